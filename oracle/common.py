"""Rounding helpers shared by the oracle modules (test infrastructure only)."""

import numpy as np
from scipy.special import erf


def f16(x):
    """Round to IEEE binary16 (round to nearest even) and return float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def ident(x):
    return np.asarray(x, dtype=np.float32)


def rounder(fp16):
    return f16 if fp16 else ident


def gelu(x):
    """Exact-erf GELU (torch F.gelu default), evaluated in float64, returned float32."""
    x64 = np.asarray(x, dtype=np.float64)
    return (0.5 * x64 * (1.0 + erf(x64 / np.sqrt(2.0)))).astype(np.float32)


def to32(a):
    return np.asarray(a, dtype=np.float32)

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


_GELU16 = None


def gelu_f16(x):
    """f16(gelu(x)) for fp16-valued x: the same values, looked up from gelu evaluated once at each of
    the 65536 fp16 inputs (the float64 erf is otherwise most of an encoder layer's CPU time)."""
    global _GELU16
    if _GELU16 is None:
        every = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
        with np.errstate(invalid='ignore', over='ignore'):
            _GELU16 = f16(gelu(every))
    h = np.asarray(x, dtype=np.float32).astype(np.float16)
    return _GELU16[h.view(np.uint16)]


def to32(a):
    return np.asarray(a, dtype=np.float32)

"""Front-end constants and the seeded synthetic clip.

The mel filterbank is the Slaney-scale, Slaney-normalised bank that WhisperFeatureExtractor builds
(transformers feature_extraction_whisper.py:95-103 -> audio_utils.mel_filter_bank, :638-744), which
the reference keeps on the GPU (custom/model.py:38). It is built here in float64 from its formulas:
mel scale linear below 1 kHz (3 f / 200) and logarithmic above (15 + ln(f / 1000) * 27 / ln 6.4),
130 equally spaced mel points over [0, 8000] Hz, triangles over the 201 FFT bin frequencies
linspace(0, 8000, 201), each scaled by 2 / (f[i+2] - f[i]).
"""

import hashlib

import numpy as np

from .config import N_FFT, N_MELS, N_SAMPLES, SAMPLE_RATE


def hz_to_mel(f):
    f = np.asarray(f, dtype=np.float64)
    lin = 3.0 * f / 200.0
    log = 15.0 + np.log(np.maximum(f, 1e-12) / 1000.0) * (27.0 / np.log(6.4))
    return np.where(f >= 1000.0, log, lin)


def mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    lin = 200.0 * m / 3.0
    log = 1000.0 * np.exp((np.log(6.4) / 27.0) * (m - 15.0))
    return np.where(m >= 15.0, log, lin)


def mel_filters(n_fft=N_FFT, n_mels=N_MELS, sr=SAMPLE_RATE, fmax=8000.0):
    """fp32[n_fft // 2 + 1, n_mels] Slaney filterbank (built in float64)."""
    bins = np.linspace(0.0, sr // 2, n_fft // 2 + 1)
    pts = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(fmax), n_mels + 2))
    lower = (bins[:, None] - pts[None, :-2]) / (pts[1:-1] - pts[:-2])[None, :]
    upper = (pts[None, 2:] - bins[:, None]) / (pts[2:] - pts[1:-1])[None, :]
    fb = np.maximum(0.0, np.minimum(lower, upper))
    fb *= (2.0 / (pts[2:] - pts[:-2]))[None, :]
    return fb.astype(np.float32)


def synthetic_clip(seed=0, n_samples=N_SAMPLES, n_tones=3, amplitude=0.1, noise_std=0.01, sr=SAMPLE_RATE):
    """Seeded 16 kHz clip: `n_tones` sinusoids with frequencies uniform in [100, 4000] Hz and uniform
    phases, amplitude 0.1 each, plus N(0, 0.01^2) noise (sigma = 0.01). Built in float64, returned fp32."""
    rng = np.random.default_rng(seed)
    freqs = rng.uniform(100.0, 4000.0, n_tones)
    phases = rng.uniform(0.0, 2.0 * np.pi, n_tones)
    t = np.arange(n_samples, dtype=np.float64) / sr
    wave = sum(amplitude * np.sin(2.0 * np.pi * f * t + p) for f, p in zip(freqs, phases))
    wave = wave + rng.standard_normal(n_samples) * noise_std
    return wave.astype(np.float32)


def sha256(array):
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()

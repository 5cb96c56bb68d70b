"""Log-mel front end in float64 (test infrastructure only).

Restates custom/model.py:93-98 (torch.stft path), whose arithmetic is
transformers feature_extraction_whisper.py:135-170 (_torch_extract_fbank_features):
  stft(n_fft=400, hop=160, periodic Hann window, center=True, reflect padding) -> drop last frame
  -> |X|^2 -> mel_filters.T @ power -> clamp(1e-10).log10() -> max(x, max - 8) -> (x + 4) / 4.
The filterbank restates transformers audio_utils.py:448-516 (Slaney mel scale), :541-560
(triangles) and :700-720 (centres, Slaney area normalisation).
"""

import numpy as np

N_FFT, HOP, N_MELS, SR = 400, 160, 128, 16000


def hann_periodic(n=N_FFT):
    return 0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(n) / n)


def _hz_to_mel(f):
    f = np.atleast_1d(np.asarray(f, dtype=np.float64))
    out = 3.0 * f / 200.0
    hi = f >= 1000.0
    out[hi] = 15.0 + np.log(f[hi] / 1000.0) * 27.0 / np.log(6.4)
    return out


def _mel_to_hz(m):
    m = np.atleast_1d(np.asarray(m, dtype=np.float64))
    out = 200.0 * m / 3.0
    hi = m >= 15.0
    out[hi] = 1000.0 * np.exp(np.log(6.4) / 27.0 * (m[hi] - 15.0))
    return out


def mel_filterbank(n_fft=N_FFT, n_mels=N_MELS, sr=SR, fmin=0.0, fmax=8000.0):
    """float64 [n_fft // 2 + 1, n_mels]."""
    fft_freqs = np.linspace(0.0, sr // 2, n_fft // 2 + 1)
    mels = np.linspace(_hz_to_mel(fmin)[0], _hz_to_mel(fmax)[0], n_mels + 2)
    centres = _mel_to_hz(mels)
    fb = np.zeros((n_fft // 2 + 1, n_mels))
    for i in range(n_mels):
        lo, c, hi = centres[i], centres[i + 1], centres[i + 2]
        rise = (fft_freqs - lo) / (c - lo)
        fall = (hi - fft_freqs) / (hi - c)
        fb[:, i] = np.maximum(0.0, np.minimum(rise, fall)) * (2.0 / (hi - lo))
    return fb


def power_spectrogram(wave, n_fft=N_FFT, hop=HOP):
    """|STFT|^2, float64 [n_fft // 2 + 1, n_frames] with the last frame dropped."""
    wave = np.asarray(wave, dtype=np.float64)
    pad = n_fft // 2
    padded = np.pad(wave, pad, mode='reflect')
    n_frames = 1 + (padded.size - n_fft) // hop
    idx = np.arange(n_fft)[None, :] + hop * np.arange(n_frames)[:, None]
    frames = padded[idx] * hann_periodic(n_fft)[None, :]
    spec = np.fft.rfft(frames, axis=1)
    return (np.abs(spec) ** 2).T[:, :-1]


def log_mel(wave, filters=None):
    """float64 [128, n_samples // 160]."""
    filters = mel_filterbank() if filters is None else np.asarray(filters, dtype=np.float64)
    mel = filters.T @ power_spectrogram(wave)
    logs = np.log10(np.maximum(mel, 1e-10))
    logs = np.maximum(logs, logs.max() - 8.0)
    return (logs + 4.0) / 4.0

"""End-to-end CPU restatement: waveform -> greedy ids (test infrastructure only).

Follows CustomModel.transcribe (custom/model.py:173-225): zero-pad to 30 s (:182-183), log-mel
(:184, oracle.logmel), fp16 mel (:188), encoder + cross K/V (:143-147, oracle.encoder), prompt +
greedy decode (:196-215, oracle.decoder.greedy).
"""

import numpy as np

from .decoder import DecoderOracle, greedy
from .encoder import cross_kv, encoder_forward
from .logmel import log_mel


def pad_wave(audio, n_samples=480000):
    wave = np.zeros(n_samples, np.float32)
    wave[: audio.size] = audio
    return wave


def transcribe_ids(params, dims, audio, prompt, n_tokens, suppress=(), begin_suppress=(), eos=(),
                   stop_at_eos=False, fp16=True, mel=None):
    """Returns dict(mel, enc, cross_kv, ids, margins). `mel` (fp16-valued [n_mels, frames]) skips the
    front end, which lets a caller feed the encoder exactly the mel another implementation produced."""
    if mel is None:
        mel = log_mel(pad_wave(audio)).astype(np.float16).astype(np.float32)
    enc = encoder_forward(params, mel, dims, fp16)
    ckv = cross_kv(params, enc, dims, fp16)
    dec = DecoderOracle(params, dims, ckv, fp16)
    out = greedy(dec, prompt, n_tokens, suppress, begin_suppress, eos, stop_at_eos)
    return dict(mel=mel, enc=enc, cross_kv=ckv, ids=out['ids'], margins=out['margins'])

"""Seeded random-init weights for the Whisper-large-v3-turbo architecture.

The reference loads the real checkpoint with ``from_pretrained`` (custom/model.py:32-36); offline
there is none, so every tensor comes from a counter-based generator (``fw_synth_normal_f16`` in
csrc/synth.hip) keyed by (seed, crc32 of the HF parameter name). The same bits come out on the host
(for the CPU oracle) and on the GPU (for the product), so both see identical weights without moving
800 M parameters around.

Initialisation: every linear/conv weight and bias, the token embedding (tied LM head) and the decoder
positions are N(0, 0.02) in fp16; LayerNorm gamma = 1, beta = 0; the encoder positions are the
sinusoids of transformers models/whisper/modeling_whisper.py:55-65. k_proj has no bias (HF
WhisperAttention, modeling_whisper.py:279).
"""

import ctypes
import math
import zlib

import numpy as np

from . import _lib
from .config import TURBO

STD = 0.02


def tensor_id(name):
    return zlib.crc32(name.encode())


def _attn(prefix, d, with_bias=True):
    out = [(f'{prefix}.q_proj.weight', (d, d), 'normal'), (f'{prefix}.q_proj.bias', (d,), 'normal'),
           (f'{prefix}.k_proj.weight', (d, d), 'normal'),
           (f'{prefix}.v_proj.weight', (d, d), 'normal'), (f'{prefix}.v_proj.bias', (d,), 'normal'),
           (f'{prefix}.out_proj.weight', (d, d), 'normal'), (f'{prefix}.out_proj.bias', (d,), 'normal')]
    return out


def _ln(prefix, d):
    return [(f'{prefix}.weight', (d,), 'one'), (f'{prefix}.bias', (d,), 'zero')]


def param_specs(dims=TURBO):
    """(name, shape, kind) for every parameter, in HF naming (model.encoder.* / model.decoder.*)."""
    d, f = dims.d_model, dims.ffn
    e, dd = 'model.encoder', 'model.decoder'
    specs = [(f'{e}.conv1.weight', (d, dims.n_mels, 3), 'normal'), (f'{e}.conv1.bias', (d,), 'normal'),
             (f'{e}.conv2.weight', (d, d, 3), 'normal'), (f'{e}.conv2.bias', (d,), 'normal'),
             (f'{e}.embed_positions.weight', (dims.enc_len, d), 'sinusoid')]
    for i in range(dims.enc_layers):
        p = f'{e}.layers.{i}'
        specs += _attn(f'{p}.self_attn', d) + _ln(f'{p}.self_attn_layer_norm', d)
        specs += [(f'{p}.fc1.weight', (f, d), 'normal'), (f'{p}.fc1.bias', (f,), 'normal'),
                  (f'{p}.fc2.weight', (d, f), 'normal'), (f'{p}.fc2.bias', (d,), 'normal')]
        specs += _ln(f'{p}.final_layer_norm', d)
    specs += _ln(f'{e}.layer_norm', d)
    specs += [(f'{dd}.embed_tokens.weight', (dims.vocab, d), 'normal'),
              (f'{dd}.embed_positions.weight', (dims.max_pos, d), 'normal')]
    for i in range(dims.dec_layers):
        p = f'{dd}.layers.{i}'
        specs += _attn(f'{p}.self_attn', d) + _ln(f'{p}.self_attn_layer_norm', d)
        specs += _attn(f'{p}.encoder_attn', d) + _ln(f'{p}.encoder_attn_layer_norm', d)
        specs += [(f'{p}.fc1.weight', (f, d), 'normal'), (f'{p}.fc1.bias', (f,), 'normal'),
                  (f'{p}.fc2.weight', (d, f), 'normal'), (f'{p}.fc2.bias', (d,), 'normal')]
        specs += _ln(f'{p}.final_layer_norm', d)
    specs += _ln(f'{dd}.layer_norm', d)
    ids = [tensor_id(n) for n, _, _ in specs]
    assert len(set(ids)) == len(ids), 'tensor id collision'
    return specs


def spec_map(dims=TURBO):
    return {n: (s, k) for n, s, k in param_specs(dims)}


def sinusoids(length, channels, max_timescale=10000.0):
    """Whisper encoder positions: [sin(t * w_i), cos(t * w_i)] with log-spaced w_i (float64)."""
    inc = math.log(max_timescale) / (channels // 2 - 1)
    inv = np.exp(-inc * np.arange(channels // 2, dtype=np.float64))
    t = np.arange(length, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.sin(t), np.cos(t)], axis=1)


def host_normal(name, shape, seed=0, std=STD, mean=0.0):
    """fp16 N(mean, std) tensor computed on the host by the same generator the GPU uses."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float16)
    _lib.check(_lib.lib().fw_synth_normal_f16_host(out.ctypes.data_as(ctypes.c_void_p), n, 0, seed,
                                                   tensor_id(name), mean, std), f'synth {name}')
    return out.reshape(shape)


def host_param(name, shape, kind, seed=0):
    if kind == 'normal':
        return host_normal(name, shape, seed)
    if kind == 'one':
        return np.ones(shape, dtype=np.float16)
    if kind == 'zero':
        return np.zeros(shape, dtype=np.float16)
    if kind == 'sinusoid':
        return sinusoids(*shape).astype(np.float16)
    raise ValueError(kind)


def host_params(dims=TURBO, seed=0, names=None):
    """Dict name -> fp16 numpy array (all parameters, or only `names`)."""
    specs = param_specs(dims)
    want = None if names is None else set(names)
    return {n: host_param(n, s, k, seed) for n, s, k in specs if want is None or n in want}


def device_fill(tensor, name, kind, seed=0, stream=None):
    """Fills a contiguous CUDA fp16 tensor with parameter `name` (same bits as host_param)."""
    import torch

    if kind == 'normal':
        s = stream if stream is not None else torch.cuda.current_stream()
        _lib.check(_lib.lib().fw_synth_normal_f16(tensor.data_ptr(), tensor.numel(), 0, seed, tensor_id(name), 0.0,
                                                  STD, s.cuda_stream), f'synth {name}')
    elif kind == 'one':
        tensor.fill_(1.0)
    elif kind == 'zero':
        tensor.zero_()
    elif kind == 'sinusoid':
        tensor.copy_(torch.from_numpy(sinusoids(*tensor.shape).astype(np.float16)))
    else:
        raise ValueError(kind)
    return tensor

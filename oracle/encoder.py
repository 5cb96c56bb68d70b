"""Whisper encoder and cross K/V projection on the CPU (test infrastructure only).

Restates transformers WhisperEncoder.forward (models/whisper/modeling_whisper.py:592-648) as the
reference runs it in fp16 (custom/model.py:32-34,143-147): every op output is rounded to fp16 with
fp32 accumulation inside the op. Rounding points (``fp16=True``):
  conv1: fp16(conv + b) -> fp16(gelu)            (:618)
  conv2 (stride 2): same, then fp16(x + positions) (:619-623, sinusoids :55-65)
  layer (:379-414): y = fp16(LN(x)); q = fp16(fp16(y Wq^T + bq) * head_dim^-0.5) (:309);
    k = fp16(y Wk^T) (no bias, :279); v = fp16(y Wv^T + bv); o = fp16(softmax(q k^T) v) (SDPA, scale 1);
    x = fp16(x + fp16(o Wo^T + bo)); y = fp16(LN(x)); u = fp16(gelu(fp16(y W1^T + b1)));
    x = fp16(x + fp16(u W2^T + b2)); clamp to +-(65504 - 1000) (:409-411)
  final: fp16(LN(x)) (:642)
With ``fp16=False`` nothing is rounded and the clamp is skipped (transformers clamps only in fp16),
which is the setting the fp32 golden vectors of a tiny transformers model pin.
Cross K/V: fp16(enc @ [k_0; v_0; k_1; ...]^T + [0; b_v0; 0; ...]) permuted to [layers, 2, heads, t, hd]
(custom/model.py:53-55, 145-146).
"""

import numpy as np

from .common import gelu, rounder, to32
from .decoder import layer_norm

CLAMP = 65504.0 - 1000.0


def conv1d(x, w, b, stride):
    """x [c_in, t], w [c_out, c_in, 3], padding 1 -> [c_out, t_out] (float32 accumulation)."""
    c_in, t = x.shape
    t_out = (t - 1) // stride + 1
    xp = np.zeros((c_in, t + 2), np.float32)
    xp[:, 1:-1] = x
    out = np.zeros((w.shape[0], t_out), np.float32)
    for tap in range(3):
        cols = xp[:, tap: tap + stride * (t_out - 1) + 1: stride]
        out += to32(w[:, :, tap]) @ cols
    return out + to32(b)[:, None]


def self_attention(y, p, heads, rnd, fp16):
    t, dm = y.shape
    hd = dm // heads
    scale = hd ** -0.5
    q = rnd(rnd(y @ p['q_w'].T + p['q_b']) * scale)
    k = rnd(y @ p['k_w'].T)
    v = rnd(y @ p['v_w'].T + p['v_b'])
    qh = q.reshape(t, heads, hd).transpose(1, 0, 2)
    kh = k.reshape(t, heads, hd).transpose(1, 0, 2)
    vh = v.reshape(t, heads, hd).transpose(1, 0, 2)
    o = np.empty((heads, t, hd), np.float32)
    for h in range(heads):  # one head at a time keeps the score matrix small
        s = qh[h] @ kh[h].T
        s -= s.max(axis=1, keepdims=True)
        e = np.exp(s)
        o[h] = (e @ vh[h]) / e.sum(axis=1, keepdims=True)
    o = rnd(o.transpose(1, 0, 2).reshape(t, dm))
    return rnd(o @ p['o_w'].T + p['o_b'])


def layer_params(params, i):
    g = lambda n: to32(params[n])
    q = f'model.encoder.layers.{i}'
    sa = f'{q}.self_attn'
    return dict(ln1=(g(f'{q}.self_attn_layer_norm.weight'), g(f'{q}.self_attn_layer_norm.bias')),
                q_w=g(f'{sa}.q_proj.weight'), q_b=g(f'{sa}.q_proj.bias'), k_w=g(f'{sa}.k_proj.weight'),
                v_w=g(f'{sa}.v_proj.weight'), v_b=g(f'{sa}.v_proj.bias'),
                o_w=g(f'{sa}.out_proj.weight'), o_b=g(f'{sa}.out_proj.bias'),
                ln2=(g(f'{q}.final_layer_norm.weight'), g(f'{q}.final_layer_norm.bias')),
                fc1_w=g(f'{q}.fc1.weight'), fc1_b=g(f'{q}.fc1.bias'),
                fc2_w=g(f'{q}.fc2.weight'), fc2_b=g(f'{q}.fc2.bias'))


def encoder_layer(x, p, heads, eps, fp16=True):
    rnd = rounder(fp16)
    y = rnd(layer_norm(x, *p['ln1'], eps))
    x = rnd(x + self_attention(y, p, heads, rnd, fp16))
    y = rnd(layer_norm(x, *p['ln2'], eps))
    u = rnd(gelu(rnd(y @ p['fc1_w'].T + p['fc1_b'])))
    x = rnd(x + rnd(u @ p['fc2_w'].T + p['fc2_b']))
    if fp16:
        x = np.clip(x, -CLAMP, CLAMP)
    return x


def embed_stem(params, mel, fp16=True):
    """mel [n_mels, 2 * t] -> x [t, d_model] (conv1, conv2, GELU, + positions)."""
    rnd = rounder(fp16)
    g = lambda n: to32(params[n])
    e = 'model.encoder'
    x = rnd(gelu(rnd(conv1d(to32(mel), g(f'{e}.conv1.weight'), g(f'{e}.conv1.bias'), 1))))
    x = rnd(gelu(rnd(conv1d(x, g(f'{e}.conv2.weight'), g(f'{e}.conv2.bias'), 2))))
    return rnd(x.T + g(f'{e}.embed_positions.weight')[: x.shape[1]])


def encoder_forward(params, mel, dims, fp16=True, n_layers=None, final_ln=True, collect=None):
    """Returns the encoder output [t, d_model] (float32, fp16-valued when fp16=True).
    `collect`, if a list, receives the hidden state after the stem and after every layer."""
    rnd = rounder(fp16)
    x = embed_stem(params, mel, fp16)
    if collect is not None:
        collect.append(x.copy())
    n = dims.enc_layers if n_layers is None else n_layers
    for i in range(n):
        x = encoder_layer(x, layer_params(params, i), dims.heads, dims.ln_eps, fp16)
        if collect is not None:
            collect.append(x.copy())
    if final_ln:
        g = lambda nm: to32(params[nm])
        x = rnd(layer_norm(x, g('model.encoder.layer_norm.weight'), g('model.encoder.layer_norm.bias'), dims.ln_eps))
    return x


def cross_kv(params, enc, dims, fp16=True):
    """[layers, 2, heads, t, hd] K/V of every decoder layer's cross-attention."""
    rnd = rounder(fp16)
    t = enc.shape[0]
    out = np.empty((dims.dec_layers, 2, dims.heads, t, dims.head_dim), np.float32)
    for i in range(dims.dec_layers):
        a = f'model.decoder.layers.{i}.encoder_attn'
        k = rnd(enc @ to32(params[f'{a}.k_proj.weight']).T)
        v = rnd(enc @ to32(params[f'{a}.v_proj.weight']).T + to32(params[f'{a}.v_proj.bias']))
        out[i, 0] = k.reshape(t, dims.heads, dims.head_dim).transpose(1, 0, 2)
        out[i, 1] = v.reshape(t, dims.heads, dims.head_dim).transpose(1, 0, 2)
    return out

"""Whisper encoder and cross K/V projection on the CPU (test infrastructure only).

Restates transformers WhisperEncoder.forward (models/whisper/modeling_whisper.py:592-648) as the
reference runs it in fp16 (custom/model.py:32-34,143-147): every op output is rounded to fp16 with
fp32 accumulation inside the op. Rounding points (``fp16=True``), one function per op so each can be
checked on its own against transformers' intermediate tensors:
  conv1: fp16(conv + b) -> fp16(gelu)            (:618)
  conv2 (stride 2): same, then fp16(x + positions) (:619-623, sinusoids :55-65)
  layer (:379-414):
    ln_op      y = fp16(LN(x))
    q_op       q = fp16(fp16(y Wq^T + bq) * head_dim^-0.5)   (q scaled after its rounding, :309)
    k_op       k = fp16(y Wk^T)                               (no bias, :279)
    v_op       v = fp16(y Wv^T + bv)
    attention_core  o = fp16(softmax(q k^T) v)                (SDPA with scale 1; fp32 softmax here)
    linear_op  fp16(o Wo^T + bo), fc1, fc2 (bias added before the single rounding)
    gelu_op    fp16(gelu(a))                                  (exact erf)
    residual_op x = fp16(x + r); after fc2, clamp(x, +-(65504 - 1000)) in fp16 (:409-411), which
                rounds the bound to fp16: +-64512
  final: fp16(LN(x)) (:642)
With ``fp16=False`` nothing is rounded and the clamp is skipped (transformers clamps only in fp16),
which is the setting the fp32 golden vectors of a tiny transformers model pin.

The attention core computes the softmax in float32 and rounds the output once. Flash-style kernels
(torch SDPA on the CPU and on CUDA, and this build's HIP kernel) round the unnormalised
probabilities to fp16 before the P.V product; that moves results by about one fp16 ulp and is inside
the 2e-3 relative tolerance the parity tests use.

Cross K/V: fp16(enc @ [k_0; v_0; k_1; ...]^T + [0; b_v0; 0; ...]) permuted to [layers, 2, heads, t, hd]
(custom/model.py:53-55, 145-146).
"""

import numpy as np

from .common import f16, gelu, gelu_f16, rounder, to32
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


def ln_op(x, ln, eps, fp16=True):
    return rounder(fp16)(layer_norm(x, *ln, eps))


def linear_op(a, w, b=None, fp16=True):
    """fp16(a W^T + b): fp32 accumulation, bias added before the single rounding."""
    out = a @ to32(w).T
    if b is not None:
        out = out + to32(b)
    return rounder(fp16)(out)


def q_op(y, p, heads, fp16=True):
    """The query as transformers hands it to SDPA: the projection is rounded, then scaled and rounded
    again (modeling_whisper.py:309); SDPA itself then runs with scale 1."""
    scale = (y.shape[-1] // heads) ** -0.5
    return rounder(fp16)(linear_op(y, p['q_w'], p['q_b'], fp16) * scale)


def k_op(y, p, fp16=True):
    return linear_op(y, p['k_w'], None, fp16)


def v_op(y, p, fp16=True):
    return linear_op(y, p['v_w'], p['v_b'], fp16)


def attention_core(q, k, v, heads, fp16=True):
    """Non-causal softmax(q k^T) v per head (q already scaled); q/k/v and the result are [t, d_model]."""
    t, dm = q.shape
    hd = dm // heads
    split = lambda a: to32(a).reshape(a.shape[0], heads, hd).transpose(1, 0, 2)
    qh, kh, vh = split(q), split(k), split(v)
    o = np.empty((heads, t, hd), np.float32)
    for h in range(heads):  # one head at a time keeps the score matrix small
        s = qh[h] @ kh[h].T
        s -= s.max(axis=1, keepdims=True)
        e = np.exp(s)
        o[h] = (e @ vh[h]) / e.sum(axis=1, keepdims=True)
    return rounder(fp16)(o.transpose(1, 0, 2).reshape(t, dm))


def gelu_op(a, fp16=True):
    if fp16 and np.array_equal(f16(a), a):  # fp16-valued input: table lookup, same values
        return gelu_f16(a)
    return rounder(fp16)(gelu(a))


def residual_op(x, r, fp16=True, clamp=False):
    """fp16(x + r); with `clamp` (the end of an fp16 layer) the result is clamped to +-CLAMP in fp16:
    torch.clamp on a half tensor rounds the bound to fp16 too, so the clamped value is 64512 (the
    fp16 nearest to 64504)."""
    rnd = rounder(fp16)
    out = rnd(to32(x) + to32(r))
    if clamp and fp16:
        out = rnd(np.clip(out, -CLAMP, CLAMP))
    return out


def self_attention(y, p, heads, fp16=True, trace=None):
    q, k, v = q_op(y, p, heads, fp16), k_op(y, p, fp16), v_op(y, p, fp16)
    o = attention_core(q, k, v, heads, fp16)
    out = linear_op(o, p['o_w'], p['o_b'], fp16)
    if trace is not None:
        trace.update(q=q, k=k, v=v, attn=o, attn_out=out)
    return out


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


def encoder_layer(x, p, heads, eps, fp16=True, trace=None):
    """One pre-LN encoder layer. `trace`, if a dict, receives every op's output by name
    (ln1, q, k, v, attn, attn_out, x_attn, ln2, fc1, gelu, fc2, out)."""
    y = ln_op(x, p['ln1'], eps, fp16)
    x_attn = residual_op(x, self_attention(y, p, heads, fp16, trace), fp16)
    y2 = ln_op(x_attn, p['ln2'], eps, fp16)
    a = linear_op(y2, p['fc1_w'], p['fc1_b'], fp16)
    u = gelu_op(a, fp16)
    m = linear_op(u, p['fc2_w'], p['fc2_b'], fp16)
    out = residual_op(x_attn, m, fp16, clamp=True)
    if trace is not None:
        trace.update(ln1=y, x_attn=x_attn, ln2=y2, fc1=a, gelu=u, fc2=m, out=out)
    return out


def embed_stem(params, mel, fp16=True):
    """mel [n_mels, 2 * t] -> x [t, d_model] (conv1, conv2, GELU, + positions)."""
    rnd = rounder(fp16)
    g = lambda n: to32(params[n])
    e = 'model.encoder'
    x = gelu_op(rnd(conv1d(to32(mel), g(f'{e}.conv1.weight'), g(f'{e}.conv1.bias'), 1)), fp16)
    x = gelu_op(rnd(conv1d(x, g(f'{e}.conv2.weight'), g(f'{e}.conv2.bias'), 2)), fp16)
    return residual_op(x.T, g(f'{e}.embed_positions.weight')[: x.shape[1]], fp16)


def encoder_forward(params, mel, dims, fp16=True, n_layers=None, final_ln=True, collect=None):
    """Returns the encoder output [t, d_model] (float32, fp16-valued when fp16=True).
    `collect`, if a list, receives the hidden state after the stem and after every layer."""
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
        x = ln_op(x, (g('model.encoder.layer_norm.weight'), g('model.encoder.layer_norm.bias')), dims.ln_eps, fp16)
    return x


def cross_kv(params, enc, dims, fp16=True):
    """[layers, 2, heads, t, hd] K/V of every decoder layer's cross-attention."""
    t = enc.shape[0]
    out = np.empty((dims.dec_layers, 2, dims.heads, t, dims.head_dim), np.float32)
    for i in range(dims.dec_layers):
        a = f'model.decoder.layers.{i}.encoder_attn'
        k = linear_op(enc, params[f'{a}.k_proj.weight'], None, fp16)
        v = linear_op(enc, params[f'{a}.v_proj.weight'], params[f'{a}.v_proj.bias'], fp16)
        out[i, 0] = k.reshape(t, dims.heads, dims.head_dim).transpose(1, 0, 2)
        out[i, 1] = v.reshape(t, dims.heads, dims.head_dim).transpose(1, 0, 2)
    return out

"""Decoder step, decode kernels and greedy loop on the CPU (test infrastructure only).

Follows the reference CUDA path:
- ``add_layernorm``: custom/kernels/whisper_kernels.cu:215-267 (fp16 residual h = fp16(h + x) at
  :232-233, two-pass fp32 statistics, y = fp16((r - mean) * rsqrt(var + eps) * gamma + beta) at :265).
- ``attention``: custom/selftest.py:26-28 (softmax(q k^T * scale) v) with the kernel's fp16 output
  (whisper_kernels.cu:212) and the fused KV-cache write of :137-145.
- ``lm_head_argmax``: whisper_kernels.cu:28-86 with pack_score :20-26 — logits rounded to fp16 before
  the argmax (:70-71), suppressed rows skipped (:72), lowest index wins ties.
- ``finalize``: whisper_kernels.cu:88-100.
- ``DecoderOracle.step``: custom/model.py:107-123 (embedding + positions :110, the layer chain
  :113-120 with the MLP residual deferred through ``pending``, final LN + LM head :121-122).
- ``greedy``: the prompt / first-token / chunked loop of custom/model.py:196-215, in the fixed-length
  mode used for the synthetic clip (no EOS stop unless asked).
"""

import numpy as np

from .common import gelu, rounder, to32


def layer_norm(r, gamma, beta, eps):
    """Textbook LayerNorm in float64 of the last axis (biased variance), returned float32."""
    r64 = np.asarray(r, dtype=np.float64)
    mean = r64.mean(axis=-1, keepdims=True)
    var = ((r64 - mean) ** 2).mean(axis=-1, keepdims=True)
    return ((r64 - mean) / np.sqrt(var + eps) * np.asarray(gamma, np.float64)
            + np.asarray(beta, np.float64)).astype(np.float32)


def add_layernorm(h, x, gamma, beta, eps=1e-5, fp16=True):
    """Returns (h_new, y). h_new = fp16(h + x) (or h when x is None), y = fp16(LN(h_new))."""
    rnd = rounder(fp16)
    r = to32(h) if x is None else rnd(to32(h) + to32(x))
    return r, rnd(layer_norm(r, gamma, beta, eps))


def attention(q, k, v, length, scale, fp16=True):
    """q [H, hd], k/v [H, >=length, hd] -> out [H * hd]: softmax over the first `length` keys."""
    q64 = np.asarray(q, np.float64)
    k64 = np.asarray(k[:, :length], np.float64)
    v64 = np.asarray(v[:, :length], np.float64)
    s = np.einsum('hd,hld->hl', q64, k64) * scale
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    out = np.einsum('hl,hld->hd', p, v64).astype(np.float32).reshape(-1)
    return rounder(fp16)(out)


def lm_head_logits(y, w, fp16=True):
    """fp32-or-better dot of every row with y, rounded to fp16 like the kernel (whisper_kernels.cu:70-71)."""
    logits = np.asarray(w, np.float32) @ np.asarray(y, np.float32)
    return rounder(fp16)(logits)


def masked_argmax(logits, suppress):
    """Highest logit among unsuppressed rows, lowest index on ties (torch.argmax / pack_score order)."""
    masked = np.where(np.asarray(suppress, bool), -np.inf, logits)
    return int(np.argmax(masked))  # np.argmax returns the first (lowest) index of the maximum


def lm_head_argmax(y, w, suppress, fp16=True):
    return masked_argmax(lm_head_logits(y, w, fp16), suppress)


def finalize(token, tokens, state, max_pos):
    """Reference argmax_finalize: returns (tokens, state, cur) after appending `token`."""
    tokens = list(tokens)
    pos, n = int(state[0]), int(state[1])
    if n < max_pos:
        if n < len(tokens):
            tokens[n] = token
    n = n + 1 if n < max_pos else n
    pos = pos + 1 if pos + 1 < max_pos else max_pos - 1
    return tokens, [pos, n], token


def top2_margin(logits, suppress):
    masked = np.where(np.asarray(suppress, bool), -np.inf, np.asarray(logits, np.float64))
    top = np.partition(masked, -2)[-2:]
    return float(top[1] - top[0])


class DecoderOracle:
    """Batch-1 decoder with a static self-attention cache, following custom/model.py:107-123."""

    def __init__(self, params, dims, cross_kv, fp16=True):
        self.dims, self.fp16, self.rnd = dims, fp16, rounder(fp16)
        g = lambda n: to32(params[n])
        p = 'model.decoder'
        self.embed = g(f'{p}.embed_tokens.weight')
        self.pos_embed = g(f'{p}.embed_positions.weight')
        self.layers = []
        for i in range(dims.dec_layers):
            q = f'{p}.layers.{i}'
            sa, ca = f'{q}.self_attn', f'{q}.encoder_attn'
            ln = lambda m: (g(f'{m}.weight'), g(f'{m}.bias'))
            zero = np.zeros(dims.d_model, np.float32)
            self.layers.append(dict(
                ln1=ln(f'{q}.self_attn_layer_norm'), ln2=ln(f'{q}.encoder_attn_layer_norm'),
                ln3=ln(f'{q}.final_layer_norm'),
                # custom/model.py:87-88: [q; k; v] with a zero k bias
                qkv_w=np.concatenate([g(f'{sa}.q_proj.weight'), g(f'{sa}.k_proj.weight'), g(f'{sa}.v_proj.weight')]),
                qkv_b=np.concatenate([g(f'{sa}.q_proj.bias'), zero, g(f'{sa}.v_proj.bias')]),
                out=(g(f'{sa}.out_proj.weight'), g(f'{sa}.out_proj.bias')),
                cross_q=(g(f'{ca}.q_proj.weight'), g(f'{ca}.q_proj.bias')),
                cross_out=(g(f'{ca}.out_proj.weight'), g(f'{ca}.out_proj.bias')),
                fc1=(g(f'{q}.fc1.weight'), g(f'{q}.fc1.bias')), fc2=(g(f'{q}.fc2.weight'), g(f'{q}.fc2.bias'))))
        self.final_ln = (g(f'{p}.layer_norm.weight'), g(f'{p}.layer_norm.bias'))
        self.cross_kv = to32(cross_kv)  # [layers, 2, heads, t, hd]
        self.self_kv = np.zeros((dims.dec_layers, 2, dims.heads, dims.max_pos, dims.head_dim), np.float32)
        self.scale = dims.head_dim ** -0.5

    def linear(self, x, wb):
        w, b = wb
        return self.rnd(w @ x + b)

    def step(self, cur, pos):
        """One decoder token at position `pos`; returns the fp16-rounded (or fp32) logits."""
        d, eps, rnd = self.dims, self.dims.ln_eps, self.rnd
        h = rnd(self.embed[cur] + self.pos_embed[pos])
        pending = None
        for i, lay in enumerate(self.layers):
            h, y = add_layernorm(h, pending, *lay['ln1'], eps, self.fp16)
            qkv = self.linear(y, (lay['qkv_w'], lay['qkv_b'])).reshape(3, d.heads, d.head_dim)
            self.self_kv[i, 0, :, pos] = qkv[1]
            self.self_kv[i, 1, :, pos] = qkv[2]
            attn = attention(qkv[0], self.self_kv[i, 0], self.self_kv[i, 1], pos + 1, self.scale, self.fp16)
            h, y = add_layernorm(h, self.linear(attn, lay['out']), *lay['ln2'], eps, self.fp16)
            q = self.linear(y, lay['cross_q']).reshape(d.heads, d.head_dim)
            ck = self.cross_kv[i, 0]
            attn = attention(q, ck, self.cross_kv[i, 1], ck.shape[1], self.scale, self.fp16)
            h, y = add_layernorm(h, self.linear(attn, lay['cross_out']), *lay['ln3'], eps, self.fp16)
            pending = self.linear(rnd(gelu(self.linear(y, lay['fc1']))), lay['fc2'])
        h, y = add_layernorm(h, pending, *self.final_ln, eps, self.fp16)
        self.last_h, self.last_y = h, y
        return lm_head_logits(y, self.embed, self.fp16)


def suppress_masks(vocab, suppress, begin_suppress):
    base = np.zeros(vocab, bool)
    base[list(suppress)] = True
    first = base.copy()
    first[list(begin_suppress)] = True
    return base, first


def greedy(oracle, prompt, n_tokens, suppress=(), begin_suppress=(), eos=(), stop_at_eos=False, teacher=None):
    """Greedy ids exactly as custom/model.py:196-215 produces them (prompt steps write the cache but
    their predictions are discarded; the last prompt step uses the begin-suppress mask).
    With `teacher` (a list of ids), each step is fed teacher[i] instead of the oracle's own choice,
    which yields per-step argmaxes for a teacher-forced comparison.
    Returns dict(ids, margins) where margins[i] is the top-2 gap of the logits that produced ids[i]."""
    dims = oracle.dims
    base, first = suppress_masks(dims.vocab, suppress, begin_suppress)
    ids, margins = [], []
    pos = 0
    for i, tok in enumerate(prompt):
        logits = oracle.step(tok, pos)
        pos = min(pos + 1, dims.max_pos - 1)
        if i == len(prompt) - 1:
            ids.append(masked_argmax(logits, first))
            margins.append(top2_margin(logits, first))
    while len(ids) < n_tokens:
        if stop_at_eos and ids[-1] in eos:
            break
        cur = ids[-1] if teacher is None else teacher[len(ids) - 1]
        logits = oracle.step(cur, pos)
        pos = min(pos + 1, dims.max_pos - 1)
        ids.append(masked_argmax(logits, base))
        margins.append(top2_margin(logits, base))
    return dict(ids=ids, margins=margins)

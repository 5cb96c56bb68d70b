"""Kernel self-checks run when a model is built (the drop-in for custom/selftest.py).

Gate interface, kept as the reference defines it (custom/selftest.py:15-19,22-23,32-101):
``run_selftest(ext)`` returns ``{'ok': bool, 'checks': [{'name', 'max_err', 'ok'}, ...]}``, ``ok`` being
true only when every check is; the reference's check names and tolerances are kept (add_layernorm
2e-2; decode_attention_self_<L> and decode_attention_cross 1e-2; kv_write_<L> exact; lm_head_argmax:
the chosen row's logit within 1e-3 of the best unsuppressed one, with the finalize bookkeeping intact);
``workspace(heads, splits)`` sizes the split-K partials; ``python -m custom.selftest --out DIR``
writes ``DIR/selftest.json``.

How the checks are made here: every input is drawn on the host from one seeded numpy generator and
uploaded, and every reference is computed on the host in float64, so no device math library takes part
in judging a kernel. The checks are grouped by kernel family (``FAMILIES``); each family is a
generator of ``(name, error, tolerance)`` triples. Besides the reference's checks, each fused kernel of
this build's decoder step is compared with the unfused ops it replaces: LN + GEMV, the one-launch
attention, the fused final LN + LM head + finalize, and the LM head with the int8 pre-pass (which must
pick the same token, bit for bit, as the fp16 head).
"""

import argparse
import json
import math
from pathlib import Path

import numpy as np
import torch

from .config import SPLIT_KEYS

HIDDEN, HEADS, HEAD_DIM, VOCAB = 1280, 20, 64, 51866
MAX_POS, ENC_LEN = 448, 1500
SELF_LENGTHS = (1, 63, 64, 65, 200, 448)
EPS = 1e-5

# tolerances of the reference gate (custom/selftest.py:44,57,64,72,86); 0 means bit for bit
TOL_LAYERNORM, TOL_ATTENTION, TOL_ARGMAX_GAP, EXACT = 2e-2, 1e-2, 1e-3, 0.0


def workspace(heads, splits, device='cuda'):
    """fp32 split-K attention partials: running max and exp-sum per (head, split), and the
    unnormalised value sum per (head, split, dim)."""
    m = torch.empty(heads * splits, device=device)
    return m, torch.empty_like(m), torch.empty(heads * splits * HEAD_DIM, device=device)


class _Inputs:
    """Seeded host inputs (fp16 values) and their device copies."""

    def __init__(self, seed=0):
        self.rng = np.random.default_rng(seed)

    def draw(self, *shape, std=1.0):
        return (self.rng.standard_normal(shape, dtype=np.float32) * std).astype(np.float16)

    @staticmethod
    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    @staticmethod
    def host(t):
        return t.detach().float().cpu().numpy().astype(np.float64)


def _ln64(r, gamma, beta):
    r = np.asarray(r, np.float64)
    mu = r.mean(-1, keepdims=True)
    var = ((r - mu) ** 2).mean(-1, keepdims=True)
    return (r - mu) / np.sqrt(var + EPS) * np.asarray(gamma, np.float64) + np.asarray(beta, np.float64)


def _attn64(q, k, v, length, scale):
    """q [H, D], k/v [H, >=length, D] -> softmax(q k^T * scale) v over the first `length` keys, [H * D]."""
    k, v = np.asarray(k[:, :length], np.float64), np.asarray(v[:, :length], np.float64)
    s = np.einsum('hd,hld->hl', np.asarray(q, np.float64), k) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum('hl,hld->hd', p, v).reshape(-1)


def _maxdiff(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def _finalize_state():
    dev = 'cuda'
    return (torch.zeros(1, dtype=torch.long, device=dev), torch.zeros(8, dtype=torch.long, device=dev),
            torch.tensor([3, 0], dtype=torch.long, device=dev), torch.zeros(1, dtype=torch.long, device=dev))


def _layernorm_family(ext, inp):
    h, x = inp.draw(1, HIDDEN), inp.draw(1, HIDDEN)
    gamma, beta = inp.draw(HIDDEN), inp.draw(HIDDEN)
    th, tx, tg, tb = inp.dev(h), inp.dev(x), inp.dev(gamma), inp.dev(beta)
    h_before = th.clone()
    y = torch.empty_like(th)
    ext.add_layernorm(th, tx, tg, tb, y, EPS)
    r = (h.astype(np.float32) + x.astype(np.float32)).astype(np.float16)  # the fp16 residual
    err = max(_maxdiff(inp.host(y), _ln64(r, gamma, beta)), _maxdiff(inp.host(th), r))
    yield 'add_layernorm', err, TOL_LAYERNORM
    # residual + LN + GEMV in one launch == add_layernorm followed by the GEMV
    w, b = inp.dev(inp.draw(3 * HIDDEN, HIDDEN, std=0.02)), inp.dev(inp.draw(3 * HIDDEN, std=0.02))
    fused, unfused = (torch.empty(3 * HIDDEN, dtype=torch.float16, device='cuda') for _ in range(2))
    h_out = torch.empty_like(th)
    ext.ln_gemv(h_before, tx, h_out, tg, tb, EPS, w, b, fused)
    ext.gemv(y, w, b, unfused)
    yield 'ln_gemv_vs_unfused', max(float((fused - unfused).abs().max()), float((h_out - th).abs().max())), EXACT


def _self_attention_family(ext, inp):
    scale = HEAD_DIM ** -0.5
    ws = workspace(HEADS, -(-ENC_LEN // SPLIT_KEYS))
    for length in SELF_LENGTHS:
        pos = length - 1
        q = inp.draw(HEADS, HEAD_DIM)
        k, v = inp.draw(HEADS, MAX_POS, HEAD_DIM), inp.draw(HEADS, MAX_POS, HEAD_DIM)
        k_new, v_new = inp.draw(HEADS, 1, HEAD_DIM), inp.draw(HEADS, 1, HEAD_DIM)
        k_want, v_want = k.copy(), v.copy()   # the cache after the fused write of row `pos`
        k_want[:, pos], v_want[:, pos] = k_new[:, 0], v_new[:, 0]
        ref = _attn64(q, k_want, v_want, length, scale)
        state = inp.dev(np.array([pos, 0], np.int64))
        tq, tkn, tvn = inp.dev(q.reshape(-1)), inp.dev(k_new), inp.dev(v_new)
        for tag, launch in (('', lambda tk, tv, out: ext.decode_attention(tq, tk, tv, out, state, tkn, tvn, *ws, scale)),
                            ('fused_', lambda tk, tv, out: ext.decode_attention_fused(tq, tk, tv, out, state, tkn,
                                                                                      tvn, scale))):
            tk, tv = inp.dev(k), inp.dev(v)
            out = torch.empty_like(tq)
            launch(tk, tv, out)
            yield f'decode_attention_{tag}self_{length}', _maxdiff(inp.host(out), ref), TOL_ATTENTION
            # the new row is written, and nothing else in the cache moves
            yield f'kv_write_{tag}{length}', max(_maxdiff(inp.host(tk), k_want), _maxdiff(inp.host(tv), v_want)), EXACT


def _cross_attention_family(ext, inp):
    scale = HEAD_DIM ** -0.5
    ws = workspace(HEADS, -(-ENC_LEN // SPLIT_KEYS))
    q = inp.draw(HEADS, HEAD_DIM)
    k, v = inp.draw(HEADS, ENC_LEN, HEAD_DIM), inp.draw(HEADS, ENC_LEN, HEAD_DIM)
    ref = _attn64(q, k, v, ENC_LEN, scale)
    tq, tk, tv = inp.dev(q.reshape(-1)), inp.dev(k), inp.dev(v)
    out = torch.empty_like(tq)
    ext.decode_attention(tq, tk, tv, out, None, None, None, *ws, scale)
    yield 'decode_attention_cross', _maxdiff(inp.host(out), ref), TOL_ATTENTION
    out = torch.empty_like(tq)
    ext.decode_attention_fused(tq, tk, tv, out, None, None, None, scale)
    yield 'decode_attention_fused_cross', _maxdiff(inp.host(out), ref), TOL_ATTENTION


def _lm_head_family(ext, inp):
    w = inp.draw(VOCAB, HIDDEN, std=0.02)
    suppress = inp.rng.random(VOCAB) < 0.01
    tw, tsup = inp.dev(w), inp.dev(suppress)
    w32 = w.astype(np.float32)

    # the reference op pair: LM head argmax into `best`, then finalize. The kernel's contract is the
    # argmax of fp16-rounded logits (lowest index on ties), so the reference logits are rounded too and
    # a correct pick has gap 0.
    y = inp.draw(HIDDEN)
    logits = (w32 @ y.astype(np.float32)).astype(np.float16).astype(np.float64)
    logits = np.where(suppress, -np.inf, logits)
    best, tokens, state, cur = _finalize_state()
    ext.lm_head_argmax(inp.dev(y[None]), tw, tsup, best)
    ext.argmax_finalize(best, tokens, state, cur, MAX_POS)
    tok = int(tokens[0])
    kept = int(cur) == tok and state.tolist() == [4, 1] and int(best) == 0
    gap = float(logits.max() - logits[tok]) if kept and 0 <= tok < VOCAB else math.inf
    yield 'lm_head_argmax', gap, TOL_ARGMAX_GAP

    # final residual + LN + LM head + finalize in one launch == add_layernorm, lm_head_argmax, finalize
    h, x = inp.dev(inp.draw(1, HIDDEN)), inp.dev(inp.draw(1, HIDDEN))
    ones = torch.ones(HIDDEN, dtype=torch.float16, device='cuda')
    zeros = torch.zeros(HIDDEN, dtype=torch.float16, device='cuda')
    results = {}
    h_unfused, y_unfused = h.clone(), torch.empty_like(h)
    ext.add_layernorm(h_unfused, x, ones, zeros, y_unfused, EPS)
    st = _finalize_state()
    ext.lm_head_argmax(y_unfused, tw, tsup, st[0])
    ext.argmax_finalize(*st, MAX_POS)
    results['unfused'] = st
    st = _finalize_state()
    ext.lm_head_argmax_fused(h, x, ones, zeros, EPS, tw, tsup, *st, MAX_POS)
    results['fused'] = st
    wq, meta = ext.lm_head_q8_table(tw)
    st = _finalize_state()
    ext.lm_head_argmax_q8(h, x, ones, zeros, EPS, tw, wq, meta, tsup, *st, MAX_POS)
    results['q8'] = st

    def same(a, b):  # token list, state and current token identical; both `best` words reset
        return (torch.equal(a[1], b[1]) and torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])
                and int(a[0]) == 0 and int(b[0]) == 0)

    yield 'lm_head_argmax_fused_vs_unfused', 0.0 if same(results['fused'], results['unfused']) else 1.0, EXACT
    yield 'lm_head_argmax_q8_vs_fused', 0.0 if same(results['q8'], results['fused']) else 1.0, EXACT


FAMILIES = (_layernorm_family, _self_attention_family, _cross_attention_family, _lm_head_family)


@torch.inference_mode()
def run_selftest(ext, seed=0):
    checks = []
    inp = _Inputs(seed)
    for family in FAMILIES:
        for name, err, tol in family(ext, inp):
            checks.append({'name': name, 'max_err': float(err), 'ok': bool(err <= tol)})
    torch.cuda.synchronize()
    return {'ok': all(c['ok'] for c in checks), 'checks': checks}


def main():
    from .ext import load_ext

    parser = argparse.ArgumentParser(description='run the kernel self-checks and write DIR/selftest.json')
    parser.add_argument('--out', type=Path, required=True)
    args = parser.parse_args()
    args.out.mkdir(parents=True, exist_ok=True)
    result = run_selftest(load_ext())
    (args.out / 'selftest.json').write_text(json.dumps(result, indent=2) + '\n')
    print(json.dumps(result))


if __name__ == '__main__':
    main()


__all__ = ['SPLIT_KEYS', 'workspace', 'run_selftest', 'main']

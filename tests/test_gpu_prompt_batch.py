"""Batched decoder launches for the prompt (several decoder positions per launch).

Every row of a batched GEMV / LN+GEMV / attention+out-projection must be bit-identical to the
single-position launch on that row, in the order the sequential prompt steps would run them (the
self attention of position v sees the fresh K/V rows of the positions before it in the same batch),
and the attention outputs also match the oracle within the decoder tolerance."""

import numpy as np
import pytest
import torch

from oracle import decoder as odec
from test_gpu_decode import close_rel, h16, np32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def ext(hip_device):
    from flash_whisper_amd.ext import load_ext

    return load_ext()


@pytest.mark.parametrize('n,k,act,nv', [(3840, 1280, 0, 4), (1280, 1280, 0, 2), (5120, 1280, 1, 3),
                                        (1280, 5120, 0, 4), (37, 1280, 0, 3), (51, 5120, 1, 2)])
def test_gemv_batch_rows_equal_single(ext, hip_device, n, k, act, nv):
    rng = np.random.default_rng(n + k + nv)
    dev = hip_device
    x = h16(rng.standard_normal((nv, k)), dev)
    w = h16(0.02 * rng.standard_normal((n, k)), dev)
    b = h16(0.02 * rng.standard_normal(n), dev)
    out = torch.empty(nv, n, dtype=torch.float16, device=dev)
    ext.gemv(x, w, b, out, act=act, nv=nv)
    for v in range(nv):
        one = torch.empty(n, dtype=torch.float16, device=dev)
        ext.gemv(x[v], w, b, one, act=act)
        assert torch.equal(out[v], one), v


@pytest.mark.parametrize('n,act,embed,nv', [(3840, 0, True, 4), (1280, 0, False, 4), (5120, 1, False, 3),
                                            (3840, 0, False, 2), (100, 0, False, 4)])
def test_ln_gemv_batch_rows_equal_single(ext, hip_device, n, act, embed, nv):
    rng = np.random.default_rng(n + nv + embed)
    dev = hip_device
    g, be = h16(1 + 0.1 * rng.standard_normal(1280), dev), h16(0.1 * rng.standard_normal(1280), dev)
    w = h16(0.02 * rng.standard_normal((n, 1280)), dev)
    bias = h16(0.02 * rng.standard_normal(n), dev)
    out = torch.empty(nv, n, dtype=torch.float16, device=dev)
    h_out = torch.empty(nv, 1280, dtype=torch.float16, device=dev)
    if embed:
        table = h16(0.02 * rng.standard_normal((300, 1280)), dev)
        pos = h16(0.02 * rng.standard_normal((40, 1280)), dev)
        cur = torch.tensor([7, 250, 123, 5][:nv], device=dev)
        state = torch.tensor([17, 0], device=dev)
        ext.ln_gemv(None, None, h_out, g, be, 1e-5, w, bias, out, act, embed=(cur, state, table, pos), nv=nv)
    else:
        h, x = h16(rng.standard_normal((nv, 1280)), dev), h16(rng.standard_normal((nv, 1280)), dev)
        ext.ln_gemv(h, x, h_out, g, be, 1e-5, w, bias, out, act, nv=nv)
    for v in range(nv):
        one, r_one = torch.empty(n, dtype=torch.float16, device=dev), torch.empty(1280, dtype=torch.float16, device=dev)
        if embed:
            st = torch.tensor([17 + v, 0], device=dev)
            ext.ln_gemv(None, None, r_one, g, be, 1e-5, w, bias, one, act, embed=(cur[v:v + 1], st, table, pos))
        else:
            ext.ln_gemv(h[v], x[v], r_one, g, be, 1e-5, w, bias, one, act)
        assert torch.equal(out[v], one) and torch.equal(h_out[v], r_one), v


@pytest.mark.parametrize('mode,pos0,nq,split', [('self', 0, 4, 64), ('self', 1, 2, 64), ('self', 61, 4, 64),
                                                ('self', 444, 4, 64), ('self', 200, 3, 128), ('cross', 0, 4, 256),
                                                ('cross', 0, 3, 192)])
def test_attention_batch_equals_sequential_steps(ext, hip_device, mode, pos0, nq, split):
    """Self mode: nq queries at positions pos0.. with their fresh K/V rows in a packed q/k/v batch, as in
    the prompt; the sequential reference runs attention_split + attn_out_gemv once per position (each
    writing its cache row before the next reads it). Cross mode: nq independent queries."""
    from flash_whisper_amd.selftest import workspace
    from oracle.common import f16

    dev, heads, dm = hip_device, 20, 1280
    rng = np.random.default_rng(pos0 + nq + split)
    max_len = 448 if mode == 'self' else 1500
    k = np.float16(rng.standard_normal((heads, max_len, 64)))
    v = np.float16(rng.standard_normal((heads, max_len, 64)))
    qkv = np.float16(rng.standard_normal((nq, 3 * dm)))
    w = np.float16(0.02 * rng.standard_normal((dm, dm)))
    b = np.float16(0.02 * rng.standard_normal(dm))
    tw, tb = h16(w, dev), h16(b, dev)
    ws = workspace(heads, nq * -(-max_len // split))
    tqkv = h16(qkv, dev)
    q, kn, vn = tqkv[:, :dm], tqkv[:, dm:2 * dm], tqkv[:, 2 * dm:]
    if mode == 'cross':
        q = h16(qkv[:, :dm], dev)
        kn = vn = None
    state = torch.tensor([pos0, 0], device=dev) if mode == 'self' else None
    tk, tv = h16(k, dev), h16(v, dev)
    out = torch.empty(nq, dm, dtype=torch.float16, device=dev)
    ext.attention_split_batch(q, tk, tv, state, kn, vn, *ws, 0.125, split_keys=split)
    ext.attn_out_gemv(*ws, state, heads, max_len, tw, tb, out, split_keys=split, nv=nq)

    sk, sv = h16(k, dev), h16(v, dev)
    k_ref, v_ref = k.copy(), v.copy()
    for z in range(nq):
        one = torch.empty(dm, dtype=torch.float16, device=dev)
        args = [None, None, None]
        length = max_len
        if mode == 'self':
            p = pos0 + z
            args = [torch.tensor([p, 0], device=dev), kn[z].contiguous(), vn[z].contiguous()]
            k_ref[:, p] = qkv[z, dm:2 * dm].reshape(heads, 64)
            v_ref[:, p] = qkv[z, 2 * dm:].reshape(heads, 64)
            length = p + 1
        ext.attention_split(q[z].contiguous(), sk, sv, *args, *ws, 0.125, split_keys=split)
        ext.attn_out_gemv(*ws, args[0], heads, max_len, tw, tb, one, split_keys=split)
        assert torch.equal(out[z], one), z
        att = odec.attention(qkv[z, :dm].reshape(heads, 64).astype(np.float32), k_ref, v_ref, length, 0.125)
        close_rel(np32(out[z]), f16(w.astype(np.float32) @ att + b.astype(np.float32)))
    assert torch.equal(tk, sk) and torch.equal(tv, sv)
    if mode == 'self':
        assert np.array_equal(tk.cpu().numpy(), k_ref) and np.array_equal(tv.cpu().numpy(), v_ref)


def test_batch_argument_checks(ext, hip_device):
    from flash_whisper_amd.selftest import workspace

    dev = hip_device
    w = torch.zeros(64, 1280, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match='nv'):
        ext.gemv(torch.zeros(5, 1280, dtype=torch.float16, device=dev), w, None,
                 torch.empty(5, 64, dtype=torch.float16, device=dev), nv=5)
    with pytest.raises(RuntimeError, match='shape'):
        ext.gemv(torch.zeros(2, 1280, dtype=torch.float16, device=dev), w, None,
                 torch.empty(64, dtype=torch.float16, device=dev), nv=2)
    k = torch.zeros(20, 64, 64, dtype=torch.float16, device=dev)
    q = torch.zeros(4, 1280, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match='workspace'):
        ext.attention_split_batch(q, k, k.clone(), None, None, None, *workspace(20, 1), 0.125)
    with pytest.raises(RuntimeError, match='view'):
        ext.attention_split_batch(q[:, 1:1281 - 8], k, k.clone(), None, None, None, *workspace(20, 8), 0.125)

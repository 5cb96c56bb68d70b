"""GPU parity of the decoder kernels against the CPU oracle (configs 2-4 of the synthetic workload).

Tolerances: "2e-3 relative in fp16" for attention and layer outputs is applied elementwise as
|gpu - ref| <= 2e-3 * |ref| + 2e-3 * rms(ref) (the rms term keeps near-zero elements meaningful);
the KV-cache write and the greedy token are bit-exact; the LM-head token must equal the oracle's
fp16-logit argmax exactly."""

import numpy as np
import pytest
import torch

from oracle import decoder as odec

pytestmark = pytest.mark.gpu
RTOL = 2e-3


def close_rel(gpu, ref, rtol=RTOL, scale=None):
    """|gpu - ref| <= rtol * scale + rtol * rms(ref), scale = |ref| unless given. When the result is a
    sum of rounded terms (a residual add), pass scale = |a| + |b|: a one-ulp difference in a large
    intermediate that cancels must be measured against the intermediate, not the small result."""
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref) if scale is None else np.asarray(scale, np.float64)
    tol = rtol * scale + rtol * np.sqrt(np.mean(ref ** 2))
    err = np.abs(gpu - ref)
    assert (err <= tol).all(), f'max err {err.max():.3e}, worst ratio {(err / tol).max():.2f}'


def h16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16)).to(dev)


def np32(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope='module')
def ext(hip_device):
    from flash_whisper_amd.ext import load_ext

    return load_ext()


def test_synth_device_matches_host(ext, hip_device):
    from flash_whisper_amd import weights

    for name, n in (('model.decoder.layers.0.fc1.weight', 5120 * 1280), ('tiny', 3), ('odd', 100001)):
        t = torch.empty(n, dtype=torch.float16, device=hip_device)
        weights.device_fill(t, name, 'normal', seed=0)
        host = weights.host_normal(name, (n,), seed=0)
        assert np.array_equal(t.cpu().numpy().view(np.uint16), host.view(np.uint16)), name


@pytest.mark.parametrize('with_x', [True, False])
def test_add_layernorm(ext, hip_device, with_x):
    rng = np.random.default_rng(10)
    h, x = rng.standard_normal(1280), rng.standard_normal(1280)
    g, b = 1 + 0.1 * rng.standard_normal(1280), 0.1 * rng.standard_normal(1280)
    h16_, x16, g16, b16 = (np.float16(a) for a in (h, x, g, b))
    th, tx, tg, tb = (h16(a, hip_device) for a in (h16_, x16, g16, b16))
    ty = torch.empty_like(th)
    ext.add_layernorm(th, tx if with_x else None, tg, tb, ty, 1e-5)
    r_ref, y_ref = odec.add_layernorm(h16_, x16 if with_x else None, g16, b16, 1e-5)
    assert np.array_equal(np32(th), r_ref)  # fp16 residual is exact
    close_rel(np32(ty), y_ref)


@pytest.mark.parametrize('n,k,act', [(3840, 1280, 0), (1280, 1280, 0), (5120, 1280, 1), (1280, 5120, 0),
                                     (37, 1280, 0), (51, 5120, 1)])
def test_gemv(ext, hip_device, n, k, act):
    rng = np.random.default_rng(n + k + act)
    x = np.float16(rng.standard_normal(k))
    w = np.float16(0.02 * rng.standard_normal((n, k)))
    b = np.float16(0.02 * rng.standard_normal(n))
    out = torch.empty(n, dtype=torch.float16, device=hip_device)
    ext.gemv(h16(x, hip_device), h16(w, hip_device), h16(b, hip_device), out, act=act)
    from oracle.common import f16, gelu

    ref = f16(w.astype(np.float32) @ x.astype(np.float32) + b.astype(np.float32))
    if act:
        ref = f16(gelu(ref))
    close_rel(np32(out), ref)


@pytest.mark.parametrize('n,act,embed', [(3840, 0, False), (1280, 0, False), (5120, 1, False), (3840, 0, True)])
def test_ln_gemv(ext, hip_device, n, act, embed):
    from oracle.common import f16, gelu

    rng = np.random.default_rng(n + act)
    dev = hip_device
    g, b = np.float16(1 + 0.1 * rng.standard_normal(1280)), np.float16(0.1 * rng.standard_normal(1280))
    w = np.float16(0.02 * rng.standard_normal((n, 1280)))
    bias = np.float16(0.02 * rng.standard_normal(n))
    out = torch.empty(n, dtype=torch.float16, device=dev)
    h_out = torch.empty(1280, dtype=torch.float16, device=dev)
    if embed:
        table = np.float16(0.02 * rng.standard_normal((300, 1280)))
        pos = np.float16(0.02 * rng.standard_normal((40, 1280)))
        cur = torch.tensor([123], device=dev)
        state = torch.tensor([17, 0], device=dev)
        ext.ln_gemv(None, None, h_out, h16(g, dev), h16(b, dev), 1e-5, h16(w, dev), h16(bias, dev), out, act,
                    embed=(cur, state, h16(table, dev), h16(pos, dev)))
        r_ref, y_ref = odec.add_layernorm(table[123], pos[17], g, b, 1e-5)
    else:
        h, x = np.float16(rng.standard_normal(1280)), np.float16(rng.standard_normal(1280))
        ext.ln_gemv(h16(h, dev), h16(x, dev), h_out, h16(g, dev), h16(b, dev), 1e-5, h16(w, dev), h16(bias, dev),
                    out, act)
        r_ref, y_ref = odec.add_layernorm(h, x, g, b, 1e-5)
    assert np.array_equal(np32(h_out), r_ref)
    ref = f16(w.astype(np.float32) @ y_ref + bias.astype(np.float32))
    if act:
        ref = f16(gelu(ref))
    # the GEMV input is the kernel's own fp16 LN output, which may differ from the oracle's by one
    # ulp in a few elements; the comparison absorbs that through the relative tolerance
    close_rel(np32(out), ref)


def _attn_inputs(rng, heads, max_len):
    q = np.float16(rng.standard_normal(heads * 64))
    k = np.float16(rng.standard_normal((heads, max_len, 64)))
    v = np.float16(rng.standard_normal((heads, max_len, 64)))
    return q, k, v


@pytest.mark.parametrize('length', [1, 63, 64, 65, 200, 224, 448])
@pytest.mark.parametrize('fused', [False, True])
def test_self_attention(ext, hip_device, length, fused):
    from flash_whisper_amd.selftest import workspace

    rng = np.random.default_rng(length)
    dev, heads, max_len, pos = hip_device, 20, 448, length - 1
    q, k, v = _attn_inputs(rng, heads, max_len)
    k_new, v_new = np.float16(rng.standard_normal((heads, 64))), np.float16(rng.standard_normal((heads, 64)))
    tk, tv = h16(k, dev), h16(v, dev)
    out = torch.empty(heads * 64, dtype=torch.float16, device=dev)
    state = torch.tensor([pos, 0], device=dev)
    ws = workspace(heads, 7)
    if fused:
        ext.decode_attention_fused(h16(q, dev), tk, tv, out, state, h16(k_new, dev), h16(v_new, dev), 0.125)
    else:
        ext.decode_attention(h16(q, dev), tk, tv, out, state, h16(k_new, dev), h16(v_new, dev), *ws, 0.125)
    k_ref, v_ref = k.copy(), v.copy()
    k_ref[:, pos], v_ref[:, pos] = k_new, v_new
    ref = odec.attention(q.reshape(heads, 64).astype(np.float32), k_ref, v_ref, length, 0.125)
    close_rel(np32(out), ref)
    assert np.array_equal(tk.cpu().numpy(), k_ref) and np.array_equal(tv.cpu().numpy(), v_ref)


@pytest.mark.parametrize('max_len,fused', [(1500, True), (1500, False), (1537, True), (3100, True), (7, True)])
def test_cross_attention(ext, hip_device, max_len, fused):
    """Cross mode over the 1500 encoder frames, plus lengths that take a partial and several 1536-key
    rounds in the single-launch kernel."""
    from flash_whisper_amd.selftest import workspace

    rng = np.random.default_rng(max_len)
    dev, heads = hip_device, 20
    q, k, v = _attn_inputs(rng, heads, max_len)
    q = np.float16(q.astype(np.float32) * 2)  # sharper softmax than the N(0, 1) default
    out = torch.empty(heads * 64, dtype=torch.float16, device=dev)
    if fused:
        ext.decode_attention_fused(h16(q, dev), h16(k, dev), h16(v, dev), out, None, None, None, 0.125)
    else:
        ext.decode_attention(h16(q, dev), h16(k, dev), h16(v, dev), out, None, None, None,
                             *workspace(heads, -(-max_len // 64)), 0.125)
    ref = odec.attention(q.reshape(heads, 64).astype(np.float32), k, v, max_len, 0.125)
    close_rel(np32(out), ref)


def _lm_setup(dev, seed=4):
    from flash_whisper_amd import weights

    rng = np.random.default_rng(seed)
    h = np.float16(rng.standard_normal(1280))
    w = torch.empty(51866, 1280, dtype=torch.float16, device=dev)
    weights.device_fill(w, 'model.decoder.embed_tokens.weight', 'normal', seed=0)
    return h, w


@pytest.mark.parametrize('fused', [False, True])
def test_lm_head_argmax_bit_exact(ext, hip_device, fused):
    from flash_whisper_amd import weights

    dev = hip_device
    h, w = _lm_setup(dev)
    w_np = weights.host_normal('model.decoder.embed_tokens.weight', (51866, 1280), seed=0)
    sup = np.zeros(51866, bool)
    sup[[1, 2, 7, 50257, 50258]] = True
    g1, b0 = np.ones(1280, np.float16), np.zeros(1280, np.float16)
    _, y_ref = odec.add_layernorm(h, None, g1, b0, 1e-5)
    logits = odec.lm_head_logits(y_ref, w_np)
    tok_ref = odec.masked_argmax(logits, sup)
    best = torch.zeros(1, dtype=torch.long, device=dev)
    tokens = torch.zeros(448, dtype=torch.long, device=dev)
    state = torch.tensor([3, 0], device=dev)
    cur = torch.zeros(1, dtype=torch.long, device=dev)
    tsup = torch.from_numpy(sup).to(dev)
    if fused:  # three steps in a row: each finalizes and leaves best zero for the next
        for i in range(3):
            ext.lm_head_argmax_fused(h16(h, dev), None, h16(g1, dev), h16(b0, dev), 1e-5, w, tsup, best, tokens,
                                     state, cur, 448)
            assert tokens[:i + 1].tolist() == [tok_ref] * (i + 1) and state.tolist() == [4 + i, 1 + i]
        state[:] = torch.tensor([4, 1])
    else:
        y = torch.empty(1280, dtype=torch.float16, device=dev)
        th = h16(h, dev)
        ext.add_layernorm(th, None, h16(g1, dev), h16(b0, dev), y, 1e-5)
        ext.lm_head_argmax(y, w, tsup, best)
        ext.argmax_finalize(best, tokens, state, cur, 448)
    assert int(tokens[0]) == tok_ref
    assert int(cur) == tok_ref and state.tolist() == [4, 1] and not best.any()


def test_lm_head_ties_and_suppression(ext, hip_device):
    """Identical rows tie exactly: the lowest index wins; suppressing it hands the win to the next."""
    dev = hip_device
    rng = np.random.default_rng(5)
    vocab = 4099
    w = np.float16(0.02 * rng.standard_normal((vocab, 1280)))
    y = np.float16(rng.standard_normal(1280))
    w[[100, 2000, 4098]] = np.float16(0.05 * np.sign(y))  # clear winners, identical rows
    tw, ty = h16(w, dev), h16(y, dev)
    for sup_idx, expect in (([], 100), ([100], 2000), ([100, 2000], 4098)):
        sup = torch.zeros(vocab, dtype=torch.bool, device=dev)
        if sup_idx:
            sup[sup_idx] = True
        best = torch.zeros(1, dtype=torch.long, device=dev)
        ext.lm_head_argmax(ty, tw, sup, best)
        tokens, state, cur = (torch.zeros(4, dtype=torch.long, device=dev), torch.tensor([0, 0], device=dev),
                              torch.zeros(1, dtype=torch.long, device=dev))
        ext.argmax_finalize(best, tokens, state, cur, 448)
        assert int(tokens[0]) == expect


def test_finalize_saturation(ext, hip_device):
    dev = hip_device
    best = torch.tensor([0], dtype=torch.long, device=dev)
    # pack (logit 1.0, idx 9): u = bits(1.0) | sign; low word = 0xFFFFFFFF - 9
    packed = ((0x3F800000 | 0x80000000) << 32) | (0xFFFFFFFF - 9)
    best.fill_(packed - (1 << 64) if packed >= (1 << 63) else packed)
    tokens = torch.zeros(4, dtype=torch.long, device=dev)
    state = torch.tensor([3, 4], device=dev)
    cur = torch.zeros(1, dtype=torch.long, device=dev)
    ext.argmax_finalize(best, tokens, state, cur, 4)
    assert state.tolist() == [3, 4] and tokens.tolist() == [0, 0, 0, 0] and int(cur) == 9 and int(best) == 0


def test_selftest_passes(ext, hip_device):
    from flash_whisper_amd.selftest import run_selftest

    res = run_selftest(ext)
    bad = [c for c in res['checks'] if not c['ok']]
    assert res['ok'], bad


@pytest.mark.parametrize('mode,length,split', [('self', 1, 64), ('self', 65, 64), ('self', 228, 64),
                                               ('self', 448, 64), ('cross', 1500, 256), ('cross', 1500, 192),
                                               ('self', 300, 128), ('self', 448, 256)])
def test_split_attention_with_fused_combine_gemv(ext, hip_device, mode, length, split):
    """attention_split + attn_out_gemv (combine in the GEMV prologue) must equal the reference-granularity
    decode_attention (split + combine launches) followed by the GEMV, bit for bit at 64-key splits, and
    match the oracle (attention, then the fp16 projection) within tolerance at any split size."""
    from flash_whisper_amd.selftest import workspace
    from oracle.common import f16

    dev, heads = hip_device, 20
    rng = np.random.default_rng(length + split)
    max_len = 448 if mode == 'self' else 1500
    q, k, v = _attn_inputs(rng, heads, max_len)
    w = np.float16(0.02 * rng.standard_normal((1280, 1280)))
    b = np.float16(0.02 * rng.standard_normal(1280))
    ws = workspace(heads, -(-max_len // min(split, 64)))
    args = [None, None, None]
    k_ref, v_ref = k.copy(), v.copy()
    if mode == 'self':
        kn, vn = np.float16(rng.standard_normal((heads, 64))), np.float16(rng.standard_normal((heads, 64)))
        args = [torch.tensor([length - 1, 0], device=dev), h16(kn, dev), h16(vn, dev)]
        k_ref[:, length - 1], v_ref[:, length - 1] = kn, vn
    tk, tv = h16(k, dev), h16(v, dev)
    out = torch.empty(1280, dtype=torch.float16, device=dev)
    ext.attention_split(h16(q, dev), tk, tv, *args, *ws, 0.125, split_keys=split)
    ext.attn_out_gemv(*ws, args[0], heads, max_len, h16(w, dev), h16(b, dev), out, split_keys=split)
    att = odec.attention(q.reshape(heads, 64).astype(np.float32), k_ref, v_ref, length, 0.125)
    close_rel(np32(out), f16(w.astype(np.float32) @ att + b.astype(np.float32)))
    if mode == 'self':
        assert np.array_equal(tk.cpu().numpy(), k_ref) and np.array_equal(tv.cpu().numpy(), v_ref)
    if split == 64 and mode == 'self':
        tk2, tv2 = h16(k, dev), h16(v, dev)
        attn, ref_out = torch.empty(1280, dtype=torch.float16, device=dev), torch.empty_like(out)
        ext.decode_attention(h16(q, dev), tk2, tv2, attn, *args, *ws, 0.125)
        ext.gemv(attn, h16(w, dev), h16(b, dev), ref_out)
        assert torch.equal(out, ref_out)

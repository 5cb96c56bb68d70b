"""GPU parity of the encoder kernels (MFMA GEMM + epilogues, implicit-GEMM conv stem, row LayerNorm,
q/k/v projection with transposed V, flash encoder attention, cross K/V scatter) against the CPU oracle. Tolerance as in
test_gpu_decode.close_rel: 2e-3 relative in fp16, elementwise with an rms floor."""

import numpy as np
import pytest
import torch

from oracle import encoder as oenc
from oracle.common import f16, gelu
from oracle.decoder import layer_norm
from test_gpu_decode import close_rel, h16, np32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def ext(hip_device):
    from flash_whisper_amd.ext import load_ext

    return load_ext()


def _gemm_ref(a, w, b, epi, res=None, q_cols=0):
    """Reference output and the magnitude scale for the relative tolerance (|res| + |term| for adds)."""
    acc = a.astype(np.float32) @ w.astype(np.float32).T
    v = f16(acc + (0 if b is None else b.astype(np.float32)))
    scale = None
    if epi == 1:
        v = f16(gelu(v))
    elif epi in (2, 3):
        scale = np.abs(res.astype(np.float32)) + np.abs(v)
        v = f16(res.astype(np.float32) + v)
        if epi == 3:  # the clamp bound 65504 - 1000 rounds to 64512 in fp16
            v = f16(np.clip(v, -64504, 64504))
    elif epi == 4:
        g = f16(gelu(v))
        scale = np.abs(g) + np.abs(res.astype(np.float32))
        v = f16(g + res.astype(np.float32))
    elif epi == 5:
        v = v.copy()
        v[:, :q_cols] = f16(v[:, :q_cols] * 0.125)
    return v, scale


# shapes cover the 256-, 192-, 128- and 64-row tile paths, a single k stage and partial last tiles
# (192-row tiles: 1500 x 3840 and 1200 x 4096)
@pytest.mark.parametrize('m,n,k,epi', [(1500, 3840, 1280, 5), (1500, 1280, 1280, 2), (1500, 5120, 1280, 1),
                                       (1500, 1280, 5120, 3), (1500, 1280, 1280, 0), (77, 128, 64, 0),
                                       (1500, 1280, 1280, 4), (300, 8192, 64, 0), (513, 16384, 192, 1),
                                       (1100, 2560, 128, 0), (1200, 4096, 128, 1)])
def test_gemm_epilogues(ext, hip_device, m, n, k, epi):
    dev = hip_device
    rng = np.random.default_rng(m + n + k + epi)
    a = np.float16(rng.standard_normal((m, k)))
    w = np.float16(0.02 * rng.standard_normal((n, k)))
    b = np.float16(0.02 * rng.standard_normal(n))
    res = np.float16(rng.standard_normal((m, n))) if epi in (2, 3, 4) else None
    out = torch.empty(m, n, dtype=torch.float16, device=dev)
    tres = h16(res, dev) if res is not None else None
    if epi in (2, 3):
        out = tres  # residual updated in place, as the encoder does
    ext.gemm(h16(a, dev), h16(w, dev), h16(b, dev), out, epi, res=tres, q_cols=n // 3 if epi == 5 else 0)
    ref, scale = _gemm_ref(a, w, b, epi, res, n // 3 if epi == 5 else 0)
    close_rel(np32(out), ref, scale=scale)


def _f16_order(v):
    """fp16 values -> integers in value order (adjacent fp16 numbers differ by 1)."""
    bits = np.asarray(v, np.float16).view(np.int16).astype(np.int32)
    return np.where(bits < 0, -(bits & 0x7FFF), bits)


def test_gelu_epilogue_within_one_ulp(ext, hip_device):
    """The GELU epilogue (erfc by a fitted exponent polynomial) against an exact GELU, 0.5 x erfc(-x / sqrt 2) in
    float64, on 16384 fp16 inputs spanning both tails, passed through the GEMM unchanged (identity
    weights): every output within one fp16 ulp, and nearly all of them equal."""
    from scipy.special import erfc

    dev = hip_device
    rng = np.random.default_rng(11)
    x = np.concatenate([np.linspace(-12, 12, 8192), rng.standard_normal(4096) * 3,
                        np.float16(rng.standard_normal(4096)) * 1e-3]).astype(np.float16)
    a = x.reshape(128, 128)
    out = torch.empty(128, 128, dtype=torch.float16, device=dev)
    ext.gemm(h16(a, dev), h16(np.eye(128), dev), None, out, 1)
    x64 = x.astype(np.float64)
    ref = np.float16(0.5 * x64 * erfc(-x64 / np.sqrt(2.0)))
    got = np.float16(np32(out).reshape(-1))
    d = np.abs(_f16_order(got) - _f16_order(ref))
    assert d.max() <= 1, (x[d.argmax()], got[d.argmax()], ref[d.argmax()])
    assert (d == 0).mean() > 0.995


@pytest.mark.parametrize('big', [False, True])
@pytest.mark.parametrize('epi', [2, 3])  # FW_EPI_BIAS_RESID, FW_EPI_BIAS_RESID_CLAMP
def test_splitk_residual_layernorm_matches_fused_path(ext, hip_device, epi, big):
    """fc2 as two k halves (fw_gemm_splitk) finished by fw_layernorm_rows_residual: the partial sums add
    up to the fp32 product, and the updated residual and its LayerNorm match the one-pass GEMM with
    the same residual epilogue followed by fw_layernorm_rows (within the fp16 tolerance: only the fp32
    summation order differs), on the encoder's fc2 shape (1500 rows: a partial last 128-row tile).
    With `big`, 8 columns of 100 rows carry a residual of +-64992, so residual + fc2 passes the
    fp16 clamp bound: the clamping epilogue must store +-64512 there (the bound 65504 - 1000 in fp16,
    as transformers' clamp of a half tensor gives) and normalise the stored values."""
    dev = hip_device
    rng = np.random.default_rng(epi + 10 * big)
    m, n, k = 1500, 1280, 5120
    a = np.float16(0.5 * rng.standard_normal((m, k)))
    w = np.float16(0.02 * rng.standard_normal((n, k)))
    b = np.float16(0.02 * rng.standard_normal(n))
    res = np.float16(rng.standard_normal((m, n)))
    rows, cols = np.arange(100) * 15, np.arange(8) * 160
    if big:
        res[np.ix_(rows, cols)] = np.float16(64992.0) * np.where(np.arange(8) % 2, -1, 1)
    g, be = h16(1 + 0.1 * rng.standard_normal(n), dev), h16(0.1 * rng.standard_normal(n), dev)
    ta, tw, tb = h16(a, dev), h16(w, dev), h16(b, dev)
    part = torch.full((2, m, n), float('nan'), dtype=torch.float32, device=dev)
    ext.gemm_splitk(ta, tw, part)
    prod = a.astype(np.float64) @ w.astype(np.float64).T
    close_rel(np32(part[0] + part[1]), prod, rtol=1e-4)
    h_ref = h16(res, dev)
    ext.gemm(ta, tw, tb, h_ref, epi, res=h_ref)
    y_ref = torch.empty_like(h_ref)
    ext.layernorm_rows(h_ref, g, be, y_ref, 1e-5)
    h = h16(res, dev)
    y = torch.full_like(h, float('nan'))
    ext.layernorm_rows_residual(part, tb, h, g, be, y, 1e-5, epi)
    close_rel(np32(h), np32(h_ref), scale=np.abs(res.astype(np.float32)) + np.abs(prod))
    close_rel(np32(y), np32(y_ref))
    # the LayerNorm of the updated residual is exactly fw_layernorm_rows of it
    y2 = torch.empty_like(h)
    ext.layernorm_rows(h, g, be, y2, 1e-5)
    assert torch.equal(y, y2)
    if big:
        sign = np.where(np.arange(8) % 2, -1.0, 1.0)
        got, one_pass = np32(h)[np.ix_(rows, cols)], np32(h_ref)[np.ix_(rows, cols)]
        if epi == 3:
            expect = oenc.residual_op(res[np.ix_(rows, cols)], f16(prod[np.ix_(rows, cols)] + b[cols]), clamp=True)
            assert np.all(expect == 64512.0 * sign)
            assert np.array_equal(got, expect) and np.array_equal(one_pass, expect)
        else:
            assert np.all(np.abs(got) > 64512.0) and np.all(np.abs(one_pass) > 64512.0)


def test_gemm_row_strided_views(ext, hip_device):
    """a, out given as column slices of wider matrices (leading dimension > k / n)."""
    dev = hip_device
    rng = np.random.default_rng(7)
    big_a = np.float16(rng.standard_normal((300, 3 * 256)))
    w = np.float16(0.02 * rng.standard_normal((128, 256)))
    ta = h16(big_a, dev)
    out_big = torch.zeros(300, 384, dtype=torch.float16, device=dev)
    ext.gemm(ta[:, 256:512], h16(w, dev), None, out_big[:, 128:256], 0)
    close_rel(np32(out_big[:, 128:256]), _gemm_ref(big_a[:, 256:512], w, None, 0)[0])
    assert float(out_big[:, :128].abs().max()) == 0 and float(out_big[:, 256:].abs().max()) == 0


@pytest.mark.parametrize('stride,c_in,t_in', [(1, 128, 3000), (2, 1280, 3000), (2, 128, 61)])
def test_conv1d(ext, hip_device, stride, c_in, t_in):
    dev = hip_device
    rng = np.random.default_rng(stride + c_in)
    x = np.float16(rng.standard_normal((t_in, c_in)))     # time-major
    w = np.float16(0.02 * rng.standard_normal((1280, c_in, 3)))
    b = np.float16(0.02 * rng.standard_normal(1280))
    wp = np.ascontiguousarray(w.transpose(0, 2, 1).reshape(1280, 3 * c_in))
    t_out = (t_in - 1) // stride + 1
    pos = np.float16(rng.standard_normal((t_out, 1280)))
    out = torch.empty(t_out, 1280, dtype=torch.float16, device=dev)
    epi = 4 if stride == 2 else 1
    ext.conv1d(h16(x, dev), stride, h16(wp, dev), h16(b, dev), out, epi, res=h16(pos, dev) if epi == 4 else None)
    ref = f16(gelu(f16(oenc.conv1d(x.T.astype(np.float32), w, b, stride)))).T
    scale = None
    if epi == 4:
        scale = np.abs(ref) + np.abs(pos.astype(np.float32))
        ref = f16(ref + pos.astype(np.float32))
    close_rel(np32(out), ref, scale=scale)


def test_layernorm_rows(ext, hip_device):
    dev = hip_device
    rng = np.random.default_rng(8)
    x = np.float16(3 * rng.standard_normal((1501, 1280)) + 0.5)
    g, b = np.float16(1 + 0.1 * rng.standard_normal(1280)), np.float16(0.1 * rng.standard_normal(1280))
    y = torch.empty(1501, 1280, dtype=torch.float16, device=dev)
    ext.layernorm_rows(h16(x, dev), h16(g, dev), h16(b, dev), y, 1e-5)
    close_rel(np32(y), f16(layer_norm(x, g, b, 1e-5)))


def _attn_ref(qkv, heads):
    seq = qkv.shape[0]
    d = heads * 64
    q = qkv[:, :d].astype(np.float64).reshape(seq, heads, 64).transpose(1, 0, 2)
    k = qkv[:, d:2 * d].astype(np.float64).reshape(seq, heads, 64).transpose(1, 0, 2)
    v = qkv[:, 2 * d:].astype(np.float64).reshape(seq, heads, 64).transpose(1, 0, 2)
    s = q @ k.transpose(0, 2, 1)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return f16((p @ v).transpose(1, 0, 2).reshape(seq, d))


@pytest.mark.parametrize('seq,heads,qscale', [(1500, 20, 0.125), (100, 2, 0.125), (1500, 20, 0.6), (33, 1, 0.3),
                                               (1496, 3, 0.2), (1, 2, 0.125), (64, 1, 0.5), (129, 2, 0.125)])
def test_encoder_attention(ext, hip_device, seq, heads, qscale):
    dev = hip_device
    rng = np.random.default_rng(seq + heads)
    qkv = rng.standard_normal((seq, 3 * heads * 64))
    qkv[:, :heads * 64] *= qscale  # q arrives pre-scaled; a larger scale sharpens the softmax
    qkv = np.float16(qkv)
    out = torch.empty(seq, heads * 64, dtype=torch.float16, device=dev)
    tq = h16(qkv, dev)
    vt = ext.encoder_vt_workspace(seq, heads)
    vt.fill_(float('nan'))  # every element, padding included, must be rewritten
    ext.encoder_pack_vt(tq, vt, heads)
    assert not torch.isnan(vt).any()
    ext.encoder_attention(tq, vt, out, heads)
    close_rel(np32(out), _attn_ref(qkv, heads))


@pytest.mark.parametrize('m', [1500, 77, 1])
def test_encoder_qkv_matches_gemm_and_pack(ext, hip_device, m):
    """The fused q/k/v projection writes the FW_EPI_SCALE_Q GEMM's q and k columns and, for v, exactly
    what fw_encoder_pack_vt makes of that GEMM's v columns (padding keys zero)."""
    dev = hip_device
    rng = np.random.default_rng(m)
    y = h16(np.float16(rng.standard_normal((m, 1280))), dev)
    w = h16(np.float16(0.02 * rng.standard_normal((3840, 1280))), dev)
    b = h16(np.float16(0.02 * rng.standard_normal(3840)), dev)
    ref = torch.empty(m, 3840, dtype=torch.float16, device=dev)
    ext.gemm(y, w, b, ref, 5, q_cols=1280)
    vt_ref = ext.encoder_vt_workspace(m, 20)
    ext.encoder_pack_vt(ref, vt_ref, 20)
    qkv = torch.full((m, 3840), 7.0, dtype=torch.float16, device=dev)
    vt = torch.full_like(vt_ref, float('nan'))
    ext.encoder_qkv(y, w, b, qkv, vt, 20)
    assert torch.equal(qkv[:, :2560], ref[:, :2560])
    assert torch.equal(qkv[:, 2560:], torch.full_like(qkv[:, 2560:], 7.0))  # v columns untouched
    assert torch.equal(vt, vt_ref)


def test_cross_kv_layout(ext, hip_device):
    from flash_whisper_amd.config import TURBO

    dev = hip_device
    rng = np.random.default_rng(9)
    enc = np.float16(rng.standard_normal((1500, 1280)))
    params = {}
    for i in range(4):
        a = f'model.decoder.layers.{i}.encoder_attn'
        params[f'{a}.k_proj.weight'] = np.float16(0.02 * rng.standard_normal((1280, 1280)))
        params[f'{a}.v_proj.weight'] = np.float16(0.02 * rng.standard_normal((1280, 1280)))
        params[f'{a}.v_proj.bias'] = np.float16(0.02 * rng.standard_normal(1280))
    w = np.concatenate([np.concatenate([params[f'model.decoder.layers.{i}.encoder_attn.k_proj.weight'],
                                        params[f'model.decoder.layers.{i}.encoder_attn.v_proj.weight']])
                        for i in range(4)])
    b = np.concatenate([np.concatenate([np.zeros(1280, np.float16),
                                        params[f'model.decoder.layers.{i}.encoder_attn.v_proj.bias']])
                        for i in range(4)])
    ckv = torch.empty(4, 2, 20, 1500, 64, dtype=torch.float16, device=dev)
    ext.cross_kv(h16(enc, dev), h16(w, dev), h16(b, dev), ckv)
    close_rel(np32(ckv), oenc.cross_kv(params, enc.astype(np.float32), TURBO))


@torch.inference_mode()
def test_encoder_layer_and_stem_vs_oracle(ext, hip_device):
    """Stem and encoder layer 0 of the seeded turbo weights, GPU vs oracle from the same input."""
    from flash_whisper_amd.config import TURBO
    from flash_whisper_amd.model import CustomModel

    model = CustomModel(selftest=False, capture=False, dims=TURBO)
    from flash_whisper_amd import weights

    names = [n for n, _, _ in weights.param_specs(TURBO)
             if n.startswith('model.encoder.layers.0.') or not n.startswith('model.encoder.layers.')]
    names = [n for n in names if n.startswith('model.encoder.')]
    params = weights.host_params(TURBO, 0, names)
    rng = np.random.default_rng(11)
    mel = np.float16(rng.standard_normal((128, 3000)) * 0.5)
    model.mel16.copy_(torch.from_numpy(np.ascontiguousarray(mel.T)))
    ext.conv1d(model.mel16, 1, model.conv1_wp, model.conv1_b, model.x1, 1)
    ext.conv1d(model.x1, 2, model.conv2_wp, model.conv2_b, model.ex, 4, res=model.enc_pos)
    stem = oenc.embed_stem(params, mel.astype(np.float32))
    close_rel(np32(model.ex), stem, scale=np.abs(stem) + np.abs(params['model.encoder.embed_positions.weight']))
    # layer 0 from the oracle's stem output, so both sides start from the same fp16 input
    model.ex.copy_(torch.from_numpy(stem.astype(np.float16)))
    lay = model.enc_layers[0]
    ext.layernorm_rows(model.ex, lay.ln1[0], lay.ln1[1], model.ey, lay.ln1[2])
    ext.encoder_qkv(model.ey, lay.qkv_w, lay.qkv_b, model.eqkv, model.evt, 20)
    ext.encoder_attention(model.eqkv, model.evt, model.eattn, 20)
    ext.gemm(model.eattn, lay.out_w, lay.out_b, model.ex, 2, res=model.ex)
    ext.layernorm_rows(model.ex, lay.ln2[0], lay.ln2[1], model.ey, lay.ln2[2])
    ext.gemm(model.ey, lay.fc1_w, lay.fc1_b, model.effn, 1)
    ext.gemm(model.effn, lay.fc2_w, lay.fc2_b, model.ex, 3, res=model.ex)
    ref = oenc.encoder_layer(stem, oenc.layer_params(params, 0), 20, 1e-5)
    # the layer output is x + attn + mlp: measure against the residual's magnitude
    close_rel(np32(model.ex), ref, scale=np.abs(stem) + np.abs(ref))


@torch.inference_mode()
def test_encoder_product_sequence_vs_oracle(ext, hip_device):
    """The product's own encoder launch sequence (CustomModel._encode: the stem, fused q/k/v + V^T,
    flash attention, out projection, fc1, fc2 as two k halves finished by the clamping residual
    LayerNorm of the next layer, the final LayerNorm, cross K/V) on the seeded turbo weights, checked
    layer by layer: each checked layer's GPU output against the oracle's layer applied to the GPU's
    input of that layer (2e-3 relative, against the residual's magnitude), the final LayerNorm and
    the cross K/V likewise. Layers 0-2 cover the first residual LayerNorms, 16 and 30-31 the depth."""
    from flash_whisper_amd import weights
    from flash_whisper_amd.config import TURBO
    from flash_whisper_amd.model import CustomModel

    check = [0, 1, 2, 16, 30, 31]
    model = CustomModel(selftest=False, capture=False, dims=TURBO)
    names = [n for n, _, _ in weights.param_specs(TURBO)
             if any(n.startswith(f'model.encoder.layers.{i}.') for i in check)
             or n.startswith('model.encoder.layer_norm') or n.startswith('model.encoder.conv')
             or n.startswith('model.encoder.embed_positions')
             or (n.startswith('model.decoder.layers.3.encoder_attn.') and ('k_proj' in n or 'v_proj' in n))]
    params = weights.host_params(TURBO, 0, names)
    rng = np.random.default_rng(12)
    mel = np.float16(rng.standard_normal((128, 3000)) * 0.5)
    model.mel16.copy_(torch.from_numpy(np.ascontiguousarray(mel.T)))
    outs = {}
    model._encode(hook=lambda i, x: outs.__setitem__(i, x.clone()))
    torch.cuda.synchronize()
    assert sorted(outs) == list(range(-1, 32))
    stem = oenc.embed_stem(params, mel.astype(np.float32))
    close_rel(np32(outs[-1]), stem, scale=np.abs(stem) + np.abs(params['model.encoder.embed_positions.weight']))
    for i in check:
        x_in = np32(outs[i - 1])
        ref = oenc.encoder_layer(x_in, oenc.layer_params(params, i), 20, 1e-5)
        close_rel(np32(outs[i]), ref, scale=np.abs(x_in) + np.abs(ref))
    x_last = np32(outs[31])
    enc_ref = oenc.ln_op(x_last, (params['model.encoder.layer_norm.weight'].astype(np.float32),
                                  params['model.encoder.layer_norm.bias'].astype(np.float32)), 1e-5)
    close_rel(np32(model.enc_out), enc_ref)
    # the cross K/V of the last decoder layer from the GPU's own encoder output
    enc = np32(model.enc_out)
    pre = 'model.decoder.layers.3.encoder_attn'
    k = oenc.linear_op(enc, params[f'{pre}.k_proj.weight'])
    v = oenc.linear_op(enc, params[f'{pre}.v_proj.weight'], params[f'{pre}.v_proj.bias'])
    close_rel(np32(model.cross_kv[3, 0]).transpose(1, 0, 2).reshape(1500, 1280), k)
    close_rel(np32(model.cross_kv[3, 1]).transpose(1, 0, 2).reshape(1500, 1280), v)

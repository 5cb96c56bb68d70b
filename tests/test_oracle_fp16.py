"""Pins the oracle's fp16 encoder semantics and its greedy protocol against transformers fixtures
recorded by tests/golden/make_golden.py (hf16, greedy). CPU only.

hf_tiny16.npz holds a tiny WhisperEncoder run in fp16 with SDPA attention, and every op's output in
every layer. Each oracle op is fed transformers' own input for that op and must reproduce
transformers' output: bit for bit for GELU and the residual add + clamp; at least 99% bit for bit
(the rest one ulp, from the summation order) for the projections and LayerNorms; and within the 2e-3
relative parity tolerance for the attention core, where torch's flash-style kernel rounds the
probabilities to fp16 and the oracle does not. Planted mistakes (query scaled before its rounding,
no clamp, a clamp bound left unrounded, an unrounded LayerNorm, attention scaled twice, the tanh GELU)
must each fail a check.

hf_greedy.json / .npz hold a tiny fp32 model's decoder, its encoder output, and its greedy ids from a
transformers loop that follows custom/pytorch_model.py:53-79; oracle.decoder.greedy must give the
same ids, and the planted protocol mistakes (begin-suppress on every step, suppress on the first step
only, no EOS stop) must not.
"""

import json

import numpy as np
import pytest

from conftest import GOLDEN
from flash_whisper_amd import weights
from flash_whisper_amd.config import WhisperDims
from oracle import decoder as odec
from oracle import encoder as oenc
from oracle.common import f16


def _dims(cfg):
    return WhisperDims(n_mels=cfg['num_mel_bins'], d_model=cfg['d_model'], heads=cfg['encoder_attention_heads'],
                       ffn=cfg['encoder_ffn_dim'], enc_layers=cfg['encoder_layers'],
                       dec_layers=cfg['decoder_layers'], vocab=cfg['vocab_size'],
                       enc_len=cfg['max_source_positions'], max_pos=cfg['max_target_positions'])


def _load(name):
    z = np.load(GOLDEN / name)
    cfg = json.loads(str(z['config']))
    params = {k[len('param:'):]: z[k].astype(np.float32) for k in z.files if k.startswith('param:')}
    trace = {k[len('trace:'):]: z[k] for k in z.files if k.startswith('trace:')}
    return _dims(cfg), params, trace, z


@pytest.fixture(scope='module')
def tiny16():
    return _load('hf_tiny16.npz')


def _ulps(a, b):
    """Distance in fp16 ulps between two fp16-valued arrays."""
    ia = np.asarray(a, np.float16).view(np.int16).astype(np.int64)
    ib = np.asarray(b, np.float16).view(np.int16).astype(np.int64)
    ia = np.where(ia < 0, -32768 - ia, ia)  # sign-magnitude -> monotonic
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


def _close_rel(got, ref, tol=2e-3):
    ref = np.asarray(ref, np.float64)
    return bool(np.all(np.abs(got - ref) <= tol * np.abs(ref) + tol * np.sqrt(np.mean(ref ** 2))))


def _op_checks(dims, params, trace, layer):
    """{op: passed} for every op of one encoder layer, each fed transformers' own input."""
    p = oenc.layer_params(params, layer)
    t = lambda n: trace[f'{layer}.{n}']
    x_in = t('out.in')

    def exact(got, ref):
        return bool(np.array_equal(got, ref))

    def gemm_like(got, ref):  # fp32 summation order (torch's, the oracle's float64) may move <1% by one ulp
        u = _ulps(got, ref)
        return bool(np.all(f16(got) == got) and u.max() <= 1 and np.mean(u == 0) >= 0.99)

    eps = dims.ln_eps
    return {
        'ln1': gemm_like(oenc.ln_op(x_in, p['ln1'], eps), t('ln1')),
        'q': gemm_like(oenc.q_op(t('ln1'), p, dims.heads), t('q')),
        'k': gemm_like(oenc.k_op(t('ln1'), p), t('k')),
        'v': gemm_like(oenc.v_op(t('ln1'), p), t('v')),
        'attn': _close_rel(oenc.attention_core(t('q'), t('k'), t('v'), dims.heads), t('attn')),
        'attn_out': gemm_like(oenc.linear_op(t('attn'), p['o_w'], p['o_b']), t('attn_out')),
        'x_attn': exact(oenc.residual_op(x_in, t('attn_out')), t('x_attn')),
        'ln2': gemm_like(oenc.ln_op(t('x_attn'), p['ln2'], eps), t('ln2')),
        'fc1': gemm_like(oenc.linear_op(t('ln2'), p['fc1_w'], p['fc1_b']), t('fc1')),
        'gelu': exact(oenc.gelu_op(t('fc1')), t('gelu')),
        'fc2': gemm_like(oenc.linear_op(t('gelu'), p['fc2_w'], p['fc2_b']), t('fc2')),
        'out': exact(oenc.residual_op(t('x_attn'), t('fc2'), clamp=True), t('out')),
    }


def test_fixture_reaches_the_clamp(tiny16):
    dims, _, trace, z = tiny16
    assert list(z['clamped_layers']) == [1, 2]
    # transformers clamps a half tensor to +-(65504 - 1000), which fp16 stores as +-64512
    for i in z['clamped_layers']:
        out = trace[f'{i}.out']
        assert out.max() == 64512.0 and out.min() == -64512.0
    # in layer 1 the residual sum itself lies past the bound (65184), so the clamp changes values
    assert np.abs(f16(trace['1.x_attn'] + trace['1.fc2'])).max() > 64512.0


def test_encoder_fp16_stem_matches_transformers(tiny16):
    dims, params, trace, z = tiny16
    assert np.array_equal(oenc.embed_stem(params, z['mel'].astype(np.float32)), trace['0.out.in'])


@pytest.mark.parametrize('layer', [0, 1, 2])
def test_encoder_fp16_ops_match_transformers(tiny16, layer):
    dims, params, trace, _ = tiny16
    checks = _op_checks(dims, params, trace, layer)
    assert all(checks.values()), {k: v for k, v in checks.items() if not v}


def test_encoder_fp16_layers_and_output_match_transformers(tiny16):
    dims, params, trace, z = tiny16
    collect = []
    enc = oenc.encoder_forward(params, z['mel'].astype(np.float32), dims, collect=collect)
    for i in range(dims.enc_layers):
        assert _close_rel(collect[i + 1], trace[f'{i}.out']), i
    assert _close_rel(enc, z['enc'].astype(np.float32))


def _planted(monkeypatch, name, fn):
    monkeypatch.setattr(oenc, name, fn)


PLANTED = {
    # query scaled in fp32 before its one rounding (transformers rounds the projection first)
    'q': ('q_op', lambda y, p, heads, fp16=True: f16(
        (y @ p['q_w'].T + p['q_b']) * (y.shape[-1] // heads) ** -0.5)),
    # the softmax scale applied again inside attention (transformers passes scaling=1.0)
    'attn': ('attention_core', lambda q, k, v, heads, fp16=True: ORIG['attention_core'](
        q * (q.shape[-1] // heads) ** -0.5, k, v, heads, fp16)),
    # the LayerNorm output kept in fp32
    'ln1': ('ln_op', lambda x, ln, eps, fp16=True: odec.layer_norm(x, *ln, eps)),
    # the tanh approximation of GELU
    'gelu': ('gelu_op', lambda a, fp16=True: f16(0.5 * a * (1 + np.tanh(np.sqrt(2 / np.pi) * (a + 0.044715 * a ** 3))))),
    # no clamp at the end of the layer
    'out': ('residual_op', lambda x, r, fp16=True, clamp=False: f16(np.asarray(x, np.float32) + r)),
}
ORIG = {n: getattr(oenc, n) for n in ('q_op', 'attention_core', 'ln_op', 'gelu_op', 'residual_op')}


@pytest.mark.parametrize('op', sorted(PLANTED))
def test_encoder_fp16_planted_mistake_is_caught(tiny16, monkeypatch, op):
    dims, params, trace, _ = tiny16
    name, fn = PLANTED[op]
    _planted(monkeypatch, name, fn)
    failed = set()
    for layer in range(dims.enc_layers):
        failed |= {k for k, v in _op_checks(dims, params, trace, layer).items() if not v}
    assert op in failed


def test_encoder_fp16_unrounded_clamp_bound_is_caught(tiny16, monkeypatch):
    """Clamping to 64504 without the fp16 rounding of the bound leaves a value fp16 cannot hold."""
    dims, params, trace, _ = tiny16

    def clamp_unrounded(x, r, fp16=True, clamp=False):
        out = f16(np.asarray(x, np.float32) + r)
        return np.clip(out, -oenc.CLAMP, oenc.CLAMP) if clamp else out

    _planted(monkeypatch, 'residual_op', clamp_unrounded)
    assert not _op_checks(dims, params, trace, 1)['out']


def test_sinusoids_match_transformers():
    z = np.load(GOLDEN / 'hf_tiny.npz')
    ref = z['param:model.encoder.embed_positions.weight']
    # transformers evaluates them in float32, this build in float64
    np.testing.assert_allclose(weights.sinusoids(*ref.shape), ref, atol=1e-6, rtol=0)
    assert np.abs(weights.sinusoids(*ref.shape) - ref).max() < 1e-6


@pytest.fixture(scope='module')
def greedy_case():
    z = np.load(GOLDEN / 'hf_greedy.npz')
    dims = _dims(json.loads(str(z['config'])))
    params = {k[len('param:'):]: z[k] for k in z.files if k.startswith('param:')}
    meta = json.loads((GOLDEN / 'hf_greedy.json').read_text())
    ckv = oenc.cross_kv(params, z['enc'], dims, fp16=False)

    def run(suppress, begin, eos=(), stop_at_eos=False):
        dec = odec.DecoderOracle(params, dims, ckv, fp16=False)
        return odec.greedy(dec, meta['prompt'], meta['limit'], suppress, begin, eos, stop_at_eos)['ids']

    return meta, run


def test_greedy_matches_transformers_loop(greedy_case):
    meta, run = greedy_case
    assert run((), ()) == meta['ids_free']
    assert run(meta['suppress'], ()) == meta['ids_suppressed']
    assert run((), meta['begin_suppress']) == meta['ids_begin_only']
    assert run(meta['suppress'], meta['begin_suppress']) == meta['ids']
    assert run(meta['suppress'], meta['begin_suppress'], meta['eos'], True) == meta['ids_eos']


def test_greedy_planted_protocol_mistakes_are_caught(greedy_case):
    meta, run = greedy_case
    sup, begin = meta['suppress'], meta['begin_suppress']
    assert run(list(sup) + list(begin), ()) != meta['ids']      # begin-suppress on every step
    assert run((), list(sup) + list(begin)) != meta['ids']      # suppress on the first step only
    assert run(sup, begin, meta['eos'], False) != meta['ids_eos']  # no EOS stop

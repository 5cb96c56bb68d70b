"""Pins the CPU oracle against third-party golden vectors (transformers, recorded by
tests/golden/make_golden.py) and against closed forms. CPU only."""

import json

import numpy as np
import pytest

from conftest import GOLDEN
from flash_whisper_amd.config import WhisperDims
from oracle import decoder as odec
from oracle import encoder as oenc
from oracle import logmel as olm


@pytest.fixture(scope='module')
def tiny():
    z = np.load(GOLDEN / 'hf_tiny.npz')
    cfg = json.loads(str(z['config']))
    dims = WhisperDims(n_mels=cfg['num_mel_bins'], d_model=cfg['d_model'], heads=cfg['encoder_attention_heads'],
                       ffn=cfg['encoder_ffn_dim'], enc_layers=cfg['encoder_layers'], dec_layers=cfg['decoder_layers'],
                       vocab=cfg['vocab_size'], enc_len=cfg['max_source_positions'],
                       max_pos=cfg['max_target_positions'])
    params = {k[len('param:'):]: z[k] for k in z.files if k.startswith('param:')}
    return dims, params, z


def test_encoder_matches_transformers_fp32(tiny):
    dims, params, z = tiny
    enc = oenc.encoder_forward(params, z['mel'], dims, fp16=False)
    np.testing.assert_allclose(enc, z['enc'], atol=2e-5, rtol=1e-4)


def test_decoder_step_matches_transformers_fp32(tiny):
    dims, params, z = tiny
    ckv = oenc.cross_kv(params, z['enc'], dims, fp16=False)
    dec = odec.DecoderOracle(params, dims, ckv, fp16=False)
    for pos, tok in enumerate(z['ids']):
        logits = dec.step(int(tok), pos)
        np.testing.assert_allclose(logits, z['logits'][pos], atol=2e-5, rtol=1e-4)


def test_decoder_oracle_detects_a_planted_mistake(tiny):
    """A plausible slip (omitting the fused v bias) must be visible at the golden vectors' tolerance."""
    dims, params, z = tiny
    bad = dict(params)
    bad['model.decoder.layers.0.self_attn.v_proj.bias'] = np.zeros_like(params['model.decoder.layers.0.self_attn.v_proj.bias'])
    dec = odec.DecoderOracle(bad, dims, oenc.cross_kv(params, z['enc'], dims, fp16=False), fp16=False)
    logits = np.stack([dec.step(int(t), p) for p, t in enumerate(z['ids'])])
    assert np.abs(logits - z['logits']).max() > 1e-3


def test_mel_filterbank_matches_transformers():
    z = np.load(GOLDEN / 'hf_logmel.npz')
    np.testing.assert_allclose(olm.mel_filterbank(), z['mel_filters'], rtol=1e-12, atol=1e-15)


def test_log_mel_matches_transformers():
    z = np.load(GOLDEN / 'hf_logmel.npz')
    np.testing.assert_allclose(olm.log_mel(z['audio']), z['log_mel'], atol=2e-5)


def test_slaney_scale_identities():
    # linear below 1 kHz (3 f / 200), log above with 27 / ln 6.4 mels per e-fold; continuous at 1 kHz
    assert olm._hz_to_mel(1000.0)[0] == pytest.approx(15.0)
    assert olm._hz_to_mel(500.0)[0] == pytest.approx(7.5)
    assert olm._hz_to_mel(6400.0)[0] == pytest.approx(42.0)
    f = np.array([10.0, 999.0, 1000.0, 2500.0, 7999.0])
    np.testing.assert_allclose(olm._mel_to_hz(olm._hz_to_mel(f)), f, rtol=1e-12)
    fb = olm.mel_filterbank()
    assert fb.shape == (201, 128) and (fb.max(axis=0) > 0).all()


def test_power_spectrum_parseval_and_pure_tone():
    rng = np.random.default_rng(0)
    wave = rng.standard_normal(4000)
    p = olm.power_spectrogram(wave)
    # Parseval on one interior frame: sum |X_k|^2 over the full spectrum == N * sum (x w)^2
    t = 7
    frame = np.pad(wave, 200, mode='reflect')[t * 160: t * 160 + 400] * olm.hann_periodic()
    full = p[:, t].sum() * 2 - p[0, t] - p[200, t]
    assert full == pytest.approx(400 * np.sum(frame ** 2), rel=1e-10)
    # a tone on bin 40 (1600 Hz): the windowed peak is (A * sum(w) / 2)^2 = (0.5 * 200 / 2)^2
    n = np.arange(16000)
    tone = 0.5 * np.cos(2 * np.pi * 1600 * n / 16000)
    pk = olm.power_spectrogram(tone)[:, 20]
    assert int(np.argmax(pk)) == 40
    assert pk[40] == pytest.approx((0.5 * 200 / 2) ** 2, rel=1e-9)


def test_layernorm_and_attention_closed_forms():
    rng = np.random.default_rng(1)
    h = rng.standard_normal(1280).astype(np.float32)
    r, y = odec.add_layernorm(h, None, np.ones(1280), np.zeros(1280), 1e-5, fp16=False)
    assert abs(float(y.mean())) < 1e-6 and float(y.std()) == pytest.approx(1.0, rel=1e-4)
    # one key -> output is that key's value row; equal scores -> mean of the values
    q = rng.standard_normal((2, 64))
    k = rng.standard_normal((2, 5, 64))
    v = rng.standard_normal((2, 5, 64))
    np.testing.assert_allclose(odec.attention(q, k, v, 1, 0.125, fp16=False).reshape(2, 64), v[:, 0], rtol=1e-6)
    np.testing.assert_allclose(odec.attention(np.zeros((2, 64)), k, v, 5, 0.125, fp16=False).reshape(2, 64),
                               v.mean(axis=1), rtol=1e-5, atol=1e-6)


def test_masked_argmax_ties_and_suppression():
    logits = np.array([1.0, 3.0, 3.0, 2.0, 3.0], np.float32)
    assert odec.masked_argmax(logits, np.zeros(5, bool)) == 1
    assert odec.masked_argmax(logits, np.array([0, 1, 0, 0, 0], bool)) == 2
    # brute force on small random sets
    rng = np.random.default_rng(2)
    for _ in range(50):
        lg = np.round(rng.standard_normal(40), 1).astype(np.float32)
        sup = rng.random(40) < 0.2
        best = max((v, -i) for i, v in enumerate(lg) if not sup[i])
        assert odec.masked_argmax(lg, sup) == -best[1]


def test_finalize_state_machine():
    # custom/selftest.py:79-85: state [3, 0] -> [4, 1], token appended, cur == token
    tokens, state, cur = odec.finalize(42, [0] * 8, [3, 0], 448)
    assert tokens[0] == 42 and state == [4, 1] and cur == 42
    # position saturates at max_pos - 1, count at max_pos
    tokens, state, cur = odec.finalize(7, [0] * 4, [3, 4], 4)
    assert state == [3, 4] and tokens == [0] * 4


def test_conv1d_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 9)).astype(np.float32)
    w = rng.standard_normal((2, 3, 3)).astype(np.float32)
    b = rng.standard_normal(2).astype(np.float32)
    for stride in (1, 2):
        out = oenc.conv1d(x, w, b, stride)
        xp = np.pad(x, ((0, 0), (1, 1)))
        t_out = (9 - 1) // stride + 1
        ref = np.array([[np.sum(w[o] * xp[:, t * stride: t * stride + 3]) + b[o] for t in range(t_out)]
                        for o in range(2)])
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_gelu_lookup_equals_direct_evaluation():
    """The oracle's fp16 GELU lookup gives exactly f16(gelu(x)) at every finite fp16 input."""
    from oracle.common import f16, gelu, gelu_f16

    every = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    every = every[np.isfinite(every)]
    assert np.array_equal(gelu_f16(every), f16(gelu(every)))

"""bench.py's accounting on the CPU: the algorithmic byte and FLOP counts against the unit sizes the
path is specified with (decode step 347 233 946 + 20 480 L bytes, LM head 132 836 514 bytes, encoder
2.313 TFLOP, log-mel 3 558 912 bytes, cross attention + MLP 33 925 120 bytes), and the selftest gate."""

import pytest

import bench
from flash_whisper_amd.config import TURBO


def test_decode_step_bytes():
    for length in (0, 1, 64, 448):
        assert bench.decode_step_bytes(TURBO, length) == 347_233_946 + 20_480 * length
    # the int8 table (1 B a weight) and its 8 B of scale and bound per row replace the fp16 table
    assert (bench.decode_step_bytes(TURBO, 5) - bench.decode_step_bytes(TURBO, 5, q8=True)
            == TURBO.vocab * TURBO.d_model - 8 * TURBO.vocab)


def test_unit_bytes_and_flops():
    assert bench.lm_head_unit_bytes(TURBO) == 132_836_514
    assert bench.encoder_flops(TURBO) == pytest.approx(2.313e12, rel=1e-3)
    # log-mel: the waveform in, the fp32 log-mel out, the filterbank
    assert bench.LOG_MEL_BYTES == 480_000 * 4 + 128 * 3000 * 4 + 201 * 128 * 4
    # cross attention + MLP: K/V of 1500 frames, fc1 and fc2 weights, and 12 fp16 1280-vectors (q, the
    # 5120 fc1 bias, the fc2 bias, gamma, beta, the residual, the attention and MLP outputs)
    d, f = TURBO.d_model, TURBO.ffn
    assert bench.CROSS_MLP_BYTES == 2 * 1500 * d * 2 + 2 * 2 * d * f + 12 * 2 * d


def test_selftest_gate():
    assert bench.selftest_gate({'ok': True, 'checks': []}) is None
    bad = {'ok': False, 'checks': [{'name': 'add_layernorm', 'max_err': 1.0, 'ok': False},
                                   {'name': 'kv_write_1', 'max_err': 0.0, 'ok': True}]}
    assert bench.selftest_gate(bad) == "selftest failed: ['add_layernorm']"
    assert bench.selftest_gate({'ok': None, 'checks': []}) == 'selftest did not run'


def test_percentile_is_linear_interpolation():
    import numpy as np

    rng = np.random.default_rng(3)
    for n in (1, 2, 5, 20, 21):
        v = list(rng.standard_normal(n))
        for p in (0.0, 0.5, 0.9, 1.0):
            assert bench.percentile(v, p) == pytest.approx(float(np.percentile(v, 100 * p)), abs=1e-12)
    # the reference's report: 20 reps 1..20 give p90 = 18.1
    assert bench.percentile(list(range(20, 0, -1)), 0.9) == pytest.approx(18.1)


def test_latency_row():
    rows = [{'e2e_s': (10 + i) * 1e-3, 'ttft_s': 4e-3 + i * 1e-4, 'n_tokens': 37} for i in range(11)]
    r = bench.latency_row(rows, 5)
    assert r['e2e_ms'] == 15.0 and r['e2e_p90_ms'] == 19.0 and r['reps'] == 11 and r['tokens'] == 37
    assert r['ttft_ms'] == pytest.approx(4.5) and r['ttft_p90_ms'] == pytest.approx(4.9)
    assert r['audio_s_per_s'] == round(5 / 15e-3, 1)

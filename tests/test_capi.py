"""The C-ABI library: every symbol declared in include/flash_whisper.h is exported, argument
validation fails before any launch with FW_EINVAL and a message, and the torch-level validators raise
RuntimeError like the reference's TORCH_CHECKs. No GPU work is started. CPU only."""

import ctypes
import re

import numpy as np
import pytest
import torch

from conftest import ROOT


def declared_symbols():
    text = (ROOT / 'include' / 'flash_whisper.h').read_text()
    return sorted(set(re.findall(r'^\s*(?:const\s+)?(?:\w+\s+)*\w+\*?\s+\**(fw_\w+)\s*\(', text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ('fw_lm_head_argmax', 'fw_argmax_finalize', 'fw_decode_attention', 'fw_add_layernorm',
              'fw_log_mel', 'fw_gemm', 'fw_conv1d', 'fw_encoder_qkv', 'fw_encoder_pack_vt', 'fw_encoder_attention',
              'fw_encoder_vt_elems', 'fw_cross_kv'):
        assert s in syms


def test_library_exports_every_declared_symbol(built_lib):
    from flash_whisper_amd import _lib

    for s in declared_symbols():
        assert hasattr(built_lib, s), s
        assert s in _lib.SIGNATURES, f'{s} has no ctypes signature'


def test_validation_errors_return_einval(built_lib):
    from flash_whisper_amd import _lib

    lib = built_lib
    assert lib.fw_gemv(None, None, None, None, 1280, 1280, 0, None) == _lib.FW_EINVAL
    assert b'null' in lib.fw_last_error()
    dummy = ctypes.c_void_p(16)
    assert lib.fw_lm_head_argmax(dummy, dummy, dummy, 51866, 1000, dummy, None) == _lib.FW_EINVAL
    assert b'hidden size must be 1280' in lib.fw_last_error()
    # len_state / k_new / v_new must come together (whisper_kernels.cu:313-314)
    rc = lib.fw_decode_attention(dummy, dummy, dummy, dummy, dummy, None, None, 20, 448, dummy, dummy, dummy,
                                 1000, 0.125, None)
    assert rc == _lib.FW_EINVAL and b'given together' in lib.fw_last_error()
    rc = lib.fw_decode_attention(dummy, dummy, dummy, dummy, None, None, None, 20, 448, dummy, dummy, dummy,
                                 20 * 7 - 1, 0.125, None)
    assert rc == _lib.FW_EINVAL and b'workspace too small' in lib.fw_last_error()
    rc = lib.fw_gemm(dummy, 1280, dummy, 1280, None, dummy, 1280, None, 0, 1500, 1000, 1280, 0, 0, None)
    assert rc == _lib.FW_EINVAL
    rc = lib.fw_gemm(dummy, 1280, dummy, 1280, None, dummy, 1280, None, 0, 1500, 1280, 1280, 2, 0, None)
    assert rc == _lib.FW_EINVAL and b'needs res' in lib.fw_last_error()
    assert lib.fw_log_mel(dummy, 100, dummy, dummy, None, dummy, 100, None) == _lib.FW_EINVAL
    assert lib.fw_log_mel_prepare(dummy, dummy, 100, None) == _lib.FW_EINVAL  # workspace too small
    assert b'workspace needs' in lib.fw_last_error()
    assert lib.fw_log_mel_prepare(None, dummy, 1 << 20, None) == _lib.FW_EINVAL
    assert lib.fw_wave_upload(None, 10, dummy, dummy, 10, 4, None) == _lib.FW_EINVAL
    assert lib.fw_wave_upload(dummy, 11, dummy, dummy, 10, 4, None) == _lib.FW_EINVAL  # more samples than room
    assert lib.fw_wave_upload(dummy, 0, dummy, dummy, 10, 4, None) == _lib.FW_EINVAL
    assert lib.fw_wave_upload(dummy, 10, dummy, dummy, 10, 0, None) == _lib.FW_EINVAL
    assert lib.fw_log_mel_run(dummy, 480000, dummy, dummy, None, dummy, 100, None) == _lib.FW_EINVAL
    assert b'workspace needs' in lib.fw_last_error()
    rc = lib.fw_encoder_qkv(dummy, dummy, None, dummy, dummy, 1500, 3, None)  # 3 * 64 is not a multiple of 128
    assert rc == _lib.FW_EINVAL and b'multiple of 128' in lib.fw_last_error()
    assert lib.fw_encoder_attention(dummy, None, dummy, 1500, 20, None) == _lib.FW_EINVAL
    rc = lib.fw_gemm_splitk(dummy, 5120, dummy, 5120, dummy, 1500, 1280, 5120, 3, None)
    assert rc == _lib.FW_EINVAL and b'splits must be 2' in lib.fw_last_error()
    rc = lib.fw_gemm_splitk(dummy, 5120, dummy, 5120, dummy, 1500, 1280, 5056, 2, None)  # k not a multiple of 128
    assert rc == _lib.FW_EINVAL
    rc = lib.fw_layernorm_rows_residual(dummy, 2, dummy, dummy, dummy, dummy, dummy, 1500, 1280, 1e-5, 0, None)
    assert rc == _lib.FW_EINVAL and b'residual epilogue' in lib.fw_last_error()
    assert lib.fw_encoder_vt_elems(1500, 20) == 20 * 64 * 1536 and lib.fw_encoder_vt_elems(0, 20) == 0


def test_decoder_step_entry_points_validate(built_lib):
    """fw_decoder_step_layers and fw_decoder_step check their arguments before any HIP call; the workspace
    size covers the control words, every layer's hand-off regions and the LM head's per-block maxima."""
    from flash_whisper_amd import _lib

    lib = built_lib
    assert lib.fw_decoder_step_max_layers() == 8
    one, two = lib.fw_decoder_step_workspace_bytes(1), lib.fw_decoder_step_workspace_bytes(2)
    layer = two - one

    assert lib.fw_decoder_step_workspace_bytes(4) == one + 3 * layer
    assert lib.fw_decoder_step_workspace_bytes(0) == 0 and lib.fw_decoder_step_workspace_bytes(9) == 0
    assert ctypes.sizeof(_lib.DecLayer) == 18 * 8 + 3 * 4 + 4 + 4 * 8  # C layout: pad before the caches
    table = (_lib.DecLayer * 4)()
    d = ctypes.c_void_p(256)
    args = [d, d, d, d, 51866, 448, 1500, 0.125, d, d, d, lib.fw_decoder_step_workspace_bytes(4), 1000, None]
    assert lib.fw_decoder_step_layers(table, 4, *args) == _lib.FW_EINVAL
    assert b'null tensor' in lib.fw_last_error()  # the layer table is empty
    assert lib.fw_decoder_step_layers(table, 9, *args) == _lib.FW_EINVAL
    assert b'n_layers' in lib.fw_last_error()
    bad = list(args)
    bad[5] = 513  # max_pos beyond 8 splits of 64 keys
    assert lib.fw_decoder_step_layers(table, 4, *bad) == _lib.FW_EINVAL and b'max_pos' in lib.fw_last_error()
    bad = list(args)
    bad[11] = 100  # workspace too small
    assert lib.fw_decoder_step_layers(table, 4, *bad) == _lib.FW_EINVAL and b'too small' in lib.fw_last_error()
    assert lib.fw_decoder_step_layers(None, 4, *args) == _lib.FW_EINVAL
    # the whole step: the LM head is required and checked like the layers
    step = [d, d, d, d, 51866, 448, 1500, 0.125, d, lib.fw_decoder_step_workspace_bytes(4), 1000, None]
    assert lib.fw_decoder_step(table, 4, None, 1, *step) == _lib.FW_EINVAL and b'null LM head' in lib.fw_last_error()
    # the float and the int are padded to the next 8-byte field; four int64 end-of-text ids
    assert ctypes.sizeof(_lib.DecHead) == 2 * 8 + 8 + 7 * 8 + 8 + 4 * 8
    head = _lib.DecHead(256, 256, 1e-5, 256, 256, 256, None, 256, None)
    assert lib.fw_decoder_step(table, 4, ctypes.byref(head), 8, *step) == _lib.FW_EINVAL
    assert b'null LM-head tensor' in lib.fw_last_error()  # no suppress mask
    head.suppress = 256
    head.wq = 264
    assert lib.fw_decoder_step(table, 4, ctypes.byref(head), 8, *step) == _lib.FW_EINVAL
    assert b'16-byte aligned' in lib.fw_last_error()
    head.wq = 256
    head.n_eos = 5
    assert lib.fw_decoder_step(table, 4, ctypes.byref(head), 8, *step) == _lib.FW_EINVAL
    assert b'n_eos' in lib.fw_last_error()
    head.n_eos = 1
    prompt = [d, d, d, d, 51866, 448, 1500, 0.125, d, lib.fw_decoder_step_workspace_bytes(4), 1000, None]
    assert lib.fw_decoder_prompt(table, 4, ctypes.byref(head), None, 4, *prompt) == _lib.FW_EINVAL
    assert lib.fw_decoder_prompt(table, 4, ctypes.byref(head), d, 3, *prompt) == _lib.FW_EINVAL
    assert b'n_prompt must be 4' in lib.fw_last_error()
    for n in (0, 1025):
        assert lib.fw_decoder_step(table, 4, ctypes.byref(head), n, *step) == _lib.FW_EINVAL
        assert b'n_steps' in lib.fw_last_error()


def test_status_becomes_runtime_error(built_lib):
    from flash_whisper_amd import _lib

    with pytest.raises(RuntimeError, match='hidden size'):
        _lib.check(built_lib.fw_lm_head_argmax(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                               10, 7, ctypes.c_void_p(16), None), 'lm_head_argmax')


def test_torch_validators_raise_before_launch(built_lib):
    from flash_whisper_amd.ext import load_ext

    ext = load_ext()
    h = torch.zeros(1280, dtype=torch.float16)  # CPU tensor: rejected like the reference's is_cuda check
    with pytest.raises(RuntimeError, match='contiguous CUDA fp16'):
        ext.add_layernorm(h, None, h, h, h, 1e-5)
    with pytest.raises(RuntimeError, match='contiguous CUDA fp16'):
        ext.lm_head_argmax(h, torch.zeros(4, 1280, dtype=torch.float16), torch.zeros(4, dtype=torch.bool),
                           torch.zeros(1, dtype=torch.long))
    with pytest.raises(RuntimeError, match='int64'):
        ext.argmax_finalize(torch.zeros(1, dtype=torch.long), torch.zeros(4, dtype=torch.int32),
                            torch.zeros(2, dtype=torch.long), torch.zeros(1, dtype=torch.long), 448)


def test_host_synth_is_standard_normal(built_lib):
    from scipy import stats

    from flash_whisper_amd import weights

    z = weights.host_normal('test.tensor', (400000,), seed=3, std=1.0).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert stats.kstest(z, 'norm').pvalue > 1e-3
    w = weights.host_normal('test.tensor', (400000,), seed=3).astype(np.float64)
    assert abs(w.std() - 0.02) < 2e-4
    # different names / seeds give independent streams; same name + seed is reproducible
    assert not np.array_equal(weights.host_normal('a', (64,)), weights.host_normal('b', (64,)))
    assert not np.array_equal(weights.host_normal('a', (64,), seed=0), weights.host_normal('a', (64,), seed=1))
    np.testing.assert_array_equal(weights.host_normal('a', (64,)), weights.host_normal('a', (64,)))


def test_product_filterbank_matches_transformers():
    from conftest import GOLDEN
    from flash_whisper_amd.audio import mel_filters

    z = np.load(GOLDEN / 'hf_logmel.npz')
    np.testing.assert_allclose(mel_filters(), z['mel_filters'].astype(np.float32), rtol=1e-6, atol=1e-9)

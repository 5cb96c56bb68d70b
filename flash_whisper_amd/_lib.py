"""ctypes binding of the C ABI in include/flash_whisper.h (libflash_whisper.so, built in-tree).

Loading never compiles: if the library is missing this raises, so no code path can silently run
without the HIP kernels. Build it with ``python -m flash_whisper_amd.build``. The environment variable
FW_LIBRARY selects another build of the same sources, e.g. the phase-timeline profiling build
``libflash_whisper_timeline.so`` (``flash_whisper_amd.step_timeline``).
"""

import ctypes
import os
import threading
from ctypes import c_float, c_int, c_int64, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get('FW_LIBRARY') or Path(__file__).resolve().parent / 'libflash_whisper.so').resolve()

FW_OK, FW_EINVAL, FW_EHIP = 0, -1, -2
NOALLOC_ATTN_SLOTS = 2048  # FW_NOALLOC_ATTN_SLOTS
ACT_NONE, ACT_GELU = 0, 1
EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESID, EPI_BIAS_RESID_CLAMP, EPI_BIAS_GELU_POS, EPI_SCALE_Q = range(6)

P = c_void_p
# name -> (restype, argtypes); mirrors include/flash_whisper.h one to one.
SIGNATURES = {
    'fw_last_error': (ctypes.c_char_p, []),
    'fw_version': (c_int, []),
    'fw_lm_head_argmax': (c_int, [P, P, P, c_int, c_int, P, P]),
    'fw_argmax_finalize': (c_int, [P, P, P, P, c_int, P]),
    'fw_decode_attention': (c_int, [P, P, P, P, P, P, P, c_int, c_int, P, P, P, c_int64, c_float, P]),
    'fw_decode_attention_noalloc': (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_float, P]),
    'fw_add_layernorm': (c_int, [P, P, P, P, P, c_int, c_float, P]),
    'fw_embed': (c_int, [P, P, P, P, c_int, c_int, P, c_int, P]),
    'fw_gemv': (c_int, [P, P, P, P, c_int, c_int, c_int, P]),
    'fw_ln_gemv': (c_int, [P, P, P, P, P, c_float, P, P, P, P, c_int, c_int, P, P, P, c_int, c_int, c_int, P]),
    'fw_decode_attention_fused': (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_float, P]),
    'fw_attention_split': (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, P, P, P, c_int64, c_float, P]),
    'fw_attn_out_gemv': (c_int, [P, P, P, c_int64, P, c_int, c_int, c_int, P, P, P, c_int, P]),
    'fw_gemv_batch': (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, P]),
    'fw_ln_gemv_batch': (c_int, [P, P, P, P, P, c_float, P, P, P, P, c_int, c_int, P, P, P, c_int, c_int, c_int, c_int,
                                 P]),
    'fw_attention_split_batch': (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, P, P, P, c_int64, c_float, c_int, c_int,
                                         c_int, P]),
    'fw_attn_out_gemv_batch': (c_int, [P, P, P, c_int64, P, c_int, c_int, c_int, P, P, P, c_int, c_int, P]),
    'fw_lm_head_argmax_fused': (c_int, [P, P, P, P, c_float, P, P, c_int, c_int, P, P, P, P, c_int, P]),
    'fw_lm_head_q8_pack': (c_int, [P, c_int, c_int, P, P, P]),
    'fw_lm_head_argmax_q8': (c_int, [P, P, P, P, c_float, P, P, P, P, c_int, c_int, P, P, P, P, c_int, P]),
    'fw_log_mel': (c_int, [P, c_int, P, P, P, P, c_int64, P]),
    'fw_log_mel_ws_floats': (c_int64, [c_int]),
    'fw_log_mel_prepare': (c_int, [P, P, c_int64, P]),
    'fw_log_mel_run': (c_int, [P, c_int, P, P, P, P, c_int64, P]),
    'fw_wave_upload': (c_int, [P, c_int64, P, P, c_int64, c_int64, P]),
    'fw_gemm': (c_int, [P, c_int, P, c_int, P, P, c_int, P, c_int, c_int, c_int, c_int, c_int, c_int, P]),
    'fw_conv1d': (c_int, [P, c_int, c_int, c_int, P, P, P, c_int, P, c_int, P]),
    'fw_layernorm_rows': (c_int, [P, P, P, P, c_int, c_int, c_float, P]),
    'fw_gemm_splitk': (c_int, [P, c_int, P, c_int, P, c_int, c_int, c_int, c_int, P]),
    'fw_layernorm_rows_residual': (c_int, [P, c_int, P, P, P, P, P, c_int, c_int, c_float, c_int, P]),
    'fw_encoder_vt_elems': (ctypes.c_longlong, [c_int, c_int]),
    'fw_encoder_qkv': (c_int, [P, P, P, P, P, c_int, c_int, P]),
    'fw_encoder_pack_vt': (c_int, [P, P, c_int, c_int, P]),
    'fw_encoder_attention': (c_int, [P, P, P, c_int, c_int, P]),
    'fw_cross_kv': (c_int, [P, c_int, P, P, P, c_int, c_int, P]),
    'fw_synth_normal_f16': (c_int, [P, c_int64, c_int64, c_uint64, c_uint64, c_float, c_float, P]),
    'fw_synth_normal_f16_host': (c_int, [P, c_int64, c_int64, c_uint64, c_uint64, c_float, c_float]),
    'fw_decoder_step_workspace_bytes': (ctypes.c_size_t, [c_int]),
    'fw_decoder_step_calibrate': (c_int, [P, c_int64, c_int, P]),
    'fw_decoder_step_calibrated': (c_int, [P]),
    'fw_decoder_step_max_layers': (c_int, []),
    'fw_decoder_step_layers': (c_int, [P, c_int, P, P, P, P, c_int, c_int, c_int, c_float, P, P, P, c_int64, c_int64,
                                       P]),
    'fw_decoder_prompt': (c_int, [P, c_int, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_float, P, c_int64, c_int64,
                                  P]),
    'fw_host_alloc_coherent': (c_void_p, [ctypes.c_size_t]),
    'fw_host_free': (None, [P]),
    'fw_final_layernorm': (c_int, [P, P, P, P, P, c_int, c_float, P]),
    'fw_decoder_step': (c_int, [P, c_int, P, c_int, P, P, P, P, c_int, c_int, c_int, c_float, P, c_int64, c_int64, P]),
    'fw_decoder_step_resident_rows': (c_int, []),
    'fw_decoder_step_check': (c_int, [c_int, c_int, c_int, c_int, c_int]),
    'fw_decoder_step_timeline': (c_int, [P, c_int64, c_int]),
    'fw_decoder_step_timeline_slots': (c_int, []),
}

DEC_LAYER_TENSORS = ('ln1_gamma', 'ln1_beta', 'qkv_w', 'qkv_b', 'out_w', 'out_b', 'ln2_gamma', 'ln2_beta',
                     'cross_q_w', 'cross_q_b', 'cross_out_w', 'cross_out_b', 'ln3_gamma', 'ln3_beta', 'fc1_w',
                     'fc1_b', 'fc2_w', 'fc2_b')


class DecLayer(ctypes.Structure):
    """struct fw_dec_layer: one decoder layer's device pointers for fw_decoder_step_layers."""
    _fields_ = ([(n, c_void_p) for n in DEC_LAYER_TENSORS] + [(f'ln{i}_eps', c_float) for i in (1, 2, 3)]
                + [(n, c_void_p) for n in ('self_k', 'self_v', 'cross_k', 'cross_v')])


class DecHead(ctypes.Structure):
    """struct fw_dec_head: the LM head of fw_decoder_step."""
    _fields_ = [('ln_gamma', c_void_p), ('ln_beta', c_void_p), ('ln_eps', c_float), ('w', c_void_p), ('wq', c_void_p),
                ('meta', c_void_p), ('suppress', c_void_p), ('tokens', c_void_p), ('y_out', c_void_p),
                ('host_tokens', c_void_p), ('n_eos', c_int), ('eos', c_int64 * 4)]


_lib = None
_lock = threading.Lock()


class FwError(RuntimeError):
    """A non-zero status from the C ABI (validation or HIP launch failure)."""


def lib():
    """The loaded library with typed entry points. Raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f'{LIB_PATH} is missing; build it with `python -m flash_whisper_amd.build`')
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = restype, argtypes
            _lib = handle
    return _lib


def check(status, what):
    if status != FW_OK:
        msg = lib().fw_last_error().decode(errors='replace')
        raise FwError(f'{what}: {msg} (status {status})')

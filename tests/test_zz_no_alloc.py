"""fw_decode_attention_noalloc (the decode attention whose split partials live in the library's static
device array, for callers that cannot allocate) against fw_decode_attention with a caller workspace,
called through the C ABI: bit-identical output and cache on two calls in a row, the second with a
smaller input (fewer heads and keys, so the static array still holds the first call's partials), in
self and cross mode; a size beyond the static array fails before any launch."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _half(rng, *shape):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float16)).cuda()


def _call_both(lib, heads, max_len, pos, rng, self_mode):
    from flash_whisper_amd._lib import check
    from flash_whisper_amd.selftest import workspace

    q = _half(rng, heads * 64)
    k, v = _half(rng, heads, max_len, 64), _half(rng, heads, max_len, 64)
    k_new, v_new = (_half(rng, heads, 64), _half(rng, heads, 64)) if self_mode else (None, None)
    state = torch.tensor([pos, 0], dtype=torch.long, device='cuda') if self_mode else None
    ptr = lambda t: None if t is None else t.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    scale = ctypes.c_float(0.125)
    splits = -(-max_len // 64)
    pm, pl, pa = workspace(heads, splits)
    k1, v1, out1 = k.clone(), v.clone(), torch.empty_like(q)
    check(lib.fw_decode_attention(ptr(q), ptr(k1), ptr(v1), ptr(out1), ptr(state), ptr(k_new), ptr(v_new), heads,
                                  max_len, ptr(pm), ptr(pl), ptr(pa), heads * splits, scale, stream), 'workspace')
    k2, v2, out2 = k.clone(), v.clone(), torch.full_like(q, float('nan'))
    check(lib.fw_decode_attention_noalloc(ptr(q), ptr(k2), ptr(v2), ptr(out2), ptr(state), ptr(k_new), ptr(v_new),
                                          heads, max_len, scale, stream), 'noalloc')
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    if self_mode:
        assert torch.equal(k2[:, pos], k_new) and torch.equal(v2[:, pos], v_new)
    return out2


@pytest.mark.parametrize('self_mode', [True, False])
def test_noalloc_matches_workspace_entry_point(hip_device, self_mode):
    from flash_whisper_amd import _lib

    lib = _lib.lib()
    rng = np.random.default_rng(5 + self_mode)
    # the largest call first (20 heads x 1500 keys = 480 slots; 448 keys in self mode), then a smaller one
    big = (20, 448, 300) if self_mode else (20, 1500, 0)
    small = (4, 100, 40) if self_mode else (3, 70, 0)
    first = _call_both(lib, *big, rng, self_mode)
    second = _call_both(lib, *small, rng, self_mode)
    assert torch.isfinite(first).all() and torch.isfinite(second).all()


def test_noalloc_rejects_sizes_beyond_the_static_workspace(hip_device):
    from flash_whisper_amd import _lib

    lib = _lib.lib()
    heads, max_len = 32, 64 * (_lib.NOALLOC_ATTN_SLOTS // 32 + 1)  # one split per head too many
    q = torch.zeros(heads * 64, dtype=torch.float16, device='cuda')
    k = torch.zeros(heads, max_len, 64, dtype=torch.float16, device='cuda')
    out = torch.zeros_like(q)
    rc = lib.fw_decode_attention_noalloc(q.data_ptr(), k.data_ptr(), k.data_ptr(), out.data_ptr(), None, None, None,
                                         heads, max_len, ctypes.c_float(0.125),
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.FW_EINVAL
    assert b'exceeds the 2048 slots' in lib.fw_last_error()

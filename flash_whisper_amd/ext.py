"""Loads the HIP kernels and exposes them as torch-tensor ops: the drop-in for custom/ext.py.

``load_ext()`` keeps the reference's name and call shape (custom/ext.py:13-18): no required
arguments, returns an object whose ops take caller-allocated torch tensors, launch on the current
stream, allocate nothing and raise ``RuntimeError`` when an argument is invalid — the contract of the
reference's ``TORCH_CHECK``s (custom/kernels/whisper_kernels.cu:269-356). The reference JIT-compiles
a pybind module with nvcc; here the kernels live in an ahead-of-time built C-ABI library
(include/flash_whisper.h) and this module is a thin ctypes layer over it. Nothing here falls back to
PyTorch math: without the library, ``load_ext()`` raises.

``python -m custom.ext`` (or ``python -m flash_whisper_amd.ext``) builds the library and prints the
compiler's per-kernel register, LDS and spill report, like the reference's ``main`` (custom/ext.py:21-50).
"""

import argparse
import ctypes
import sys

import numpy as np
import torch

from . import _lib
from ._lib import ACT_GELU, ACT_NONE, EPI_BIAS  # noqa: F401  (re-exported constants)
from .config import SPLIT_KEYS

HIDDEN, HEAD_DIM = 1280, 64
MAX_BATCH = 4  # decoder positions per batched launch (the prompt)
WAVE_CHUNK = 240000  # samples per staged chunk of the waveform upload (half of 30 s: smaller chunks measured slower)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _require(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def check_half(t, name):
    """Reference check_half (whisper_kernels.cu:272-274)."""
    _require(isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous() and t.dtype == torch.float16,
             f'{name} must be contiguous CUDA fp16')


def _check_rows(t, name, cols):
    """A [rows, cols] fp16 CUDA view with unit column stride and a 16-byte-aligned row stride; returns rows."""
    _require(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float16 and t.dim() == 2
             and t.size(1) == cols and t.stride(1) == 1 and (t.size(0) == 1 or t.stride(0) >= cols)
             and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0,
             f'{name} must be a CUDA fp16 [rows, {cols}] view with unit column stride and 16-byte aligned rows')
    return t.size(0)


def _check(t, name, dtype, what):
    _require(isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous() and t.dtype == dtype,
             f'{name} must be contiguous CUDA {what}')


class HostTokens:
    """n int64 of pinned host memory that device stores reach while a kernel runs (fw_host_alloc_coherent):
    the one-launch decode stores each token here as it is decoded and the host polls `array`."""

    def __init__(self, lib, n):
        import numpy as np

        self._lib = lib
        self.address = lib.fw_host_alloc_coherent(8 * n)
        if not self.address:
            raise RuntimeError(f'host_alloc_coherent: {lib.fw_last_error().decode(errors="replace")}')
        self.array = np.ctypeslib.as_array((ctypes.c_int64 * n).from_address(self.address))

    def __del__(self):
        if getattr(self, 'address', None):
            self.array = None
            self._lib.fw_host_free(self.address)
            self.address = None


class WhisperExt:
    """The op set of the reference extension plus the fused/encoder/front-end ops of this build."""

    def __init__(self):
        self.lib = _lib.lib()

    def _call(self, name, *args):
        _lib.check(getattr(self.lib, name)(*args), name)

    # ---- reference ops -------------------------------------------------------------------
    def lm_head_argmax(self, h, w, suppress, best):
        """whisper_kernels.cu:278-289."""
        check_half(h, 'h')
        check_half(w, 'w')
        _require(h.numel() == HIDDEN and w.dim() == 2 and w.size(1) == HIDDEN, f'hidden size must be {HIDDEN}')
        _require(suppress.dtype == torch.bool and suppress.is_cuda and suppress.is_contiguous()
                 and suppress.numel() == w.size(0), 'suppress must be bool [vocab]')
        _require(best.dtype == torch.int64 and best.is_cuda and best.numel() == 1, 'best must be int64 [1]')
        self._call('fw_lm_head_argmax', h.data_ptr(), w.data_ptr(), suppress.data_ptr(), w.size(0), HIDDEN,
                   best.data_ptr(), _stream())

    def argmax_finalize(self, best, tokens, state, cur, max_pos):
        """whisper_kernels.cu:291-298."""
        for t, n in ((tokens, 'tokens'), (state, 'state'), (cur, 'cur')):
            _require(t.dtype == torch.int64, 'tokens, state and cur must be int64')
            _require(t.is_cuda and t.is_contiguous(), f'{n} must be a contiguous CUDA tensor')
        _require(best.dtype == torch.int64 and best.is_cuda and best.numel() == 1, 'best must be int64 [1]')
        self._call('fw_argmax_finalize', best.data_ptr(), tokens.data_ptr(), state.data_ptr(), cur.data_ptr(),
                   int(max_pos), _stream())

    def _attn_checks(self, q, k, v, out, len_state, k_new, v_new, part_m, part_l, part_acc, split_keys):
        for t, n in ((q, 'q'), (k, 'k'), (v, 'v'), (out, 'out')):
            check_half(t, n)
        _require(k.dim() == 3 and k.size(2) == HEAD_DIM and k.shape == v.shape, 'k, v must be [heads, max_len, 64]')
        heads, max_len = k.size(0), k.size(1)
        splits = -(-max_len // split_keys)
        _require(q.numel() == heads * HEAD_DIM and out.numel() == heads * HEAD_DIM, 'q, out must be [heads * 64]')
        _require((k_new is None) == (v_new is None) == (len_state is None),
                 'len_state, k_new and v_new must be given together')
        if k_new is not None:
            check_half(k_new, 'k_new')
            check_half(v_new, 'v_new')
            _require(k_new.numel() == heads * HEAD_DIM and v_new.numel() == heads * HEAD_DIM,
                     'k_new, v_new must be [heads, 64]')
            _require(len_state.dtype == torch.int64 and len_state.is_cuda, 'len_state must be CUDA int64')
        for t in (part_m, part_l, part_acc):
            _require(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32,
                     'workspace must be contiguous CUDA fp32')
        slots = min(part_m.numel(), part_l.numel(), part_acc.numel() // HEAD_DIM)
        _require(slots >= heads * splits, f'workspace too small for {splits} splits')
        return heads, max_len, slots

    def decode_attention(self, q, k, v, out, len_state, k_new, v_new, part_m, part_l, part_acc, scale):
        """whisper_kernels.cu:300-339: split kernel (64 keys per split) + combine kernel."""
        heads, max_len, slots = self._attn_checks(q, k, v, out, len_state, k_new, v_new, part_m, part_l, part_acc,
                                                  SPLIT_KEYS)
        self._call('fw_decode_attention', q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _ptr(len_state),
                   _ptr(k_new), _ptr(v_new), heads, max_len, part_m.data_ptr(), part_l.data_ptr(),
                   part_acc.data_ptr(), slots, float(scale), _stream())

    def add_layernorm(self, h, x, gamma, beta, y, eps):
        """whisper_kernels.cu:341-356."""
        for t, n in ((h, 'h'), (gamma, 'gamma'), (beta, 'beta'), (y, 'y')):
            check_half(t, n)
        _require(h.numel() == HIDDEN, f'hidden size must be {HIDDEN}')
        if x is not None:
            check_half(x, 'x')
        self._call('fw_add_layernorm', h.data_ptr(), _ptr(x), gamma.data_ptr(), beta.data_ptr(), y.data_ptr(),
                   HIDDEN, float(eps), _stream())

    # ---- fused decoder ops ---------------------------------------------------------------
    def embed(self, cur, state, embed, pos_embed, h):
        check_half(embed, 'embed')
        check_half(pos_embed, 'pos_embed')
        check_half(h, 'h')
        self._call('fw_embed', cur.data_ptr(), state.data_ptr(), embed.data_ptr(), pos_embed.data_ptr(),
                   embed.size(0), pos_embed.size(0), h.data_ptr(), HIDDEN, _stream())

    def gemv(self, x, w, bias, out, act=ACT_NONE, nv=1):
        """out = act(w x + b); with nv > 1, x and out hold nv rows (a batch of decoder positions)."""
        check_half(x, 'x')
        check_half(w, 'w')
        check_half(out, 'out')
        _require(1 <= nv <= MAX_BATCH, f'nv must be in [1, {MAX_BATCH}]')
        _require(w.dim() == 2 and x.numel() == nv * w.size(1) and out.numel() == nv * w.size(0),
                 'gemv shape mismatch')
        if bias is not None:
            check_half(bias, 'bias')
            _require(bias.numel() == w.size(0), 'bias must be [n_out]')
        args = (x.data_ptr(), w.data_ptr(), _ptr(bias), out.data_ptr(), w.size(0), w.size(1), act)
        if nv == 1:
            self._call('fw_gemv', *args, _stream())
        else:
            self._call('fw_gemv_batch', *args, nv, _stream())

    def ln_gemv(self, h, x, h_out, gamma, beta, eps, w, bias, out, act=ACT_NONE, embed=None, nv=1):
        """r = fp16(h + x) -> h_out; y = LN(r); out = act(w y + b). embed = (cur, state, table, pos_table).
        With nv > 1, h, x, h_out and out hold nv rows and cur nv tokens (positions state[0] + v)."""
        for t, n in ((gamma, 'gamma'), (beta, 'beta'), (w, 'w'), (out, 'out')):
            check_half(t, n)
        _require(1 <= nv <= MAX_BATCH, f'nv must be in [1, {MAX_BATCH}]')
        _require(w.dim() == 2 and w.size(1) == HIDDEN and out.numel() == nv * w.size(0), 'ln_gemv shape mismatch')
        cur = state = table = pos_table = None
        if embed is not None:
            cur, state, table, pos_table = embed
            check_half(table, 'embed')
            check_half(pos_table, 'pos_embed')
            _check(cur, 'cur', torch.int64, 'int64')
            _require(cur.numel() >= nv, 'embedding mode needs nv tokens in cur')
        else:
            check_half(h, 'h')
            _require(h.numel() == nv * HIDDEN, 'h must hold nv rows of the hidden size')
        for t, n in ((x, 'x'), (h_out, 'h_out')):
            if t is not None:
                check_half(t, n)
                _require(t.numel() == nv * HIDDEN, f'{n} must hold nv rows of the hidden size')
        if bias is not None:
            check_half(bias, 'bias')
        args = (_ptr(h), _ptr(x), _ptr(h_out), gamma.data_ptr(), beta.data_ptr(), float(eps),
                _ptr(cur), _ptr(state), _ptr(table), _ptr(pos_table),
                0 if table is None else table.size(0), 0 if pos_table is None else pos_table.size(0),
                w.data_ptr(), _ptr(bias), out.data_ptr(), w.size(0), HIDDEN, act)
        if nv == 1:
            self._call('fw_ln_gemv', *args, _stream())
        else:
            self._call('fw_ln_gemv_batch', *args, nv, _stream())

    def _attn_io_checks(self, q, k, v, out, len_state, k_new, v_new):
        for t, n in ((q, 'q'), (k, 'k'), (v, 'v'), (out, 'out')):
            check_half(t, n)
        _require(k.dim() == 3 and k.size(2) == HEAD_DIM and k.shape == v.shape, 'k, v must be [heads, max_len, 64]')
        heads, max_len = k.size(0), k.size(1)
        _require(q.numel() == heads * HEAD_DIM and out.numel() == heads * HEAD_DIM, 'q, out must be [heads * 64]')
        _require((k_new is None) == (v_new is None) == (len_state is None),
                 'len_state, k_new and v_new must be given together')
        if k_new is not None:
            check_half(k_new, 'k_new')
            check_half(v_new, 'v_new')
            _require(k_new.numel() == heads * HEAD_DIM and v_new.numel() == heads * HEAD_DIM,
                     'k_new, v_new must be [heads, 64]')
            _require(len_state.dtype == torch.int64 and len_state.is_cuda, 'len_state must be CUDA int64')
        return heads, max_len

    def decode_attention_fused(self, q, k, v, out, len_state, k_new, v_new, scale):
        """decode_attention in a single launch (one block per head, no workspace)."""
        heads, max_len = self._attn_io_checks(q, k, v, out, len_state, k_new, v_new)
        self._call('fw_decode_attention_fused', q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                   _ptr(len_state), _ptr(k_new), _ptr(v_new), heads, max_len, float(scale), _stream())

    def decode_attention_noalloc(self, q, k, v, out, len_state, k_new, v_new, scale):
        """decode_attention with its split partials in the library's static device array: no workspace,
        no allocation (heads * ceil(max_len / 64) <= 2048; calls that overlap on one GPU race)."""
        heads, max_len = self._attn_io_checks(q, k, v, out, len_state, k_new, v_new)
        self._call('fw_decode_attention_noalloc', q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                   _ptr(len_state), _ptr(k_new), _ptr(v_new), heads, max_len, float(scale), _stream())

    def attention_split(self, q, k, v, len_state, k_new, v_new, part_m, part_l, part_acc, scale, split_keys=SPLIT_KEYS):
        """Split half of decode_attention: (m, l, acc) partials per (head, split) into the workspace."""
        heads, max_len, slots = self._attn_checks(q, k, v, q, len_state, k_new, v_new, part_m, part_l, part_acc,
                                                  split_keys)
        self._call('fw_attention_split', q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(len_state), _ptr(k_new),
                   _ptr(v_new), heads, max_len, int(split_keys), part_m.data_ptr(), part_l.data_ptr(),
                   part_acc.data_ptr(), slots, float(scale), _stream())

    def attention_split_batch(self, q, k, v, len_state, k_new, v_new, part_m, part_l, part_acc, scale,
                              split_keys=SPLIT_KEYS):
        """attention_split for nq = q.size(0) queries at positions len_state[0] + z (self mode). q, k_new
        and v_new are [nq, heads * 64] row views (the row stride may exceed the row, e.g. slices of a
        packed q/k/v batch); partials land query-major for attn_out_gemv(nv=nq)."""
        check_half(k, 'k')
        check_half(v, 'v')
        _require(k.dim() == 3 and k.size(2) == HEAD_DIM and k.shape == v.shape, 'k, v must be [heads, max_len, 64]')
        heads, max_len = k.size(0), k.size(1)
        nq = _check_rows(q, 'q', heads * HEAD_DIM)
        _require(1 <= nq <= MAX_BATCH, f'at most {MAX_BATCH} queries')
        _require((k_new is None) == (v_new is None) == (len_state is None),
                 'len_state, k_new and v_new must be given together')
        kv_stride = 0
        if k_new is not None:
            _require(_check_rows(k_new, 'k_new', heads * HEAD_DIM) == nq == _check_rows(v_new, 'v_new', heads * HEAD_DIM)
                     and k_new.stride(0) == v_new.stride(0), 'k_new, v_new must be [nq, heads * 64] with one stride')
            _require(len_state.dtype == torch.int64 and len_state.is_cuda, 'len_state must be CUDA int64')
            kv_stride = k_new.stride(0)
        for t in (part_m, part_l, part_acc):
            _require(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32,
                     'workspace must be contiguous CUDA fp32')
        slots = min(part_m.numel(), part_l.numel(), part_acc.numel() // HEAD_DIM)
        _require(slots >= nq * heads * -(-max_len // split_keys), 'workspace too small')
        self._call('fw_attention_split_batch', q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(len_state),
                   _ptr(k_new), _ptr(v_new), heads, max_len, int(split_keys), part_m.data_ptr(), part_l.data_ptr(),
                   part_acc.data_ptr(), slots, float(scale), nq, q.stride(0), kv_stride, _stream())

    def attn_out_gemv(self, part_m, part_l, part_acc, len_state, heads, max_len, w, bias, out, split_keys=SPLIT_KEYS,
                      nv=1):
        """Combine of attention_split partials + output projection: out = fp16(w . combine + bias); with
        nv > 1 the partials of attention_split_batch, out nv rows."""
        for t in (part_m, part_l, part_acc):
            _require(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32,
                     'workspace must be contiguous CUDA fp32')
        check_half(w, 'w')
        check_half(out, 'out')
        _require(1 <= nv <= MAX_BATCH, f'nv must be in [1, {MAX_BATCH}]')
        _require(w.dim() == 2 and w.size(1) == heads * HEAD_DIM == HIDDEN and out.numel() == nv * w.size(0),
                 'attn_out_gemv shape mismatch')
        if bias is not None:
            check_half(bias, 'bias')
        if len_state is not None:
            _require(len_state.dtype == torch.int64 and len_state.is_cuda, 'len_state must be CUDA int64')
        slots = min(part_m.numel(), part_l.numel(), part_acc.numel() // HEAD_DIM)
        args = (part_m.data_ptr(), part_l.data_ptr(), part_acc.data_ptr(), slots, _ptr(len_state), heads,
                int(max_len), int(split_keys), w.data_ptr(), _ptr(bias), out.data_ptr(), w.size(0))
        if nv == 1:
            self._call('fw_attn_out_gemv', *args, _stream())
        else:
            self._call('fw_attn_out_gemv_batch', *args, nv, _stream())

    # ---- the decoder layers of one token in one launch --------------------------------------
    def decoder_step_supported(self, n_layers, vocab, max_pos, enc_len, prompt=False):
        """(True, '') if the one-launch step (or, with `prompt`, the one-launch prompt pass) can run these
        sizes on the current device, else (False, the reason) (fw_decoder_step_check)."""
        st = self.lib.fw_decoder_step_check(int(n_layers), int(vocab), int(max_pos), int(enc_len), int(bool(prompt)))
        return (True, '') if st == _lib.FW_OK else (False, self.lib.fw_last_error().decode(errors='replace'))

    def decoder_step_workspace(self, n_layers):
        """Zero-filled workspace of fw_decoder_step_layers for n_layers (one per decoding stream), its
        hand-off pages placed for the device's two halves (fw_decoder_step_calibrate)."""
        nbytes = self.lib.fw_decoder_step_workspace_bytes(int(n_layers))
        _require(nbytes > 0, f'decoder_step: n_layers must be in [1, {self.lib.fw_decoder_step_max_layers()}]')
        ws = torch.zeros(nbytes, dtype=torch.uint8, device='cuda')
        self._call('fw_decoder_step_calibrate', ws.data_ptr(), nbytes, int(n_layers), _stream())
        return ws

    def decoder_step_calibrated(self, ws):
        """True if the workspace's hand-off pages were placed by a complete calibration (synchronises)."""
        st = self.lib.fw_decoder_step_calibrated(ws.data_ptr())
        _require(st >= 0, self.lib.fw_last_error().decode(errors='replace'))
        return st == 1

    def decoder_layer_table(self, layers):
        """The fw_dec_layer array for decoder_step_layers. `layers`: one dict per layer with the tensors
        named in _lib.DEC_LAYER_TENSORS (biases may be None), ln{1,2,3}_eps, and self_k / self_v
        ([heads, max_pos, 64]), cross_k / cross_v ([heads, enc_len, 64]). The table holds raw pointers:
        the tensors must outlive it."""
        table = (_lib.DecLayer * len(layers))()
        shapes = {'qkv_w': (3 * HIDDEN, HIDDEN), 'out_w': (HIDDEN, HIDDEN), 'cross_q_w': (HIDDEN, HIDDEN),
                  'cross_out_w': (HIDDEN, HIDDEN), 'fc1_w': (4 * HIDDEN, HIDDEN), 'fc2_w': (HIDDEN, 4 * HIDDEN)}
        rows = {'qkv_b': 3 * HIDDEN, 'fc1_b': 4 * HIDDEN}
        for i, lay in enumerate(layers):
            for name in _lib.DEC_LAYER_TENSORS:
                t = lay.get(name)
                if t is None:
                    _require(name.endswith('_b'), f'layer {i}: {name} is required')
                    continue
                check_half(t, f'layer {i} {name}')
                if name in shapes:
                    _require(tuple(t.shape) == shapes[name], f'layer {i}: {name} must be {list(shapes[name])}')
                else:
                    _require(t.numel() == rows.get(name, HIDDEN), f'layer {i}: {name} has the wrong size')
                setattr(table[i], name, t.data_ptr())
            for n in ('self_k', 'self_v', 'cross_k', 'cross_v'):
                t = lay[n]
                check_half(t, f'layer {i} {n}')
                _require(t.dim() == 3 and t.size(0) * HEAD_DIM == HIDDEN and t.size(2) == HEAD_DIM,
                         f'layer {i}: {n} must be [heads, len, 64]')
                setattr(table[i], n, t.data_ptr())
            _require(lay['self_k'].shape == lay['self_v'].shape and lay['cross_k'].shape == lay['cross_v'].shape,
                     f'layer {i}: K and V shapes differ')
            _require(lay['self_k'].shape == layers[0]['self_k'].shape
                     and lay['cross_k'].shape == layers[0]['cross_k'].shape, f'layer {i}: cache shapes differ')
            for j in (1, 2, 3):
                setattr(table[i], f'ln{j}_eps', float(lay[f'ln{j}_eps']))
        # the cache lengths, checked against max_pos / enc_len by every launch that takes the table
        table.self_len, table.cross_len = layers[0]['self_k'].size(1), layers[0]['cross_k'].size(1)
        return table

    @staticmethod
    def _check_table(table, max_pos, enc_len):
        _require(int(max_pos) <= table.self_len, f'max_pos {max_pos} exceeds the self-attention cache ({table.self_len})')
        _require(int(enc_len) == table.cross_len, f'enc_len {enc_len} differs from the cross K/V length ({table.cross_len})')

    @staticmethod
    def _check_head(head, vocab, embed, max_pos):
        _require(int(vocab) == head.vocab, f"vocab {vocab} differs from the LM head's rows ({head.vocab})")
        _require(embed.size(0) >= int(vocab), f'the embedding has {embed.size(0)} rows for a vocabulary of {vocab}')
        _require(head.tokens_len >= int(max_pos), f'the token list holds {head.tokens_len} ids, fewer than max_pos')

    def decoder_step_layers(self, table, cur, state, embed, pos_embed, max_pos, enc_len, scale, h_out, x_out, ws,
                            spin_limit=2_000_000):
        """Every decoder layer of one token in one launch (fw_decoder_step_layers): from the embedding of
        cur[0] at state[0] to the residual h_out and the last fc2 output x_out, K/V rows written at
        state[0]. Nothing else may run on the device meanwhile. A wait past spin_limit ticks (100 MHz)
        sets the workspace's error word; read it with decoder_step_error."""
        for t, n in ((embed, 'embed'), (pos_embed, 'pos_embed'), (h_out, 'h_out'), (x_out, 'x_out')):
            check_half(t, n)
        _require(embed.dim() == 2 and embed.size(1) == HIDDEN and pos_embed.dim() == 2 and pos_embed.size(1) == HIDDEN
                 and pos_embed.size(0) >= max_pos, 'embed / pos_embed must be [rows, 1280]')
        _require(h_out.numel() == HIDDEN and x_out.numel() == HIDDEN, 'h_out, x_out must be [1280]')
        self._check_table(table, max_pos, enc_len)
        for t, n in ((cur, 'cur'), (state, 'state')):
            _require(t.dtype == torch.int64 and t.is_cuda and t.is_contiguous(), f'{n} must be contiguous CUDA int64')
        _require(ws.dtype == torch.uint8 and ws.is_cuda and ws.is_contiguous(), 'workspace must be CUDA uint8')
        self._call('fw_decoder_step_layers', ctypes.addressof(table), len(table), cur.data_ptr(), state.data_ptr(),
                   embed.data_ptr(), pos_embed.data_ptr(), embed.size(0), int(max_pos), int(enc_len), float(scale),
                   h_out.data_ptr(), x_out.data_ptr(), ws.data_ptr(), ws.numel(), int(spin_limit), _stream())

    def final_layernorm(self, h, x, gamma, beta, y, eps):
        """The LM-head kernels' final LayerNorm (their reduction order): y = LN(fp16(h + x))."""
        for t, n in ((h, 'h'), (gamma, 'gamma'), (beta, 'beta'), (y, 'y')):
            check_half(t, n)
        if x is not None:
            check_half(x, 'x')
        _require(h.numel() == HIDDEN and y.numel() == HIDDEN, f'hidden size must be {HIDDEN}')
        self._call('fw_final_layernorm', h.data_ptr(), _ptr(x), gamma.data_ptr(), beta.data_ptr(), y.data_ptr(),
                   HIDDEN, float(eps), _stream())

    def host_tokens(self, n):
        """HostTokens: n int64 of device-coherent pinned host memory (fw_dec_head.host_tokens)."""
        return HostTokens(self.lib, n)

    def decoder_head(self, gamma, beta, eps, w, wq, meta, suppress, tokens, y_out=None, host_tokens=None, eos=()):
        """The fw_dec_head of decoder_step (raw pointers: the tensors and host_tokens must outlive it).
        eos: up to 4 end-of-text ids at which a launch stops (set_eos changes them later)."""
        for t, n in ((gamma, 'gamma'), (beta, 'beta'), (w, 'w')):
            check_half(t, n)
        _require(w.dim() == 2 and w.size(1) == HIDDEN, f'hidden size must be {HIDDEN}')
        _check(wq, 'wq', torch.int8, 'int8')
        _check(meta, 'meta', torch.float32, 'fp32')
        _require(tuple(wq.shape) == tuple(w.shape) and tuple(meta.shape) == (w.size(0), 2),
                 'wq must match w and meta be [vocab, 2]')
        _require(suppress.dtype == torch.bool and suppress.is_cuda and suppress.is_contiguous()
                 and suppress.numel() == w.size(0), 'suppress must be bool [vocab]')
        _check(tokens, 'tokens', torch.int64, 'int64')
        if y_out is not None:
            check_half(y_out, 'y_out')
            _require(y_out.numel() == HIDDEN, f'y_out must be [{HIDDEN}]')
        head = _lib.DecHead(gamma.data_ptr(), beta.data_ptr(), float(eps), w.data_ptr(), wq.data_ptr(), meta.data_ptr(),
                            suppress.data_ptr(), tokens.data_ptr(), _ptr(y_out),
                            host_tokens.address if host_tokens is not None else None)
        # checked against every launch that takes the head
        head.vocab, head.tokens_len = w.size(0), tokens.numel()
        self.set_eos(head, eos)
        return head

    @staticmethod
    def set_eos(head, eos):
        """The end-of-text ids a decoder_step launch stops at (at most 4)."""
        eos = [int(e) for e in eos]
        _require(len(eos) <= 4, 'at most 4 end-of-text ids')
        head.n_eos = len(eos)
        for i, e in enumerate(eos):
            head.eos[i] = e

    def decoder_step(self, table, head, cur, state, embed, pos_embed, max_pos, enc_len, scale, ws, vocab,
                     spin_limit=2_000_000, n_steps=1):
        """n_steps whole decoder steps in one launch (fw_decoder_step): each runs the layers of
        decoder_step_layers, then the final LN, the int8-pre-pass LM head, the argmax and the finalize
        (tokens, state and cur advance after every step)."""
        check_half(embed, 'embed')
        check_half(pos_embed, 'pos_embed')
        _require(pos_embed.size(0) >= int(max_pos), 'pos_embed has fewer rows than max_pos')
        self._check_table(table, max_pos, enc_len)
        self._check_head(head, vocab, embed, max_pos)
        for t, n in ((cur, 'cur'), (state, 'state')):
            _require(t.dtype == torch.int64 and t.is_cuda and t.is_contiguous(), f'{n} must be contiguous CUDA int64')
        _require(ws.dtype == torch.uint8 and ws.is_cuda and ws.is_contiguous(), 'workspace must be CUDA uint8')
        self._call('fw_decoder_step', ctypes.addressof(table), len(table), ctypes.addressof(head), int(n_steps),
                   cur.data_ptr(), state.data_ptr(), embed.data_ptr(), pos_embed.data_ptr(), int(vocab), int(max_pos), int(enc_len),
                   float(scale), ws.data_ptr(), ws.numel(), int(spin_limit), _stream())

    def decoder_prompt(self, table, head, prompt, cur, state, embed, pos_embed, max_pos, enc_len, scale, ws, vocab,
                       spin_limit=2_000_000):
        """The 4-token prompt pass in one launch (fw_decoder_prompt): the cache rows, state, cur and first
        token of 4 steps whose first 3 predictions are discarded."""
        check_half(embed, 'embed')
        check_half(pos_embed, 'pos_embed')
        _require(pos_embed.size(0) >= int(max_pos), 'pos_embed has fewer rows than max_pos')
        self._check_table(table, max_pos, enc_len)
        self._check_head(head, vocab, embed, max_pos)
        for t, n in ((prompt, 'prompt'), (cur, 'cur'), (state, 'state')):
            _require(t.dtype == torch.int64 and t.is_cuda and t.is_contiguous(), f'{n} must be contiguous CUDA int64')
        _require(ws.dtype == torch.uint8 and ws.is_cuda and ws.is_contiguous(), 'workspace must be CUDA uint8')
        self._call('fw_decoder_prompt', ctypes.addressof(table), len(table), ctypes.addressof(head), prompt.data_ptr(),
                   prompt.numel(), cur.data_ptr(), state.data_ptr(), embed.data_ptr(), pos_embed.data_ptr(),
                   int(vocab), int(max_pos), int(enc_len), float(scale), ws.data_ptr(), ws.numel(), int(spin_limit),
                   _stream())

    @staticmethod
    def decoder_step_error(ws, clear=True):
        """The workspace's error word (nonzero: a wait of the step timed out); synchronises."""
        word = ws[8:12].view(torch.int32)
        err = int(word.item())
        if err and clear:
            word.zero_()
        return err

    def lm_head_argmax_fused(self, h, x, gamma, beta, eps, w, suppress, best, tokens, state, cur, max_pos):
        """Final residual + LN + lm_head_argmax + argmax_finalize (finalize skipped when tokens, state and
        cur are all None)."""
        for t, n in ((h, 'h'), (gamma, 'gamma'), (beta, 'beta'), (w, 'w')):
            check_half(t, n)
        if x is not None:
            check_half(x, 'x')
        _require(w.dim() == 2 and w.size(1) == HIDDEN, f'hidden size must be {HIDDEN}')
        _require(suppress.dtype == torch.bool and suppress.is_cuda and suppress.numel() == w.size(0),
                 'suppress must be bool [vocab]')
        fin = (tokens, state, cur)
        _require(all(t is None for t in fin) or all(t is not None for t in fin),
                 'tokens, state and cur must be given together')
        for t in (best,) + tuple(t for t in fin if t is not None):
            _require(t.dtype == torch.int64 and t.is_cuda and t.is_contiguous(), 'tokens, state and cur must be int64')
        self._call('fw_lm_head_argmax_fused', h.data_ptr(), _ptr(x), gamma.data_ptr(), beta.data_ptr(), float(eps),
                   w.data_ptr(), suppress.data_ptr(), w.size(0), HIDDEN, best.data_ptr(), _ptr(tokens),
                   _ptr(state), _ptr(cur), int(max_pos), _stream())

    def lm_head_q8_table(self, w):
        """Allocates and fills the int8 table of w for lm_head_argmax_q8 (init time): (wq, meta)."""
        wq = torch.empty(w.size(0), HIDDEN, dtype=torch.int8, device=w.device)
        meta = torch.empty(w.size(0), 2, dtype=torch.float32, device=w.device)
        self.lm_head_q8_pack(w, wq, meta)
        return wq, meta

    def lm_head_q8_pack(self, w, wq, meta):
        """Fills wq int8 [vocab, 1280] and meta fp32 [vocab, 2] (scale, error bound) from w."""
        check_half(w, 'w')
        _require(w.dim() == 2 and w.size(1) == HIDDEN, f'hidden size must be {HIDDEN}')
        vocab = w.size(0)
        _check(wq, 'wq', torch.int8, 'int8')
        _check(meta, 'meta', torch.float32, 'fp32')
        _require(tuple(wq.shape) == (vocab, HIDDEN) and tuple(meta.shape) == (vocab, 2),
                 'wq must be [vocab, 1280] and meta [vocab, 2]')
        self._call('fw_lm_head_q8_pack', w.data_ptr(), vocab, HIDDEN, wq.data_ptr(), meta.data_ptr(), _stream())
        return wq, meta

    def lm_head_argmax_q8(self, h, x, gamma, beta, eps, w, wq, meta, suppress, best, tokens, state, cur, max_pos):
        """lm_head_argmax_fused with the same result, bit for bit, from the int8 table (wq, meta) of w."""
        for t, n in ((h, 'h'), (gamma, 'gamma'), (beta, 'beta'), (w, 'w')):
            check_half(t, n)
        if x is not None:
            check_half(x, 'x')
        _require(w.dim() == 2 and w.size(1) == HIDDEN, f'hidden size must be {HIDDEN}')
        _check(wq, 'wq', torch.int8, 'int8')
        _check(meta, 'meta', torch.float32, 'fp32')
        _require(tuple(wq.shape) == tuple(w.shape) and tuple(meta.shape) == (w.size(0), 2),
                 'wq must match w and meta be [vocab, 2]')
        _require(suppress.dtype == torch.bool and suppress.is_cuda and suppress.numel() == w.size(0),
                 'suppress must be bool [vocab]')
        fin = (tokens, state, cur)
        _require(all(t is None for t in fin) or all(t is not None for t in fin),
                 'tokens, state and cur must be given together')
        for t in (best,) + tuple(t for t in fin if t is not None):
            _require(t.dtype == torch.int64 and t.is_cuda and t.is_contiguous(), 'tokens, state and cur must be int64')
        self._call('fw_lm_head_argmax_q8', h.data_ptr(), _ptr(x), gamma.data_ptr(), beta.data_ptr(), float(eps),
                   w.data_ptr(), wq.data_ptr(), meta.data_ptr(), suppress.data_ptr(), w.size(0), HIDDEN,
                   best.data_ptr(), _ptr(tokens), _ptr(state), _ptr(cur), int(max_pos), _stream())

    # ---- log-mel front end -------------------------------------------------------------
    def log_mel_workspace(self, n_samples, device='cuda'):
        return torch.empty(int(self.lib.fw_log_mel_ws_floats(int(n_samples))), dtype=torch.float32, device=device)

    def _log_mel_checks(self, wave, filters, out, out16, ws):
        _check(wave, 'wave', torch.float32, 'fp32')
        _check(filters, 'filters', torch.float32, 'fp32')
        _check(out, 'out', torch.float32, 'fp32')
        _check(ws, 'ws', torch.float32, 'fp32')
        n_frames = wave.numel() // 160
        _require(filters.shape == (201, 128), 'filters must be [201, 128]')
        _require(out.numel() == 128 * n_frames, f'out must be [128, {n_frames}]')
        if out16 is not None:
            check_half(out16, 'out16')
            _require(out16.numel() == 128 * n_frames, f'out16 must be [{n_frames}, 128]')

    def log_mel(self, wave, filters, out, out16, ws):
        """Log-mel of one clip: log_mel_prepare then log_mel_run."""
        self._log_mel_checks(wave, filters, out, out16, ws)
        self._call('fw_log_mel', wave.data_ptr(), wave.numel(), filters.data_ptr(), out.data_ptr(), _ptr(out16),
                   ws.data_ptr(), ws.numel(), _stream())

    def wave_upload(self, audio, staging, wave, chunk=WAVE_CHUNK):
        """audio (1-D float32 NumPy array) -> wave[:audio.size], zeros after it, through the pinned
        ``staging`` tensor in chunks whose copies start as each is staged (custom/model.py:103-104)."""
        _require(isinstance(audio, np.ndarray) and audio.dtype == np.float32 and audio.ndim == 1,
                 'audio must be a one-dimensional float32 NumPy array')
        _check(wave, 'wave', torch.float32, 'fp32')
        _require(staging.dtype == torch.float32 and staging.is_pinned() and staging.is_contiguous(),
                 'staging must be a contiguous pinned fp32 host tensor')
        _require(0 < audio.size <= min(staging.numel(), wave.numel()), 'audio must fit staging and wave')
        audio = np.ascontiguousarray(audio)
        self._call('fw_wave_upload', audio.ctypes.data, audio.size, staging.data_ptr(), wave.data_ptr(), wave.numel(),
                   int(chunk), _stream())

    def log_mel_prepare(self, filters, ws):
        """Writes the FFT twiddles and the compacted filterbank of ``filters`` to the start of ``ws``."""
        _check(filters, 'filters', torch.float32, 'fp32')
        _check(ws, 'ws', torch.float32, 'fp32')
        _require(filters.shape == (201, 128), 'filters must be [201, 128]')
        self._call('fw_log_mel_prepare', filters.data_ptr(), ws.data_ptr(), ws.numel(), _stream())

    def log_mel_run(self, wave, filters, out, out16, ws):
        """Log-mel of one clip on a workspace that log_mel_prepare filled from the same ``filters``."""
        self._log_mel_checks(wave, filters, out, out16, ws)
        self._call('fw_log_mel_run', wave.data_ptr(), wave.numel(), filters.data_ptr(), out.data_ptr(), _ptr(out16),
                   ws.data_ptr(), ws.numel(), _stream())

    # ---- encoder ---------------------------------------------------------------------------
    def gemm(self, a, w, bias, out, epilogue=EPI_BIAS, res=None, q_cols=0):
        """out[m, n] = epilogue(a[m, :k] . w[n, :k]); a, out, res may be row-strided 2-D views."""
        for t, n in ((a, 'a'), (w, 'w'), (out, 'out')):
            _require(t.is_cuda and t.dtype == torch.float16 and t.dim() == 2 and t.stride(1) == 1,
                     f'{n} must be a 2-D CUDA fp16 tensor with unit column stride')
        m, k = a.shape
        n = w.size(0)
        _require(w.size(1) == k and out.shape == (m, n), 'gemm shape mismatch')
        if bias is not None:
            check_half(bias, 'bias')
        ldr = 0
        if res is not None:
            _require(res.is_cuda and res.dtype == torch.float16 and res.shape == (m, n) and res.stride(1) == 1,
                     'res must be [m, n] CUDA fp16')
            ldr = res.stride(0)
        self._call('fw_gemm', a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), _ptr(bias), out.data_ptr(),
                   out.stride(0), _ptr(res), ldr, m, n, k, epilogue, q_cols, _stream())

    def conv1d(self, x, stride, wp, bias, out, epilogue, res=None):
        check_half(x, 'x')
        check_half(wp, 'wp')
        check_half(out, 'out')
        t_in, c_in = x.shape
        c_out = wp.size(0)
        _require(wp.shape == (c_out, 3 * c_in), 'wp must be [c_out, 3 * c_in]')
        _require(out.shape == ((t_in - 1) // stride + 1, c_out), 'out shape mismatch')
        if res is not None:
            check_half(res, 'res')
            _require(res.shape == out.shape, 'res must match out')
        self._call('fw_conv1d', x.data_ptr(), t_in, c_in, stride, wp.data_ptr(), _ptr(bias), out.data_ptr(), c_out,
                   _ptr(res), epilogue, _stream())

    def layernorm_rows(self, x, gamma, beta, y, eps):
        for t, n in ((x, 'x'), (gamma, 'gamma'), (beta, 'beta'), (y, 'y')):
            check_half(t, n)
        _require(x.dim() == 2 and x.size(1) == HIDDEN and y.shape == x.shape, 'layernorm_rows shape mismatch')
        self._call('fw_layernorm_rows', x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), y.data_ptr(), x.size(0),
                   HIDDEN, float(eps), _stream())

    def gemm_splitk(self, a, w, part, splits=2):
        """part[s] <- the fp32 product of a and w^T over the s-th k half (a [m, k], w [n, k], part [2, m, n])."""
        check_half(a, 'a')
        check_half(w, 'w')
        _check(part, 'part', torch.float32, 'float32')
        m, k = a.shape
        n = w.size(0)
        _require(a.dim() == 2 and w.dim() == 2 and w.size(1) == k and part.shape == (splits, m, n),
                 'gemm_splitk shape mismatch')
        self._call('fw_gemm_splitk', a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), part.data_ptr(), m, n, k,
                   int(splits), _stream())

    def layernorm_rows_residual(self, part, bias, h, gamma, beta, y, eps, epilogue):
        """h <- residual epilogue(part[0] + part[1], bias) in place, then y <- LN(h) (part from gemm_splitk)."""
        for t, n in ((bias, 'bias'), (h, 'h'), (gamma, 'gamma'), (beta, 'beta'), (y, 'y')):
            check_half(t, n)
        _check(part, 'part', torch.float32, 'float32')
        rows = h.size(0)
        _require(h.dim() == 2 and h.size(1) == HIDDEN and y.shape == h.shape and part.shape == (2, rows, HIDDEN),
                 'layernorm_rows_residual shape mismatch')
        self._call('fw_layernorm_rows_residual', part.data_ptr(), 2, bias.data_ptr(), h.data_ptr(), gamma.data_ptr(),
                   beta.data_ptr(), y.data_ptr(), rows, HIDDEN, float(eps), int(epilogue), _stream())

    def encoder_vt_workspace(self, seq, heads):
        """Transposed-V buffer for encoder_qkv / encoder_pack_vt / encoder_attention (layout private)."""
        n = self.lib.fw_encoder_vt_elems(seq, heads)
        _require(n > 0, 'encoder_vt_workspace: seq and heads must be positive')
        return torch.zeros(n, dtype=torch.float16, device='cuda')

    def _check_vt(self, vt, seq, heads):
        check_half(vt, 'vt')
        _require(vt.numel() == self.lib.fw_encoder_vt_elems(seq, heads), 'vt must hold fw_encoder_vt_elems(seq, heads)')

    def encoder_qkv(self, y, w, bias, qkv, vt, heads):
        """q/k/v projection of an encoder layer: q (scaled by 1/8) and k into qkv, v into vt."""
        for t, n in ((y, 'y'), (w, 'w'), (qkv, 'qkv')):
            check_half(t, n)
        seq, d = y.shape
        _require(d == heads * HEAD_DIM and w.shape == (3 * d, d) and qkv.shape == (seq, 3 * d),
                 'encoder_qkv shape mismatch')
        if bias is not None:
            check_half(bias, 'bias')
        self._check_vt(vt, seq, heads)
        self._call('fw_encoder_qkv', y.data_ptr(), w.data_ptr(), _ptr(bias), qkv.data_ptr(), vt.data_ptr(), seq, heads,
                   _stream())

    def encoder_pack_vt(self, qkv, vt, heads):
        check_half(qkv, 'qkv')
        seq = qkv.size(0)
        _require(qkv.shape == (seq, 3 * heads * HEAD_DIM), 'encoder_pack_vt shape mismatch')
        self._check_vt(vt, seq, heads)
        self._call('fw_encoder_pack_vt', qkv.data_ptr(), vt.data_ptr(), seq, heads, _stream())

    def encoder_attention(self, qkv, vt, out, heads):
        check_half(qkv, 'qkv')
        check_half(out, 'out')
        seq = qkv.size(0)
        _require(qkv.shape == (seq, 3 * heads * HEAD_DIM) and out.shape == (seq, heads * HEAD_DIM),
                 'encoder_attention shape mismatch')
        self._check_vt(vt, seq, heads)
        self._call('fw_encoder_attention', qkv.data_ptr(), vt.data_ptr(), out.data_ptr(), seq, heads, _stream())

    def cross_kv(self, enc, w, bias, cross_kv):
        check_half(enc, 'enc')
        check_half(w, 'w')
        check_half(cross_kv, 'cross_kv')
        layers, _, heads, t, _ = cross_kv.shape
        _require(enc.shape == (t, HIDDEN) and w.shape == (layers * 2 * HIDDEN, HIDDEN), 'cross_kv shape mismatch')
        if bias is not None:
            check_half(bias, 'bias')
        self._call('fw_cross_kv', enc.data_ptr(), t, w.data_ptr(), _ptr(bias), cross_kv.data_ptr(), layers, heads,
                   _stream())


_ext = None


def load_ext(verbose=False):
    """Returns the extension object (custom/ext.py:13). Raises if the library has not been built."""
    global _ext
    if _ext is None:
        if verbose:
            print(f'loading {_lib.LIB_PATH}', file=sys.stderr)
        _ext = WhisperExt()
    return _ext


def main():
    from . import build as build_mod

    parser = argparse.ArgumentParser(description='Build the HIP library and print per-kernel resource usage.')
    parser.parse_args()
    lib = build_mod.build()
    for line in build_mod.resource_usage():
        if any(k in line for k in ('Function Name', 'VGPRs', 'Spill', 'LDS Size', 'Occupancy')):
            print(line.split('remark: ')[-1].replace(' [-Rpass-analysis=kernel-resource-usage]', ''))
    print(f'built: [{lib}]')


if __name__ == '__main__':
    main()

"""The decoder step as one persistent launch against the 34-launch step of the same weights: the layers
alone (fw_decoder_step_layers: K/V cache, residual, last fc2 output) and the whole step with the final
LayerNorm, int8-pre-pass LM head, argmax and finalize (fw_decoder_step: K/V cache, final LayerNorm
output, token list, state, current token), bit-identical after every step, at positions across the
self-attention split boundaries and up to the end of the cache; the error word after a flagged wait.
The 224-id oracle fixture runs through the one-launch step in tests/test_gpu_model.py (it is the
model's default)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def model(hip_device):
    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.model import CustomModel

    m = CustomModel(seed=0, selftest=False, capture=False)
    m.transcribe(synthetic_clip(0), max_new_tokens=1, stop_at_eos=False)  # fills the cross K/V
    return m


def _start(model, pos, cur, kv0):
    model.self_kv.copy_(kv0)
    model.state.copy_(torch.tensor([pos, 0], device='cuda'))
    model.cur.fill_(cur)
    model.tokens.zero_()
    model.best.zero_()


def _run(model, persistent, pos, cur, kv0, steps):
    """`steps` steps from position pos with cache kv0, the persistent form without its LM head; per step
    the tensors both step forms produce."""
    model.persistent_step = persistent
    model.persistent_head = False
    model.self_kv.copy_(kv0)
    model.state.copy_(torch.tensor([pos, 0], device='cuda'))
    model.cur.fill_(cur)
    model.tokens.zero_()
    model.best.zero_()
    out = []
    b = (model.dims.dec_layers - 1) % 2  # the 32-launch step's final residual buffer (layer l writes h[l % 2])
    for _ in range(steps):
        model._step()
        h, x = (model.h_fin, model.x_fin) if persistent else (model.h[b], model.pending)
        out.append([t.clone() for t in (model.self_kv, h, x, model.tokens, model.state, model.cur)])
    torch.cuda.synchronize()
    model.persistent_head = True
    return out


def _run_full(model, persistent, pos, cur, kv0, steps, y):
    """`steps` whole steps (LM head included); per step the cache, the final LayerNorm output (written
    by the one-launch step into y, recomputed for the launch chain with the LM-head kernels' final
    LayerNorm), tokens, state and current token."""
    model.persistent_step = persistent
    _start(model, pos, cur, kv0)
    b = (model.dims.dec_layers - 1) % 2
    g, be, eps = model.final_ln
    out = []
    for _ in range(steps):
        model._step()
        if not persistent:
            model.ext.final_layernorm(model.h[b], model.pending, g, be, y, eps)
        out.append([t.clone() for t in (model.self_kv, y, model.tokens, model.state, model.cur)])
    torch.cuda.synchronize()
    return out


@torch.inference_mode()
@pytest.mark.parametrize('pos', [0, 60, 126, 250, 440])
def test_persistent_step_matches_launch_chain(model, pos):
    g = torch.Generator(device='cuda').manual_seed(pos)
    kv0 = (torch.randn(model.self_kv.shape, generator=g, device='cuda') * 0.7).half()
    steps = min(6, model.max_pos - pos)
    names = ('self_kv', 'h', 'x', 'tokens', 'state', 'cur')
    try:
        ref = _run(model, False, pos, 1234, kv0, steps)
        got = _run(model, True, pos, 1234, kv0, steps)
    finally:
        model.persistent_step = True
    assert model.ext.decoder_step_error(model.step_ws) == 0
    for s, (a, b) in enumerate(zip(got, ref)):
        for name, ta, tb in zip(names, a, b):
            assert torch.equal(ta, tb), f'step {s} (position {pos + s}): {name} differs'


@torch.inference_mode()
@pytest.mark.parametrize('pos', [0, 60, 126, 250, 443])
def test_one_launch_step_matches_launch_chain(model, pos):
    """The whole step in one launch: the LM head's int8 pre-pass, fp16 rescoring, block maxima and
    finalize inside the persistent kernel pick the chain's token at every step; from the last start
    position the steps reach the cache's last row, where the finalize holds the position."""
    g = torch.Generator(device='cuda').manual_seed(1000 + pos)
    kv0 = (torch.randn(model.self_kv.shape, generator=g, device='cuda') * 0.7).half()
    steps = 6
    y = torch.zeros(model.dims.d_model, dtype=torch.float16, device='cuda')
    names = ('self_kv', 'final LN', 'tokens', 'state', 'cur')
    try:
        model._make_step_head(y)
        got = _run_full(model, True, pos, 1234, kv0, steps, y)
        ref = _run_full(model, False, pos, 1234, kv0, steps, y)
    finally:
        model.persistent_step = True
        model._make_step_head()
    assert model.ext.decoder_step_error(model.step_ws) == 0
    for s, (a, b) in enumerate(zip(got, ref)):
        for name, ta, tb in zip(names, a, b):
            assert torch.equal(ta, tb), f'step {s} (position {pos + s}): {name} differs'
    assert int(got[-1][3][1]) == steps and int(got[-1][3][0]) == min(pos + steps, model.max_pos - 1)
    toks = got[-1][2][:steps]
    assert int(toks.min()) >= 0 and int(toks.max()) < model.dims.vocab


@torch.inference_mode()
@pytest.mark.parametrize('pos,steps', [(0, 8), (120, 8), (437, 12)])
def test_multi_step_launch_matches_launch_chain(model, pos, steps):
    """Several steps in one launch (each step takes the previous one's token and position from the
    finalizing block's broadcast, and the self-attention blocks read back cache rows written earlier in
    the same launch) against as many 34-launch steps: cache, final LayerNorm output of the last step,
    tokens, state and current token bit-identical; from position 437 the steps run into the cache's
    last row and stay there."""
    g = torch.Generator(device='cuda').manual_seed(2000 + pos)
    kv0 = (torch.randn(model.self_kv.shape, generator=g, device='cuda') * 0.7).half()
    y = torch.zeros(model.dims.d_model, dtype=torch.float16, device='cuda')
    try:
        model._make_step_head(y)
        ref = _run_full(model, False, pos, 4321, kv0, steps, y)[-1]
        model.persistent_step = True
        _start(model, pos, 4321, kv0)
        model._steps(steps)
        torch.cuda.synchronize()
        got = [t.clone() for t in (model.self_kv, y, model.tokens, model.state, model.cur)]
    finally:
        model.persistent_step = True
        model._make_step_head()
    assert model.ext.decoder_step_error(model.step_ws) == 0
    for name, ta, tb in zip(('self_kv', 'final LN', 'tokens', 'state', 'cur'), got, ref):
        assert torch.equal(ta, tb), f'{steps} steps from position {pos}: {name} differs'
    assert int(got[3][1]) == steps


@torch.inference_mode()
def test_persistent_step_repeats_exactly(model):
    """Two runs of the same steps (the epoch moves on every launch) give the same bits."""
    g = torch.Generator(device='cuda').manual_seed(7)
    kv0 = (torch.randn(model.self_kv.shape, generator=g, device='cuda') * 0.7).half()
    a = _run(model, True, 100, 4242, kv0, 4)
    b = _run(model, True, 100, 4242, kv0, 4)
    for x, y in zip(a, b):
        for ta, tb in zip(x, y):
            assert torch.equal(ta, tb)


@torch.inference_mode()
def test_flagged_error_ends_waits_and_is_reported(model):
    """A step launched with the error word already set stops waiting after a few polls and completes;
    the word stays set, transcribe-level checks raise, and reading it clears it."""
    ws = model.step_ws
    word = ws[8:12].view(torch.int32)
    word.fill_(1)
    model.state.copy_(torch.tensor([10, 0], device='cuda'))
    model.cur.fill_(50)
    model._step()
    torch.cuda.synchronize()
    assert int(word.item()) == 1
    with pytest.raises(RuntimeError, match='timed out'):
        model._check_step_error()
    assert int(word.item()) == 0
    # the next steps are valid again
    kv0 = torch.zeros_like(model.self_kv)
    ref = _run(model, False, 3, 77, kv0, 2)
    got = _run(model, True, 3, 77, kv0, 2)
    model.persistent_step = True
    for x, y in zip(got, ref):
        for ta, tb in zip(x, y):
            assert torch.equal(ta, tb)


@torch.inference_mode()
def test_flagged_transcribe_falls_back_to_launch_chain(model):
    """transcribe with the error word set before it starts: the persistent prompt pass and decode stop
    waiting at once and their tokens are discarded; the clip is decoded again on the 34-launch step in
    the same call, which gives the oracle fixture's 224 ids and reports decode_fallback; the word is
    clear afterwards and the next call runs the persistent step again (custom/model.py:149-171,189-192
    falls back to eager execution the same way when its graph capture fails)."""
    import json

    from conftest import GOLDEN
    from flash_whisper_amd.audio import synthetic_clip

    fx = json.loads((GOLDEN / 'e2e_turbo_seed0.json').read_text())
    clip = synthetic_clip(0)
    word = model.step_ws[8:12].view(torch.int32)
    word.fill_(1)
    res = model.transcribe(clip, max_new_tokens=fx['n_tokens'], stop_at_eos=False)
    assert res['decode_fallback'] is True
    assert res['token_ids'] == fx['ids']
    assert int(word.item()) == 0 and model.persistent_step
    res = model.transcribe(clip, max_new_tokens=fx['n_tokens'], stop_at_eos=False)
    assert res['decode_fallback'] is False and res['token_ids'] == fx['ids']



@torch.inference_mode()
def test_streamed_decode_matches_chunked_decode(model):
    """transcribe's whole decode as one launch, its tokens polled from host memory as they are stored,
    gives the ids of the chunked decode (8-step launches, tokens copied after each chunk): 224 fixed
    tokens, and with an end-of-text id the launch stops itself at its first occurrence."""
    from flash_whisper_amd.audio import synthetic_clip

    clip = synthetic_clip(0)
    saved = model.eos
    try:
        model.stream_decode = False
        ref = model.transcribe(clip, max_new_tokens=224, stop_at_eos=False)['token_ids']
        model.stream_decode = True
        got = model.transcribe(clip, max_new_tokens=224, stop_at_eos=False)['token_ids']
        assert got == ref
        model.eos = {ref[30], ref[50]}  # the launch stops at the first of them
        first = min(ref.index(ref[30]), ref.index(ref[50]))
        got = model.transcribe(clip)['token_ids']
        assert got == ref[:first + 1]
        assert int(model.state[1]) == first + 1  # the device stopped there too
    finally:
        model.eos = saved
        model.stream_decode = True
    assert model.ext.decoder_step_error(model.step_ws) == 0


@torch.inference_mode()
@pytest.mark.parametrize('pos', [0, 100, 444])
def test_prompt_pass_in_one_launch_matches_batched_launches(model, pos):
    """The 4-token prompt pass as one persistent launch (every phase on 4 vectors; the self attention of
    position pos + z sees the fresh K/V rows of positions pos .. pos + z) against the batched
    34-launch pass: the whole cache, tokens, state and current token bit-identical, from the start of
    the cache, from a filled cache and up to its last row."""
    g = torch.Generator(device='cuda').manual_seed(3000 + pos)
    kv0 = (torch.randn(model.self_kv.shape, generator=g, device='cuda') * 0.7).half()
    first = model.first_mask.clone()

    def run():
        out = []
        try:
            for persistent in (False, True):
                model.persistent_prompt = persistent
                _start(model, pos, 4321, kv0)
                if not persistent:  # the batched launches read the decode mask, set to the first step's
                    model.suppress.copy_(model.first_mask)
                model._prefill()
                model.suppress.copy_(model.base_mask)
                torch.cuda.synchronize()
                out.append([t.clone() for t in (model.self_kv, model.tokens, model.state, model.cur)])
        finally:
            model.persistent_prompt = True
        assert model.ext.decoder_step_error(model.step_ws) == 0
        for name, ta, tb in zip(('self_kv', 'tokens', 'state', 'cur'), out[1], out[0]):
            assert torch.equal(ta, tb), f'prompt at position {pos}: {name} differs'
        assert out[1][2].tolist() == [min(pos + 4, model.max_pos - 1), 1]
        return int(out[1][3])

    try:
        tok = run()
        model.first_mask[tok] = True  # the one-launch pass reads the first step's mask itself
        assert run() != tok
    finally:
        model.first_mask.copy_(first)


@torch.inference_mode()
def test_hand_off_pages_calibrated(model):
    """fw_decoder_step_calibrate measured every logical page of the model's workspace: one bit per
    logical page, the half of the device its first physical page is local to. Memory alternates between
    the I/O dies every 8 KB within each 2 MB page, so the first pages of the 16 KB groups in one 2 MB page
    all sit on the same die: their bits agree."""
    ext, ws = model.ext, model.step_ws
    assert ext.decoder_step_calibrated(ws)
    n_pages = -(-(model.dims.dec_layers * 4 * 18880 + 2 * 1024 + 8) // 1024)
    words = ws[256:512].cpu().view(torch.int32)
    bits = [bool((int(words[j // 32]) >> (j % 32)) & 1) for j in range(n_pages)]
    area = (ws.data_ptr() + 256 + 256 + 2 * 2048 * 4 + 16383) // 16384 * 16384
    regions = {}
    for j, b in enumerate(bits):
        regions.setdefault((area + j * 16384) >> 21, []).append(b)
    for r, bs in regions.items():
        agree = max(bs.count(True), bs.count(False)) / len(bs)
        assert agree > 0.9, (r, bs)


@torch.inference_mode()
def test_decode_independent_of_page_placement(model):
    """The placement only decides which copy a block polls: with the group bits cleared (as in a workspace
    never calibrated) and inverted (every block polling the copy on the other half's memory), the decode
    gives the same 224 ids."""
    from flash_whisper_amd.audio import synthetic_clip

    clip = synthetic_clip(0)
    ws = model.step_ws
    saved = ws[256:512].clone()
    ref = model.transcribe(clip, max_new_tokens=224, stop_at_eos=False)['token_ids']
    try:
        for fill in (0, 255):
            ws[256:512].fill_(fill)
            res = model.transcribe(clip, max_new_tokens=224, stop_at_eos=False)
            assert res['token_ids'] == ref and res['decode_fallback'] is False, fill
    finally:
        ws[256:512].copy_(saved)
    assert model.ext.decoder_step_error(ws) == 0

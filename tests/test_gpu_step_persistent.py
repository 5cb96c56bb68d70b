"""The decoder layers of a step as one persistent launch (fw_decoder_step_layers) against the 32-launch
step of the same layers: K/V cache, residual, last fc2 output, token, state and current token
bit-identical after every step, at positions across the self-attention split boundaries and up to the
end of the cache; the error word after a flagged wait. The 224-id oracle fixture runs through the
persistent step in tests/test_gpu_model.py (it is the model's default)."""

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


def _run(model, persistent, pos, cur, kv0, steps):
    """`steps` steps from position pos with cache kv0; per step the tensors both step forms produce."""
    model.persistent_step = persistent
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


"""Several clips in flight on separate lanes and streams (flash_whisper_amd.serve) must produce exactly
the token ids of one-at-a-time CustomModel.transcribe, in fixed-length and EOS-stopping modes; in
fixed-length mode the seeded clip 0 must give the oracle's ids (tests/golden/e2e_turbo_seed0.json)."""

import json

import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def model(hip_device):
    from flash_whisper_amd.model import CustomModel

    return CustomModel(seed=0, selftest=False)


@pytest.mark.parametrize('lanes,stop_at_eos', [(2, False), (3, True)])
def test_lanes_match_sequential_transcribe(model, lanes, stop_at_eos):
    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.serve import Scheduler

    clips = [synthetic_clip(s) for s in (0, 1, 2, 3)]
    clips[3] = clips[3][:5 * 16000]  # a short clip too
    saved = set(model.eos)
    try:
        if stop_at_eos:  # an EOS that the first clip produces at its 13th token, so that clip stops early
            first = model.transcribe(clips[0], max_new_tokens=30, stop_at_eos=False)['token_ids']
            model.eos.clear()
            model.eos.add(first[12])  # in place: the lanes share this set
        ref = [model.transcribe(c, max_new_tokens=30, stop_at_eos=stop_at_eos)['token_ids'] for c in clips]
        if stop_at_eos:
            assert len(ref[0]) <= 13 and ref[0][-1] in model.eos
        sched = Scheduler(model, lanes=lanes)
        out = sched.transcribe_many(clips, max_new_tokens=30, stop_at_eos=stop_at_eos)
        if not stop_at_eos:
            fx = json.loads((GOLDEN / 'e2e_turbo_seed0.json').read_text())
            assert out[0]['token_ids'] == fx['ids'][:30]
        assert [r['token_ids'] for r in out] == ref
        assert all(r['wall_s'] >= r['e2e_s'] > 0 for r in out)
        # the lanes stay usable one at a time
        assert sched.lanes[-1].transcribe(clips[0], max_new_tokens=30, stop_at_eos=stop_at_eos)['token_ids'] == ref[0]
    finally:
        model.eos.clear()
        model.eos.update(saved)

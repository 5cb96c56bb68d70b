"""A local checkpoint directory (config.json, model.safetensors, generation_config.json, tokenizer.json)
written from the seeded turbo weights must give the oracle's greedy ids for the seeded clip
(tests/golden/e2e_turbo_seed0.json), with the prompt and suppress ids taken from those files and the
text from the tokenizer. The same weights with the decoder scaled (tests/weights_varied.py), whose
greedy ids vary from step to step (62 distinct), must give the oracle's 224 ids of that model
(tests/golden/e2e_turbo_seed0_varied.json) bit for bit."""

import json

from conftest import GOLDEN

import pytest
import torch

from test_checkpoint import hf_config, special_tokenizer

pytestmark = pytest.mark.gpu
N_TOKENS = 24


def _write_checkpoint(root, arrays):
    from safetensors.torch import save_file

    from flash_whisper_amd.config import (BEGIN_SUPPRESS_IDS, EOS_IDS, PROMPT_IDS, SUPPRESS_IDS, TURBO)

    params = {n: torch.from_numpy(a) for n, a in arrays.items()}
    save_file(params, str(root / 'model.safetensors'))
    del params
    cfg = hf_config(TURBO)
    cfg['eos_token_id'] = EOS_IDS[0]
    (root / 'config.json').write_text(json.dumps(cfg))
    (root / 'generation_config.json').write_text(json.dumps(
        {'eos_token_id': EOS_IDS[0], 'suppress_tokens': list(SUPPRESS_IDS),
         'begin_suppress_tokens': list(BEGIN_SUPPRESS_IDS)}))
    names = ('<|startoftranscript|>', '<|en|>', '<|transcribe|>', '<|notimestamps|>')
    specials = dict(zip(names, PROMPT_IDS))
    specials['<|endoftext|>'] = EOS_IDS[0]
    special_tokenizer(TURBO.vocab, specials).save(str(root / 'tokenizer.json'))
    return root


@pytest.fixture(scope='module')
def checkpoint_dir(tmp_path_factory):
    from flash_whisper_amd import weights as W
    from flash_whisper_amd.config import TURBO

    return _write_checkpoint(tmp_path_factory.mktemp('turbo_ckpt'), W.host_params(TURBO, seed=0))


def test_checkpoint_model_matches_synthetic(checkpoint_dir, hip_device):
    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.config import PROMPT_IDS
    from flash_whisper_amd.model import CustomModel

    fx = json.loads((GOLDEN / 'e2e_turbo_seed0.json').read_text())
    clip = synthetic_clip(0)
    m = CustomModel(str(checkpoint_dir), None, selftest=False)
    assert m.checkpoint == str(checkpoint_dir) and tuple(m.prompt) == PROMPT_IDS
    assert m.setup.suppress == tuple(fx['suppress']) and m.setup.begin_suppress == tuple(fx['begin_suppress'])
    out = m.transcribe(clip, max_new_tokens=N_TOKENS, stop_at_eos=False)
    assert out['token_ids'] == fx['ids'][:N_TOKENS]
    words = [f'w{i}' for i in out['token_ids'] if i < 50257]
    assert out['text'] == ' '.join(words)


@torch.inference_mode()
def test_varied_checkpoint_matches_oracle_ids(tmp_path_factory, hip_device):
    import gc

    from flash_whisper_amd import weights as W
    from flash_whisper_amd.audio import sha256, synthetic_clip
    from flash_whisper_amd.config import TURBO
    from flash_whisper_amd.model import CustomModel
    from weights_varied import FIXTURE_NAME, scaled_decoder

    fx = json.loads((GOLDEN / FIXTURE_NAME).read_text())
    assert fx['distinct'] >= 50
    root = _write_checkpoint(tmp_path_factory.mktemp('turbo_varied'), scaled_decoder(W.host_params(TURBO, seed=0)))
    clip = synthetic_clip(0)
    assert sha256(clip) == fx['clip_sha256']
    m = CustomModel(str(root), None, selftest=False)
    try:
        ids = m.transcribe(clip, max_new_tokens=fx['n_tokens'], stop_at_eos=False)['token_ids']
    finally:
        del m
        gc.collect()
        torch.cuda.empty_cache()
    first = next((i for i, (a, b) in enumerate(zip(ids, fx['ids'])) if a != b), None)
    assert first is None and len(ids) == len(fx['ids']), (
        f'first mismatch at {first}: gpu {ids[first:first + 4]} oracle {fx["ids"][first:first + 4]} '
        f'margin {fx["margins"][first]}')
    assert len(set(ids)) == fx['distinct']

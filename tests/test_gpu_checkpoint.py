"""A local checkpoint directory (config.json, model.safetensors, generation_config.json, tokenizer.json)
written from the seeded turbo weights must give the same greedy ids as the synthetic model, with the
prompt and suppress ids taken from those files and the text from the tokenizer."""

import json

import pytest
import torch

from test_checkpoint import hf_config, special_tokenizer

pytestmark = pytest.mark.gpu
N_TOKENS = 24


@pytest.fixture(scope='module')
def checkpoint_dir(tmp_path_factory):
    from safetensors.torch import save_file

    from flash_whisper_amd import weights as W
    from flash_whisper_amd.config import (BEGIN_SUPPRESS_IDS, EOS_IDS, PROMPT_IDS, SUPPRESS_IDS, TURBO)

    root = tmp_path_factory.mktemp('turbo_ckpt')
    params = {n: torch.from_numpy(a) for n, a in W.host_params(TURBO, seed=0).items()}
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


def test_checkpoint_model_matches_synthetic(checkpoint_dir, hip_device):
    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.config import PROMPT_IDS
    from flash_whisper_amd.model import CustomModel

    clip = synthetic_clip(0)
    ref = CustomModel(seed=0, selftest=False).transcribe(clip, max_new_tokens=N_TOKENS, stop_at_eos=False)
    torch.cuda.empty_cache()
    m = CustomModel(str(checkpoint_dir), None, selftest=False)
    assert m.checkpoint == str(checkpoint_dir) and tuple(m.prompt) == PROMPT_IDS
    out = m.transcribe(clip, max_new_tokens=N_TOKENS, stop_at_eos=False)
    assert out['token_ids'] == ref['token_ids']
    words = [f'w{i}' for i in out['token_ids'] if i < 50257]
    assert out['text'] == ' '.join(words)

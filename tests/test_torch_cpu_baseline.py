"""oracle.torch_cpu (the reference's PyTorch path in fp32 on the CPU, the timed CPU baseline): its greedy
loop over the HF KV cache gives the ids transformers' own generation loop gave on the tiny greedy model
(tests/golden/hf_greedy.*: suppress on every step, begin-suppress on the first), and a planted protocol
mistake (no begin-suppress) is caught; the seeded turbo parameter names load with nothing missing."""

import json

import numpy as np
import pytest

from conftest import GOLDEN

torch = pytest.importorskip('torch')
transformers = pytest.importorskip('transformers')


@pytest.fixture(scope='module')
def tiny_cpu():
    from flash_whisper_amd.config import DecodeSetup, WhisperDims
    from oracle.torch_cpu import TorchCpuWhisper

    z = np.load(GOLDEN / 'hf_greedy.npz')
    cfg = json.loads(str(z['config']))
    meta = json.loads((GOLDEN / 'hf_greedy.json').read_text())
    dims = WhisperDims(n_mels=cfg['num_mel_bins'], d_model=cfg['d_model'], heads=cfg['encoder_attention_heads'],
                       ffn=cfg['encoder_ffn_dim'], enc_layers=cfg['encoder_layers'], dec_layers=cfg['decoder_layers'],
                       vocab=cfg['vocab_size'], enc_len=cfg['max_source_positions'],
                       max_pos=cfg['max_target_positions'])
    setup = DecodeSetup(prompt=tuple(meta['prompt']), eos=tuple(meta['eos']), suppress=tuple(meta['suppress']),
                        begin_suppress=tuple(meta['begin_suppress']))
    params = {k[len('param:'):]: z[k] for k in z.files if k.startswith('param:')}
    cpu = TorchCpuWhisper(params, dims, setup, threads=2, config=transformers.WhisperConfig(**cfg), decoder_only=True)
    enc = (torch.from_numpy(z['enc'])[None],)
    return cpu, enc, meta


def test_greedy_loop_matches_transformers_ids(tiny_cpu):
    cpu, enc, meta = tiny_cpu
    ids, step_s, first = cpu.decode(enc, meta['limit'])
    assert ids == meta['ids'] and len(step_s) == meta['limit'] and first is not None


def test_greedy_loop_planted_mistake_is_caught(tiny_cpu):
    cpu, enc, meta = tiny_cpu
    saved = cpu.begin_suppress
    cpu.begin_suppress = []
    try:
        ids = cpu.decode(enc, meta['limit'])[0]
    finally:
        cpu.begin_suppress = saved
    assert ids == meta['ids_suppressed'] != meta['ids']


def test_turbo_parameter_names_match_transformers():
    from transformers import WhisperForConditionalGeneration

    from flash_whisper_amd import weights
    from flash_whisper_amd.config import TURBO
    from oracle.torch_cpu import hf_config

    with torch.device('meta'):
        model = WhisperForConditionalGeneration(hf_config(TURBO, 50257))
    names = {s[0]: s[1] for s in weights.param_specs(TURBO)}
    state = {n: tuple(t.shape) for n, t in model.state_dict().items()}
    assert set(state) - set(names) == {'proj_out.weight'}  # tied to the token embedding
    assert set(names) <= set(state) and all(state[n] == tuple(s) for n, s in names.items())

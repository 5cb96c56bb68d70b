"""Local-checkpoint loading (flash_whisper_amd.checkpoint) on the CPU: config -> dims, safetensors
weights (single and sharded files, dtype conversion), hub-cache resolution, tokenizer prompt ids,
generation-config lists and detokenisation. The GPU test in test_gpu_model.py loads a full checkpoint
written from the seeded weights and checks the token ids against the synthetic model."""

import json

import numpy as np
import pytest
import torch

from flash_whisper_amd import checkpoint as C
from flash_whisper_amd import weights as W
from flash_whisper_amd.config import TURBO, WhisperDims

TINY = WhisperDims(n_mels=8, d_model=64, heads=2, ffn=128, enc_layers=1, dec_layers=1, vocab=120, enc_len=10,
                   max_pos=16)


def hf_config(d):
    return {'num_mel_bins': d.n_mels, 'd_model': d.d_model, 'decoder_attention_heads': d.heads,
            'encoder_attention_heads': d.heads, 'decoder_ffn_dim': d.ffn, 'encoder_ffn_dim': d.ffn,
            'encoder_layers': d.enc_layers, 'decoder_layers': d.dec_layers, 'vocab_size': d.vocab,
            'max_source_positions': d.enc_len, 'max_target_positions': d.max_pos, 'activation_function': 'gelu',
            'eos_token_id': 100}


def special_tokenizer(vocab_size, specials):
    """WordLevel tokenizer: ordinary tokens 'w<i>', the given special tokens at their ids."""
    from tokenizers import AddedToken, Tokenizer
    from tokenizers.models import WordLevel
    from tokenizers.pre_tokenizers import WhitespaceSplit

    vocab = {f'w{i}': i for i in range(vocab_size)}
    for tok, i in specials.items():
        vocab.pop(f'w{i}')
        vocab[tok] = i
    tk = Tokenizer(WordLevel(vocab, unk_token='w0'))
    tk.pre_tokenizer = WhitespaceSplit()
    tk.add_special_tokens([AddedToken(t, special=True) for t in specials])
    return tk


def write_checkpoint(root, d, params, shards=1, tokenizer=None, gen=None):
    from safetensors.torch import save_file

    root.mkdir(parents=True, exist_ok=True)
    (root / 'config.json').write_text(json.dumps(hf_config(d)))
    names = sorted(params)
    if shards == 1:
        save_file({n: params[n] for n in names}, str(root / C.WEIGHT_FILE))
    else:
        index = {}
        for s in range(shards):
            part = names[s::shards]
            fname = f'model-{s + 1:05d}-of-{shards:05d}.safetensors'
            save_file({n: params[n] for n in part}, str(root / fname))
            index.update({n: fname for n in part})
        (root / C.INDEX_FILE).write_text(json.dumps({'metadata': {}, 'weight_map': index}))
    if tokenizer is not None:
        tokenizer.save(str(root / 'tokenizer.json'))
    if gen is not None:
        (root / 'generation_config.json').write_text(json.dumps(gen))
    return root


def tiny_params(seed=0, dtype=torch.float32):
    rng = np.random.default_rng(seed)
    return {n: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).to(dtype) for n, s, _ in W.param_specs(TINY)}


@pytest.mark.parametrize('shards,dtype', [(1, torch.float32), (3, torch.bfloat16), (1, torch.float16)])
def test_weights_single_and_sharded_with_fp16_conversion(tmp_path, shards, dtype):
    params = tiny_params(dtype=dtype)
    root = write_checkpoint(tmp_path / 'ckpt', TINY, params, shards=shards)
    assert C.load_dims(root) == TINY
    w = C.Weights(root)
    for name, shape, _ in W.param_specs(TINY):
        t = w.get(name, shape)
        assert t.dtype == torch.float16 and torch.equal(t, params[name].to(torch.float16)), name
    with pytest.raises(C.CheckpointError, match='shape'):
        w.get('model.encoder.conv1.bias', (3,))
    with pytest.raises(C.CheckpointError, match='lacks'):
        w.get('model.encoder.nonexistent', (1,))


def test_supported_dims():
    C.check_supported(TURBO)
    with pytest.raises(NotImplementedError, match='d_model'):
        C.check_supported(TINY)
    deeper = WhisperDims(enc_layers=8, dec_layers=2, vocab=51865)  # depth and vocabulary may vary
    C.check_supported(deeper)


def test_resolve_directory_and_hub_cache(tmp_path):
    d = write_checkpoint(tmp_path / 'plain', TINY, tiny_params())
    assert C.resolve(str(d)) == d
    snap = tmp_path / 'hub' / 'models--org--whisper-x' / 'snapshots' / 'abc123'
    write_checkpoint(snap, TINY, tiny_params())
    (tmp_path / 'hub' / 'models--org--whisper-x' / 'refs').mkdir()
    (tmp_path / 'hub' / 'models--org--whisper-x' / 'refs' / 'main').write_text('abc123')
    assert C.resolve('org/whisper-x', cache_dir=str(tmp_path / 'hub')) == snap
    with pytest.raises(FileNotFoundError, match='nothing is downloaded'):
        C.resolve('org/absent', cache_dir=str(tmp_path / 'hub'))
    (tmp_path / 'noconfig').mkdir()
    with pytest.raises(C.CheckpointError, match='config.json'):
        C.resolve(str(tmp_path / 'noconfig'))


def test_decode_setup_and_detokenize(tmp_path):
    specials = {'<|endoftext|>': 100, '<|startoftranscript|>': 101, '<|en|>': 102, '<|transcribe|>': 103,
                '<|notimestamps|>': 104}
    tk = special_tokenizer(TINY.vocab, specials)
    gen = {'eos_token_id': 100, 'suppress_tokens': [1, 2, 3], 'begin_suppress_tokens': [5, 100]}
    root = write_checkpoint(tmp_path / 'ckpt', TINY, tiny_params(), tokenizer=tk, gen=gen)
    tok = C.load_tokenizer(root)
    setup = C.decode_setup(root, tok, TINY)
    assert setup.prompt == (101, 102, 103, 104) and setup.eos == (100,)
    assert setup.suppress == (1, 2, 3) and setup.begin_suppress == (5, 100)
    assert C.detokenize(tok, [101, 102, 103, 104, 7, 8, 100]) == 'w7 w8'
    assert C.detokenize(None, [1, 2]) == ''
    # without a tokenizer the prompt cannot be derived
    with pytest.raises(C.CheckpointError, match='tokenizer.json'):
        C.decode_setup(root, None, TINY)
    # ids outside the vocabulary are rejected
    (root / 'generation_config.json').write_text(json.dumps({**gen, 'suppress_tokens': [TINY.vocab + 5]}))
    with pytest.raises(C.CheckpointError, match='outside the vocabulary'):
        C.decode_setup(root, tok, TINY)


def test_decode_setup_fallbacks(tmp_path):
    """As transformers' generation config (custom/model.py:45-46,57-61): lists missing from
    generation_config.json come from config.json, a null list is empty, and without any EOS id
    nothing stops the decode."""
    specials = {'<|endoftext|>': 100, '<|startoftranscript|>': 101, '<|en|>': 102, '<|transcribe|>': 103,
                '<|notimestamps|>': 104}
    tk = special_tokenizer(TINY.vocab, specials)
    root = write_checkpoint(tmp_path / 'ckpt', TINY, tiny_params(), tokenizer=tk, gen={'eos_token_id': 100})
    cfg = json.loads((root / 'config.json').read_text())
    cfg.update(suppress_tokens=[7, 9], begin_suppress_tokens=[11], eos_token_id=99)
    (root / 'config.json').write_text(json.dumps(cfg))
    tok = C.load_tokenizer(root)
    setup = C.decode_setup(root, tok, TINY)
    assert setup.suppress == (7, 9) and setup.begin_suppress == (11,) and setup.eos == (100,)
    # null in generation_config.json wins over config.json and means empty
    (root / 'generation_config.json').write_text(json.dumps({'suppress_tokens': None, 'begin_suppress_tokens': None}))
    setup = C.decode_setup(root, tok, TINY)
    assert setup.suppress == () and setup.begin_suppress == () and setup.eos == (99,)
    # neither file names any list or EOS id
    (root / 'generation_config.json').unlink()
    for key in ('suppress_tokens', 'begin_suppress_tokens', 'eos_token_id'):
        cfg.pop(key)
    (root / 'config.json').write_text(json.dumps(cfg))
    setup = C.decode_setup(root, tok, TINY)
    assert setup.suppress == () and setup.begin_suppress == () and setup.eos == ()
    # a single EOS id or a list of them
    (root / 'generation_config.json').write_text(json.dumps({'eos_token_id': [100, 98]}))
    assert C.decode_setup(root, tok, TINY).eos == (100, 98)

"""Local Whisper checkpoints: weights, dimensions, decoding setup and tokenizer from files on disk.

The reference builds its model with ``from_pretrained(model_id, cache_dir=...)`` plus the checkpoint's
tokenizer and generation config (custom/model.py:32-36,40-62) and detokenises the greedy ids at the end
of ``transcribe`` (custom/model.py:216-217). This module reads the same files without any network
access:

- ``model_id`` may be a directory holding ``config.json`` and ``model.safetensors`` (or sharded
  ``model-*.safetensors`` with ``model.safetensors.index.json``), or a hub id already present in a
  Hugging Face cache (``<cache_dir>/models--org--name/snapshots/<rev>/``, ``cache_dir`` defaulting to
  ``$HF_HUB_CACHE`` or ``$HF_HOME/hub``). Nothing is ever downloaded.
- Tensor names are the transformers ``WhisperForConditionalGeneration`` state-dict names, which are the
  names ``weights.param_specs`` uses; fp32 / bf16 tensors are converted to fp16 as the reference's
  ``dtype=torch.float16`` load does. The LM head is ``proj_out.weight`` when the file has it, else the
  tied ``model.decoder.embed_tokens.weight``.
- ``tokenizer.json`` (a tokenizers-library file) gives the prompt ids of the reference's four prompt
  tokens and the text; ``generation_config.json`` gives the EOS and suppress lists.
"""

import json
import os
from pathlib import Path

from .config import DecodeSetup, WhisperDims

PROMPT_TOKENS = ('<|startoftranscript|>', '<|en|>', '<|transcribe|>', '<|notimestamps|>')  # custom/model.py:22
WEIGHT_FILE = 'model.safetensors'
INDEX_FILE = 'model.safetensors.index.json'


class CheckpointError(ValueError):
    pass


def _hub_cache(cache_dir):
    if cache_dir:
        return Path(cache_dir)
    if os.environ.get('HF_HUB_CACHE'):
        return Path(os.environ['HF_HUB_CACHE'])
    home = os.environ.get('HF_HOME') or os.path.join(os.path.expanduser('~'), '.cache', 'huggingface')
    return Path(home) / 'hub'


def resolve(model_id, cache_dir=None):
    """Directory of the checkpoint `model_id`: the path itself, or its snapshot in the local hub cache."""
    p = Path(model_id)
    if p.is_dir():
        if not (p / 'config.json').is_file():
            raise CheckpointError(f'{p} has no config.json')
        return p
    repo = _hub_cache(cache_dir) / ('models--' + str(model_id).replace('/', '--'))
    snaps = repo / 'snapshots'
    if snaps.is_dir():
        ref = repo / 'refs' / 'main'
        if ref.is_file() and (snaps / ref.read_text().strip() / 'config.json').is_file():
            return snaps / ref.read_text().strip()
        found = sorted(d for d in snaps.iterdir() if (d / 'config.json').is_file())
        if found:
            return found[-1]
    raise FileNotFoundError(f'checkpoint {model_id!r} is neither a directory nor in the local hub cache '
                            f'{_hub_cache(cache_dir)} (nothing is downloaded)')


def load_dims(path):
    """WhisperDims from a transformers WhisperConfig ``config.json``."""
    cfg = json.loads((Path(path) / 'config.json').read_text())
    try:
        d = WhisperDims(n_mels=cfg['num_mel_bins'], d_model=cfg['d_model'], heads=cfg['decoder_attention_heads'],
                        ffn=cfg['decoder_ffn_dim'], enc_layers=cfg['encoder_layers'], dec_layers=cfg['decoder_layers'],
                        vocab=cfg['vocab_size'], enc_len=cfg['max_source_positions'],
                        max_pos=cfg['max_target_positions'])
    except KeyError as e:
        raise CheckpointError(f'config.json lacks {e}') from None
    if (cfg.get('encoder_attention_heads', d.heads) != d.heads or cfg.get('encoder_ffn_dim', d.ffn) != d.ffn):
        raise CheckpointError('encoder and decoder must share heads and FFN width')
    if cfg.get('activation_function', 'gelu') != 'gelu':
        raise CheckpointError(f'unsupported activation {cfg["activation_function"]!r}')
    return d


def check_supported(dims):
    """The kernels are specialised for the large-v3 layer width; depth, vocabulary and lengths may vary."""
    want = dict(n_mels=128, d_model=1280, heads=20, ffn=5120, enc_len=1500)
    bad = {k: getattr(dims, k) for k, v in want.items() if getattr(dims, k) != v}
    if bad:
        raise NotImplementedError(f'kernels need {want}; checkpoint has {bad}')
    if dims.max_pos > 512:
        raise NotImplementedError('at most 512 decoder positions (8 self-attention splits of 64 keys)')


class Weights:
    """Lazy tensor access over one or several safetensors files (CPU torch tensors)."""

    def __init__(self, path):
        from safetensors import safe_open

        path = Path(path)
        if (path / INDEX_FILE).is_file():
            index = json.loads((path / INDEX_FILE).read_text())['weight_map']
            files = sorted(set(index.values()))
        elif (path / WEIGHT_FILE).is_file():
            files = [WEIGHT_FILE]
        else:
            raise CheckpointError(f'{path} has neither {WEIGHT_FILE} nor {INDEX_FILE}')
        self._handles = [safe_open(str(path / f), framework='pt') for f in files]
        self._where = {}
        for h in self._handles:
            for k in h.keys():
                self._where[k] = h

    def __contains__(self, name):
        return name in self._where

    def get(self, name, shape):
        """fp16 tensor `name` with the expected `shape`."""
        import torch

        if name not in self._where:
            raise CheckpointError(f'checkpoint lacks {name}')
        t = self._where[name].get_tensor(name)
        if tuple(t.shape) != tuple(shape):
            raise CheckpointError(f'{name}: shape {tuple(t.shape)}, expected {tuple(shape)}')
        return t.to(torch.float16) if t.dtype != torch.float16 else t


def load_tokenizer(path):
    """tokenizers.Tokenizer from ``tokenizer.json``, or None when the checkpoint has none."""
    f = Path(path) / 'tokenizer.json'
    if not f.is_file():
        return None
    from tokenizers import Tokenizer

    return Tokenizer.from_file(str(f))


def _ids(value):
    """A token-id list from a config value: null is empty, a single id is a one-element list."""
    if value is None:
        return ()
    return tuple(value) if isinstance(value, (list, tuple)) else (value,)


def decode_setup(path, tokenizer, dims):
    """Prompt, EOS and suppress ids as the reference derives them (custom/model.py:44-46,57-61): from
    the generation config, whose fields transformers fills from config.json when the checkpoint has
    no generation_config.json; a missing or null suppress list is empty (``gen.suppress_tokens or []``),
    and a missing EOS id means no EOS stop."""
    prompt = None
    if tokenizer is not None:
        ids = [tokenizer.token_to_id(t) for t in PROMPT_TOKENS]
        if all(i is not None for i in ids):
            prompt = tuple(ids)
    cfg = json.loads((Path(path) / 'config.json').read_text())
    gen_file = Path(path) / 'generation_config.json'
    gen = json.loads(gen_file.read_text()) if gen_file.is_file() else {}
    field = lambda key: gen[key] if key in gen else cfg.get(key)
    eos = gen.get('eos_token_id')
    eos = _ids(cfg.get('eos_token_id') if eos is None else eos)
    suppress, begin = _ids(field('suppress_tokens')), _ids(field('begin_suppress_tokens'))
    if prompt is None:
        raise CheckpointError('the prompt tokens need tokenizer.json with ' + ', '.join(PROMPT_TOKENS))
    for name, ids in (('prompt', prompt), ('eos', eos), ('suppress', suppress), ('begin_suppress', begin)):
        if any(not 0 <= i < dims.vocab for i in ids):
            raise CheckpointError(f'{name} ids outside the vocabulary of {dims.vocab}')
    return DecodeSetup(prompt=prompt, eos=eos, suppress=suppress, begin_suppress=begin)


def detokenize(tokenizer, ids):
    """Text of the greedy ids without special tokens (custom/model.py:217)."""
    return '' if tokenizer is None else tokenizer.decode(list(ids), skip_special_tokens=True)

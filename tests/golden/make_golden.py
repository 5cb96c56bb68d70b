"""Writes the committed golden fixtures. Run in the development container only (never on a GPU run).

  python tests/golden/make_golden.py hf      # transformers vectors (third-party arithmetic spec)
  python tests/golden/make_golden.py hf16    # transformers fp16 encoder, op by op
  python tests/golden/make_golden.py greedy  # transformers greedy loop with prompt / suppress / EOS
  python tests/golden/make_golden.py e2e     # oracle greedy ids on the full synthetic model
  python tests/golden/make_golden.py varied  # the same with the decoder scaled (ids that vary)

``hf`` imports the installed third-party ``transformers`` (5.15.0 here; the reference pins 5.20.2 in
requirements.lock:681) on the CPU, with random init and no download, to record:
  - hf_logmel.npz: WhisperFeatureExtractor(feature_size=128).mel_filters and the log-mel its numpy
    path gives for a seeded 2 s waveform (feature_extraction_whisper.py:105-131);
  - hf_tiny.npz: a tiny WhisperForConditionalGeneration (fp32, eval) — all parameters, a mel input,
    the encoder output (modeling_whisper.py:592-648) and the decoder logits for a fixed id sequence
    given that encoder output. These pin the structure of the oracle's encoder and decoder.
``hf16`` records hf_tiny16.npz: a tiny WhisperEncoder run in fp16 on the CPU (SDPA attention, as
custom/model.py:32-33 loads it), with head_dim 8 so the fp16 rounding of the pre-scaled query
(modeling_whisper.py:309) is observable, and fc2 biases that push two residual channels past
65504 - 1000 so the fp16 clamp (:409-411) acts. Every op's output inside every layer is recorded:
the LayerNorms, the query / key / value exactly as the attention function receives them, the
attention output, out_proj, fc1, the GELU, fc2 and the clamped layer output.
``greedy`` records hf_greedy.json / .npz: a tiny fp32 model (hf_tiny.npz's config, its own seed)
decoding greedily with its own
KV cache through a loop that follows custom/pytorch_model.py:53-79 (the whole prompt in one forward,
its last position's logits give the first token; suppress ids masked on every step, begin-suppress
ids on the first step only; stop after an EOS id or after max_target_positions - len(prompt) ids).
The suppress, begin-suppress and EOS ids are chosen from unconstrained runs so that each one changes
the result.
``e2e`` runs the oracle (fp16 rounding points) on the seeded whisper-large-v3-turbo-shaped weights and
the seeded 30 s clip and records the 224 greedy ids with their top-2 margins, plus checksums and row
samples of the intermediate tensors (e2e_turbo_seed0.json / .npz).
``varied`` does the same on those weights with the decoder scaled as tests/weights_varied.py defines
(e2e_turbo_seed0_varied.json): the seed-0 ids repeat three ids, these vary from step to step.
"""

import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
OUT = Path(__file__).resolve().parent

TINY = dict(vocab_size=96, num_mel_bins=8, d_model=64, encoder_layers=2, decoder_layers=2,
            encoder_attention_heads=4, decoder_attention_heads=4, encoder_ffn_dim=128, decoder_ffn_dim=128,
            max_source_positions=16, max_target_positions=24, pad_token_id=0, bos_token_id=1, eos_token_id=2,
            decoder_start_token_id=3, activation_function='gelu', scale_embedding=False)
TINY_IDS = [3, 5, 7, 11, 13, 17, 19, 23]


def make_hf():
    import torch
    from transformers import WhisperConfig, WhisperFeatureExtractor, WhisperForConditionalGeneration

    import transformers

    fe = WhisperFeatureExtractor(feature_size=128)
    rng = np.random.default_rng(1234)
    audio = (rng.standard_normal(2 * 16000) * 0.1).astype(np.float32)
    feats = fe._np_extract_fbank_features(audio[None], 'cpu')[0]
    np.savez_compressed(OUT / 'hf_logmel.npz', mel_filters=fe.mel_filters.astype(np.float64), audio=audio,
                        log_mel=feats.astype(np.float64), transformers_version=transformers.__version__)

    torch.manual_seed(0)
    cfg = WhisperConfig(**TINY)
    model = WhisperForConditionalGeneration(cfg).eval()
    with torch.no_grad():
        # random-init biases are zero in transformers; give every parameter a random value so the
        # fixture also pins where biases enter
        for name, p in model.named_parameters():
            if 'embed_positions' in name and 'encoder' in name:
                continue
            if p.dim() == 1 and 'layer_norm' not in name:
                p.normal_(0.0, 0.05)
            elif 'layer_norm' in name:
                p.normal_(1.0 if name.endswith('weight') else 0.0, 0.1)
        mel = torch.randn(1, cfg.num_mel_bins, 2 * cfg.max_source_positions)
        enc = model.model.encoder(mel).last_hidden_state
        ids = torch.tensor([TINY_IDS])
        out = model(encoder_outputs=(enc,), decoder_input_ids=ids)
    params = {n: p.detach().numpy().astype(np.float32) for n, p in model.state_dict().items()}
    np.savez_compressed(OUT / 'hf_tiny.npz', mel=mel[0].numpy(), enc=enc[0].numpy(), ids=np.array(TINY_IDS),
                        logits=out.logits[0].numpy(), config=json.dumps(TINY),
                        transformers_version=transformers.__version__,
                        **{f'param:{n}': v for n, v in params.items()})
    print('wrote hf_logmel.npz, hf_tiny.npz with transformers', transformers.__version__)


TINY16 = dict(TINY, encoder_attention_heads=8, decoder_attention_heads=8, encoder_layers=3)
CLAMP_BIAS = {0: 33000.0, 1: 32200.0}  # fc2 bias of channel 3 (+) and channel 7 (-) per layer


def _randomize(model):
    """Random values for every parameter (transformers initialises biases to zero)."""
    import torch

    with torch.no_grad():
        for name, p in model.named_parameters():
            if 'embed_positions' in name and 'encoder' in name:
                continue
            if p.dim() == 1 and 'layer_norm' not in name:
                p.normal_(0.0, 0.05)
            elif 'layer_norm' in name:
                p.normal_(1.0 if name.endswith('weight') else 0.0, 0.1)


def make_hf16():
    import torch
    from transformers import WhisperConfig, WhisperForConditionalGeneration
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    import transformers

    torch.manual_seed(16)
    cfg = WhisperConfig(**TINY16, attn_implementation='sdpa')
    model = WhisperForConditionalGeneration(cfg).eval()
    _randomize(model)
    with torch.no_grad():
        for i, b in CLAMP_BIAS.items():
            fc2 = model.model.encoder.layers[i].fc2.bias
            fc2[3], fc2[7] = b, -b
    model = model.half()
    enc = model.model.encoder
    rec = {}

    def keep(name, t):
        rec[name] = t.detach()[0].float().numpy().copy()

    sdpa = ALL_ATTENTION_FUNCTIONS['sdpa']
    layer_of = {id(lay.self_attn): i for i, lay in enumerate(enc.layers)}

    def recording_sdpa(module, query, key, value, attention_mask, **kw):
        out = sdpa(module, query, key, value, attention_mask, **kw)
        i = layer_of[id(module)]
        flat = lambda t: t.transpose(1, 2).reshape(t.shape[0], t.shape[2], -1)  # [b, h, t, hd] -> [b, t, h*hd]
        keep(f'{i}.q', flat(query))
        keep(f'{i}.k', flat(key))
        keep(f'{i}.v', flat(value))
        keep(f'{i}.attn', out[0].reshape(out[0].shape[0], out[0].shape[1], -1))
        return out

    def hook(name, inputs=False):
        def f(mod, args, kwargs, out):
            if inputs:
                keep(name + '.in', args[0] if args else kwargs['hidden_states'])
            keep(name, out if torch.is_tensor(out) else out[0])
        return f

    for i, lay in enumerate(enc.layers):
        lay.register_forward_hook(hook(f'{i}.out', inputs=True), with_kwargs=True)
        lay.self_attn_layer_norm.register_forward_hook(hook(f'{i}.ln1'), with_kwargs=True)
        lay.self_attn.out_proj.register_forward_hook(hook(f'{i}.attn_out'), with_kwargs=True)
        lay.final_layer_norm.register_forward_hook(hook(f'{i}.ln2', inputs=True), with_kwargs=True)
        lay.fc1.register_forward_hook(hook(f'{i}.fc1'), with_kwargs=True)
        lay.fc2.register_forward_hook(hook(f'{i}.fc2', inputs=True), with_kwargs=True)
    ALL_ATTENTION_FUNCTIONS['sdpa'] = recording_sdpa
    try:
        mel = (torch.randn(1, cfg.num_mel_bins, 2 * cfg.max_source_positions) * 2).half()
        with torch.no_grad():
            out = enc(mel).last_hidden_state
    finally:
        del ALL_ATTENTION_FUNCTIONS['sdpa']
    # x_attn is the final LayerNorm's input; the GELU output is fc2's input
    for i in range(cfg.encoder_layers):
        rec[f'{i}.x_attn'] = rec.pop(f'{i}.ln2.in')
        rec[f'{i}.gelu'] = rec.pop(f'{i}.fc2.in')
    clamped = [i for i in range(cfg.encoder_layers) if np.abs(rec[f'{i}.out']).max() >= 65504.0 - 1000.0]
    assert clamped, 'no layer reached the fp16 clamp'
    params = {n: p.detach().numpy() for n, p in model.state_dict().items()}
    np.savez_compressed(OUT / 'hf_tiny16.npz', mel=mel[0].numpy(), enc=out[0].detach().numpy(),
                        config=json.dumps(TINY16), transformers_version=transformers.__version__,
                        torch_version=torch.__version__, clamped_layers=np.array(clamped),
                        **{f'param:{n}': v for n, v in params.items()}, **{f'trace:{k}': v for k, v in rec.items()})
    print('wrote hf_tiny16.npz; layers reaching the clamp:', clamped)


def _greedy_model():
    """A tiny fp32 model whose greedy ids vary from step to step: the model of hf_tiny.npz's config with
    N(0, 0.5) token embeddings and N(0, 0.3) decoder projections (smaller values make random-init
    decoders repeat one id)."""
    import torch
    from transformers import WhisperConfig, WhisperForConditionalGeneration

    torch.manual_seed(2)
    model = WhisperForConditionalGeneration(WhisperConfig(**TINY)).eval()
    _randomize(model)
    with torch.no_grad():
        model.model.decoder.embed_tokens.weight.normal_(0, 0.5)
        for lay in model.model.decoder.layers:
            for lin in (lay.fc1, lay.fc2, lay.self_attn.q_proj, lay.self_attn.k_proj, lay.self_attn.v_proj,
                        lay.self_attn.out_proj):
                lin.weight.normal_(0, 0.3)
    mel = torch.randn(1, TINY['num_mel_bins'], 2 * TINY['max_source_positions'])
    return model, mel


def _hf_greedy(model, enc, prompt, suppress, begin_suppress, eos):
    """Greedy ids with transformers' own KV cache, in the order of custom/pytorch_model.py:53-79."""
    import torch

    limit = model.config.max_target_positions - len(prompt)
    ids, margins, past = [], [], None
    inp = torch.tensor([prompt])
    with torch.no_grad():
        for step in range(limit):
            out = model(encoder_outputs=(enc,), decoder_input_ids=inp, past_key_values=past, use_cache=True)
            logits = out.logits[0, -1].float().clone()
            mask = list(suppress) + (list(begin_suppress) if step == 0 else [])
            if mask:
                logits[mask] = -float('inf')
            top = torch.topk(logits, 2).values
            tok = int(logits.argmax())
            ids.append(tok)
            margins.append(float(top[0] - top[1]))
            if tok in eos:
                break
            past = out.past_key_values
            inp = torch.tensor([[tok]])
    return ids, margins


def make_greedy():
    import torch

    import transformers

    model, mel = _greedy_model()
    with torch.no_grad():
        enc = model.model.encoder(mel).last_hidden_state
    prompt = [3, 50, 51, 52]
    run = lambda sup, begin, eos=(): _hf_greedy(model, enc, prompt, sup, begin, eos)
    free, _ = run([], [])
    # begin-suppress the first free token and an id x; suppress an id that the begin-only run produces
    # after its first step. Each protocol slip then changes the ids: suppressing only on the first
    # step gives the begin-only run, and begin-suppressing on every step removes x, which the final
    # run produces later.
    found = None
    for x in dict.fromkeys(free[1:]):
        begin = [free[0], x] if x != free[0] else [free[0]]
        begin_only, _ = run([], begin)
        for tok in dict.fromkeys(begin_only[1:]):
            if tok in begin or tok == begin_only[0]:
                continue
            full, margins = run([tok], begin)
            if full != begin_only and any(t in begin for t in full[1:]):
                found = (begin, begin_only, [tok], full, margins)
                break
        if found:
            break
    if not found:
        raise RuntimeError('no suppress / begin-suppress ids separate the protocol variants')
    begin, begin_only, suppress, full, margins = found
    sup_run, _ = run(suppress, [])
    assert sup_run != full and free != sup_run
    eos_at = next(i for i in range(3, len(full)) if full[i] not in full[:i])
    eos = [full[eos_at]]
    stopped, _ = run(suppress, begin, eos)
    assert stopped == full[:eos_at + 1]
    assert min(margins) > 1e-3, min(margins)
    meta = dict(prompt=prompt, suppress=suppress, begin_suppress=begin, eos=eos,
                ids_free=free, ids_suppressed=sup_run, ids_begin_only=begin_only, ids=full, margins=margins, ids_eos=stopped,
                limit=model.config.max_target_positions - len(prompt),
                transformers_version=transformers.__version__,
                note='tiny fp32 model; parameters and encoder output in hf_greedy.npz')
    (OUT / 'hf_greedy.json').write_text(json.dumps(meta, indent=1) + '\n')
    dec = {n: p.detach().numpy() for n, p in model.state_dict().items() if n.startswith('model.decoder.')}
    np.savez_compressed(OUT / 'hf_greedy.npz', enc=enc[0].numpy(), config=json.dumps(TINY),
                        **{f'param:{n}': v for n, v in dec.items()})
    print('wrote hf_greedy.json', full, 'eos', eos, 'min margin', min(margins))


def make_e2e(seed=0, n_tokens=224):
    from flash_whisper_amd import audio as fw_audio
    from flash_whisper_amd import weights
    from flash_whisper_amd.config import DecodeSetup, TURBO
    from oracle.pipeline import transcribe_ids

    t0 = time.time()
    params = weights.host_params(TURBO, seed)
    clip = fw_audio.synthetic_clip(seed)
    setup = DecodeSetup()
    print(f'weights {time.time() - t0:.1f}s', flush=True)
    res = transcribe_ids(params, TURBO, clip, setup.prompt, n_tokens, setup.suppress, setup.begin_suppress)
    print(f'oracle e2e {time.time() - t0:.1f}s', flush=True)
    rows = np.array([0, 1, 2, 3, 500, 749, 750, 1000, 1496, 1497, 1498, 1499])
    enc, ckv = res['enc'], res['cross_kv']
    np.savez_compressed(OUT / f'e2e_turbo_seed{seed}.npz', rows=rows, enc_rows=enc[rows].astype(np.float16),
                        cross_k_rows=ckv[:, 0, :, rows].astype(np.float16),
                        mel_cols=res['mel'][:, rows].astype(np.float16))
    meta = dict(seed=seed, n_tokens=n_tokens, ids=[int(i) for i in res['ids']],
                margins=[float(m) for m in res['margins']], clip_sha256=fw_audio.sha256(clip),
                prompt=list(setup.prompt), suppress=list(setup.suppress), begin_suppress=list(setup.begin_suppress),
                enc_abs_mean=float(np.abs(enc).mean()), enc_std=float(enc.std()),
                mel_mean=float(res['mel'].mean()), mel_max=float(res['mel'].max()),
                note='oracle fp16 rounding points; weights from fw_synth_normal_f16 with this seed')
    (OUT / f'e2e_turbo_seed{seed}.json').write_text(json.dumps(meta, indent=1) + '\n')
    m = np.array(res['margins'])
    print('ids', res['ids'][:32], '... min margin', m.min(), 'n<2e-3', int((m < 2e-3).sum()))


def make_varied(seed=0, n_tokens=224):
    from flash_whisper_amd import audio as fw_audio
    from flash_whisper_amd import weights
    from flash_whisper_amd.config import DecodeSetup, TURBO
    from oracle.pipeline import transcribe_ids

    sys.path.insert(0, str(OUT.parent))
    import weights_varied as V

    t0 = time.time()
    params = V.scaled_decoder(weights.host_params(TURBO, seed))
    clip = fw_audio.synthetic_clip(seed)
    setup = DecodeSetup()
    res = transcribe_ids(params, TURBO, clip, setup.prompt, n_tokens, setup.suppress, setup.begin_suppress)
    print(f'oracle e2e {time.time() - t0:.1f}s', flush=True)
    ids = [int(i) for i in res['ids']]
    meta = dict(seed=seed, n_tokens=n_tokens, ids=ids, margins=[float(m) for m in res['margins']],
                distinct=len(set(ids)), embed_scale=V.EMBED_SCALE, proj_scale=V.PROJ_SCALE,
                clip_sha256=fw_audio.sha256(clip), prompt=list(setup.prompt), suppress=list(setup.suppress),
                begin_suppress=list(setup.begin_suppress),
                note='oracle fp16 rounding points; seed-0 weights with the decoder scaled (tests/weights_varied.py)')
    (OUT / V.FIXTURE_NAME).write_text(json.dumps(meta, indent=1) + '\n')
    m = np.array(res['margins'])
    print('distinct', len(set(ids)), 'min margin', m.min(), 'n<2e-3', int((m < 2e-3).sum()))


if __name__ == '__main__':
    what = sys.argv[1] if len(sys.argv) > 1 else 'all'
    if what in ('hf', 'all'):
        make_hf()
    if what in ('hf16', 'all'):
        make_hf16()
    if what in ('greedy', 'all'):
        make_greedy()
    if what in ('e2e', 'all'):
        make_e2e()
    if what in ('varied', 'all'):
        make_varied()

"""Writes the committed golden fixtures. Run in the development container only (never on a GPU run).

  python tests/golden/make_golden.py hf    # transformers vectors (third-party arithmetic spec)
  python tests/golden/make_golden.py e2e   # oracle greedy ids on the full synthetic model

``hf`` imports the installed third-party ``transformers`` (5.15.0 here; the reference pins 5.20.2 in
requirements.lock:681) on the CPU, with random init and no download, to record:
  - hf_logmel.npz: WhisperFeatureExtractor(feature_size=128).mel_filters and the log-mel its numpy
    path gives for a seeded 2 s waveform (feature_extraction_whisper.py:105-131);
  - hf_tiny.npz: a tiny WhisperForConditionalGeneration (fp32, eval) — all parameters, a mel input,
    the encoder output (modeling_whisper.py:592-648) and the decoder logits for a fixed id sequence
    given that encoder output. These pin the structure of the oracle's encoder and decoder.
``e2e`` runs the oracle (fp16 rounding points) on the seeded whisper-large-v3-turbo-shaped weights and
the seeded 30 s clip and records the 224 greedy ids with their top-2 margins, plus checksums and row
samples of the intermediate tensors (e2e_turbo_seed0.json / .npz).
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


if __name__ == '__main__':
    what = sys.argv[1] if len(sys.argv) > 1 else 'all'
    if what in ('hf', 'all'):
        make_hf()
    if what in ('e2e', 'all'):
        make_e2e()

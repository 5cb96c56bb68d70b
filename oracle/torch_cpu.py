"""The reference's PyTorch path in fp32 on the host CPU: a timed baseline (test infrastructure only).

The reference's plain-PyTorch backend (custom/pytorch_model.py:29-89) runs transformers'
WhisperForConditionalGeneration in fp16 on CUDA, with the feature extractor's log-mel on the host and a
manual greedy loop over the HF KV cache. This module runs the same modules and loop on the CPU in fp32
(the natural CPU precision): the seeded fp16 weights upcast to fp32, ``WhisperFeatureExtractor``'s
torch log-mel (``torch.stft``), ``get_encoder()``, then one forward per token with ``past_key_values``,
the suppress lists applied to the last position's logits and the begin-suppress list at the first
step (pytorch_model.py:49-80). Decoding runs a fixed number of tokens (random-init weights never emit
EOS), so its ids are fp32 greedy ids and may part from the fp16 GPU ids after a near tie; the numpy
oracle (oracle.pipeline) is the id check, this module only the timing baseline. ``config_rows`` times
the path's per-config units the same way (fp32, on the host's cores).
"""

import os
import statistics
import time


def host_threads():
    """Threads for torch's CPU pool: the host's CPU count, capped by OMP_NUM_THREADS where that is set."""
    n = os.cpu_count() or 1
    env = os.environ.get('OMP_NUM_THREADS', '')
    return min(n, int(env)) if env.isdigit() and int(env) > 0 else n


def hf_config(dims, eos_id):
    from transformers import WhisperConfig

    return WhisperConfig(num_mel_bins=dims.n_mels, d_model=dims.d_model, decoder_attention_heads=dims.heads,
                         encoder_attention_heads=dims.heads, decoder_ffn_dim=dims.ffn, encoder_ffn_dim=dims.ffn,
                         encoder_layers=dims.enc_layers, decoder_layers=dims.dec_layers, vocab_size=dims.vocab,
                         max_source_positions=dims.enc_len, max_target_positions=dims.max_pos,
                         activation_function='gelu', eos_token_id=eos_id)


class TorchCpuWhisper:
    """transformers Whisper in fp32 on the CPU with the given fp16 numpy parameters (HF names)."""

    def __init__(self, params, dims, setup, threads=None, config=None, decoder_only=False):
        import torch
        from transformers import WhisperFeatureExtractor, WhisperForConditionalGeneration

        self.threads = threads or host_threads()
        torch.set_num_threads(self.threads)
        config = config or hf_config(dims, setup.eos[0] if setup.eos else None)
        with torch.device('meta'):  # no random init: every tensor is assigned from `params` below
            model = WhisperForConditionalGeneration(config)
        state = {n: torch.from_numpy(a).float() for n, a in params.items()}
        missing, unexpected = model.load_state_dict(state, strict=False, assign=True)
        model.tie_weights()  # proj_out is the token embedding
        skip = ('proj_out.weight',) + (('model.encoder.',) if decoder_only else ())  # decoder_only: no encoder run
        if unexpected or [m for m in missing if not m.startswith(skip)]:
            raise RuntimeError(f'parameter names do not match: missing {missing}, unexpected {unexpected}')
        self.model = model.eval()
        self.features = WhisperFeatureExtractor(feature_size=dims.n_mels)
        self.prompt = list(setup.prompt)
        self.suppress = list(setup.suppress)
        self.begin_suppress = list(setup.begin_suppress)

    def transcribe(self, audio, max_new_tokens):
        """pytorch_model.py:29-89 on the CPU, for `max_new_tokens` tokens: the reference's timing dict
        plus ``step_s`` (each token's forward + argmax, the first including the prompt)."""
        import torch

        with torch.inference_mode():
            start = time.perf_counter()
            feats = self.features(audio, sampling_rate=16000, return_tensors='pt').input_features
            mel_s = time.perf_counter() - start
            t = time.perf_counter()
            enc = self.model.get_encoder()(feats)
            encoder_s = time.perf_counter() - t
            decode_start = time.perf_counter()
            tokens, step_s, first = self.decode(enc, max_new_tokens)
            decode_s = time.perf_counter() - decode_start
        return dict(token_ids=tokens, ttft_s=first - start, e2e_s=time.perf_counter() - start, mel_s=mel_s,
                    encoder_s=encoder_s, decode_s=decode_s, step_s=step_s)

    def decode(self, enc, max_new_tokens):
        """The greedy loop of pytorch_model.py:58-80 (no EOS stop) over encoder outputs `enc`: returns
        (token ids, each step's seconds, perf_counter time of the first token)."""
        import torch

        ids = torch.tensor([self.prompt], dtype=torch.long)
        past, tokens, step_s, first = None, [], [], None
        with torch.inference_mode():
            for step in range(max_new_tokens):
                t = time.perf_counter()
                out = self.model(encoder_outputs=enc, decoder_input_ids=ids, past_key_values=past, use_cache=True)
                logits = out.logits[0, -1].float()
                if self.suppress:
                    logits[self.suppress] = -float('inf')
                if step == 0 and self.begin_suppress:
                    logits[self.begin_suppress] = -float('inf')
                token = int(logits.argmax().item())
                step_s.append(time.perf_counter() - t)
                if first is None:
                    first = time.perf_counter()
                tokens.append(token)
                past = out.past_key_values
                ids = torch.tensor([[token]], dtype=torch.long)
        return tokens, step_s, first


def _median_us(fn, reps):
    fn()  # warm-up
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return round(statistics.median(ts) * 1e6, 1)


def config_rows(cpu, clip, reps=50, seed=1234):
    """Median us over `reps` of each per-config unit, fp32 on the CPU, with the model's own layer-0
    decoder weights and tied embedding where the unit has weights:
    - log_mel: the feature extractor on the 30 s clip (pytorch_model.py:37-39);
    - self_attention L in {1, 64, 224, 448}: softmax(q K^T / 8) V for 20 heads x 64 (q, K, V ~ N(0, 1));
    - cross_attention_mlp: the same over 1500 frames, then residual, LayerNorm, fc1, GELU, fc2, residual;
    - lm_head: final LayerNorm, logits over the 51866-row embedding, argmax (h ~ N(0, 1)).
    The inputs stay the same from rep to rep, so whatever fits the host's caches is read from them."""
    import torch
    import torch.nn.functional as F

    model = cpu.model
    dec = model.model.decoder
    layer = dec.layers[0]
    heads, dm = model.config.decoder_attention_heads, model.config.d_model
    hd = dm // heads
    g = torch.Generator().manual_seed(seed)
    randn = lambda *s: torch.randn(*s, generator=g)
    rows = {}
    with torch.inference_mode():
        rows['log_mel'] = _median_us(lambda: cpu.features(clip, sampling_rate=16000, return_tensors='pt'), reps)
        q = randn(heads, 1, hd)
        sa = {}
        for length in (1, 64, 224, 448):
            k, v = randn(heads, length, hd), randn(heads, length, hd)
            sa[f'L{length}'] = _median_us(lambda: torch.softmax(q @ k.transpose(1, 2) * hd ** -0.5, -1) @ v, reps)
        rows['self_attention'] = sa
        k, v, h = randn(heads, 1500, hd), randn(heads, 1500, hd), randn(1, dm)

        def cross_mlp():
            a = (torch.softmax(q @ k.transpose(1, 2) * hd ** -0.5, -1) @ v).reshape(1, dm)
            r = h + a
            y = F.layer_norm(r, (dm,), layer.final_layer_norm.weight, layer.final_layer_norm.bias, 1e-5)
            return r + layer.fc2(F.gelu(layer.fc1(y)))

        rows['cross_attention_mlp'] = _median_us(cross_mlp, reps)
        ln = dec.layer_norm
        w = model.proj_out.weight

        def lm_head():
            y = F.layer_norm(h, (dm,), ln.weight, ln.bias, 1e-5)
            return int((y @ w.t()).argmax())

        rows['lm_head'] = _median_us(lm_head, reps)
    return rows


def baseline(params, dims, setup, clip, tokens, reps=5, config_reps=50, progress=None):
    """`reps` end-to-end transcribes of `clip` for `tokens` tokens after a short warm-up (8 tokens), and
    the per-config units over `config_reps`; medians and p90 of the reference's timing fields, with each
    token's step time pooled over the reps (the first step of each, which includes the prompt, left out)."""
    cpu = TorchCpuWhisper(params, dims, setup)
    cpu.transcribe(clip, 8)
    runs = []
    for i in range(reps):
        runs.append(cpu.transcribe(clip, tokens))
        if progress:
            progress(f'fp32 PyTorch transcribe {i + 1}/{reps}: {runs[-1]["e2e_s"]:.1f} s')
    steps = [s for r in runs for s in r['step_s'][1:]]
    med = lambda k: round(statistics.median(r[k] for r in runs) * 1e3, 1)
    e2e = sorted(r['e2e_s'] * 1e3 for r in runs)
    pos = 0.9 * (len(e2e) - 1)
    lo, hi = int(pos), min(int(pos) + 1, len(e2e) - 1)
    return dict(step_us=round(statistics.median(steps) * 1e6, 1), e2e_ms=med('e2e_s'),
                e2e_p90_ms=round(e2e[lo] + (e2e[hi] - e2e[lo]) * (pos - lo), 1), ttft_ms=med('ttft_s'),
                mel_ms=med('mel_s'), encoder_ms=med('encoder_s'), decode_ms=med('decode_s'), reps=reps,
                threads=cpu.threads, token_ids=runs[-1]['token_ids'],
                configs=config_rows(cpu, clip, config_reps))

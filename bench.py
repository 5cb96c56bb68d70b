"""Benchmark of the batch-1 Whisper-large-v3-turbo hot path on one MI355X.

Workload (one "step"): a full ``CustomModel.transcribe`` of a seeded 30 s synthetic clip — HIP log-mel,
32-layer MFMA encoder + cross K/V in a hipGraph, then the 4-token prompt pass and the first token in one
persistent launch, then the other 223 greedy tokens in one more (``decoder_step_kernel``, which streams
each token to host memory; fixed length, no EOS stop) — with seeded random-init weights of the
whisper-large-v3-turbo architecture. The reference's timing boundary is kept: the clock starts at an
in-memory waveform and stops at the token-id list (reference custom/model.py:179-225). Each timed
transcribe runs inside a roctx range (``bench:30s:rep<i>``; flash_whisper_amd.trace).

Reported metric: decode-step us (median GPU time per decoder step: HIP events around the one launch
that decodes every token after the first, divided by its steps, inside the timed transcribes), the rate
of the step's algorithmic bytes (the per-step bytes of the path, fp16 LM head included: the decoder
weights, cross K/V, self K/V rows and the tied embedding), the 30 s-clip E2E ms and TTFT (median and p90).

``roofline`` covers the dominant kernel, the persistent decoder step (per step the 4 decoder layers,
final LN, int8 pre-pass LM head, argmax and finalize): ``achieved`` is the step's algorithmic bytes
(fp16 LM head, as the unit is defined) over its time, HIP events around that launch on the stream it
runs on, divided by its steps (``us_per_launch`` / ``steps_per_launch``); ``achieved_read`` counts the
bytes the step must read with the int8 table instead. ``traffic`` is the kernel's calibrated PMC fetch +
write bytes per step from profiles/decoder_step_kernel_traffic.md. ``lm_head`` times the 34-launch
step's LM-head kernel alone (final LN + int8 pre-pass + exact fp16 candidates + argmax, h ~ N(0, 1))
over rotating copies of its table (more than the 256 MB MALL) in a hipGraph between HIP events on the
graph's stream; with ``--fp16-lm-head`` the step is not one launch and ``roofline`` is that kernel's.

``clips`` holds the reference's clip-length rows: 5 s and 15 s seeded clips, 20 transcribes each with
the token budget scaled to the clip (37 and 112), and the 30 s timed transcribes; E2E and TTFT median
and p90. ``configs`` times the path's per-config units: standalone (each over rotating buffers of more
than 300 MB so every call streams from HBM: the log-mel front end, the 34-launch step's split-K self
attention at L in {1, 64, 224, 448}, and its cross attention over 1500 frames + LN/GELU MLP), and
``in_kernel``: the same units as phases of the persistent step, from its profiling build. Every row
names its code path. ``cpu_baseline`` times the reference's PyTorch path in fp32 on this host's cores
(oracle.torch_cpu; 5 end-to-end transcribes and 50 reps per config unit) and runs the numpy oracle once
end to end as the id check.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

METRIC = 'decode-step µs + achieved HBM GB/s; 30 s-clip E2E ms & TTFT, batch 1'
HBM_PEAK_GBPS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
LM_KERNEL = {False: 'lm_head_kernel<true> (final LN + LM head GEMV + argmax)',
             True: 'lm_head_q8_kernel<true> (final LN + int8 pre-pass over the LM head + exact fp16 candidates + argmax)'}
LM_TRAFFIC = {False: 'profiles/lm_head_kernel_traffic.md', True: 'profiles/lm_head_q8_kernel_traffic.md'}
STEP_KERNEL = ('decoder_step_kernel (persistent: every token after the first in one launch; per step 4 decoder '
               'layers, final LN, int8 pre-pass LM head with exact fp16 candidates, argmax, finalize)')
STEP_TRAFFIC = 'profiles/decoder_step_kernel_traffic.md'
ROTATE_BYTES = 300 << 20  # more than the 256 MB MALL
LOG_MEL_BYTES = 3_558_912          # 480000 fp32 in, 128 x 3000 fp32 out, the 201 x 128 filterbank
CROSS_MLP_BYTES = 33_925_120       # cross K/V 7.68 MB + fc1, fc2 26.2 MB + vectors


def decode_step_bytes(dims, length, q8=False):
    """Algorithmic bytes of one decoder step attending over `length` cached positions: every decoder
    weight, bias and LayerNorm vector once, the tied 51866 x 1280 LM head once (fp16; with `q8` the
    int8 table and its per-row scale and bound instead), the cross K/V of all layers, the self K/V rows
    0..length-1 of all layers, the two embedding rows and the suppress mask."""
    d, f, L = dims.d_model, dims.ffn, dims.dec_layers
    per_layer = 2 * (3 * d * d + 3 * d * d + 2 * d * f) + 2 * (3 * d + d + d + d + f + d) + 2 * 6 * d
    weights = L * per_layer + 2 * 2 * d  # + final LN
    lm_head = (dims.vocab * d + 8 * dims.vocab) if q8 else 2 * dims.vocab * d
    cross = L * 2 * dims.heads * dims.enc_len * dims.head_dim * 2
    self_kv = L * 2 * dims.heads * length * dims.head_dim * 2
    return weights + lm_head + cross + self_kv + 2 * 2 * d + dims.vocab


def encoder_flops(dims):
    """Algorithmic FLOPs of the encoder stage: the conv stem (conv1 over 2 x enc_len frames, conv2 with
    stride 2), every layer's q/k/v, attention (Q K^T and P V), out, fc1 and fc2 products, and the cross
    K/V projection of all decoder layers (2.313 TFLOP for whisper-large-v3-turbo)."""
    t, d, f = dims.enc_len, dims.d_model, dims.ffn
    stem = 2 * (2 * t) * d * (3 * dims.n_mels) + 2 * t * d * (3 * d)
    layer = 2 * t * (3 * d) * d + 2 * 2 * t * t * d + 2 * t * d * d + 2 * 2 * t * f * d
    return stem + dims.enc_layers * layer + 2 * t * (dims.dec_layers * 2 * d) * d


def measured_traffic(path, per='launch'):
    """HBM bytes per launch (or per step) of a kernel from its committed, copy-calibrated rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE passes), or None when that summary is absent."""
    import pathlib
    import re

    f = pathlib.Path(__file__).resolve().parent / path
    if not f.exists():
        return None
    m = re.search(rf'^traffic_bytes_per_{per}:\s*(\d+)', f.read_text(), re.M)
    return int(m.group(1)) if m else None


def lm_head_bytes(dims, q8):
    """Bytes one fused LM-head launch must read. fp16 kernel: the embedding, the suppress mask, h, x,
    gamma, beta (the unit's algorithmic bytes). int8 pre-pass kernel: the int8 table, its per-row scale
    and error bound (8 B a row), the mask and the four vectors; the fp16 rows of the candidates it
    re-scores (a few per block, data-dependent) are not counted."""
    vec = dims.vocab + 4 * 2 * dims.d_model
    return (dims.vocab * dims.d_model + 8 * dims.vocab + vec) if q8 else (2 * dims.vocab * dims.d_model + vec)


def lm_head_unit_bytes(dims):
    """The LM-head unit's algorithmic bytes: the fp16 table, the suppress mask, h, gamma, beta and the
    8-byte packed result (132 836 514 B for whisper-large-v3-turbo)."""
    return 2 * dims.vocab * dims.d_model + dims.vocab + 3 * 2 * dims.d_model + 8


def selftest_gate(selftest):
    """None when every kernel self-check passed, else the reason to refuse to report: like the
    reference, which counts its custom path as verified only when selftest['ok'] is True
    (reference bench.py:147, reporting.py:107-108)."""
    if selftest.get('ok') is True:
        return None
    failed = [c['name'] for c in selftest.get('checks', []) if not c.get('ok')]
    return f'selftest failed: {failed}' if failed else 'selftest did not run'


def graph_time_us(call, reps, replays=7):
    """Per-call time of `call(i)` (enqueues call i on the current stream): a hipGraph of `reps` calls is
    captured on a side stream and replayed `replays` times between HIP events recorded on that
    stream; the median of the replays' per-call averages."""
    import torch

    stream = torch.cuda.Stream()
    with torch.inference_mode(), torch.cuda.stream(stream):
        for i in range(min(reps, 8)):
            call(i)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                call(i)
        graph.replay()
        per_call = []
        for _ in range(replays):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            graph.replay()
            end.record(stream)
            end.synchronize()
            per_call.append(start.elapsed_time(end) * 1e3 / reps)
    del graph
    return statistics.median(per_call)


def time_lm_head(model, reps, q8):
    """Average us per launch of the LN + LM-head + argmax kernel alone (no finalize launch), over
    copies of its table (>= 256 MB in all, more than the MALL, so each launch reads its table from HBM)."""
    import torch

    ext, d = model.ext, model.dims
    copies = 5 if q8 else 3
    if q8:
        tables = [(model.lm_q8, model.lm_meta)] + [(model.lm_q8.clone(), model.lm_meta.clone())
                                                   for _ in range(copies - 1)]
    else:
        tables = [model.lm_head] + [model.lm_head.clone() for _ in range(copies - 1)]
    best = torch.zeros(1, dtype=torch.long, device='cuda')
    g, b, eps = model.final_ln
    gen = torch.Generator(device='cuda').manual_seed(4)
    h = torch.randn(d.d_model, generator=gen, device='cuda').half()  # the LM-head unit's input, N(0, 1)
    x = torch.zeros_like(h)

    def launch(i):
        if q8:
            wq, meta = tables[i % copies]
            ext.lm_head_argmax_q8(h, x, g, b, eps, model.lm_head, wq, meta, model.suppress, best, None, None, None,
                                  d.max_pos)
        else:
            ext.lm_head_argmax_fused(h, x, g, b, eps, tables[i % copies], model.suppress, best, None, None, None,
                                     d.max_pos)

    us = graph_time_us(launch, reps)
    del tables
    return us


def launch_floor_us(model, reps=200):
    """Cost of one dependent launch at the decode step's granularity: a chain of add_layernorm launches
    (one block: each reads the residual the previous launch wrote, adds, normalises, writes)."""
    import torch

    ext, dm = model.ext, model.dims.d_model
    h = torch.randn(dm, dtype=torch.float16, device='cuda') * 0.01
    x = torch.zeros_like(h)
    y = torch.empty_like(h)
    g, b = torch.ones_like(h), torch.zeros_like(h)
    return graph_time_us(lambda i: ext.add_layernorm(h, x, g, b, y, 1e-5), reps)


def log(msg):
    """A progress line on stderr (stdout carries only the JSON line)."""
    print(f'bench: {msg}', file=sys.stderr, flush=True)


def percentile(values, p):
    """Linear interpolation between the order statistics, as the reference's report (reporting.py:31-38)."""
    v = sorted(values)
    pos = (len(v) - 1) * p
    lo, hi = int(pos), min(int(pos) + 1, len(v) - 1)
    return v[lo] + (v[hi] - v[lo]) * (pos - lo)


def latency_row(results, seconds):
    """E2E / TTFT median and p90 (ms) over `results` (transcribe dicts), audio seconds per second."""
    e2e, ttft = [r['e2e_s'] * 1e3 for r in results], [r['ttft_s'] * 1e3 for r in results]
    med = statistics.median(e2e)
    return {'e2e_ms': round(med, 3), 'e2e_p90_ms': round(percentile(e2e, 0.9), 3),
            'ttft_ms': round(statistics.median(ttft), 3), 'ttft_p90_ms': round(percentile(ttft, 0.9), 3),
            'audio_s_per_s': round(seconds / (med * 1e-3), 1), 'reps': len(results),
            'tokens': results[0]['n_tokens']}


def clip_rows(model, reps, tokens_30s):
    """The reference's 5 s and 15 s clip rows (runner.py:185-194: 20 reps per length, distinct audio per
    rep): seeded synthetic clips of that length (the encoder still runs the zero-padded 30 s window), with
    the 30 s token budget scaled to the clip (37 and 112 of 224: random-init weights never emit EOS)."""
    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.trace import trace_range

    rows = {}
    for seconds in (5, 15):
        tokens = round(tokens_30s * seconds / 30)
        clips = [synthetic_clip(200 + i, n_samples=seconds * 16000) for i in range(reps)]
        model.transcribe(clips[0], max_new_tokens=tokens, stop_at_eos=False)  # warm-up at this length
        res = []
        for i, clip in enumerate(clips):
            with trace_range(f'bench:{seconds}s:rep{i}'):
                res.append(model.transcribe(clip, max_new_tokens=tokens, stop_at_eos=False))
        rows[f'{seconds}s'] = latency_row(res, seconds)
    return rows


def _row(us, nbytes, launches, sample):
    gbps = nbytes / (us * 1e-6) / 1e9
    return {'us': round(us, 2), 'bytes': int(nbytes), 'gbps': round(gbps, 1), 'frac': round(gbps / HBM_PEAK_GBPS, 4),
            'launches': launches, 'sample': sample}


def config_rows(model, reps):
    """The path's per-config units, each as the median over 7 replays of a hipGraph of `reps` calls
    cycling through more than 300 MB of distinct inputs (so every call reads from HBM, not the MALL)."""
    import torch

    from flash_whisper_amd._lib import ACT_GELU
    from flash_whisper_amd.selftest import workspace

    ext, d = model.ext, model.dims
    half, dev = torch.float16, 'cuda'
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    randn = lambda *shape, std=1.0: (torch.randn(*shape, generator=gen, device=dev) * std).to(half)
    rows = {}

    # config 1: log-mel of a 30 s waveform (3 tones + noise like the benchmark clip, different seeds)
    from flash_whisper_amd.audio import synthetic_clip

    per = 480000 * 4 + 128 * 3000 * 4 + 3000 * 128 * 2
    n = -(-ROTATE_BYTES // per)
    waves = [torch.from_numpy(synthetic_clip(1000 + i)).to(dev) for i in range(n)]
    outs = [(torch.empty(128, 3000, device=dev), torch.empty(3000, 128, dtype=half, device=dev)) for _ in range(n)]
    ws = ext.log_mel_workspace(480000)
    ext.log_mel_prepare(model.mel_filters, ws)  # once per filterbank, as the model does
    us = graph_time_us(lambda i: ext.log_mel_run(waves[i % n], model.mel_filters, outs[i % n][0], outs[i % n][1],
                                                 ws), reps)
    rows['log_mel'] = _row(us, LOG_MEL_BYTES, 2, f'{n} distinct 30 s clips, {reps} calls per graph (per-clip '
                           'frames + finalize launches; the filterbank prepared once)')
    rows['log_mel']['code_path'] = 'logmel_frames_kernel + logmel_finalize_kernel, as transcribe runs them'
    del waves, outs, ws

    # config 2: split-K self attention (split + combine, the reference op) over an fp16 K/V cache
    heads, hd, max_pos = d.heads, d.head_dim, d.max_pos
    per = 2 * heads * max_pos * hd * 2
    n = -(-ROTATE_BYTES // per)
    caches = [(randn(heads, max_pos, hd), randn(heads, max_pos, hd)) for _ in range(n)]
    q, kn, vn = randn(heads * hd), randn(heads, hd), randn(heads, hd)
    out = torch.empty(heads * hd, dtype=half, device=dev)
    pm, pl, pa = workspace(heads, -(-max_pos // 64))
    self_rows = {}
    for length in (1, 64, 224, 448):
        state = torch.tensor([length - 1, 0], dtype=torch.long, device=dev)
        us = graph_time_us(lambda i: ext.decode_attention(q, caches[i % n][0], caches[i % n][1], out, state, kn, vn,
                                                          pm, pl, pa, hd ** -0.5), reps)
        self_rows[f'L{length}'] = _row(us, 5120 * length + 15360, 2,
                                       f'{n} distinct [20, 448, 64] K/V caches, {reps} calls per graph')
    self_rows['code_path'] = ('attn_split_kernel + attn_combine_kernel (decode_attention: the 34-launch step\'s '
                              'kernels, the reference op\'s granularity); the product\'s in-kernel phase is '
                              'in_kernel.self_attention')
    rows['self_attention'] = self_rows
    del caches

    # config 3: cross attention over 1500 frames, then residual + LN + fc1 + GELU, then fc2
    dm, ffn, t = d.d_model, d.ffn, d.enc_len
    per = CROSS_MLP_BYTES
    n = -(-ROTATE_BYTES // per)
    sets = [dict(k=randn(heads, t, hd), v=randn(heads, t, hd), w1=randn(ffn, dm, std=0.02), b1=randn(ffn, std=0.02),
                 w2=randn(dm, ffn, std=0.02), b2=randn(dm, std=0.02)) for _ in range(n)]
    q, h = randn(dm), randn(dm)
    g, b = torch.ones(dm, dtype=half, device=dev), torch.zeros(dm, dtype=half, device=dev)
    attn, h_out = torch.empty(dm, dtype=half, device=dev), torch.empty(dm, dtype=half, device=dev)
    f, mlp = torch.empty(ffn, dtype=half, device=dev), torch.empty(dm, dtype=half, device=dev)
    pm, pl, pa = workspace(heads, -(-t // 64))

    def cross_mlp(i):
        s = sets[i % n]
        ext.decode_attention(q, s['k'], s['v'], attn, None, None, None, pm, pl, pa, hd ** -0.5)
        ext.ln_gemv(h, attn, h_out, g, b, 1e-5, s['w1'], s['b1'], f, act=ACT_GELU)
        ext.gemv(f, s['w2'], s['b2'], mlp)

    us = graph_time_us(cross_mlp, reps)
    rows['cross_attention_mlp'] = _row(us, CROSS_MLP_BYTES, 4, f'{n} distinct K/V + MLP weight sets, {reps} calls '
                                       'per graph; the MLP residual is added by the next LayerNorm, as in the step')
    rows['cross_attention_mlp']['code_path'] = ('decode_attention + ln_gemv(GELU) + gemv: the 34-launch step\'s '
                                                'kernels; the product\'s phases are in_kernel.cross_attention_mlp')
    del sets
    torch.cuda.empty_cache()
    return rows


def in_kernel_rows(tokens, dims, timeout_s=600):
    """Configs 2-4 as the product runs them: phases of the persistent decoder step, timed by its
    profiling build (flash_whisper_amd.step_timeline: the 100 MHz wall clock stored by every block at
    fixed points of each step; a child process on this GPU while this one is idle). Each row is the
    phases' share of the step (from the previous phase's last output to this phase's last output,
    hand-off included), median over the steps and the 4 layers, on the config's algorithmic bytes."""
    import tempfile

    root = os.path.dirname(os.path.abspath(__file__))
    lib = os.path.join(root, 'flash_whisper_amd', 'libflash_whisper_timeline.so')
    if not os.path.exists(lib):
        return {'skipped': f'{lib} not built'}
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, 'phases.json')
        env = dict(os.environ, FW_LIBRARY=lib)
        proc = subprocess.run([sys.executable, '-m', 'flash_whisper_amd.step_timeline', '--tokens', str(tokens),
                               '--json', path], cwd=root, env=env, capture_output=True, text=True, timeout=timeout_s)
        if proc.returncode != 0:
            return {'skipped': f'step_timeline exited with {proc.returncode}: {proc.stderr[-400:]}'}
        with open(path) as f:
            tl = json.load(f)
    ph = tl['phases']
    rows = {'code_path': 'decoder_step_kernel<1> phases (the product\'s decode), from its profiling build '
                         '(libflash_whisper_timeline.so); medians over a 224-token decode and 8 steps from '
                         'position 440, all 4 layers',
            'step_period_us': tl['step_period_us']}
    rows['self_attention'] = {
        k: dict(_row(v['dur_us'], 5120 * int(k[1:]) + 15360, 0, f'{v["samples"]} layer-steps with L in '
                     f'[{int(k[1:]) - 4}, {int(k[1:])}]'), block_work_us=v['work_us'])
        for k, v in tl['self_attention_by_length'].items()}
    cross = ph['cross attention']['dur_us'] + ph['LN3 + fc1 + GELU']['dur_us'] + ph['fc2']['dur_us']
    rows['cross_attention_mlp'] = dict(
        _row(cross, CROSS_MLP_BYTES, 0, 'cross attention + LN3/fc1/GELU + fc2 phases per layer (the cross-out '
             'projection between them is its own phase, cross_out_us)'),
        cross_attention_us=ph['cross attention']['dur_us'], cross_out_us=ph['cross-out']['dur_us'],
        fc1_us=ph['LN3 + fc1 + GELU']['dur_us'], fc2_us=ph['fc2']['dur_us'])
    rows['lm_head'] = _row(tl['lm_head_us'], lm_head_unit_bytes(dims), 0, 'final LN + int8 pre-pass + exact fp16 '
                           'candidates + argmax + finalize, from the last fc2 output to the token stored')
    read = lm_head_bytes(dims, True)  # what the phase reads: the int8 table, its scales and bounds
    rows['lm_head'].update(bytes_read=read, frac_read=round(read / (tl['lm_head_us'] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4))
    rows['phases'] = ph
    return rows


def serving_throughput(model, lanes, clips, tokens):
    """Clips per second with `lanes` clips in flight (flash_whisper_amd.serve) against one at a time, on
    `clips` seeded 30 s clips of `tokens` greedy tokens each (fixed length)."""
    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.serve import Scheduler

    batch = [synthetic_clip(100 + i) for i in range(clips)]
    out = {'lanes': lanes, 'clips': clips, 'tokens_per_clip': tokens}
    for n in (1, lanes):
        sched = Scheduler(model, lanes=n)
        sched.transcribe_many(batch[:n], max_new_tokens=tokens, stop_at_eos=False)  # warm-up
        res = sched.transcribe_many(batch, max_new_tokens=tokens, stop_at_eos=False)
        out[f'clips_per_s_{n}_lane' + ('s' if n > 1 else '')] = round(clips / res[0]['wall_s'], 2)
        del sched
    return out


def _host_description():
    model_line = None
    try:
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
        model_line = next((ln.split(':', 1)[1].strip() for ln in out.splitlines() if ln.startswith('Model name')), None)
    except (OSError, subprocess.SubprocessError):
        pass
    return model_line or platform.processor() or platform.machine()


def _blas_threads():
    """(library, threads) of the BLAS numpy uses, as threadpoolctl reports it."""
    try:
        from threadpoolctl import threadpool_info

        info = [i for i in threadpool_info() if i.get('user_api') == 'blas']
        if info:
            return f"{info[0].get('internal_api')} {info[0].get('version')}", int(info[0]['num_threads'])
    except ImportError:
        pass
    return 'unknown', os.cpu_count()


def cpu_baseline(model, tokens, gpu_ids, reps, config_reps):
    """Two CPU legs on this host, on the benchmark clip and the same seeded weights.

    - The reference's PyTorch path in fp32 (oracle.torch_cpu: transformers Whisper, torch.stft log-mel,
      greedy loop over the HF KV cache; custom/pytorch_model.py:29-89): `reps` end-to-end transcribes of
      `tokens` tokens and the per-config units over `config_reps` each. `value` is its median decoder step
      (each token's forward + argmax, pooled over the reps).
    - The numpy oracle once end to end (log-mel, fp16-rounded encoder, cross K/V, every decoder step in
      fp32 with the reference's fp16 rounding points): its ids are checked against the GPU's bit for bit."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from flash_whisper_amd import weights
    from flash_whisper_amd.audio import synthetic_clip
    from oracle.decoder import DecoderOracle, masked_argmax, suppress_masks
    from oracle.encoder import cross_kv, encoder_forward
    from oracle.logmel import log_mel
    from oracle.pipeline import pad_wave
    from oracle.torch_cpu import baseline

    d, setup = model.dims, model.setup
    specs = weights.param_specs(d)
    with ThreadPoolExecutor(16) as pool:  # the host generator runs in C and releases the GIL
        arrays = list(pool.map(lambda s: weights.host_param(*s, seed=model.seed), specs))
    params = {s[0]: a for s, a in zip(specs, arrays)}
    del arrays
    log('cpu baseline: host parameters generated')
    clip = synthetic_clip(0)
    base, first = suppress_masks(d.vocab, setup.suppress, setup.begin_suppress)
    step_s = []

    t0 = time.perf_counter()
    mel = log_mel(pad_wave(clip)).astype(np.float16).astype(np.float32)
    t_mel = time.perf_counter()
    enc = encoder_forward(params, mel, d)
    ckv = cross_kv(params, enc, d)
    t_enc = time.perf_counter()
    dec = DecoderOracle(params, d, ckv)
    ids, pos = [], 0
    for i, tok in enumerate(setup.prompt):
        s0 = time.perf_counter()
        logits = dec.step(tok, pos)
        step_s.append(time.perf_counter() - s0)
        pos += 1
        if i == len(setup.prompt) - 1:
            ids.append(masked_argmax(logits, first))
    t_first = time.perf_counter()
    while len(ids) < tokens:
        s0 = time.perf_counter()
        logits = dec.step(ids[-1], pos)
        step_s.append(time.perf_counter() - s0)
        pos += 1
        ids.append(masked_argmax(logits, base))
    t_end = time.perf_counter()
    del dec, enc, ckv
    lib, threads = _blas_threads()
    ms = lambda a, b: round((b - a) * 1e3, 1)
    oracle = dict(kind='numpy oracle, fp32 math with the reference\'s fp16 rounding points', runs=1,
                  step_us=round(statistics.median(step_s) * 1e6, 1), e2e_ms=ms(t0, t_end), ttft_ms=ms(t0, t_first),
                  mel_ms=ms(t0, t_mel), encoder_ms=ms(t_mel, t_enc), decode_ms=ms(t_enc, t_end),
                  ids_match_gpu=ids == list(gpu_ids), blas=lib, blas_threads=threads)

    log(f'cpu baseline: numpy oracle done ({oracle["e2e_ms"] / 1e3:.1f} s end to end)')
    torch_cpu = baseline(params, d, setup, clip, tokens, reps=reps, config_reps=config_reps,
                         progress=lambda m: log(f'cpu baseline: {m}'))
    log('cpu baseline: fp32 PyTorch path done')
    cpu_ids = torch_cpu.pop('token_ids')
    first_diff = next((i for i, (a, b) in enumerate(zip(cpu_ids, gpu_ids)) if a != b), None)
    import torch

    return dict(value=torch_cpu['step_us'], unit='us/decode-step', cores=torch_cpu['threads'], kind='port',
                sample=f'the reference\'s PyTorch path (transformers Whisper + greedy loop over the HF KV cache) '
                       f'in fp32 on {torch_cpu["threads"]} host threads: {reps} end-to-end transcribes of the '
                       f'benchmark clip ({tokens} tokens each, after an 8-token warm-up), value = median decoder '
                       f'step pooled over them; configs = the per-config units, median of {config_reps} each',
                precision='fp32', e2e_ms=torch_cpu['e2e_ms'], e2e_p90_ms=torch_cpu['e2e_p90_ms'],
                ttft_ms=torch_cpu['ttft_ms'], mel_ms=torch_cpu['mel_ms'], encoder_ms=torch_cpu['encoder_ms'],
                decode_ms=torch_cpu['decode_ms'], reps=reps, configs=torch_cpu['configs'],
                fp32_ids_first_difference_from_gpu=first_diff, torch_threads=torch_cpu['threads'],
                torch=torch.__version__, nproc=os.cpu_count(), host=_host_description(), oracle=oracle)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=10, help='timed transcribes')
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--tokens', type=int, default=224)
    ap.add_argument('--kernel-reps', type=int, default=100)
    ap.add_argument('--clip-reps', type=int, default=20, help='transcribes per 5 s and 15 s clip row (0: skip)')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--cpu-reps', type=int, default=5, help='end-to-end transcribes of the fp32 PyTorch CPU baseline')
    ap.add_argument('--cpu-config-reps', type=int, default=50, help='reps per config unit of the CPU baseline')
    ap.add_argument('--no-configs', action='store_true', help='skip the per-config rows')
    ap.add_argument('--lanes', type=int, default=4, help='clips in flight for the serving-throughput extra (0: skip)')
    ap.add_argument('--fp16-lm-head', action='store_true',
                    help='decode with the fp16 LM-head kernel instead of the int8 pre-pass one (same tokens)')
    ap.add_argument('--copy-calibration', action='store_true',
                    help='also run 4 plain 256 MiB device copies (the reference kernel for PMC byte counters)')
    ap.add_argument('--decode-replays', type=int, default=0,
                    help='profiling aid: after one transcribe, replay the 8-step decoder graph N times and exit')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (--gpus {args.gpus} requested): this build runs the batch-1 path on '
              f'a single MI355X; independent clips would shard one per GPU with no exchange.', file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.config import CHUNK
    from flash_whisper_amd.model import CustomModel
    from flash_whisper_amd.trace import trace_range

    model = CustomModel(seed=0, lm_q8=not args.fp16_lm_head)
    reason = selftest_gate(model.selftest)
    if reason:
        print(reason, file=sys.stderr)
        sys.exit(1)
    clip = synthetic_clip(0)
    if args.decode_replays:
        model.transcribe(clip, max_new_tokens=args.tokens, stop_at_eos=False)
        for _ in range(args.decode_replays):
            model.graph_chunk.replay()
        if args.copy_calibration:
            src = torch.empty(128 << 20, dtype=torch.float16, device='cuda')
            dst = torch.empty_like(src)
            for _ in range(4):
                dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'decode_replays': args.decode_replays, 'steps_per_replay': CHUNK}), flush=True)
        return
    for i in range(args.warmup):
        with trace_range(f'bench:warmup:rep{i}'):
            model.transcribe(clip, max_new_tokens=args.tokens, stop_at_eos=False)

    model.record_events = True
    rows, step_us = [], []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    launch_us, launch_steps = [], 0
    for i in range(args.steps):
        with trace_range(f'bench:30s:rep{i}'):
            res = model.transcribe(clip, max_new_tokens=args.tokens, stop_at_eos=False)
        rows.append(res)
        if model.decode_events:  # the whole decode as one launch
            (a, b, n), = model.decode_events
            launch_us.append(a.elapsed_time(b) * 1e3)
            launch_steps = n
            step_us.append(launch_us[-1] / n)
        else:
            chunk_ms = [a.elapsed_time(b) for a, b in model.chunk_events]
            step_us.append(sum(chunk_ms) * 1e3 / (len(chunk_ms) * CHUNK))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    model.record_events = False

    log(f'{args.steps} timed 30 s transcribes done')
    q8 = model.use_lm_q8
    clips = clip_rows(model, args.clip_reps, args.tokens) if args.clip_reps > 0 else {}
    clips['30s'] = latency_row(rows, 30)
    log('5 s and 15 s clip rows done')
    with trace_range('bench:lm_head'):
        lm_us = time_lm_head(model, args.kernel_reps, q8)
        lm16_us = time_lm_head(model, args.kernel_reps, False) if q8 else lm_us
    with trace_range('bench:launch_floor'):
        floor_us = launch_floor_us(model)
    with trace_range('bench:configs'):
        configs = None if args.no_configs else config_rows(model, args.kernel_reps)
    if configs is not None:
        log('standalone config rows done')
        configs['in_kernel'] = in_kernel_rows(args.tokens, model.dims)
        log('in-kernel phase rows done')
    log('LM-head, launch-floor and config rows done')
    with trace_range('bench:serving'):
        serve = serving_throughput(model, args.lanes, 2 * args.lanes, args.tokens) if args.lanes > 1 else None
    if args.copy_calibration:
        src = torch.empty(128 << 20, dtype=torch.float16, device='cuda')
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    lm_bytes, lm_bytes_s8d = lm_head_bytes(model.dims, q8), lm_head_unit_bytes(model.dims)
    lm_gbps = lm_bytes / (lm_us * 1e-6) / 1e9
    lm_gbps_s8d = lm_bytes_s8d / (lm_us * 1e-6) / 1e9
    lm16_gbps = lm_bytes_s8d / (lm16_us * 1e-6) / 1e9

    # mean cached length over the decode: positions 4 .. 4 + tokens - 1 attend over pos + 1 keys
    lengths = np.arange(len(model.prompt) + 1, len(model.prompt) + args.tokens + 1)
    step_bytes = float(np.mean([decode_step_bytes(model.dims, int(L)) for L in lengths]))
    read_bytes = float(np.mean([decode_step_bytes(model.dims, int(L), q8) for L in lengths]))
    med_step = statistics.median(step_us)
    step_gbps = step_bytes / (med_step * 1e-6) / 1e9
    med = lambda k: statistics.median(r[k] for r in rows) * 1e3
    enc_tflops = encoder_flops(model.dims) / (med('encoder_s') * 1e-3) / 1e12

    out = {
        'metric': METRIC, 'value': round(med_step, 2), 'unit': 'us/decode-step', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(elapsed * 1e3 / args.steps, 3),
        'higher_is_better': False, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'fp16',
        'data': 'synthetic: seeded 30 s clip (3 tones + noise), seeded random-init N(0, 0.02) fp16 weights',
        'config': {'workload': f'whisper-large-v3-turbo batch 1: 30 s clip -> log-mel -> 32-layer encoder -> '
                               f'{args.tokens} greedy tokens (prompt pass and decode each one persistent launch)',
                   'clip_s': 30, 'tokens': args.tokens, 'batch': 1},
        'decode_step_us': round(med_step, 2),
        # the step's algorithmic bytes (fp16 LM head) over its time; 214 MB of them (decoder weights,
        # cross K/V) stay resident in the 256 MB MALL across steps, so this is not an HBM rate
        'decode_step_bytes': int(step_bytes), 'decode_step_algorithmic_gbps': round(step_gbps, 1),
        'decode_step_roofline_frac': round(step_gbps / HBM_PEAK_GBPS, 4),
        'decode_step_bytes_read': int(read_bytes),
        'decode_launch_floor_us': round(floor_us, 2),
        'e2e_ms': round(med('e2e_s'), 3), 'ttft_ms': round(med('ttft_s'), 3),
        'e2e_p90_ms': clips['30s']['e2e_p90_ms'], 'ttft_p90_ms': clips['30s']['ttft_p90_ms'],
        'mel_ms': round(med('mel_s'), 3),
        'encoder_ms': round(med('encoder_s'), 3), 'decode_ms': round(med('decode_s'), 3),
        'encoder_tflops': round(enc_tflops, 1), 'encoder_mfma_frac': round(enc_tflops / MFMA_FP16_PEAK_TFLOPS, 4),
        'n_tokens': rows[-1]['n_tokens'],
        # int8 LM-head rows each block of the step kernel keeps in LDS for the whole launch
        'decode_step_lm_resident_rows': int(model.ext.lib.fw_decoder_step_resident_rows()),
    }
    lm_head = {'kernel': LM_KERNEL[q8], 'bound': 'hbm', 'achieved': round(lm_gbps, 1),
               'peak': HBM_PEAK_GBPS, 'unit': 'GB/s', 'frac': round(lm_gbps / HBM_PEAK_GBPS, 4),
               'traffic': measured_traffic(LM_TRAFFIC[q8]), 'traffic_source': LM_TRAFFIC[q8],
               'us_per_launch': round(lm_us, 2), 'bytes_per_launch': lm_bytes,
               'bytes_s8d': lm_bytes_s8d, 'achieved_s8d': round(lm_gbps_s8d, 1),
               'frac_s8d': round(lm_gbps_s8d / HBM_PEAK_GBPS, 4),
               'fp16_head': {'kernel': LM_KERNEL[False], 'us_per_launch': round(lm16_us, 2),
                             'achieved': round(lm16_gbps, 1), 'frac': round(lm16_gbps / HBM_PEAK_GBPS, 4),
                             'traffic': measured_traffic(LM_TRAFFIC[False])}}
    if model.persistent_step and model.persistent_head and q8:
        read_gbps = read_bytes / (med_step * 1e-6) / 1e9
        out['roofline'] = {'kernel': STEP_KERNEL, 'bound': 'hbm', 'achieved': round(step_gbps, 1),
                           'peak': HBM_PEAK_GBPS, 'unit': 'GB/s', 'frac': round(step_gbps / HBM_PEAK_GBPS, 4),
                           'traffic': measured_traffic(STEP_TRAFFIC, 'step'), 'traffic_per': 'step',
                           'traffic_source': STEP_TRAFFIC,
                           'us_per_step': round(med_step, 2), 'bytes_per_step': round(step_bytes),
                           'bytes_read': round(read_bytes), 'achieved_read': round(read_gbps, 1),
                           'frac_read': round(read_gbps / HBM_PEAK_GBPS, 4)}
        if launch_us:  # one launch decodes every token after the first
            out['roofline'].update({'steps_per_launch': launch_steps,
                                    'us_per_launch': round(statistics.median(launch_us), 1),
                                    'bytes_per_launch': round(step_bytes * launch_steps)})
        out['lm_head'] = lm_head
    else:
        out['roofline'] = lm_head
    out['clips'] = clips
    if configs is not None:
        out['configs'] = configs
    if serve is not None:
        out['serving'] = serve
    if not args.no_cpu_baseline:
        with trace_range('bench:cpu_baseline'):
            out['cpu_baseline'] = cpu_baseline(model, args.tokens, rows[-1]['token_ids'], args.cpu_reps,
                                               args.cpu_config_reps)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()

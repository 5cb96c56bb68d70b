"""Benchmark of the batch-1 Whisper-large-v3-turbo hot path on one MI355X.

Workload (one "step"): a full ``CustomModel.transcribe`` of a seeded 30 s synthetic clip — HIP log-mel,
32-layer MFMA encoder + cross K/V in a hipGraph, 4-token prompt, then 224 greedy tokens with the 8-step
decoder hipGraph (fixed length, no EOS stop), with seeded random-init weights of the
whisper-large-v3-turbo architecture. The reference's timing boundary is kept: the clock starts at an
in-memory waveform and stops at the token-id list (reference custom/model.py:179-225).

Reported metric: decode-step us (median GPU time per decoder step, HIP events around every 8-step graph
replay inside the timed transcribes), its achieved HBM GB/s from the algorithmic bytes of a step, the
30 s-clip E2E ms and TTFT. ``roofline`` covers the step's LM-head kernel (final LN + int8 pre-pass over
the tied embedding + exact fp16 logits of the candidate rows + argmax; ``--fp16-lm-head`` decodes with
the fp16 LM-head kernel instead, same tokens), timed standalone: a hipGraph of launches over rotating
copies of its table, so it streams from HBM as inside the step, between HIP events on the graph's
stream. ``cpu_baseline`` times the CPU oracle's decoder step on this host.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

import argparse
import json
import os
import platform
import statistics
import sys
import time

METRIC = 'decode-step µs + achieved HBM GB/s; 30 s-clip E2E ms & TTFT, batch 1'
HBM_PEAK_GBPS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
LM_KERNEL = {False: 'lm_head_kernel<true> (final LN + LM head GEMV + argmax)',
             True: 'lm_head_q8_kernel<true> (final LN + int8 pre-pass over the LM head + exact fp16 candidates + argmax)'}
LM_TRAFFIC = {False: 'profiles/lm_head_kernel_traffic.md', True: 'profiles/lm_head_q8_kernel_traffic.md'}


def decode_step_bytes(dims, length, q8=False):
    """Algorithmic HBM bytes of one decoder step attending over `length` cached positions: every decoder
    weight, bias and LayerNorm vector once, the tied 51866 x 1280 LM head once, the cross K/V of all
    layers, the self K/V rows 0..length-1 of all layers, the two embedding rows and the suppress mask."""
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


def measured_traffic(path):
    """HBM bytes per LM-head launch from the committed, copy-calibrated rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE passes), or None when that summary is absent."""
    import pathlib
    import re

    f = pathlib.Path(__file__).resolve().parent / path
    if not f.exists():
        return None
    m = re.search(r'^traffic_bytes_per_launch:\s*(\d+)', f.read_text(), re.M)
    return int(m.group(1)) if m else None


def lm_head_bytes(dims, q8):
    """Algorithmic bytes of one fused LM-head launch. fp16 kernel: the embedding, the suppress mask, h, x,
    gamma, beta. int8 pre-pass kernel: the int8 table, its per-row scale and error bound (8 B a row),
    the mask and the four vectors; the fp16 rows of the candidates it re-scores (a few per block,
    data-dependent) are not counted."""
    vec = dims.vocab + 4 * 2 * dims.d_model
    return (dims.vocab * dims.d_model + 8 * dims.vocab + vec) if q8 else (2 * dims.vocab * dims.d_model + vec)


def time_lm_head(model, reps, q8):
    """Average us per launch of the LN + LM-head + argmax kernel alone (no finalize launch): `reps`
    launches rotating over copies of its table (>= 256 MB in all, more than the MALL, so each launch
    reads its table from HBM) are captured in one hipGraph on a side stream and replayed between HIP
    events recorded on that stream."""
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
    h, x = model.h[0], model.pending
    stream = torch.cuda.Stream()

    def launch(i):
        if q8:
            wq, meta = tables[i % copies]
            ext.lm_head_argmax_q8(h, x, g, b, eps, model.lm_head, wq, meta, model.suppress, best, None, None, None,
                                  d.max_pos)
        else:
            ext.lm_head_argmax_fused(h, x, g, b, eps, tables[i % copies], model.suppress, best, None, None, None,
                                     d.max_pos)

    with torch.inference_mode(), torch.cuda.stream(stream):
        for i in range(2 * copies):
            launch(i)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                launch(i)
        graph.replay()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
    del tables, graph
    return start.elapsed_time(end) * 1e3 / reps


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


def cpu_baseline(model, seconds, tokens):
    """The CPU oracle's decoder step (numpy fp32 with the reference's fp16 rounding points) on this host,
    on the GPU model's cross K/V, for a bounded number of steps."""
    import numpy as np

    from flash_whisper_amd import weights
    from oracle.decoder import DecoderOracle

    d = model.dims
    names = [n for n, _, _ in weights.param_specs(d) if n.startswith('model.decoder.')]
    params = weights.host_params(d, model.seed, names)
    oracle = DecoderOracle(params, d, model.cross_kv.float().cpu().numpy())
    del params
    # the workload's step positions: the prompt and then the generated tokens (0 .. prompt + tokens - 1)
    n_steps = min(d.max_pos, len(model.prompt) + tokens - 1)
    tok, pos, times = model.prompt[0], 0, []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(times) < n_steps:
        t0 = time.perf_counter()
        logits = oracle.step(tok, pos)
        times.append(time.perf_counter() - t0)
        tok, pos = int(np.argmax(logits)), pos + 1
    threads = int(os.environ.get('OPENBLAS_NUM_THREADS') or os.environ.get('OMP_NUM_THREADS') or os.cpu_count())
    return dict(value=round(statistics.median(times) * 1e6, 1), unit='us/decode-step', cores=threads,
                kind='port',
                sample=f'{len(times)} decoder steps (positions 0..{len(times) - 1}) of the numpy oracle, fp32 math '
                       f'with fp16 rounding points, median; host {platform.processor() or platform.machine()}, '
                       f'nproc {os.cpu_count()}')


def main():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=10, help='timed transcribes')
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--tokens', type=int, default=224)
    ap.add_argument('--kernel-reps', type=int, default=60)
    ap.add_argument('--cpu-seconds', type=float, default=12.0)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--lanes', type=int, default=4, help='clips in flight for the serving-throughput extra (0: skip)')
    ap.add_argument('--fp16-lm-head', action='store_true',
                    help='decode with the fp16 LM-head kernel instead of the int8 pre-pass one (same tokens)')
    ap.add_argument('--copy-calibration', action='store_true',
                    help='also run 4 plain 256 MiB device copies (the reference kernel for PMC byte counters)')
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

    model = CustomModel(seed=0, lm_q8=not args.fp16_lm_head)
    if not model.selftest['ok']:
        print(f'selftest failed: {[c for c in model.selftest["checks"] if not c["ok"]]}', file=sys.stderr)
        sys.exit(1)
    clip = synthetic_clip(0)
    for _ in range(args.warmup):
        model.transcribe(clip, max_new_tokens=args.tokens, stop_at_eos=False)

    model.record_events = True
    rows, step_us = [], []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = model.transcribe(clip, max_new_tokens=args.tokens, stop_at_eos=False)
        rows.append(res)
        chunk_ms = [a.elapsed_time(b) for a, b in model.chunk_events]
        step_us.append(sum(chunk_ms) * 1e3 / (len(chunk_ms) * CHUNK))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    model.record_events = False

    q8 = model.use_lm_q8
    lm_us = time_lm_head(model, args.kernel_reps, q8)
    lm16_us = time_lm_head(model, args.kernel_reps, False) if q8 else lm_us
    serve = serving_throughput(model, args.lanes, 2 * args.lanes, args.tokens) if args.lanes > 1 else None
    if args.copy_calibration:
        src = torch.empty(128 << 20, dtype=torch.float16, device='cuda')
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    lm_bytes = lm_head_bytes(model.dims, q8)
    lm_gbps = lm_bytes / (lm_us * 1e-6) / 1e9

    # mean cached length over the decode: positions 4 .. 4 + tokens - 1 attend over pos + 1 keys
    lengths = np.arange(len(model.prompt) + 1, len(model.prompt) + args.tokens + 1)
    step_bytes = float(np.mean([decode_step_bytes(model.dims, int(L), q8) for L in lengths]))
    ref_step_bytes = float(np.mean([decode_step_bytes(model.dims, int(L)) for L in lengths]))
    med_step = statistics.median(step_us)
    step_gbps = step_bytes / (med_step * 1e-6) / 1e9
    med = lambda k: statistics.median(r[k] for r in rows) * 1e3

    out = {
        'metric': METRIC, 'value': round(med_step, 2), 'unit': 'us/decode-step', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(elapsed * 1e3 / args.steps, 3),
        'higher_is_better': False, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'fp16',
        'data': 'synthetic: seeded 30 s clip (3 tones + noise), seeded random-init N(0, 0.02) fp16 weights',
        'config': {'workload': f'whisper-large-v3-turbo batch 1: 30 s clip -> log-mel -> 32-layer encoder -> '
                               f'{args.tokens} greedy tokens (8-step decoder hipGraph)',
                   'clip_s': 30, 'tokens': args.tokens, 'batch': 1},
        'decode_step_us': round(med_step, 2), 'decode_step_bytes': int(step_bytes),
        'decode_step_bytes_fp16_head': int(ref_step_bytes),
        'decode_step_hbm_gbps': round(step_gbps, 1), 'decode_step_roofline_frac': round(step_gbps / HBM_PEAK_GBPS, 4),
        'e2e_ms': round(med('e2e_s'), 3), 'ttft_ms': round(med('ttft_s'), 3), 'mel_ms': round(med('mel_s'), 3),
        'encoder_ms': round(med('encoder_s'), 3), 'decode_ms': round(med('decode_s'), 3),
        'encoder_tflops': round(encoder_flops(model.dims) / (med('encoder_s') * 1e-3) / 1e12, 1),
        'encoder_mfma_frac': round(encoder_flops(model.dims) / (med('encoder_s') * 1e-3) / 1e12
                                   / MFMA_FP16_PEAK_TFLOPS, 4),
        'n_tokens': rows[-1]['n_tokens'],
        'roofline': {'kernel': LM_KERNEL[q8], 'bound': 'hbm', 'achieved': round(lm_gbps, 1),
                     'peak': HBM_PEAK_GBPS, 'unit': 'GB/s', 'frac': round(lm_gbps / HBM_PEAK_GBPS, 4),
                     'traffic': measured_traffic(LM_TRAFFIC[q8]), 'traffic_source': LM_TRAFFIC[q8],
                     'us_per_launch': round(lm_us, 2), 'bytes_per_launch': lm_bytes,
                     'fp16_head_us_per_launch': round(lm16_us, 2)},
    }
    if serve is not None:
        out['serving'] = serve
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline(model, args.cpu_seconds, args.tokens)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()

"""Phase timeline of the persistent decoder step (``decoder_step_kernel``), from the profiling build.

    FW_LIBRARY=flash_whisper_amd/libflash_whisper_timeline.so python -m flash_whisper_amd.step_timeline

The profiling build (``libflash_whisper_timeline.so``, linked by ``python -m flash_whisper_amd.build``)
is the product library with the decoder step compiled with FW_STEP_TIMELINE=1: thread 0 of every block
stores the 100 MHz wall clock at fixed points of each step (fw_decoder_step_timeline in
include/flash_whisper.h lists them); nothing else changes. This module builds the seeded model,
transcribes the benchmark clip once (warm-up), runs the log-mel, encoder and prompt pass of a second
transcribe, then records the decode launch that follows (every token after the first, one launch, as
``transcribe`` runs it) and prints, per layer and phase, the median over the decode's steps of:

- ``in``: when the phase's input was in its blocks (first / median / last block, after the wait and
  the phase's prologue: residual catch-up and LayerNorm, or the attention vector's words);
- ``out``: when the last of its blocks had stored its output (for the cross attention, the heads'
  combined outputs);
- ``dur``: ``out`` less the previous phase's ``out``: the phase's share of the step;
- ``wait``: the median block's ``in`` less the previous phase's ``out``: hand-off and prologue;

all in us from the step's start (the first block to read the previous step's token). With
``--from-pos P --steps N`` it also records N steps from position P of a cache filled by the warm-up
(self attention over up to 448 keys), and prints the self-attention phase at every step.
"""

import argparse
import os
import statistics
import sys

import numpy as np

TICK_US = 0.01  # the 100 MHz wall clock
PHASES = ('LN1 + q/k/v', 'self attention', 'out', 'LN2 + cross q', 'cross attention', 'cross-out',
          'LN3 + fc1 + GELU', 'fc2')
TL_LAYERS, TL_LM, TL_SA = 4, 129, 141
TL_CLK = TL_SA + 8  # shader clock at the step's start and end, wall clock at its end
TL_WAVE = TL_CLK + 3  # layer 0's self attention: each wave's partials done
LM_POINTS = ('arrived', 'final LN done', 'y digits ready', 'first HBM batches scored', 'resident rows scored',
             'all rows scored', 'candidates listed', 'block maximum stored', 'every block maximum gathered',
             'token and state stored (last block)', 'residual caught up (thread 0; before the final LN)',
             'first HBM batch of wave 0 in registers (after the y digits)')


def tl_phase(layer, phase):
    return 1 + (layer * 8 + phase - 1) * 4


def record(model, n_steps, setup):
    """Runs setup() (enqueues whatever precedes the recorded launch), then records the timeline of the
    next n_steps decoder steps (one launch); returns int64 [steps, grid, slots] ticks (0: not reached)."""
    import torch

    lib = model.ext.lib
    slots = lib.fw_decoder_step_timeline_slots()
    if slots <= 0:
        raise RuntimeError('this library records no timeline: set FW_LIBRARY to libflash_whisper_timeline.so')
    grid = min(torch.cuda.get_device_properties(0).multi_processor_count, 1024)
    buf = torch.zeros(n_steps, grid, slots, dtype=torch.int64, device='cuda')
    setup()
    torch.cuda.synchronize()
    model.ext._call('fw_decoder_step_timeline', buf.data_ptr(), buf.numel() * 8, n_steps)
    model._steps(n_steps)
    torch.cuda.synchronize()
    model.ext._call('fw_decoder_step_timeline', None, 0, 0)
    model._check_step_error()
    return buf.cpu().numpy()


def step_stats(tl, n_layers):
    """Per step: the statistics above in us from the step's start."""
    out = []
    for st in range(tl.shape[0]):
        s = tl[st]
        if not (s[:, 0] > 0).any():
            break  # the launch stopped early
        t0 = s[s[:, 0] > 0, 0].min()
        us = lambda v: (float(v) - float(t0)) * TICK_US
        row, prev_out = {}, 0.0
        for layer in range(min(n_layers, TL_LAYERS)):
            for p in range(1, 9):
                base = tl_phase(layer, p)
                act = s[:, base + 2] > 0
                ins = np.sort(s[act, base + 1])
                outs = s[act, base + 3 if p == 5 else base + 2]
                outs = outs[outs > 0]
                if p == 5 and not len(outs):  # one query: the heads are combined by the cross-out blocks
                    outs = s[act, base + 2]
                if not len(ins) or not len(outs):
                    continue
                per = (s[act, base + 2] - s[act, base + 1]) * TICK_US  # each block's input -> its stores
                r = dict(blocks=int(act.sum()), in_first=us(ins[0]), in_med=us(np.median(ins)), in_last=us(ins[-1]),
                         out=us(outs.max()), enter=us(np.median(s[act, base])), enter_last=us(s[act, base].max()),
                         work=float(np.median(per)), work_max=float(per.max()))
                if p == 5:
                    r['part'] = us(s[act, base + 2].max())  # the split partials stored
                if p in (1, 4, 7):  # thread 0's residual contributions added, before the LayerNorm
                    r['resid'] = us(np.median(s[act, base + 3]))
                r['dur'], r['wait'] = r['out'] - prev_out, r['in_med'] - prev_out
                prev_out = r['out']
                row[(layer, p)] = r
        lm = s[:, TL_LM:TL_LM + len(LM_POINTS)]
        for k, name in enumerate(LM_POINTS):
            v = lm[:, k][lm[:, k] > 0]
            if len(v):
                row[('lm', k)] = dict(med=us(np.median(v)), last=us(v.max()), blocks=len(v))
        base = tl_phase(0, 2)
        act = s[:, base + 2] > 0
        if act.any():  # layer 0's self attention inside: each block's times after its input was in
            t_in = s[act, base + 1].astype(np.float64)
            for k, name in enumerate(('fresh row written', 'wave 0 partials (every round)', 'splits merged')):
                row[('sa', k)] = float(np.median(s[act, TL_SA + k] - t_in)) * TICK_US
            if (s[act, TL_SA + 3] > 0).all():
                row[('sa', 5)] = float(np.median(s[act, TL_SA + 3] - t_in)) * TICK_US
            row[('sa', 3)] = float(np.median(s[act, base + 3] - t_in)) * TICK_US
            for w in range(8):
                v = s[act, TL_WAVE + w]
                if (v > 0).all():
                    row[('wave', w)] = float(np.median(v - t_in)) * TICK_US
            row[('sa', 4)] = float(np.median(s[act, base + 2] - t_in)) * TICK_US
        ok = (s[:, TL_CLK] > 0) & (s[:, TL_CLK + 2] > s[:, 0]) & (s[:, 0] > 0)
        if ok.any():  # shader clock ticks over wall-clock ticks (100 MHz), per block: the core clock in MHz
            mhz = (s[ok, TL_CLK + 1] - s[ok, TL_CLK]) / ((s[ok, TL_CLK + 2] - s[ok, 0]) * TICK_US)
            row['clock_mhz'] = float(np.median(mhz))
        nxt = tl[st + 1][:, 0] if st + 1 < tl.shape[0] else None
        if nxt is not None and (nxt > 0).any():
            row['period'] = (float(nxt[nxt > 0].min()) - float(t0)) * TICK_US
        out.append(row)
    return out


def median_over(rows, key, field):
    vals = [r[key][field] for r in rows if key in r]
    return statistics.median(vals) if vals else float('nan')


def report(rows, n_layers, title):
    lines = [f'### {title}', '',
             f'Steps: {len(rows)} (medians over them); step period (start to the next step\'s start): '
             f'{statistics.median(r["period"] for r in rows if "period" in r):.2f} us; shader clock (s_memtime '
             f'ticks over wall-clock time, median block): '
             f'{statistics.median(r["clock_mhz"] for r in rows if "clock_mhz" in r):.0f} MHz', '',
             '| Layer | Phase | Blocks | entered (median / last) | in first | in median | in last | out | dur | wait | '
             'block work (median / max) |',
             '|---:|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|']
    for layer in range(min(n_layers, TL_LAYERS)):
        for p in range(1, 9):
            key = (layer, p)
            if not any(key in r for r in rows):
                continue
            m = lambda f: median_over(rows, key, f)
            name = PHASES[p - 1] + (f' (partials stored {m("part"):.2f})' if p == 5 else '') + \
                (f' (residual in {m("resid"):.2f})' if p in (1, 4, 7) else '')
            lines.append(f'| {layer} | {name} | {int(m("blocks"))} | {m("enter"):.2f} / {m("enter_last"):.2f} | '
                         f'{m("in_first"):.2f} | {m("in_med"):.2f} | {m("in_last"):.2f} | {m("out"):.2f} | '
                         f'{m("dur"):.2f} | {m("wait"):.2f} | {m("work"):.2f} / {m("work_max"):.2f} |')
    lines += ['', '| Layer 0 self attention, after its input (median block) | us |', '|---|---:|']
    for k, name in enumerate(('fresh row written', 'wave 0 partials (every round)', 'splits merged',
                              'combined (or merged, more than 2 splits)', 'output stored',
                              'past the barrier after the partials')):
        if any(('sa', k) in r for r in rows):
            lines.append(f'| {name} | {statistics.median(r[("sa", k)] for r in rows if ("sa", k) in r):.2f} |')
    waves = [w for w in range(8) if any(('wave', w) in r for r in rows)]
    if waves:
        lines += ['', '| Layer 0 self attention: wave w\'s partials done, after the input (median block) | ' +
                  ' | '.join(f'w{w}' for w in waves) + ' |', '|---|' + '---:|' * len(waves),
                  '| us | ' + ' | '.join(f'{statistics.median(r[("wave", w)] for r in rows if ("wave", w) in r):.2f}'
                                         for w in waves) + ' |']
    lines += ['', '| LM head point | median block | last block |', '|---|---:|---:|']
    for k, name in enumerate(LM_POINTS):
        key = ('lm', k)
        if any(key in r for r in rows):
            lines.append(f'| {name} | {median_over(rows, key, "med"):.2f} | {median_over(rows, key, "last"):.2f} |')
    return '\n'.join(lines)


def summary(rows, rows2, n_layers, pos0, from_pos):
    """Machine-readable medians: per phase over the decode's steps and layers (``dur``: its share of the
    step, ``work``: the median block's input-to-stores time), layer-by-layer self attention at cache
    lengths L in {64, 224, 448} (the 5 steps ending at L, all layers), the LM head (from the last fc2's
    output to the token stored) and the step period."""
    layers = range(min(n_layers, TL_LAYERS))
    med = lambda v: round(statistics.median(v), 3) if v else None
    phases = {}
    for p in range(1, 9):
        hits = [r[(l, p)] for r in rows for l in layers if (l, p) in r]
        phases[PHASES[p - 1]] = {'dur_us': med([h['dur'] for h in hits]), 'work_us': med([h['work'] for h in hits])}
    steps = [(pos0 + i + 1, r) for i, r in enumerate(rows)] + [(from_pos + i + 1, r) for i, r in enumerate(rows2)]
    by_len = {}
    for length in (64, 224, 448):
        hits = [r[(l, 2)] for L, r in steps if length - 4 <= L <= length for l in layers if (l, 2) in r]
        by_len[f'L{length}'] = {'dur_us': med([h['dur'] for h in hits]), 'work_us': med([h['work'] for h in hits]),
                                'samples': len(hits)}
    last = (len(layers) - 1, 8)
    stored = LM_POINTS.index('token and state stored (last block)')
    lm = [r[('lm', stored)]['last'] - r[last]['out'] for r in rows if ('lm', stored) in r and last in r]
    return {'phases': phases, 'self_attention_by_length': by_len, 'lm_head_us': med(lm),
            'step_period_us': med([r['period'] for r in rows if 'period' in r]), 'steps': len(rows),
            'shader_clock_mhz': med([r['clock_mhz'] for r in rows if 'clock_mhz' in r])}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--tokens', type=int, default=224)
    ap.add_argument('--from-pos', type=int, default=440, help='start of the extra run (self attention over long caches)')
    ap.add_argument('--steps', type=int, default=8, help='steps of the extra run (0: none)')
    ap.add_argument('--json', help='also write the medians of summary() to this file')
    args = ap.parse_args()
    if not os.environ.get('FW_LIBRARY'):
        print('set FW_LIBRARY=flash_whisper_amd/libflash_whisper_timeline.so (the profiling build)', file=sys.stderr)
        sys.exit(2)

    import torch

    from flash_whisper_amd.audio import synthetic_clip
    from flash_whisper_amd.model import CustomModel

    torch.set_grad_enabled(False)
    model = CustomModel(seed=0, selftest=False)
    clip = synthetic_clip(0)
    model.transcribe(clip, max_new_tokens=args.tokens, stop_at_eos=False)  # warm-up
    n_layers = model.dims.dec_layers
    n = args.tokens - 1
    model.ext.set_eos(model.step_head, ())
    tl = record(model, n, lambda: model.transcribe(clip, max_new_tokens=1, stop_at_eos=False))
    rows = step_stats(tl, n_layers)
    print(f'# device: {torch.cuda.get_device_name(0)}, grid {tl.shape[1]} blocks, '
          f'{model.ext.lib.fw_decoder_step_resident_rows()} resident LM-head rows per block')
    print()
    print(report(rows[1:], n_layers, f'Decode launch of a {args.tokens}-token transcribe: steps 1..{len(rows) - 1} '
                                     f'(positions 5..{4 + len(rows) - 1}; step 0 also loads the resident rows)'))
    print()
    pos0 = 4  # the decode starts after the 4-token prompt
    sa = [(pos0 + i + 1, r[(0, 2)]['dur'], r[(0, 2)]['in_med'] - r[(0, 1)]['out']) for i, r in enumerate(rows)
          if (0, 2) in r and (0, 1) in r]
    pick = [x for x in sa if x[0] in (64, 128, 224)]
    rows2 = []
    if args.steps > 0:
        def setup():
            with torch.inference_mode():
                model.state.copy_(torch.tensor([args.from_pos, 0], device='cuda'))
                model.cur.fill_(int(model.tokens[0]))
        tl2 = record(model, args.steps, setup)
        rows2 = step_stats(tl2, n_layers)
        print(report(rows2, n_layers, f'{args.steps} steps from position {args.from_pos} (cache rows from the '
                                      f'warm-up transcribe and earlier steps)'))
        print()
        pick += [(args.from_pos + i + 1, r[(0, 2)]['dur'], r[(0, 2)]['in_med'] - r[(0, 1)]['out'])
                 for i, r in enumerate(rows2) if (0, 2) in r and (0, 1) in r]
    print('### Self attention (layer 0) by cache length L = position + 1', '')
    print('| L | dur (us) | wait (us) |', '|---:|---:|---:|', sep='\n')
    for L, dur, wait in pick:
        print(f'| {L} | {dur:.2f} | {wait:.2f} |')
    if args.json:
        import json

        out = summary(rows[1:], rows2, n_layers, pos0 + 1, args.from_pos)
        out.update(device=torch.cuda.get_device_name(0), grid=int(tl.shape[1]),
                   resident_rows=int(model.ext.lib.fw_decoder_step_resident_rows()), tokens=args.tokens)
        with open(args.json, 'w') as f:
            json.dump(out, f)


if __name__ == '__main__':
    main()

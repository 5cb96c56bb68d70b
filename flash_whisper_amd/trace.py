"""roctx ranges around the path's passes, and a per-range summary of a kernel trace that recorded them.

The reference wraps each profiled pass in an NVTX range and captures by range (runner.py:166-184,
bench.py:185-197). Here ``transcribe`` runs inside a ``transcribe`` range (the model's selftest
inside ``selftest``), and bench.py names each timed pass (``bench:30s:rep3``, ``bench:5s:rep0``, ...).
The ranges go through ROCm's roctx (librocprofiler-sdk-roctx): while no tool traces markers a push
and a pop cost a library call each; under

    rocprofv3 --marker-trace --kernel-trace --output-format csv -d OUT -o run -- python3 bench.py

they are recorded, and

    python -m flash_whisper_amd.trace OUT

lists, per range name (``rep<i>`` suffixes grouped), the passes, the kernels whose GPU interval lies
inside each pass, and their GPU time (median over the passes). A ``transcribe`` range is pushed after
the host has synchronised the device and popped after its last token is on the host, so the kernels
inside it are that transcribe's.
"""

import contextlib
import csv
import os
import re
import statistics
import sys

_ROCTX = None


def _roctx():
    """The roctx library (ctypes), or None where it is not installed (the ranges are then no-ops)."""
    global _ROCTX
    if _ROCTX is None:
        import ctypes

        _ROCTX = False
        root = os.environ.get('ROCM_PATH', '/opt/rocm')
        for name in (os.path.join(root, 'lib', 'librocprofiler-sdk-roctx.so.1'), 'librocprofiler-sdk-roctx.so.1'):
            try:
                lib = ctypes.CDLL(name)
            except OSError:
                continue
            lib.roctxRangePushA.argtypes, lib.roctxRangePushA.restype = [ctypes.c_char_p], ctypes.c_int
            lib.roctxRangePop.argtypes, lib.roctxRangePop.restype = [], ctypes.c_int
            _ROCTX = lib
            break
    return _ROCTX or None


@contextlib.contextmanager
def trace_range(name):
    """A roctx range named `name` around the block (on this host thread)."""
    lib = _roctx()
    if lib is not None:
        lib.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        if lib is not None:
            lib.roctxRangePop()


def _rows(path):
    with open(path, newline='') as f:
        return list(csv.DictReader(f))


def _find(root, suffix):
    hits = []
    for d, _, files in os.walk(root):
        hits += [os.path.join(d, f) for f in files if f.endswith(suffix)]
    if not hits:
        raise FileNotFoundError(f'no *{suffix} under {root}')
    return sorted(hits)


def _col(row, *names):
    for n in names:
        if n in row:
            return row[n]
    raise KeyError(f'none of {names} in the trace columns {sorted(row)}')


def load(root):
    """(ranges, kernels) from a rocprofv3 CSV output directory: ranges as (name, start_ns, end_ns),
    kernels as (name, start_ns, end_ns)."""
    ranges = []
    for path in _find(root, 'marker_api_trace.csv'):
        for r in _rows(path):
            name = _col(r, 'Function', 'Operation', 'Name')
            if name in ('roctxRangePushA', 'roctxRangePop', 'roctxMarkA'):
                continue  # the API calls themselves; the ranges carry their message as the name
            ranges.append((name, int(_col(r, 'Start_Timestamp')), int(_col(r, 'End_Timestamp'))))
    kernels = []
    for path in _find(root, 'kernel_trace.csv'):
        for r in _rows(path):
            kernels.append((_col(r, 'Kernel_Name'), int(_col(r, 'Start_Timestamp')), int(_col(r, 'End_Timestamp'))))
    kernels.sort(key=lambda k: k[1])
    return ranges, kernels


def kernel_name(name):
    """name<template args> of a traced kernel name, without namespaces and parameters."""
    from .build import _plain_name

    if name.startswith('_Z'):
        return _plain_name(name)
    name = name.removeprefix('void ').replace('fw::(anonymous namespace)::', '')
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):  # the parameter list starts at the first '(' outside template brackets
        depth += ch == '<'
        depth -= ch == '>'
        if ch == '(' and depth == 0:
            cut = i
            break
    return name[:cut]


def summarize(ranges, kernels):
    """Markdown: per range group, the passes, kernels per pass and their GPU time (median over passes),
    then the kernels of the ``transcribe`` passes by name."""
    import bisect

    starts = [k[1] for k in kernels]
    groups = {}
    for name, t0, t1 in ranges:
        outer = [r for r in ranges if r[1] <= t0 and t1 <= r[2] and r != (name, t0, t1)]
        if outer:  # a nested range is named with its innermost enclosing one: bench:30s:rep* > transcribe
            name = re.sub(r'rep\d+$', 'rep*', min(outer, key=lambda r: r[2] - r[1])[0]) + ' > ' + name
        i = bisect.bisect_left(starts, t0)
        inside = []
        while i < len(kernels) and kernels[i][1] < t1:
            if kernels[i][2] <= t1:
                inside.append(kernels[i])
            i += 1
        groups.setdefault(re.sub(r'rep\d+$', 'rep*', name), []).append((t1 - t0, inside))
    lines = ['| Range | Passes | Wall (median, ms) | Kernels per pass (median) | GPU kernel time (median, ms) |',
             '|---|---:|---:|---:|---:|']
    for g in sorted(groups):
        passes = groups[g]
        lines.append(f'| {g} | {len(passes)} | {statistics.median(p[0] for p in passes) / 1e6:.3f} | '
                     f'{statistics.median(len(p[1]) for p in passes):.0f} | '
                     f'{statistics.median(sum(k[2] - k[1] for k in p[1]) for p in passes) / 1e6:.3f} |')
    for g in sorted(groups):
        if not g.endswith('transcribe'):
            continue
        per = {}
        for _, inside in groups[g]:
            seen = {}
            for k in inside:
                seen.setdefault(k[0], []).append(k[2] - k[1])
            for n, v in seen.items():
                per.setdefault(n, []).append((len(v), sum(v)))
        lines += ['', f'Kernels of the `{g}` passes ({len(groups[g])}), by GPU time per pass:', '',
                  '| Kernel | Launches per pass | GPU time per pass (median, us) |', '|---|---:|---:|']
        for n, v in sorted(per.items(), key=lambda kv: -statistics.median(x[1] for x in kv[1])):
            short = kernel_name(n)
            lines.append(f'| `{short}` | {statistics.median(x[0] for x in v):.0f} | '
                         f'{statistics.median(x[1] for x in v) / 1e3:.1f} |')
    return '\n'.join(lines)


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 1:
        print('usage: python -m flash_whisper_amd.trace ROCPROFV3_OUTPUT_DIR', file=sys.stderr)
        return 2
    ranges, kernels = load(argv[0])
    print(f'{len(ranges)} ranges, {len(kernels)} kernels')
    print()
    print(summarize(ranges, kernels))
    return 0


if __name__ == '__main__':
    sys.exit(main())

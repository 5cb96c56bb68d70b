"""Builds the HIP kernels into the in-tree C-ABI library ``flash_whisper_amd/libflash_whisper.so``.

``python -m flash_whisper_amd.build`` compiles every ``csrc/*.hip`` for gfx950 with hipcc (in
parallel, one object per source) and links them. The library exports the entry points declared in
``include/flash_whisper.h``. It also links the profiling build ``libflash_whisper_timeline.so``: the
same objects with the decoder step compiled with FW_STEP_TIMELINE=1, which records the phase timeline
that ``python -m flash_whisper_amd.step_timeline`` reads (selected with FW_LIBRARY; never the default). This replaces the reference's JIT extension build (custom/ext.py:13-18),
which ran nvcc through torch.utils.cpp_extension; here the build is ahead-of-time and in-tree so the
built library travels with the source tree.
"""

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
BUILD_DIR = Path(os.environ.get('FW_BUILD_DIR', PKG / '_build'))
LIB = PKG / 'libflash_whisper.so'
TIMELINE_LIB = PKG / 'libflash_whisper_timeline.so'
TIMELINE_SRC = 'decode_step.hip'  # the one source the profiling build compiles differently
ARCH = os.environ.get('FW_OFFLOAD_ARCH', 'gfx950')
HIPCC = os.environ.get('HIPCC', shutil.which('hipcc') or '/opt/rocm/bin/hipcc')

COMMON_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-Wall', '-Wno-unused-function',
    # packed fp32 (v_pk_*_f32) codegen stays off on this target
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Xarch_host', '-mfma',
]
# The synthetic-weight generator must round identically on host and device: no FMA contraction.
PER_FILE_FLAGS = {
    'synth.hip': ['-ffp-contract=off'],
    # MFMA results in VGPRs: the attention softmax reads every score and rescales O in place
    'attention_enc.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form'],
}


def sources():
    return sorted(CSRC.glob('*.hip'))


def _compile(src, verbose, defines=(), suffix=''):
    obj = BUILD_DIR / (src.stem + suffix + '.o')
    cmd = [HIPCC, *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), *defines, '-c', str(src), '-o', str(obj)]
    if verbose:
        print(' '.join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and says so; that is harmless.
    noise = ('packed-fp32-ops', 'not a recognized feature', 'ignoring feature')
    msg = '\n'.join(line for line in (proc.stdout + proc.stderr).splitlines()
                    if not any(n in line for n in noise))
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{msg}')
    if verbose and msg.strip():
        print(msg, flush=True)
    return obj


def _link(objs, lib, verbose):
    tmp = lib.with_suffix('.so.tmp')
    cmd = [HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', str(tmp), *map(str, objs), '-lpthread']
    if verbose:
        print(' '.join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'link failed:\n{proc.stdout}{proc.stderr}')
    os.replace(tmp, lib)  # atomic: a process that already mapped the old file keeps it


def build(verbose=False, jobs=None):
    """Compiles all sources and links the shared library and its phase-timeline profiling build. Always
    rebuilds. Returns the product library's path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    tl_src = next(s for s in srcs if s.name == TIMELINE_SRC)
    jobs = jobs or min(len(srcs) + 1, max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as pool:
        tl_obj = pool.submit(_compile, tl_src, verbose, ('-DFW_STEP_TIMELINE=1',), '_timeline')
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
        tl_obj = tl_obj.result()
    _link(objs, LIB, verbose)
    _link([tl_obj if o.stem == tl_src.stem else o for o in objs], TIMELINE_LIB, verbose)
    return LIB


RESOURCE_FIELDS = (('VGPRs', 'VGPRs'), ('AGPRs', 'AGPRs'), ('TotalSGPRs', 'SGPRs'),
                   ('ScratchSize [bytes/lane]', 'scratch B/lane'), ('Occupancy [waves/SIMD]', 'waves/SIMD'),
                   ('LDS Size [bytes/block]', 'static LDS B/block'), ('VGPRs Spill', 'VGPR spill'),
                   ('SGPRs Spill', 'SGPR spill'))


def _plain_name(sym):
    """name<int args> of an Itanium-mangled nested name that c++filt left as it was (it does not know
    the _Float16 parameter code DF16_)."""
    import re

    if not sym.startswith('_ZN'):
        return sym
    i, parts = 3, []
    while i < len(sym) and sym[i].isdigit():
        j = i
        while sym[j].isdigit():
            j += 1
        n = int(sym[i:j])
        parts.append(sym[j:j + n])
        i = j + n
    if not parts:
        return sym
    name = parts[-1]
    if sym[i:i + 1] == 'I':
        args = re.findall(r'L([ib])(\d+)E', sym[i:sym.find('EE', i) + 2])
        name += '<' + ', '.join(('true' if v == '1' else 'false') if k == 'b' else v for k, v in args) + '>'
    return name


def _demangle(names):
    tool = shutil.which('c++filt')
    if not tool or not names:
        return names
    out = subprocess.run([tool], input='\n'.join(names), capture_output=True, text=True).stdout.splitlines()
    return out if len(out) == len(names) else names


def resource_usage(variants=(('', ()), (' (profiling build)', ('-DFW_STEP_TIMELINE=1',)))):
    """Per-kernel VGPR/AGPR/SGPR/scratch/occupancy/LDS/spill report from the compiler
    (-Rpass-analysis=kernel-resource-usage) for every source as the library builds it, as markdown.
    The decoder step's dynamic LDS (the resident LM-head rows) is sized at launch and not counted."""
    rows = []
    for src in sources():
        for tag, extra in variants:
            if extra and src.stem != 'decode_step':
                continue
            cmd = [HIPCC, *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), *extra, '--cuda-device-only',
                   '-Rpass-analysis=kernel-resource-usage', '-c', str(src), '-o', os.devnull]
            proc = subprocess.run(cmd, capture_output=True, text=True)
            cur = None
            for line in proc.stderr.splitlines():
                if 'remark:' not in line:
                    continue
                body = line.split('remark:', 1)[1].split('[-Rpass', 1)[0].strip()
                key, _, val = body.partition(':')
                if key == 'Function Name':
                    cur = {'file': src.name + tag, 'name': val.strip()}
                    rows.append(cur)
                elif cur is not None:
                    cur[key.strip()] = val.strip()
    names = _demangle([r['name'] for r in rows])
    out = ['| Source | Kernel | ' + ' | '.join(h for _, h in RESOURCE_FIELDS) + ' |',
           '|---|---|' + '---:|' * len(RESOURCE_FIELDS)]
    for r, name in zip(rows, names):
        short = _plain_name(name) if name.startswith('_Z') else \
            name.replace('fw::(anonymous namespace)::', '').split('(')[0].removeprefix('void ')
        out.append(f'| {r["file"]} | `{short}` | ' + ' | '.join(r.get(k, '') for k, _ in RESOURCE_FIELDS) + ' |')
    return out


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument('-v', '--verbose', action='store_true')
    parser.add_argument('--resource-usage', action='store_true', help='print per-kernel register/LDS usage')
    args = parser.parse_args()
    lib = build(verbose=args.verbose)
    print(f'built: {lib}')
    if args.resource_usage:
        print('\n'.join(resource_usage()))


if __name__ == '__main__':
    sys.exit(main())

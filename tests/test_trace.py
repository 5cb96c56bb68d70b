"""flash_whisper_amd.trace on the CPU: a roctx range is harmless without a profiler, and the summary
attributes each kernel to the range that holds its whole GPU interval, grouping rep<i> names."""

import csv

from flash_whisper_amd import trace


def test_trace_range_without_a_profiler():
    with trace.trace_range('test:outer'):
        with trace.trace_range('test:inner'):
            pass


def _write(path, header, rows):
    with open(path, 'w', newline='') as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summary_attributes_kernels_to_ranges(tmp_path):
    d = tmp_path / 'run' / 'host'
    d.mkdir(parents=True)
    _write(d / 'run_marker_api_trace.csv', ['Domain', 'Function', 'Start_Timestamp', 'End_Timestamp'],
           [['MARKER_CORE_API', 'bench:30s:rep0', 1000, 2000], ['MARKER_CORE_API', 'bench:30s:rep1', 3000, 4200],
            ['MARKER_CORE_API', 'transcribe', 1010, 1990], ['MARKER_CORE_API', 'transcribe', 3010, 4190],
            ['MARKER_CORE_API', 'roctxRangePop', 1990, 1991]])
    _write(d / 'run_kernel_trace.csv', ['Kernel_Name', 'Start_Timestamp', 'End_Timestamp'],
           [['enc', 1100, 1400], ['step', 1500, 1900], ['enc', 3100, 3300], ['step', 3400, 4000],
            ['late', 4150, 4300], ['outside', 2100, 2200]])
    ranges, kernels = trace.load(str(tmp_path))
    assert len(ranges) == 4 and len(kernels) == 6
    text = trace.summarize(ranges, kernels)
    # both reps hold 2 kernels ('late' ends after rep1's end); GPU time per pass 700 and 800 ns
    assert '| bench:30s:rep* | 2 | 0.001 | 2 | 0.001 |' in text
    assert '| bench:30s:rep* > transcribe | 2 |' in text  # named with its enclosing range
    assert '| `step` | 1 | 0.5 |' in text  # (400 + 600) / 2 ns = 0.5 us
    assert 'outside' not in text

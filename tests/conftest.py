"""Shared pytest setup: the `gpu` marker and small helpers used across the suites."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / 'tests' / 'golden'


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (HIP device) and the built library')


@pytest.fixture(scope='session')
def built_lib():
    """The in-tree C-ABI library; builds it when it is missing (CPU-only build is fine)."""
    from flash_whisper_amd import _lib, build

    if not _lib.LIB_PATH.exists():
        build.build()
    return _lib.lib()


@pytest.fixture(scope='session')
def hip_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip('no HIP device')
    from flash_whisper_amd import _lib

    if not _lib.LIB_PATH.exists():
        raise RuntimeError('libflash_whisper.so is not built; run `python -m flash_whisper_amd.build` first')
    return torch.device('cuda', 0)

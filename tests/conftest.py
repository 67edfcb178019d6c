"""pytest configuration: the `gpu` marker and shared fixtures.

`-m "not gpu"` runs the oracle pins, host logic and library-load checks on the
CPU; `-m gpu` runs the parity tests against the HIP library on an MI355X.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from cachalot_amd import _lib

    _lib.lib()  # fail loudly if the library is missing
    return torch.device("cuda:0")


@pytest.fixture(params=["two_kernel_mx", "two_kernel_bf16"])
def q2_path(request, monkeypatch):
    """The 2-bit decode runs as two kernels on the block-scaled fp8 x fp4 matrix
    cores by default; the bf16-MFMA kernel pair (the path for shapes outside the
    matrix-core kernels' envelope) is selected with CACHALOT_DECODE_BF16=1.  Both
    are pinned."""
    monkeypatch.setenv("CACHALOT_DECODE_BF16", "1" if request.param == "two_kernel_bf16" else "0")
    return request.param


@pytest.fixture(params=["mx", "bf16"])
def prefill_path(request, monkeypatch):
    """FP4 and 2-bit g128 prefill run on the block-scaled fp8 x fp4 matrix cores by
    default; the bf16-MFMA kernels are selected with CACHALOT_PREFILL_BF16=1.  Both are
    pinned."""
    monkeypatch.setenv("CACHALOT_PREFILL_BF16", "1" if request.param == "bf16" else "0")
    return request.param

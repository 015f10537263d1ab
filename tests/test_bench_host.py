"""CPU-side tests of bench.py's set-up code (no GPU needed): a weight
scratch too small for a projection's N x K fp32 weights is refused on the
host, before any device call writes into it."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


class FakeBuf:
    """Stands in for a capi.DevBuf; any device call on it would fail."""

    def __init__(self, nbytes):
        self.ptr = 0x1000
        self.nbytes = nbytes


class NoDevice:
    def __getattr__(self, name):
        raise AssertionError(f"device call {name} reached with an undersized scratch")


def test_scratch_too_small_raises_before_any_device_call(monkeypatch):
    monkeypatch.setattr(bench, "capi", NoDevice())
    # the shape whose fill once overran a smaller scratch: 17920 x 1536 fp32
    with pytest.raises(ValueError):
        bench.rotation(FakeBuf(8960 * 1536 * 4), 1, 17920, 1536, False, False, 1)
    with pytest.raises(ValueError):
        bench.Linear(None, FakeBuf(896 * 896 * 4 - 4), 1, 896, 896, False, False, 1)
    with pytest.raises(TypeError):
        bench.Linear(None, 0x1000, 1, 896, 896, False, False, 1)  # a bare pointer carries no size


def test_scratch_of_exact_size_passes_the_check():
    bench.check_scratch(FakeBuf(896 * 896 * 4), 896, 896)

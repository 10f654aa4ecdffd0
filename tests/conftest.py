"""Shared test setup: the `gpu` marker, import paths for the product binding and the oracle, and
helpers to read the reference's golden-vector format."""
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gpt-sovits-native_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_terminal_summary(terminalreporter):
    """Session total of 16-bit output elements that passed only through the one-storage-step
    clause of the parity bar (tests/gpu_util.py)."""
    try:
        from gpu_util import WIDENED
    except Exception:
        return
    if WIDENED["elements"]:
        terminalreporter.write_line(
            f"16-bit parity: {WIDENED['widened']} of {WIDENED['elements']} compared elements "
            f"passed only within one storage step (|d| > 2e-3)")


def load_bin(name):
    """Reference fixture format `[u32 rank][u32 dims x rank][raw little-endian data]`
    (tools/export_kern_golden.py:4-6, 26-36; reader tests/test_kern.cpp:30-57)."""
    path = os.path.join(GOLDEN, name)
    raw = open(path, "rb").read()
    (rank,) = struct.unpack_from("<I", raw, 0)
    dims = struct.unpack_from(f"<{rank}I", raw, 4)
    dt = np.float16 if name.endswith(".f16") else np.float32
    data = np.frombuffer(raw, dtype=dt, offset=4 + 4 * rank)
    assert data.size == int(np.prod(dims)), name
    return data.reshape(dims).copy()


def check_close(got, want, max_rel, min_cos):
    """The reference's gate (tests/test_kern.cpp:60-80): running peak |want| normalises each error
    (peak is updated before the element's error is formed) and cosine similarity in double."""
    g = np.asarray(got, dtype=np.float64).ravel()
    w = np.asarray(want, dtype=np.float64).ravel()
    assert g.size == w.size
    peak = np.maximum.accumulate(np.abs(w))
    with np.errstate(divide="ignore", invalid="ignore"):
        err = np.abs(g - w) / peak
    worst = float(np.nanmax(err)) if err.size else 0.0
    cos = float(np.dot(g, w) / np.sqrt(np.dot(g, g) * np.dot(w, w)))
    return worst <= max_rel and cos >= min_cos, worst, cos


@pytest.fixture(scope="session")
def gsvk_lib():
    import gsvk
    return gsvk.lib()


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    return oracle.lib()

"""The measurement library behind `bench.py --diag` (libgsvk_diag.so) on the CPU: it loads, exports
its two entry points, and rejects unknown forms and sizes its kernels do not take before any HIP
call (every call here fails validation, so no device is needed)."""
import ctypes
import os

import pytest

from conftest import ROOT

LIB = os.path.join(ROOT, "gpt-sovits-native_amd", "libgsvk_diag.so")


@pytest.fixture(scope="module")
def diag():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (make -C gpt-sovits-native_amd libgsvk_diag.so)")
    lib = ctypes.CDLL(LIB)
    lib.gsvk_diag_copy.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_size_t, ctypes.c_void_p]
    lib.gsvk_diag_stream_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_copy_rejects_before_launch(diag):
    a16, b16 = 1 << 20, 2 << 20  # 16-byte aligned stand-ins, never dereferenced
    assert diag.gsvk_diag_copy(4, a16, b16, 8, 1024, None) == -1
    assert diag.gsvk_diag_copy(-1, a16, b16, 8, 1024, None) == -1
    assert diag.gsvk_diag_copy(0, None, b16, 8, 1024, None) == -2
    assert diag.gsvk_diag_copy(0, a16 + 4, b16, 8, 1024, None) == -2   # misaligned
    assert diag.gsvk_diag_copy(0, a16, b16, 8, 1000, None) == -2       # not whole 16-byte chunks
    assert diag.gsvk_diag_copy(0, a16, b16, 0, 1024, None) == -2
    assert diag.gsvk_diag_copy(1, a16, b16, 8, 512 * 16 * 16 + 16, None) == -2  # row over 128 KiB
    assert diag.gsvk_diag_copy(2, a16, b16, 3, 1024, None) == -2       # not whole 32 KiB blocks


def test_stream_read_rejects_before_launch(diag):
    w, sink = 1 << 20, 2 << 20
    assert diag.gsvk_diag_stream_read(5, w, 64, sink, None) == -1
    assert diag.gsvk_diag_stream_read(0, w, 48, sink, None) == -2       # not whole 32-row batches
    assert diag.gsvk_diag_stream_read(0, w, 0, sink, None) == -2
    assert diag.gsvk_diag_stream_read(0, None, 64, sink, None) == -2
    assert diag.gsvk_diag_stream_read(0, w, 64, None, None) == -2
    assert diag.gsvk_diag_stream_read(0, w + 8, 64, sink, None) == -2   # misaligned

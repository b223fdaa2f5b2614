"""dllm_hip_sum_squares_noalloc (the allocation-free variant of dllm_hip_sum_squares, its scratch in a fixed device
array) against the workspace entry point, bit for bit, through the C ABI: two calls in a row, the second on a smaller
input, so the second call runs over the first call's leftover scratch contents. Also the size limit's error."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

MAX_VALUES = 1 << 29


@pytest.fixture(scope="module")
def lib():
    from etalii_dllm_amd.kernels import lib

    lib.dllm_hip_sum_squares_noalloc.argtypes = [C.c_void_p, C.c_size_t, C.POINTER(C.c_double), C.c_void_p]
    return lib


def with_workspace(lib, dev, n: int) -> float:
    from etalii_dllm_amd.kernels import Device, check

    ws = Device(lib.dllm_hip_sum_squares_workspace(n))
    out = C.c_double()
    check(lib.dllm_hip_sum_squares(dev.ptr, n, C.byref(out), ws.ptr, ws.nbytes, None))
    return out.value


def no_alloc(lib, dev, n: int) -> float:
    from etalii_dllm_amd.kernels import check

    out = C.c_double()
    check(lib.dllm_hip_sum_squares_noalloc(dev.ptr, n, C.byref(out), None))
    return out.value


def bits(x: float) -> bytes:
    return np.float64(x).tobytes()


def test_no_alloc_sum_squares_equals_the_workspace_entry_point(lib):
    from etalii_dllm_amd.kernels import Device

    big = O.gaussian(71, 40 * 8192 + 1234)
    big[5000] = np.float32(3e18)  # a binade jump in the middle
    small = O.gaussian(72, 3 * 8192 + 77, scale=1e-3)
    for values in (big, small, small[:1], np.zeros(0, np.float32)):
        dev = Device.of(values)
        want = with_workspace(lib, dev, values.size)
        got = no_alloc(lib, dev, values.size)
        assert bits(got) == bits(want), (values.size, got, want)
        if values.size:
            assert bits(got) == bits(O.oracle_kernels().sum_squares(values))


def test_no_alloc_sum_squares_at_its_size_limit(lib):
    """The largest input the fixed scratch serves (2^29 values) equals the workspace entry point; one more value is
    an invalid argument, refused before any launch."""
    from etalii_dllm_amd.kernels import Device, check

    values = np.full(MAX_VALUES, np.float32(0.5))
    values[::4097] = np.float32(1.25)
    dev = Device.of(values)
    assert bits(no_alloc(lib, dev, MAX_VALUES)) == bits(with_workspace(lib, dev, MAX_VALUES))
    assert bits(no_alloc(lib, dev, 1000)) == bits(with_workspace(lib, dev, 1000))
    out = C.c_double()
    with pytest.raises(ValueError, match="at most 2\\^29"):
        check(lib.dllm_hip_sum_squares_noalloc(dev.ptr, MAX_VALUES + 1, C.byref(out), None))

"""The float functions the decoder kernels use, pinned on the host.

rusticide's softmax and SiLU call f32::exp, which is libm's expf
(crates/rusticide-kernels/src/portable/{norm.rs:17-30,elementwise.rs:6-9}).
rh_expf_host runs the same source the device kernels run; it must give the
bits of libm's expf on every input (an exhaustive sweep of all 2^32 inputs
agrees; this test covers every 61st float and the special cases).

RMSNorm's f32::sqrt (crates/rusticide-kernels/src/portable/norm.rs:8-14) is
rounded to nearest; the device's native square root is only within one ulp,
so the kernels correct it from fma residuals. rh_sqrt_host runs that
correction from starts one ulp below, at and above the nearest float (an
exhaustive sweep of every positive float agrees; this test covers every 37th).
"""

import ctypes

import numpy as np
import pytest

import oracle as O
import rusticide_amd as R


def host_expf(x):
    L = R.lib()
    L.rh_expf_host.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    L.rh_expf_host(x.ctypes.data, y.ctypes.data, len(x))
    return y


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


SPECIAL = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 88.0, -88.0, 88.72283, 88.72284, 88.7229,
                    -103.97207, -103.97208, -103.9721, -87.33655, -87.3366, 1e-45, -1e-45, 1e-38, -1e-38,
                    np.float32(2 ** -24), 100.0, -200.0], np.float32)


def test_expf_special_values():
    assert same(host_expf(SPECIAL), O.expf(SPECIAL))


@pytest.mark.parametrize("part", range(4))
def test_expf_matches_libm_on_a_stride_of_all_floats(part):
    # every 61st bit pattern, in four quarters of the 32-bit range
    start, stop = part << 30, (part + 1) << 30
    for lo in range(start, stop, 61 << 22):
        bits = np.arange(lo, min(lo + (61 << 22), stop), 61, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        assert same(host_expf(x), O.expf(x)), f"first mismatch near bits {lo:#x}"


def test_expf_is_not_the_correctly_rounded_exp():
    # the two differ (libm's expf is not correctly rounded everywhere); the
    # kernels follow libm, which is what makes their softmax bits the CPU path's
    x = np.linspace(-30, 0, 2_000_001, dtype=np.float32)
    cr = np.exp(x.astype(np.float64)).astype(np.float32)
    assert not same(O.expf(x), cr)
    assert same(host_expf(x), O.expf(x))


def host_sqrt(x, start=None):
    L = R.lib()
    L.rh_sqrt_host.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    st = None if start is None else np.ascontiguousarray(start, np.float32)
    L.rh_sqrt_host(x.ctypes.data, None if st is None else st.ctypes.data, y.ctypes.data, len(x))
    return y


def test_sqrt_special_values():
    x = np.array([0.0, -0.0, np.inf, -1.0, -np.inf, np.nan, 1e-45, 2 ** -126, 2 ** -64, 2 ** -65, 1.0, 2.0, 4.0,
                  3.4028235e38, 1e-5, 1.0000001e-5], np.float32)
    assert same(host_sqrt(x), np.sqrt(x))


@pytest.mark.parametrize("part", range(2))
def test_sqrt_correction_from_one_ulp_either_side(part):
    # numpy's float32 sqrt is the IEEE one (rounded to nearest); starts one
    # ulp off must come back to it for every x >= 2^-64
    first = np.float32(2.0 ** -64).view(np.uint32)
    start, stop = (first, 0x5F800000) if part == 0 else (0x5F800000, 0x7F800000)
    for lo in range(int(start), stop, 37 << 22):
        bits = np.arange(lo, min(lo + (37 << 22), stop), 37, dtype=np.uint64).astype(np.uint32)
        x = bits.view(np.float32)
        want = np.sqrt(x)
        for d in (-1, 0, 1):
            s = (want.view(np.uint32) + np.uint32(d & 0xFFFFFFFF)).view(np.float32)
            assert same(host_sqrt(x, s), want), f"start {d:+d} ulp, near bits {lo:#x}"
        assert same(host_sqrt(x), want)


def test_sqrt_below_two_to_the_minus_64_scales_exactly():
    bits = np.arange(1, np.float32(2.0 ** -64).view(np.uint32), 101, dtype=np.uint32)
    x = bits.view(np.float32)
    assert same(host_sqrt(x), np.sqrt(x))

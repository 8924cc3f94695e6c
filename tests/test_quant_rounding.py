"""The element quantization of the HIP kernels, restated in float32 numpy,
against the reference's formula over every fp16 input.

cider/kernels/w8a8_quantize.metal:82-85 defines q = clamp(round(x * inv),
-128, 127) with Metal's round (half away from zero) and NaN -> -128; the
oracle computes that in float64 (``rha``, ``clamp_i8``).  The kernels
(cider_amd/csrc/quant_common.hpp) compute it differently:

    r = x * inv                       (binary32; an fma with +0 on the GPU)
    r = fmin(fmax(r, -128), 127)      (clamp first; NaN -> -128)
    q = trunc(r + copysign(0.5 - 2^-25, r))

This test checks that the two agree for all 65536 fp16 bit patterns of x
(NaN, inf, subnormals, exact .5 ties) at several hundred scales inv,
including 1.0 (s == 1) and 127 / amax for amax across the fp16 range.  A
plausible slip -- adding 0.5 instead of the largest float below it (wrong at
0.49999997), rounding before a half-even conversion, clamping after the
truncation -- fails here.
"""
import numpy as np

from oracle import cider_oracle as O

F32 = np.float32


def kernel_q(x16: np.ndarray, inv: np.float32) -> np.ndarray:
    r = (x16.astype(F32) * F32(inv)).astype(F32)
    r = np.fmin(np.fmax(r, F32(-128.0)), F32(127.0)).astype(F32)
    t = (r + np.copysign(F32(np.nextafter(F32(0.5), F32(0.0))), r)).astype(F32)
    return np.trunc(t).astype(np.int64)


def reference_q(x16: np.ndarray, inv: np.float32) -> np.ndarray:
    v = (x16.astype(F32) * F32(inv)).astype(F32)
    return O.clamp_i8(O.rha(v)).astype(np.int64)


def _inv_values():
    amax = np.arange(0x0001, 0x7C00, 97, dtype=np.uint16).view(np.float16).astype(F32)
    s = (amax / F32(127.0)).astype(F32)
    s = np.where(s == F32(0.0), F32(1.0), s).astype(F32)
    inv = (F32(1.0) / s).astype(F32)
    extra = np.array([1.0, 0.5, 2.0, 127.0, 1.0 / 127.0, 3.0e4, 1e-4], dtype=F32)
    # scales that put x * inv on the float just below a .5 (x = 1, 2, ...):
    # where adding 0.5 instead of 0.5 - 2^-25 would round up
    below = np.nextafter(np.array([0.5, 1.5, 2.5, 126.5, 0.25], dtype=F32), F32(0.0)).astype(F32)
    return np.concatenate([inv, extra, below])


def test_kernel_rounding_equals_reference_for_every_fp16_input():
    x16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    with np.errstate(invalid="ignore", over="ignore"):
        _check_all(x16)


def _check_all(x16):
    for inv in _inv_values():
        a = kernel_q(x16, inv)
        b = reference_q(x16, inv)
        bad = np.nonzero(a != b)[0]
        assert bad.size == 0, (float(inv), hex(int(x16.view(np.uint16)[bad[0]])),
                               int(a[bad[0]]), int(b[bad[0]]))


def test_half_offset_is_needed():
    """Adding exactly 0.5 rounds 0.49999997 up: the offset must be the float
    below 0.5, which the test above would catch through x * inv = 0.49999997."""
    r = F32(np.nextafter(F32(0.5), F32(0.0)))
    assert np.trunc((r + F32(0.5)).astype(F32)) == 1.0
    assert np.trunc((r + np.nextafter(F32(0.5), F32(0.0))).astype(F32)) == 0.0
    # and the kernel formula meets that value at some fp16 x and inv: x = 1, inv = r
    x16 = np.array([1.0], dtype=np.float16)
    assert kernel_q(x16, r)[0] == reference_q(x16, r)[0] == 0

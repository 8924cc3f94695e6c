"""Parity of the HIP path (through cider_amd -> C ABI) with the CPU oracle.

Bar: bit-exact for quantized activations, scales, int32 accumulators and
every GEMM output (per-channel, W4A8, per-group and W4 per-group at every M:
each kernel keeps the reference's fp32 operation order, including the
sequential per-group chain).  The fp16-activation MV (M == 1) sums each row
in its own order (the reference's Metal simd_sum tree is unspecified): it
must meet the MV bar of tests/util.py (north-star 1e-3 relative / 1 fp16 ulp
of the oracle, or the fp32 summation bound of the exact value); shapes
outside the streaming MV's table run the lane-order MV, which reproduces the
oracle's restated order bit for bit.
"""

import hashlib

import numpy as np
import pytest

from oracle import cider_oracle as O
from tests.golden.make_golden import bitexact_inputs
from tests.util import assert_pergroup_linear_close, assert_bits_equal, assert_mv_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cider_amd as C

DEV = "cuda"


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def H(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def synth_pc(M, N, K, seed, bias=True):
    x = O.synth_activations(M, K, seed)
    w = O.synth_weights_i8(N, K, seed + 1)
    sw = O.synth_scales(N, seed + 2)
    b = ((np.random.default_rng(seed + 3).standard_normal(N) * 0.1).astype(np.float16)
         if bias else None)
    return x, w, sw, b


# --------------------------------------------------------------------------
# a1 quantize_per_token: bit-exact
# --------------------------------------------------------------------------


@pytest.mark.parametrize("M,K", [(1, 8), (4, 2560), (7, 513), (33, 4097), (5, 10240),
                                 (3, 16392), (2, 20000), (9, 64), (6, 6)])
def test_quantize_bitexact(M, K):
    x = O.synth_activations(M, K, 11 + M + K)
    q, sa = C.quantize_per_token(T(x))
    qe, sae = O.quantize_per_token(x)
    assert_bits_equal(H(q), qe, "q")
    assert_bits_equal(H(sa), sae, "scale_a")


def test_quantize_special_rows():
    K = 256
    x = np.zeros((6, K), np.float16)
    # row 0 all zeros -> s = 1, q = 0
    # row 1 amax 127 -> s = 1: ties at .5 round away from zero (half-even would differ)
    x[1, :6] = [127.0, 2.5, -3.5, 0.5, -0.5, 1.5]
    # row 2 NaN is ignored by the absmax and quantizes to -128
    x[2, :3] = [np.nan, 3.0, -6.0]
    # row 3 inf: s = inf, inv = 0 -> 0 * inf = NaN -> -128, finite -> 0
    x[3, :3] = [np.inf, 1.0, -2.0]
    # row 4 subnormal fp16 only
    x[4, :4] = np.array([6e-8, -1.2e-7, 3e-8, 0], np.float16)
    # row 5 fp16 max
    x[5, :3] = [65504.0, -65504.0, 1.0]
    q, sa = C.quantize_per_token(T(x))
    qe, sae = O.quantize_per_token(x)
    assert_bits_equal(H(q), qe, "q")
    assert_bits_equal(H(sa), sae, "scale_a")
    qh = H(q)
    assert list(qh[1, :6]) == [127, 3, -4, 1, -1, 2]


# --------------------------------------------------------------------------
# a3 int8_matmul_int32: the reference's own 14 shapes, bit-exact
# --------------------------------------------------------------------------


def test_int8_matmul_reference_shapes(bitexact_shapes):
    for rec in bitexact_shapes:
        a, b = bitexact_inputs(rec["M"], rec["K"], rec["N"])
        c = H(C.int8_matmul_int32(T(a), T(b)))
        assert c.dtype == np.int32 and c.shape == (rec["M"], rec["N"])
        assert sha(c) == rec["sha_c"], (rec["M"], rec["K"], rec["N"])


# M > 64, K % 128 == 0, N % 8 == 0: the LDS-DMA kernel at each int32 tile the
# dispatcher picks (64x64: 256x256 and 300x520; the mixed 256x256 + 128x256
# grid: 2048x10240; 128x256: 2048x4096; 128x128: 1024x4096; 128x64: 128x10240;
# 64x128: 192x10240; 256x256: 4096x8192; 192x256: 1100x10240).
@pytest.mark.parametrize("M,N,K", [(65, 64, 64), (256, 256, 128), (300, 520, 384),
                                   (1000, 130, 1000), (2, 3, 1), (70, 90, 17),
                                   (2048, 10240, 128), (1024, 4096, 256), (128, 10240, 128),
                                   (192, 10240, 128), (4096, 8192, 256), (2048, 4096, 256),
                                   (1100, 10240, 128)])
def test_int8_matmul_more_shapes(M, N, K):
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int8)
    b = rng.integers(-128, 128, (N, K), dtype=np.int8)
    assert_bits_equal(H(C.int8_matmul_int32(T(a), T(b))), O.int8_matmul_int32(a, b))


def test_int8_matmul_extremes():
    K = 65536  # |acc| = 2^30, exact in int32
    for M in (3, 130):
        a = np.full((M, K), -128, np.int8)
        b = np.full((5, K), -128, np.int8)
        b[1] = 127
        c = H(C.int8_matmul_int32(T(a), T(b)))
        assert (c[:, 0] == 16384 * K).all() and (c[:, 1] == -128 * 127 * K).all()


# --------------------------------------------------------------------------
# a2 per-channel linear
# --------------------------------------------------------------------------


# Shapes cover every GEMM variant: skinny (M <= 64), the register-staged tiled
# kernel (K % 128 != 0 or N % 8 != 0) and the LDS-DMA kernel at each tile the
# dispatcher picks: 128x64 (M=128, N=10240), 64x64 (M=300/257), 128x128
# (M=2048, N=2048), 128x256 (M=600), 192x256 (M=1024, N=10240), 256x256
# (M=4096, N=8192), and the mixed 256x256 + 128x256 grid (M=2048, N=10240;
# M=1000, N=16640 with a partial last tile row; the full-size tests below);
# 64x128 in the midpoint test below.
@pytest.mark.parametrize("M,N,K", [(2, 16, 64), (7, 33, 130), (16, 1000, 2560), (33, 257, 513),
                                   (64, 128, 256), (65, 200, 320), (128, 10240, 2560),
                                   (300, 1000, 1024), (257, 512, 4096), (100, 70, 100),
                                   (1024, 10240, 2560), (2048, 2048, 1024), (600, 8192, 768),
                                   (2048, 10240, 256), (1000, 16640, 128), (4096, 8192, 128)])
def test_perchannel_linear_bitexact(M, N, K):
    for bias in (True, False):
        x, w, sw, b = synth_pc(M, N, K, 1000 + M + N + K, bias)
        y = C.perchannel_linear(T(x), T(w), T(sw), None if b is None else T(b))
        assert y.dtype == torch.float16 and tuple(y.shape) == (M, N)
        assert_bits_equal(H(y), O.perchannel_linear(x, w, sw, b), f"pc {M}x{N}x{K}")


def test_perchannel_gemm_matches_linear():
    M, N, K = 200, 384, 768
    x, w, sw, b = synth_pc(M, N, K, 77)
    q, sa = C.quantize_per_token(T(x))
    y1 = C.perchannel_gemm(q, sa, T(w), T(sw), T(b))
    y2 = C.perchannel_linear(T(x), T(w), T(sw), T(b))
    assert_bits_equal(H(y1), H(y2))


# The epilogue rounds f32(f32(acc) * sa) * sw to binary32 and then to fp16.  A
# fused multiply-and-convert (one rounding, straight to fp16) agrees except
# where the binary32 product lands exactly on an fp16 midpoint.  Random int8
# operands with random binary32 scales put a few hundred such elements in each
# case (the test asserts that they are there); the shapes select, in order,
# the 128 x 64, 64 x 64 (twice), 64 x 128 and 192 x 256 LDS-DMA tiles, the
# mixed grid, the register-staged kernel (K % 128 != 0), the skinny kernel and
# the GEMV.
@pytest.mark.parametrize("M,N,K,rows", [
    (128, 10240, 2560, None), (128, 2560, 10240, None), (1000, 1000, 1024, None),
    (192, 10240, 2560, None), (1100, 10240, 256, None),
    (4096, 10240, 2560, np.r_[0:64, 4032:4096]), (300, 1000, 1000, None),
    (48, 4096, 4096, None), (3, 10240, 2560, None)])
def test_perchannel_gemm_double_rounding_midpoints(M, N, K, rows):
    rng = np.random.default_rng(M + N + K)
    q = rng.integers(-127, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = (rng.random(M) * 0.01).astype(np.float32)
    sw = (rng.random(N) * 0.01).astype(np.float32)
    y = H(C.perchannel_gemm(T(q), T(sa), T(w), T(sw)))
    if rows is not None:
        y, q, sa = y[rows], q[rows], sa[rows]
    acc = O.int8_matmul_int32(q, w)
    p1 = (acc.astype(np.float32) * sa[:, None]).astype(np.float32)
    exact = p1.astype(np.float64) * sw.astype(np.float64)[None, :]   # exact: 48-bit product
    once = exact.astype(np.float16)                                   # numpy rounds once
    twice = exact.astype(np.float32).astype(np.float16)
    n_mid = int(np.sum(once.view(np.uint16) != twice.view(np.uint16)))
    assert n_mid > 0, "the data holds no double-rounding midpoint"
    assert_bits_equal(y, O.dequant_perchannel(acc, sa, sw, None), f"midpoints {M}x{N}x{K}")


# The same for the int4-weight per-channel GEMM (128 x 64 and 64 x 64 DMA
# tiles at M=128) and the per-group kernels, against their oracles.
@pytest.mark.parametrize("M,N,K", [(128, 10240, 2560), (128, 2560, 10240)])
def test_w4_and_pergroup_midpoint_shapes(M, N, K):
    rng = np.random.default_rng(M * 7 + N + K)
    x = (rng.standard_normal((M, K)) * 4).astype(np.float16)
    wf = rng.standard_normal((K, N)).astype(np.float32)
    packed, sw = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw)))
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw), f"w4 midpoints {M}x{N}x{K}")
    w8 = rng.integers(-127, 128, (N, K), dtype=np.int8)
    for gs in (64, 128):
        sc = (rng.random((K // gs, N)) * 0.01).astype(np.float32)
        y = H(C.pergroup_linear(T(x), T(w8), T(sc), gs))
        assert_pergroup_linear_close(y, x, w8, sc, None, gs, O.pergroup_linear(x, w8, sc, gs, None),
                                     f"pergroup gs{gs} midpoints {M}x{N}x{K}")


# K % 256 == 0 with 1024 <= K <= 16384 (in the streaming MV's table) runs the
# streaming MV: R rows per wave, 16-byte chunks, v_dot2 products; N=9 and
# N=130 leave the last wave partly past N.  Of those, K from 10240 to 16384
# with K % 1024 == 0 runs the k-split MV (KS = 4 or 5 waves share each row's
# k range; N=9, 3 and 1001 leave the last workgroup partly past N, N=2560
# takes KS = 5).  K=256 / 8 / 300 / 16640 run the lane-order MV
# (bounds-checked tail for K=300 and K=8).
@pytest.mark.parametrize("N,K", [(40, 256), (130, 1024), (10240, 2560), (2560, 10240),
                                 (100, 300), (7, 8), (8, 1280), (9, 1536), (100, 16384),
                                 (33, 16640), (4096, 12288), (12288, 4096), (1000, 3584),
                                 (50, 7680), (70, 3840), (9, 11264), (3, 10240),
                                 (1001, 13312), (64, 14336), (255, 15360)])
def test_perchannel_mv(N, K):
    x, w, sw, b = synth_pc(1, N, K, 500 + N + K)
    y = H(C.perchannel_linear(T(x), T(w), T(sw), T(b)))
    assert_mv_close(y, x, w, sw, b, 0, f"mv {N}x{K}")
    y0 = H(C.perchannel_linear(T(x), T(w), T(sw)))       # no bias: no add
    assert_mv_close(y0, x, w, sw, None, 0, f"mv {N}x{K} no bias")


# The lane-order MV (shapes outside the streaming MV's table) keeps the
# oracle's 32-lane / block / butterfly order: bit-exact.
@pytest.mark.parametrize("N,K", [(40, 256), (100, 300), (7, 8), (33, 16640), (64, 768)])
def test_lane_order_mv_bitexact(N, K):
    x, w, sw, b = synth_pc(1, N, K, 510 + N + K)
    y = H(C.perchannel_linear(T(x), T(w), T(sw), T(b)))
    assert_bits_equal(y, O.perchannel_linear(x, w, sw, b), f"lane-order mv {N}x{K}")
    gs = 64 if K % 64 == 0 else 0
    if gs:
        swg = O.synth_scales((K // gs, N), 511)
        yg = H(C.pergroup_linear(T(x), T(w), T(swg), gs, T(b)))
        assert_bits_equal(yg, O.pergroup_linear(x, w, swg, gs, b), f"lane-order pg mv {N}x{K}")


def test_bf16_and_fp32_inputs_roundtrip():
    M, N, K = 70, 96, 256
    x, w, sw, b = synth_pc(M, N, K, 9)
    xb = torch.from_numpy(x.astype(np.float32)).to(DEV).to(torch.bfloat16)
    y = C.perchannel_linear(xb, T(w), T(sw), T(b))
    assert y.dtype == torch.bfloat16
    x16 = xb.to(torch.float16).cpu().numpy()
    exp = torch.from_numpy(O.perchannel_linear(x16, w, sw, b)).to(torch.bfloat16)
    assert torch.equal(y.cpu(), exp)
    yf = C.perchannel_linear(T(x.astype(np.float32)), T(w), T(sw), T(b))
    assert yf.dtype == torch.float32
    assert_bits_equal(H(yf).astype(np.float16), O.perchannel_linear(x, w, sw, b))


def test_full_size_config1_row_slices_and_determinism():
    M, N, K = 4096, 10240, 2560
    x, w, sw, b = synth_pc(M, N, K, 20261202, bias=False)
    xd, wd, swd = T(x), T(w), T(sw)
    y1 = C.perchannel_linear(xd, wd, swd)
    y2 = C.perchannel_linear(xd, wd, swd)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16)), "non-deterministic"
    yh = H(y1)
    rows = np.r_[0:64, M - 64:M, np.random.default_rng(5).choice(M, 64, replace=False)]
    exp = O.perchannel_linear(x[rows], w, sw, None)
    assert_bits_equal(yh[rows], exp, "config1 rows")


def test_full_size_down_proj_rows():
    M, N, K = 1024, 2560, 10240
    x, w, sw, b = synth_pc(M, N, K, 31, bias=True)
    y = H(C.perchannel_linear(T(x), T(w), T(sw), T(b)))
    rows = np.r_[0:32, M - 32:M]
    assert_bits_equal(y[rows], O.perchannel_linear(x[rows], w, sw, b), "down rows")


# --------------------------------------------------------------------------
# a5/a6 per-group
# --------------------------------------------------------------------------


# M > 64 with K % 128 == 0 and N % 8 == 0 runs the LDS-DMA per-group kernel
# (one k-stage (K=128), two (K=256), an odd count (K=384), ragged M and N;
# gs 256 groups span two stages and their sets alternate over a 4-stage
# period: K=256 / 768 / 1280 end it after 2 stages, K=512 / 1024 after 4);
# K=320 runs the register-staged kernel.
@pytest.mark.parametrize("gs", [64, 128, 256])
@pytest.mark.parametrize("M,N,K", [(1, 72, 512), (1, 10240, 2560), (5, 48, 256), (16, 130, 512),
                                   (64, 100, 1024), (65, 96, 512), (300, 520, 1024),
                                   (130, 64, 320), (128, 256, 128), (200, 1024, 256),
                                   (257, 136, 384), (129, 264, 768), (96, 1032, 1280)])
def test_pergroup_linear(gs, M, N, K):
    if K % gs:
        pytest.skip("K not a multiple of gs")
    x = O.synth_activations(M, K, 40 + M + gs)
    w = O.synth_weights_i8(N, K, 41 + N)
    sw = O.synth_scales((K // gs, N), 42 + K)
    b = (np.random.default_rng(43).standard_normal(N) * 0.1).astype(np.float16)
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    if M == 1:
        assert_mv_close(y, x, w, sw, b, gs, f"pg mv gs{gs} {N}x{K}")
        return
    # M >= 2: the per-group bar (the GEMM kernels flush with fma; the small-M
    # kernels keep the sequential chain and are also checked bit for bit by
    # the small-M tests)
    assert_pergroup_linear_close(y, x, w, sw, b, gs, O.pergroup_linear(x, w, sw, gs, b),
                                 f"pg gs{gs} {M}x{N}x{K}")


@pytest.mark.parametrize("gs", [64, 128, 256])
@pytest.mark.parametrize("N,K", [(9, 16384), (4096, 12288), (2560, 10240), (17, 256)])
def test_pergroup_mv_shapes(gs, N, K):
    if K % gs:
        pytest.skip("K not a multiple of gs")
    x = O.synth_activations(1, K, 60 + gs)
    w = O.synth_weights_i8(N, K, 61 + N)
    sw = O.synth_scales((K // gs, N), 62 + K)
    b = (np.random.default_rng(63).standard_normal(N) * 0.1).astype(np.float16)
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    assert_mv_close(y, x, w, sw, b, gs, f"pg mv gs{gs} {N}x{K}")


@pytest.mark.parametrize("gs", [64, 128, 256])
@pytest.mark.parametrize("M,N,K", [(1024, 10240, 2560), (512, 2560, 10240)])
def test_pergroup_full_size_rows(gs, M, N, K):
    x = O.synth_activations(M, K, 50 + gs)
    w = O.synth_weights_i8(N, K, 51)
    sw = O.synth_scales((K // gs, N), 52)
    b = (np.random.default_rng(53).standard_normal(N) * 0.1).astype(np.float16)
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    rows = np.r_[0:16, M - 16:M]
    exp = O.pergroup_gemm(*O.quantize_per_token(x[rows]), w, sw, b, gs)
    assert_pergroup_linear_close(y[rows], x[rows], w, sw, b, gs, exp, f"pg gs{gs} {M}x{N}x{K} rows")


# --------------------------------------------------------------------------
# a7 W4A8 (reference layout) and the per-group int4 extension
# --------------------------------------------------------------------------


def test_w4_repack_matches_unpack():
    rng = np.random.default_rng(3)
    for K, N in [(2, 1), (64, 70), (130, 129), (4096, 256)]:
        src = rng.integers(0, 256, (K // 2, N), dtype=np.uint8)
        dst = H(C.repack_w4_ref(T(src)))
        assert dst.shape == (N, K // 2)
        np.testing.assert_array_equal(O.unpack_w4_lo_first(dst), O.unpack_w4_ref(src).T)


# M > 64, K % 128 == 0, N % 8 == 0 runs the LDS-DMA kernel with int4 weights
# (512x640, 256x1024 and 300x136 -- an odd stage count -- on 64x64 tiles,
# 192x6144 and 192x10240 on 64x128, 2048x2048 on 128x128, 2048x4096 on
# 128x256, 2048x10240 on the mixed grid, 1024x10240 on 192x256; 256x256 in the
# full-size test and 128x64 in the midpoint test below); N % 8 != 0 the
# register-staged kernel; M <= 64 the skinny kernel.
@pytest.mark.parametrize("M,N,K", [(1, 32, 64), (9, 70, 160), (1, 12288, 4096),
                                   (16, 4096, 12288), (64, 300, 1024), (100, 300, 1024),
                                   (512, 640, 2048), (7, 33, 98), (256, 1024, 512),
                                   (300, 136, 384), (2048, 10240, 256), (192, 6144, 1024),
                                   (192, 10240, 2560), (2048, 2048, 1024), (2048, 4096, 1024),
                                   (1024, 10240, 256)])
def test_w4a8_linear_ref_layout(M, N, K):
    x = O.synth_activations(M, K, 60 + M)
    wf = np.random.default_rng(61 + N).standard_normal((K, N)).astype(np.float32)
    packed, sw = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw)))
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw), f"w4 {M}x{N}x{K}")


def test_w4a8_full_size_rows():
    M, N, K = 4096, 12288, 4096
    x = O.synth_activations(M, K, 62)
    wf = np.random.default_rng(63).standard_normal((K, N)).astype(np.float32)
    packed, sw = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw)))
    rows = np.r_[0:16, M - 16:M]
    assert_bits_equal(y[rows], O.w4a8_linear(x[rows], packed, sw), "w4 full-size rows")


# M > 64, K % 128 == 0 and N % 8 == 0 runs the LDS-DMA per-group kernel with
# int4 weights (100x96, 512x640, one stage at K=128, an odd stage count at
# K=384).
@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("M,N,K", [(1, 48, 256), (16, 300, 1024), (17, 40, 512),
                                   (100, 96, 512), (512, 640, 2048), (128, 256, 128),
                                   (257, 136, 384)])
def test_w4a8_pergroup(gs, M, N, K):
    x = O.synth_activations(M, K, 70 + M)
    w4 = np.random.default_rng(71 + N).integers(-8, 8, (N, K), dtype=np.int8)
    packed = O.pack_w4_lo_first(w4)
    sc = O.synth_scales((K // gs, N), 72 + K).astype(np.float16)
    y = H(C.w4a8_pergroup_linear(T(x), T(packed), T(sc), gs))
    exp = O.w4a8_pergroup_linear(x, packed, sc, gs)
    if (M, N, K) == (512, 640, 2048):
        # split K in two (fp32 chains of the slices, added): the per-group bar
        assert_pergroup_linear_close(y, x, w4, sc, None, gs, exp, f"w4g gs{gs} {M}x{N}x{K}")
    else:
        # the small-M kernels and the two-set DMA kernel (exact fast flush of
        # fp16 scales) keep the sequential chain
        assert_bits_equal(y, exp, f"w4g gs{gs} {M}x{N}x{K}")


@pytest.mark.parametrize("gs", [64, 128])
def test_w4a8_pergroup_full_size_rows(gs):
    M, N, K = 4096, 12288, 4096
    x = O.synth_activations(M, K, 73 + gs)
    w4 = np.random.default_rng(74).integers(-8, 8, (N, K), dtype=np.int8)
    packed = O.pack_w4_lo_first(w4)
    sc = O.synth_scales((K // gs, N), 75).astype(np.float16)
    y = H(C.w4a8_pergroup_linear(T(x), T(packed), T(sc), gs))
    rows = np.r_[0:16, M - 16:M]
    exp = O.w4a8_pergroup_linear(x[rows], packed, sc, gs)
    assert_pergroup_linear_close(y[rows], x[rows], w4, sc, None, gs, exp, f"w4g gs{gs} full-size rows")


# fp16 group scales take the fast flush (each group's int32 sum starts from
# the bit pattern of 1.5 * 2^23 and one fma of those bits rounds D * s once);
# a tile whose scales include +-inf or NaN gives NaN there and is redone with
# the exact flush.  Special scales sit in a few columns (so some tiles stay
# fast and some are redone), rows of zeros give D_g = 0 against the infinite
# scales (NaN in the reference), and every tile shape runs: 128 x 128 of
# 8 waves (gs 64, 2048 x 1280), two 128 x 64 workgroups per CU (gs 128),
# 64 x 64 tiles (128 x 512), M = 48, the M <= 16 weight stream, the decode
# GEMV (M = 1, 3) and the register-staged kernel (N % 8 != 0).  Infinite
# scales in group 0 also check the flush before the first group, which must
# add +0.0 whatever group 0's scales are.
_SPECIAL_SCALES = {(0, 6): np.inf, (0, 78): -np.inf, (1, 5): np.inf, (2, 77): -np.inf,
                   (0, 200): np.nan, (3, 300): 0.0, (1, 301): -0.0, (0, 302): 2.0 ** -24,
                   (2, 303): 65504.0, (1, 304): -65504.0, (0, 1100): np.inf}


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("M,N,K", [(2048, 1280, 512), (128, 512, 1024), (48, 1280, 1024),
                                   (8, 1280, 2048), (3, 1280, 2048), (1, 1280, 2048),
                                   (300, 1004, 384)])
def test_w4a8_pergroup_special_scales(gs, M, N, K):
    x = O.synth_activations(M, K, 80 + M)
    if M > 2:                                      # (no zero row at M <= 2)
        x[5 % M, :] = 0
    if M > 130:
        x[130, :] = 0
    w4 = np.random.default_rng(81 + N).integers(-8, 8, (N, K), dtype=np.int8)
    w4[:, :gs] = -8                                # |D| at its largest in group 0
    packed = O.pack_w4_lo_first(w4)
    sc = O.synth_scales((K // gs, N), 82 + K).astype(np.float16)
    for (g, n), v in _SPECIAL_SCALES.items():
        if n < N:
            sc[g % (K // gs), n] = v
    b = (np.random.default_rng(83).standard_normal(N) * 0.1).astype(np.float16)
    y = H(C.w4a8_pergroup_linear(T(x), T(packed), T(sc), gs, T(b)))
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.w4a8_pergroup_linear(x, packed, sc, gs, b)
    assert np.isinf(exp).any() and np.isnan(exp).any()
    assert_bits_equal(y, exp, f"w4g special scales gs{gs} {M}x{N}x{K}")


# The same special scales (fp32) on int8 weights: every per-group tile shape
# and group size, including the 8-wave gs 256 tile (2048 x 1280).
@pytest.mark.parametrize("gs", [64, 128, 256])
@pytest.mark.parametrize("M,N,K", [(2048, 1280, 1024), (128, 512, 1024), (48, 1280, 1024),
                                   (8, 1280, 2048), (3, 1280, 2048), (300, 1004, 768)])
def test_pergroup_special_scales(gs, M, N, K):
    x, w, _, b = synth_pc(M, N, K, 84 + M)
    if M > 2:
        x[5 % M, :] = 0
    w[:, :gs] = -127
    sw = O.synth_scales((K // gs, N), 85 + gs)
    for (g, n), v in _SPECIAL_SCALES.items():
        if n < N:
            sw[g % (K // gs), n] = v
    sw[1, 6] = np.float32(3.0e38)                  # the product overflows to inf
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.pergroup_linear(x, w, sw, gs, b)
    assert np.isinf(exp).any() and np.isnan(exp).any()
    # tiles with these scales take the exact chain, the others the fma flush
    assert_pergroup_linear_close(y, x, w, sw, b, gs, exp, f"pg special scales gs{gs} {M}x{N}x{K}")


# Grids of at least 512 tiles of 128 x 128 run the one-set per-group kernel
# (64 x 64 waves, int8 weights with fp32 scales): ragged M and N (the last
# tile row and column partly outside), every group size, special scales in
# the first and the last tile column; rows of the first tile row, across
# tile-row boundaries, in the middle and of the last tile row.
@pytest.mark.parametrize("gs", [64, 128, 256])
def test_pergroup_one_set_tiles(gs):
    M, N, K = 4059, 8200, 768                      # 32 x 65 tiles of 128 x 128
    x, w, _, b = synth_pc(M, N, K, 86 + gs)
    x[5, :] = 0
    w[:, :gs] = -127
    sw = O.synth_scales((K // gs, N), 87 + gs)
    for (g, n), v in _SPECIAL_SCALES.items():
        sw[g % (K // gs), n] = v
        sw[(g + 1) % (K // gs), N - 1 - n % 64] = v
    sw[1, 6] = np.float32(3.0e38)                  # the product overflows to inf
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    rows = np.r_[0:8, 250:262, 2000:2004, M - 27:M]
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.pergroup_gemm(*O.quantize_per_token(x[rows]), w, sw, b, gs)
    assert np.isinf(exp).any() and np.isnan(exp).any()
    assert_pergroup_linear_close(y[rows], x[rows], w, sw, b, gs, exp,
                                 f"pg one-set tiles gs{gs} {M}x{N}x{K} rows")


# Few rows on a very wide N also reach the one-set kernel (M <= 64 with N >= 8192
# takes the per-group DMA tiles; 512 tiles of 128 x 128 from N = 65536): every
# tile has one partial tile row, and the last tile column is ragged.
@pytest.mark.parametrize("gs", [64, 128])
def test_pergroup_one_set_few_rows(gs):
    M, N, K = 40, 65544, 256
    x, w, _, b = synth_pc(M, N, K, 98 + gs)
    sw = O.synth_scales((K // gs, N), 99 + gs)
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    assert_pergroup_linear_close(y, x, w, sw, b, gs, O.pergroup_linear(x, w, sw, gs, b),
                                 f"pg one-set few rows gs{gs}")


# The one-set kernel at its shortest k-loops: one and two stages of 128 (the
# loop body never runs; the prologue's reload of the last stage fills the
# second ring slot), 512 tiles of 128 x 128.
@pytest.mark.parametrize("gs,K", [(64, 128), (128, 128), (64, 256), (128, 256), (256, 256)])
def test_pergroup_one_set_short_k(gs, K):
    M, N = 2048, 4096
    x, w, _, b = synth_pc(M, N, K, 92 + gs + K)
    sw = O.synth_scales((K // gs, N), 93 + gs)
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    rows = np.r_[0:4, 1020:1030, M - 6:M]
    exp = O.pergroup_gemm(*O.quantize_per_token(x[rows]), w, sw, b, gs)
    assert_pergroup_linear_close(y[rows], x[rows], w, sw, b, gs, exp,
                                 f"pg one-set short K gs{gs} {M}x{N}x{K} rows")


# The same kernel with int4 weights and fp16 group scales.
@pytest.mark.parametrize("gs", [64, 128])
def test_w4a8_pergroup_one_set_tiles(gs):
    M, N, K = 4059, 8200, 768
    x = O.synth_activations(M, K, 88 + gs)
    x[5, :] = 0
    w4 = np.random.default_rng(89).integers(-8, 8, (N, K), dtype=np.int8)
    w4[:, :gs] = -8
    packed = O.pack_w4_lo_first(w4)
    sc = O.synth_scales((K // gs, N), 90 + gs).astype(np.float16)
    for (g, n), v in _SPECIAL_SCALES.items():
        sc[g % (K // gs), n] = v
        sc[(g + 1) % (K // gs), N - 1 - n % 64] = v
    b = (np.random.default_rng(91).standard_normal(N) * 0.1).astype(np.float16)
    y = H(C.w4a8_pergroup_linear(T(x), T(packed), T(sc), gs, T(b)))
    rows = np.r_[0:8, 250:262, 2000:2004, M - 27:M]
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.w4a8_pergroup_linear(x[rows], packed, sc, gs, b)
    assert np.isinf(exp).any() and np.isnan(exp).any()
    assert_pergroup_linear_close(y[rows], x[rows], w4, sc, b, gs, exp,
                                 f"w4g one-set tiles gs{gs} {M}x{N}x{K} rows")


# Decode-sized GEMV on quantized activations (M <= 4, K <= 16384, K % 16 == 0
# for int8 / % 32 for int4): one wave per weight row, v_dot4 products; N=17
# leaves most waves of the last workgroup without a row.
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("N,K", [(17, 256), (300, 2560), (1024, 16384), (64, 12288)])
def test_gemv_q_exact(M, N, K):
    x, w, sw, b = synth_pc(M, N, K, 100 + M + N)
    if M > 1:  # M == 1 on W8 runs the fp16 MV
        y = H(C.perchannel_linear(T(x), T(w), T(sw), T(b)))
        assert_bits_equal(y, O.perchannel_linear(x, w, sw, b), f"gemv pc {M}x{N}x{K}")
        for gs in (64, 128, 256):
            swg = O.synth_scales((K // gs, N), 101 + gs)
            yg = H(C.pergroup_linear(T(x), T(w), T(swg), gs, T(b)))
            assert_bits_equal(yg, O.pergroup_linear(x, w, swg, gs, b), f"gemv pg{gs} {M}x{N}x{K}")
    q = np.random.default_rng(102).integers(-128, 128, (M, K), dtype=np.int8)
    assert np.array_equal(C.int8_matmul_int32(T(q), T(w)).cpu().numpy(),
                          O.int8_matmul_int32(q, w)), f"gemv i32 {M}x{N}x{K}"
    wf = np.random.default_rng(103).standard_normal((K, N)).astype(np.float32)
    packed, sw4 = O.pack_weight_int4(wf)
    assert_bits_equal(H(C.w4a8_linear(T(x), T(packed), T(sw4))),
                      O.w4a8_linear(x, packed, sw4), f"gemv w4 {M}x{N}x{K}")
    w4 = np.random.default_rng(104).integers(-8, 8, (N, K), dtype=np.int8)
    for gs in (64, 128):
        sc = O.synth_scales((K // gs, N), 105 + gs).astype(np.float16)
        pk = O.pack_w4_lo_first(w4)
        assert_bits_equal(H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, T(b))),
                          O.w4a8_pergroup_linear(x, pk, sc, gs, b), f"gemv w4g{gs} {M}x{N}x{K}")


# W4A8 per-group at M == 1 with K a multiple of 1024 from 2048 (of 2048 past
# 8192) and N % 8 == 0: the streaming GEMV (4 rows per wave up to K = 8192, 1
# row per wave in 8-wave workgroups above), x quantized in the kernel.  N of
# 8, 24, 1032 and 4104 leave the last workgroup partly outside; special
# scales in the first rows.
@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("N,K", [(1032, 4096), (8, 8192), (24, 10240), (4104, 3072),
                                 (256, 16384), (520, 2048)])
def test_w4a8_gemv1_stream(gs, N, K):
    x = O.synth_activations(1, K, 94 + N)
    w4 = np.random.default_rng(95 + K).integers(-8, 8, (N, K), dtype=np.int8)
    w4[:, :gs] = -8
    pk = O.pack_w4_lo_first(w4)
    sc = O.synth_scales((K // gs, N), 96 + gs).astype(np.float16)
    sc[0, 0], sc[1 % (K // gs), 1] = np.inf, np.nan
    sc[0, 2], sc[0, 3] = 0.0, 65504.0
    for bias in (True, False):
        b = (np.random.default_rng(97).standard_normal(N) * 0.1).astype(np.float16) if bias else None
        y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, None if b is None else T(b)))
        with np.errstate(invalid="ignore", over="ignore"):
            exp = O.w4a8_pergroup_linear(x, pk, sc, gs, b)
        assert_bits_equal(y, exp, f"w4g M=1 stream gs{gs} N={N} K={K} bias={bias}")


# The same streaming GEMV with per-channel fp32 scales (the reference's own
# W4A8, weights in its [K/2, N] layout, no bias).
@pytest.mark.parametrize("N,K", [(1032, 4096), (8, 8192), (24, 10240), (4104, 3072),
                                 (256, 16384), (520, 2048), (12288, 4096)])
def test_w4a8_gemv1_stream_perchannel(N, K):
    x = O.synth_activations(1, K, 98 + N)
    wf = np.random.default_rng(99 + K).standard_normal((K, N)).astype(np.float32)
    packed, sw = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw)))
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw), f"w4 pc M=1 stream N={N} K={K}")


# M <= 16 with K % 512 == 0 and K >= 1536: the weight stream through LDS
# (skinny_dma.hip) for every format.  Covered: 8 and 16 activation slots
# (M <= 8 re-reads rows for the MFMA's columns past 8), one to four blocks of
# 16 rows per workgroup, N past the last block (1000, 8196, 4100; per-group
# needs N % 8 == 0, so 8196 and 4100 take the other kernels there), the fewest
# stages the ring takes (K = 1536: 3 stages of 512), long K (12288: 24
# stages), a grid of more than one round (N = 20480, 4 blocks per workgroup:
# 320 workgroups), and per-group chains over 8 / 4 / 2 groups per stage (gs
# 64 / 128 / 256, the last summing two waves' halves of a group).
@pytest.mark.parametrize("M,N,K", [(5, 1000, 1536), (8, 2560, 10240), (9, 8196, 2048),
                                   (12, 4100, 12288), (16, 20480, 2560), (16, 10240, 2560),
                                   (13, 12288, 4096), (6, 4096, 2048), (16, 64, 1536)])
def test_skinny_dma_exact(M, N, K):
    x, w, sw, b = synth_pc(M, N, K, 140 + M)
    for bias in (b, None):
        y = H(C.perchannel_linear(T(x), T(w), T(sw), None if bias is None else T(bias)))
        assert_bits_equal(y, O.perchannel_linear(x, w, sw, bias), f"skinny dma pc {M}x{N}x{K}")
    q = np.random.default_rng(141).integers(-128, 128, (M, K), dtype=np.int8)
    q[0, :] = -128  # the extremes: -128 * -127 summed over K
    w2 = w.copy()
    w2[: min(N, 5), :] = -127
    c = C.int8_matmul_int32(T(q), T(w2)).cpu().numpy()
    assert np.array_equal(c, O.int8_matmul_int32(q, w2)), f"skinny dma i32 {M}x{N}x{K}"
    for gs in (64, 128, 256):
        swg = O.synth_scales((K // gs, N), 142 + gs)
        y = H(C.pergroup_linear(T(x), T(w), T(swg), gs, T(b)))
        assert_bits_equal(y, O.pergroup_linear(x, w, swg, gs, b), f"skinny dma pg{gs} {M}x{N}x{K}")
    w4 = np.random.default_rng(143).integers(-8, 8, (N, K), dtype=np.int8)
    w4[0, :] = -8
    pk = O.pack_w4_lo_first(w4)
    for gs in (64, 128):
        sc = O.synth_scales((K // gs, N), 144 + gs).astype(np.float16)
        for bias in (b, None):
            y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, None if bias is None else T(bias)))
            assert_bits_equal(y, O.w4a8_pergroup_linear(x, pk, sc, gs, bias),
                              f"skinny dma w4g{gs} {M}x{N}x{K}")
    wf = np.random.default_rng(145).standard_normal((K, N)).astype(np.float32)
    packed, sw4 = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw4)))
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw4), f"skinny dma w4 {M}x{N}x{K}")


# Special activation rows through the small-M kernels (the fused decode GEMV
# at (2, 2560, 1536), the LDS weight stream at the others): zeros (s = 1),
# NaN (-128), one inf (s = inf: NaN and +-inf outputs), fp16 maxima,
# subnormals; every format and epilogue against the oracle, and per-channel
# also against the quantize and GEMM entry points called one after the other.
@pytest.mark.parametrize("M,N,K", [(2, 2560, 1536), (5, 1000, 4096), (8, 10240, 2560),
                                   (9, 4096, 2048), (16, 12288, 4096), (16, 64, 1536)])
def test_small_m_special_rows(M, N, K):
    x, w, sw, b = synth_pc(M, N, K, 170 + M)
    x[0, :] = 0
    x[1, :3] = [np.nan, 3.0, -6.0]
    if M > 2:
        x[2, 7] = np.inf
    if M > 3:
        x[3, :] = np.where(np.arange(K) % 3 == 0, -65504.0, 65504.0)
    if M > 4:
        x[4, :] = 0
        x[4, :4] = np.array([6e-8, -1.2e-7, 3e-8, 0], np.float16)
    with np.errstate(invalid="ignore", over="ignore"):
        for bias in (b, None):
            y = H(C.perchannel_linear(T(x), T(w), T(sw), None if bias is None else T(bias)))
            assert_bits_equal(y, O.perchannel_linear(x, w, sw, bias), f"small-M pc {M}x{N}x{K}")
            q, sa = C.quantize_per_token(T(x))
            y2 = H(C.perchannel_gemm(q, sa, T(w), T(sw), None if bias is None else T(bias)))
            assert_bits_equal(y, y2, f"small-M pc vs quantize + gemm {M}x{N}x{K}")
        for gs in (64, 128, 256):
            swg = O.synth_scales((K // gs, N), 171 + gs)
            y = H(C.pergroup_linear(T(x), T(w), T(swg), gs, T(b)))
            assert_bits_equal(y, O.pergroup_linear(x, w, swg, gs, b), f"small-M pg{gs} {M}x{N}x{K}")
        w4 = np.random.default_rng(172).integers(-8, 8, (N, K), dtype=np.int8)
        pk = O.pack_w4_lo_first(w4)
        for gs in (64, 128):
            sc = O.synth_scales((K // gs, N), 173 + gs).astype(np.float16)
            y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, T(b)))
            assert_bits_equal(y, O.w4a8_pergroup_linear(x, pk, sc, gs, b),
                              f"small-M w4g{gs} {M}x{N}x{K}")
        wf = np.random.default_rng(174).standard_normal((K, N)).astype(np.float32)
        packed, sw4 = O.pack_weight_int4(wf)
        y = H(C.w4a8_linear(T(x), T(packed), T(sw4)))
        assert_bits_equal(y, O.w4a8_linear(x, packed, sw4), f"small-M w4 {M}x{N}x{K}")


# Per-group at mid M on small N: 64 x 64 tiles of four 32 x 32 waves, where the
# 128-row tiles would fill at most half the CUs, and their split-K form
# (K slices of fp32 chains, summed) where even those fill at most half the
# CUs: (65, 2560, 10240) leaves a one-row tile (split in 4), (128, 2560,
# 10240) splits in 4, (200, 1032, 2048) a ragged row tile and N past the
# last 64-column tile; every group size and both weight formats, against
# the per-group bar.
@pytest.mark.parametrize("M,N,K", [(65, 2560, 10240), (128, 2560, 10240), (200, 1032, 2048),
                                   (512, 4096, 4096)])
def test_pergroup_small_tiles(M, N, K):
    x, w, _, b = synth_pc(M, N, K, 160 + M)
    for gs in (64, 128, 256):
        swg = O.synth_scales((K // gs, N), 161 + gs)
        y = H(C.pergroup_linear(T(x), T(w), T(swg), gs, T(b)))
        assert_pergroup_linear_close(y, x, w, swg, b, gs, O.pergroup_linear(x, w, swg, gs, b),
                                     f"pg64 tiles gs{gs} {M}x{N}x{K}")
    w4 = np.random.default_rng(162).integers(-8, 8, (N, K), dtype=np.int8)
    pk = O.pack_w4_lo_first(w4)
    for gs in (64, 128):
        sc = O.synth_scales((K // gs, N), 163 + gs).astype(np.float16)
        y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, T(b)))
        assert_pergroup_linear_close(y, x, w4, sc, b, gs, O.w4a8_pergroup_linear(x, pk, sc, gs, b),
                                     f"pg64 tiles w4g{gs} {M}x{N}x{K}")


# Split-K per-group with special scales: the slices whose tiles hold
# them take the exact chain from global memory (fp32 scales) or redo the
# fast flush exactly (fp16 scales), the others flush with fma; the slices'
# partial sums then carry the infinities and NaNs into the sum.
@pytest.mark.parametrize("M,N,gs", [(128, 2560, 64), (128, 2560, 128), (128, 2560, 256),
                                    (256, 2560, 64), (256, 2560, 128), (256, 2560, 256),
                                    (512, 4096, 64), (512, 4096, 128), (512, 4096, 256)])
def test_pergroup_splitk_special_scales(M, N, gs):
    # two K slices of the two-set kernel: 40 tiles of 128 x 64 at M=128, of
    # 128 x 128 at M=256; gs 256 at M=128: four, of 80 tiles of 64 x 64.
    # M=512 N=4096: four slices of the one-set kernel's 128 tiles.
    K = 4096
    x, w, _, b = synth_pc(M, N, K, 164 + gs)
    x[5, :] = 0
    w[:, :gs] = -127
    sw = O.synth_scales((K // gs, N), 165 + gs)
    for (g, n), v in _SPECIAL_SCALES.items():
        sw[(g * 7) % (K // gs), n] = v              # spread over the slices
    sw[20 % (K // gs), 6] = np.float32(3.0e38)
    y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.pergroup_linear(x, w, sw, gs, b)
    assert np.isinf(exp).any() and np.isnan(exp).any()
    assert_pergroup_linear_close(y, x, w, sw, b, gs, exp, f"pg split-K special M={M} gs{gs}")
    if gs == 256:
        return                                     # the W4A8 formats define gs 64 / 128
    w4 = np.random.default_rng(166).integers(-8, 8, (N, K), dtype=np.int8)
    w4[:, :gs] = -8
    pk = O.pack_w4_lo_first(w4)
    sc = O.synth_scales((K // gs, N), 167 + gs).astype(np.float16)
    for (g, n), v in _SPECIAL_SCALES.items():
        sc[(g * 7) % (K // gs), n] = v
    y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, T(b)))
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.w4a8_pergroup_linear(x, pk, sc, gs, b)
    assert np.isinf(exp).any() and np.isnan(exp).any()
    assert_pergroup_linear_close(y, x, w4, sc, b, gs, exp, f"w4g split-K special M={M} gs{gs}")


# Split-K per-channel GEMM (M from 17 to 512 where the tiles fill at most a
# quarter of the CUs): int32 partial sums of K slices, summed (exact) by the
# dequant kernel in the tile epilogue's operation order.  Slices:
# (128, 2560, 10240) and (64, 2560, 10240) eight, (17, 4096, 12288) eight,
# (130, 2560, 4096) four with a ragged row tile, (256, 2560, 10240) four,
# (200, 1000, 4096) four with N past the last 128-column tile; (512, 2560,
# 2560) has 80 tiles and runs one pass, and so does (512, 2048, 2048), whose
# 64 x 64 tiles fill the CUs.  The extremes (-127 everywhere) are summed over
# the longest slices.
@pytest.mark.parametrize("M,N,K", [(128, 2560, 10240), (64, 2560, 10240), (17, 4096, 12288),
                                   (130, 2560, 4096), (256, 2560, 10240), (200, 1000, 4096),
                                   (512, 2560, 2560), (512, 2048, 2048)])
def test_splitk_perchannel_exact(M, N, K):
    x, w, sw, b = synth_pc(M, N, K, 150 + M)
    x[0, :] = 0                                  # s = 1, q = 0
    x[1, :3] = [65504.0, -65504.0, 1.0]
    for bias in (b, None):
        y = H(C.perchannel_linear(T(x), T(w), T(sw), None if bias is None else T(bias)))
        assert_bits_equal(y, O.perchannel_linear(x, w, sw, bias), f"split-K pc {M}x{N}x{K}")
    xe = np.full((M, K), -60000.0, dtype=np.float16)   # quantizes to -127 everywhere
    we = np.full((N, K), -127, dtype=np.int8)
    y = H(C.perchannel_linear(T(xe), T(we), T(sw), T(b)))
    assert_bits_equal(y, O.perchannel_linear(xe, we, sw, b), f"split-K extremes {M}x{N}x{K}")


# Skinny kernel (M <= 64) at shapes where N alone gives few workgroups, so the
# K range is split over 8 or 16 waves per workgroup (int32 sums exact in any
# order); per-group deals the groups to the waves round-robin and keeps the
# sequential group chain, so it is bit-exact too (K = 12288 at gs = 64: 192
# groups, a chain long enough for any other order to show).
@pytest.mark.parametrize("M,N,K", [(16, 2560, 10240), (32, 1024, 8192), (3, 256, 16384),
                                   (48, 512, 4096)])
def test_skinny_wave_splits_exact(M, N, K):
    x, w, sw, b = synth_pc(M, N, K, 90 + M)
    y = H(C.perchannel_linear(T(x), T(w), T(sw), T(b)))
    assert_bits_equal(y, O.perchannel_linear(x, w, sw, b), f"skinny pc {M}x{N}x{K}")
    q = np.random.default_rng(91).integers(-128, 128, (M, K), dtype=np.int8)
    c = C.int8_matmul_int32(T(q), T(w)).cpu().numpy()
    assert np.array_equal(c, O.int8_matmul_int32(q, w)), f"skinny i32 {M}x{N}x{K}"
    wf = np.random.default_rng(92).standard_normal((K, N)).astype(np.float32)
    packed, sw4 = O.pack_weight_int4(wf)
    y4 = H(C.w4a8_linear(T(x), T(packed), T(sw4)))
    assert_bits_equal(y4, O.w4a8_linear(x, packed, sw4), f"skinny w4 {M}x{N}x{K}")


# 5 <= M <= 64 with at least 128 column tiles of 64 (or M > 48) runs the
# LDS-DMA kernel's 64 x 64 tiles (int4 weights; per-channel and int32 at
# M > 16 or K not a multiple of 512) instead of the skinny kernel: rows past M
# are loaded from the last valid row and never stored.  Per-group at >= 128 column tiles runs the 128-row per-group DMA
# tiles for M > 32, and for int8 weights at gs 128 at every M: (16, 10240,
# 2560) and (5, 12288, 512) int8 gs 128; (33, 8192, 1024) and (64, 8192, 512)
# every per-group variant, (17, 10240, 2560) and (24, 8192, 1024) int8
# per-group at M <= 32; the others stay on the skinny kernel ((64, 512, 4096)
# and (40, 2560, 2048): per-group with 4 row blocks and 8 waves per workgroup).
@pytest.mark.parametrize("M,N,K", [(16, 10240, 2560), (5, 12288, 512), (33, 8192, 1024),
                                   (64, 8192, 512), (64, 512, 4096), (40, 2560, 2048),
                                   (49, 96, 256), (17, 10240, 2560), (24, 8192, 1024)])
def test_small_m_dma_tiles(M, N, K):
    x, w, sw, b = synth_pc(M, N, K, 98 + M)
    y = H(C.perchannel_linear(T(x), T(w), T(sw), T(b)))
    assert_bits_equal(y, O.perchannel_linear(x, w, sw, b), f"small-M dma pc {M}x{N}x{K}")
    q = np.random.default_rng(99).integers(-128, 128, (M, K), dtype=np.int8)
    c = C.int8_matmul_int32(T(q), T(w)).cpu().numpy()
    assert np.array_equal(c, O.int8_matmul_int32(q, w)), f"small-M dma i32 {M}x{N}x{K}"
    wf = np.random.default_rng(100).standard_normal((K, N)).astype(np.float32)
    packed, sw4 = O.pack_weight_int4(wf)
    y4 = H(C.w4a8_linear(T(x), T(packed), T(sw4)))
    assert_bits_equal(y4, O.w4a8_linear(x, packed, sw4), f"small-M dma w4 {M}x{N}x{K}")
    # per-group at the same shapes: the skinny kernels keep the sequential
    # group chain (bit-exact); the per-group DMA tiles (int8 weights on wide
    # N) flush fp32 scales with fma (the per-group bar); with fp16 scales
    # (W4A8) they keep the exact fast flush
    for gs in (64, 128):
        if K % gs:
            continue
        swg = O.synth_scales((K // gs, N), 101 + gs)
        yg = H(C.pergroup_linear(T(x), T(w), T(swg), gs))
        exp = O.pergroup_linear(x, w, swg, gs)
        if N >= 8192:
            assert_pergroup_linear_close(yg, x, w, swg, None, gs, exp,
                                         f"small-M dma pg{gs} {M}x{N}x{K}")
        else:
            assert_bits_equal(yg, exp, f"small-M dma pg{gs} {M}x{N}x{K}")
        w4 = np.random.default_rng(102).integers(-8, 8, (N, K), dtype=np.int8)
        pk = O.pack_w4_lo_first(w4)
        sc = O.synth_scales((K // gs, N), 103).astype(np.float16)
        yw = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs))
        assert_bits_equal(yw, O.w4a8_pergroup_linear(x, pk, sc, gs),
                          f"small-M dma w4g{gs} {M}x{N}x{K}")


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 12288), (16, 4096, 12288), (5, 2560, 10240)])
def test_skinny_wave_splits_pergroup(gs, M, N, K):
    x = O.synth_activations(M, K, 93 + M)
    w4 = np.random.default_rng(94).integers(-8, 8, (N, K), dtype=np.int8)
    sc = O.synth_scales((K // gs, N), 95).astype(np.float16)
    y = H(C.w4a8_pergroup_linear(T(x), T(O.pack_w4_lo_first(w4)), T(sc), gs))
    assert_bits_equal(y, O.w4a8_pergroup_linear(x, O.pack_w4_lo_first(w4), sc, gs),
                      f"skinny w4g gs{gs} {M}x{N}x{K}")
    if M > 1:
        w = O.synth_weights_i8(N, K, 96)
        sw = O.synth_scales((K // gs, N), 97)
        y8 = H(C.pergroup_linear(T(x), T(w), T(sw), gs))
        assert_bits_equal(y8, O.pergroup_linear(x, w, sw, gs), f"skinny pg gs{gs} {M}x{N}x{K}")


# --------------------------------------------------------------------------
# committed golden fixtures
# --------------------------------------------------------------------------


def test_golden_fixtures(golden_cases):
    d = golden_cases
    for i in range(4):
        x, w, sw, b = (d[f"pc{i}_{k}"] for k in ("x", "w", "sw", "bias"))
        q, sa = C.quantize_per_token(T(x))
        assert_bits_equal(H(q), d[f"pc{i}_q"])
        assert_bits_equal(H(sa), d[f"pc{i}_sa"])
        assert_bits_equal(H(C.perchannel_linear(T(x), T(w), T(sw), T(b))), d[f"pc{i}_y"])
    for i in range(2):
        x, w, sw, b = (d[f"mv{i}_{k}"] for k in ("x", "w", "sw", "bias"))
        assert_mv_close(H(C.perchannel_linear(T(x), T(w), T(sw), T(b))), x, w, sw, b, 0,
                        f"golden mv{i}", ref=d[f"mv{i}_y"])
    for i in range(4):
        x, w, sw, b = (d[f"pg{i}_{k}"] for k in ("x", "w", "sw", "bias"))
        gs = int(d[f"pg{i}_gs"])
        y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
        if x.shape[0] == 1:
            assert_mv_close(y, x, w, sw, b, gs, f"golden pg{i}", ref=d[f"pg{i}_y"])
        else:
            assert_bits_equal(y, d[f"pg{i}_y"])
    for i in range(2):
        x, p, sw = (d[f"w4r{i}_{k}"] for k in ("x", "packed", "sw"))
        assert_bits_equal(H(C.w4a8_linear(T(x), T(p), T(sw))), d[f"w4r{i}_y"])
    for i in range(2):
        x, p, sc = (d[f"w4g{i}_{k}"] for k in ("x", "packed", "scale"))
        gs = int(d[f"w4g{i}_gs"])
        assert_bits_equal(H(C.w4a8_pergroup_linear(T(x), T(p), T(sc), gs)), d[f"w4g{i}_y"])


# --------------------------------------------------------------------------
# modules, streams, errors on the device path
# --------------------------------------------------------------------------


def test_cider_linear_from_float_and_convert():
    torch.manual_seed(0)
    lin = torch.nn.Linear(256, 96, bias=True).to(DEV).half()
    for gs in (None, 64):
        layer = C.CiderLinear.from_float(lin, target_group_size=gs)
        x = torch.randn(3, 5, 256, device=DEV, dtype=torch.float16)
        y = layer(x)
        assert y.shape == (3, 5, 96)
        wq = layer.w_int8.cpu().numpy()
        sw = layer.scale_w.cpu().numpy()
        b = layer.bias.cpu().numpy()
        x2 = x.reshape(-1, 256).cpu().numpy()
        exp = (O.perchannel_linear(x2, wq, sw, b) if gs is None
               else O.pergroup_linear(x2, wq, sw, gs, b))
        assert_bits_equal(H(y).reshape(-1, 96), exp)
    model = torch.nn.Sequential(torch.nn.Linear(128, 64), torch.nn.ReLU(),
                                torch.nn.Sequential(torch.nn.Linear(64, 32))).to(DEV)
    w0, b0 = (model[0].weight.detach().float().cpu().numpy(),
              model[0].bias.detach().half().cpu().numpy())
    w1, b1 = (model[2][0].weight.detach().float().cpu().numpy(),
              model[2][0].bias.detach().half().cpu().numpy())
    stats = C.convert_model(model, verbose=False)
    assert stats["n_converted"] == 2
    assert isinstance(model[0], C.CiderLinear) and isinstance(model[2][0], C.CiderLinear)
    # the converted weights are the reference quantizer's, and the converted
    # model's output is the oracle's linear -> ReLU -> linear chain
    q0, s0 = O.quantize_weight_int8(w0)
    q1, s1 = O.quantize_weight_int8(w1)
    assert_bits_equal(model[0].w_int8.cpu().numpy(), q0, "converted w0")
    assert_bits_equal(model[0].scale_w.cpu().numpy(), s0, "converted scale 0")
    assert_bits_equal(model[2][0].w_int8.cpu().numpy(), q1, "converted w1")
    xm = torch.randn(4, 128, device=DEV, dtype=torch.float16)
    out = model(xm)
    assert out.shape == (4, 32)
    y0 = O.perchannel_linear(xm.cpu().numpy(), q0, s0, b0)
    r0 = np.where(y0 > 0, y0, np.float16(0)).astype(np.float16)
    assert_bits_equal(H(out), O.perchannel_linear(r0, q1, s1, b1), "converted model")


def test_w4a8_module():
    K, N = 256, 80
    wf = np.random.default_rng(8).standard_normal((K, N)).astype(np.float32)
    layer = C.W4A8Linear.from_weights(wf, device=DEV)
    x = O.synth_activations(6, K, 81)
    y = H(layer(T(x)))
    packed, sw = O.pack_weight_int4(wf)
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw))


def test_explicit_stream():
    M, N, K = 130, 256, 512
    x, w, sw, b = synth_pc(M, N, K, 5)
    s = torch.cuda.Stream()
    xd, wd, swd, bd = T(x), T(w), T(sw), T(b)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        y = C.perchannel_linear(xd, wd, swd, bd, stream=s)
    s.synchronize()
    assert_bits_equal(y.cpu().numpy(), O.perchannel_linear(x, w, sw, b))


def test_device_errors():
    x = torch.zeros(4, 64, device=DEV, dtype=torch.float16)
    w = torch.zeros(8, 64, device=DEV, dtype=torch.int8)
    s = torch.ones(8, device=DEV)
    with pytest.raises(ValueError):
        C.perchannel_linear(x[0], w, s)
    with pytest.raises(ValueError):
        C.perchannel_linear(x, w[:, :32], s)
    with pytest.raises(ValueError):
        C.pergroup_linear(x, w, torch.ones(1, 8, device=DEV), 100)
    with pytest.raises(ValueError):
        C.pergroup_linear(x, w, torch.ones(8, device=DEV), 64)
    with pytest.raises(RuntimeError):
        C.perchannel_linear(x.cpu(), w.cpu(), s.cpu())
    y = C.perchannel_linear(x[:0], w, s)
    assert tuple(y.shape) == (0, 8)


# 5 <= M <= 16, per-group or int4 weights: the weight-stream kernel
# (skinny_stream.hip).  K=12288 at gs 64 has 192 groups, taken in three
# phases; K=10240 at gs 128 runs 8-wave workgroups; int4 loads pairs of
# k-steps (K % 128 == 0, per-channel and gs 128) or single k-steps (gs 64);
# N=100 / 260 / 36 leave the last 16-row block partly past N.
@pytest.mark.parametrize("M,N,K", [(5, 100, 12288), (16, 260, 10240), (9, 4096, 2560),
                                   (16, 36, 4096), (12, 64, 128)])
def test_stream_small_m_exact(M, N, K):
    x = O.synth_activations(M, K, 120 + M + K)
    w = O.synth_weights_i8(N, K, 121 + N)
    b = (np.random.default_rng(122).standard_normal(N) * 0.1).astype(np.float16)
    for gs in (64, 128, 256):
        if K % gs:
            continue
        sw = O.synth_scales((K // gs, N), 123 + gs)
        y = H(C.pergroup_linear(T(x), T(w), T(sw), gs, T(b)))
        assert_bits_equal(y, O.pergroup_linear(x, w, sw, gs, b), f"stream pg{gs} {M}x{N}x{K}")
    w4 = np.random.default_rng(124).integers(-8, 8, (N, K), dtype=np.int8)
    pk = O.pack_w4_lo_first(w4)
    for gs in (64, 128):
        sc = O.synth_scales((K // gs, N), 125 + gs).astype(np.float16)
        y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs, T(b)))
        assert_bits_equal(y, O.w4a8_pergroup_linear(x, pk, sc, gs, b), f"stream w4g{gs} {M}x{N}x{K}")
    wf = np.random.default_rng(126).standard_normal((K, N)).astype(np.float32)
    packed, sw4 = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw4)))
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw4), f"stream w4 {M}x{N}x{K}")


# 2 <= M <= 16 through the quantizing linears, with rows of special values:
# q and scale_a must be those of the quantize kernel whichever kernel runs
# (the fused decode GEMV at small N, or quantize + GEMV / stream / DMA tiles),
# and the output of a row with inf or NaN is then NaN / +-inf exactly as the
# oracle's.  K=64 leaves 7 of 8 waves of the stream kernel without a k-step;
# N=24 / 264 / 8200 leave the last workgroup partly past N.
@pytest.mark.parametrize("M,N,K", [(2, 24, 64), (3, 40, 128), (7, 264, 320), (16, 4096, 2560),
                                   (16, 12288, 4096), (11, 8200, 4096), (5, 1024, 1024)])
def test_small_m_quantized_exact(M, N, K):
    x = O.synth_activations(M, K, 130 + M + K)
    if M >= 5:
        x[1, :] = 0                                 # s = 1, q = 0
        x[2, :4] = [np.nan, 3.0, -6.0, 0.5]         # NaN ignored by the absmax, q = -128
        x[3, 7] = np.inf                            # s = inf
        x[4, :3] = [65504.0, -65504.0, 1.0]
    w = O.synth_weights_i8(N, K, 131 + N)
    sw = O.synth_scales(N, 132)
    b = (np.random.default_rng(133).standard_normal(N) * 0.1).astype(np.float16)
    for bias in (b, None):
        y = H(C.perchannel_linear(T(x), T(w), T(sw), None if bias is None else T(bias)))
        assert_bits_equal(y, O.perchannel_linear(x, w, sw, bias), f"small-M pc {M}x{N}x{K}")
    for gs in (64, 128):
        if K % gs:
            continue
        swg = O.synth_scales((K // gs, N), 134 + gs)
        y = H(C.pergroup_linear(T(x), T(w), T(swg), gs, T(b)))
        assert_bits_equal(y, O.pergroup_linear(x, w, swg, gs, b), f"small-M pg{gs} {M}x{N}x{K}")
    w4 = np.random.default_rng(135).integers(-8, 8, (N, K), dtype=np.int8)
    pk = O.pack_w4_lo_first(w4)
    for gs in (64, 128):
        if K % gs:
            continue
        sc = O.synth_scales((K // gs, N), 136 + gs).astype(np.float16)
        for bias in (b, None):
            y = H(C.w4a8_pergroup_linear(T(x), T(pk), T(sc), gs,
                                         None if bias is None else T(bias)))
            assert_bits_equal(y, O.w4a8_pergroup_linear(x, pk, sc, gs, bias),
                              f"small-M w4g{gs} {M}x{N}x{K}")
    wf = np.random.default_rng(137).standard_normal((K, N)).astype(np.float32)
    packed, sw4 = O.pack_weight_int4(wf)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw4)))
    assert_bits_equal(y, O.w4a8_linear(x, packed, sw4), f"small-M w4 {M}x{N}x{K}")

"""CPU oracle for cider's fused quantize -> int8 GEMM -> dequant linear.

TEST INFRASTRUCTURE ONLY.  This module is the checker: it is imported by
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` and by nothing else.  The product package (``cider_amd``) never
imports it, links it or falls back to it.

Every function restates, in numpy, the arithmetic of one reference kernel or
helper and cites the reference file:line it follows (paths relative to the
reference checkout root).  The order of floating-point operations is the
one written in the reference source, evaluated left to right in IEEE binary32
with round-to-nearest-even and no fused multiply-add:

* ``f32(.)``  - IEEE binary32 RNE (numpy float32 ufuncs round every op);
* ``h(.)``    - binary32 -> binary16 RNE (numpy ``astype(np.float16)``);
* ``rha(.)``  - round half away from zero (Metal ``round``).

Integer dot products are exact: they run as float64 BLAS products, which
cannot round while every partial sum stays below 2**53 (true for
K < 2**39 int8 x int8 terms), and are then wrapped to int32 the way the
reference's own bit-exact test wraps its int64 result
(``benchmarks/test_bitexact.py:55``).

Behaviour the reference leaves undefined is fixed here and used by the HIP
kernels identically:

* NaN inputs are ignored by the row absmax (Metal ``max`` is ``fmax``);
  a NaN product quantizes to -128 (``fmin(fmax(v, -128), 127)``).
* The MV kernels have no K tail in the reference (K % 256 == 0 at every
  reference call); the oracle treats missing tail elements as zeros.
* ``simd_sum`` over the 32 lanes of an MV row is an xor butterfly
  (offsets 16, 8, 4, 2, 1).  Metal does not specify its tree; the MV
  parity bar is therefore a tolerance, not bit equality.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------


def rha(v: np.ndarray) -> np.ndarray:
    """Round half away from zero of float32 values (Metal ``round``).

    Computed in float64, where ``|v| + 0.5`` is exact for every float32
    ``|v| < 2**29``, so no double rounding can move a value across .5.
    Returns float64 with NaN preserved.
    """
    v64 = np.asarray(v, dtype=np.float64)
    return np.copysign(np.floor(np.abs(v64) + 0.5), v64)


def clamp_i8(v: np.ndarray) -> np.ndarray:
    """``fmin(fmax(v, -128), 127)`` then int8; NaN -> -128.

    Follows ``clamp(round(v), -128.0f, 127.0f)`` in
    ``cider/kernels/w8a8_quantize.metal:84``.
    """
    v = np.asarray(v, dtype=np.float64)
    out = np.clip(v, -128.0, 127.0)
    out = np.where(np.isnan(v), -128.0, out)
    return out.astype(np.int8)


def int_dot_nt(a: np.ndarray, b_nk: np.ndarray) -> np.ndarray:
    """Exact ``a @ b_nk.T`` for integer matrices, wrapped to int32.

    a: [M, K] integer, b_nk: [N, K] integer.  float64 BLAS is exact here
    (all partial sums are integers below 2**53).
    """
    a64 = np.asarray(a, dtype=np.float64)
    b64 = np.asarray(b_nk, dtype=np.float64)
    if a64.shape[1] != b64.shape[1]:
        raise ValueError("K mismatch")
    if a64.shape[1] >= (1 << 39):
        raise ValueError("K too large for the exact float64 product")
    c = a64 @ b64.T
    return c.astype(np.int64).astype(np.int32)


# ---------------------------------------------------------------------------
# a1: per-token activation quantization
# ---------------------------------------------------------------------------


def quantize_per_token(x: np.ndarray):
    """Per-token symmetric int8 quantization.

    Follows ``cider/kernels/w8a8_quantize.metal:33-86``:
    ``amax = max_k |x|`` (:34-38, 55-61), ``s = amax / 127`` with
    ``s == 0 -> 1`` (:64-67), ``inv = 1 / s`` (:71), then
    ``q = clamp(round(x * inv), -128, 127)`` (:82-85).

    x: [M, K] float16.  Returns (q int8 [M, K], sa float32 [M]).
    """
    x = np.asarray(x)
    if x.dtype != np.float16:
        raise TypeError("quantize_per_token expects float16 input")
    xf = x.astype(F32)
    if xf.shape[1] == 0:
        amax = np.zeros(xf.shape[0], dtype=F32)
    else:
        # fmax semantics: NaN never wins the max (all-NaN row -> NaN).
        amax = np.fmax.reduce(np.abs(xf), axis=1).astype(F32)
        amax = np.where(np.isnan(amax), F32(0.0), amax).astype(F32)
    s = (amax / F32(127.0)).astype(F32)
    s = np.where(s == F32(0.0), F32(1.0), s).astype(F32)
    inv = (F32(1.0) / s).astype(F32)
    v = (xf * inv[:, None]).astype(F32)
    q = clamp_i8(rha(v))
    return q, s


# ---------------------------------------------------------------------------
# a3: raw int8 x int8 -> int32
# ---------------------------------------------------------------------------


def int8_matmul_int32(a: np.ndarray, b_nk: np.ndarray) -> np.ndarray:
    """``C = A @ B^T`` in int32, B given as [N, K].

    Follows ``cider/kernels/w8a8_matmul.metal:301-453`` and the reference
    test's expected value ``benchmarks/test_bitexact.py:55``.
    """
    return int_dot_nt(np.asarray(a, np.int8), np.asarray(b_nk, np.int8))


# ---------------------------------------------------------------------------
# a2: per-channel epilogue and linear
# ---------------------------------------------------------------------------


def dequant_perchannel(acc: np.ndarray, sa: np.ndarray, sw: np.ndarray,
                       bias: np.ndarray | None) -> np.ndarray:
    """``h( f32(f32(f32(acc) * sa[m]) * sw[n]) + f32(bias[n]) )``.

    Follows ``cider/kernels/w8a8_matmul.metal:74-77`` (bias present) and
    ``cider/kernels/w4a8_matmul.metal:83`` (``bias is None``: no add).
    """
    accf = np.asarray(acc, dtype=np.int32).astype(F32)
    v = (accf * np.asarray(sa, F32)[:, None]).astype(F32)
    v = (v * np.asarray(sw, F32)[None, :]).astype(F32)
    if bias is not None:
        v = (v + np.asarray(bias, np.float16).astype(F32)[None, :]).astype(F32)
    return v.astype(np.float16)


def mv_perchannel(x: np.ndarray, w: np.ndarray, sw: np.ndarray,
                  bias: np.ndarray) -> np.ndarray:
    """M == 1 decode: fp16 activation x int8 weight, no activation quant.

    Follows ``cider/kernels/w8a8_int8_mv.metal:26-70``: lane ``l`` of 32
    owns elements ``256 b + 8 l + i`` (i < 8) of each 256-wide block ``b``;
    ``dot`` is the sequential sum of the 8 exact products (:46-49),
    ``result += dot`` per block (:50), ``simd_sum`` over lanes (:58) and
    ``y = h(f32(sw * R) + f32(bias))`` (:66-67).

    x: [1, K] or [K] float16, w: [N, K] int8 -> [1, N] float16.
    """
    xv = np.asarray(x, np.float16).reshape(-1).astype(F32)
    w = np.asarray(w, np.int8)
    N, K = w.shape
    nb = (K + 255) // 256
    kp = nb * 256
    xp = np.zeros(kp, F32)
    xp[:K] = xv
    wp = np.zeros((N, kp), F32)
    wp[:, :K] = w.astype(F32)
    prod = (wp * xp[None, :]).astype(F32).reshape(N, nb, 32, 8)  # exact
    d = prod[..., 0]
    for i in range(1, 8):
        d = (d + prod[..., i]).astype(F32)
    r = np.zeros((N, 32), F32)
    for b in range(nb):
        r = (r + d[:, b, :]).astype(F32)
    R = _butterfly_sum(r)
    y = (np.asarray(sw, F32) * R).astype(F32)
    y = (y + np.asarray(bias, np.float16).astype(F32)).astype(F32)
    return y.astype(np.float16)[None, :]


def _butterfly_sum(r: np.ndarray) -> np.ndarray:
    """Sum over the last axis (32 lanes) by an xor butterfly; lane 0 result."""
    lanes = np.arange(r.shape[-1])
    v = r.astype(F32)
    off = r.shape[-1] // 2
    while off >= 1:
        v = (v + v[..., lanes ^ off]).astype(F32)
        off //= 2
    return v[..., 0]


def perchannel_linear(x: np.ndarray, w: np.ndarray, sw: np.ndarray,
                      bias: np.ndarray | None = None) -> np.ndarray:
    """Per-channel W8A8 linear with the reference's dispatch.

    Follows ``csrc/src/w8a8_primitive.mm:157-251``: M == 1 takes the fp16
    MV; otherwise quantize (a1) then int GEMM with the fused per-channel
    epilogue (a2).  A missing bias is zeros fp16 (``cider/ops.py:143-144``).
    """
    x = np.asarray(x, np.float16)
    w = np.asarray(w, np.int8)
    N = w.shape[0]
    if bias is None:
        bias = np.zeros(N, np.float16)
    if x.shape[0] == 1:
        return mv_perchannel(x, w, sw, bias)
    q, sa = quantize_per_token(x)
    acc = int_dot_nt(q, w)
    return dequant_perchannel(acc, sa, sw, bias)


# ---------------------------------------------------------------------------
# a5 / a6: per-group
# ---------------------------------------------------------------------------


def pergroup_gemm(q: np.ndarray, sa: np.ndarray, w: np.ndarray,
                  sw_gn: np.ndarray, bias: np.ndarray | None,
                  group_size: int) -> np.ndarray:
    """Per-group GEMM with in-register fp32 flush.

    Follows ``cider/kernels/pergroup_int8_gemm.metal:90-191``: int32
    ``D_g`` over each group's K slice (:99-150), ``acc += f32(D_g) * sw[g, n]``
    sequentially in g (:154-168), then ``h(f32(acc * sa[m]) + f32(bias[n]))``
    (:184-186).  sw_gn is [G, N] (``cider/ops.py:184,204``).
    """
    M, K = q.shape
    N = w.shape[0]
    if K % group_size:
        raise ValueError("K must be a multiple of group_size")
    G = K // group_size
    sw_gn = np.asarray(sw_gn, F32).reshape(G, N)
    acc = np.zeros((M, N), F32)
    for g in range(G):
        sl = slice(g * group_size, (g + 1) * group_size)
        dg = int_dot_nt(q[:, sl], w[:, sl]).astype(F32)
        acc = (acc + (dg * sw_gn[g][None, :]).astype(F32)).astype(F32)
    v = (acc * np.asarray(sa, F32)[:, None]).astype(F32)
    if bias is not None:
        v = (v + np.asarray(bias, np.float16).astype(F32)[None, :]).astype(F32)
    return v.astype(np.float16)


def mv_pergroup(x: np.ndarray, w: np.ndarray, sw_gn: np.ndarray,
                bias: np.ndarray, group_size: int) -> np.ndarray:
    """M == 1 per-group decode MV (fp16 activation).

    Follows ``cider/kernels/pergroup_int8_mv.metal:22-106``: per lane and
    block, ``g = (256 b + 8 l) / gs`` (:58), ``dot`` over 8 exact products
    left to right (:77-78), ``result += f32(sw[g, n] * dot)`` (:81-82),
    ``simd_sum`` (:94) and ``y = h(f32(R + f32(bias)))`` (:102).
    """
    xv = np.asarray(x, np.float16).reshape(-1).astype(F32)
    w = np.asarray(w, np.int8)
    N, K = w.shape
    G = K // group_size
    sw_gn = np.asarray(sw_gn, F32).reshape(G, N)
    nb = (K + 255) // 256
    kp = nb * 256
    xp = np.zeros(kp, F32)
    xp[:K] = xv
    wp = np.zeros((N, kp), F32)
    wp[:, :K] = w.astype(F32)
    prod = (wp * xp[None, :]).astype(F32).reshape(N, nb, 32, 8)
    d = prod[..., 0]
    for i in range(1, 8):
        d = (d + prod[..., i]).astype(F32)
    lane_k = (np.arange(nb)[:, None] * 256 + np.arange(32)[None, :] * 8)
    gidx = np.minimum(lane_k // group_size, G - 1)            # [nb, 32]
    swb = sw_gn[gidx]                                          # [nb, 32, N]
    swb = np.moveaxis(swb, -1, 0)                              # [N, nb, 32]
    r = np.zeros((N, 32), F32)
    for b in range(nb):
        r = (r + (swb[:, b, :] * d[:, b, :]).astype(F32)).astype(F32)
    R = _butterfly_sum(r)
    y = (R + np.asarray(bias, np.float16).astype(F32)).astype(F32)
    return y.astype(np.float16)[None, :]


def pergroup_linear(x: np.ndarray, w: np.ndarray, sw_gn: np.ndarray,
                    group_size: int, bias: np.ndarray | None = None):
    """Per-group linear with the reference dispatch.

    Follows ``csrc/src/pergroup_primitive.mm:159-276`` (M == 1 -> MV,
    else quantize + per-group GEMM) and ``cider/ops.py:195-196`` (zero bias).
    """
    x = np.asarray(x, np.float16)
    w = np.asarray(w, np.int8)
    if group_size not in (64, 128, 256):
        raise ValueError("group_size must be 64, 128 or 256")
    N = w.shape[0]
    if bias is None:
        bias = np.zeros(N, np.float16)
    if x.shape[0] == 1:
        return mv_pergroup(x, w, sw_gn, bias, group_size)
    q, sa = quantize_per_token(x)
    return pergroup_gemm(q, sa, w, sw_gn, bias, group_size)


# ---------------------------------------------------------------------------
# a7: W4A8 (reference layout) and the per-group extension
# ---------------------------------------------------------------------------


def unpack_w4_ref(packed_kn: np.ndarray) -> np.ndarray:
    """Reference W4 layout -> int8 [K, N].

    ``packed[K/2, N]``, high nibble = even k, low nibble = odd k, value =
    nibble - 8.  Follows ``cider/kernels/w4a8_matmul.metal:47-70,216-219``
    and ``cider/ops.py:114-115``.
    """
    p = np.asarray(packed_kn, np.uint8)
    hi = (p >> 4).astype(np.int16) - 8
    lo = (p & 0xF).astype(np.int16) - 8
    K2, N = p.shape
    out = np.empty((2 * K2, N), np.int8)
    out[0::2] = hi
    out[1::2] = lo
    return out


def w4a8_linear(x: np.ndarray, packed_kn: np.ndarray, sw: np.ndarray):
    """W4A8 linear, reference layout, per-column fp32 scale, no bias.

    Follows ``csrc/src/w4a8_primitive.mm:175-264`` (always quantize + GEMM,
    M == 1 included) and ``cider/kernels/w4a8_matmul.metal:83``
    (``h(f32(f32(acc) * sa) * sw)``).
    """
    x = np.asarray(x, np.float16)
    q, sa = quantize_per_token(x)
    w_kn = unpack_w4_ref(packed_kn)
    acc = int_dot_nt(q, w_kn.T)
    return dequant_perchannel(acc, sa, sw, None)


def unpack_w4_lo_first(packed_nk: np.ndarray) -> np.ndarray:
    """Per-group W4 extension layout -> int8 [N, K].

    ``packed[N, K/2]``: byte ``k >> 1`` of row n holds element k in its low
    nibble when k is even and in its high nibble when k is odd; each nibble
    is a two's-complement int4 in [-8, 7].  No reference kernel uses this
    layout; it is the layout of the W4A8 per-group benchmark configuration.
    """
    p = np.asarray(packed_nk, np.uint8)
    lo = (p & 0xF).astype(np.int16)
    hi = (p >> 4).astype(np.int16)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    N, K2 = p.shape
    out = np.empty((N, 2 * K2), np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def pack_w4_lo_first(w_nk: np.ndarray) -> np.ndarray:
    """Inverse of :func:`unpack_w4_lo_first` (int8 in [-8, 7], K even)."""
    w = np.asarray(w_nk, np.int16)
    if w.shape[1] % 2:
        raise ValueError("K must be even")
    if w.min(initial=0) < -8 or w.max(initial=0) > 7:
        raise ValueError("int4 values must lie in [-8, 7]")
    nib = (w & 0xF).astype(np.uint8)
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)


def w4a8_pergroup_linear(x: np.ndarray, packed_nk: np.ndarray,
                         scale_gn_f16: np.ndarray, group_size: int,
                         bias: np.ndarray | None = None) -> np.ndarray:
    """W4A8 per-group extension: A5's group flush over int4 weights.

    ``acc = sum_g f32(f32(D_g) * f32(scale[g, n]))`` sequentially in g,
    ``y = h(f32(acc * sa) [+ f32(bias)])``.  This is the natural
    generalization of ``cider/kernels/pergroup_int8_gemm.metal:152-189`` to
    int4 weights and fp16 scales; no reference kernel pins it (the
    reference has no per-group W4), so its parity rests on the checks in
    ``tests/test_oracle.py``.
    """
    x = np.asarray(x, np.float16)
    q, sa = quantize_per_token(x)
    w = unpack_w4_lo_first(packed_nk)
    sw = np.asarray(scale_gn_f16, np.float16).astype(F32)
    return pergroup_gemm(q, sa, w, sw, bias, group_size)


# ---------------------------------------------------------------------------
# a14: offline weight quantizers (host side in the reference too)
# ---------------------------------------------------------------------------


def quantize_weight_int8(w: np.ndarray):
    """Per-row symmetric int8: ``cider/ops.py:73-90`` (np.round = half-even)."""
    w = np.asarray(w).astype(np.float32)
    row_max = np.max(np.abs(w), axis=1)
    scale = row_max / np.float32(127.0)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    q = np.clip(np.round(w / scale[:, None]), -128, 127).astype(np.int8)
    return q, scale


def quantize_weight_pergroup(w: np.ndarray, group_size: int):
    """Per-group symmetric int8: ``cider/nn.py:34-59``.

    Returns (q int8 [N, K], scale float32 [N, G]); callers transpose the
    scale to [G, N] (``cider/nn.py:166,187``).
    """
    w = np.asarray(w).astype(np.float32)
    N, K = w.shape
    if K % group_size:
        raise ValueError("K not divisible by group_size")
    G = K // group_size
    wr = w.reshape(N, G, group_size)
    gmax = np.max(np.abs(wr), axis=2)
    scale = gmax / np.float32(127.0)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    q = np.clip(np.round(wr / scale[:, :, None]), -128, 127)
    return q.astype(np.int8).reshape(N, K), scale


def pack_weight_int4(w: np.ndarray, zero_point: int = 8):
    """Per-column W4 quantize + pack, reference layout: ``cider/ops.py:93-116``.

    w: [K, N] float -> (packed uint8 [K/2, N], scale float32 [N]).
    """
    K, N = w.shape
    if K % 2:
        raise ValueError("K must be even")
    w = np.asarray(w).astype(np.float32)
    col_max = np.max(np.abs(w), axis=0)
    scale = col_max / np.float32(7.0)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    wq = np.clip(np.round(w / scale[None, :]) + zero_point, 0, 15).astype(np.uint8)
    packed = (wq[0::2, :] << 4) | wq[1::2, :]
    return packed.astype(np.uint8), scale


# ---------------------------------------------------------------------------
# synthetic inputs of the benchmark configurations
# ---------------------------------------------------------------------------


def synth_activations(M: int, K: int, seed: int) -> np.ndarray:
    """X fp16 ~ N(0, 1) with K // 100 columns scaled x20 (outlier channels)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    n_out = K // 100
    if n_out:
        cols = rng.choice(K, size=n_out, replace=False)
        x[:, cols] *= np.float32(20.0)
    return x.astype(np.float16)


def synth_weights_i8(N: int, K: int, seed: int) -> np.ndarray:
    """W int8 uniform in [-127, 127]."""
    rng = np.random.default_rng(seed)
    return rng.integers(-127, 128, size=(N, K), dtype=np.int8)


def synth_scales(shape, seed: int) -> np.ndarray:
    """fp32 scales uniform in [1e-3, 1e-2]."""
    rng = np.random.default_rng(seed)
    return rng.uniform(1e-3, 1e-2, size=shape).astype(np.float32)

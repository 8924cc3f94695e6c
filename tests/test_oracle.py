"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against something other than its own
formula: the reference's golden vectors (``benchmarks/test_bitexact.py``),
textbook routines (int64 matmul, brute force loops), an exact-rational model
of IEEE rounding (``tests/exact_fp.py``), invariants, and known-answer cases
chosen so that a plausible mistake (half-even instead of half-away rounding,
division instead of reciprocal multiply, a different fp32 association or a
fused multiply-add, a swapped nibble) fails.  The C restatement is checked
against the numpy one on the same inputs.
"""

import hashlib
from fractions import Fraction

import numpy as np
import pytest

from oracle import cider_oracle as O
from oracle import c_oracle as C
from tests import exact_fp as X
from tests.golden.make_golden import bitexact_inputs
from tests.util import f16_ulp

F32 = np.float32


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# --------------------------------------------------------------------------
# a3: the reference's own golden vectors
# --------------------------------------------------------------------------


def test_bitexact_golden_vectors(bitexact_shapes):
    """All 14 shapes of benchmarks/test_bitexact.py:19-35, bit for bit."""
    assert len(bitexact_shapes) == 14
    for rec in bitexact_shapes:
        a, b = bitexact_inputs(rec["M"], rec["K"], rec["N"])
        assert sha(a) == rec["sha_a"] and sha(b) == rec["sha_b"], "legacy RNG drifted"
        c = O.int8_matmul_int32(a, b)
        assert c.dtype == np.int32 and c.shape == (rec["M"], rec["N"])
        assert sha(c) == rec["sha_c"], rec
        if "c" in rec:
            np.testing.assert_array_equal(c, np.array(rec["c"], np.int32))


def test_int_gemm_brute_force():
    rng = np.random.default_rng(1)
    for M, N, K in [(1, 1, 1), (3, 4, 5), (2, 7, 33)]:
        a = rng.integers(-128, 128, (M, K), dtype=np.int8)
        b = rng.integers(-128, 128, (N, K), dtype=np.int8)
        ref = [[sum(int(a[m, k]) * int(b[n, k]) for k in range(K)) for n in range(N)]
               for m in range(M)]
        np.testing.assert_array_equal(O.int8_matmul_int32(a, b), np.array(ref, np.int32))


def test_int_gemm_extremes():
    # -128 * -128 * K is the largest accumulator; must stay exact
    K = 4097
    a = np.full((2, K), -128, np.int8)
    b = np.full((3, K), -128, np.int8)
    assert (O.int8_matmul_int32(a, b) == 16384 * K).all()
    b[1] = 127
    assert O.int8_matmul_int32(a, b)[0, 1] == -128 * 127 * K


# --------------------------------------------------------------------------
# a1: quantize
# --------------------------------------------------------------------------


def _exact_quant_row(xrow):
    xs = [Fraction(float(v)) for v in xrow.astype(np.float32)]
    amax = max(abs(v) for v in xs)
    s = X.f32(amax / 127)
    if s == 0:
        s = Fraction(1)
    inv = X.f32(1 / s)
    q = [max(-128, min(127, X.rha(X.f32(v * inv)))) for v in xs]
    return q, s


def test_quantize_exact_model():
    x = O.synth_activations(12, 96, 7)
    x[3] = 0
    q, sa = O.quantize_per_token(x)
    for m in range(x.shape[0]):
        qe, se = _exact_quant_row(x[m])
        assert Fraction(float(sa[m])) == se
        assert q[m].tolist() == qe


def test_quantize_ties_round_half_away():
    # amax 127 -> s = 1, inv = 1: x * inv is x itself, ties are exact .5
    x = np.array([[127, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5]], np.float16)
    q, sa = O.quantize_per_token(x)
    assert sa[0] == 1.0
    assert q[0].tolist() == [127, 3, -3, 1, -1, 2, -127]  # half-even would give 2,-2,0,0


def test_quantize_reciprocal_not_division():
    # x * fl(1/s) = 63.499996 -> 63, while x / s = 63.5 -> 64
    x = np.array([[33.9, 16.95]], np.float16)
    q, _ = O.quantize_per_token(x)
    assert q[0, 1] == 63
    qe, _ = _exact_quant_row(x[0])
    assert qe[1] == 63


def test_quantize_invariants():
    x = O.synth_activations(32, 300, 11)
    x[5] = 0
    q, sa = O.quantize_per_token(x)
    assert sa[5] == 1.0 and (q[5] == 0).all()          # zero row -> s = 1
    assert np.abs(q.astype(np.int32)).max() <= 127      # never -128 for finite x
    am = np.argmax(np.abs(x.astype(np.float32)), axis=1)
    for m in range(32):
        if m != 5:
            assert abs(int(q[m, am[m]])) == 127
    # scale equivariance under powers of two (fp16 exact)
    x4 = (x.astype(np.float32) / 4).astype(np.float16)
    assert (x4.astype(np.float32) * 4 == x.astype(np.float32)).all()
    q4, sa4 = O.quantize_per_token(x4)
    np.testing.assert_array_equal(q4[np.arange(32) != 5], q[np.arange(32) != 5])
    np.testing.assert_array_equal(sa4[np.arange(32) != 5] * 4, sa[np.arange(32) != 5])


def test_quantize_nonfinite_defined():
    x = np.array([[np.nan, 1.0, -2.0], [np.inf, 1.0, 0.0]], np.float16)
    q, sa = O.quantize_per_token(x)
    assert sa[0] == np.float32(2.0) / np.float32(127.0)
    assert q[0].tolist() == [-128, 64, -127]
    assert np.isinf(sa[1])
    assert q[1].tolist() == [-128, 0, 0]


# --------------------------------------------------------------------------
# a2: per-channel epilogue
# --------------------------------------------------------------------------


def _exact_pc(acc, sa, sw, bias):
    v = X.f32(Fraction(int(acc)))
    v = X.f32(v * Fraction(float(sa)))
    v = X.f32(v * Fraction(float(sw)))
    if bias is not None:
        v = X.f32(v + Fraction(float(bias)))
    return X.f16(v)


def test_perchannel_epilogue_exact_model():
    rng = np.random.default_rng(3)
    M, N = 6, 40
    acc = rng.integers(-(1 << 26), 1 << 26, (M, N)).astype(np.int32)   # > 2^24: inexact cast
    sa = rng.uniform(1e-4, 1e-1, M).astype(F32)
    sw = rng.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (rng.standard_normal(N) * 3).astype(np.float16)
    y = O.dequant_perchannel(acc, sa, sw, bias)
    for m in range(M):
        for n in range(N):
            assert Fraction(float(y[m, n])) == _exact_pc(acc[m, n], sa[m], sw[n], bias[n]), (m, n)


# (acc, sa, sw, bias, y): the reference order ((acc*sa)*sw)+bias; the
# association acc*(sa*sw) or a fused final multiply-add gives another fp16.
EPILOGUE_KATS = [
    (61931469, 0.03303958, 0.004302384, 0.507, 8808.0),
    (63957425, 0.09057191, 0.0062665623, 3.4, 36288.0),
    (44281141, 0.015257112, 0.009841958, 4.75, 6652.0),
    (21671822, 0.0964681, 0.007847651, 1.39, 16416.0),
    (58364924, 0.09889701, 0.009920192, 3.494, 57280.0),
]


def test_perchannel_epilogue_kats_order_and_no_fma():
    for acc, sa, sw, b, yexp in EPILOGUE_KATS:
        sa, sw, b = F32(sa), F32(sw), np.float16(b)
        y = O.dequant_perchannel(np.array([[acc]], np.int32), np.array([sa]), np.array([sw]),
                                 np.array([b]))
        assert float(y[0, 0]) == yexp
        assert Fraction(yexp) == _exact_pc(acc, sa, sw, b)
        alt = X.f16(X.f32(X.f32(X.f32(Fraction(acc)) * X.f32(Fraction(float(sa)) * Fraction(float(sw))))
                          + Fraction(float(b))))
        fused = X.f16(X.f32(X.f32(X.f32(Fraction(acc)) * Fraction(float(sa))) * Fraction(float(sw))
                            + Fraction(float(b))))
        assert alt != Fraction(yexp) or fused != Fraction(yexp)


def test_perchannel_epilogue_special_cases():
    acc = np.array([[0, 1, -1, 2048, 70000, -70000]], np.int32)
    ones_a = np.ones(1, F32)
    ones_w = np.ones(6, F32)
    y = O.dequant_perchannel(acc, ones_a, ones_w, np.zeros(6, np.float16))
    np.testing.assert_array_equal(y, acc.astype(np.float64).astype(np.float16))
    assert np.isinf(y[0, 4]) and np.isinf(y[0, 5])
    # acc = 0: y == bias; sign of zero: -0 * s + 0 -> +0, no bias keeps -0
    bias = np.array([1.5, -2.0, 0.0, 0.0, 0.0, 0.0], np.float16)
    acc0 = np.zeros((1, 6), np.int32)
    np.testing.assert_array_equal(O.dequant_perchannel(acc0, ones_a, ones_w, bias)[0], bias)
    neg = O.dequant_perchannel(np.array([[-1]], np.int32), np.array([1e-30], F32),
                               np.array([1e-30], F32), None)
    assert np.signbit(neg[0, 0]) and neg[0, 0] == 0


def test_perchannel_linear_gemm_path_composes():
    x = O.synth_activations(9, 160, 21)
    w = O.synth_weights_i8(50, 160, 22)
    sw = O.synth_scales(50, 23)
    y = O.perchannel_linear(x, w, sw)
    q, sa = O.quantize_per_token(x)
    acc = (q.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
    np.testing.assert_array_equal(y, O.dequant_perchannel(acc, sa, sw, np.zeros(50, np.float16)))
    # and within the activation-quantization error bound of the float product:
    # |x - q*sa| <= sa/2 per element, so |err| <= sa/2 * sum_k |w*sw| (+ fp16 ulp)
    ref = x.astype(np.float64) @ (w.astype(np.float64) * sw[:, None]).T
    err = np.abs(y.astype(np.float64) - ref)
    bound = (sa[:, None].astype(np.float64) / 2) * (np.abs(w).sum(1) * sw)[None, :]
    bound += np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (err <= bound * 1.0001).all()


# --------------------------------------------------------------------------
# a4: M == 1 MV
# --------------------------------------------------------------------------


def _exact_mv_row(xr, wr, sw, bias):
    K = len(xr)
    nb = (K + 255) // 256
    r = [Fraction(0)] * 32
    for b in range(nb):
        for l in range(32):
            d = None
            for i in range(8):
                k = 256 * b + 8 * l + i
                p = Fraction(int(wr[k])) * Fraction(float(xr[k])) if k < K else Fraction(0)
                d = p if d is None else X.f32(d + p)
            r[l] = X.f32(r[l] + d)
    off = 16
    while off:
        r = [X.f32(r[l] + r[l ^ off]) for l in range(32)]
        off //= 2
    v = X.f32(Fraction(float(sw)) * r[0])
    return X.f16(X.f32(v + Fraction(float(bias))))


def test_mv_exact_model_and_closed_form():
    x = O.synth_activations(1, 512, 31)
    w = O.synth_weights_i8(6, 512, 32)
    sw = O.synth_scales(6, 33)
    bias = np.array([0, 0.5, -1, 0, 0, 2], np.float16)
    y = O.mv_perchannel(x, w, sw, bias)
    for n in range(6):
        assert Fraction(float(y[0, n])) == _exact_mv_row(x[0], w[n], sw[n], bias[n])
    # closed form: the exact dot in float64, within one fp16 ulp + fp32 sum error
    ref = sw * (w.astype(np.float64) @ x[0].astype(np.float64)) + bias.astype(np.float64)
    tol = np.maximum(np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64), 1e-6)
    assert (np.abs(y[0].astype(np.float64) - ref) <= tol).all()


def test_mv_dispatch_only_at_m1():
    x = O.synth_activations(2, 256, 41)
    w = O.synth_weights_i8(8, 256, 42)
    sw = O.synth_scales(8, 43)
    y2 = O.perchannel_linear(x, w, sw)
    y1 = O.perchannel_linear(x[:1], w, sw)
    np.testing.assert_array_equal(y1, O.mv_perchannel(x[:1], w, sw, np.zeros(8, np.float16)))
    q, sa = O.quantize_per_token(x)
    np.testing.assert_array_equal(y2, O.dequant_perchannel(O.int8_matmul_int32(q, w), sa, sw,
                                                           np.zeros(8, np.float16)))


# --------------------------------------------------------------------------
# a5 / a6: per-group
# --------------------------------------------------------------------------


def test_pergroup_exact_model():
    rng = np.random.default_rng(5)
    M, N, K, gs = 3, 5, 256, 64
    x = O.synth_activations(M, K, 51)
    w = O.synth_weights_i8(N, K, 52)
    sw = rng.uniform(1e-3, 1e-2, (K // gs, N)).astype(F32)
    bias = (rng.standard_normal(N)).astype(np.float16)
    y = O.pergroup_linear(x, w, sw, gs, bias)
    q, sa = O.quantize_per_token(x)
    for m in range(M):
        for n in range(N):
            acc = Fraction(0)
            for g in range(K // gs):
                d = int(np.dot(q[m, g * gs:(g + 1) * gs].astype(np.int64),
                               w[n, g * gs:(g + 1) * gs].astype(np.int64)))
                acc = X.f32(acc + X.f32(Fraction(d) * Fraction(float(sw[g, n]))))
            v = X.f16(X.f32(X.f32(acc * Fraction(float(sa[m]))) + Fraction(float(bias[n]))))
            assert Fraction(float(y[m, n])) == v


def test_pergroup_sequential_group_order():
    # D_g * sw_g = 2^24, 1, 1, -2^24: sequential fp32 gives 0, the reverse
    # order gives 2 and a pairwise tree gives 1
    gs = 64
    q = np.zeros((1, 4 * gs), np.int8)
    w = np.zeros((1, 4 * gs), np.int8)
    for g, d in enumerate([1, 1, 1, -1]):
        q[0, g * gs], w[0, g * gs] = 1, d
    sw = np.array([[2.0 ** 24], [1.0], [1.0], [2.0 ** 24]], F32)
    y = O.pergroup_gemm(q, np.ones(1, F32), w, sw, None, gs)
    assert y[0, 0] == 0.0
    rev = lambda a: a.reshape(1, 4, gs)[:, ::-1].reshape(1, 4 * gs).copy()
    y_rev = O.pergroup_gemm(rev(q), np.ones(1, F32), rev(w), sw[::-1].copy(), None, gs)
    assert y_rev[0, 0] == 2.0


def test_pergroup_mv_exact_model():
    x = O.synth_activations(1, 512, 61)
    w = O.synth_weights_i8(4, 512, 62)
    for gs in (64, 128, 256):
        sw = O.synth_scales((512 // gs, 4), 63)
        bias = np.array([0.25, 0, -1, 3], np.float16)
        y = O.mv_pergroup(x, w, sw, bias, gs)
        for n in range(4):
            r = [Fraction(0)] * 32
            for b in range(2):
                for l in range(32):
                    d = None
                    for i in range(8):
                        k = 256 * b + 8 * l + i
                        p = Fraction(int(w[n, k])) * Fraction(float(x[0, k]))
                        d = p if d is None else X.f32(d + p)
                    g = (256 * b + 8 * l) // gs
                    r[l] = X.f32(r[l] + X.f32(Fraction(float(sw[g, n])) * d))
            off = 16
            while off:
                r = [X.f32(r[l] + r[l ^ off]) for l in range(32)]
                off //= 2
            assert Fraction(float(y[0, n])) == X.f16(X.f32(r[0] + Fraction(float(bias[n]))))


def _pg_mv_closed_form(x, w, sw_gn, bias, gs):
    """float64 value of sum_g sw[g,n] * sum_{k in g} w[n,k] x[k] + bias[n] and
    sum of |terms|, straight from the definition (no lanes, no blocks)."""
    K = w.shape[1]
    G = K // gs
    xv = x.reshape(-1).astype(np.float64)
    prod = w.astype(np.float64) * xv[None, :]                          # [N, K]
    dg = prod.reshape(w.shape[0], G, gs).sum(axis=2)                   # [N, G]
    ag = np.abs(prod).reshape(w.shape[0], G, gs).sum(axis=2)
    sw = sw_gn.astype(np.float64).T                                    # [N, G]
    return (sw * dg).sum(axis=1) + bias.astype(np.float64), (np.abs(sw) * ag).sum(axis=1)


@pytest.mark.parametrize("gs", [64, 128, 256])
def test_pergroup_mv_closed_form_and_layout_kats(gs):
    """mv_pergroup against the float64 definition with a derived fp32 bound.

    Every term w*x is exact in fp32 (8-bit by 11-bit significands); a term
    then passes through at most 7 in-chunk adds, one scale multiply, nb block
    adds, 5 butterfly adds and the bias add, so the fp32 result is within
    gamma_(14+nb) * sum|sw*w*x| (+ u*|bias|) of the exact value (Higham,
    Accuracy and Stability, 2nd ed., Lemma 3.1 and section 4.2), and the fp16
    output within half an fp16 ulp of that.  The scales span 2^-16 .. 2^-3
    across groups and columns, so reading them transposed ([N, G]) or with a
    wrong group index (the block's group, or the lane's offset without the
    block's) moves outputs by orders of magnitude more than the bound."""
    rng = np.random.default_rng(gs)
    N, K = 24, 1024
    G = K // gs
    x = rng.standard_normal((1, K)).astype(np.float16)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sw = np.ldexp(1.0, rng.integers(-16, -3, (G, N))).astype(F32) * \
        rng.uniform(1.0, 2.0, (G, N)).astype(F32)
    bias = (rng.standard_normal(N) * 0.5).astype(np.float16)
    y = O.mv_pergroup(x, w, sw, bias, gs)[0].astype(np.float64)
    exact, mag = _pg_mv_closed_form(x, w, sw, bias, gs)
    u = 2.0 ** -24
    nb = K // 256
    n = 14 + nb
    bound = n * u / (1 - n * u) * mag + u * np.abs(bias.astype(np.float64))
    half_ulp = 0.5 * f16_ulp(exact)
    assert (np.abs(y - exact) <= bound + half_ulp * (1 + 1e-9)).all()
    # the plausible mistakes fail the same check
    mistakes = {
        "transposed scale": np.ascontiguousarray(sw.T).reshape(G, N),
        "groups in reverse": np.ascontiguousarray(sw[::-1]),
    }
    if gs < 256:
        mistakes["group of the block"] = sw[np.arange(G) * gs // 256 * 256 // gs]
    for name, swm in mistakes.items():
        ym = O.mv_pergroup(x, w, swm, bias, gs)[0].astype(np.float64)
        assert not (np.abs(ym - exact) <= bound + half_ulp).all(), name


def test_pergroup_mv_group_index_kat():
    """Hand-worked: K=512, gs=64, one nonzero product per group, scale of
    group g = 2^g; the output is sum_g 2^g * (g+1) = 1793 exactly."""
    gs, K = 64, 512
    x = np.zeros((1, K), np.float16)
    w = np.zeros((1, K), np.int8)
    for g in range(K // gs):
        k = g * gs + 37 % gs          # not the first element of its 8-lane chunk
        x[0, k] = 1.0
        w[0, k] = g + 1
    sw = np.array([[2.0 ** g] for g in range(K // gs)], F32)
    y = O.mv_pergroup(x, w, sw, np.zeros(1, np.float16), gs)
    assert float(y[0, 0]) == sum(2.0 ** g * (g + 1) for g in range(K // gs)) == 1793.0


def test_pergroup_validation():
    x = O.synth_activations(2, 192, 1)
    w = O.synth_weights_i8(4, 192, 2)
    with pytest.raises(ValueError):
        O.pergroup_linear(x, w, np.ones((3, 4), F32), 32)
    with pytest.raises(ValueError):
        O.pergroup_gemm(*O.quantize_per_token(x), w, np.ones((1, 4), F32), None, 128)


# --------------------------------------------------------------------------
# a7: W4
# --------------------------------------------------------------------------


def test_w4_ref_nibble_order():
    packed = np.array([[0x1F, 0x80]], np.uint8)      # [K/2=1, N=2]
    w = O.unpack_w4_ref(packed)
    assert w.tolist() == [[1 - 8, 8 - 8], [15 - 8, 0 - 8]]   # hi nibble = even k


def test_w4_ref_pack_roundtrip_and_linear():
    rng = np.random.default_rng(8)
    K, N = 64, 12
    wf = rng.standard_normal((K, N)).astype(F32)
    packed, sw = O.pack_weight_int4(wf)
    w = O.unpack_w4_ref(packed).astype(np.int32)
    assert w.min() >= -8 and w.max() <= 7
    assert (np.abs(w * sw[None, :] - wf) <= sw[None, :] * 0.5 + 1e-7).all()
    x = O.synth_activations(3, K, 9)
    y = O.w4a8_linear(x, packed, sw)
    q, sa = O.quantize_per_token(x)
    acc = (q.astype(np.int64) @ w.astype(np.int64)).astype(np.int32)
    for m in range(3):
        for n in range(N):
            assert Fraction(float(y[m, n])) == _exact_pc(acc[m, n], sa[m], sw[n], None)


def test_w4_lo_first_layout():
    packed = np.array([[0x8F, 0x70]], np.uint8)      # [N=1, K/2=2]
    assert O.unpack_w4_lo_first(packed).tolist() == [[-1, -8, 0, 7]]
    rng = np.random.default_rng(10)
    w = rng.integers(-8, 8, (7, 40), dtype=np.int8)
    np.testing.assert_array_equal(O.unpack_w4_lo_first(O.pack_w4_lo_first(w)), w)


def test_w4_pergroup_equals_int8_pergroup_on_same_values():
    rng = np.random.default_rng(12)
    N, K, gs = 10, 256, 64
    w = rng.integers(-8, 8, (N, K), dtype=np.int8)
    sc = O.synth_scales((K // gs, N), 13).astype(np.float16)
    x = O.synth_activations(4, K, 14)
    y4 = O.w4a8_pergroup_linear(x, O.pack_w4_lo_first(w), sc, gs)
    q, sa = O.quantize_per_token(x)
    np.testing.assert_array_equal(y4, O.pergroup_gemm(q, sa, w, sc.astype(F32), None, gs))


# --------------------------------------------------------------------------
# a14: weight quantizers
# --------------------------------------------------------------------------


def test_weight_quantizer_half_even_and_zero_rows():
    w = np.array([[127, 2.5, 3.5, -2.5, -127], [0, 0, 0, 0, 0]], F32)
    q, s = O.quantize_weight_int8(w)
    assert s.tolist() == [1.0, 1.0]
    assert q.tolist() == [[127, 2, 4, -2, -127], [0, 0, 0, 0, 0]]
    qg, sg = O.quantize_weight_pergroup(np.tile(w, (1, 2))[:, :8], 4)
    assert sg.shape == (2, 2)


def test_weight_quantizer_pergroup_whole_row_equals_per_channel():
    """gs = K is one group per row: bit for bit the per-channel quantizer."""
    rng = np.random.default_rng(21)
    for N, K in [(7, 64), (33, 256), (5, 1000)]:
        w = (rng.standard_normal((N, K)) * rng.uniform(0.01, 10, (N, 1))).astype(F32)
        w[1] = 0.0
        qg, sg = O.quantize_weight_pergroup(w, K)
        q, s = O.quantize_weight_int8(w)
        assert sg.shape == (N, 1)
        np.testing.assert_array_equal(qg, q)
        np.testing.assert_array_equal(sg[:, 0].view(np.uint32), s.view(np.uint32))


def test_weight_quantizer_pergroup_kat_and_exact_model():
    """Hand-worked values: row 0 has groups of max 4 and 40, row 1 of 127
    and 0; 2/(4/127) = 63.5 rounds half to even (64), and the all-zero
    group gets scale 1.  Reshaping along the wrong axis (groups taken down
    the columns) gives other scales."""
    w = np.array([[1, 2, 3, 4, 10, 20, 30, 40],
                  [127, -2.5, 3.5, 1, 0, 0, 0, 0]], F32)
    q, s = O.quantize_weight_pergroup(w, 4)
    np.testing.assert_array_equal(s, np.array([[4 / 127, 40 / 127], [1.0, 1.0]], F32))
    assert q.tolist() == [[32, 64, 95, 127, 32, 64, 95, 127], [127, -2, 4, 1, 0, 0, 0, 0]]
    wrong = np.abs(w.T.reshape(2, 4, 2)).max(axis=1) / F32(127.0)
    assert not np.array_equal(wrong, s)
    # exact-rational model, element by element
    rng = np.random.default_rng(22)
    w = (rng.standard_normal((3, 192)) * 3).astype(F32)
    for gs in (64, 96):
        q, s = O.quantize_weight_pergroup(w, gs)
        for n in range(3):
            for g in range(192 // gs):
                seg = w[n, g * gs:(g + 1) * gs]
                sc = X.f32(Fraction(float(np.max(np.abs(seg)))) / 127)
                assert Fraction(float(s[n, g])) == sc
                for j, v in enumerate(seg):
                    e = max(-128, min(127, X.rne(X.f32(Fraction(float(v)) / sc))))
                    assert int(q[n, g * gs + j]) == e


# --------------------------------------------------------------------------
# the C restatement agrees with the numpy one
# --------------------------------------------------------------------------


def test_c_f16_conversions_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = C.f16_to_f32(h)
    ref = h.astype(np.float32)
    same = (f == ref) | (np.isnan(f) & np.isnan(ref))
    assert same.all()
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 1 << 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([bits.view(np.float32),
                           np.array([65504, 65519.99, 65520, 6e-8, 2.98e-8, 2.9802322e-08,
                                     -0.0, 1.0009765625, 1.00048828125, 1.00146484375], F32)])
    got = C.f32_to_f16(vals)
    exp = vals.astype(np.float16)
    ok = (got.view(np.uint16) == exp.view(np.uint16)) | (np.isnan(got) & np.isnan(exp))
    assert ok.all()


def test_c_oracle_matches_numpy(golden_cases):
    g = golden_cases
    for i in range(4):
        x, w, sw, bias = g[f"pc{i}_x"], g[f"pc{i}_w"], g[f"pc{i}_sw"], g[f"pc{i}_bias"]
        q, sa = C.quantize_per_token(x)
        np.testing.assert_array_equal(q, g[f"pc{i}_q"])
        np.testing.assert_array_equal(sa, g[f"pc{i}_sa"])
        y = C.perchannel_linear_gemm(x, w, sw, bias)
        np.testing.assert_array_equal(y.view(np.uint16), g[f"pc{i}_y"].view(np.uint16))
    for i in range(2):
        y = C.mv_perchannel(g[f"mv{i}_x"], g[f"mv{i}_w"], g[f"mv{i}_sw"], g[f"mv{i}_bias"])
        np.testing.assert_array_equal(y.view(np.uint16), g[f"mv{i}_y"].view(np.uint16))
    for i in range(4):
        gs = int(g[f"pg{i}_gs"])
        x = g[f"pg{i}_x"]
        if x.shape[0] == 1:
            continue
        q, sa = O.quantize_per_token(x)
        y = C.pergroup_gemm(q, sa, g[f"pg{i}_w"], g[f"pg{i}_sw"], g[f"pg{i}_bias"], gs)
        np.testing.assert_array_equal(y.view(np.uint16), g[f"pg{i}_y"].view(np.uint16))


def test_c_oracle_bitexact_shapes_subset(bitexact_shapes):
    for rec in bitexact_shapes:
        if rec["M"] * rec["N"] * rec["K"] > 40_000_000:
            continue
        a, b = bitexact_inputs(rec["M"], rec["K"], rec["N"])
        assert sha(C.int8_matmul_int32(a, b)) == rec["sha_c"]


def test_golden_cases_reproduce(golden_cases):
    """The committed fixtures are what the oracle computes today."""
    g = golden_cases
    for i in range(4):
        np.testing.assert_array_equal(
            O.perchannel_linear(g[f"pc{i}_x"], g[f"pc{i}_w"], g[f"pc{i}_sw"], g[f"pc{i}_bias"]).view(np.uint16),
            g[f"pc{i}_y"].view(np.uint16))
    for i in range(4):
        np.testing.assert_array_equal(
            O.pergroup_linear(g[f"pg{i}_x"], g[f"pg{i}_w"], g[f"pg{i}_sw"], int(g[f"pg{i}_gs"]),
                              g[f"pg{i}_bias"]).view(np.uint16),
            g[f"pg{i}_y"].view(np.uint16))
    for i in range(2):
        np.testing.assert_array_equal(
            O.w4a8_linear(g[f"w4r{i}_x"], g[f"w4r{i}_packed"], g[f"w4r{i}_sw"]).view(np.uint16),
            g[f"w4r{i}_y"].view(np.uint16))
        np.testing.assert_array_equal(
            O.w4a8_pergroup_linear(g[f"w4g{i}_x"], g[f"w4g{i}_packed"], g[f"w4g{i}_scale"],
                                   int(g[f"w4g{i}_gs"])).view(np.uint16),
            g[f"w4g{i}_y"].view(np.uint16))


@pytest.mark.parametrize("gs", [0, 64, 128])
def test_mv_bar_accepts_the_oracle_and_rejects_planted_mistakes(gs):
    """The MV parity bar (tests/util.py assert_mv_close) passes the oracle's
    own output and fails outputs with one product dropped, one product
    counted twice, or a scale off by 1 %."""
    from tests.util import assert_mv_close
    N, K = 64, 2560
    x = O.synth_activations(1, K, 71)
    w = O.synth_weights_i8(N, K, 72)
    sw = O.synth_scales(N if gs == 0 else (K // gs, N), 73)
    b = (np.random.default_rng(74).standard_normal(N) * 0.1).astype(np.float16)

    def run(ww, ss):
        return (O.mv_perchannel(x, ww, ss, b) if gs == 0 else O.mv_pergroup(x, ww, ss, b, gs))

    assert_mv_close(run(w, sw), x, w, sw, b, gs, "oracle")
    k = int(np.argmax(np.abs(x[0].astype(np.float32))))
    dropped = w.copy()
    dropped[:, k] = 0
    doubled = w.astype(np.int16)
    doubled[:, k] = np.clip(2 * doubled[:, k], -127, 127)
    for name, bad in (("dropped product", run(dropped, sw)),
                      ("doubled product", run(doubled.astype(np.int8), sw)),
                      ("scale off by 1%", run(w, (sw * F32(1.01)).astype(F32)))):
        with pytest.raises(AssertionError):
            assert_mv_close(bad, x, w, sw, b, gs, name)


def test_sum_bar_compares_non_finite_outputs_per_element():
    """The tolerance bar of tests/util.py (assert_sum_close, under the MV
    bar) requires the oracle's NaN positions and inf signs element by
    element: -inf for +inf, a NaN moved to another output, or a finite value
    for a NaN fail it; a matching NaN / NaN pair and matching infinities
    pass."""
    from tests.util import assert_sum_close
    ref = np.array([1.0, np.inf, np.nan, -np.inf, 2.0], np.float16)
    exact = np.array([1.0, np.inf, np.nan, -np.inf, 2.0])
    mag = np.abs(np.nan_to_num(exact, nan=0.0, posinf=0.0, neginf=0.0))
    assert_sum_close(ref.copy(), ref, exact, mag, 8, "same")
    for name, bad in (("inf sign", [1.0, -np.inf, np.nan, -np.inf, 2.0]),
                      ("NaN moved", [np.nan, np.inf, 3.0, -np.inf, 2.0]),
                      ("NaN lost", [1.0, np.inf, 0.0, -np.inf, 2.0]),
                      ("finite off", [1.0, np.inf, np.nan, -np.inf, 2.5])):
        with pytest.raises(AssertionError):
            assert_sum_close(np.array(bad, np.float16), ref, exact, mag, 8, name)


def _fma_pergroup_chain(q, sa, w, sw, bias, gs, slices=1):
    """The per-group GEMM as the fma-flush kernels evaluate it: per K slice a
    chain acc = fma(f32(D_g), s, acc) (the fma's single rounding from the
    exact float64 value, exact here since |D s| < 2^75 with 46-bit products
    and the addend at most 2^64), the slices added in order, then the
    reference's epilogue operations."""
    M, K = q.shape
    N = w.shape[0]
    G = K // gs
    s = sw.astype(np.float64).reshape(G, N)
    per = G // slices
    total = None
    for sl in range(slices):
        acc = np.zeros((M, N), F32)
        for g in range(sl * per, (sl + 1) * per):
            D = q[:, g * gs:(g + 1) * gs].astype(np.int64) @ w[:, g * gs:(g + 1) * gs].astype(np.int64).T
            acc = (acc.astype(np.float64) + D.astype(np.float64) * s[g][None, :]).astype(F32)
        total = acc if total is None else (total + acc).astype(F32)
    v = (total * sa.astype(F32)[:, None]).astype(F32)
    if bias is not None:
        v = (v + bias.astype(F32)[None, :]).astype(F32)
    return v.astype(np.float16)


@pytest.mark.parametrize("gs", [64, 128])
def test_pergroup_bar_accepts_fma_chains_and_rejects_planted_mistakes(gs):
    """The per-group tolerance bar (tests/util.py assert_pergroup_close)
    passes the oracle's sequential chain, an fma chain and a 4-slice split
    of it, and fails a dropped group, a group counted twice, the scales of
    the next group, a column-shifted scale row and a scale off by 1 %."""
    from tests.util import assert_pergroup_close
    M, N, K = 24, 96, 1024
    x = O.synth_activations(M, K, 171)
    w = O.synth_weights_i8(N, K, 172)
    sw = O.synth_scales((K // gs, N), 173)
    b = (np.random.default_rng(174).standard_normal(N) * 0.1).astype(np.float16)
    q, sa = O.quantize_per_token(x)
    ref = O.pergroup_gemm(q, sa, w, sw, b, gs)

    def bar(y, what):
        assert_pergroup_close(y, q, sa, w, sw, b, gs, ref, what)

    bar(ref, "oracle")
    fma1 = _fma_pergroup_chain(q, sa, w, sw, b, gs)
    fma4 = _fma_pergroup_chain(q, sa, w, sw, b, gs, slices=4)
    bar(fma1, "fma chain")
    bar(fma4, "4 slices")
    G = K // gs
    dropped = sw.copy()
    dropped[3] = 0
    doubled = sw.copy()
    doubled[3] *= F32(2)
    nextg = np.roll(sw, -1, axis=0)
    shifted = np.roll(sw, 1, axis=1)
    off = (sw * F32(1.01)).astype(F32)
    for name, s_bad in (("dropped group", dropped), ("group twice", doubled),
                        ("next group's scales", nextg), ("column-shifted scales", shifted),
                        ("scale off by 1%", off)):
        with pytest.raises(AssertionError):
            bar(O.pergroup_gemm(q, sa, w, s_bad, b, gs), name)
    assert G >= 8

"""Shared test helpers: fp16 tolerance, GPU gating, tensor conversion."""

import numpy as np
import pytest


def has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def f16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of fp16 values at |v| (subnormal spacing below 2^-14)."""
    a = np.abs(np.asarray(v, np.float16)).astype(np.float64)
    a = np.where(np.isfinite(a), a, 65504.0)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def assert_f16_close(got, exp, rel=1e-3, ulps=1, what=""):
    """fp16 parity bar: every element within ``ulps`` fp16 ulp of the expected
    value or within ``rel`` relative error; NaN and inf must match exactly."""
    got = np.asarray(got, np.float16)
    exp = np.asarray(exp, np.float16)
    assert got.shape == exp.shape, (got.shape, exp.shape)
    gf = got.astype(np.float64)
    ef = exp.astype(np.float64)
    nan_g, nan_e = np.isnan(gf), np.isnan(ef)
    assert (nan_g == nan_e).all(), f"{what}: NaN pattern differs"
    inf_g, inf_e = np.isinf(gf), np.isinf(ef)
    assert (inf_g == inf_e).all() and (gf[inf_g] == ef[inf_e]).all(), f"{what}: inf differs"
    fin = ~(nan_e | inf_e)
    d = np.abs(gf[fin] - ef[fin])
    ok = (d <= ulps * f16_ulp(ef[fin])) | (d <= rel * np.abs(ef[fin]))
    if not ok.all():
        idx = np.flatnonzero(~ok)[:5]
        raise AssertionError(
            f"{what}: {np.count_nonzero(~ok)} of {ok.size} elements outside "
            f"{ulps} ulp / {rel} rel; e.g. got {gf[fin][idx]} expected {ef[fin][idx]}")


def assert_bits_equal(got, exp, what=""):
    """Bit-for-bit equality (fp16 compared as uint16 patterns, NaN payloads
    compared as 'is NaN')."""
    got = np.asarray(got)
    exp = np.asarray(exp)
    assert got.shape == exp.shape and got.dtype == exp.dtype, (got.shape, exp.shape,
                                                               got.dtype, exp.dtype)
    if got.dtype == np.float16:
        gn, en = np.isnan(got), np.isnan(exp)
        assert (gn == en).all(), f"{what}: NaN pattern differs"
        g = got.view(np.uint16)[~gn]
        e = exp.view(np.uint16)[~en]
    else:
        g, e = got, exp
    if not np.array_equal(g, e):
        bad = np.flatnonzero(g.reshape(-1) != e.reshape(-1))
        raise AssertionError(f"{what}: {bad.size} of {g.size} elements differ; first at "
                             f"{bad[:5]}: got {g.reshape(-1)[bad[:5]]} exp {e.reshape(-1)[bad[:5]]}")


gpu = pytest.mark.gpu


def mv_exact(x, w, sw, bias, gs):
    """float64 value and magnitude of the M == 1 MV, from its definition:
    y[n] = sum_k s(n, k) w[n, k] x[k] + bias[n], s = sw[n] per channel
    (gs 0) or sw[k // gs, n] per group; returns (exact [N], sum of |terms|
    [N] including |bias|)."""
    xv = np.asarray(x, np.float16).reshape(-1).astype(np.float64)
    prod = np.asarray(w).astype(np.float64) * xv[None, :]
    N, K = prod.shape
    if gs == 0:
        s = np.asarray(sw, np.float32).astype(np.float64).reshape(N, 1)
        exact, mag = s[:, 0] * prod.sum(1), np.abs(s[:, 0]) * np.abs(prod).sum(1)
    else:
        G = K // gs
        s = np.asarray(sw, np.float32).astype(np.float64).reshape(G, N).T      # [N, G]
        exact = (s * prod.reshape(N, G, gs).sum(2)).sum(1)
        mag = (np.abs(s) * np.abs(prod).reshape(N, G, gs).sum(2)).sum(1)
    b = np.zeros(N) if bias is None else np.asarray(bias, np.float16).astype(np.float64)
    return exact + b, mag + np.abs(b)


def assert_mv_close(got, x, w, sw, bias, gs, what="", ref=None):
    """Bar for the fp16-activation MV (M == 1), whose reduction order the
    reference leaves to Metal's ``simd_sum`` (unspecified).  Every output must
    be within the north-star bar of the oracle's order -- 1e-3 relative or
    1 fp16 ulp -- or, where cancellation makes the sum small, within the
    fp32 error bound of an evaluation of depth d of the exact value:
    gamma_d * sum|terms| + 1 fp16 ulp, with d = 2 * ceil(K / 64) + 16, which
    covers a 64-lane split of each row with paired products, the cross-lane
    tree, the scale multiply and the bias add (and the oracle's 32-lane
    order).  Dropping, duplicating or misplacing a single product, or a
    wrong scale, fails both parts.  ``ref``: the oracle's output if already
    at hand (e.g. a committed fixture)."""
    from oracle import cider_oracle as O
    got = np.asarray(got, np.float16).reshape(-1)
    x = np.asarray(x, np.float16)
    N, K = np.asarray(w).shape
    if bias is None:
        bias = np.zeros(N, np.float16)
    if ref is None:
        ref = (O.mv_perchannel(x, w, sw, bias) if gs == 0 else
               O.mv_pergroup(x, w, sw, bias, gs))
    ref = np.asarray(ref, np.float16).reshape(-1)
    exact, mag = mv_exact(x, w, sw, bias, gs)
    assert_sum_close(got, ref, exact, mag, 2 * (-(-K // 64)) + 16, what, "MV bar")


def assert_sum_close(got, ref, exact, mag, depth, what="", bar="bar"):
    """fp16 outputs of a sum whose fp32 evaluation order is free (any tree,
    fma or not): every output is within 1e-3 relative or 1 fp16 ulp of the
    oracle's output ``ref``, or within gamma_depth * mag + 1 fp16 ulp of the
    float64 value ``exact`` (``mag``: the sum of the absolute terms), the
    fp32 error bound of any evaluation of that depth.  Non-finite outputs
    must match the oracle element by element (NaN positions, inf signs); the
    bar applies to the elements finite in both."""
    g = np.asarray(got, np.float16).reshape(-1).astype(np.float64)
    r = np.asarray(ref, np.float16).reshape(-1).astype(np.float64)
    exact = np.asarray(exact, np.float64).reshape(-1)
    mag = np.asarray(mag, np.float64).reshape(-1)
    assert g.shape == r.shape, (g.shape, r.shape)
    nan_g, nan_r = np.isnan(g), np.isnan(r)
    assert (nan_g == nan_r).all(), f"{what}: NaN positions differ from the oracle's"
    inf_g, inf_r = np.isinf(g), np.isinf(r)
    assert (inf_g == inf_r).all() and (g[inf_g] == r[inf_r]).all(), \
        f"{what}: inf outputs differ from the oracle's"
    fin = ~(nan_r | inf_r)
    g, r, exact, mag = g[fin], r[fin], exact[fin], mag[fin]
    u = 2.0 ** -24
    bound = depth * u / (1 - depth * u) * mag + f16_ulp(exact)
    near_ref = (np.abs(g - r) <= f16_ulp(r)) | (np.abs(g - r) <= 1e-3 * np.abs(r))
    near_exact = np.abs(g - exact) <= bound
    ok = near_ref | near_exact
    if not ok.all():
        idx = np.flatnonzero(~ok)[:5]
        raise AssertionError(
            f"{what}: {np.count_nonzero(~ok)} of {ok.size} outputs outside the {bar}; "
            f"e.g. at {idx}: got {g[idx]} oracle {r[idx]} exact {exact[idx]} bound {bound[idx]}")


def pergroup_exact(q, sa, w, sw_gn, bias, gs):
    """float64 value and magnitude of the per-group GEMM from its definition:
    y[m, n] = sa[m] * sum_g D_g[m, n] * s[g, n] + bias[n], D_g the exact
    int dot product of group g; returns (exact [M, N], sum of |terms| with
    the same factors, plus |bias|)."""
    qf = np.asarray(q).astype(np.float64)
    wf = np.asarray(w).astype(np.float64)
    M, K = qf.shape
    N = wf.shape[0]
    G = K // gs
    s = np.asarray(sw_gn, np.float32).astype(np.float64).reshape(G, N)
    exact = np.zeros((M, N))
    mag = np.zeros((M, N))
    with np.errstate(invalid="ignore", over="ignore"):
        for g in range(G):
            D = qf[:, g * gs:(g + 1) * gs] @ wf[:, g * gs:(g + 1) * gs].T   # exact below 2^53
            t = D * s[g][None, :]
            exact += t
            mag += np.abs(t)
        sa64 = np.asarray(sa, np.float32).astype(np.float64).reshape(M, 1)
        b = (np.zeros(N) if bias is None else
             np.asarray(bias, np.float16).astype(np.float64)).reshape(1, N)
        return exact * sa64 + b, mag * np.abs(sa64) + np.abs(b)


def assert_pergroup_close(got, q, sa, w, sw_gn, bias, gs, ref, what=""):
    """Bar for the per-group GEMM's fp16 outputs (M >= 2): the int32 group sums
    D_g are exact, the fp32 chain over the groups may be evaluated in any
    order and with fused multiply-adds (the kernels flush with
    fma(f32(D_g), s, acc), and split-K adds the chains of K slices), so
    every output is within 1e-3 relative / 1 fp16 ulp of the oracle's
    sequential chain ``ref``, or within gamma_d * sum|terms| + 1 fp16 ulp of
    the float64 value with d = 2 G + 8 (G groups: a product and an add each,
    then the slice sums, the per-token scale and the bias).  Non-finite
    outputs must match the oracle element by element.  ``q``, ``sa``: the
    quantized activations; ``w``: int8 weights [N, K] (int4 values widened).
    A dropped or duplicated group, a scale of the wrong group or column, or a
    scale off by 1 % fails it (tests/test_oracle.py)."""
    G = np.asarray(q).shape[1] // gs
    exact, mag = pergroup_exact(q, sa, w, sw_gn, bias, gs)
    assert_sum_close(got, ref, exact, mag, 2 * G + 8, what, "per-group bar")


def assert_pergroup_linear_close(got, x, w, sw_gn, bias, gs, ref, what=""):
    """assert_pergroup_close for fp16 activation rows x (quantized here with
    the oracle's per-token quantization, which the kernels match bit for
    bit)."""
    from oracle import cider_oracle as O
    q, sa = O.quantize_per_token(np.asarray(x, np.float16))
    assert_pergroup_close(got, q, sa, w, sw_gn, bias, gs, ref, what)

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

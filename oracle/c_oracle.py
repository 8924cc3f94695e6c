"""ctypes wrapper of ``oracle/libcider_oracle.so`` (the C restatement).

TEST INFRASTRUCTURE ONLY: used by tests/ and by the cpu_baseline leg of
bench.py.  The library is built by ``make -C oracle`` (``__graft_entry__.build``).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcider_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64


def lib():
    """Load the C oracle, raising if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"C oracle not built: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        sigs = {
            "oracle_h2f_array": [_P, _P, _I64],
            "oracle_f2h_array": [_P, _P, _I64],
            "oracle_quantize_per_token": [_P, _I, _I, _P, _P],
            "oracle_i8_gemm_nt": [_P, _P, _I, _I, _I, _P],
            "oracle_dequant_perchannel": [_P, _P, _P, _P, _I, _I, _P],
            "oracle_mv_perchannel": [_P, _P, _P, _P, _I, _I, _P],
            "oracle_pergroup_gemm": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
            "oracle_perchannel_linear": [_P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P],
            "oracle_num_threads": [],
            "oracle_set_num_threads": [_I],
        }
        for name, argtypes in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = _I if name == "oracle_num_threads" else None
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f2h_array(_ptr(f), _ptr(out), f.size)
    return out.view(np.float16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.float16).view(np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_h2f_array(_ptr(h), _ptr(out), h.size)
    return out


def quantize_per_token(x):
    x = _c(x, np.float16)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    sa = np.empty(M, np.float32)
    lib().oracle_quantize_per_token(_ptr(x), M, K, _ptr(q), _ptr(sa))
    return q, sa


def int8_matmul_int32(a, b_nk):
    a = _c(a, np.int8)
    b = _c(b_nk, np.int8)
    M, K = a.shape
    N = b.shape[0]
    c = np.empty((M, N), np.int32)
    lib().oracle_i8_gemm_nt(_ptr(a), _ptr(b), M, N, K, _ptr(c))
    return c


def dequant_perchannel(acc, sa, sw, bias):
    acc = _c(acc, np.int32)
    M, N = acc.shape
    sa = _c(sa, np.float32)
    sw = _c(sw, np.float32)
    y = np.empty((M, N), np.float16)
    if bias is None:
        bp = None
    else:
        bias = _c(bias, np.float16)
        bp = _ptr(bias)
    lib().oracle_dequant_perchannel(_ptr(acc), _ptr(sa), _ptr(sw), bp, M, N, _ptr(y))
    return y


def mv_perchannel(x, w, sw, bias):
    x = _c(x, np.float16).reshape(-1)
    w = _c(w, np.int8)
    N, K = w.shape
    sw = _c(sw, np.float32)
    bias = _c(bias, np.float16)
    y = np.empty(N, np.float16)
    lib().oracle_mv_perchannel(_ptr(x), _ptr(w), _ptr(sw), _ptr(bias), N, K, _ptr(y))
    return y[None, :]


def pergroup_gemm(q, sa, w, sw_gn, bias, group_size):
    q = _c(q, np.int8)
    M, K = q.shape
    w = _c(w, np.int8)
    N = w.shape[0]
    sa = _c(sa, np.float32)
    sw_gn = _c(sw_gn, np.float32)
    y = np.empty((M, N), np.float16)
    if bias is None:
        bp = None
    else:
        bias = _c(bias, np.float16)
        bp = _ptr(bias)
    lib().oracle_pergroup_gemm(_ptr(q), _ptr(sa), _ptr(w), _ptr(sw_gn), bp,
                               M, N, K, group_size, _ptr(y))
    return y


def perchannel_linear_gemm(x, w, sw, bias):
    """M >= 2 per-channel linear (quantize + GEMM + epilogue) in C."""
    x = _c(x, np.float16)
    M, K = x.shape
    w = _c(w, np.int8)
    N = w.shape[0]
    sw = _c(sw, np.float32)
    bias = _c(bias, np.float16)
    q = np.empty((M, K), np.int8)
    sa = np.empty(M, np.float32)
    acc = np.empty((M, N), np.int32)
    y = np.empty((M, N), np.float16)
    lib().oracle_perchannel_linear(_ptr(x), _ptr(w), _ptr(sw), _ptr(bias), M, N, K,
                                   _ptr(q), _ptr(sa), _ptr(acc), _ptr(y))
    return y


def num_threads() -> int:
    return lib().oracle_num_threads()


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(n)

"""ctypes binding of ``cider_amd/lib/libcider_hip.so`` (the C ABI in
``include/cider_hip.h``).

Counterpart of the reference's extension loader ``cider/ops.py:31-47``, which
imports the nanobind module ``_cider_prim`` from ``cider/lib`` and raises
``RuntimeError`` when it is missing.  Here the extension is a plain C shared
library; a missing or unloadable library raises ``RuntimeError`` the same way,
and there is no fallback of any kind.

torch is imported before the library is opened: PyTorch-ROCm ships its own
HIP runtime (SONAME ``libamdhip64.so.7``), and loading it first makes the
dynamic loader resolve this library's HIP dependency to that same copy, so
device pointers and streams from torch are valid in our calls.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede CDLL: shares torch's HIP runtime)

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libcider_hip.so")

CIDER_OK = 0
CIDER_E_INVALID = -1
CIDER_E_HIP = -2
CIDER_E_UNSUPPORTED = -3

CIDER_OP_PERCHANNEL = 1
CIDER_OP_PERGROUP = 2
CIDER_OP_W4A8 = 3
CIDER_OP_W4A8_PERGROUP = 4
CIDER_OP_W4A8_REF = 5

CIDER_NOALLOC_SCRATCH_BYTES = 32 << 20

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); exactly the symbols declared in include/cider_hip.h
SIGNATURES = {
    "cider_version": (_I, []),
    "cider_last_error": (ctypes.c_char_p, []),
    "cider_workspace_bytes": (_SZ, [_I, _I64, _I64, _I64, _I]),
    "cider_quantize_per_token": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "cider_int8_matmul_int32": (_I, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "cider_perchannel_linear": (_I, [_P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _P]),
    "cider_perchannel_linear_noalloc": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cider_perchannel_gemm": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cider_pergroup_linear": (_I, [_P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I, _P]),
    "cider_w4_repack_ref": (_I, [_P, _P, _I64, _I64, _P]),
    "cider_w4a8_linear": (_I, [_P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _P]),
    "cider_w4a8_linear_ref": (_I, [_P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _P]),
    "cider_w4a8_pergroup_linear": (_I, [_P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I, _P]),
    "cider_rmsnorm_quantize": (_I, [_P, _P, _P, _P, _F, _P, _P, _P, _I64, _I64, _P]),
    "cider_silu_mul_quantize": (_I, [_P, _P, _P, _P, _I64, _I64, _P]),
    "cider_qk_norm_rope": (_I, [_P, _P, _P, _F, _P, _P, _I64, _P, _P, _P, _P, _P,
                                _I64, _I64, _I64, _I64, _I64, _P]),
    "cider_attn_decode_workspace_bytes": (_SZ, [_I64, _I64]),
    "cider_attn_decode": (_I, [_P, _P, _P, _P, _F, _P, _SZ, _P, _I64, _I64, _I64, _I64, _P]),
    "cider_attn_prefill_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "cider_attn_prefill": (_I, [_P, _P, _P, _F, _P, _SZ, _P, _I64, _I64, _P, _I64, _I64, _I64,
                                _I64, _P]),
    "cider_attn_prefill_quantize_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "cider_attn_prefill_quantize": (_I, [_P, _P, _P, _F, _P, _SZ, _P, _P, _I64, _I64, _P, _I64,
                                         _I64, _I64, _I64, _P]),
    "cider_rmsnorm_mv": (_I, [_P, _P, _P, _P, _F, _P, _P, _P, _P, _I64, _I64, _P]),
    "cider_swiglu_mv": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _P]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Open the library (once) and bind every entry point; RuntimeError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"cider_amd HIP extension not built: {LIB_PATH} is missing "
                "(run `python -c 'import __graft_entry__ as g; g.build()'` or "
                "`make -C cider_amd/csrc`)")
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - depends on the machine
            raise RuntimeError(f"cider_amd HIP extension failed to load: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as e:
                raise RuntimeError(
                    f"cider_amd HIP extension at {LIB_PATH} lacks {name}: it is older "
                    "than its sources; rebuild it") from e
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    """Raise for a negative return code, with the library's message."""
    if rc == CIDER_OK:
        return
    msg = (load().cider_last_error() or b"").decode(errors="replace")
    if rc == CIDER_E_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg or f"cider error {rc}")


def workspace_bytes(op: int, M: int, N: int, K: int, group_size: int = 0) -> int:
    return int(load().cider_workspace_bytes(op, M, N, K, group_size))

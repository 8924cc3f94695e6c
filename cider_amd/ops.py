"""cider_amd.ops - functional API of the fused quantize -> int8 GEMM -> dequant
linear on MI355X, a drop-in for the reference's ``cider/ops.py``.

Same function names, argument order and meaning as the reference
(``cider/ops.py:73-255``), on ``torch`` tensors that live on a ROCm GPU
instead of ``mx.array``:

* ``perchannel_linear(x, w, scale_w, bias=None, stream=None)``
* ``pergroup_linear(x, w, scale_w, group_size, bias=None, new_bias=None, stream=None)``
* ``w4a8_linear(x, packed_w, scale_w, stream=None)``
* ``int8_matmul_int32(a, b, stream=None)``
* ``quantize_weight_int8(w)``, ``pack_weight_int4(w, zero_point=8)`` (numpy)
* ``is_available()``, ``kernel_dir()``

Where MLX returns a lazy array evaluated at ``mx.eval``, these functions
enqueue the kernels on the current (or given) torch stream and return at once.
Errors follow the reference: bad ranks, shapes and group sizes raise
``ValueError`` (``std::invalid_argument`` there), a missing extension or a
device failure raises ``RuntimeError``.  There is no CPU implementation (the
reference's ``eval_cpu`` throws, ``csrc/include/w8a8_primitive.h:32-36``):
CPU tensors raise ``RuntimeError``.

Extensions beyond the reference surface (same kernels): ``quantize_per_token``,
``perchannel_gemm``, ``repack_w4_ref``, ``pack_weight_int4_pergroup`` and
``w4a8_pergroup_linear`` (the per-group int4 format with fp16 scales).
"""

from __future__ import annotations

import collections
import ctypes
import threading
import weakref
from typing import Optional

import numpy as np
import torch

from . import _lib

# --------------------------------------------------------------------------
# availability
# --------------------------------------------------------------------------


def kernel_dir() -> str:
    """Directory of the compiled kernels (``cider/ops.py:19-24``; kept for
    signature compatibility: the HIP kernels are linked into the library)."""
    return _lib.LIB_DIR


def is_available() -> bool:
    """True when the HIP extension loads and a gfx950 (MI355X) GPU is visible.

    Counterpart of the reference's Apple-M5 gate (``cider/ops.py:52-68``)."""
    try:
        _lib.load()
    except RuntimeError:
        return False
    if not torch.cuda.is_available():
        return False
    try:
        arch = torch.cuda.get_device_properties(0).gcnArchName
    except Exception:  # pragma: no cover
        return False
    return arch.split(":")[0] == "gfx950"


# --------------------------------------------------------------------------
# host-side weight quantizers (numpy, as in the reference)
# --------------------------------------------------------------------------


def quantize_weight_int8(w: np.ndarray) -> tuple:
    """Per-output-row symmetric int8 (``cider/ops.py:73-90``).

    w: [N, K] float.  scale = max|w[n]| / 127 (1 where 0);
    q = clip(np.round(w / scale), -128, 127)  (np.round: half to even).
    Returns (q int8 [N, K], scale float32 [N]).
    """
    wf = np.asarray(w).astype(np.float32)
    scale = np.max(np.abs(wf), axis=1) / 127.0
    scale = np.where(scale == 0, 1.0, scale)
    q = np.clip(np.round(wf / scale[:, None]), -128, 127).astype(np.int8)
    return q, scale.astype(np.float32)


def quantize_weight_pergroup(w: np.ndarray, group_size: int) -> tuple:
    """Per-group symmetric int8 (``cider/nn.py:34-59``).

    Returns (q int8 [N, K], scale float32 [N, K // group_size]); layers store
    the scale transposed to [K // group_size, N] (``cider/nn.py:166``).
    """
    wf = np.asarray(w).astype(np.float32)
    N, K = wf.shape
    if K % group_size:
        raise ValueError(f"K={K} not divisible by group_size={group_size}")
    wg = wf.reshape(N, K // group_size, group_size)
    scale = np.max(np.abs(wg), axis=2) / 127.0
    scale = np.where(scale == 0, 1.0, scale)
    q = np.clip(np.round(wg / scale[:, :, None]), -128, 127).astype(np.int8)
    return q.reshape(N, K), scale.astype(np.float32)


def pack_weight_int4(w: np.ndarray, zero_point: int = 8) -> tuple:
    """Per-column symmetric int4, reference packing (``cider/ops.py:93-116``).

    w: [K, N] float, K even.  scale = max|w[:, n]| / 7 (1 where 0);
    nibble = clip(np.round(w / scale) + zero_point, 0, 15);
    packed[k/2, n] = nibble[k] << 4 | nibble[k+1]  (high nibble = even k).
    Returns (packed uint8 [K/2, N], scale float32 [N]).
    """
    wf = np.asarray(w).astype(np.float32)
    K, _ = wf.shape
    if K % 2:
        raise ValueError(f"K must be even, got {K}")
    scale = np.max(np.abs(wf), axis=0) / 7.0
    scale = np.where(scale == 0, 1.0, scale)
    nib = np.clip(np.round(wf / scale[None, :]) + zero_point, 0, 15).astype(np.uint8)
    packed = (nib[0::2, :] << 4) | nib[1::2, :]
    return packed.astype(np.uint8), scale.astype(np.float32)


def pack_weight_int4_pergroup(w: np.ndarray, group_size: int) -> tuple:
    """Per-group symmetric int4 in the library layout (extension).

    w: [N, K] float.  Per group of ``group_size`` consecutive k of row n:
    scale = fp16(max|w| / 7) (1 where 0), q = clip(np.round(w / f32(scale)),
    -8, 7); packed[n, k/2] holds element k in its low nibble for even k and
    in its high nibble for odd k (two's complement).
    Returns (packed uint8 [N, K/2], scales float16 [K/group_size, N]).
    """
    wf = np.asarray(w).astype(np.float32)
    N, K = wf.shape
    if K % group_size or K % 2:
        raise ValueError(f"K={K} must be even and divisible by group_size={group_size}")
    wg = wf.reshape(N, K // group_size, group_size)
    scale = (np.max(np.abs(wg), axis=2) / 7.0).astype(np.float16)
    scale = np.where(scale == 0, np.float16(1.0), scale).astype(np.float16)
    q = np.clip(np.round(wg / scale.astype(np.float32)[:, :, None]), -8, 7)
    q = q.astype(np.int16).reshape(N, K)
    nib = (q & 0xF).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return packed, np.ascontiguousarray(scale.T)


# --------------------------------------------------------------------------
# device plumbing
# --------------------------------------------------------------------------


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_gpu(fn: str, *tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{fn}: expected torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{fn}: tensors must be on a ROCm GPU (got {t.device}); "
                "there is no CPU implementation")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{fn}: tensors on different devices ({dev} and {t.device})")
    return dev


def _stream_ptr(dev: torch.device, stream) -> ctypes.c_void_p:
    s = torch.cuda.current_stream(dev) if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


class _on_stream:
    """Makes `stream` current (so scratch is allocated in its pool) if given."""

    def __init__(self, dev, stream):
        self.ctx = torch.cuda.stream(stream) if stream is not None else None
        self.dev = torch.cuda.device(dev)

    def __enter__(self):
        self.dev.__enter__()
        if self.ctx is not None:
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)
        self.dev.__exit__(*exc)


def _as(t: torch.Tensor, dtype) -> torch.Tensor:
    return t.to(dtype).contiguous()


def _workspace(op: int, M: int, N: int, K: int, gs: int, dev) -> Optional[torch.Tensor]:
    nbytes = _lib.workspace_bytes(op, M, N, K, gs)
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=dev)


def _nbytes(ws: Optional[torch.Tensor]) -> int:
    return 0 if ws is None else ws.numel()


def _check_2d(fn: str, name: str, t: torch.Tensor, what: str):
    if t.dim() != 2:
        raise ValueError(f"{fn}: {name} must be 2D {what}")


def _cast_out(y: torch.Tensor, dtype) -> torch.Tensor:
    return y if dtype == torch.float16 else y.to(dtype)


# --------------------------------------------------------------------------
# primitive API (reference surface)
# --------------------------------------------------------------------------


def quantize_per_token(x: torch.Tensor, stream=None):
    """Per-token int8 quantization of x [M, K] (any float dtype, rounded to
    fp16 first).  Returns (q int8 [M, K], scale_a float32 [M]).

    The first dispatch of the reference's W8A8 path
    (``cider/kernels/w8a8_quantize.metal:17-87``, ``csrc/src/w8a8_primitive.mm:191-202``).
    """
    fn = "quantize_per_token"
    dev = _require_gpu(fn, x)
    _check_2d(fn, "x", x, "[M,K]")
    lib = _lib.load()
    with _on_stream(dev, stream):
        xh = _as(x, torch.float16)
        M, K = xh.shape
        q = torch.empty((M, K), dtype=torch.int8, device=dev)
        sa = torch.empty((M,), dtype=torch.float32, device=dev)
        _lib.check(lib.cider_quantize_per_token(_ptr(xh), _ptr(q), _ptr(sa), M, K,
                                                _stream_ptr(dev, stream)))
    return q, sa


def perchannel_linear(x: torch.Tensor, w: torch.Tensor, scale_w: torch.Tensor,
                      bias: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """W8A8 per-channel linear (``cider/ops.py:121-148``).

    x [M, K] float16/bfloat16 (other floats are cast to fp16), w int8 [N, K],
    scale_w float32 [N], bias float16 [N] (zeros if None).  M == 1 runs the
    fp16-activation MV, M >= 2 quantizes x per token and runs the int8 GEMM
    with the fused per-channel epilogue.  Returns [M, N] in x's dtype.
    """
    fn = "perchannel_linear"
    dev = _require_gpu(fn, x, w, scale_w, bias)
    _check_2d(fn, "x", x, "[M,K]")
    _check_2d(fn, "w", w, "[N,K]")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"{fn}: x is [M,{K}] but w is [{N},{w.shape[1]}]")
    if scale_w.numel() != N:
        raise ValueError(f"{fn}: scale_w has {scale_w.numel()} elements, expected N={N}")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"{fn}: bias has {bias.numel()} elements, expected N={N}")
    out_dtype = x.dtype
    lib = _lib.load()
    with _on_stream(dev, stream):
        xh = _as(x, torch.float16)
        wq = _as(w, torch.int8)
        sw = _as(scale_w.reshape(-1), torch.float32)
        b = (torch.zeros(N, dtype=torch.float16, device=dev) if bias is None
             else _as(bias.reshape(-1), torch.float16))
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = _workspace(_lib.CIDER_OP_PERCHANNEL, M, N, K, 0, dev)
        _lib.check(lib.cider_perchannel_linear(
            _ptr(xh), _ptr(wq), _ptr(sw), _ptr(b), _ptr(y), _ptr(ws),
            _nbytes(ws), M, N, K, _stream_ptr(dev, stream)))
    return _cast_out(y, out_dtype)


def perchannel_gemm(q: torch.Tensor, scale_a: torch.Tensor, w: torch.Tensor,
                    scale_w: torch.Tensor, bias: Optional[torch.Tensor] = None,
                    stream=None) -> torch.Tensor:
    """Per-channel int8 GEMM + epilogue on pre-quantized activations
    (the second dispatch of ``csrc/src/w8a8_primitive.mm:207-247``), any M.
    Returns float16 [M, N]."""
    fn = "perchannel_gemm"
    dev = _require_gpu(fn, q, scale_a, w, scale_w, bias)
    _check_2d(fn, "q", q, "[M,K]")
    _check_2d(fn, "w", w, "[N,K]")
    M, K = q.shape
    N = w.shape[0]
    if w.shape[1] != K or scale_a.numel() != M or scale_w.numel() != N:
        raise ValueError(f"{fn}: inconsistent shapes")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"{fn}: bias has {bias.numel()} elements, expected N={N}")
    lib = _lib.load()
    with _on_stream(dev, stream):
        qq = _as(q, torch.int8)
        sa = _as(scale_a.reshape(-1), torch.float32)
        wq = _as(w, torch.int8)
        sw = _as(scale_w.reshape(-1), torch.float32)
        b = None if bias is None else _as(bias.reshape(-1), torch.float16)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        _lib.check(lib.cider_perchannel_gemm(_ptr(qq), _ptr(sa), _ptr(wq), _ptr(sw), _ptr(b),
                                             _ptr(y), M, N, K, _stream_ptr(dev, stream)))
    return y


def pergroup_linear(x: torch.Tensor, w: torch.Tensor, scale_w: torch.Tensor,
                    group_size: int, bias: Optional[torch.Tensor] = None,
                    new_bias: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Per-group W8A8 linear (``cider/ops.py:161-209``).

    scale_w float32 [K // group_size, N] (the reference's transposed layout),
    group_size in {64, 128, 256}.  M == 1 runs the per-group fp16 MV, M >= 2
    the per-group GEMM.  ``new_bias`` is accepted and ignored, as the
    reference's kernels ignore it (``cider/ops.py:151-158,197-201``).
    """
    fn = "pergroup_linear"
    del new_bias
    dev = _require_gpu(fn, x, w, scale_w, bias)
    _check_2d(fn, "x", x, "[M,K]")
    _check_2d(fn, "w", w, "[N,K]")
    if scale_w.dim() != 2:
        raise ValueError(f"{fn}: scale_w must be 2D [num_groups,N]")
    if group_size not in (64, 128, 256):
        raise ValueError(f"{fn}: group_size must be 64, 128, or 256")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"{fn}: x is [M,{K}] but w is [{N},{w.shape[1]}]")
    if K % group_size:
        raise ValueError(f"{fn}: K={K} is not a multiple of group_size={group_size}")
    if tuple(scale_w.shape) != (K // group_size, N):
        raise ValueError(f"{fn}: scale_w is {tuple(scale_w.shape)}, expected "
                         f"[{K // group_size},{N}] ([num_groups,N])")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"{fn}: bias has {bias.numel()} elements, expected N={N}")
    out_dtype = x.dtype
    lib = _lib.load()
    with _on_stream(dev, stream):
        xh = _as(x, torch.float16)
        wq = _as(w, torch.int8)
        sw = _as(scale_w, torch.float32)
        b = (torch.zeros(N, dtype=torch.float16, device=dev) if bias is None
             else _as(bias.reshape(-1), torch.float16))
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = _workspace(_lib.CIDER_OP_PERGROUP, M, N, K, group_size, dev)
        _lib.check(lib.cider_pergroup_linear(
            _ptr(xh), _ptr(wq), _ptr(sw), _ptr(b), _ptr(y), _ptr(ws),
            _nbytes(ws), M, N, K, group_size, _stream_ptr(dev, stream)))
    return _cast_out(y, out_dtype)


def repack_w4_ref(packed_w: torch.Tensor, stream=None) -> torch.Tensor:
    """Reference W4 layout uint8 [K/2, N] -> library layout uint8 [N, K/2]."""
    fn = "repack_w4_ref"
    dev = _require_gpu(fn, packed_w)
    _check_2d(fn, "packed_w", packed_w, "[K/2,N]")
    K2, N = packed_w.shape
    lib = _lib.load()
    with _on_stream(dev, stream):
        src = _as(packed_w, torch.uint8)
        dst = torch.empty((N, K2), dtype=torch.uint8, device=dev)
        _lib.check(lib.cider_w4_repack_ref(_ptr(src), _ptr(dst), N, 2 * K2,
                                           _stream_ptr(dev, stream)))
    return dst


class _RepackCache:
    """Repacked copies of reference-layout W4 tensors.

    An entry is valid while its source tensor is alive and unmodified: same
    object, version counter, storage address and shape.  The dict is guarded
    by a lock (callers may run on several threads).  A repack runs on the
    stream of the call that misses; an event recorded after it makes every
    later caller's stream wait for it, and the copy is marked as used by that
    stream so the caching allocator keeps its memory until the stream's work
    is done, even if the entry is evicted meanwhile.  An entry leaves when its
    source tensor is freed (``weakref.finalize``) or, least recently used
    first, when the cache is full.
    """

    def __init__(self, capacity: int = 16):
        self.capacity = capacity
        self.entries = collections.OrderedDict()
        # id(source) -> (weakref, finalizer): one finalizer per live source
        # tensor, however often its entry is replaced (in-place updates) or
        # evicted and made again
        self._fins = {}
        self._lock = threading.Lock()

    @staticmethod
    def _sig(t: torch.Tensor):
        return (t._version, t.data_ptr(), tuple(t.shape), t.device)

    def _drop(self, key, ref):
        with self._lock:
            e = self.entries.get(key)
            if e is not None and e[0] is ref:
                del self.entries[key]
            f = self._fins.get(key)
            if f is not None and f[0] is ref:
                del self._fins[key]

    def get(self, t: torch.Tensor, stream) -> torch.Tensor:
        use = torch.cuda.current_stream(t.device) if stream is None else stream
        key = id(t)
        with self._lock:
            e = self.entries.get(key)
            if e is not None and e[0]() is t and e[1] == self._sig(t):
                self.entries.move_to_end(key)
                out, done = e[2], e[3]
            else:
                out = None
        if out is not None:
            use.wait_event(done)
            out.record_stream(use)
            return out
        out = repack_w4_ref(t, stream)
        done = torch.cuda.Event()
        done.record(use)
        with self._lock:
            f = self._fins.get(key)
            if f is not None and f[0]() is t and f[1].alive:
                ref = f[0]
            else:
                ref = weakref.ref(t)
                self._fins[key] = (ref, weakref.finalize(t, self._drop, key, ref))
            self.entries[key] = (ref, self._sig(t), out, done)
            self.entries.move_to_end(key)
            while len(self.entries) > self.capacity:
                self.entries.popitem(last=False)
        return out


_repack_cache = _RepackCache()


def w4a8_linear_packed(x: torch.Tensor, w4_nk: torch.Tensor, scale_w: torch.Tensor,
                       stream=None) -> torch.Tensor:
    """W4A8 linear on weights already in the library layout [N, K/2]."""
    fn = "w4a8_linear"
    dev = _require_gpu(fn, x, w4_nk, scale_w)
    _check_2d(fn, "x", x, "[M,K]")
    M, K = x.shape
    N = w4_nk.shape[0]
    if K % 2 or w4_nk.shape[1] * 2 != K:
        raise ValueError(f"{fn}: x is [M,{K}] but packed weights hold K={2 * w4_nk.shape[1]}")
    if scale_w.numel() != N:
        raise ValueError(f"{fn}: scale_w has {scale_w.numel()} elements, expected N={N}")
    out_dtype = x.dtype
    lib = _lib.load()
    with _on_stream(dev, stream):
        xh = _as(x, torch.float16)
        sw = _as(scale_w.reshape(-1), torch.float32)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = _workspace(_lib.CIDER_OP_W4A8, M, N, K, 0, dev)
        _lib.check(lib.cider_w4a8_linear(_ptr(xh), _ptr(w4_nk), _ptr(sw), _ptr(y), _ptr(ws),
                                         _nbytes(ws), M, N, K, _stream_ptr(dev, stream)))
    return _cast_out(y, out_dtype)


def w4a8_linear(x: torch.Tensor, packed_w: torch.Tensor, scale_w: torch.Tensor,
                stream=None) -> torch.Tensor:
    """W4A8 linear (``cider/ops.py:212-235``): packed_w uint8 [K/2, N] in the
    reference layout (high nibble = even k, zero point 8), scale_w float32 [N],
    no bias.  Always quantize + GEMM, M == 1 included
    (``csrc/src/w4a8_primitive.mm:175-264``).  The weight is repacked to the
    library layout once and cached while the tensor is unchanged."""
    fn = "w4a8_linear"
    _require_gpu(fn, x, packed_w, scale_w)
    _check_2d(fn, "x", x, "[M,K]")
    _check_2d(fn, "packed_w", packed_w, "[K/2,N]")
    if packed_w.shape[0] * 2 != x.shape[1]:
        raise ValueError(f"{fn}: x is [M,{x.shape[1]}] but packed_w is "
                         f"{list(packed_w.shape)} ([K/2,N])")
    w4 = _repack_cache.get(packed_w, stream)
    return w4a8_linear_packed(x, w4, scale_w, stream)


def w4a8_pergroup_linear(x: torch.Tensor, w4_nk: torch.Tensor, scales: torch.Tensor,
                         group_size: int, bias: Optional[torch.Tensor] = None,
                         stream=None) -> torch.Tensor:
    """W4A8 per-group linear (extension): w4_nk uint8 [N, K/2] low nibble first,
    scales float16 [K // group_size, N], group_size in {64, 128}."""
    fn = "w4a8_pergroup_linear"
    dev = _require_gpu(fn, x, w4_nk, scales, bias)
    _check_2d(fn, "x", x, "[M,K]")
    _check_2d(fn, "w4_nk", w4_nk, "[N,K/2]")
    if group_size not in (64, 128):
        raise ValueError(f"{fn}: group_size must be 64 or 128")
    M, K = x.shape
    N = w4_nk.shape[0]
    if w4_nk.shape[1] * 2 != K or K % group_size:
        raise ValueError(f"{fn}: inconsistent K (x has {K}, weights {2 * w4_nk.shape[1]})")
    if tuple(scales.shape) != (K // group_size, N):
        raise ValueError(f"{fn}: scales is {tuple(scales.shape)}, expected [{K // group_size},{N}]")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"{fn}: bias has {bias.numel()} elements, expected N={N}")
    out_dtype = x.dtype
    lib = _lib.load()
    with _on_stream(dev, stream):
        xh = _as(x, torch.float16)
        w4 = _as(w4_nk, torch.uint8)
        sc = _as(scales, torch.float16)
        b = None if bias is None else _as(bias.reshape(-1), torch.float16)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = _workspace(_lib.CIDER_OP_W4A8_PERGROUP, M, N, K, group_size, dev)
        _lib.check(lib.cider_w4a8_pergroup_linear(
            _ptr(xh), _ptr(w4), _ptr(sc), _ptr(b), _ptr(y), _ptr(ws), _nbytes(ws),
            M, N, K, group_size, _stream_ptr(dev, stream)))
    return _cast_out(y, out_dtype)


def int8_matmul_int32(a: torch.Tensor, b: torch.Tensor, stream=None) -> torch.Tensor:
    """Raw int8 x int8 -> int32 matmul, b given as [N, K]
    (``cider/ops.py:238-255``).  Returns int32 [M, N], bit-exact."""
    fn = "int8_matmul_int32"
    dev = _require_gpu(fn, a, b)
    _check_2d(fn, "a", a, "[M,K]")
    _check_2d(fn, "b", b, "[N,K]")
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError(f"{fn}: a is [M,{K}] but b is [{N},{b.shape[1]}]")
    lib = _lib.load()
    with _on_stream(dev, stream):
        aa = _as(a, torch.int8)
        bb = _as(b, torch.int8)
        c = torch.empty((M, N), dtype=torch.int32, device=dev)
        _lib.check(lib.cider_int8_matmul_int32(_ptr(aa), _ptr(bb), _ptr(c), M, N, K,
                                               _stream_ptr(dev, stream)))
    return c

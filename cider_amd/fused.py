"""Producers of the W8A8 linear's input, with the per-token quantization fused
in, prefill-chunk and single-query decode attention (HIP kernels behind the C ABI of
``include/cider_hip.h``: ``cider_rmsnorm_quantize``, ``cider_silu_mul_quantize``,
``cider_qk_norm_rope``, ``cider_attn_decode``, ``cider_attn_prefill``,
``cider_attn_prefill_quantize``, the last one the attention as the producer of
the o projection's input).

The reference library quantizes a linear's fp16 input inside the linear
(``cider/kernels/w8a8_quantize.metal:17-87``); its models produce that input
with MLX ops (RMSNorm before q/k/v and gate/up, SwiGLU before down_proj,
``cider/fused_hybrid.py:209``).  Here the producer kernel ends in the same
quantization, and hands ``(q, scale_a)`` to ``ops.perchannel_gemm``: q and
scale_a are bit-identical to ``ops.quantize_per_token`` applied to the fp16
output the producer computes.

Every function runs on the GPU only; there is no CPU path.
"""

from __future__ import annotations

import collections
from typing import Optional

import torch

from . import _lib
from .ops import _on_stream, _ptr, _require_gpu, _stream_ptr

Normed = collections.namedtuple("Normed", "y q scale_a h")


def _f16(fn: str, name: str, t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.float16 or not t.is_contiguous():
        raise ValueError(f"{fn}: {name} must be a contiguous float16 tensor")
    return t


def rmsnorm_quantize(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                     add: Optional[torch.Tensor] = None, sum_out: Optional[torch.Tensor] = None,
                     want_y: bool = True, want_q: bool = True, stream=None) -> Normed:
    """RMSNorm of x [M, K] (fp16) by weight [K], optionally after a residual add.

    With ``add``, h = fp16(x + add) is written to ``sum_out`` (a new tensor if
    None; may be ``x`` itself) and normalised.  Returns ``Normed(y, q,
    scale_a, h)``: y fp16 [M, K] if want_y, q int8 [M, K] and scale_a fp32 [M]
    if want_q, h the summed input (x when no add).
    """
    fn = "rmsnorm_quantize"
    dev = _require_gpu(fn, x, weight, add, sum_out)
    if x.dim() != 2:
        raise ValueError(f"{fn}: x must be 2D [M,K]")
    M, K = x.shape
    _f16(fn, "x", x)
    _f16(fn, "weight", weight)
    if weight.numel() != K:
        raise ValueError(f"{fn}: weight has {weight.numel()} elements, expected K={K}")
    if add is not None:
        _f16(fn, "add", add)
        if add.shape != x.shape:
            raise ValueError(f"{fn}: add is {tuple(add.shape)}, x is {tuple(x.shape)}")
    lib = _lib.load()
    with _on_stream(dev, stream):
        h = None
        if add is not None:
            h = torch.empty_like(x) if sum_out is None else _f16(fn, "sum_out", sum_out)
            if h.shape != x.shape:
                raise ValueError(f"{fn}: sum_out has the wrong shape")
        y = torch.empty_like(x) if want_y else None
        q = torch.empty((M, K), dtype=torch.int8, device=dev) if want_q else None
        sa = torch.empty((M,), dtype=torch.float32, device=dev) if want_q else None
        _lib.check(lib.cider_rmsnorm_quantize(_ptr(x), _ptr(add), _ptr(h), _ptr(weight),
                                              float(eps), _ptr(y), _ptr(q), _ptr(sa), M, K,
                                              _stream_ptr(dev, stream)))
    return Normed(y, q, sa, x if h is None else h)


def silu_mul_quantize(gate_up: torch.Tensor, want_y: bool = True, want_q: bool = True,
                      stream=None):
    """SwiGLU of the fused gate+up output [M, 2I] (gate first).  Returns
    (y fp16 [M, I] or None, q int8 [M, I] or None, scale_a fp32 [M] or None)."""
    fn = "silu_mul_quantize"
    dev = _require_gpu(fn, gate_up)
    if gate_up.dim() != 2 or gate_up.shape[1] % 2 != 0:
        raise ValueError(f"{fn}: gate_up must be 2D [M, 2I]")
    _f16(fn, "gate_up", gate_up)
    M, I2 = gate_up.shape
    I = I2 // 2
    lib = _lib.load()
    with _on_stream(dev, stream):
        y = torch.empty((M, I), dtype=torch.float16, device=dev) if want_y else None
        q = torch.empty((M, I), dtype=torch.int8, device=dev) if want_q else None
        sa = torch.empty((M,), dtype=torch.float32, device=dev) if want_q else None
        _lib.check(lib.cider_silu_mul_quantize(_ptr(gate_up), _ptr(y), _ptr(q), _ptr(sa), M, I,
                                               _stream_ptr(dev, stream)))
    return y, q, sa


def qk_norm_rope(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                 eps: float, cos: torch.Tensor, sin: torch.Tensor, rope_row: torch.Tensor,
                 slot: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 num_heads: int, num_kv_heads: int, q_out: Optional[torch.Tensor] = None,
                 stream=None) -> torch.Tensor:
    """Per-head q/k RMSNorm + rotate-half RoPE over a fused projection
    qkv [L, (H + 2 KV) * 128]; k and v go into the caches (k_cache and
    v_cache, both [KV, T, 128]) at positions ``slot`` (int64 [L]); cos / sin are
    fp16 tables [P, 128] read at rows ``rope_row`` (int64 [L]).  Returns q
    [L, H, 128]."""
    fn = "qk_norm_rope"
    dev = _require_gpu(fn, qkv, q_norm_w, k_norm_w, cos, sin, rope_row, slot, k_cache, v_cache)
    D = 128
    H, KV = int(num_heads), int(num_kv_heads)
    if qkv.dim() != 2 or qkv.shape[1] != (H + 2 * KV) * D:
        raise ValueError(f"{fn}: qkv must be [L, {(H + 2 * KV) * D}]")
    for name, t in (("qkv", qkv), ("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("cos", cos),
                    ("sin", sin), ("k_cache", k_cache), ("v_cache", v_cache)):
        _f16(fn, name, t)
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != D:
        raise ValueError(f"{fn}: cos and sin must be [P, {D}]")
    if k_cache.dim() != 3 or k_cache.shape[0] != KV or k_cache.shape[2] != D:
        raise ValueError(f"{fn}: k_cache must be [{KV}, T, {D}]")
    T = k_cache.shape[1]
    if tuple(v_cache.shape) != (KV, T, D):
        raise ValueError(f"{fn}: v_cache must be [{KV}, {T}, {D}]")
    L = qkv.shape[0]
    for name, t in (("rope_row", rope_row), ("slot", slot)):
        if t.dtype != torch.int64 or t.numel() != L or not t.is_contiguous():
            raise ValueError(f"{fn}: {name} must be a contiguous int64 tensor of {L} elements")
    lib = _lib.load()
    with _on_stream(dev, stream):
        if q_out is None:
            q_out = torch.empty((L, H, D), dtype=torch.float16, device=dev)
        _lib.check(lib.cider_qk_norm_rope(
            _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), float(eps), _ptr(cos), _ptr(sin),
            cos.shape[0], _ptr(rope_row), _ptr(slot), _ptr(q_out), _ptr(k_cache),
            _ptr(v_cache), L, H, KV, D, T, _stream_ptr(dev, stream)))
    return q_out


def attn_decode_workspace(num_heads: int, capacity: int, device) -> torch.Tensor:
    nbytes = _lib.load().cider_attn_decode_workspace_bytes(num_heads, capacity)
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


def attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                n_valid: torch.Tensor, scale: float, ws: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Single-query grouped-query attention: q [H, 128] (or [1, H, 128])
    against the first n = n_valid[0] positions of k_cache and v_cache (both
    [KV, T, 128]).  Returns fp16 [H * 128]."""
    fn = "attn_decode"
    dev = _require_gpu(fn, q, k_cache, v_cache, n_valid, ws, out)
    D = 128
    _f16(fn, "q", q)
    H = q.numel() // D
    if q.numel() != H * D:
        raise ValueError(f"{fn}: q must hold H x {D} values")
    KV, T, d = k_cache.shape
    if tuple(v_cache.shape) != (KV, T, d):
        raise ValueError(f"{fn}: v_cache must match k_cache [KV, T, {d}]")
    if n_valid.dtype != torch.int64 or n_valid.numel() < 1:
        raise ValueError(f"{fn}: n_valid must be an int64 tensor")
    lib = _lib.load()
    with _on_stream(dev, stream):
        if ws is None:
            ws = attn_decode_workspace(H, T, dev)
        if out is None:
            out = torch.empty(H * D, dtype=torch.float16, device=dev)
        _lib.check(lib.cider_attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(n_valid),
                                         float(scale), _ptr(ws), ws.numel(), _ptr(out), H, KV, d,
                                         T, _stream_ptr(dev, stream)))
    return out


def attn_prefill_workspace(c: int, n: int, num_heads: int, device) -> Optional[torch.Tensor]:
    """The workspace a chunk of c queries over n slots splits its keys into
    (None when the launch does not split)."""
    nbytes = _lib.load().cider_attn_prefill_workspace_bytes(c, n, num_heads)
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def attn_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, n: int,
                 scale: float, out: Optional[torch.Tensor] = None,
                 ws: Optional[torch.Tensor] = None, split: bool = True,
                 n_dev: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Causal grouped-query attention of a prefill chunk: q [c, H, 128] holds
    the queries of cache slots n - c .. n - 1, whose keys and values are
    already in k_cache / v_cache [KV, T, 128]; query i attends slots
    0 .. n - c + i.  Returns fp16 [c, H * 128] (the reference hands this to
    MLX's fused SDPA, ``cider/fused_hybrid.py:179-196``).  A launch with few
    query blocks splits its keys over several workgroups into a workspace
    (allocated here unless ``ws`` is given); ``split=False`` runs unsplit.
    ``n_dev`` (int64 [1] on the device): the length is read there, clamped to
    [c, n], with n its upper bound -- for a call captured in a graph that
    serves chunks at any cache offset."""
    fn = "attn_prefill"
    dev = _require_gpu(fn, q, k_cache, v_cache, out, ws, n_dev)
    if n_dev is not None and (n_dev.dtype != torch.int64 or n_dev.numel() < 1):
        raise ValueError(f"{fn}: n_dev must be an int64 tensor")
    _f16(fn, "q", q)
    _f16(fn, "k_cache", k_cache)
    _f16(fn, "v_cache", v_cache)
    if q.dim() != 3:
        raise ValueError(f"{fn}: q must be [c, H, D]")
    c, H, D = q.shape
    KV, T, d = k_cache.shape
    if tuple(v_cache.shape) != (KV, T, d) or d != D:
        raise ValueError(f"{fn}: the caches must be [KV, T, {D}]")
    lib = _lib.load()
    with _on_stream(dev, stream):
        if out is None:
            out = torch.empty(c, H * D, dtype=torch.float16, device=dev)
        elif out.dtype != torch.float16 or not out.is_contiguous() or out.numel() != c * H * D:
            raise ValueError(f"{fn}: out must be a contiguous float16 tensor of c x H x {D}")
        if ws is None and split:
            ws = attn_prefill_workspace(c, int(n), H, dev)
        wsp, wsb = (_ptr(ws), ws.numel()) if (ws is not None and split) else (None, 0)
        _lib.check(lib.cider_attn_prefill(_ptr(q), _ptr(k_cache), _ptr(v_cache), float(scale),
                                          wsp, wsb, _ptr(out), c, int(n), _ptr(n_dev), H, KV, D,
                                          T, _stream_ptr(dev, stream)))
    return out


def attn_prefill_quantize_workspace(c: int, n: int, num_heads: int, device) -> torch.Tensor:
    """The workspace of ``attn_prefill_quantize`` for a chunk of c queries over
    n slots: the key parts' partials when the launch splits, else the fp16
    output before its quantization."""
    nbytes = _lib.load().cider_attn_prefill_quantize_workspace_bytes(c, n, num_heads)
    if nbytes == 0:
        raise ValueError(f"attn_prefill_quantize: unsupported shape c={c} n={n} H={num_heads}")
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def attn_prefill_quantize(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, n: int,
                          scale: float, ws: Optional[torch.Tensor] = None,
                          n_dev: Optional[torch.Tensor] = None, stream=None):
    """``attn_prefill`` with its output quantized per token for the o
    projection: returns (q int8 [c, H * 128], scale_a fp32 [c]), bit-identical
    to ``ops.quantize_per_token`` of ``attn_prefill``'s output, for
    ``CiderLinear.forward_quantized``.  A launch that splits its keys
    quantizes where it merges the parts, with no fp16 output in HBM.  ``ws``:
    ``attn_prefill_quantize_workspace(c, n, H)`` (allocated here if None)."""
    fn = "attn_prefill_quantize"
    dev = _require_gpu(fn, q, k_cache, v_cache, ws, n_dev)
    if n_dev is not None and (n_dev.dtype != torch.int64 or n_dev.numel() < 1):
        raise ValueError(f"{fn}: n_dev must be an int64 tensor")
    _f16(fn, "q", q)
    _f16(fn, "k_cache", k_cache)
    _f16(fn, "v_cache", v_cache)
    if q.dim() != 3:
        raise ValueError(f"{fn}: q must be [c, H, D]")
    c, H, D = q.shape
    KV, T, d = k_cache.shape
    if tuple(v_cache.shape) != (KV, T, d) or d != D:
        raise ValueError(f"{fn}: the caches must be [KV, T, {D}]")
    lib = _lib.load()
    with _on_stream(dev, stream):
        if ws is None:
            ws = attn_prefill_quantize_workspace(c, int(n), H, dev)
        qo = torch.empty(c, H * D, dtype=torch.int8, device=dev)
        sa = torch.empty(c, dtype=torch.float32, device=dev)
        _lib.check(lib.cider_attn_prefill_quantize(_ptr(q), _ptr(k_cache), _ptr(v_cache),
                                                   float(scale), _ptr(ws), ws.numel(), _ptr(qo),
                                                   _ptr(sa), c, int(n), _ptr(n_dev), H, KV, D, T,
                                                   _stream_ptr(dev, stream)))
    return qo, sa


def _mv_linear(fn: str, linear, K: int):
    """(w_int8, scale_w, bias, N) of a per-channel int8 CiderLinear with in_features K."""
    if getattr(linear, "group_size", None) != 0 or not hasattr(linear, "w_int8"):
        raise ValueError(f"{fn}: linear must be a per-channel int8 CiderLinear")
    N, Kw = linear.w_int8.shape
    if Kw != K:
        raise ValueError(f"{fn}: linear takes K={Kw}, the input has K={K}")
    return linear.w_int8, linear.scale_w, linear.bias, N


def rmsnorm_mv(x: torch.Tensor, weight: torch.Tensor, eps: float, linear,
               add: Optional[torch.Tensor] = None, stream=None):
    """Decode (one token): ``linear(RMSNorm(h))`` in one launch, with
    h = x, or h = fp16(x + add) when ``add`` is given.  Bit-identical to
    ``linear(rmsnorm_quantize(x, weight, eps, add).y)``.  Returns (h, y): h
    [1, K] (a new tensor when add is given, else x) and y [1, N] fp16.  x and
    add are [1, K] or [K] fp16; linear is a per-channel int8 CiderLinear."""
    fn = "rmsnorm_mv"
    dev = _require_gpu(fn, x, weight, add)
    K = x.numel()
    _f16(fn, "x", x)
    _f16(fn, "weight", weight)
    if weight.numel() != K:
        raise ValueError(f"{fn}: weight has {weight.numel()} elements, expected K={K}")
    if add is not None:
        _f16(fn, "add", add)
        if add.numel() != K:
            raise ValueError(f"{fn}: add has {add.numel()} elements, x has {K}")
    w, sw, bias, N = _mv_linear(fn, linear, K)
    lib = _lib.load()
    with _on_stream(dev, stream):
        h = torch.empty((1, K), dtype=torch.float16, device=dev) if add is not None else None
        y = torch.empty((1, N), dtype=torch.float16, device=dev)
        _lib.check(lib.cider_rmsnorm_mv(_ptr(x), _ptr(add), _ptr(h), _ptr(weight), float(eps),
                                        _ptr(w), _ptr(sw), _ptr(bias), _ptr(y), N, K,
                                        _stream_ptr(dev, stream)))
    return (x.reshape(1, K) if h is None else h), y


def swiglu_mv(gate_up: torch.Tensor, linear, stream=None) -> torch.Tensor:
    """Decode (one token): ``linear(SwiGLU(gate_up))`` in one launch, gate_up
    [1, 2I] (gate first).  Bit-identical to
    ``linear(silu_mul_quantize(gate_up, want_q=False)[0])``.  Returns y [1, N]."""
    fn = "swiglu_mv"
    dev = _require_gpu(fn, gate_up)
    _f16(fn, "gate_up", gate_up)
    if gate_up.numel() % 2:
        raise ValueError(f"{fn}: gate_up must hold [gate | up] of equal halves")
    K = gate_up.numel() // 2
    w, sw, bias, N = _mv_linear(fn, linear, K)
    lib = _lib.load()
    with _on_stream(dev, stream):
        y = torch.empty((1, N), dtype=torch.float16, device=dev)
        _lib.check(lib.cider_swiglu_mv(_ptr(gate_up), _ptr(w), _ptr(sw), _ptr(bias), _ptr(y),
                                       N, K, _stream_ptr(dev, stream)))
    return y

"""cider_amd.nn - quantized Linear modules (drop-in for ``cider/nn.py``).

``CiderLinear`` holds one copy of the weights: int8 [N, K] plus fp32 scales,
per-channel ([N]) or per-group ([K // group_size, N], the reference's
transposed layout, ``cider/nn.py:85-89,166``).  Its forward flattens the
leading dimensions, calls ``ops.perchannel_linear`` / ``ops.pergroup_linear``
(which dispatch M == 1 to the MV and M >= 2 to quantize + GEMM) and restores
the shape (``cider/nn.py:102-113``).  ``W8A8Linear`` is an alias, as in the
reference (``cider/nn.py:212``).  ``W4A8Linear`` holds reference-layout packed
int4 weights (``cider/nn.py:216-241``) and keeps a repacked copy in the
library layout, made on its first forward on the GPU and made again when the
packed weights change (in-place update, ``load_state_dict``).
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import _lib, ops


def set_mode(mode: str):
    """No-op, kept for compatibility (``cider/nn.py:24-26``)."""


def get_mode() -> str:
    """Always 'auto' (``cider/nn.py:28-30``)."""
    return "auto"


def _symmetric_quantize_pergroup(w_fp: np.ndarray, group_size: int):
    """[N, K] float -> (int8 [N, K], fp32 [N, K // group_size]) (``cider/nn.py:34-59``)."""
    return ops.quantize_weight_pergroup(w_fp, group_size)


def _device_of(*ts) -> torch.device:
    for t in ts:
        if isinstance(t, torch.Tensor):
            return t.device
    return torch.device("cpu")


class CiderLinear(torch.nn.Module):
    """INT8 linear: prefill (M >= 2) runs W8A8 quantize + int8 GEMM, decode
    (M == 1) the fp16-activation MV; per-channel (group_size 0) or per-group
    (64/128/256).  Mirrors ``cider/nn.py:63-208``."""

    def __init__(self, w_int8: torch.Tensor, scale_w: torch.Tensor, group_size: int,
                 in_features: int, out_features: int, bias: Optional[torch.Tensor] = None):
        super().__init__()
        if group_size == 0:
            self._mode = "per_channel"
        elif group_size in (64, 128, 256):
            self._mode = "per_group"
        else:
            raise ValueError(
                f"Unsupported group_size={group_size}. Use 0 (per-channel) or 64/128/256.")
        dev = _device_of(w_int8, scale_w)
        self.register_buffer("w_int8", torch.as_tensor(w_int8, dtype=torch.int8, device=dev)
                             .contiguous())
        self.register_buffer("scale_w", torch.as_tensor(scale_w, dtype=torch.float32, device=dev)
                             .contiguous())
        if bias is None:
            bias = torch.zeros(out_features, dtype=torch.float16, device=dev)
        self.register_buffer("bias", torch.as_tensor(bias, device=dev).to(torch.float16)
                             .contiguous())
        self.group_size = group_size
        self._in_features = in_features
        self._out_features = out_features
        self._ws_cache = {}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x2 = x.reshape(-1, self._in_features)
        if (self._mode == "per_channel" and x2.dtype == torch.float16 and x2.is_cuda
                and x2.is_contiguous() and x2.device == self.w_int8.device):
            y = self._perchannel_direct(x2)
        elif self._mode == "per_channel":
            y = ops.perchannel_linear(x2, self.w_int8, self.scale_w, self.bias)
        else:
            y = ops.pergroup_linear(x2, self.w_int8, self.scale_w, self.group_size, self.bias)
        return y.reshape(*orig_shape[:-1], self._out_features)

    def _perchannel_direct(self, x2: torch.Tensor) -> torch.Tensor:
        """Per-channel call straight into the C ABI for the common case (fp16,
        contiguous, same device): the buffers are already in the library's
        types, so only the output and the workspace are allocated.  The
        launch goes to the current stream, so it can be captured in a graph."""
        lib = _lib.load()
        M = x2.shape[0]
        N, K = self._out_features, self._in_features
        dev = x2.device
        nb = self._ws_cache.get(M)
        if nb is None:
            nb = _lib.workspace_bytes(_lib.CIDER_OP_PERCHANNEL, M, N, K, 0)
            self._ws_cache[M] = nb
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev) if nb else None
        rc = lib.cider_perchannel_linear(
            x2.data_ptr(), self.w_int8.data_ptr(), self.scale_w.data_ptr(), self.bias.data_ptr(),
            y.data_ptr(), ws.data_ptr() if ws is not None else None, nb, M, N, K,
            torch.cuda.current_stream(dev).cuda_stream)
        if rc != 0:
            _lib.check(rc)
        return y

    def forward_quantized(self, q: torch.Tensor, scale_a: torch.Tensor) -> torch.Tensor:
        """Per-channel linear on activations already quantized per token
        (q int8 [M, K], scale_a fp32 [M]), as a producer kernel with the
        quantization fused in hands them over (``cider_amd.fused``).  Equal to
        ``forward`` on the fp16 tensor that q and scale_a were quantized from
        (for M >= 2, where ``forward`` quantizes too)."""
        if self._mode != "per_channel":
            raise ValueError("forward_quantized: per-channel layers only")
        M, K = q.shape
        if K != self._in_features or scale_a.numel() != M:
            raise ValueError("forward_quantized: q / scale_a do not match the layer")
        lib = _lib.load()
        N = self._out_features
        y = torch.empty((M, N), dtype=torch.float16, device=q.device)
        rc = lib.cider_perchannel_gemm(
            q.data_ptr(), scale_a.data_ptr(), self.w_int8.data_ptr(), self.scale_w.data_ptr(),
            self.bias.data_ptr(), y.data_ptr(), M, N, K,
            torch.cuda.current_stream(q.device).cuda_stream)
        if rc != 0:
            _lib.check(rc)
        return y

    @staticmethod
    def from_float(layer: torch.nn.Module, target_group_size: Optional[int] = None,
                   device=None) -> "CiderLinear":
        """From a ``torch.nn.Linear`` (or any module with ``weight`` [N, K] and
        optional ``bias``): symmetric requant, per-channel unless
        ``target_group_size`` is given (``cider/nn.py:173-192``).  An
        MLX-style affine-quantized layer (``weight`` words, ``scales``,
        ``biases``, ``group_size``, ``bits``) is dequantized and requantized
        as ``cider/nn.py:127-171`` does (``cider_amd.ingest.from_affine``)."""
        if hasattr(layer, "scales") and hasattr(layer, "bits"):
            from .ingest import from_affine
            return from_affine(layer, target_group_size, device)
        if not hasattr(layer, "weight"):
            raise TypeError(f"Unsupported layer: {type(layer)}")
        weight = layer.weight.detach()
        out_f, in_f = weight.shape
        dev = device if device is not None else weight.device
        lin_bias = getattr(layer, "bias", None)
        if lin_bias is not None:
            lin_bias = lin_bias.detach().to(device=dev, dtype=torch.float16)
        tgs = target_group_size or 0
        w_np = weight.to(torch.float32).cpu().numpy()
        if tgs == 0:
            q, s = ops.quantize_weight_int8(w_np)
        else:
            q, s = _symmetric_quantize_pergroup(w_np, tgs)
            s = np.ascontiguousarray(s.T)  # [N, G] -> [G, N]
        return CiderLinear(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), tgs,
                           in_f, out_f, lin_bias)

    @property
    def in_features(self) -> int:
        return self._in_features

    @property
    def out_features(self) -> int:
        return self._out_features

    @property
    def input_dims(self) -> int:
        return self._in_features

    @property
    def output_dims(self) -> int:
        return self._out_features

    def extra_repr(self) -> str:
        return (f"in={self._in_features}, out={self._out_features}, mode={self._mode}, "
                f"gs={self.group_size}")

    def __repr__(self):
        return f"CiderLinear({self.extra_repr()})"


W8A8Linear = CiderLinear


class W4A8Linear(torch.nn.Module):
    """Packed int4 weight x int8 activation linear (``cider/nn.py:216-241``).

    ``packed_weight`` uint8 [K/2, N] (reference layout), ``scale`` fp32 [N]."""

    def __init__(self, packed_weight: torch.Tensor, scale: torch.Tensor, K: int):
        super().__init__()
        dev = _device_of(packed_weight, scale)
        self.register_buffer("packed_weight",
                             torch.as_tensor(packed_weight, dtype=torch.uint8, device=dev)
                             .contiguous())
        self.register_buffer("scale", torch.as_tensor(scale, dtype=torch.float32, device=dev)
                             .contiguous())
        self._K = K
        # library layout, made on first use on the GPU; valid for the
        # (version, address, shape, device) of packed_weight it was made from.
        # _w4_done: event recorded after the repack on the stream that made it
        self._w4_nk = None
        self._w4_sig = None
        self._w4_done = None

    def _packed_nk(self) -> torch.Tensor:
        """The library-layout copy, ordered for the current stream: a repack
        runs on the calling stream and records an event; every use waits for
        that event on its own stream and marks the copy as used there, so the
        caching allocator keeps the memory until that stream's work is done
        even after a later repack replaces the copy."""
        w = self.packed_weight
        use = torch.cuda.current_stream(w.device)
        sig = (w._version, w.data_ptr(), tuple(w.shape), w.device)
        if self._w4_nk is None or self._w4_sig != sig:
            out = ops.repack_w4_ref(w)
            done = torch.cuda.Event()
            done.record(use)
            self._w4_nk, self._w4_sig, self._w4_done = out, sig, done
            return out
        use.wait_event(self._w4_done)
        self._w4_nk.record_stream(use)
        return self._w4_nk

    def _load_from_state_dict(self, *args, **kwargs):
        self._w4_nk = None
        self._w4_sig = None
        self._w4_done = None
        super()._load_from_state_dict(*args, **kwargs)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        y = ops.w4a8_linear_packed(x.reshape(-1, self._K), self._packed_nk(), self.scale)
        return y.reshape(*orig_shape[:-1], self.output_dims)

    @staticmethod
    def from_weights(w: np.ndarray, zero_point: int = 8, device=None) -> "W4A8Linear":
        """From an fp16/fp32 numpy weight [K, N] (``cider/nn.py:229-234``)."""
        K = w.shape[0]
        packed, scale = ops.pack_weight_int4(w, zero_point)
        dev = device if device is not None else ("cuda" if torch.cuda.is_available() else "cpu")
        return W4A8Linear(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev), K)

    @property
    def input_dims(self) -> int:
        return self._K

    @property
    def output_dims(self) -> int:
        return self.packed_weight.shape[1]


class W4A8GroupLinear(torch.nn.Module):
    """Per-group int4 weight x int8 activation linear (extension): packed
    [N, K/2] low nibble first, fp16 scales [K // group_size, N]."""

    def __init__(self, packed_nk: torch.Tensor, scales: torch.Tensor, group_size: int,
                 bias: Optional[torch.Tensor] = None):
        super().__init__()
        if group_size not in (64, 128):
            raise ValueError(f"Unsupported group_size={group_size}. Use 64 or 128.")
        dev = _device_of(packed_nk, scales)
        self.register_buffer("packed_weight", torch.as_tensor(packed_nk, dtype=torch.uint8,
                                                              device=dev).contiguous())
        self.register_buffer("scales", torch.as_tensor(scales, dtype=torch.float16, device=dev)
                             .contiguous())
        self.bias = None if bias is None else torch.as_tensor(bias, device=dev).half()
        self.group_size = group_size
        self._K = 2 * self.packed_weight.shape[1]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        y = ops.w4a8_pergroup_linear(x.reshape(-1, self._K), self.packed_weight, self.scales,
                                     self.group_size, self.bias)
        return y.reshape(*orig_shape[:-1], self.packed_weight.shape[0])

    @staticmethod
    def from_float(layer: torch.nn.Module, group_size: int = 128, device=None):
        weight = layer.weight.detach()
        dev = device if device is not None else weight.device
        packed, scales = ops.pack_weight_int4_pergroup(weight.float().cpu().numpy(), group_size)
        bias = getattr(layer, "bias", None)
        return W4A8GroupLinear(torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev),
                               group_size, None if bias is None else bias.detach().to(dev))

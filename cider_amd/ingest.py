"""cider_amd.ingest - weight ingestion: packed low-bit checkpoints into the
library's weight formats.

Two sources, both stored as 32-bit words holding ``32 / bits`` codes each,
code i of a word in bits ``[bits*i, bits*(i+1))`` (low bits first):

* **MLX affine-quantized linears** (what ``nn.QuantizedLinear`` holds:
  ``weight`` uint32 [N, K*bits/32], ``scales`` and ``biases`` [N, K/gs],
  ``group_size``, ``bits``), dequantized as ``w = q * scale + bias``
  (``cider/ops.py:171-173``).  ``CiderLinear.from_float`` turns such a layer
  into a symmetric int8 layer the way the reference does
  (``cider/nn.py:127-171``): dequantize, then requantize per group when the
  source is 8-bit with group size 64/128/256 (or ``target_group_size`` asks
  for it), per channel otherwise.  The reference calls ``mx.dequantize`` from
  MLX (>= 0.31, not vendored); this module restates the affine formula above
  in fp32.  No reference test pins MLX's own rounding of that formula, so
  this step's parity is unpinned; only ``32 % bits == 0`` packings (2, 4, 8
  bits) are accepted.

* **compressed-tensors "pack-quantized" checkpoints** (LLMCompressor), the
  format ``tools/convert_compressed_tensors_to_mlx.py:31-183`` reads: per
  quantized layer ``<name>.weight_packed`` int32 [N, K/(32/bits)],
  ``<name>.weight_scale`` [N, G] (G = 1 per channel), optional
  ``<name>.weight_shape`` [2] = (N, K); value = code - 2^(bits-1), weight =
  value * scale of its group; config.json ``quantization_config`` gives bits,
  group size and strategy; a layer's tensors may sit in different shards.
  ``load_compressed_tensors`` maps each layer straight onto a library format
  without requantization where one exists:
    - 8-bit, per channel or group 64/128/256 -> ``CiderLinear`` (int8 values
      exact, fp32 scales);
    - 4-bit, group 64/128 -> ``W4A8GroupLinear`` (int4 values exact, fp16
      scales, as the reference's converter also casts them);
    - 4-bit per channel -> ``W4A8Linear`` (reference W4 layout, fp32 scales);
    - anything else -> dequantized, then ``CiderLinear`` per-channel int8.

Files are read with safetensors (no pickle).  Everything here runs on the
host; the resulting modules run on the GPU.
"""

from __future__ import annotations

import dataclasses
import glob
import json
import os
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import ops
from .nn import CiderLinear, W4A8GroupLinear, W4A8Linear, _symmetric_quantize_pergroup


# --------------------------------------------------------------------------
# packed words
# --------------------------------------------------------------------------


def unpack_words(words: np.ndarray, bits: int, K: Optional[int] = None) -> np.ndarray:
    """[N, W] 32-bit words -> unsigned codes [N, K] (K = W * 32 / bits by
    default); code i of word w is element w * (32/bits) + i."""
    if bits not in (2, 4, 8):
        raise ValueError(f"unsupported bit width {bits}: words must hold whole codes")
    w = np.ascontiguousarray(words).view(np.uint32)
    per = 32 // bits
    mask = np.uint32((1 << bits) - 1)
    codes = np.empty(w.shape[:-1] + (w.shape[-1], per), dtype=np.uint8)
    for i in range(per):
        codes[..., i] = ((w >> np.uint32(bits * i)) & mask).astype(np.uint8)
    codes = codes.reshape(w.shape[:-1] + (w.shape[-1] * per,))
    if K is not None:
        if K > codes.shape[-1]:
            raise ValueError(f"K={K} exceeds the {codes.shape[-1]} packed codes")
        codes = codes[..., :K]
    return codes


def pack_words(codes: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of ``unpack_words`` (codes [N, K], K a multiple of 32/bits) ->
    uint32 words [N, K * bits / 32]."""
    if bits not in (2, 4, 8):
        raise ValueError(f"unsupported bit width {bits}")
    per = 32 // bits
    c = np.asarray(codes).astype(np.uint32)
    if c.shape[-1] % per:
        raise ValueError(f"K={c.shape[-1]} is not a multiple of {per}")
    c = c.reshape(c.shape[:-1] + (c.shape[-1] // per, per))
    out = np.zeros(c.shape[:-1], dtype=np.uint32)
    for i in range(per):
        out |= c[..., i] << np.uint32(bits * i)
    return out


def _expand_groups(s: np.ndarray, K: int) -> Tuple[np.ndarray, int]:
    """Per-row group values [N, G] -> [N, K] and the group size."""
    G = s.shape[1]
    if K % G:
        raise ValueError(f"K={K} is not a multiple of the {G} groups")
    gs = K // G
    return np.repeat(s, gs, axis=1), gs


# --------------------------------------------------------------------------
# MLX affine quantization
# --------------------------------------------------------------------------


@dataclasses.dataclass
class AffineQuantized:
    """The tensors of an MLX ``nn.QuantizedLinear``: ``weight`` uint32 words
    [N, K*bits/32], ``scales`` / ``biases`` [N, K/group_size], optional
    ``bias`` [N]."""

    weight: np.ndarray
    scales: np.ndarray
    biases: Optional[np.ndarray]
    group_size: int
    bits: int
    bias: Optional[np.ndarray] = None

    @property
    def out_features(self) -> int:
        return int(np.asarray(self.scales).shape[0])

    @property
    def in_features(self) -> int:
        return int(np.asarray(self.scales).shape[1]) * self.group_size


class QuantizedLinear(torch.nn.Module):
    """An affine-quantized linear layer as MLX's ``nn.QuantizedLinear`` holds
    it, on torch tensors: ``weight`` 32-bit words [N, K*bits/32] (int32
    storage of the uint32 words), ``scales`` and ``biases`` [N, K/group_size],
    ``group_size``, ``bits`` and an optional ``bias`` [N].

    It is the source layer ``convert_model`` and ``CiderLinear.from_float``
    convert, as the reference's converter does with ``nn.QuantizedLinear``
    (``cider/convert.py:25``, ``cider/nn.py:127-171``).  Its own forward
    dequantizes with torch ops (``w = q * scale + bias`` per group) and runs
    a floating-point matmul; it is the unconverted model, not a path of this
    library.
    """

    def __init__(self, weight, scales, biases, group_size: int, bits: int, bias=None):
        super().__init__()
        if bits not in (2, 4, 8):
            raise ValueError(f"unsupported bit width {bits}")
        w = torch.as_tensor(weight)
        if w.dtype != torch.int32:
            w = torch.from_numpy(np.ascontiguousarray(_np(w)).astype(np.uint32).view(np.int32))
        self.register_buffer("weight", w.contiguous())
        self.register_buffer("scales", torch.as_tensor(scales).contiguous())
        self.register_buffer("biases", None if biases is None
                             else torch.as_tensor(biases).contiguous())
        self.register_buffer("bias", None if bias is None else torch.as_tensor(bias).contiguous())
        self.group_size = int(group_size)
        self.bits = int(bits)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        per = 32 // self.bits
        words = self.weight.to(torch.int64) & 0xFFFFFFFF
        shifts = torch.arange(per, device=words.device, dtype=torch.int64) * self.bits
        q = ((words[..., None] >> shifts) & ((1 << self.bits) - 1)).reshape(words.shape[0], -1)
        K = self.scales.shape[1] * self.group_size
        s = self.scales.float().repeat_interleave(self.group_size, dim=1)
        w = q[:, :K].float() * s
        if self.biases is not None:
            w = w + self.biases.float().repeat_interleave(self.group_size, dim=1)
        b = None if self.bias is None else self.bias.to(x.dtype)
        return torch.nn.functional.linear(x, w.to(x.dtype), b)

    @property
    def out_features(self) -> int:
        return int(self.scales.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.scales.shape[1]) * self.group_size


def is_affine_quantized(layer) -> bool:
    """True for a layer holding affine-quantized weights (``QuantizedLinear``
    or any object with ``weight``, ``scales``, ``group_size`` and ``bits``)."""
    return all(hasattr(layer, a) for a in ("weight", "scales", "group_size", "bits"))


def affine_dequantize(weight, scales, biases, group_size: int, bits: int) -> np.ndarray:
    """w = q * scale + bias per group (fp32; biases None -> 0)."""
    s = np.asarray(scales, dtype=np.float32)
    N, G = s.shape
    K = G * group_size
    q = unpack_words(np.asarray(weight), bits, K).astype(np.float32)
    if q.shape[0] != N:
        raise ValueError("weight and scales disagree on the number of rows")
    se, _ = _expand_groups(s, K)
    w = q * se
    if biases is not None:
        be, _ = _expand_groups(np.asarray(biases, dtype=np.float32), K)
        w = w + be
    return w.astype(np.float32)


def from_affine(layer, target_group_size: Optional[int] = None, device=None) -> CiderLinear:
    """``CiderLinear`` from an MLX-style affine-quantized layer (any object
    with ``weight``, ``scales``, ``biases``, ``group_size``, ``bits`` and
    optionally ``bias``), as ``cider/nn.py:127-171`` converts
    ``nn.QuantizedLinear``: dequantize, then symmetric int8 per group
    (target_group_size, or the source's group size when it is 8-bit with
    gs in {64, 128, 256}) or per channel."""
    bits, gs = int(layer.bits), int(layer.group_size)
    scales = _np(layer.scales).astype(np.float32)
    out_f, in_f = scales.shape[0], scales.shape[1] * gs
    if target_group_size is not None:
        tgs = target_group_size
    elif bits == 8 and gs in (64, 128, 256):
        tgs = gs
    else:
        tgs = 0
    biases = getattr(layer, "biases", None)
    w = affine_dequantize(_np(layer.weight), scales, None if biases is None else _np(biases),
                          gs, bits)
    if device is not None:
        dev = torch.device(device)
    elif isinstance(layer.weight, torch.Tensor):
        dev = layer.weight.device
    else:
        dev = torch.device("cpu")
    lin_bias = getattr(layer, "bias", None)
    if lin_bias is not None:
        lin_bias = torch.as_tensor(_np(lin_bias)).to(device=dev, dtype=torch.float16)
    if tgs == 0:
        q, s = ops.quantize_weight_int8(w)
    else:
        q, s = _symmetric_quantize_pergroup(w, tgs)
        s = np.ascontiguousarray(s.T)  # [N, G] -> [G, N]
    return CiderLinear(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), tgs, in_f,
                       out_f, lin_bias)


def _np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            t = t.float()
        return t.numpy()
    return np.asarray(t)


# --------------------------------------------------------------------------
# compressed-tensors checkpoints
# --------------------------------------------------------------------------


@dataclasses.dataclass
class PackedLayer:
    """One compressed-tensors quantized layer."""

    name: str
    codes: np.ndarray        # unsigned codes [N, K]
    scale: np.ndarray        # fp32 [N, G] (G = 1: per channel)
    bits: int

    @property
    def shape(self) -> Tuple[int, int]:
        return self.codes.shape

    @property
    def values(self) -> np.ndarray:
        """Signed integer values [N, K] = code - 2^(bits-1)."""
        return self.codes.astype(np.int16) - (1 << (self.bits - 1))

    @property
    def group_size(self) -> int:
        """K for per-channel scales, else K / G."""
        return self.codes.shape[1] // self.scale.shape[1]

    def dequantize(self) -> np.ndarray:
        se, _ = _expand_groups(self.scale, self.codes.shape[1])
        return (self.values.astype(np.float32) * se).astype(np.float32)


def _read_config(model_dir: str) -> dict:
    with open(os.path.join(model_dir, "config.json")) as f:
        cfg = json.load(f)
    q = cfg.get("quantization_config", {})
    w = q.get("config_groups", {}).get("group_0", {}).get("weights", {})
    return {"bits": int(w.get("num_bits", 4)), "group_size": w.get("group_size"),
            "strategy": w.get("strategy", "group"), "symmetric": w.get("symmetric", True),
            "ignore": list(q.get("ignore", [])), "config": cfg}


def read_compressed_tensors(model_dir: str):
    """Reads every ``*.safetensors`` shard of a compressed-tensors model.
    Returns (layers {name: PackedLayer}, plain {key: torch.Tensor}, info)."""
    from safetensors.torch import load_file

    info = _read_config(model_dir)
    bits = info["bits"]
    files = sorted(glob.glob(os.path.join(model_dir, "model*.safetensors")))
    if not files:
        files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no .safetensors shards in {model_dir}")
    tensors: Dict[str, torch.Tensor] = {}
    for f in files:  # a layer's parts may sit in different shards
        tensors.update(load_file(f))
    parts: Dict[str, Dict[str, torch.Tensor]] = {}
    plain: Dict[str, torch.Tensor] = {}
    for key, t in tensors.items():
        for suffix, part in ((".weight_packed", "packed"), (".weight_scale", "scale"),
                             (".weight_shape", "shape")):
            if key.endswith(suffix):
                parts.setdefault(key[: -len(suffix)], {})[part] = t
                break
        else:
            plain[key] = t
    per_word = 32 // bits
    layers = {}
    for name, p in sorted(parts.items()):
        if "packed" not in p or "scale" not in p:
            raise ValueError(f"{name}: weight_packed and weight_scale are both required")
        packed = p["packed"].numpy()
        if "shape" in p:
            N, K = (int(v) for v in p["shape"].tolist())
        else:
            N, K = packed.shape[0], packed.shape[1] * per_word
        codes = unpack_words(packed, bits, K)
        if codes.shape[0] != N:
            raise ValueError(f"{name}: weight_shape says {N} rows, weight_packed has "
                             f"{codes.shape[0]}")
        scale = p["scale"].float().numpy().reshape(N, -1).astype(np.float32)
        if K % scale.shape[1]:
            raise ValueError(f"{name}: K={K} is not a multiple of {scale.shape[1]} groups")
        layers[name] = PackedLayer(name, codes, scale, bits)
    return layers, plain, info


def to_module(layer: PackedLayer, device=None) -> torch.nn.Module:
    """The library module for one packed layer (see the module docstring)."""
    dev = torch.device(device) if device is not None else torch.device("cpu")
    N, K = layer.shape
    G = layer.scale.shape[1]
    gs = K // G
    if layer.bits == 8 and (G == 1 or gs in (64, 128, 256)):
        q = layer.values.astype(np.int8)
        if G == 1:
            return CiderLinear(torch.from_numpy(q).to(dev),
                               torch.from_numpy(np.ascontiguousarray(layer.scale[:, 0])).to(dev),
                               0, K, N)
        return CiderLinear(torch.from_numpy(q).to(dev),
                           torch.from_numpy(np.ascontiguousarray(layer.scale.T)).to(dev),
                           gs, K, N)
    if layer.bits == 4 and G > 1 and gs in (64, 128) and K % 2 == 0:
        v = layer.values
        nib = (v & 0xF).astype(np.uint8)
        packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)       # [N, K/2]
        scales = np.ascontiguousarray(layer.scale.T).astype(np.float16)       # [G, N]
        return W4A8GroupLinear(torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev),
                               gs)
    if layer.bits == 4 and G == 1 and K % 2 == 0:
        nib = (layer.values + 8).astype(np.uint8).T                            # [K, N] in 0..15
        packed = ((nib[0::2, :] << 4) | nib[1::2, :]).astype(np.uint8)       # reference layout
        return W4A8Linear(torch.from_numpy(packed).to(dev),
                          torch.from_numpy(np.ascontiguousarray(layer.scale[:, 0])).to(dev), K)
    q, s = ops.quantize_weight_int8(layer.dequantize())
    return CiderLinear(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), 0, K, N)


def load_compressed_tensors(model_dir: str, device=None):
    """Reads a compressed-tensors checkpoint and builds one library module per
    quantized layer.  Returns (modules {name: Module}, plain {key: Tensor},
    info)."""
    layers, plain, info = read_compressed_tensors(model_dir)
    return {n: to_module(l, device) for n, l in layers.items()}, plain, info


def replace_modules(model: torch.nn.Module, modules: Dict[str, torch.nn.Module]) -> int:
    """Puts each module at its dotted path in ``model`` (replacing what is
    there, typically an ``nn.Linear``); returns how many were placed."""
    n = 0
    for name, mod in modules.items():
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, child, mod)
        n += 1
    return n

"""Weight ingestion (cider_amd/ingest.py): packed 32-bit words, the MLX
affine-quantized layer conversion of cider/nn.py:127-171, and compressed-tensors
checkpoints (the format of tools/convert_compressed_tensors_to_mlx.py:31-183)
mapped onto the library's weight formats.

The checkpoints are synthetic: a config.json and safetensors shards written
here with known codes and scales (the reference ships no checkpoint).  The
packing is pinned by brute-force bit extraction on small inputs; the mapped
library weights by the oracle's own unpackers of the library layouts.
MLX's rounding of its affine dequantization is not pinned by any reference
test (MLX is not vendored): that step is checked against its formula only.
"""

import json
import math

import numpy as np
import pytest
import torch

from cider_amd import ingest as I
from cider_amd import nn as cnn
from oracle import cider_oracle as O


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unpack_words_bit_by_bit(bits):
    rng = np.random.default_rng(bits)
    words = rng.integers(0, 2 ** 32, (3, 5), dtype=np.uint64).astype(np.uint32)
    codes = I.unpack_words(words, bits)
    per = 32 // bits
    assert codes.shape == (3, 5 * per)
    for r in range(3):
        for wi in range(5):
            w = int(words[r, wi])
            for i in range(per):
                exp = (w >> (bits * i)) & ((1 << bits) - 1)
                assert codes[r, wi * per + i] == exp
    assert np.array_equal(I.pack_words(codes, bits), words)
    # int32 words (compressed-tensors stores them signed) read the same bits
    assert np.array_equal(I.unpack_words(words.view(np.int32), bits), codes)
    # a K that does not fill the last word
    assert np.array_equal(I.unpack_words(words, bits, 5 * per - 3), codes[:, :-3])
    with pytest.raises(ValueError):
        I.unpack_words(words, 3)


def test_affine_dequantize_formula():
    rng = np.random.default_rng(1)
    N, K, gs, bits = 3, 64, 32, 4
    codes = rng.integers(0, 16, (N, K))
    scales = rng.uniform(0.01, 0.1, (N, K // gs)).astype(np.float32)
    biases = rng.uniform(-1, 1, (N, K // gs)).astype(np.float32)
    w = I.affine_dequantize(I.pack_words(codes, bits), scales, biases, gs, bits)
    for n in range(N):
        for k in range(K):
            exp = np.float32(codes[n, k]) * scales[n, k // gs] + biases[n, k // gs]
            assert w[n, k] == np.float32(exp)
    w0 = I.affine_dequantize(I.pack_words(codes, bits), scales, None, gs, bits)
    assert np.array_equal(w0, (codes * np.repeat(scales, gs, 1)).astype(np.float32))


def test_from_float_on_symmetric_8bit_affine_layer_keeps_the_values():
    """An 8-bit affine layer with biases = -128 * scale holds symmetric values
    v = q - 128 in [-127, 127] with one value per group at +-127: the
    reference's per-group requant (cider/nn.py:150-163) gives back exactly v
    and the source scales."""
    rng = np.random.default_rng(2)
    N, K, gs = 6, 256, 128
    v = rng.integers(-127, 128, (N, K))
    v[:, ::gs] = 127 * np.where(rng.random((N, K // gs)) < 0.5, 1, -1)
    scales = rng.uniform(1e-3, 1e-2, (N, K // gs)).astype(np.float32)
    layer = I.AffineQuantized(weight=I.pack_words(v + 128, 8), scales=scales,
                              biases=-128.0 * scales, group_size=gs, bits=8)
    m = cnn.CiderLinear.from_float(layer)
    assert m.group_size == gs and m.in_features == K and m.out_features == N
    assert np.array_equal(m.w_int8.numpy(), v.astype(np.int8))
    np.testing.assert_allclose(m.scale_w.numpy(), scales.T, rtol=2e-7)
    # 4-bit source: per-channel unless asked otherwise (cider/nn.py:137-142)
    l4 = I.AffineQuantized(weight=I.pack_words(rng.integers(0, 16, (N, K)), 4),
                           scales=scales, biases=-8.0 * scales, group_size=gs, bits=4)
    assert cnn.CiderLinear.from_float(l4).group_size == 0
    assert cnn.CiderLinear.from_float(l4, target_group_size=64).group_size == 64
    w = I.affine_dequantize(l4.weight, l4.scales, l4.biases, gs, 4)
    q, s = O.quantize_weight_int8(w)
    m4 = cnn.CiderLinear.from_float(l4)
    assert np.array_equal(m4.w_int8.numpy(), q) and np.array_equal(m4.scale_w.numpy(), s)


def test_quantized_linear_module_forward_and_conversion_walk():
    """The torch QuantizedLinear holds MLX's affine tensors; its float forward
    is the affine formula, and the conversion walk (cider/convert.py:28-47)
    replaces it, an nn.Linear and a duck-typed affine module, keeping the
    source's 8-bit group size as cider/nn.py:134-139 does."""
    from cider_amd import convert as cconv
    rng = np.random.default_rng(4)
    N, K, gs = 16, 256, 64
    codes = rng.integers(0, 256, (N, K))
    scales = rng.uniform(1e-3, 1e-2, (N, K // gs)).astype(np.float32)
    biases = (-128.0 * scales).astype(np.float32)
    words = I.pack_words(codes, 8)
    ql = I.QuantizedLinear(words, scales, biases, gs, 8)
    assert ql.in_features == K and ql.out_features == N
    assert ql.weight.dtype == torch.int32
    x = torch.from_numpy(rng.standard_normal((3, K)).astype(np.float32))
    w = I.affine_dequantize(words, scales, biases, gs, 8)
    np.testing.assert_allclose(ql(x).numpy(), x.numpy() @ w.T, rtol=1e-5, atol=1e-5)

    class Duck(torch.nn.Module):   # an affine layer of another class
        def __init__(self):
            super().__init__()
            self.weight = I.pack_words(rng.integers(0, 16, (8, 128)), 4)
            self.scales = np.full((8, 2), 0.01, np.float32)
            self.biases = np.full((8, 2), -0.08, np.float32)
            self.group_size, self.bits = 64, 4

    model = torch.nn.Sequential(ql, torch.nn.ReLU(),
                                torch.nn.Sequential(torch.nn.Linear(16, 128), Duck()))
    counter = [0]
    cconv._convert_children(model, counter, set(), None)
    assert counter[0] == 3
    assert isinstance(model[0], cnn.CiderLinear) and model[0].group_size == gs
    qe, se = O.quantize_weight_pergroup(w, gs)
    assert np.array_equal(model[0].w_int8.numpy(), qe)
    assert np.array_equal(model[0].scale_w.numpy(), np.ascontiguousarray(se.T))
    assert isinstance(model[2][0], cnn.CiderLinear) and model[2][0].group_size == 0
    assert isinstance(model[2][1], cnn.CiderLinear) and model[2][1].group_size == 0
    # group_size given: every layer per-group at that size
    model2 = torch.nn.Sequential(I.QuantizedLinear(words, scales, biases, gs, 8),
                                 torch.nn.Linear(128, 64))
    cconv._convert_children(model2, [0], set(), 128)
    assert model2[0].group_size == 128 and model2[1].group_size == 128


# --------------------------------------------------------------------------
# compressed-tensors
# --------------------------------------------------------------------------


def _write_ct(tmp_path, bits, group_size, strategy, layers, plain):
    """layers: {name: (codes [N, K], scale [N, G])}; splits the first layer's
    tensors over two shards."""
    from safetensors.torch import save_file
    per = 32 // bits
    cfg = {"model_type": "qwen3", "quantization_config": {
        "config_groups": {"group_0": {"weights": {"num_bits": bits, "group_size": group_size,
                                                  "strategy": strategy, "symmetric": True}}},
        "ignore": ["lm_head"]}}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    s1, s2 = {}, {}
    for i, (name, (codes, scale)) in enumerate(layers.items()):
        N, K = codes.shape
        padded = np.zeros((N, math.ceil(K / per) * per), np.int64)
        padded[:, :K] = codes
        words = I.pack_words(padded, bits).view(np.int32)
        s1[f"{name}.weight_packed"] = torch.from_numpy(words.copy())
        dst = s2 if i == 0 else s1   # the first layer's scale / shape live in shard 2
        dst[f"{name}.weight_scale"] = torch.from_numpy(scale).to(torch.bfloat16)
        dst[f"{name}.weight_shape"] = torch.tensor([N, K], dtype=torch.int64)
    s2.update(plain)
    save_file(s1, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(s2, str(tmp_path / "model-00002-of-00002.safetensors"))


def _bf16(a):
    return torch.from_numpy(a).to(torch.bfloat16).float().numpy()


def test_compressed_tensors_w4_group_maps_exactly(tmp_path):
    rng = np.random.default_rng(3)
    N, K, gs = 24, 256, 128
    codes = rng.integers(0, 16, (N, K))
    scale = rng.uniform(1e-3, 1e-2, (N, K // gs)).astype(np.float32)
    codes_b = rng.integers(0, 16, (8, 128))
    scale_b = rng.uniform(1e-3, 1e-2, (8, 1)).astype(np.float32)
    emb = torch.randn(10, 4)
    _write_ct(tmp_path, 4, gs, "group", {"model.layers.0.mlp.down_proj": (codes, scale),
                                         "model.layers.0.self_attn.o_proj": (codes_b, scale_b)},
              {"model.embed_tokens.weight": emb})
    layers, plain, info = I.read_compressed_tensors(str(tmp_path))
    assert info["bits"] == 4 and set(plain) == {"model.embed_tokens.weight"}
    assert torch.equal(plain["model.embed_tokens.weight"], emb)
    L = layers["model.layers.0.mlp.down_proj"]
    assert np.array_equal(L.values, codes - 8)
    np.testing.assert_array_equal(L.dequantize(),
                                  ((codes - 8) * np.repeat(_bf16(scale), gs, 1)).astype(np.float32))
    mods, _, _ = I.load_compressed_tensors(str(tmp_path))
    m = mods["model.layers.0.mlp.down_proj"]
    assert isinstance(m, cnn.W4A8GroupLinear) and m.group_size == gs
    assert np.array_equal(O.unpack_w4_lo_first(m.packed_weight.numpy()), codes - 8)
    assert np.array_equal(m.scales.numpy(), _bf16(scale).T.astype(np.float16))
    # per-channel 4-bit -> the reference W4 layout (cider/ops.py:93-116)
    mb = mods["model.layers.0.self_attn.o_proj"]
    assert isinstance(mb, cnn.W4A8Linear)
    assert np.array_equal(O.unpack_w4_ref(mb.packed_weight.numpy()), (codes_b - 8).T)
    assert np.array_equal(mb.scale.numpy(), _bf16(scale_b)[:, 0])


@pytest.mark.parametrize("strategy,G", [("channel", 1), ("group", 4)])
def test_compressed_tensors_w8_maps_exactly(tmp_path, strategy, G):
    rng = np.random.default_rng(4)
    N, K = 16, 512
    codes = rng.integers(1, 256, (N, K))
    scale = rng.uniform(1e-3, 1e-2, (N, G)).astype(np.float32)
    _write_ct(tmp_path, 8, None if G == 1 else K // G, strategy, {"proj": (codes, scale)}, {})
    m = I.load_compressed_tensors(str(tmp_path))[0]["proj"]
    assert isinstance(m, cnn.CiderLinear)
    assert np.array_equal(m.w_int8.numpy(), (codes - 128).astype(np.int8))
    if G == 1:
        assert m.group_size == 0 and np.array_equal(m.scale_w.numpy(), _bf16(scale)[:, 0])
    else:
        assert m.group_size == K // G and np.array_equal(m.scale_w.numpy(), _bf16(scale).T)


def test_compressed_tensors_2bit_and_ragged_k_requantize(tmp_path):
    rng = np.random.default_rng(5)
    N, K = 8, 100                         # 100 codes in 7 words of 16
    codes = rng.integers(0, 4, (N, K))
    scale = rng.uniform(1e-2, 1e-1, (N, 1)).astype(np.float32)
    _write_ct(tmp_path, 2, None, "channel", {"proj": (codes, scale)}, {})
    layers, _, _ = I.read_compressed_tensors(str(tmp_path))
    assert layers["proj"].shape == (N, K)
    w = ((codes - 2) * _bf16(scale)).astype(np.float32)
    np.testing.assert_array_equal(layers["proj"].dequantize(), w)
    m = I.to_module(layers["proj"])
    q, s = O.quantize_weight_int8(w)
    assert m.group_size == 0
    assert np.array_equal(m.w_int8.numpy(), q) and np.array_equal(m.scale_w.numpy(), s)


def test_replace_modules():
    model = torch.nn.Sequential()
    model.add_module("block", torch.nn.Sequential())
    model.block.add_module("proj", torch.nn.Linear(8, 4))
    new = cnn.CiderLinear(torch.zeros(4, 8, dtype=torch.int8), torch.ones(4), 0, 8, 4)
    assert I.replace_modules(model, {"block.proj": new}) == 1
    assert model.block.proj is new


@pytest.mark.gpu
def test_compressed_tensors_w4_group_forward_on_gpu(tmp_path):
    rng = np.random.default_rng(6)
    N, K, gs = 512, 1024, 128
    codes = rng.integers(0, 16, (N, K))
    scale = rng.uniform(1e-3, 1e-2, (N, K // gs)).astype(np.float32)
    _write_ct(tmp_path, 4, gs, "group", {"proj": (codes, scale)}, {})
    layers, _, _ = I.read_compressed_tensors(str(tmp_path))
    m = I.to_module(layers["proj"], "cuda")
    # M > 64 on 16 tiles: the two-set per-group DMA kernel, whose flush of fp16
    # group scales is bit-exact (one fma from the biased group sum)
    x = torch.randn(100, K, device="cuda").half()
    y = m(x).float()
    # exact per-group reference on the same quantized activations
    xq = x.cpu().numpy()
    exp = O.w4a8_pergroup_linear(xq, m.packed_weight.cpu().numpy(), m.scales.cpu().numpy(),
                                 gs, None)
    assert np.array_equal(y.half().cpu().numpy().view(np.uint16), exp.view(np.uint16))

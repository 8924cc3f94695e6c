"""Qwen3-VL-shaped chunked prefill (cider_amd/qwen3vl.py).

CPU: the 3-axis positions of get_rope_index (vlm_service/custom_qwen3vl.py:
143-295) on a hand-worked prompt; M-RoPE reduces to 1-D RoPE on text; the
interleaved axis pattern.  GPU: chunked prefill against one-shot prefill and
against an fp32 restatement of the model with the same per-token cos / sin;
decode continues the M-RoPE positions (decode logits against prefilling the
same token); graph replays against eager decoding.
"""

import math

import pytest
import torch

from cider_amd import qwen3 as Q
from cider_amd import qwen3vl as V

TINY = Q.Qwen3Config(hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4,
                     num_kv_heads=2, head_dim=128, vocab_size=1000, rope_theta=5e6)


def test_rope_index_hand_worked():
    pos = V.rope_index([("text", 3), ("image", (1, 2, 3)), ("text", 2)])
    assert pos.tolist() == [
        [0, 1, 2, 3, 3, 3, 3, 3, 3, 6, 7],
        [0, 1, 2, 3, 3, 3, 4, 4, 4, 6, 7],
        [0, 1, 2, 3, 4, 5, 3, 4, 5, 6, 7]]
    # two frames: t advances; the next run starts after the block's maximum
    pos = V.rope_index([("text", 1), ("image", (2, 1, 2)), ("text", 1)])
    assert pos.tolist() == [[0, 1, 1, 2, 2, 3], [0, 1, 1, 1, 1, 3], [0, 1, 2, 1, 2, 3]]


def test_mrope_on_text_is_1d_rope():
    L, D = 50, 128
    p = torch.arange(L).expand(3, L)
    cos, sin = V.mrope_cos_sin(p, D, 5e6)
    c1, s1 = Q.rope_tables(D, L, 5e6, "cpu")
    assert torch.equal(cos, c1) and torch.equal(sin, s1)


def test_mrope_axis_interleave():
    D = 128
    inv = 1.0 / (5e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    for axis in range(3):
        p = torch.zeros(3, 1, dtype=torch.int64)
        p[axis, 0] = 7
        cos, sin = V.mrope_cos_sin(p, D, 5e6)
        for i in range(D // 2):
            if i < 60 and i % 3 == 1:
                src = 1
            elif i < 60 and i % 3 == 2:
                src = 2
            else:
                src = 0
            ang = 7 * inv[i].item() if src == axis else 0.0
            for col in (i, i + D // 2):
                assert abs(sin[0, col].item() - math.sin(ang)) < 1e-3
                assert abs(cos[0, col].item() - math.cos(ang)) < 1e-3


def test_synth_segments():
    segs = V.synth_segments(1334, 2, seed=1)
    assert sum(v if k == "text" else 256 for k, v in segs) == 1334
    assert [k for k, _ in segs].count("image") == 2 and segs[-1][0] == "text"
    pos = V.rope_index(segs)
    assert pos.shape == (3, 1334) and int(pos.max()) < 1334


# --------------------------------------------------------------------------
# GPU
# --------------------------------------------------------------------------


def _ref_forward(m, x, cos, sin):
    """fp32 restatement of the model on embeddings x [L, h] with per-token
    cos / sin [L, D]: dequantized weights, no activation quantization."""
    c = m.cfg
    L = x.shape[0]
    lin = lambda t, l: t @ (l.w_int8.float() * l.scale_w[:, None]).T  # noqa: E731

    def norm(t, w):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + c.rms_eps) * w.float()

    cos, sin = cos.float()[:, None, :], sin.float()[:, None, :]
    x = x.float()
    causal = torch.full((L, L), float("-inf"), device=x.device).triu(1)
    for ly in m.layers:
        qkv = lin(norm(x, ly.input_norm), ly.qkv)
        q, k, v = qkv.split([c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim,
                             c.num_kv_heads * c.head_dim], -1)
        q = Q.apply_rope(norm(q.reshape(L, c.num_heads, c.head_dim), ly.q_norm), cos, sin)
        k = Q.apply_rope(norm(k.reshape(L, c.num_kv_heads, c.head_dim), ly.k_norm), cos, sin)
        v = v.reshape(L, c.num_kv_heads, c.head_dim)
        rep = c.num_heads // c.num_kv_heads
        k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
        s = torch.matmul(q.permute(1, 0, 2).contiguous(), k.permute(1, 2, 0).contiguous())
        p = torch.softmax(s / math.sqrt(c.head_dim) + causal, -1)
        o = torch.matmul(p, v.permute(1, 0, 2).contiguous()).permute(1, 0, 2).reshape(L, -1)
        x = x + lin(o, ly.o)
        gu = lin(norm(x, ly.post_norm), ly.gate_up)
        x = x + lin(torch.nn.functional.silu(gu[:, :c.intermediate_size])
                    * gu[:, c.intermediate_size:], ly.down)
    return norm(x, m.final_norm) @ m.lm_head.float().T


def _close(a, b, tol, what):
    a, b = a.float(), b.float()
    rel = (a - b).abs().max().item() / b.abs().max().item()
    cos = torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0).item()
    assert rel < tol and cos > 0.999, f"{what}: max rel {rel:.4f}, cosine {cos:.6f}"


SEGS = [("text", 9), ("image", (1, 4, 5)), ("text", 14), ("image", (2, 2, 3)), ("text", 6)]


@pytest.mark.gpu
def test_chunked_prefill_matches_one_shot_and_fp32():
    m = V.Qwen3VL(TINY, max_len=128, seed=11)
    x, _ = m.embed_prompt(SEGS, seed=3)
    pos3 = V.rope_index(SEGS)
    L = x.shape[0]
    one = m.prefill_chunked(x, pos3, chunk=L)
    k1 = m.k_cache[:, :, :L].clone()
    chunked = m.prefill_chunked(x, pos3, chunk=16)
    # one-shot runs SDPA's causal kernel, the chunks its lower-right-masked
    # one: attention outputs equal up to fp16 rounding, which moves single
    # activations' int8 rounding in the linears after it
    _close(chunked, one, 5e-2, "chunked vs one-shot")
    # layer 0 sees the same inputs in both runs: its cache is identical
    assert torch.equal(m.k_cache[0, :, :L], k1[0])
    _close(m.k_cache[:, :, :L], k1, 5e-2, "k cache chunked vs one-shot")
    cos, sin = V.mrope_cos_sin(pos3.cuda(), TINY.head_dim, TINY.rope_theta)
    ref = _ref_forward(m, x, cos, sin)[-1:]
    _close(chunked, ref, 8e-2, "chunked vs fp32 model")
    assert m._rope_delta.item() == int(pos3.max()) + 1 - L


@pytest.mark.gpu
@pytest.mark.parametrize("chunk", [16, 61, 24])
def test_graph_chunked_prefill_matches_eager(chunk):
    """Chunks replayed from one captured graph (the last one padded to the
    chunk: 61 tokens in chunks of 16 and 24) give the eager chunks' logits
    and cache (the attention's rounding apart), and leave the slots past the
    prompt's end to decode."""
    m = V.Qwen3VL(TINY, max_len=128, seed=14)
    x, _ = m.embed_prompt(SEGS, seed=6)
    pos3 = V.rope_index(SEGS)
    L = x.shape[0]
    eager = m.prefill_chunked(x, pos3, chunk=chunk, graph=False)
    ke, ve = m.k_cache[:, :, :L].clone(), m.v_cache[:, :, :L].clone()
    m.k_cache.zero_()
    m.v_cache.zero_()
    g1 = m.prefill_chunked(x, pos3, chunk=chunk, graph=True)
    g2 = m.prefill_chunked(x, pos3, chunk=chunk, graph=True)  # a second replay of the graph
    assert torch.isfinite(g1.float()).all()
    assert torch.equal(g1, g2)
    _close(g1, eager, 5e-2, "graph vs eager chunks")
    # layer 0 sees the same rows in both: its cache is bit-identical
    assert torch.equal(m.k_cache[0, :, :L], ke[0]) and torch.equal(m.v_cache[0, :, :L], ve[0])
    _close(m.k_cache[:, :, :L], ke, 5e-2, "k cache graph vs eager")
    # decode from the graph-prefilled cache continues like the eager one
    tok = torch.argmax(g1[-1].float()).reshape(1)
    dg = m.decode_step(tok, torch.tensor([L], device="cuda"))
    m2 = V.Qwen3VL(TINY, max_len=128, seed=14)
    m2.prefill_chunked(x, pos3, chunk=chunk, graph=False)
    de = m2.decode_step(tok, torch.tensor([L], device="cuda"))
    _close(dg[0], de[0], 5e-2, "decode after graph vs eager prefill")


@pytest.mark.gpu
def test_decode_continues_mrope_positions():
    m = V.Qwen3VL(TINY, max_len=128, seed=12)
    x, _ = m.embed_prompt(SEGS, seed=4)
    pos3 = V.rope_index(SEGS)
    L = x.shape[0]
    logits = m.prefill_chunked(x, pos3, chunk=8)
    tok = torch.argmax(logits[-1].float()).reshape(1)
    dec = m.decode_step(tok, torch.tensor([L], device="cuda"))
    # the same token appended to the prompt as text, prefilled in one go
    x2 = torch.cat([x, m.embed.index_select(0, tok)])
    p2 = torch.cat([pos3, torch.full((3, 1), int(pos3.max()) + 1)], 1)
    m2 = V.Qwen3VL(TINY, max_len=128, seed=12)
    full = m2.prefill_chunked(x2, p2, chunk=8)
    # decode: fp16-activation MV; prefill: W8A8 GEMM (activation quantization)
    _close(dec[0], full[0], 8e-2, "decode vs prefill of the same token")


@pytest.mark.gpu
def test_graph_generate_equals_eager():
    a = V.Qwen3VL(TINY, max_len=128, seed=13)
    b = V.Qwen3VL(TINY, max_len=128, seed=13)
    ta = a.generate_from_prompt(SEGS, 10, seed=5, chunk=16, graph=True)
    tb = b.generate_from_prompt(SEGS, 10, seed=5, chunk=16, graph=False)
    assert torch.equal(ta, tb)

"""cider_amd.qwen3 - a Qwen3-shaped decoder stack whose every projection is a
W8A8 per-channel ``CiderLinear`` (the callers of the hot path).

Shape defaults are Qwen3-8B (hidden 4096, SwiGLU intermediate 12288, 36
layers, 32 query / 8 KV heads of 128, RMSNorm with eps 1e-6 including the
per-head q/k norms, RoPE base 1e6, vocabulary 151936 with an fp16 lm_head).
Weights are random: int8 uniform in [-127, 127] with per-channel scales chosen
so that every linear keeps unit-variance inputs at unit variance; embedding
and norm weights are fp16.

Projections are fused the way the reference fuses them for prefill
(``cider/fused_hybrid.py:142-213,240-263``): q, k and v are one linear of
N = (32 + 8 + 8) * 128 = 6144 outputs, gate and up one linear of 2 * 12288
outputs; o_proj and down_proj stay single.  Prefill (M = prompt length) runs
the quantize + int8 GEMM path; decode (M = 1) runs the fp16-activation MV,
exactly as ``CiderLinear`` dispatches for the reference (``cider/nn.py:102-113``).

With ``fused=True`` (the default) the producers of each linear's input are
HIP kernels of this library (``cider_amd.fused``): the residual add and
RMSNorm before q/k/v and gate/up, and the SwiGLU before down_proj, end in the
per-token quantization, so prefill hands (q, scale_a) straight to the int8
GEMM; the per-head q/k RMSNorm and RoPE write k and v into the cache in the
same kernel; decode attention is a single-query split-K kernel over the
cache; prefill attention is this library's causal flash-attention kernel over
the cache (grouped query heads; a chunk that follows earlier cache slots
attends them all).  ``fused=False`` runs those steps as plain PyTorch ops
instead (the A/B reference; its attention is batched matmuls with the 4 query
heads of each KV head grouped along rows).  The embedding lookup and the fp16
lm_head are PyTorch on the GPU in both modes.  Both caches are [KV, T, 128]
(position-major).

Decode keeps the position, the next token and the KV cache on the device, so a
whole decode step (embedding to argmax) can be captured once as a HIP graph and
replayed for every generated token with no host synchronisation
(``Qwen3.generate(..., graph=True)``).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Optional

import torch
import torch.nn.functional as F

from . import fused as FK
from .nn import CiderLinear


@dataclasses.dataclass
class Qwen3Config:
    hidden_size: int = 4096
    intermediate_size: int = 12288
    num_layers: int = 36
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6

    @property
    def qkv_out(self) -> int:
        return (self.num_heads + 2 * self.num_kv_heads) * self.head_dim

    def linear_shapes(self):
        """(name, N, K) of the four W8A8 linears of one layer."""
        h, i = self.hidden_size, self.intermediate_size
        return [("qkv", self.qkv_out, h), ("o", h, self.num_heads * self.head_dim),
                ("gate_up", 2 * i, h), ("down", h, i)]

    def linear_macs_per_token(self) -> int:
        return self.num_layers * sum(n * k for _, n, k in self.linear_shapes())


QWEN3_8B = Qwen3Config()

# standard deviation of an int8 drawn uniformly from [-127, 127]
_INT8_UNIFORM_STD = math.sqrt((255 ** 2 - 1) / 12.0)


def random_w8a8_linear(n: int, k: int, gen: torch.Generator, device) -> CiderLinear:
    """W8A8 per-channel linear with random int8 weights [n, k] and scales that
    give each output unit variance for unit-variance inputs (+-10% per channel)."""
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=device, generator=gen)
    base = 1.0 / (_INT8_UNIFORM_STD * math.sqrt(k))
    s = base * (0.9 + 0.2 * torch.rand(n, device=device, generator=gen, dtype=torch.float32))
    return CiderLinear(w, s, 0, k, n)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dimension in fp32, scaled by w after the cast back."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def rope_tables(head_dim: int, max_pos: int, theta: float, device):
    """cos, sin [max_pos, head_dim] (fp16) for the rotate-half form of RoPE."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32)
                           / head_dim))
    f = torch.outer(torch.arange(max_pos, device=device, dtype=torch.float32), inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().half(), emb.sin().half()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [L, heads, d]; cos, sin [L, 1, d]."""
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * cos + rot * sin


class Qwen3Layer(torch.nn.Module):
    def __init__(self, cfg: Qwen3Config, gen: torch.Generator, device):
        super().__init__()
        self.cfg = cfg
        self.fuse_mv = True  # decode: producers inside the consuming MV (A/B switch)
        h = cfg.hidden_size
        ones = lambda n: torch.ones(n, dtype=torch.float16, device=device)  # noqa: E731
        self.input_norm = ones(h)
        self.post_norm = ones(h)
        self.q_norm = ones(cfg.head_dim)
        self.k_norm = ones(cfg.head_dim)
        self.qkv = random_w8a8_linear(cfg.qkv_out, h, gen, device)
        self.o = random_w8a8_linear(h, cfg.num_heads * cfg.head_dim, gen, device)
        self.gate_up = random_w8a8_linear(2 * cfg.intermediate_size, h, gen, device)
        self.down = random_w8a8_linear(h, cfg.intermediate_size, gen, device)

    def _qkv(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        c = self.cfg
        L = x.shape[0]
        qkv = self.qkv(rms_norm(x, self.input_norm, c.rms_eps))
        q, k, v = qkv.split([c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim,
                             c.num_kv_heads * c.head_dim], dim=-1)
        q = apply_rope(rms_norm(q.reshape(L, c.num_heads, c.head_dim), self.q_norm, c.rms_eps),
                       cos, sin)
        k = apply_rope(rms_norm(k.reshape(L, c.num_kv_heads, c.head_dim), self.k_norm,
                                c.rms_eps), cos, sin)
        return q, k, v.reshape(L, c.num_kv_heads, c.head_dim)

    def _attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                mask: torch.Tensor) -> torch.Tensor:
        """Attention as batched matmuls (the PyTorch-producer reference path):
        q [L, heads, d]; k, v [kv, T, d]; mask broadcastable to [kv, group, L,
        T] (0 or -inf).  Returns [L, heads * d]."""
        c = self.cfg
        L = q.shape[0]
        g = c.num_heads // c.num_kv_heads
        T = k.shape[1]
        kT = k.transpose(1, 2).contiguous()  # [kv, d, T]: no transposed bmm operand
        # q head j * g + r belongs to KV head j
        qg = (q * (1.0 / math.sqrt(c.head_dim))).reshape(L, c.num_kv_heads, g, c.head_dim)
        qg = qg.permute(1, 2, 0, 3).reshape(c.num_kv_heads, g * L, c.head_dim)
        s = torch.bmm(qg, kT).float().reshape(c.num_kv_heads, g, L, T) + mask
        p = torch.softmax(s, dim=-1).to(torch.float16).reshape(c.num_kv_heads, g * L, T)
        o = torch.bmm(p, v).reshape(c.num_kv_heads, g, L, c.head_dim)
        return o.permute(2, 0, 1, 3).reshape(L, c.num_heads * c.head_dim)

    def _mlp(self, x: torch.Tensor) -> torch.Tensor:
        i = self.cfg.intermediate_size
        gu = self.gate_up(rms_norm(x, self.post_norm, self.cfg.rms_eps))
        return self.down(F.silu(gu[:, :i]) * gu[:, i:])

    def prefill(self, x, cos, sin, k_cache, v_cache, mask):
        """x [L, hidden] at positions 0..L-1; fills cache[:, :L]."""
        L = x.shape[0]
        q, k, v = self._qkv(x, cos, sin)
        k_cache[:, :L, :].copy_(k.permute(1, 0, 2))
        v_cache[:, :L, :].copy_(v.permute(1, 0, 2))
        x = x + self.o(self._attend(q, k_cache[:, :L, :], v_cache[:, :L, :], mask))
        return x + self._mlp(x)

    def decode(self, x, cos, sin, pos, k_cache, v_cache, mask):
        """x [1, hidden] at device position `pos` ([1] int64); attends over the
        whole cache with `mask` (-inf past pos)."""
        q, k, v = self._qkv(x, cos, sin)
        k_cache.index_copy_(1, pos, k.permute(1, 0, 2))
        v_cache.index_copy_(1, pos, v.permute(1, 0, 2))
        x = x + self.o(self._attend(q, k_cache, v_cache, mask))
        return x + self._mlp(x)

    # ---- fused producers (HIP kernels) -------------------------------------
    # The residual stream is carried as (x, pending): the layer's true input is
    # h(x + pending); the add happens inside the next RMSNorm kernel, which
    # writes the sum back over x.

    def _norm(self, x, pending, w, want_y, want_q):
        return FK.rmsnorm_quantize(x, w, self.cfg.rms_eps, add=pending,
                                   sum_out=x if pending is not None else None,
                                   want_y=want_y, want_q=want_q)

    def prefill_fused(self, x, pending, tables, rope_row, slot, k_cache, v_cache, n,
                      attn_ws=None, n_dev=None):
        """x [L, hidden] (+ pending) at cache slots n - L .. n - 1 (`slot`);
        attends causally over cache slots 0..n-1, the attention's output
        quantized for o_proj in the attention (``attn_ws``: its workspace for
        this (L, n), ``fused.attn_prefill_quantize_workspace``, shared by the
        layers; ``n_dev``: n
        read on the device, the host n its upper bound).  Returns
        (x, pending)."""
        c = self.cfg
        a = self._norm(x, pending, self.input_norm, False, True)
        qkv = self.qkv.forward_quantized(a.q, a.scale_a)
        q = FK.qk_norm_rope(qkv, self.q_norm, self.k_norm, c.rms_eps, tables[0], tables[1],
                            rope_row, slot, k_cache, v_cache, c.num_heads, c.num_kv_heads)
        qa, sa = FK.attn_prefill_quantize(q, k_cache, v_cache, n, 1.0 / math.sqrt(c.head_dim),
                                          ws=attn_ws, n_dev=n_dev)
        b = self._norm(a.h, self.o.forward_quantized(qa, sa), self.post_norm, False, True)
        gu = self.gate_up.forward_quantized(b.q, b.scale_a)
        _, qd, sd = FK.silu_mul_quantize(gu, want_y=False, want_q=True)
        return b.h, self.down.forward_quantized(qd, sd)

    def decode_fused(self, x, pending, tables, pos, n_valid, k_cache, v_cache, ws,
                     rope_pos=None):
        """One token x [1, hidden] (+ pending) at device cache slot `pos`
        ([1] int64; RoPE row `rope_pos`, default pos), attending over
        n_valid = pos + 1 cache positions."""
        c = self.cfg
        # RMSNorm (+ residual add) and SwiGLU run inside the x staging of the
        # MV that consumes them (bit-identical to the separate launches; one
        # kernel fewer each) where that pays: every workgroup of the MV redoes
        # the producer, so only for MVs of few workgroups / short rows
        fuse_in = self.fuse_mv and _fuse_norm_into(c.hidden_size, c.qkv_out)
        fuse_post = self.fuse_mv and _fuse_norm_into(c.hidden_size, 2 * c.intermediate_size)
        fuse_act = self.fuse_mv and _fuse_swiglu_into(c.intermediate_size)
        if fuse_in:
            h, qkv = FK.rmsnorm_mv(x, self.input_norm, c.rms_eps, self.qkv, add=pending)
        else:
            a = self._norm(x, pending, self.input_norm, True, False)
            h, qkv = a.h, self.qkv(a.y)
        q = FK.qk_norm_rope(qkv, self.q_norm, self.k_norm, c.rms_eps, tables[0], tables[1],
                            pos if rope_pos is None else rope_pos, pos, k_cache, v_cache,
                            c.num_heads, c.num_kv_heads)
        attn = FK.attn_decode(q, k_cache, v_cache, n_valid, 1.0 / math.sqrt(c.head_dim), ws=ws)
        o = self.o(attn.reshape(1, -1))
        if fuse_post:
            h2, gu = FK.rmsnorm_mv(h, self.post_norm, c.rms_eps, self.gate_up, add=o)
        else:
            b = self._norm(h, o, self.post_norm, True, False)
            h2, gu = b.h, self.gate_up(b.y)
        if fuse_act:
            return h2, FK.swiglu_mv(gu, self.down)
        hs, _, _ = FK.silu_mul_quantize(gu, want_y=True, want_q=False)
        return h2, self.down(hs)


def _mv_fusable(k: int) -> bool:
    """A producer can run inside the M == 1 linear's x staging (cider_rmsnorm_mv,
    cider_swiglu_mv): K a multiple of 256 up to 16384."""
    return k % 256 == 0 and k <= 16384


def _fuse_norm_into(k: int, n: int) -> bool:
    """RMSNorm inside an M == 1 linear of n outputs (n / 8 workgroups, each of
    which redoes the norm): measured to pay up to 2048 workgroups (Qwen3-8B
    qkv: 9.6 us fused vs 15.6 us as two launches; gate_up, 3072 workgroups:
    23.4 vs ~22.5 us)."""
    return _mv_fusable(k) and n <= 16384


def _fuse_swiglu_into(k: int) -> bool:
    """SwiGLU inside an M == 1 linear with K = k: every workgroup evaluates k
    exponentials, which pays for short rows only (Qwen3-8B down, K = 12288:
    21.1 us fused vs 18.5 us as two launches; Qwen3-VL-2B, K = 6144: faster)."""
    return _mv_fusable(k) and k <= 8192


class Qwen3(torch.nn.Module):
    """Random-init Qwen3-shaped causal LM over W8A8 per-channel linears."""

    def __init__(self, cfg: Qwen3Config = QWEN3_8B, max_len: int = 4096, seed: int = 0,
                 device="cuda", fused: bool = True, capacity_multiple: int = 8):
        super().__init__()
        if fused and cfg.head_dim != 128:
            raise ValueError("Qwen3(fused=True): the q/k-norm, RoPE and attention kernels "
                             "take head_dim 128")
        self.fused = fused
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("Qwen3: the W8A8 linears run on a ROCm GPU only")
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.cfg = cfg
        self.max_len = max_len
        # cache capacity: a multiple of 8 positions (the decode attention's
        # 8-position groups), or of capacity_multiple (a chunked prefill that
        # pads its last chunk to the chunk size writes that far)
        mult = max(8, (capacity_multiple + 7) // 8 * 8)
        cap = (max_len + mult - 1) // mult * mult
        self.capacity = cap
        self.device = dev
        h = cfg.hidden_size
        self.embed = (torch.randn(cfg.vocab_size, h, device=dev, generator=gen) * 0.02).half()
        self.layers = torch.nn.ModuleList(Qwen3Layer(cfg, gen, dev)
                                          for _ in range(cfg.num_layers))
        self.final_norm = torch.ones(h, dtype=torch.float16, device=dev)
        self.lm_head = (torch.randn(cfg.vocab_size, h, device=dev, generator=gen)
                        * (1.0 / math.sqrt(h))).half()
        self.cos, self.sin = rope_tables(cfg.head_dim, cap, cfg.rope_theta, dev)
        kv, d = cfg.num_kv_heads, cfg.head_dim
        # zero-filled: decode attends over the whole cache, masked entries
        # must hold finite values
        self.k_cache = torch.zeros(cfg.num_layers, kv, cap, d, dtype=torch.float16,
                                   device=dev)
        self.v_cache = torch.zeros(cfg.num_layers, kv, cap, d, dtype=torch.float16,
                                   device=dev)
        self._attn_ws = FK.attn_decode_workspace(cfg.num_heads, cap, dev) if fused else None
        # RoPE row = cache slot + this offset in decode (device [1] int64; None
        # = 0); multimodal prompts whose M-RoPE positions run behind their
        # length set it after prefill
        self._rope_delta = None
        self._graph = None

    # ---- prefill ----------------------------------------------------------
    @torch.no_grad()
    def prefill(self, ids: torch.Tensor, last_only: bool = False) -> torch.Tensor:
        """ids [L] int64 on the device; fills the KV cache for positions
        0..L-1 and returns the logits [L, vocab] (fp16), or with last_only
        those of the last position [1, vocab] -- what generation needs; the
        reference's prefill evaluates only the cache, and the last token's
        logits come from its first step (vlm_service/custom_qwen3vl.py:598-660)."""
        L = ids.shape[0]
        if L > self.max_len:
            raise ValueError(f"prompt of {L} tokens exceeds max_len={self.max_len}")
        x = self.embed.index_select(0, ids)
        if self.fused:
            pos = torch.arange(L, device=self.device)
            pending = None
            ws = FK.attn_prefill_quantize_workspace(L, L, self.cfg.num_heads, self.device)
            for i, layer in enumerate(self.layers):
                x, pending = layer.prefill_fused(x, pending, (self.cos, self.sin), pos, pos,
                                                 self.k_cache[i], self.v_cache[i], L, ws)
            if last_only:
                x, pending = x[-1:].clone(), pending[-1:].clone()
            return F.linear(self._final_norm(x, pending), self.lm_head)
        cos, sin = self.cos[:L, None, :], self.sin[:L, None, :]
        mask = torch.full((L, L), float("-inf"), device=self.device).triu_(1)
        for i, layer in enumerate(self.layers):
            x = layer.prefill(x, cos, sin, self.k_cache[i], self.v_cache[i], mask)
        if last_only:
            x = x[-1:]
        return F.linear(rms_norm(x, self.final_norm, self.cfg.rms_eps), self.lm_head)

    def _final_norm(self, x, pending):
        return FK.rmsnorm_quantize(x, self.final_norm, self.cfg.rms_eps, add=pending,
                                   sum_out=x, want_y=True, want_q=False).y

    # ---- decode -----------------------------------------------------------
    @torch.no_grad()
    def decode_step(self, tok: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """One token: tok [1] int64, pos [1] int64 (both on the device).
        Returns the logits [1, vocab]."""
        x = self.embed.index_select(0, tok)
        if self.fused:
            n_valid = pos + 1
            rope_pos = None if self._rope_delta is None else pos + self._rope_delta
            pending = None
            for i, layer in enumerate(self.layers):
                x, pending = layer.decode_fused(x, pending, (self.cos, self.sin), pos, n_valid,
                                                self.k_cache[i], self.v_cache[i], self._attn_ws,
                                                rope_pos)
            return F.linear(self._final_norm(x, pending), self.lm_head)
        if self._rope_delta is not None:
            raise ValueError("decode_step: a RoPE position offset needs fused=True")
        cos = self.cos.index_select(0, pos)[:, None, :]
        sin = self.sin.index_select(0, pos)[:, None, :]
        ar = torch.arange(self.capacity, device=self.device)
        mask = torch.where(ar <= pos, 0.0, float("-inf"))
        for i, layer in enumerate(self.layers):
            x = layer.decode(x, cos, sin, pos, self.k_cache[i], self.v_cache[i], mask)
        return F.linear(rms_norm(x, self.final_norm, self.cfg.rms_eps), self.lm_head)

    def _greedy_step(self, state: dict):
        """Device-resident greedy step: reads state['tok'], state['pos'],
        writes the argmax into state['tok'] and state['out'][state['i']],
        advances pos and i."""
        logits = self.decode_step(state["tok"], state["pos"])
        nxt = torch.argmax(logits[0].float()).reshape(1)
        state["out"].index_copy_(0, state["i"], nxt)
        state["tok"].copy_(nxt)
        state["pos"].add_(1)
        state["i"].add_(1)

    @torch.no_grad()
    def generate(self, ids: torch.Tensor, steps: int, graph: bool = True) -> torch.Tensor:
        """Greedy decoding: prefill `ids`, then `steps` tokens.  Returns the
        generated ids [steps] (device).  graph=True captures one decode step
        as a HIP graph and replays it."""
        L = ids.shape[0]
        if L + steps > self.max_len:
            raise ValueError("prompt + steps exceeds max_len")
        logits = self.prefill(ids, last_only=True)
        first = torch.argmax(logits[-1].float()).reshape(1)
        state = {"tok": first.clone(), "pos": torch.tensor([L], device=self.device),
                 "i": torch.zeros(1, dtype=torch.int64, device=self.device),
                 "out": torch.zeros(steps + 1, dtype=torch.int64, device=self.device)}
        state["out"][0] = first[0]
        state["i"].fill_(1)
        if steps == 0:
            return state["out"][:1]
        if not graph:
            for _ in range(steps):
                self._greedy_step(state)
            return state["out"][1:]
        g, s = self.capture_decode(state)
        for _ in range(steps):
            g.replay()
        return state["out"][1:]

    def capture_decode(self, state: dict):
        """Captures one greedy step over the buffers in `state`.  The capture
        runs the step once eagerly first (warm-up on a side stream, as graph
        capture requires); the state is restored afterwards, so the graph's
        first replay computes the next token."""
        saved = {k: v.clone() for k, v in state.items()}
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._greedy_step(state)
        torch.cuda.current_stream(self.device).wait_stream(side)
        for k in state:
            state[k].copy_(saved[k])
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._greedy_step(state)
        for k in state:
            state[k].copy_(saved[k])
        torch.cuda.synchronize(self.device)
        return g, side

"""cider_amd.qwen3vl - a Qwen3-VL-2B-shaped text decoder with multimodal
(3-axis M-RoPE) prompts, chunked prefill and graph-captured decode over the
W8A8 linears (the caller the reference's VLM service puts on the path,
``vlm_service/custom_qwen3vl.py``).

Shape (Qwen3-VL-2B text model): hidden 2048, SwiGLU intermediate 6144, 28
layers, 16 query / 8 KV heads of 128, RMSNorm eps 1e-6 with per-head q/k
norms, RoPE base 5e6 with interleaved M-RoPE sections (24, 20, 20), vocabulary
151936, lm_head tied to the embedding.  Weights are random (no checkpoint);
the vision tower is out of scope: image tokens enter as fp16 embeddings
drawn from N(0, 0.02), 256 per image (a 32 x 32 patch grid after the 2 x 2
spatial merge: t = 1, h = w = 16).

Positions follow ``get_rope_index`` (``vlm_service/custom_qwen3vl.py:143-295``):
text runs count up on all three axes; an image block of grid (t, h, w) takes
(t_i, h_i, w_i) + text_len + start over its tokens, and the next run starts
at the block's maximum + 1.  They are computed over the whole prompt before
chunking (``custom_qwen3vl.py:576-595``), then the prompt is prefilled in
chunks of 512 tokens (``custom_qwen3vl.py:602-643``), each chunk attending to
the cache the chunks before it filled; the logits of the prompt's last token
give the first generated token.  Decode continues on all axes at
``slot + delta`` with ``delta = max position + 1 - prompt length``.

M-RoPE (the interleaved form of the Qwen3-VL text model, which mlx-vlm and
transformers implement; neither is vendored, so this restatement is
"parity unpinned" beyond its invariants): frequency i of the head_dim / 2
rotary frequencies takes its position from axis H when i % 3 == 1 and
i < 3 * 20, from axis W when i % 3 == 2 and i < 3 * 20, else from axis T;
cos / sin are then laid out as [f, f] for the rotate-half form.  With equal
positions on the three axes (text) this is the ordinary 1-D RoPE.
"""

from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import torch
import torch.nn.functional as F

from . import fused as FK
from .qwen3 import Qwen3, Qwen3Config

QWEN3_VL_2B = Qwen3Config(hidden_size=2048, intermediate_size=6144, num_layers=28, num_heads=16,
                          num_kv_heads=8, head_dim=128, vocab_size=151936, rope_theta=5.0e6,
                          rms_eps=1.0e-6)
MROPE_SECTION = (24, 20, 20)
IMAGE_GRID = (1, 16, 16)          # (t, h, w) after the spatial merge: 256 tokens
PREFILL_CHUNK = 512

# Segment = ("text", n_tokens) or ("image", (t, h, w))
Segment = Tuple[str, object]


def rope_index(segments: Sequence[Segment]) -> torch.Tensor:
    """3-axis positions [3, L] (int64) of a prompt given as text runs and
    image blocks, as ``get_rope_index`` builds them."""
    parts: List[torch.Tensor] = []
    nxt = 0
    for kind, val in segments:
        if kind == "text":
            n = int(val)
            idx = torch.arange(n, dtype=torch.int64) + nxt
            parts.append(idx.expand(3, n))
            nxt = nxt + n
        elif kind == "image":
            t, h, w = (int(v) for v in val)
            ti = torch.arange(t).view(t, 1, 1).expand(t, h, w).reshape(-1)
            hi = torch.arange(h).view(1, h, 1).expand(t, h, w).reshape(-1)
            wi = torch.arange(w).view(1, 1, w).expand(t, h, w).reshape(-1)
            block = torch.stack([ti, hi, wi]).to(torch.int64) + nxt
            parts.append(block)
            nxt = int(block.max()) + 1
        else:
            raise ValueError(f"unknown segment kind {kind!r}")
    return torch.cat(parts, dim=1) if parts else torch.zeros(3, 0, dtype=torch.int64)


def mrope_cos_sin(pos3: torch.Tensor, head_dim: int, theta: float,
                  section: Sequence[int] = MROPE_SECTION):
    """cos, sin [L, head_dim] (fp16) for 3-axis positions pos3 [3, L]."""
    half = head_dim // 2
    if sum(section) != half:
        raise ValueError(f"M-RoPE sections {tuple(section)} must add up to {half}")
    dev = pos3.device
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=dev, dtype=torch.float32)
                           / head_dim))
    f = pos3.to(torch.float32)[..., None] * inv          # [3, L, half]
    ft = f[0].clone()
    for axis, offset in ((1, 1), (2, 2)):
        sl = slice(offset, 3 * section[axis], 3)
        ft[:, sl] = f[axis][:, sl]
    emb = torch.cat([ft, ft], dim=-1)
    return emb.cos().half(), emb.sin().half()


def synth_segments(total: int, n_images: int, seed: int) -> List[Segment]:
    """A prompt of `total` tokens: text runs of random length around
    `n_images` image blocks of 256 tokens (vision start / end markers are
    text tokens, counted in the runs)."""
    img = IMAGE_GRID[0] * IMAGE_GRID[1] * IMAGE_GRID[2]
    text = total - n_images * img
    if text < n_images + 1:
        raise ValueError("prompt too short for its images")
    g = torch.Generator().manual_seed(seed)
    cuts = sorted(torch.randperm(text - 1, generator=g)[:n_images].add(1).tolist())
    runs = [b - a for a, b in zip([0] + cuts, cuts + [text])]
    segs: List[Segment] = []
    for i, r in enumerate(runs):
        segs.append(("text", r))
        if i < n_images:
            segs.append(("image", IMAGE_GRID))
    return segs


class Qwen3VL(Qwen3):
    """Qwen3-VL-shaped text decoder: ``Qwen3`` with a tied lm_head, M-RoPE
    prompts and chunked prefill (fused producers only)."""

    def __init__(self, cfg: Qwen3Config = QWEN3_VL_2B, max_len: int = 4096, seed: int = 0,
                 device="cuda", section: Sequence[int] = MROPE_SECTION):
        # capacity a multiple of the chunk: the graph prefill pads its last chunk
        super().__init__(cfg, max_len=max_len, seed=seed, device=device, fused=True,
                         capacity_multiple=PREFILL_CHUNK)
        self.section = tuple(section)
        self.lm_head = self.embed          # tied, as the 2B model
        self._chunk_graph = None           # (chunk, graph, static buffers, outputs)

    def embed_prompt(self, segments: Sequence[Segment], seed: int = 0) -> Tuple[torch.Tensor,
                                                                             torch.Tensor]:
        """Synthetic prompt embeddings [L, hidden] (text ids uniform over the
        vocabulary through the embedding; image tokens fp16 N(0, 0.02)) and
        the ids [L] (-1 at image tokens)."""
        g = torch.Generator(device=self.device).manual_seed(seed)
        xs, ids = [], []
        for kind, val in segments:
            if kind == "text":
                t = torch.randint(0, self.cfg.vocab_size, (int(val),), device=self.device,
                                  generator=g)
                xs.append(self.embed.index_select(0, t))
                ids.append(t)
            else:
                n = int(val[0]) * int(val[1]) * int(val[2])
                xs.append((torch.randn(n, self.cfg.hidden_size, device=self.device, generator=g)
                           * 0.02).half())
                ids.append(torch.full((n,), -1, dtype=torch.int64, device=self.device))
        return torch.cat(xs), torch.cat(ids)

    def _chunk_layers(self, xc, rows, tables, slots, n, ws, n_dev=None):
        """The 28 layers over one chunk xc [c, hidden] at cache slots `slots`."""
        pc = None
        for i, layer in enumerate(self.layers):
            xc, pc = layer.prefill_fused(xc, pc, tables, rows, slots, self.k_cache[i],
                                         self.v_cache[i], n, ws, n_dev)
        return xc, pc

    def _capture_chunk(self, chunk: int):
        """One HIP graph of the layers over a chunk of `chunk` rows whose
        inputs (embeddings, RoPE rows, cache slots, valid length) are static
        device buffers: every chunk of a prompt replays it after filling them.
        The warm-up and capture run with slots outside the cache, which the
        q/k-norm kernel writes nowhere, so they leave the cache as it was."""
        dev, h = self.device, self.cfg.hidden_size
        buf = {"x": torch.zeros(chunk, h, dtype=torch.float16, device=dev),
               "cos": torch.zeros(chunk, self.cfg.head_dim, dtype=torch.float16, device=dev),
               "sin": torch.zeros(chunk, self.cfg.head_dim, dtype=torch.float16, device=dev),
               "rows": torch.arange(chunk, device=dev),
               "slots": torch.full((chunk,), -1, dtype=torch.int64, device=dev),
               "n": torch.tensor([chunk], dtype=torch.int64, device=dev)}
        cap = self.capacity
        ws = FK.attn_prefill_quantize_workspace(chunk, cap, self.cfg.num_heads, dev)

        def run():
            return self._chunk_layers(buf["x"], buf["rows"], (buf["cos"], buf["sin"]),
                                      buf["slots"], cap, ws, buf["n"])

        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            run()
        torch.cuda.current_stream(dev).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = run()
        torch.cuda.synchronize(dev)
        self._chunk_graph = (chunk, g, buf, out, ws)

    @torch.no_grad()
    def prefill_chunked(self, x: torch.Tensor, pos3: torch.Tensor,
                        chunk: int = PREFILL_CHUNK, graph: bool = True) -> torch.Tensor:
        """Prefills embeddings x [L, hidden] at M-RoPE positions pos3 [3, L]
        in chunks, into cache slots 0..L-1.  Returns the logits [1, vocab] of
        the last token, and sets the decode RoPE offset.

        graph=True: every chunk is one replay of a captured graph of the
        layers over `chunk` rows; the last chunk is padded with zero rows at
        the following slots (within the cache capacity, a multiple of the
        chunk; where the padded prompt would not fit, the chunks run eagerly).  Causal attention keeps the real tokens from seeing the
        padded keys, and every other step is row-wise, so the real rows get
        what the eager chunks compute (up to the attention's rounding); the
        padded slots past L are rewritten by decode before it reads them."""
        L = x.shape[0]
        if L > self.max_len:
            raise ValueError(f"prompt of {L} tokens exceeds max_len={self.max_len}")
        if pos3.shape != (3, L):
            raise ValueError("pos3 must be [3, L]")
        pos3 = pos3.to(self.device)
        if graph and (L + chunk - 1) // chunk * chunk <= self.capacity:
            return self._prefill_chunked_graph(x, pos3, chunk)
        cos, sin = mrope_cos_sin(pos3, self.cfg.head_dim, self.cfg.rope_theta, self.section)
        slots = torch.arange(L, device=self.device)
        out = None
        for s in range(0, L, chunk):
            e = min(L, s + chunk)
            c = e - s
            xc = x[s:e].clone()
            rows = torch.arange(c, device=self.device)
            pc = None
            ws = FK.attn_prefill_quantize_workspace(e - s, e, self.cfg.num_heads, self.device)
            for i, layer in enumerate(self.layers):
                # query i (slot s + i) sees slots 0 .. s + i
                xc, pc = layer.prefill_fused(xc, pc, (cos[s:e], sin[s:e]), rows,
                                             slots[s:e], self.k_cache[i], self.v_cache[i], e, ws)
            out = (xc, pc)
        xl, pl = out
        return self._prefill_logits(xl[-1:], pl[-1:], pos3, L)

    def _prefill_logits(self, xl, pl, pos3, L):
        logits = F.linear(self._final_norm(xl.clone(), pl.clone()), self.lm_head)
        delta = int(pos3.max()) + 1 - L
        self._rope_delta = torch.tensor([delta], dtype=torch.int64, device=self.device)
        return logits

    def _prefill_chunked_graph(self, x, pos3, chunk):
        L = x.shape[0]
        if self._chunk_graph is None or self._chunk_graph[0] != chunk:
            self._capture_chunk(chunk)
        _, g, buf, (xo, po), _ = self._chunk_graph
        nch = (L + chunk - 1) // chunk
        Lp = nch * chunk
        # positions of the padded rows repeat the last one (any finite RoPE row serves)
        pos_p = torch.cat([pos3, pos3[:, -1:].expand(3, Lp - L)], dim=1) if Lp > L else pos3
        cos, sin = mrope_cos_sin(pos_p, self.cfg.head_dim, self.cfg.rope_theta, self.section)
        for k in range(nch):
            s, e = k * chunk, min(L, (k + 1) * chunk)
            buf["x"][: e - s].copy_(x[s:e])
            if e - s < chunk:
                buf["x"][e - s:].zero_()
            buf["cos"].copy_(cos[s:s + chunk])
            buf["sin"].copy_(sin[s:s + chunk])
            torch.arange(s, s + chunk, device=self.device, out=buf["slots"])
            buf["n"].fill_(s + chunk)
            g.replay()
        r = (L - 1) - (nch - 1) * chunk  # the last real row of the last chunk
        return self._prefill_logits(xo[r:r + 1], po[r:r + 1], pos3, L)

    @torch.no_grad()
    def generate_from_prompt(self, segments: Sequence[Segment], steps: int, seed: int = 0,
                             chunk: int = PREFILL_CHUNK, graph: bool = True) -> torch.Tensor:
        """Chunked prefill of a synthetic multimodal prompt, then `steps`
        greedy tokens (decode step captured as a HIP graph)."""
        x, _ = self.embed_prompt(segments, seed)
        L = x.shape[0]
        if L + steps > self.max_len:
            raise ValueError("prompt + steps exceeds max_len")
        logits = self.prefill_chunked(x, rope_index(segments), chunk)
        first = torch.argmax(logits[-1].float()).reshape(1)
        state = {"tok": first.clone(), "pos": torch.tensor([L], device=self.device),
                 "i": torch.zeros(1, dtype=torch.int64, device=self.device),
                 "out": torch.zeros(steps, dtype=torch.int64, device=self.device)}
        if not graph:
            for _ in range(steps):
                self._greedy_step(state)
            return state["out"]
        g, _ = self.capture_decode(state)
        for _ in range(steps):
            g.replay()
        return state["out"]

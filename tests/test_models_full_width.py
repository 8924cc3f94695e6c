"""configs[3] and configs[4] at their real width and depth.

* 2-layer slices at full width (Qwen3-8B: hidden 4096, intermediate 12288,
  32 q / 8 kv heads; Qwen3-VL-2B: hidden 2048, intermediate 6144, 16 / 8
  heads; both with the 151936-token vocabulary) against the fp32
  restatements of tests/test_qwen3.py and tests/test_qwen3vl.py (no
  activation quantization).  The per-token int8 rounding of the linears'
  inputs is the difference; at this width, with SwiGLU outputs' heavy
  tails, it measured cosine 0.99897 (VL-2B, one logits row) to 0.9990 and
  a max relative error of 0.044; the bar is cosine > 0.998 and max relative
  error 8e-2.  (Quantizing the reference's activations too does not tighten
  this: the GPU's fp16 intermediates move some of the rounding decisions,
  so the two roundings are independent noise.)  A wrong head grouping,
  RoPE or cache index drops the cosine far below (tests/test_qwen3.py).
* The full-depth models (36 / 28 layers) at the BASELINE workloads
  (configs[3]: a 2048-token prefill and 128 greedy decode steps; configs[4]:
  the 1334 / 2393 / 3455-token prompts with 2 / 3 / 4 images) through
  properties that need no float reference: finite logits, decode continuing
  a prefill agrees with prefilling one token more (the decode MV has no
  activation quantization, so the two differ by that noise over 4 linears
  per layer; measured cosine above 0.999 at both depths, the bar is 0.995),
  chunked prefill of a multimodal prompt agrees with one-shot prefill, and
  HIP-graph decode reproduces eager decode token for token.
"""

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from cider_amd import qwen3 as Q  # noqa: E402
from cider_amd import qwen3vl as V  # noqa: E402
from tests import test_qwen3 as T3  # noqa: E402
from tests import test_qwen3vl as TV  # noqa: E402


def _cos(a, b):
    return torch.nn.functional.cosine_similarity(a.float().flatten(), b.float().flatten(),
                                                 dim=0).item()


def _close_width(a, b, what):
    a, b = a.float(), b.float()
    rel = (a - b).abs().max().item() / b.abs().max().item()
    c = _cos(a, b)
    assert rel < 8e-2 and c > 0.998, f"{what}: max rel {rel:.4f}, cosine {c:.6f}"


def test_qwen3_8b_width_two_layers_vs_fp32():
    cfg = Q.Qwen3Config(num_layers=2)           # every other field is Qwen3-8B's
    m = Q.Qwen3(cfg, max_len=128, seed=21)
    ids = torch.randint(0, cfg.vocab_size, (96,), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(22))
    got = m.prefill(ids)
    assert got.shape == (96, 151936) and torch.isfinite(got).all()
    ref = T3._ref_forward(m, ids)
    print(f"qwen3-8b width, 2 layers: cosine {_cos(got, ref):.6f}", flush=True)
    _close_width(got, ref, "qwen3-8b width, 2 layers")


def test_qwen3_vl_2b_width_two_layers_vs_fp32():
    cfg = Q.Qwen3Config(hidden_size=2048, intermediate_size=6144, num_layers=2, num_heads=16,
                        num_kv_heads=8, head_dim=128, vocab_size=151936,
                        rope_theta=V.QWEN3_VL_2B.rope_theta)
    m = V.Qwen3VL(cfg, max_len=600, seed=23)
    segs = V.synth_segments(540, 1, seed=24)
    x, _ = m.embed_prompt(segs, seed=25)
    pos3 = V.rope_index(segs)
    got = m.prefill_chunked(x, pos3, chunk=512)
    cos, sin = V.mrope_cos_sin(pos3.cuda(), cfg.head_dim, cfg.rope_theta)
    ref = TV._ref_forward(m, x, cos, sin)[-1:]
    print(f"qwen3-vl-2b width, 2 layers: cosine {_cos(got, ref):.6f}", flush=True)
    _close_width(got, ref, "qwen3-vl-2b width, 2 layers")


def test_qwen3_8b_config3_workload():
    """configs[3] at its workload: the full 36-layer Qwen3-8B shape, a prefill
    of 2048 ids uniform over the vocabulary, then 128 greedy decode steps.
    Checked by properties: finite logits over the whole prefill; decode at
    position 2048 agrees with prefilling one token more; the 128 steps
    replayed from a HIP graph equal eager decoding token for token; and the
    last step, attending over 2175 cached positions, agrees with a prefill of
    the whole generated sequence."""
    cfg = Q.QWEN3_8B
    assert cfg.num_layers == 36 and cfg.hidden_size == 4096 and cfg.vocab_size == 151936
    L, steps = 2048, 128
    a = Q.Qwen3(cfg, max_len=L + steps + 2, seed=31)
    ids = torch.randint(0, cfg.vocab_size, (L + 1,), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(32))
    full = a.prefill(ids)                        # positions 0..L
    assert full.shape == (L + 1, cfg.vocab_size) and torch.isfinite(full).all()
    a.prefill(ids[:L])                           # cache for 0..L-1
    dec = a.decode_step(ids[L:L + 1], torch.tensor([L], device="cuda"))
    assert torch.isfinite(dec).all()
    c = _cos(dec[0], full[L])
    print(f"qwen3-8b configs[3]: decode vs prefill at {L}: cosine {c:.6f}", flush=True)
    assert c > 0.995, f"decode vs prefill at position {L}: cosine {c:.5f}"
    del full
    # 128 greedy steps: graph replays reproduce eager decoding token for token
    ta = a.generate(ids[:L], steps, graph=True)
    tb = a.generate(ids[:L], steps, graph=False)
    assert ta.shape == (steps,) and torch.equal(ta, tb), \
        f"graph and eager decoding differ at step {int((ta != tb).nonzero()[0])}"
    print(f"qwen3-8b configs[3]: {steps} graph steps = eager, "
          f"{int(ta.unique().numel())} distinct tokens", flush=True)
    # the last decode step (slot L + steps - 1, 2175 positions) against a
    # prefill of prompt + generated tokens
    seq = torch.cat([ids[:L], ta])               # L + steps ids
    last = L + steps - 1
    ref = a.prefill(seq)[last]
    a.prefill(seq[:last])
    dec = a.decode_step(seq[last:last + 1], torch.tensor([last], device="cuda"))
    c = _cos(dec[0], ref)
    print(f"qwen3-8b configs[3]: decode vs prefill at {last}: cosine {c:.6f}", flush=True)
    assert c > 0.995, f"decode vs prefill at position {last}: cosine {c:.5f}"
    del a
    torch.cuda.empty_cache()


@pytest.mark.parametrize("L,n_img", [(1334, 2), (2393, 3), (3455, 4)])
def test_qwen3_vl_2b_config4_prompts(L, n_img):
    """configs[4] at its three prompts (1334 / 2393 / 3455 tokens with 2 / 3 /
    4 image blocks of 256 tokens, 3-axis M-RoPE positions), full 28-layer
    Qwen3-VL-2B shape: chunked prefill (chunk 512) agrees with one-shot
    prefill; decode continues the M-RoPE positions (the next token decoded
    agrees with prefilling it); HIP-graph decode reproduces eager decode
    token for token over 32 steps."""
    cfg = V.QWEN3_VL_2B
    assert cfg.num_layers == 28 and cfg.hidden_size == 2048 and cfg.vocab_size == 151936
    segs = V.synth_segments(L, n_img, seed=41 + L)
    assert sum(1 for kind, _ in segs if kind == "image") == n_img
    steps = 32
    m = V.Qwen3VL(cfg, max_len=L + steps + 2, seed=42)
    x, _ = m.embed_prompt(segs, seed=43)
    assert x.shape == (L, cfg.hidden_size)
    pos3 = V.rope_index(segs)
    chunked = m.prefill_chunked(x, pos3, chunk=512)
    assert torch.isfinite(chunked).all()
    one = m.prefill_chunked(x, pos3, chunk=L)
    c = _cos(chunked, one)
    print(f"qwen3-vl-2b {L} tokens: chunked vs one-shot cosine {c:.6f}", flush=True)
    assert c > 0.995, f"chunked vs one-shot prefill at {L} tokens: cosine {c:.5f}"
    # decode continues the M-RoPE positions: the next token decoded equals
    # prefilling it as text at the next position
    m.prefill_chunked(x, pos3, chunk=512)
    tok = torch.argmax(chunked[-1].float()).reshape(1)
    dec = m.decode_step(tok, torch.tensor([L], device="cuda"))
    x2 = torch.cat([x, m.embed.index_select(0, tok)])
    p2 = torch.cat([pos3, torch.full((3, 1), int(pos3.max()) + 1)], 1)
    full = m.prefill_chunked(x2, p2, chunk=512)
    c = _cos(dec[0], full[0])
    print(f"qwen3-vl-2b {L} tokens: decode vs prefill cosine {c:.6f}", flush=True)
    assert c > 0.995, f"decode vs prefill of the same token: cosine {c:.5f}"
    ta = m.generate_from_prompt(segs, steps, seed=43, chunk=512, graph=True)
    tb = m.generate_from_prompt(segs, steps, seed=43, chunk=512, graph=False)
    assert torch.equal(ta, tb)
    del m
    torch.cuda.empty_cache()

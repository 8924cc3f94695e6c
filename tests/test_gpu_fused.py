"""GPU parity of the producer kernels (RMSNorm / SwiGLU with the per-token
quantization fused in, per-head q/k norm + RoPE + cache write) and of the
single-query decode and prefill-chunk attention.

Bars:
  * quantization: q and scale_a bit-identical to the oracle's
    quantize_per_token (restating cider/kernels/w8a8_quantize.metal:33-86)
    applied to the fp16 tensor the producer itself returns;
  * residual add: bit-identical to fp16 addition;
  * RMSNorm / SwiGLU / RoPE outputs: the same chain of fp16 roundings
    evaluated in float64 on the CPU.  The kernel's fp32 sum of squares and exp
    differ from float64 in the last bits, which can move the rounding of the
    chain's first fp16 intermediate by one step: the output must equal the
    chain's for that intermediate or a neighbour (RoPE: within the error bound
    that step propagates to), and almost all elements must be identical;
  * decode attention: float64 softmax attention on the CPU, within fp16
    output rounding plus fp32 accumulation error (rtol 4e-3, atol 2e-3);
  * prefill attention: float64 causal softmax attention, within 3e-3 + 5e-3
    |ref| (the kernel rounds the probabilities to fp16 for the P.V product, as
    fused SDPA kernels do; PyTorch's SDPA lands at the same error).
"""

import math

import numpy as np
import pytest
import torch

from cider_amd import fused as F
from oracle import cider_oracle as O

pytestmark = pytest.mark.gpu


def _f16(a):
    return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float64)


def _ulp16(v):
    """fp16 ulp at |v| (normal range), as float64."""
    a = np.maximum(np.abs(v), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - 10)


def _rms_parts(h, w, eps):
    """float64 RMSNorm chain: t = h(h * r) and the weight, y = h(w * t)."""
    r = 1.0 / np.sqrt((h * h).sum(-1, keepdims=True) / h.shape[-1] + eps)
    return _f16(h * r), w


def _rms_ref(h, w, eps):
    t, w = _rms_parts(h, w, eps)
    return _f16(w * t)


def _assert_chain(got, t, w, what, max_frac=0.02):
    """got == h(w * t') with t' equal to t or one fp16 step either side: t is
    the float64 chain's rounded intermediate (h(h * r) for RMSNorm, h(silu(g))
    for SwiGLU); the kernel's fp32 sum of squares / exp may move that rounding
    by one step, which w scales before the final rounding."""
    t16 = t.astype(np.float16)
    lo = np.nextafter(t16, np.float16(-np.inf)).astype(np.float64)
    hi = np.nextafter(t16, np.float16(np.inf)).astype(np.float64)
    got = got.astype(np.float64)
    ok = (got == _f16(w * t)) | (got == _f16(w * lo)) | (got == _f16(w * hi))
    assert np.all(ok), f"{what}: {int(np.sum(~ok))} elements off by more than one step of t"
    frac = np.mean(got != _f16(w * t))
    assert frac <= max_frac, f"{what}: {frac:.4f} of the elements differ"


def _assert_rms(got, h, w, eps, what):
    t, w = _rms_parts(h, w, eps)
    _assert_chain(got, t, w, what)


def _quant_check(y_t, q_t, sa_t, what):
    y = y_t.cpu().numpy()
    q_ref, sa_ref = O.quantize_per_token(y)
    assert np.array_equal(q_t.cpu().numpy(), q_ref), f"{what}: q differs from the oracle"
    assert np.array_equal(sa_t.cpu().numpy().view(np.uint32),
                          np.asarray(sa_ref, dtype=np.float32).view(np.uint32)), \
        f"{what}: scale_a differs from the oracle"


RMS_SHAPES = [(1, 4096), (7, 2560), (300, 4096), (33, 12288), (5, 20480), (64, 8), (4, 264)]


@pytest.mark.parametrize("M,K", RMS_SHAPES)
@pytest.mark.parametrize("with_add", [False, True])
def test_rmsnorm_quantize(M, K, with_add):
    g = torch.Generator(device="cuda").manual_seed(M * 131 + K)
    x = (torch.randn(M, K, device="cuda", generator=g) * 3).half()
    w = (torch.rand(K, device="cuda", generator=g) * 2).half()
    add = (torch.randn(M, K, device="cuda", generator=g)).half() if with_add else None
    r = F.rmsnorm_quantize(x, w, 1e-6, add=add)
    torch.cuda.synchronize()
    h = x if add is None else x + add
    if add is not None:
        assert torch.equal(r.h, h), "residual sum is not the fp16 sum"
    _assert_rms(r.y.cpu().numpy(), h.double().cpu().numpy(), w.double().cpu().numpy(), 1e-6,
                f"rmsnorm y M={M} K={K}")
    _quant_check(r.y, r.q, r.scale_a, f"rmsnorm q M={M} K={K}")
    # q-only launch computes the same q
    r2 = F.rmsnorm_quantize(x, w, 1e-6, add=add, want_y=False)
    assert torch.equal(r2.q, r.q) and torch.equal(r2.scale_a, r.scale_a)


def test_rmsnorm_in_place_residual_and_special_rows():
    K = 1024
    x = torch.randn(6, K, device="cuda").half()
    x[1] = 0                       # zero row: y = 0, scale 1, q = 0
    x[2] = 2.5                     # constant row: y = h(w * h(2.5 / sqrt(6.25 + eps)))
    add = torch.zeros_like(x)
    w = torch.ones(K, device="cuda", dtype=torch.float16)
    x0 = x.clone()
    r = F.rmsnorm_quantize(x, w, 1e-6, add=add, sum_out=x)   # h written over x
    torch.cuda.synchronize()
    assert torch.equal(x, x0) and r.h.data_ptr() == x.data_ptr()
    assert torch.all(r.y[1] == 0) and torch.all(r.q[1] == 0) and r.scale_a[1].item() == 1.0
    one = np.float16(2.5 / math.sqrt(6.25 + 1e-6))
    assert torch.all(r.y[2].cpu() == torch.tensor(float(one)).half())
    assert torch.all(r.q[2] == 127)


# a workgroup per row up to I = 16384 at every M (ragged last vector group at
# I = 6152), a wave per row streaming above (I = 24576, 16392)
SWI_SHAPES = [(1, 12288), (3, 6144), (129, 4096), (2, 24576), (16, 8), (300, 12288),
              (517, 6152), (70, 16392)]


@pytest.mark.parametrize("M,I", SWI_SHAPES)
def test_silu_mul_quantize(M, I):
    g = torch.Generator(device="cuda").manual_seed(M + I)
    gu = (torch.randn(M, 2 * I, device="cuda", generator=g) * 3).half()
    y, q, sa = F.silu_mul_quantize(gu)
    torch.cuda.synchronize()
    a = gu[:, :I].double().cpu().numpy()
    u = gu[:, I:].double().cpu().numpy()
    _assert_chain(y.cpu().numpy(), _f16(a / (1.0 + np.exp(-a))), u, f"swiglu M={M} I={I}")
    _quant_check(y, q, sa, f"swiglu q M={M} I={I}")
    _, q2, sa2 = F.silu_mul_quantize(gu, want_y=False)
    assert torch.equal(q2, q) and torch.equal(sa2, sa)


def _rope_tables(P, D=128, theta=1e6):
    inv = 1.0 / (theta ** (np.arange(0, D, 2) / D))
    f = np.outer(np.arange(P), inv)
    emb = np.concatenate([f, f], -1)
    return np.cos(emb).astype(np.float16), np.sin(emb).astype(np.float16)


@pytest.mark.parametrize("L,H,KV", [(1, 32, 8), (37, 16, 8), (5, 4, 4)])
def test_qk_norm_rope_and_cache(L, H, KV):
    D, T, P = 128, 96, 200
    g = torch.Generator(device="cuda").manual_seed(L * 7 + H)
    qkv = (torch.randn(L, (H + 2 * KV) * D, device="cuda", generator=g) * 2).half()
    qw = (torch.rand(D, device="cuda", generator=g) + 0.5).half()
    kw = (torch.rand(D, device="cuda", generator=g) + 0.5).half()
    cos_np, sin_np = _rope_tables(P)
    cos, sin = torch.from_numpy(cos_np).cuda(), torch.from_numpy(sin_np).cuda()
    rope_row = torch.randint(0, P, (L,), device="cuda", generator=g)
    slot = torch.randperm(T, device="cuda", generator=g)[:L].contiguous()
    kc = torch.zeros(KV, T, D, dtype=torch.float16, device="cuda")
    vc = torch.zeros(KV, T, D, dtype=torch.float16, device="cuda")
    q = F.qk_norm_rope(qkv, qw, kw, 1e-6, cos, sin, rope_row, slot, kc, vc, H, KV)
    torch.cuda.synchronize()

    x = qkv.double().cpu().numpy().reshape(L, H + 2 * KV, D)
    rr = rope_row.cpu().numpy()
    c, s = cos_np.astype(np.float64)[rr][:, None, :], sin_np.astype(np.float64)[rr][:, None, :]

    def ref(part, w):
        """(expected out, error bound): the norm output n may be one step of
        its intermediate off (scaled by w, then rounded), which the rotation
        carries with |cos| and |sin| into two rounded products and a rounded
        sum; bound = 2 fp16 steps of each product plus one of the result."""
        n = _rms_ref(part, w.double().cpu().numpy(), 1e-6)
        rot = np.concatenate([-n[..., D // 2:], n[..., :D // 2]], -1)
        a, b = _f16(n * c), _f16(rot * s)
        out = _f16(a + b)
        return out, 2 * (_ulp16(a) + _ulp16(b)) + _ulp16(out)

    def check(got, exp_bound, what):
        exp, bound = exp_bound
        diff = np.abs(got.astype(np.float64) - exp)
        assert np.all(diff <= bound), f"{what}: {int(np.sum(diff > bound))} beyond the bound"
        assert np.mean(diff > 0) <= 0.03, f"{what}: {np.mean(diff > 0):.4f} differ"

    check(q.cpu().numpy(), ref(x[:, :H], qw), "q")
    k_exp = ref(x[:, H:H + KV], kw)
    sl = slot.cpu().numpy()
    k_got = kc.cpu().numpy().astype(np.float64)[:, sl, :].transpose(1, 0, 2)   # [L, KV, D]
    check(k_got, k_exp, "k cache")
    v_got = vc.cpu().numpy()[:, sl, :].transpose(1, 0, 2)
    assert np.array_equal(v_got, qkv.cpu().numpy().reshape(L, H + 2 * KV, D)[:, H + KV:])
    untouched = np.setdiff1d(np.arange(T), sl)
    assert np.all(kc.cpu().numpy()[:, untouched, :] == 0)
    assert np.all(vc.cpu().numpy()[:, untouched, :] == 0)


def test_qk_norm_rope_skips_out_of_range_slots():
    H, KV, D, T = 4, 2, 128, 16
    qkv = torch.randn(2, (H + 2 * KV) * D, device="cuda").half()
    w = torch.ones(D, device="cuda", dtype=torch.float16)
    cos_np, sin_np = _rope_tables(8)
    cos, sin = torch.from_numpy(cos_np).cuda(), torch.from_numpy(sin_np).cuda()
    kc = torch.zeros(KV, T, D, dtype=torch.float16, device="cuda")
    vc = torch.zeros(KV, T, D, dtype=torch.float16, device="cuda")
    rope_row = torch.tensor([1, 2], device="cuda")
    slot = torch.tensor([3, T], device="cuda")     # the second token has no slot
    F.qk_norm_rope(qkv, w, w, 1e-6, cos, sin, rope_row, slot, kc, vc, H, KV)
    torch.cuda.synchronize()
    written = (kc != 0).any(dim=2).any(dim=0).cpu().numpy()
    assert written[3] and written.sum() == 1
    assert torch.equal(vc[:, 3], qkv[0].reshape(H + 2 * KV, D)[H + KV:])
    # a token without a RoPE row: its q heads are NaN (not stale memory), and
    # it writes no k row even where its slot is valid
    kc.zero_()
    q = F.qk_norm_rope(qkv, w, w, 1e-6, cos, sin, torch.tensor([1, 8], device="cuda"),
                       torch.tensor([3, 5], device="cuda"), kc, vc, H, KV)
    torch.cuda.synchronize()
    assert torch.isfinite(q[0]).all() and torch.isnan(q[1]).all()
    written = (kc != 0).any(dim=2).any(dim=0).cpu().numpy()
    assert written[3] and written.sum() == 1


def _attn_ref(q, kc, vc, n, scale):
    H, D = q.shape
    KV = kc.shape[0]
    G = H // KV
    out = np.zeros((H, D))
    for h in range(H):
        j = h // G
        s = scale * (kc[j][:n] @ q[h])
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vc[j][:n]
    return out


@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("n", [1, 127, 128, 129, 600, 640, 645])
def test_attn_decode(G, n):
    KV, D, T = 2, 128, 640
    H = KV * G
    g = torch.Generator(device="cuda").manual_seed(G * 1000 + n)
    q = torch.randn(H, D, device="cuda", generator=g).half()
    kc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    vc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    # positions >= n hold garbage that must not leak into the result
    nn = min(n, T)
    kc[:, nn:, :] = float("nan")
    vc[:, nn:, :] = float("nan")
    nv = torch.tensor([n], device="cuda")
    scale = 1.0 / math.sqrt(D)
    out = F.attn_decode(q, kc, vc, nv, scale)
    torch.cuda.synchronize()
    exp = _attn_ref(q.double().cpu().numpy(), kc.double().cpu().numpy()[:, :nn],
                    vc.double().cpu().numpy()[:, :nn], nn, scale)
    got = out.double().cpu().numpy().reshape(H, D)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, exp, rtol=4e-3, atol=2e-3)


def test_attn_decode_graph_replays_follow_device_length():
    KV, G, D, T = 8, 4, 128, 512
    H = KV * G
    q = torch.randn(H, D, device="cuda").half()
    kc = torch.randn(KV, T, D, device="cuda").half()
    vc = torch.randn(KV, T, D, device="cuda").half()
    nv = torch.tensor([1], device="cuda")
    ws = F.attn_decode_workspace(H, T, "cuda")
    out = torch.empty(H * D, dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        F.attn_decode(q, kc, vc, nv, 0.1, ws=ws, out=out)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        F.attn_decode(q, kc, vc, nv, 0.1, ws=ws, out=out)
    for n in (3, 130, 257, 512, 40):
        nv.fill_(n)
        eager = F.attn_decode(q, kc, vc, nv, 0.1)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"n={n}"


def _prefill_ref(q, kc, vc, c, n, scale):
    """float64 causal attention of the chunk q [c, H, D] (cache slots
    n - c .. n - 1) over kc / vc [KV, >= n, D], on the GPU in float64."""
    H, D = q.shape[1], q.shape[2]
    KV = kc.shape[0]
    G = H // KV
    allowed = torch.ones(c, n, dtype=torch.bool, device=q.device).tril(diagonal=n - c)
    out = torch.empty(c, H, D, dtype=torch.float64, device=q.device)
    for h in range(H):
        j = h // G
        k = kc[j, :n].double()
        s = scale * (q[:, h].double() @ k.T.contiguous())
        s = s.masked_fill(~allowed, float("-inf"))
        out[:, h] = torch.softmax(s, dim=-1) @ vc[j, :n].double()
    return out


# (c, n, H, KV, T, q scale): the Qwen3-8B 2048-token prefill, Qwen3-VL chunks
# after earlier slots, ragged lengths and capacities (the last stage past n),
# one query, every grouping 1..8, KV not a multiple of 8 (the plain item
# order), and peaked softmaxes (large logits exercise the running-max slack).
PREFILL_CASES = [
    (2048, 2048, 32, 8, 2048, 1.0), (512, 2048, 16, 8, 2304, 1.0), (777, 777, 32, 8, 800, 1.0),
    (100, 1000, 16, 8, 1024, 1.0), (1, 37, 32, 8, 64, 1.0), (130, 130, 8, 8, 136, 1.0),
    (64, 200, 64, 8, 256, 1.0), (300, 300, 12, 4, 320, 1.0), (257, 513, 5, 1, 520, 1.0),
    (640, 1280, 32, 8, 1280, 6.0), (300, 1500, 16, 8, 1536, 10.0), (129, 129, 16, 8, 4096, 1.0),
    # chunk offsets n - c between 32 and 64: a wave's queries straddle key 64, so some lanes
    # find every key of their set's first block masked while others do not
    (100, 140, 8, 8, 144, 1.0), (60, 105, 16, 8, 128, 3.0), (24, 72, 4, 2, 512, 1.0),
]


@pytest.mark.parametrize("c,n,H,KV,T,qs", PREFILL_CASES)
def test_attn_prefill(c, n, H, KV, T, qs):
    D = 128
    g = torch.Generator(device="cuda").manual_seed(c * 7 + n + H)
    q = (torch.randn(c, H, D, device="cuda", generator=g) * qs).half()
    kc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    vc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    # slots >= n hold garbage that must not leak into the result
    kc[:, n:, :] = float("nan")
    vc[:, n:, :] = float("nan")
    scale = 1.0 / math.sqrt(D)
    out = F.attn_prefill(q, kc, vc, n, scale)
    torch.cuda.synchronize()
    exp = _prefill_ref(q, kc, vc, c, n, scale)
    got = out.double().reshape(c, H, D)
    assert torch.isfinite(got).all()
    err = (got - exp).abs()
    tol = 3e-3 + 5e-3 * exp.abs()
    assert bool((err <= tol).all()), f"max err {err.max().item():.3e}"


# chunks whose query blocks fill few CUs split their keys over parts (a first
# chunk of 1024: the first query block's first part holds no stage at all;
# later chunks: 2-8 parts); the unsplit launch is held to the same bar
SPLIT_CASES = [(1024, 1024, 8, 8, 1024), (512, 2048, 16, 8, 2048), (383, 3455, 16, 8, 3584),
               (100, 1000, 32, 8, 1024), (128, 4096, 8, 8, 4096)]


@pytest.mark.parametrize("c,n,H,KV,T", SPLIT_CASES)
def test_attn_prefill_split_and_unsplit(c, n, H, KV, T):
    from cider_amd import _lib
    D = 128
    assert _lib.load().cider_attn_prefill_workspace_bytes(c, n, H) > 0, "expected a split launch"
    g = torch.Generator(device="cuda").manual_seed(c + 3 * n)
    q = torch.randn(c, H, D, device="cuda", generator=g).half()
    kc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    vc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    kc[:, n:, :] = float("nan")
    vc[:, n:, :] = float("nan")
    scale = 1.0 / math.sqrt(D)
    ws = F.attn_prefill_workspace(c, n, H, "cuda")
    ws.fill_(0xFF)  # stale partials must not matter
    split = F.attn_prefill(q, kc, vc, n, scale, ws=ws)
    plain = F.attn_prefill(q, kc, vc, n, scale, split=False)
    torch.cuda.synchronize()
    exp = _prefill_ref(q, kc, vc, c, n, scale)
    for got in (split, plain):
        got = got.double().reshape(c, H, D)
        assert torch.isfinite(got).all()
        err = (got - exp).abs()
        assert bool((err <= 3e-3 + 5e-3 * exp.abs()).all()), f"max err {err.max().item():.3e}"


# The attention with its output quantized for o_proj: q and sa are, bit for
# bit, the oracle's quantize_per_token of attn_prefill's fp16 output with the
# same key split -- split launches (quantized in the merge), launches that fill
# the GPU (the fp16 output staged in the workspace), 1..128 heads (one to
# eight vectors per merge thread), a workspace of c * H * 256 bytes (one part),
# the length read on the device, and stale workspace contents.
QUANT_CASES = SPLIT_CASES + [(2048, 2048, 32, 8, 2048), (1, 37, 32, 8, 64), (100, 140, 8, 8, 144),
                             (257, 2000, 5, 1, 2048), (64, 1200, 64, 8, 1280),
                             (16, 1100, 128, 8, 1152), (16, 300, 128, 8, 320)]


@pytest.mark.parametrize("c,n,H,KV,T", QUANT_CASES)
def test_attn_prefill_quantize_bits(c, n, H, KV, T):
    D = 128
    print(f"attn_prefill_quantize c={c} n={n} H={H} KV={KV} T={T}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(c + 5 * n + H)
    q = (torch.randn(c, H, D, device="cuda", generator=g) * 2).half()
    kc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    vc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    kc[:, n:, :] = float("nan")
    vc[:, n:, :] = float("nan")
    scale = 1.0 / math.sqrt(D)
    wsq = F.attn_prefill_quantize_workspace(c, n, H, "cuda")
    wsq.fill_(0xFF)
    qa, sa = F.attn_prefill_quantize(q, kc, vc, n, scale, ws=wsq)
    out = F.attn_prefill(q, kc, vc, n, scale, ws=F.attn_prefill_workspace(c, n, H, "cuda"))
    _quant_check(out, qa, sa, f"attn q c={c} n={n} H={H}")
    n_dev = torch.tensor([n], dtype=torch.int64, device="cuda")
    qd, sd = F.attn_prefill_quantize(q, kc, vc, n, scale, ws=wsq, n_dev=n_dev)
    assert torch.equal(qd, qa) and torch.equal(sd, sa), "device length"
    small = torch.full((c * H * 256,), 0xFF, dtype=torch.uint8, device="cuda")
    q1, s1 = F.attn_prefill_quantize(q, kc, vc, n, scale, ws=small)
    plain = F.attn_prefill(q, kc, vc, n, scale, split=False)
    _quant_check(plain, q1, s1, f"attn q one part c={c} n={n} H={H}")


def test_attn_prefill_chunks_match_one_shot():
    """Chunks of 512 after earlier slots (the Qwen3-VL prefill) give what one
    launch over the whole prompt gives, within the same bar."""
    c, H, KV, D, T = 1500, 16, 8, 128, 1536
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn(c, H, D, device="cuda", generator=g).half()
    kc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    vc = torch.randn(KV, T, D, device="cuda", generator=g).half()
    one = F.attn_prefill(q, kc, vc, c, 0.09).double()
    parts = [F.attn_prefill(q[s:s + 512].contiguous(), kc, vc, min(s + 512, c), 0.09).double()
             for s in range(0, c, 512)]
    torch.cuda.synchronize()
    err = (torch.cat(parts) - one).abs()
    assert bool((err <= 3e-3 + 5e-3 * one.abs()).all()), f"max err {err.max().item():.3e}"


# Decode producers run inside the consuming M == 1 linear: bit-identical to
# the producer launch followed by the linear on its fp16 output.
def _pc_linear(N, K, seed):
    from cider_amd import nn as cnn
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    sw = torch.rand(N, device="cuda", generator=g) * 9e-3 + 1e-3
    b = (torch.randn(N, device="cuda", generator=g) * 0.1).half()
    return cnn.CiderLinear(w, sw, 0, K, N, b)


@pytest.mark.parametrize("N,K,with_add", [(6144, 4096, True), (24576, 4096, True),
                                          (4096, 2048, False), (33, 16384, True),
                                          (40, 256, False), (3000, 2560, True),
                                          (2560, 10240, False), (2560, 10240, True),
                                          (4096, 12288, True)])
def test_rmsnorm_mv_equals_two_launches(N, K, with_add):
    g = torch.Generator(device="cuda").manual_seed(N + K)
    x = (torch.randn(1, K, device="cuda", generator=g) * 3).half()
    add = torch.randn(1, K, device="cuda", generator=g).half() if with_add else None
    w = (torch.rand(K, device="cuda", generator=g) * 2).half()
    lin = _pc_linear(N, K, N * 3 + K)
    h, y = F.rmsnorm_mv(x, w, 1e-6, lin, add=add)
    r = F.rmsnorm_quantize(x, w, 1e-6, add=add, want_q=False)
    y2 = lin(r.y)
    torch.cuda.synchronize()
    assert torch.equal(h.view(-1), r.h.view(-1)), "residual sum differs"
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), f"rmsnorm_mv {N}x{K}"


@pytest.mark.parametrize("N,I", [(4096, 12288), (2048, 6144), (33, 512), (4096, 16384),
                                 (2560, 10240), (7, 15360)])
def test_swiglu_mv_equals_two_launches(N, I):
    g = torch.Generator(device="cuda").manual_seed(N + I)
    gu = (torch.randn(1, 2 * I, device="cuda", generator=g) * 3).half()
    lin = _pc_linear(N, I, N * 5 + I)
    y = F.swiglu_mv(gu, lin)
    hs, _, _ = F.silu_mul_quantize(gu, want_y=True, want_q=False)
    y2 = lin(hs)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), f"swiglu_mv {N}x{I}"


def test_producer_mv_rejects_unsupported_shapes():
    lin = _pc_linear(16, 264, 1)
    x = torch.randn(1, 264, device="cuda").half()
    w = torch.ones(264, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="256"):
        F.rmsnorm_mv(x, w, 1e-6, lin)

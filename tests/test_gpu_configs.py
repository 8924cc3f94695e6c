"""Parity at every BASELINE configuration's workload size.

configs[1] (W8A8, both shapes, per-channel / per-group gs 128 / gs 64, M in
{1, 128, 1024, 4096, 8192}) and configs[2] (W4A8, both shapes, M in {1, 16,
512, 4096}: the per-group int4 format with fp16 scales at gs 64 / 128, and
the reference's per-column int4 layout, through the functional API and
through the one-call C entry ``cider_w4a8_linear_ref``).  Each case runs the
whole problem on the GPU (so the dispatcher picks the kernel and grid it
picks in production) and compares rows against the CPU oracle: all rows at
M <= 16, otherwise the first 16, the last 16 and 16 seeded random rows.
Bar: bit-exact for the per-channel GEMMs and the reference W4 layout; the
per-group formats within the per-group bar of tests/util.py (their DMA
kernels flush with fused multiply-adds and split K at mid M); the M == 1 MV
within the MV bar.
"""

import ctypes
import functools

import numpy as np
import pytest

from oracle import cider_oracle as O
from tests.util import assert_bits_equal, assert_mv_close, assert_pergroup_linear_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import cider_amd as C
    from cider_amd import _lib

DEV = "cuda"
SHAPES_W8 = [(10240, 2560), (2560, 10240)]
SHAPES_W4 = [(12288, 4096), (4096, 12288)]


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def H(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rows_of(M, seed):
    if M <= 16:
        return np.arange(M)
    rnd = np.random.default_rng(seed).choice(np.arange(16, M - 16), 16, replace=False)
    return np.unique(np.r_[0:16, M - 16:M, rnd])


@functools.lru_cache(maxsize=2)
def acts(M, K):
    return O.synth_activations(M, K, 20261201 + M + K)


@functools.lru_cache(maxsize=2)
def w8(N, K):
    return O.synth_weights_i8(N, K, 20261202 + N)


@functools.lru_cache(maxsize=2)
def w4_values(N, K):
    return np.random.default_rng(20261203 + N).integers(-8, 8, (N, K), dtype=np.int8)


@functools.lru_cache(maxsize=2)
def w4_ref_layout(N, K):
    wf = np.random.default_rng(20261204 + N).standard_normal((K, N)).astype(np.float32)
    return O.pack_weight_int4(wf)


@pytest.mark.parametrize("mode", ["pc", "gs128", "gs64"])
@pytest.mark.parametrize("N,K", SHAPES_W8)
@pytest.mark.parametrize("M", [1, 128, 1024, 4096, 8192])
def test_config1_w8a8(M, N, K, mode):
    print(f"config1 M={M} N={N} K={K} {mode}", flush=True)
    x, w = acts(M, K), w8(N, K)
    rows = rows_of(M, M + N)
    if mode == "pc":
        sw = O.synth_scales(N, 7)
        y = H(C.perchannel_linear(T(x), T(w), T(sw)))
        if M == 1:
            assert_mv_close(y, x, w, sw, None, 0, f"pc mv {N}x{K}")
            return
        exp = O.perchannel_linear(x[rows], w, sw)
    else:
        gs = int(mode[2:])
        sw = O.synth_scales((K // gs, N), 8 + gs)
        y = H(C.pergroup_linear(T(x), T(w), T(sw), gs))
        if M == 1:
            assert_mv_close(y, x, w, sw, None, gs, f"pg{gs} mv {N}x{K}")
            return
        exp = O.pergroup_gemm(*O.quantize_per_token(x[rows]), w, sw, np.zeros(N, np.float16), gs)
        assert y.shape == (M, N)
        assert_pergroup_linear_close(y[rows], x[rows], w, sw, None, gs, exp,
                                     f"config1 {mode} {M}x{N}x{K}")
        return
    assert y.shape == (M, N)
    assert_bits_equal(y[rows], exp, f"config1 {mode} {M}x{N}x{K}")


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("N,K", SHAPES_W4)
@pytest.mark.parametrize("M", [1, 16, 512, 4096])
def test_config2_w4a8_pergroup(M, N, K, gs):
    print(f"config2 pergroup M={M} N={N} K={K} gs={gs}", flush=True)
    x = acts(M, K)
    packed = O.pack_w4_lo_first(w4_values(N, K))
    sc = O.synth_scales((K // gs, N), 9 + gs).astype(np.float16)
    y = H(C.w4a8_pergroup_linear(T(x), T(packed), T(sc), gs))
    rows = rows_of(M, M + N + gs)
    assert y.shape == (M, N)
    assert_pergroup_linear_close(y[rows], x[rows], w4_values(N, K), sc, None, gs,
                                 O.w4a8_pergroup_linear(x[rows], packed, sc, gs),
                                 f"config2 w4g{gs} {M}x{N}x{K}")


def _w4a8_linear_ref_capi(x, packed, sw):
    """cider_w4a8_linear_ref through the C ABI, workspace from torch."""
    lib = _lib.load()
    M, K = x.shape
    N = packed.shape[1]
    xd, pd, sd = T(x), T(packed), T(sw)
    y = torch.empty((M, N), dtype=torch.float16, device=DEV)
    nb = _lib.workspace_bytes(_lib.CIDER_OP_W4A8_REF, M, N, K)
    ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
    rc = lib.cider_w4a8_linear_ref(xd.data_ptr(), pd.data_ptr(), sd.data_ptr(), y.data_ptr(),
                                   ws.data_ptr(), nb, M, N, K,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc)
    return H(y)


@pytest.mark.parametrize("N,K", SHAPES_W4)
@pytest.mark.parametrize("M", [1, 16, 512, 4096])
def test_config2_w4a8_reference_layout(M, N, K):
    print(f"config2 ref layout M={M} N={N} K={K}", flush=True)
    x = acts(M, K)
    packed, sw = w4_ref_layout(N, K)
    rows = rows_of(M, M + N)
    exp = O.w4a8_linear(x[rows], packed, sw)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw)))
    assert_bits_equal(y[rows], exp, f"config2 w4 ref {M}x{N}x{K}")
    y1 = _w4a8_linear_ref_capi(x, packed, sw)
    assert_bits_equal(y1, y, f"one-call C entry {M}x{N}x{K}")


# int4 weights at the configs[1] shapes: the 192 x 256 tile runs its 4-slot
# ring past the wrap at K=2560 (M=1024) and at M=4096, N=2560, K=10240.
@pytest.mark.parametrize("M,N,K", [(1024, 10240, 2560), (4096, 2560, 10240)])
def test_w4_reference_layout_at_config1_shapes(M, N, K):
    x = acts(M, K)
    packed, sw = w4_ref_layout(N, K)
    rows = rows_of(M, M + K)
    y = H(C.w4a8_linear(T(x), T(packed), T(sw)))
    assert_bits_equal(y[rows], O.w4a8_linear(x[rows], packed, sw), f"w4 {M}x{N}x{K}")


def test_w4a8_module_follows_weight_updates():
    """W4A8Linear remakes its library-layout copy when packed_weight changes:
    in place, and through load_state_dict."""
    K, N = 512, 96
    rng = np.random.default_rng(31)
    wa = rng.standard_normal((K, N)).astype(np.float32)
    wb = rng.standard_normal((K, N)).astype(np.float32)
    layer = C.W4A8Linear.from_weights(wa, device=DEV)
    x = O.synth_activations(5, K, 32)
    pa, sa = O.pack_weight_int4(wa)
    pb, sb = O.pack_weight_int4(wb)
    assert_bits_equal(H(layer(T(x))), O.w4a8_linear(x, pa, sa), "before")
    other = C.W4A8Linear.from_weights(wb, device=DEV)
    layer.load_state_dict(other.state_dict())
    assert_bits_equal(H(layer(T(x))), O.w4a8_linear(x, pb, sb), "after load_state_dict")
    with torch.no_grad():
        layer.packed_weight.copy_(T(pa))
        layer.scale.copy_(T(sa))
    assert_bits_equal(H(layer(T(x))), O.w4a8_linear(x, pa, sa), "after copy_")


def test_functional_w4a8_cache_across_streams():
    """The repack cache hands a copy made on one stream to a call on another:
    that call waits for the repack, and an in-place update of the source is
    seen by the next call."""
    K, N, M = 1024, 256, 70
    rng = np.random.default_rng(33)
    packed, sw = O.pack_weight_int4(rng.standard_normal((K, N)).astype(np.float32))
    x = O.synth_activations(M, K, 34)
    pd, sd, xd = T(packed), T(sw), T(x)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        y1 = C.w4a8_linear(xd, pd, sd, stream=s1)
    with torch.cuda.stream(s2):
        y2 = C.w4a8_linear(xd, pd, sd, stream=s2)
    torch.cuda.synchronize()
    exp = O.w4a8_linear(x, packed, sw)
    assert_bits_equal(y1.cpu().numpy(), exp, "stream 1")
    assert_bits_equal(y2.cpu().numpy(), exp, "stream 2")
    packed2, sw2 = O.pack_weight_int4(rng.standard_normal((K, N)).astype(np.float32))
    pd.copy_(T(packed2))
    sd.copy_(T(sw2))
    assert_bits_equal(H(C.w4a8_linear(xd, pd, sd)), O.w4a8_linear(x, packed2, sw2), "updated")


def test_w4a8_module_across_streams():
    """W4A8Linear's library-layout copy, made on one stream, is used on
    another: the second stream waits for the repack."""
    K, N, M = 1024, 192, 40
    rng = np.random.default_rng(35)
    w = rng.standard_normal((K, N)).astype(np.float32)
    layer = C.W4A8Linear.from_weights(w, device=DEV)
    packed, sw = O.pack_weight_int4(w)
    x = O.synth_activations(M, K, 36)
    xd = T(x)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        y1 = layer(xd)
    with torch.cuda.stream(s2):
        y2 = layer(xd)
    torch.cuda.synchronize()
    exp = O.w4a8_linear(x, packed, sw)
    assert_bits_equal(y1.cpu().numpy(), exp, "stream 1 (repack)")
    assert_bits_equal(y2.cpu().numpy(), exp, "stream 2 (cached copy)")


def test_repack_cache_one_finalizer_per_source():
    """Repeated misses on one live source tensor (in-place updates) replace
    its cache entry without stacking finalizers."""
    from cider_amd import ops as OPS
    K, N = 256, 64
    rng = np.random.default_rng(37)
    packed, sw = O.pack_weight_int4(rng.standard_normal((K, N)).astype(np.float32))
    x = O.synth_activations(3, K, 38)
    pd, sd, xd = T(packed), T(sw), T(x)
    cache = OPS._repack_cache
    for i in range(4):
        packed_i, sw_i = O.pack_weight_int4(rng.standard_normal((K, N)).astype(np.float32))
        pd.copy_(T(packed_i))
        sd.copy_(T(sw_i))
        assert_bits_equal(H(C.w4a8_linear(xd, pd, sd)), O.w4a8_linear(x, packed_i, sw_i),
                          f"update {i}")
        fin = cache._fins[id(pd)][1]
        if i == 0:
            first = fin
        assert fin is first and fin.alive
    del pd
    import gc
    gc.collect()
    assert not first.alive

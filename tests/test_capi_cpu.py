"""CPU tier: the C-ABI library loads, exports every symbol that
include/cider_hip.h declares, and validates arguments without touching a GPU;
the host-side weight quantizers match the oracle; CPU tensors are rejected.
"""

import ctypes
import os
import re

import numpy as np
import pytest

from oracle import cider_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cider_hip.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(cider_[a-z0-9_]+)\(",
                                 text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from cider_amd import _lib
    return _lib.load()


def test_header_declares_entry_points():
    syms = header_symbols()
    assert "cider_perchannel_linear" in syms and "cider_int8_matmul_int32" in syms
    assert len(syms) == 24, syms


@pytest.mark.parametrize("lang,compiler", [("c", "gcc"), ("c++", "g++")])
def test_header_compiles_as_c_and_cpp(lang, compiler, tmp_path):
    """The header is what a binding (cgo, JNI, ctypes' C stub) includes: it
    must compile on its own as C and as C++."""
    import shutil
    import subprocess
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    r = subprocess.run([compiler, "-fsyntax-only", "-Wall", "-Werror", "-x", lang, HEADER],
                       capture_output=True, text=True, cwd=tmp_path)
    assert r.returncode == 0, r.stderr


def test_library_exports_every_header_symbol(lib):
    from cider_amd import _lib
    syms = header_symbols()
    assert sorted(_lib.SIGNATURES) == syms
    for s in syms:
        assert hasattr(lib, s), s
    assert lib.cider_version() >= 100


def test_workspace_bytes(lib):
    from cider_amd import _lib
    ws = _lib.workspace_bytes
    assert ws(_lib.CIDER_OP_PERCHANNEL, 1, 10240, 2560) == 0
    assert ws(_lib.CIDER_OP_PERGROUP, 1, 10240, 2560, 128) == 0
    # quantized activations + per-token scales, each 256-byte aligned
    assert ws(_lib.CIDER_OP_PERCHANNEL, 4096, 10240, 2560) == 4096 * 2560 + 4096 * 4
    assert ws(_lib.CIDER_OP_W4A8, 1, 64, 64) == 256 + 256
    assert ws(_lib.CIDER_OP_PERCHANNEL, 3, 8, 10) == 256 + 256
    assert ws(_lib.CIDER_OP_PERCHANNEL, 0, 8, 10) == 0
    # the one-call reference-layout W4A8 adds room for the repacked weights
    assert ws(_lib.CIDER_OP_W4A8_REF, 4096, 12288, 4096) == \
        4096 * 4096 + 4096 * 4 + 12288 * 2048
    assert ws(_lib.CIDER_OP_W4A8_REF, 1, 70, 64) == 256 + 256 + 2304


def test_splitk_workspace_respects_32bit_tile_offsets(lib):
    """The split-K GEMM's tiles address rows by 32-bit per-lane offsets; K
    with K * 256 >= 2**32 must run one pass (no partial-sum part in the
    workspace), while the usual mid-M shapes keep their K slices."""
    from cider_amd import _lib
    ws = _lib.workspace_bytes

    def quant(M, K):
        a = lambda v: (v + 255) // 256 * 256
        return a(M * K) + a(4 * M)

    # M=128 N=2560 K=10240: 20 tiles of 128 x 128, 8 slices of the int32 sums
    assert ws(_lib.CIDER_OP_PERCHANNEL, 128, 2560, 10240) == \
        quant(128, 10240) + 8 * 128 * 2560 * 4
    # M=256 N=2560 K=10240: 160 tiles of 64 x 64 leave CUs idle, 4 slices
    assert ws(_lib.CIDER_OP_PERCHANNEL, 256, 2560, 10240) == \
        quant(256, 10240) + 4 * 256 * 2560 * 4
    # M=512 N=2048 K=2048: 64 tiles of 128 x 128, but 256 tiles of 64 x 64
    # fill the CUs, so one pass
    assert ws(_lib.CIDER_OP_PERCHANNEL, 512, 2048, 2048) == quant(512, 2048)
    # one tile, K = 2**26: 2**26 * 256 = 2**34 bytes of offsets, no split
    assert ws(_lib.CIDER_OP_PERCHANNEL, 32, 128, 1 << 26) == quant(32, 1 << 26)
    # just below the limit the split still applies
    k = (1 << 24) - 1024
    assert ws(_lib.CIDER_OP_PERCHANNEL, 32, 128, k) > quant(32, k)


def test_pergroup_splitk_workspace(lib):
    """The per-group linears size fp32 partial chains of their K slices (256
    CUs assumed without a GPU): 40 tiles of 128 x 64 at M=128 N=2560 K=10240
    take 4 slices, and so do its 80 tiles of 64 x 64 at gs 256; the 128 tiles
    of 128 x 128 at M=512 N=4096 K=12288 take 4 (512 workgroups of the
    one-set kernel); grids that fill the CUs, short K and M <= 64 take none."""
    from cider_amd import _lib
    ws = _lib.workspace_bytes

    def quant(M, K):
        a = lambda v: (v + 255) // 256 * 256
        return a(M * K) + a(4 * M)

    assert ws(_lib.CIDER_OP_PERGROUP, 128, 2560, 10240, 128) == \
        quant(128, 10240) + 4 * 128 * 2560 * 4
    assert ws(_lib.CIDER_OP_PERGROUP, 128, 2560, 10240, 256) == \
        quant(128, 10240) + 4 * 128 * 2560 * 4
    assert ws(_lib.CIDER_OP_W4A8_PERGROUP, 512, 4096, 12288, 64) == \
        quant(512, 12288) + 4 * 512 * 4096 * 4
    assert ws(_lib.CIDER_OP_PERGROUP, 128, 10240, 2560, 128) == quant(128, 2560)
    assert ws(_lib.CIDER_OP_W4A8_PERGROUP, 512, 12288, 4096, 128) == quant(512, 4096)
    assert ws(_lib.CIDER_OP_PERGROUP, 64, 2560, 10240, 64) == quant(64, 10240)


def _err(lib):
    return lib.cider_last_error().decode()


def test_validation_errors_without_gpu(lib):
    from cider_amd import _lib
    p = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    n = None
    # bad group size (csrc/src/pergroup_primitive.mm:291-295)
    rc = lib.cider_pergroup_linear(p, p, p, n, p, p, 1 << 20, 4, 8, 256, 100, n)
    assert rc == _lib.CIDER_E_INVALID and "group_size" in _err(lib)
    rc = lib.cider_pergroup_linear(p, p, p, n, p, p, 1 << 20, 4, 8, 320, 128, n)
    assert rc == _lib.CIDER_E_INVALID and "multiple" in _err(lib)
    rc = lib.cider_w4a8_pergroup_linear(p, p, p, n, p, p, 1 << 20, 4, 8, 256, 256, n)
    assert rc == _lib.CIDER_E_INVALID
    # negative dims
    rc = lib.cider_int8_matmul_int32(p, p, p, -1, 4, 4, n)
    assert rc == _lib.CIDER_E_INVALID and "negative" in _err(lib)
    # NULL operands
    rc = lib.cider_perchannel_linear(n, p, p, n, p, p, 1 << 20, 4, 8, 16, n)
    assert rc == _lib.CIDER_E_INVALID and "x is NULL" in _err(lib)
    # workspace missing / too small / misaligned
    rc = lib.cider_perchannel_linear(p, p, p, n, p, n, 0, 4, 8, 16, n)
    assert rc == _lib.CIDER_E_INVALID and "workspace" in _err(lib)
    rc = lib.cider_perchannel_linear(p, p, p, n, p, p, 16, 4, 8, 16, n)
    assert rc == _lib.CIDER_E_INVALID and "workspace" in _err(lib)
    rc = lib.cider_perchannel_linear(p, p, p, n, p, ctypes.c_void_p(0x1010), 1 << 20, 4, 8, 16, n)
    assert rc == _lib.CIDER_E_INVALID and "aligned" in _err(lib)
    # odd K for int4
    rc = lib.cider_w4a8_linear(p, p, p, p, p, 1 << 20, 4, 8, 15, n)
    assert rc == _lib.CIDER_E_INVALID and "even" in _err(lib)
    rc = lib.cider_w4_repack_ref(p, p, 8, 15, n)
    assert rc == _lib.CIDER_E_INVALID
    # the one-call reference-layout W4A8: odd K, and a workspace without room
    # for the repacked weights
    rc = lib.cider_w4a8_linear_ref(p, p, p, p, p, 1 << 20, 4, 8, 15, n)
    assert rc == _lib.CIDER_E_INVALID and "even" in _err(lib)
    need = _lib.workspace_bytes(_lib.CIDER_OP_W4A8_REF, 4, 4096, 4096)
    rc = lib.cider_w4a8_linear_ref(p, p, p, p, p, need - 1, 4, 4096, 4096, n)
    assert rc == _lib.CIDER_E_INVALID and "workspace" in _err(lib)
    # the entry point without a workspace rejects problems beyond its scratch
    rc = lib.cider_perchannel_linear_noalloc(p, p, p, n, p, 8192, 16, 8192, n)
    assert rc == _lib.CIDER_E_INVALID and "scratch" in _err(lib)
    assert _lib.workspace_bytes(_lib.CIDER_OP_PERCHANNEL, 4096, 16, 8000) <= \
        _lib.CIDER_NOALLOC_SCRATCH_BYTES
    # empty problems are no-ops that succeed
    assert lib.cider_perchannel_linear_noalloc(n, n, n, n, n, 0, 8, 16, n) == _lib.CIDER_OK
    assert lib.cider_perchannel_linear(n, n, n, n, n, n, 0, 0, 8, 16, n) == _lib.CIDER_OK
    assert lib.cider_int8_matmul_int32(n, n, n, 5, 0, 16, n) == _lib.CIDER_OK
    assert _err(lib) == ""


def test_producer_and_attention_validation_without_gpu(lib):
    from cider_amd import _lib
    p = ctypes.c_void_p(0x1000)
    n = None
    E = _lib.CIDER_E_INVALID
    # K must be a multiple of 8; something must be requested; add needs sum
    assert lib.cider_rmsnorm_quantize(p, n, n, p, 1e-6, p, n, n, 4, 12, n) == E
    assert "multiple of 8" in _err(lib)
    assert lib.cider_rmsnorm_quantize(p, n, n, p, 1e-6, n, n, n, 4, 16, n) == E
    assert "neither" in _err(lib)
    assert lib.cider_rmsnorm_quantize(p, p, n, p, 1e-6, p, n, n, 4, 16, n) == E
    assert "sum" in _err(lib)
    assert lib.cider_rmsnorm_quantize(p, n, n, p, -1.0, p, n, n, 4, 16, n) == E
    assert lib.cider_rmsnorm_quantize(p, n, n, p, 1e-6, n, p, n, 4, 16, n) == E
    assert "sa is NULL" in _err(lib)
    assert lib.cider_rmsnorm_quantize(p, n, n, p, 1e-6, ctypes.c_void_p(0x1008), n, n,
                                      4, 16, n) == E
    assert "aligned" in _err(lib)
    assert lib.cider_rmsnorm_quantize(p, n, n, p, 1e-6, p, n, n, 4, 16, n) == E
    assert "alias" in _err(lib)
    assert lib.cider_silu_mul_quantize(p, p, n, n, 4, 20, n) == E
    assert lib.cider_silu_mul_quantize(p, n, n, n, 4, 16, n) == E
    # head_dim 128 only; sizes; NULL tables
    args = [p, p, p, 1e-6, p, p, 64, p, p, p, p, p, 3, 8, 2, 128, 64, n]
    bad = list(args)
    bad[15] = 64
    assert lib.cider_qk_norm_rope(*bad) == E and "head_dim" in _err(lib)
    bad = list(args)
    bad[4] = n
    assert lib.cider_qk_norm_rope(*bad) == E and "cos is NULL" in _err(lib)
    bad = list(args)
    bad[16] = 0
    assert lib.cider_qk_norm_rope(*bad) == E
    # attention: group ratio, capacity multiple of 8, workspace
    wsb = lib.cider_attn_decode_workspace_bytes(32, 4096)
    assert wsb == 32 * 32 * 130 * 4  # 32 chunks of 128 positions, 32 heads
    assert lib.cider_attn_decode(p, p, p, p, 0.1, p, wsb, p, 24, 8, 128, 4096, n) == E
    assert lib.cider_attn_decode(p, p, p, p, 0.1, p, wsb, p, 32, 8, 128, 4092, n) == E
    assert lib.cider_attn_decode(p, p, p, p, 0.1, p, 16, p, 32, 8, 128, 4096, n) == E
    assert "workspace" in _err(lib)
    assert lib.cider_attn_decode(p, p, p, p, 0.1, p, wsb, p, 32, 8, 64, 4096, n) == E
    # prefill attention: head_dim, grouping, 1 <= c <= n <= T, pointers, alignment
    assert lib.cider_attn_prefill(p, p, p, 0.1, n, 0, p, 16, 32, n, 32, 8, 64, 64, n) == E
    assert "head_dim" in _err(lib)
    assert lib.cider_attn_prefill(p, p, p, 0.1, n, 0, p, 16, 32, n, 30, 8, 128, 64, n) == E
    assert lib.cider_attn_prefill(p, p, p, 0.1, n, 0, p, 33, 32, n, 32, 8, 128, 64, n) == E
    assert lib.cider_attn_prefill(p, p, p, 0.1, n, 0, p, 0, 32, n, 32, 8, 128, 64, n) == E
    assert lib.cider_attn_prefill(p, p, p, 0.1, n, 0, p, 16, 65, n, 32, 8, 128, 64, n) == E
    assert lib.cider_attn_prefill(n, p, p, 0.1, n, 0, p, 16, 32, n, 32, 8, 128, 64, n) == E
    assert "q is NULL" in _err(lib)
    assert lib.cider_attn_prefill(p, p, p, 0.1, n, 0, ctypes.c_void_p(0x1008), 16,
                                  32, n, 32, 8, 128, 64, n) == E
    assert "aligned" in _err(lib)
    assert lib.cider_attn_prefill(p, p, p, 0.1, ctypes.c_void_p(0x1010), 4096, p, 16,
                                  32, n, 32, 8, 128, 64, n) == E
    assert "256-byte" in _err(lib)
    # the workspace is what a split launch needs: none for a launch that fills the GPU
    assert lib.cider_attn_prefill_workspace_bytes(2048, 2048, 32) == 0
    assert lib.cider_attn_prefill_workspace_bytes(0, 2048, 32) == 0
    # a 512-query chunk over 2048 slots with 16 heads (64 query blocks): 4 parts of fp32 partials
    assert lib.cider_attn_prefill_workspace_bytes(512, 2048, 16) == 4 * 512 * 16 * 130 * 4
    # prefill attention quantized for o_proj: as above, plus H <= 128, the
    # output pointers, and a workspace of at least c * H * 256 bytes (each call
    # below breaks one argument, so none launches)
    good = [p, p, p, 0.1, p, 1 << 30, p, p, 16, 32, n, 32, 8, 128, 64, n]

    def apq(i, v):
        a = list(good)
        a[i] = v
        return lib.cider_attn_prefill_quantize(*a)

    assert apq(13, 64) == E and "head_dim" in _err(lib)
    assert apq(11, 256) == E and "H <= 128" in _err(lib)
    assert apq(11, 30) == E
    assert apq(8, 33) == E and apq(8, 0) == E and apq(9, 65) == E
    assert apq(0, n) == E and "q is NULL" in _err(lib)
    assert apq(6, n) == E and "q_out is NULL" in _err(lib)
    assert apq(7, n) == E and "sa_out is NULL" in _err(lib)
    assert apq(4, n) == E and "ws is NULL" in _err(lib)
    assert apq(6, ctypes.c_void_p(0x1008)) == E and "aligned" in _err(lib)
    assert apq(4, ctypes.c_void_p(0x1010)) == E and "256-byte" in _err(lib)
    assert apq(5, 16 * 32 * 256 - 1) == E and "needs at least" in _err(lib)
    # its workspace: the fp16 output of an unsplit launch, the partials of a split one
    wq = lib.cider_attn_prefill_quantize_workspace_bytes
    assert wq(2048, 2048, 32) == 2048 * 32 * 256
    assert wq(512, 2048, 16) == 4 * 512 * 16 * 130 * 4
    assert wq(16, 16, 256) == 0 and wq(0, 16, 8) == 0
    # empty problems succeed
    assert lib.cider_rmsnorm_quantize(n, n, n, n, 1e-6, p, n, n, 0, 16, n) == _lib.CIDER_OK
    assert lib.cider_qk_norm_rope(*(args[:12] + [0] + args[13:])) == _lib.CIDER_OK



def test_producer_mv_validation_without_gpu(lib):
    """cider_rmsnorm_mv / cider_swiglu_mv reject bad shapes, pointers and
    overlaps before any launch (no GPU needed)."""
    from cider_amd import _lib
    E, U = _lib.CIDER_E_INVALID, _lib.CIDER_E_UNSUPPORTED
    n = None
    x, a, sm, nw, w, sw, y = (ctypes.c_void_p(v) for v in
                              (0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000, 0x70000))
    K, N = 4096, 6144
    # K % 256 != 0 or K > 16384 or misaligned x / w: unsupported (use the two calls)
    assert lib.cider_rmsnorm_mv(x, n, n, nw, 1e-6, w, sw, n, y, N, 4000, n) == U
    assert lib.cider_rmsnorm_mv(x, n, n, nw, 1e-6, w, sw, n, y, N, 16640, n) == U
    assert lib.cider_rmsnorm_mv(ctypes.c_void_p(0x10008), n, n, nw, 1e-6, w, sw, n, y, N, K,
                                n) == U
    assert "256" in _err(lib)
    # add without sum, sum without add
    assert lib.cider_rmsnorm_mv(x, a, n, nw, 1e-6, w, sw, n, y, N, K, n) == E
    assert lib.cider_rmsnorm_mv(x, n, sm, nw, 1e-6, w, sw, n, y, N, K, n) == E
    assert "together" in _err(lib)
    # sum overlapping x (another workgroup still reads x), y overlapping inputs
    assert lib.cider_rmsnorm_mv(x, a, ctypes.c_void_p(0x10000 + 4096), nw, 1e-6, w, sw, n, y,
                                N, K, n) == E
    assert "sum must not overlap" in _err(lib)
    assert lib.cider_rmsnorm_mv(x, a, sm, nw, 1e-6, w, sw, n, ctypes.c_void_p(0x30000 + 64),
                                N, K, n) == E
    assert "y must not overlap" in _err(lib)
    # NULLs, eps, sizes
    assert lib.cider_rmsnorm_mv(x, n, n, n, 1e-6, w, sw, n, y, N, K, n) == E
    assert "norm_w is NULL" in _err(lib)
    assert lib.cider_rmsnorm_mv(x, n, n, nw, -1.0, w, sw, n, y, N, K, n) == E
    assert lib.cider_rmsnorm_mv(x, n, n, nw, 1e-6, w, n, n, y, N, K, n) == E
    assert lib.cider_rmsnorm_mv(x, n, n, nw, 1e-6, w, sw, n, y, 0, K, n) == E
    # SwiGLU: gate_up is [2K]; y must not overlap it
    assert lib.cider_swiglu_mv(x, w, sw, n, y, N, 12290, n) == U
    assert lib.cider_swiglu_mv(x, w, sw, n, ctypes.c_void_p(0x10000 + 2 * 4096 + 2), N, K,
                               n) == E
    assert "overlap" in _err(lib)
    assert lib.cider_swiglu_mv(x, n, sw, n, y, N, K, n) == E


def test_check_maps_codes_to_exceptions(lib):
    from cider_amd import _lib
    lib.cider_int8_matmul_int32(None, None, None, -1, 1, 1, None)
    with pytest.raises(ValueError, match="negative"):
        _lib.check(_lib.CIDER_E_INVALID)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.CIDER_E_HIP)


def test_host_quantizers_match_oracle():
    import cider_amd as C
    rng = np.random.default_rng(0)
    w = rng.standard_normal((37, 256)).astype(np.float32)
    w[3] = 0
    q, s = C.quantize_weight_int8(w)
    qe, se = O.quantize_weight_int8(w)
    np.testing.assert_array_equal(q, qe)
    np.testing.assert_array_equal(s, se)
    assert s[3] == 1.0 and (q[3] == 0).all()
    qg, sg = C.quantize_weight_pergroup(w, 64)
    qge, sge = O.quantize_weight_pergroup(w, 64)
    np.testing.assert_array_equal(qg, qge)
    np.testing.assert_array_equal(sg, sge)
    wk = rng.standard_normal((64, 24)).astype(np.float32)
    p, s4 = C.pack_weight_int4(wk)
    pe, s4e = O.pack_weight_int4(wk)
    np.testing.assert_array_equal(p, pe)
    np.testing.assert_array_equal(s4, s4e)


def test_pergroup_int4_packer_roundtrip():
    import cider_amd as C
    rng = np.random.default_rng(1)
    w = rng.standard_normal((20, 256)).astype(np.float32)
    packed, sc = C.pack_weight_int4_pergroup(w, 64)
    assert packed.shape == (20, 128) and sc.shape == (4, 20) and sc.dtype == np.float16
    q = O.unpack_w4_lo_first(packed)
    assert q.min() >= -8 and q.max() <= 7
    # each group's largest |w| maps to +-7 (half-to-even of exactly 7.0 or near it)
    deq = q.reshape(20, 4, 64) * sc.T.astype(np.float32)[:, :, None]
    err = np.abs(deq.reshape(20, 256) - w)
    assert (err <= np.repeat(sc.T.astype(np.float32), 64, axis=1) * 0.5 + 1e-3).all()


def test_cpu_tensors_rejected():
    torch = pytest.importorskip("torch")
    import cider_amd as C
    x = torch.zeros(2, 8, dtype=torch.float16)
    w = torch.zeros(4, 8, dtype=torch.int8)
    s = torch.ones(4)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        C.perchannel_linear(x, w, s)
    with pytest.raises(RuntimeError):
        C.int8_matmul_int32(w, w)
    if not torch.cuda.is_available():
        assert C.is_available() is False
        with pytest.raises(RuntimeError):
            C.convert_model(torch.nn.Linear(4, 4), verbose=False)


def test_reference_import_path():
    """``import cider`` and its submodules resolve to this implementation
    (the reference's surface, cider/__init__.py:18-57)."""
    import cider
    import cider.convert
    import cider_amd
    from cider.nn import CiderLinear, W4A8Linear, W8A8Linear
    from cider.ops import (int8_matmul_int32, pack_weight_int4, perchannel_linear,
                           pergroup_linear, quantize_weight_int8, w4a8_linear)
    assert cider.ops is cider_amd.ops and cider.nn is cider_amd.nn
    assert cider.convert is cider_amd.convert
    assert CiderLinear is cider_amd.CiderLinear and W8A8Linear is CiderLinear
    for name in ("convert_model", "set_mode", "get_mode", "CiderLinear", "W8A8Linear",
                 "W4A8Linear", "perchannel_linear", "w4a8_linear", "pergroup_linear",
                 "int8_matmul_int32", "quantize_weight_int8", "pack_weight_int4",
                 "is_available", "kernel_dir"):
        assert hasattr(cider, name), name
    assert callable(perchannel_linear) and callable(pergroup_linear)
    assert callable(int8_matmul_int32) and callable(w4a8_linear)
    assert callable(pack_weight_int4) and callable(quantize_weight_int8)
    assert W4A8Linear is cider_amd.W4A8Linear

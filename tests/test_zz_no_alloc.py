"""cider_perchannel_linear_noalloc (the entry point that allocates nothing)
against cider_perchannel_linear with a caller workspace, through the C ABI.

Two calls in a row on the same GPU share the library's scratch; the second
is smaller, so stale quantized rows of the first must not leak into it.
Bar: bit-exact (both run the same kernels on the same integers).
"""

import ctypes

import numpy as np
import pytest

from oracle import cider_oracle as O
from tests.util import assert_bits_equal

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


def _call_both(lib, _lib, x, w, sw, b):
    M, K = x.shape
    N = w.shape[0]
    xd, wd, sd = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in (x, w, sw))
    bd = None if b is None else torch.from_numpy(b).to(DEV)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    y_ws = torch.empty((M, N), dtype=torch.float16, device=DEV)
    nb = _lib.workspace_bytes(_lib.CIDER_OP_PERCHANNEL, M, N, K)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=DEV)
    _lib.check(lib.cider_perchannel_linear(
        xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), None if bd is None else bd.data_ptr(),
        y_ws.data_ptr(), ws.data_ptr() if nb else None, nb, M, N, K, s))
    y_na = torch.empty((M, N), dtype=torch.float16, device=DEV)
    _lib.check(lib.cider_perchannel_linear_noalloc(
        xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), None if bd is None else bd.data_ptr(),
        y_na.data_ptr(), M, N, K, s))
    torch.cuda.synchronize()
    return y_ws.cpu().numpy(), y_na.cpu().numpy()


def test_noalloc_matches_workspace_entry_twice_then_smaller():
    from cider_amd import _lib
    lib = _lib.load()
    # (128, 2560, 10240): the workspace entry runs the split-K GEMM (eight K
    # slices), the scratch entry one pass over K: the same bits either way
    cases = [(4096, 2560, 2560, True), (300, 1000, 1024, False), (1, 512, 1024, True),
             (3, 256, 512, True), (128, 2560, 10240, True)]
    for M, N, K, bias in cases:
        print(f"noalloc M={M} N={N} K={K}", flush=True)
        x = O.synth_activations(M, K, 7000 + M)
        w = O.synth_weights_i8(N, K, 7001 + N)
        sw = O.synth_scales(N, 7002)
        b = (np.random.default_rng(7003).standard_normal(N) * 0.1).astype(np.float16) \
            if bias else None
        y_ws, y_na = _call_both(lib, _lib, x, w, sw, b)
        assert_bits_equal(y_na, y_ws, f"noalloc vs workspace {M}x{N}x{K}")
        if M > 1:
            rows = np.r_[0:min(M, 8), max(0, M - 8):M]
            assert_bits_equal(y_na[rows], O.perchannel_linear(x[rows], w, sw, b),
                              f"noalloc vs oracle {M}x{N}x{K}")


def test_noalloc_rejects_problems_beyond_its_scratch():
    from cider_amd import _lib
    lib = _lib.load()
    M, K = 8192, 8192          # M*K = 64 MiB > 32 MiB
    rc = lib.cider_perchannel_linear_noalloc(ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000),
                                             ctypes.c_void_p(0x1000), None,
                                             ctypes.c_void_p(0x1000), M, 16, K, None)
    assert rc == _lib.CIDER_E_INVALID
    assert "scratch" in lib.cider_last_error().decode()

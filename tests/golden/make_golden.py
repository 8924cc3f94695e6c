"""Writes the committed golden fixtures under tests/golden/.

1. ``bitexact_shapes.json``: the 14 shapes of the reference's only
   results-pinning test (``benchmarks/test_bitexact.py:19-35``).  Inputs are
   numpy's legacy RNG, exactly as that test draws them
   (``np.random.seed(42)``; ``randint(-128, 128, (M, K))`` then
   ``randint(-128, 128, (N, K))``, ``test_bitexact.py:45-47``); the expected
   output is the test's own int64 product cast to int32 (``:55``).  The
   fixture stores SHA-256 digests of the inputs and of the expected int32
   output, plus the full output for the small shapes, so a test can rebuild
   the inputs and compare without storing 100+ MB.
2. ``cases.npz``: small seeded cases of every function on the path, with
   outputs from the numpy oracle (regression pins for the GPU tests).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import cider_oracle as O  # noqa: E402

SHAPES = [  # (M, K, N), benchmarks/test_bitexact.py:19-35
    (1, 2, 2), (2, 4, 2), (1, 128, 128), (1, 4096, 4096), (4, 2048, 2048),
    (16, 4096, 4096), (32, 4096, 4096), (64, 4096, 4096), (128, 4096, 4096),
    (16, 4096, 8192), (16, 8192, 4096), (64, 2048, 4096), (7, 513, 1025),
    (33, 4097, 4095),
]


def bitexact_inputs(M, K, N):
    np.random.seed(42)
    a = np.random.randint(-128, 128, (M, K), dtype=np.int8)
    b = np.random.randint(-128, 128, (N, K), dtype=np.int8)
    return a, b


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def make_bitexact():
    out = []
    for M, K, N in SHAPES:
        a, b = bitexact_inputs(M, K, N)
        c = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.int32)
        rec = {"M": M, "K": K, "N": N, "sha_a": sha(a), "sha_b": sha(b),
               "sha_c": sha(c), "c_sum_int64": int(c.astype(np.int64).sum())}
        if M * N <= 4096:
            rec["c"] = c.tolist()
        out.append(rec)
    with open(os.path.join(HERE, "bitexact_shapes.json"), "w") as f:
        json.dump({"source": "benchmarks/test_bitexact.py:19-55", "shapes": out}, f, indent=1)


def make_cases():
    d = {}
    # per-channel GEMM path (M >= 2), odd sizes included
    for i, (M, N, K) in enumerate([(2, 16, 64), (7, 33, 130), (33, 257, 513), (64, 128, 256)]):
        x = O.synth_activations(M, K, 100 + i)
        w = O.synth_weights_i8(N, K, 200 + i)
        sw = O.synth_scales(N, 300 + i)
        bias = (np.random.default_rng(400 + i).standard_normal(N) * 0.1).astype(np.float16)
        q, sa = O.quantize_per_token(x)
        d[f"pc{i}_x"], d[f"pc{i}_w"], d[f"pc{i}_sw"], d[f"pc{i}_bias"] = x, w, sw, bias
        d[f"pc{i}_q"], d[f"pc{i}_sa"] = q, sa
        d[f"pc{i}_y"] = O.perchannel_linear(x, w, sw, bias)
    # M == 1 MV path
    for i, (N, K) in enumerate([(40, 256), (130, 1024)]):
        x = O.synth_activations(1, K, 500 + i)
        w = O.synth_weights_i8(N, K, 600 + i)
        sw = O.synth_scales(N, 700 + i)
        bias = np.zeros(N, np.float16)
        d[f"mv{i}_x"], d[f"mv{i}_w"], d[f"mv{i}_sw"], d[f"mv{i}_bias"] = x, w, sw, bias
        d[f"mv{i}_y"] = O.perchannel_linear(x, w, sw, bias)
    # per-group GEMM and MV
    for i, (M, N, K, gs) in enumerate([(5, 48, 256, 64), (16, 130, 512, 128), (1, 72, 512, 64),
                                       (3, 64, 512, 256)]):
        x = O.synth_activations(M, K, 800 + i)
        w = O.synth_weights_i8(N, K, 900 + i)
        sw = O.synth_scales((K // gs, N), 1000 + i)
        bias = (np.random.default_rng(1100 + i).standard_normal(N) * 0.1).astype(np.float16)
        d[f"pg{i}_x"], d[f"pg{i}_w"], d[f"pg{i}_sw"], d[f"pg{i}_bias"] = x, w, sw, bias
        d[f"pg{i}_gs"] = np.array(gs)
        d[f"pg{i}_y"] = O.pergroup_linear(x, w, sw, gs, bias)
    # W4A8, reference layout
    for i, (M, N, K) in enumerate([(1, 32, 64), (9, 70, 160)]):
        x = O.synth_activations(M, K, 1200 + i)
        wf = np.random.default_rng(1300 + i).standard_normal((K, N)).astype(np.float32)
        packed, sw = O.pack_weight_int4(wf)
        d[f"w4r{i}_x"], d[f"w4r{i}_packed"], d[f"w4r{i}_sw"] = x, packed, sw
        d[f"w4r{i}_y"] = O.w4a8_linear(x, packed, sw)
    # W4A8 per-group extension
    for i, (M, N, K, gs) in enumerate([(4, 48, 256, 64), (17, 40, 512, 128)]):
        x = O.synth_activations(M, K, 1400 + i)
        w4 = np.random.default_rng(1500 + i).integers(-8, 8, size=(N, K), dtype=np.int8)
        packed = O.pack_w4_lo_first(w4)
        sc = O.synth_scales((K // gs, N), 1600 + i).astype(np.float16)
        d[f"w4g{i}_x"], d[f"w4g{i}_packed"], d[f"w4g{i}_scale"] = x, packed, sc
        d[f"w4g{i}_gs"] = np.array(gs)
        d[f"w4g{i}_y"] = O.w4a8_pergroup_linear(x, packed, sc, gs)
    np.savez_compressed(os.path.join(HERE, "cases.npz"), **d)


if __name__ == "__main__":
    make_bitexact()
    make_cases()
    print("golden fixtures written to", HERE)

"""Benchmark of the fused W8A8 linear on one MI355X.

Workload (the configuration the metric is quoted
on): per-channel W8A8 linear, M=4096, N=10240, K=2560.  One step is one pass
of the hot path over that batch, i.e. exactly the two kernels
cider_perchannel_linear launches (per-token quantize, then int8 GEMM with the
fused per-channel epilogue), enqueued through the C ABI as
cider_quantize_per_token + cider_perchannel_gemm.  The K timed steps are
enqueued as K quantize launches followed by K GEMM launches, with a HIP event
at each boundary, so the GEMM kernel's average duration (the roofline figure)
comes from back-to-back launches.  Inputs are resident in HBM before timing
starts.

Also reported, in the same run:
  * decode: the M == 1 MV (N=10240, K=2560), cycling over enough weight copies
    (>= 2x the 256 MB Infinity Cache) that every launch streams from HBM, in a
    HIP graph and as eager back-to-back launches, beside the read probe of
    cider_amd/csrc/probe.hip (one launch reading the same bytes in the MV's
    layout: the read ceiling of the M == 1 roofline);
  * mfma_ceiling: the sustained int8 MFMA rate and shader clock of a probe
    kernel with register-resident operands (random and zero bytes), the
    ceiling of the GEMM roofline on this part;
  * sweep: the other configs[1] / configs[2] cases (per-group, W4A8, M = 1,
    16, 128, 1024, 8192 and the N=2560 K=10240 shape), each a HIP graph of
    back-to-back calls; up to M = 512 the weights rotate past the MALL;
  * qwen3: configs[3], the Qwen3-8B-shaped stack, 2048-token prefill and
    128 graph-replayed greedy decode steps;
  * cpu_baseline: the C restatement of the reference math (oracle/) on rows
    0..127 of the same inputs (= configs[0], M=128), all host threads, and a
    bit-exact comparison of those rows with the GPU output.

Prints ONE JSON line.
"""

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
# the cpu_baseline leg's OpenMP threads are bound to cores (read when the
# oracle's OpenMP runtime starts): unbound, the C timing of the same sample
# ranged 12-32 ms over runs on 16 host threads
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POPS
HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
MALL_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=250.0,
                    help="before the warmup steps, repeat the step until this much GPU time "
                         "has passed, so the timed steps run at settled clocks (0 = off)")
    ap.add_argument("--M", type=int, default=4096)
    ap.add_argument("--N", type=int, default=10240)
    ap.add_argument("--K", type=int, default=2560)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the M=1 decode leg")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the compact sweep (per-group, W4A8, M=1 / 16 / 8192 cases)")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the sustained-MFMA probe (cider_amd/csrc/probe.hip)")
    ap.add_argument("--only-decode", action="store_true",
                    help="print only the decode leg (M=1 MV of N x K) as one JSON line, e.g. "
                         "to pair it with a kernel trace of the same launches")
    ap.add_argument("--no-qwen3", action="store_true",
                    help="skip the compact configs[3] leg (Qwen3-8B prefill / decode)")
    ap.add_argument("--qwen3", action="store_true",
                    help="instead of the default line, print one JSON line for configs[3]: "
                         "Qwen3-8B-shaped W8A8 stack, 2048-token prefill + 128 greedy "
                         "decode steps (decode step captured as a HIP graph)")
    ap.add_argument("--qwen3vl", action="store_true",
                    help="instead of the default line, print one JSON line for configs[4]: "
                         "Qwen3-VL-2B-shaped W8A8 text decoder, chunked prefill (512) of "
                         "1334 / 2393 / 3455-token multimodal prompts, then graph decode")
    ap.add_argument("--attn", action="store_true",
                    help="instead of the default line, print one JSON line for the prefill "
                         "attention kernel (cider_attn_prefill) at the configs[3] shape "
                         "(2048 queries, 32 / 8 heads) and a configs[4] chunk (512 queries "
                         "after 1536 cached, 16 / 8 heads), with PyTorch's SDPA beside it")
    ap.add_argument("--torch-producers", action="store_true",
                    help="with --qwen3: run RMSNorm, SwiGLU, q/k norm + RoPE and decode "
                         "attention as PyTorch ops instead of the fused HIP kernels (A/B)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="first run three 256 MiB device-to-device copies, the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--sweep", action="store_true",
                    help="instead of the default line, print one JSON line per configs[1] / "
                         "configs[2] case (M sweep x shapes x scale modes)")
    return ap.parse_args()


def synth_inputs(torch, M, N, K, seed, dev):
    """X fp16 ~ N(0,1) with K//100 outlier columns x20; W int8 U[-127,127];
    scale_w fp32 U[1e-3,1e-2]; bias zeros (the reference default)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g, dtype=torch.float32)
    cols = torch.randperm(K, generator=g)[: K // 100]
    x[:, cols] *= 20.0
    x = x.to(torch.float16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g, dtype=torch.float32) * 9e-3 + 1e-3
    bias = torch.zeros(N, dtype=torch.float16)
    return [t.to(dev) for t in (x, w, sw, bias)]


def vp(t):
    return ctypes.c_void_p(t.data_ptr())


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by output columns with no collective; see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from cider_amd import _lib

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    lib = _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.sweep:
        sweep(torch, args, dev)
        return
    if args.qwen3:
        bench_qwen3(torch, args, dev)
        return
    if args.qwen3vl:
        bench_qwen3vl(torch, args, dev)
        return
    if args.attn:
        bench_attn(torch, args, dev)
        return
    if args.only_decode:
        stream = torch.cuda.current_stream(dev)
        print(json.dumps({"decode": bench_decode(torch, lib, _lib, args.N, args.K, args, dev,
                                                 stream)}), flush=True)
        return
    M, N, K = args.M, args.N, args.K
    x, w, sw, bias = synth_inputs(torch, M, N, K, args.seed, dev)
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    sa = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)

    def quant():
        _lib.check(lib.cider_quantize_per_token(vp(x), vp(q), vp(sa), M, K, sp))

    def gemm():
        _lib.check(lib.cider_perchannel_gemm(vp(q), vp(sa), vp(w), vp(sw), vp(bias), vp(y),
                                             M, N, K, sp))

    if args.copy_calib:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # Settle: the first ~50 launches after the host-side setup run 10-15%
    # slower while the GPU clock ramps up; repeat the step (untimed) for
    # settle_ms of GPU time before the W warmup steps.
    settled_ms = 0.0
    if args.settle_ms > 0:
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        while settled_ms < args.settle_ms:
            for _ in range(20):
                quant()
                gemm()
            s1.record(stream)
            s1.synchronize()
            settled_ms = s0.elapsed_time(s1)
    for _ in range(args.warmup):
        quant()
        gemm()
    torch.cuda.synchronize()
    # Timed region: K quantize launches, then K GEMM launches (every GEMM reads
    # the quantized activations the launches before it wrote), one HIP event at
    # each boundary on the launch stream, so each kernel's average comes from
    # back-to-back launches with no event in between.
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for _ in range(args.steps):
        quant()
    ev[1].record(stream)
    for _ in range(args.steps):
        gemm()
    ev[2].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / args.steps
    quant_avg = ev[0].elapsed_time(ev[1]) / args.steps
    gemm_avg = ev[1].elapsed_time(ev[2]) / args.steps
    step_ms = ev[0].elapsed_time(ev[2]) / args.steps
    ops = 2.0 * M * N * K
    value_tops = ops / (step_ms * 1e-3) / 1e12
    gemm_tops = ops / (gemm_avg * 1e-3) / 1e12

    result = {
        "metric": "W8A8 GEMM TOPS (% INT8 peak) at M=4096; GB/s (% HBM peak) at M=1",
        "value": round(value_tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": round(settled_ms, 1),
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "configs[1]: W8A8 per-channel linear (quantize + int8 GEMM + "
                               "fused dequant), X fp16 N(0,1) with 1% outlier columns x20",
                   "M": M, "N": N, "K": K, "seed": args.seed, "parallelism": "none (1 GPU)"},
        "kernels": {"quantize_ms": round(quant_avg, 4), "gemm_ms": round(gemm_avg, 4),
                    "host_wall_ms_per_step": round(wall_ms, 4),
                    "gemm_tops": round(gemm_tops, 2),
                    "frac_of_int8_peak_whole_step": round(value_tops / INT8_PEAK_TOPS, 4)},
        "roofline": {"bound": "mfma", "kernel": gemm_kernel_name(M, N, K, dev),
                     "achieved": round(gemm_tops, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TOPS", "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
                     "traffic": load_traffic()},
    }

    if not args.no_decode:
        result["decode"] = bench_decode(torch, lib, _lib, N, K, args, dev, stream)
    if not args.no_sweep:
        result["sweep"] = compact_sweep(torch, lib, _lib, args, dev, stream)

    if not args.no_ceiling:
        result["mfma_ceiling"] = mfma_ceiling(torch, args, dev, stream)

    if not args.no_qwen3:
        result["qwen3"] = qwen3_summary(torch, args, dev)

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(x, w, sw, bias, y, N, K)
    print(json.dumps(result), flush=True)


def bench_decode(torch, lib, _lib, N, K, args, dev, stream):
    """M == 1 fp16-activation MV, weights rotated across >= 2x MALL."""
    wbytes = N * K
    copies = max(2, -(-2 * MALL_BYTES // wbytes) + 1)
    g = torch.Generator(device="cpu").manual_seed(args.seed + 1)
    ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
          for _ in range(copies)]
    sw = (torch.rand(N, generator=g) * 9e-3 + 1e-3).to(dev)
    bias = torch.zeros(N, dtype=torch.float16, device=dev)
    x = torch.randn(1, K, generator=g).to(torch.float16).to(dev)
    y = torch.empty((1, N), dtype=torch.float16, device=dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    iters = max(args.steps, copies * 4)

    def call(i):
        _lib.check(lib.cider_perchannel_linear(vp(x), vp(ws[i % copies]), vp(sw), vp(bias), vp(y),
                                               None, 0, 1, N, K, sp))

    for i in range(max(args.warmup, copies)):
        call(i)
    torch.cuda.synchronize()

    def graph_us(fn, n):
        """Per-call time of n back-to-back calls captured in one HIP graph (no
        host launch cost), median of 5 replays after a 50 ms settle."""
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(n):
                fn(i)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        while True:
            gr.replay()
            s1.record(stream)
            s1.synchronize()
            if s0.elapsed_time(s1) >= 50.0:
                break
        ts = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            gr.replay()
            e1.record(stream)
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) / n * 1e3)
        return sorted(ts)[2]

    def cur():  # graph capture runs on a stream of its own
        return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def gcall(i):
        _lib.check(lib.cider_perchannel_linear(vp(x), vp(ws[i % copies]), vp(sw), vp(bias), vp(y),
                                               None, 0, 1, N, K, cur()))

    us = graph_us(gcall, iters)
    # The same calls launched one by one on the stream (no graph): the
    # per-call time that a kernel trace of back-to-back launches pairs with.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(iters):
        call(i)
    e0.record(stream)
    for i in range(iters):
        call(i)
    e1.record(stream)
    e1.synchronize()
    us_eager = e0.elapsed_time(e1) / iters * 1e3
    # The read probe (cider_amd/csrc/probe.hip) over the same weight copies in
    # the same graph form: one launch reading N*K bytes in the MV's layout,
    # with no x staging, arithmetic or output beyond 4 bytes per wave.
    plib = load_probe()
    rsink = torch.empty(N * K // 5120, dtype=torch.int32, device=dev)

    def rcall(i):
        rc = plib.cider_probe_read(vp(ws[i % copies]), N * K, vp(rsink), cur())
        if rc != 0:
            raise RuntimeError(f"cider_probe_read failed ({rc})")

    read_us = graph_us(rcall, iters) if (N * K) % 20480 == 0 else None
    # The same call with 8 weight rows: the per-launch cost of the MV in the
    # graph (dispatch, x staging, drain) with almost no weight traffic.
    w8 = ws[0][:8].contiguous()

    def gfloor(i):
        _lib.check(lib.cider_perchannel_linear(vp(x), vp(w8), vp(sw), vp(bias), vp(y),
                                               None, 0, 1, 8, K, cur()))

    floor_us = graph_us(gfloor, iters)
    nbytes = N * K + 2 * K + 4 * N + 2 * N + 2 * N  # W, x, scale_w, bias, y
    gbs = nbytes / (us * 1e-6) / 1e9
    above = nbytes / ((us - floor_us) * 1e-6) / 1e9 if us > floor_us else None
    return {"workload": "M=1 per-channel MV (configs[1] decode)", "N": N, "K": K,
            "weight_copies": copies, "calls": iters, "timing": "HIP graph of %d calls" % iters,
            "us_per_call": round(us, 3), "algorithmic_bytes": nbytes,
            "achieved_gbs": round(gbs, 1), "peak_gbs": HBM_PEAK_GBS,
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bound": "hbm",
            "kernel": "mv_stream_kernel<2, 5, per-channel> (cider_amd/csrc/mv_stream.hip)",
            "us_per_call_eager": round(us_eager, 3),
            "launch_floor_us": round(floor_us, 3),
            "streaming_gbs_above_floor": None if above is None else round(above, 1),
            "read_ceiling": None if read_us is None else {
                "probe": "probe_read_kernel (cider_amd/csrc/probe.hip): one launch reading "
                         "the N*K weight bytes in the MV's layout, same copies and graph",
                "us_per_call": round(read_us, 3),
                "gbs": round(N * K / (read_us * 1e-6) / 1e9, 1),
                "frac_of_hbm_peak": round(N * K / (read_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "mv_frac_of_read": round(read_us / us, 4)}}


_probe = None


def load_probe():
    """ctypes binding of cider_amd/lib/libcider_probe.so (the measurement
    probes of cider_amd/csrc/probe.hip, not part of the linear's C ABI)."""
    global _probe
    if _probe is None:
        path = os.path.join(ROOT, "cider_amd", "lib", "libcider_probe.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build with make -C cider_amd/csrc")
        lib = ctypes.CDLL(path)
        P, I, LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
        lib.cider_probe_mfma.argtypes = [P, I, I, P, P, I, P]
        lib.cider_probe_mfma.restype = I
        lib.cider_probe_mfma_round_ops.argtypes = [I]
        lib.cider_probe_mfma_round_ops.restype = LL
        lib.cider_probe_mfma_src_bytes.argtypes = []
        lib.cider_probe_mfma_src_bytes.restype = LL
        lib.cider_probe_read.argtypes = [P, LL, P, P]
        lib.cider_probe_read.restype = I
        _probe = lib
    return _probe


def mfma_ceiling(torch, args, dev, stream):
    """The int8 MFMA rate the chip sustains with no memory traffic (probe
    kernel probe_mfma_kernel, cider_amd/csrc/probe.hip): one 8-wave workgroup
    per CU, the MFMAs of a 128 x 64 wave tile per round from register-
    resident operands, about 0.3-0.5 ms per launch; settled for 300 ms, then
    the median of 10 timed launches.  The GEMM's instruction
    (v_mfma_i32_32x32x32_i8) and v_mfma_i32_16x16x64_i8, on random operand
    bytes (the weights' statistics) and on all-zero operands; the shader clock
    is s_memtime over s_memrealtime (100 MHz) of every wave, median."""
    plib = load_probe()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    nsrc = cus * int(plib.cider_probe_mfma_src_bytes())
    g = torch.Generator(device="cpu").manual_seed(args.seed + 11)
    rnd = torch.randint(-128, 128, (nsrc,), generator=g, dtype=torch.int8).to(dev)
    zeros = torch.zeros_like(rnd)
    clocks = torch.zeros(cus * 8 * 4, dtype=torch.int64, device=dev)
    sink = torch.empty(cus * 512, dtype=torch.int32, device=dev)
    iters = 400
    sp = ctypes.c_void_p(stream.cuda_stream)
    out = {"probe": "probe_mfma_kernel (cider_amd/csrc/probe.hip): %d workgroups x 8 waves, "
                    "%d rounds per wave" % (cus, iters)}
    for form, fname in ((0, "mfma_i32_32x32x32_i8"), (1, "mfma_i32_16x16x64_i8")):
        ops = float(plib.cider_probe_mfma_round_ops(form)) * iters * cus * 8
        rec = {}
        for name, src in (("random_int8", rnd), ("zeros", zeros)):
            def launch():
                rc = plib.cider_probe_mfma(vp(src), form, iters, vp(clocks), vp(sink), cus, sp)
                if rc != 0:
                    raise RuntimeError(f"cider_probe_mfma failed ({rc})")
            s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s0.record(stream)
            while True:
                for _ in range(20):
                    launch()
                s1.record(stream)
                s1.synchronize()
                if s0.elapsed_time(s1) >= 300.0:
                    break
            ts = []
            for _ in range(10):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                launch()
                e1.record(stream)
                e1.synchronize()
                ts.append(e0.elapsed_time(e1))
            ms = statistics.median(ts)
            c = clocks.view(-1, 4).cpu().double()
            ghz = ((c[:, 1] - c[:, 0]) / (c[:, 3] - c[:, 2]) * 0.1).median().item()
            tops = ops / (ms * 1e-3) / 1e12
            rec[name] = {"ms_per_launch": round(ms, 4), "tops": round(tops, 1),
                         "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                         "shader_clock_ghz": round(ghz, 3),
                         "frac_of_peak_at_that_clock": round(tops / INT8_PEAK_TOPS * 2.4 / ghz, 4)}
        out[fname] = rec
    return out


def time_case(torch, stream, settle_ms, name, call_for, ncopies, M, N, K, nbytes_alg, ops,
              mode):
    """GPU time per call of call_for(i) (i cycling over ncopies weight copies):
    a run of calls captured in one HIP graph, replayed (untimed) for settle_ms
    of GPU time, then timed over 5 replays; the median per call."""
    reps = max(24, 2 * ncopies)
    for i in range(max(4, ncopies)):
        call_for(i % ncopies)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(reps):
            call_for(i % ncopies)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    while True:
        g.replay()
        s1.record(stream)
        s1.synchronize()
        if s0.elapsed_time(s1) >= settle_ms:
            break
    times = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / reps)
    ms = statistics.median(times)
    del g
    return {"case": name, "mode": mode, "M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
            "tops": round(ops / (ms * 1e-3) / 1e12, 1),
            "frac_int8_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
            "gbs": round(nbytes_alg / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes_alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "weight_copies": ncopies, "timing": "HIP graph of %d calls" % reps}


def compact_sweep(torch, lib, _lib, args, dev, stream):
    """The cases of the configs[1] / configs[2] sweep that the headline line
    does not cover, timed as in sweep(): per-group gs 128 / 64 at M=4096, the
    M=1 MV on the down-projection shape, W4A8 per-group gs 128 at M=4096 and
    M=16 (the decode-batch path), per-channel at M=16, 128, 1024, 4096 and
    8192 on both configs[1] shapes, per-group at M=128, the M=16 per-group
    cases of the LDS weight stream (int8 gs 128, W4A8 gs 64), and W4A8 gs 128
    at M=1 (the streaming GEMV with the quantization fused).  Up to M = 512
    the weights rotate over copies past the MALL, so they stream from HBM."""
    vp = ctypes.c_void_p

    def cur():
        return vp(torch.cuda.current_stream(dev).cuda_stream)

    g = torch.Generator(device="cpu").manual_seed(args.seed + 7)

    def synth_x(M, K):
        x = torch.randn(M, K, generator=g)
        x[:, torch.randperm(K, generator=g)[: K // 100]] *= 20.0
        return x.to(torch.float16).to(dev)

    def copies(M, wbytes):
        # up to M = 512 the linear is near the memory ridge: weights stream
        # from HBM as in a model (>= 2x the MALL of copies, rotated)
        return max(1, -(-2 * MALL_BYTES // wbytes) + 1) if M <= 512 else 1

    recs = []

    def w8_case(M, N, K, gs):
        nc = copies(M, N * K)
        ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
              for _ in range(nc)]
        sw = ((torch.rand(N, generator=g) * 9e-3 + 1e-3) if gs == 0 else
              (torch.rand(K // gs, N, generator=g) * 9e-3 + 1e-3)).to(dev)
        bias = torch.zeros(N, dtype=torch.float16, device=dev)
        x = synth_x(M, K)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        op = _lib.CIDER_OP_PERCHANNEL if gs == 0 else _lib.CIDER_OP_PERGROUP
        nb = _lib.workspace_bytes(op, M, N, K, gs)
        wsp = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)

        def call_for(i):
            if gs == 0:
                _lib.check(lib.cider_perchannel_linear(
                    vp(x.data_ptr()), vp(ws[i].data_ptr()), vp(sw.data_ptr()),
                    vp(bias.data_ptr()), vp(y.data_ptr()), vp(wsp.data_ptr()), nb, M, N, K,
                    cur()))
            else:
                _lib.check(lib.cider_pergroup_linear(
                    vp(x.data_ptr()), vp(ws[i].data_ptr()), vp(sw.data_ptr()),
                    vp(bias.data_ptr()), vp(y.data_ptr()), vp(wsp.data_ptr()), nb, M, N, K, gs,
                    cur()))
        sbytes = 4 * N if gs == 0 else 4 * N * (K // gs)
        nbytes = N * K + 2 * M * K + sbytes + 2 * N + 2 * M * N
        mode = "per-channel" if gs == 0 else f"per-group-{gs}"
        recs.append(time_case(torch, stream, args.settle_ms, "configs[1]", call_for, nc, M, N,
                              K, nbytes, 2.0 * M * N * K, mode))

    def w4_case(M, N, K, gs):
        nc = copies(M, N * K // 2)
        pk = [torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8).to(dev)
              for _ in range(nc)]
        sc = (torch.rand(K // gs, N, generator=g) * 9e-3 + 1e-3).to(torch.float16).to(dev)
        x = synth_x(M, K)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        nb = _lib.workspace_bytes(_lib.CIDER_OP_W4A8_PERGROUP, M, N, K, gs)
        wsp = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)

        def call_for(i):
            _lib.check(lib.cider_w4a8_pergroup_linear(
                vp(x.data_ptr()), vp(pk[i].data_ptr()), vp(sc.data_ptr()), None,
                vp(y.data_ptr()), vp(wsp.data_ptr()), nb, M, N, K, gs, cur()))
        nbytes = N * K // 2 + 2 * M * K + 2 * N * (K // gs) + 2 * M * N
        recs.append(time_case(torch, stream, args.settle_ms, "configs[2]", call_for, nc, M, N,
                              K, nbytes, 2.0 * M * N * K, f"w4a8-per-group-{gs}"))

    w8_case(4096, 10240, 2560, 128)
    w8_case(4096, 10240, 2560, 64)
    w8_case(1, 2560, 10240, 0)
    w8_case(16, 10240, 2560, 0)
    w8_case(8192, 10240, 2560, 0)
    w8_case(4096, 2560, 10240, 0)
    for M in (128, 1024):
        w8_case(M, 10240, 2560, 0)
        w8_case(M, 2560, 10240, 0)
    w8_case(128, 10240, 2560, 128)
    w8_case(128, 2560, 10240, 64)
    w4_case(4096, 12288, 4096, 128)
    w4_case(16, 12288, 4096, 128)
    w8_case(16, 10240, 2560, 128)
    w4_case(16, 12288, 4096, 64)
    w4_case(1, 12288, 4096, 128)
    torch.cuda.synchronize()
    return recs


def sweep(torch, args, dev):
    """per-channel / per-group gs 128 and 64, M in {1,128,1024,4096,8192},
    (N,K) in {(10240,2560),(2560,10240)}, plus per-group gs 256 (a group size
    the reference's per-group op also takes); configs[2]: W4A8 per-group gs 64 / 128,
    (N,K) in {(12288,4096),(4096,12288)}, M in {1,16,512,4096}.

    Each case is the whole linear (per-token quantize + GEMM, or the MV at
    M == 1) called through the C ABI with preallocated output and workspace.
    A run of calls is captured in a HIP graph and replayed, so the time per
    call is GPU time, free of Python and launch overhead.  Weights rotate over
    >= 2x the MALL when a call is memory-bound (M <= 64) so every call streams
    them from HBM."""
    from cider_amd import _lib
    lib = _lib.load()
    vp = ctypes.c_void_p
    stream = torch.cuda.current_stream(dev)

    def cur():  # the current stream (graph capture runs on a stream of its own)
        return vp(torch.cuda.current_stream(dev).cuda_stream)

    def synth_x(M, K, seed):
        g = torch.Generator(device="cpu").manual_seed(seed)
        x = torch.randn(M, K, generator=g)
        x[:, torch.randperm(K, generator=g)[: K // 100]] *= 20.0
        return x.to(torch.float16).to(dev)

    def run(name, call_for, ncopies, M, N, K, nbytes_alg, ops, mode):
        print(json.dumps(time_case(torch, stream, args.settle_ms, name, call_for, ncopies, M,
                                   N, K, nbytes_alg, ops, mode)), flush=True)

    def copies_for(M, wbytes):
        return max(1, -(-2 * MALL_BYTES // wbytes) + 1) if M <= 512 else 1

    g = torch.Generator(device="cpu").manual_seed(args.seed)
    for (N, K) in [(10240, 2560), (2560, 10240)]:
        nw = -(-2 * MALL_BYTES // (N * K)) + 1
        ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
              for _ in range(nw)]
        bias = torch.zeros(N, dtype=torch.float16, device=dev)
        for mode, gs in [("per-channel", 0), ("per-group-128", 128), ("per-group-64", 64),
                         ("per-group-256", 256)]:
            sw = ((torch.rand(N, generator=g) * 9e-3 + 1e-3) if gs == 0 else
                  (torch.rand(K // gs, N, generator=g) * 9e-3 + 1e-3)).to(dev)
            sbytes = 4 * N if gs == 0 else 4 * N * (K // gs)
            for M in (1, 128, 1024, 4096, 8192):
                x = synth_x(M, K, args.seed + M)
                y = torch.empty((M, N), dtype=torch.float16, device=dev)
                op = _lib.CIDER_OP_PERCHANNEL if gs == 0 else _lib.CIDER_OP_PERGROUP
                nb = _lib.workspace_bytes(op, M, N, K, gs)
                wsp = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
                if gs == 0:
                    def call_for(i, x=x, y=y, wsp=wsp, nb=nb, sw=sw, M=M):
                        _lib.check(lib.cider_perchannel_linear(
                            vp(x.data_ptr()), vp(ws[i].data_ptr()), vp(sw.data_ptr()),
                            vp(bias.data_ptr()), vp(y.data_ptr()), vp(wsp.data_ptr()), nb,
                            M, N, K, cur()))
                else:
                    def call_for(i, x=x, y=y, wsp=wsp, nb=nb, sw=sw, M=M, gs=gs):
                        _lib.check(lib.cider_pergroup_linear(
                            vp(x.data_ptr()), vp(ws[i].data_ptr()), vp(sw.data_ptr()),
                            vp(bias.data_ptr()), vp(y.data_ptr()), vp(wsp.data_ptr()), nb,
                            M, N, K, gs, cur()))
                nbytes = N * K + 2 * M * K + sbytes + 2 * N + 2 * M * N
                run("configs[1]", call_for, copies_for(M, N * K), M, N, K, nbytes,
                    2.0 * M * N * K, mode)
        del ws
    for (N, K) in [(12288, 4096), (4096, 12288)]:
        nw = -(-2 * MALL_BYTES // (N * K // 2)) + 1
        pk = [torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8).to(dev)
              for _ in range(nw)]
        for gs in (128, 64):
            sc = (torch.rand(K // gs, N, generator=g) * 9e-3 + 1e-3).to(torch.float16).to(dev)
            for M in (1, 16, 512, 4096):
                x = synth_x(M, K, args.seed + M)
                y = torch.empty((M, N), dtype=torch.float16, device=dev)
                nb = _lib.workspace_bytes(_lib.CIDER_OP_W4A8_PERGROUP, M, N, K, gs)
                wsp = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)

                def call_for(i, x=x, y=y, wsp=wsp, nb=nb, sc=sc, M=M, gs=gs):
                    _lib.check(lib.cider_w4a8_pergroup_linear(
                        vp(x.data_ptr()), vp(pk[i].data_ptr()), vp(sc.data_ptr()), None,
                        vp(y.data_ptr()), vp(wsp.data_ptr()), nb, M, N, K, gs, cur()))
                nbytes = N * K // 2 + 2 * M * K + 2 * N * (K // gs) + 2 * M * N
                run("configs[2]", call_for, copies_for(M, N * K // 2), M, N, K, nbytes,
                    2.0 * M * N * K, f"w4a8-per-group-{gs}")
        del pk


def cpu_baseline(x, w, sw, bias, y, N, K):
    """The reference math on the host, on rows 0..127 of the workload
    (= configs[0], M=128): the oracle's C restatement (all host threads) is
    the reported value; BASELINE.md's two numpy restatements are timed beside
    it (per-token quantize, then (i) a literal int32 np.matmul -- numpy runs
    integer matmul single-threaded without BLAS -- or (ii) an exact float64
    BLAS GEMM, then the dequant in the reference order).  The GPU's rows are
    checked bit for bit against the C result."""
    import numpy as np

    from oracle import c_oracle
    from oracle import cider_oracle as O

    rows = 128
    xs = x[:rows].cpu().numpy()
    wn = w.cpu().numpy()
    swn = sw.cpu().numpy()
    bn = bias.cpu().numpy()
    threads = c_oracle.num_threads()

    def timed(fn, runs, budget_s):
        times, out = [], None
        deadline = time.perf_counter() + budget_s
        for _ in range(runs):
            t0 = time.perf_counter()
            out = fn()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > deadline:
                break
        return statistics.median(times), len(times), out

    c_oracle.perchannel_linear_gemm(xs[:4], wn, swn, bn)  # warm-up: threads, pages
    med, nruns, out = timed(lambda: c_oracle.perchannel_linear_gemm(xs, wn, swn, bn), 7, 30.0)
    gpu_rows = y[:rows].cpu().numpy()
    exact = bool(np.array_equal(gpu_rows.view(np.uint16), out.view(np.uint16)))

    # numpy restatements; the int32 matmul runs on 16 of the rows (its rate
    # does not depend on M), the float64 BLAS one on all 128
    w32, w64 = wn.astype(np.int32), wn.astype(np.float64)

    def np_int32(xr):
        q, sa = O.quantize_per_token(xr)
        acc = np.matmul(q.astype(np.int32), w32.T)
        return O.dequant_perchannel(acc, sa, swn, bn)

    def np_f64(xr):
        q, sa = O.quantize_per_token(xr)
        acc = (q.astype(np.float64) @ w64.T).astype(np.int64).astype(np.int32)
        return O.dequant_perchannel(acc, sa, swn, bn)

    r32 = 16
    m32, n32, o32 = timed(lambda: np_int32(xs[:r32]), 3, 20.0)
    np_f64(xs[:4])  # warm-up
    m64, n64, o64 = timed(lambda: np_f64(xs), 7, 10.0)
    np_exact = bool(np.array_equal(o64.view(np.uint16), out.view(np.uint16)) and
                    np.array_equal(o32.view(np.uint16), out[:r32].view(np.uint16)))
    # the reported value: the faster of the two full-size faithful variants
    # (both bit-exact against each other and the GPU rows)
    best_c = med <= m64 or not np_exact
    best = med if best_c else m64
    return {"value": round(2.0 * rows * N * K / best / 1e12, 4), "unit": "TOPS",
            "cores": threads, "kind": "port",
            "sample": f"rows 0..{rows - 1} of the M=4096 workload (configs[0] shape "
                      f"M={rows},N={N},K={K}); quantize + int32 GEMM + dequant; the faster "
                      f"of the C oracle ({nruns} runs) and numpy float64 BLAS ({n64} runs), "
                      f"median after one warm-up run, threads bound to cores",
            "variant": "C oracle (AVX2 4x2 register blocks, OpenMP)" if best_c else
                       "numpy float64 BLAS",
            "ms": round(best * 1e3, 2), "c_oracle_ms": round(med * 1e3, 2),
            "cpu": cpu_model(), "nproc": os.cpu_count(),
            "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "openblas_num_threads": os.environ.get("OPENBLAS_NUM_THREADS"),
            "gpu_rows_bit_exact": exact,
            "numpy": {
                "int32_matmul": {"ms": round(m32 * 1e3, 2), "rows": r32, "runs": n32,
                                 "tops": round(2.0 * r32 * N * K / m32 / 1e12, 5),
                                 "threads": 1},
                "float64_blas": {"ms": round(m64 * 1e3, 2), "rows": rows, "runs": n64,
                                 "tops": round(2.0 * rows * N * K / m64 / 1e12, 4),
                                 "threads": "BLAS default"},
                "bit_exact_vs_c": np_exact}}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def measure_qwen3(torch, args, dev, torch_producers=False):
    """random-init Qwen3-8B-shaped stack (cider_amd/qwen3.py), all
    projections W8A8 per-channel; prefill of 2048 synthetic ids uniform over
    the vocabulary, then 128 greedy decode steps, each one replay of a HIP
    graph of the whole step (MV linears, attention over the device-resident
    KV cache, fp16 lm_head, argmax).  Returns (prefill_ms, decode_ms, tokens
    distinct, build_s, cfg)."""
    from cider_amd import qwen3 as Q
    cfg = Q.QWEN3_8B
    L, steps = 2048, 128
    t0 = time.perf_counter()
    m = Q.Qwen3(cfg, max_len=L + steps + 1, seed=args.seed, device=dev,
                fused=not torch_producers)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ids = torch.randint(0, cfg.vocab_size, (L,), device=dev, generator=gen)
    stream = torch.cuda.current_stream(dev)
    m.prefill(ids, last_only=True)  # warm-up
    torch.cuda.synchronize()
    reps = 3
    e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    e[0].record(stream)
    for _ in range(reps):
        logits = m.prefill(ids, last_only=True)
    e[1].record(stream)
    torch.cuda.synchronize()
    prefill_ms = e[0].elapsed_time(e[1]) / reps
    first = torch.argmax(logits[-1].float()).reshape(1)
    state = {"tok": first.clone(), "pos": torch.tensor([L], device=dev),
             "i": torch.zeros(1, dtype=torch.int64, device=dev),
             "out": torch.zeros(steps, dtype=torch.int64, device=dev)}
    g, _ = m.capture_decode(state)
    e[0].record(stream)
    for _ in range(steps):
        g.replay()
    e[1].record(stream)
    torch.cuda.synchronize()
    decode_ms = e[0].elapsed_time(e[1]) / steps
    distinct = int(state["out"].unique().numel())
    del g, m, logits
    torch.cuda.empty_cache()
    return prefill_ms, decode_ms, distinct, build_s, cfg


def bench_attn(torch, args, dev):
    """--attn: the causal prefill attention kernel per launch (HIP events on the
    launch stream), against the 2.5 PFLOP/s dense fp16 MFMA peak, with
    PyTorch's fused SDPA at the same shapes (the path the models used before);
    and the form the models call, which ends in o_proj's per-token
    quantization (cider_attn_prefill_quantize), beside the attention followed
    by a quantize launch."""
    import math

    import torch.nn.functional as TF
    from torch.nn.attention.bias import causal_lower_right

    from cider_amd import _lib
    from cider_amd import fused as FK
    from cider_amd import ops as OPS
    D, reps = 128, 20
    stream = torch.cuda.current_stream(dev)
    cases = []
    for name, c, n, H, KV in (("configs[3] Qwen3-8B prefill, 2048 tokens", 2048, 2048, 32, 8),
                              ("configs[4] Qwen3-VL chunk of 512 after 1536 cached", 512, 2048,
                               16, 8)):
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + c + n)
        q = torch.randn(c, H, D, device=dev, generator=g).half()
        kc = torch.randn(KV, n, D, device=dev, generator=g).half()
        vc = torch.randn(KV, n, D, device=dev, generator=g).half()
        scale = 1.0 / math.sqrt(D)
        out = torch.empty(c, H * D, dtype=torch.float16, device=dev)
        ws = FK.attn_prefill_workspace(c, n, H, dev)
        wsq = FK.attn_prefill_quantize_workspace(c, n, H, dev)
        qq, kk, vv = q.permute(1, 0, 2).unsqueeze(0), kc.unsqueeze(0), vc.unsqueeze(0)
        mask = None if c == n else causal_lower_right(c, n)

        def ours():
            FK.attn_prefill(q, kc, vc, n, scale, out=out, ws=ws)

        def quantized():
            FK.attn_prefill_quantize(q, kc, vc, n, scale, ws=wsq)

        def then_quantize():
            FK.attn_prefill(q, kc, vc, n, scale, out=out, ws=ws)
            OPS.quantize_per_token(out)

        def sdpa():
            if mask is None:
                return TF.scaled_dot_product_attention(qq, kk, vv, is_causal=True, enable_gqa=True)
            return TF.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, enable_gqa=True)

        times = {}
        for key, fn in (("kernel", ours), ("quantized", quantized), ("then_quantize", then_quantize),
                        ("sdpa", sdpa)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            times[key] = e0.elapsed_time(e1) / reps * 1e3  # us per launch
        # causal flops: 2 products of 2 D flops per (query, allowed key) pair
        flops = 4.0 * H * D * (c * (n - c) + c * (c + 1) / 2)
        tf = flops / times["kernel"] / 1e6
        cases.append({"case": name, "c": c, "n": n, "heads": H, "kv_heads": KV,
                      "key_parts": _lib.load().cider_attn_prefill_workspace_bytes(c, n, H)
                      // max(1, c * H * 130 * 4) or 1,
                      "kernel_us": round(times["kernel"], 2), "tflops": round(tf, 1),
                      "frac_fp16_peak": round(tf / 2500.0, 4),
                      "quantized_us": round(times["quantized"], 2),
                      "attention_then_quantize_us": round(times["then_quantize"], 2),
                      "sdpa_us": round(times["sdpa"], 2),
                      "speedup_vs_sdpa": round(times["sdpa"] / times["kernel"], 2)})
    print(json.dumps({"metric": "causal prefill attention (cider_attn_prefill) per launch",
                      "unit": "us", "higher_is_better": False, "dtype": "fp16 (fp32 softmax)",
                      "data": "synthetic N(0,1) q/k/v", "peak_tflops_fp16_dense": 2500.0,
                      "cases": cases}), flush=True)


def qwen3_summary(torch, args, dev):
    """The compact configs[3] figures of the default line."""
    L, steps = 2048, 128
    prefill_ms, decode_ms, distinct, _, cfg = measure_qwen3(torch, args, dev)
    return {"workload": "configs[3]: Qwen3-8B-shaped W8A8 per-channel stack, 36 layers, "
                        "random init; prefill of 2048 synthetic ids, then 128 greedy decode "
                        "steps (one HIP-graph replay per step)",
            "prefill_ms": round(prefill_ms, 3),
            "prefill_tokens_per_s": round(L / prefill_ms * 1e3, 1),
            "decode_ms_per_token": round(decode_ms, 4),
            "decode_tokens_per_s": round(1e3 / decode_ms, 1),
            "decode_steps": steps, "tokens_distinct": distinct}


def bench_qwen3(torch, args, dev):
    """configs[3] as its own JSON line (--qwen3)."""
    L, steps = 2048, 128
    prefill_ms, decode_ms, distinct, build_s, cfg = measure_qwen3(
        torch, args, dev, args.torch_producers)
    macs = cfg.linear_macs_per_token()
    w_bytes = macs + cfg.vocab_size * cfg.hidden_size * 2  # int8 linears + fp16 lm_head
    print(json.dumps({
        "metric": "Qwen3-8B-shaped W8A8 stack: prefill ms (2048 tokens), decode ms/token",
        "value": round(prefill_ms, 3), "unit": "ms", "higher_is_better": False,
        "n_gpus": 1, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "configs[3]: 36 layers, hidden 4096, intermediate 12288, "
                               "32 q / 8 kv heads of 128, vocab 151936 (fp16 lm_head), "
                               "random init, prefill 2048 ids + 128 greedy decode steps",
                   "seed": args.seed},
        "prefill": {"ms": round(prefill_ms, 3), "tokens_per_s": round(L / prefill_ms * 1e3, 1),
                    "linear_tops": round(2 * L * macs / (prefill_ms * 1e-3) / 1e12, 1)},
        "decode": {"ms_per_token": round(decode_ms, 4),
                   "tokens_per_s": round(1e3 / decode_ms, 1),
                   "weight_gbs": round(w_bytes / (decode_ms * 1e-3) / 1e9, 1),
                   "steps": steps, "graph": True,
                   "tokens_distinct": distinct},
        "producers": ("pytorch ops" if args.torch_producers else
                      "fused HIP kernels (RMSNorm/SwiGLU + quantize, q/k norm + RoPE, "
                      "decode attention)"),
        "build_s": round(build_s, 1),
    }), flush=True)


def bench_qwen3vl(torch, args, dev):
    """random-init Qwen3-VL-2B-shaped text decoder
    (cider_amd/qwen3vl.py), W8A8 per-channel projections, prompts of 1334 /
    2393 / 3455 tokens with 2 / 3 / 4 synthetic 256-token image blocks at
    3-axis M-RoPE positions, chunked prefill (chunk 512), then 64 greedy
    decode steps per prompt, each one replay of the captured decode step."""
    from cider_amd import qwen3vl as V
    cfg = V.QWEN3_VL_2B
    prompts = [(1334, 2), (2393, 3), (3455, 4)]
    steps = 64
    t0 = time.perf_counter()
    m = V.Qwen3VL(cfg, max_len=max(p for p, _ in prompts) + steps + 1, seed=args.seed,
                  device=dev)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    stream = torch.cuda.current_stream(dev)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    rows = []
    for i, (L, n_img) in enumerate(prompts):
        segs = V.synth_segments(L, n_img, args.seed + i)
        x, _ = m.embed_prompt(segs, seed=args.seed + i)
        pos3 = V.rope_index(segs)
        m.prefill_chunked(x, pos3)      # warm-up (also fills the cache)
        torch.cuda.synchronize()
        reps = 3
        e[0].record(stream)
        for _ in range(reps):
            logits = m.prefill_chunked(x, pos3)
        e[1].record(stream)
        torch.cuda.synchronize()
        pre_ms = e[0].elapsed_time(e[1]) / reps
        first = torch.argmax(logits[-1].float()).reshape(1)
        state = {"tok": first.clone(), "pos": torch.tensor([L], device=dev),
                 "i": torch.zeros(1, dtype=torch.int64, device=dev),
                 "out": torch.zeros(steps, dtype=torch.int64, device=dev)}
        g, _ = m.capture_decode(state)
        e[0].record(stream)
        for _ in range(steps):
            g.replay()
        e[1].record(stream)
        torch.cuda.synchronize()
        dec_ms = e[0].elapsed_time(e[1]) / steps
        rows.append({"prompt_tokens": L, "images": n_img,
                     "prefill_ms": round(pre_ms, 3),
                     "prefill_tokens_per_s": round(L / pre_ms * 1e3, 1),
                     "decode_ms_per_token": round(dec_ms, 4),
                     "decode_tokens_per_s": round(1e3 / dec_ms, 1),
                     "tokens_distinct": int(state["out"].unique().numel())})
    print(json.dumps({
        "metric": "Qwen3-VL-2B-shaped W8A8 text decoder: chunked-prefill tokens/s and decode "
                  "tokens/s at 1334 / 2393 / 3455-token multimodal prompts",
        "value": rows[-1]["prefill_tokens_per_s"], "unit": "tokens/s (prefill, 3455 tokens)",
        "higher_is_better": True, "n_gpus": 1, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "configs[4]: 28 layers, hidden 2048, intermediate 6144, 16 q / 8 kv "
                               "heads of 128, vocab 151936 (tied fp16 lm_head), random init; "
                               "text ids + 256-token fp16 N(0,0.02) image blocks at M-RoPE "
                               "positions; chunk 512; 64 graph-replayed greedy decode steps",
                   "seed": args.seed},
        "prompts": rows,
        "reference_m5pro_w8a8_pc": {"prefill_tokens_per_s": [3242, 2983, 2796],
                                    "decode_tokens_per_s": [104, 100, 95],
                                    "note": "different hardware and the full VLM service"},
        "build_s": round(build_s, 1),
    }), flush=True)


# (bm, bn, rate) for int8 weights, as pick_tile in cider_amd/csrc/gemm_dma.hip
_TILES_I8 = [(256, 256, 1.0), (128, 256, 0.87), (128, 128, 0.75), (128, 64, 0.517),
             (64, 128, 0.508), (64, 64, 0.40), (192, 256, 0.90)]


def gemm_kernel_name(M, N, K, dev):
    """The GEMM kernel the library's dispatcher launches for this shape
    (int8 weights, per-channel; cider_amd/csrc/gemm_dma.hip, pick_tile)."""
    import torch
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    if K % 128 == 0 and N % 8 == 0 and M > 64:
        best, best_cost = None, None
        for bm, bn, rate in _TILES_I8:
            tiles = -(-M // bm) * -(-N // bn)
            full, rest = divmod(tiles, cus)
            rounds = full + (0.6 + 0.4 * rest / cus if rest else 0.0)
            cost = rounds * bm * bn / rate
            if best_cost is None or cost < best_cost * 0.999:
                best, best_cost = (bm, bn), cost
        tm, tn = -(-M // 256), -(-N // 256)
        T = tm * tn
        R = T % cus
        if T > cus and 0 < R and 2 * R <= cus and R % tm == 0:
            tail = (0.6 + 0.4 * 2 * R / cus) * 128 * 256 / 0.87
            if (T // cus) * 256 * 256 + tail < best_cost * 0.999:
                return ("gemm_dma_mixed_kernel<PC, I8, 8> (256x256 tiles + 128x256 tiles, "
                        "half of them first and half last, 8 waves)")
        waves = 8 if best[1] == 256 else 4
        return "gemm_dma_kernel<%d, %d, 128, PC, I8, %d> (%dx%d tiles, %d waves)" % (
            best[0], best[1], waves, best[0], best[1], waves)
    return "gemm_kernel<PC>"


def load_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 PMC summary, if any."""
    p = os.path.join(ROOT, "profiles", "gemm_pc_m4096_traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


if __name__ == "__main__":
    main()

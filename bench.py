"""Benchmark of the MI355X KuDNN Linear/GEMM path (one JSON line on stdout).

Workload ("C3"): bf16 Linear + GELU(tanh) + residual add,
X[4096,4096] x W[11008,4096]^T, zero bias, residual R[4096,11008], fp32 accumulate, bf16 out. One step
is one call of the fused Linear post-op chain through the C ABI on inputs already resident in HBM.

Also reported (not `value`): the decode-shaped skinny Linear at M in {1, 4, 16}, K=4096, N in {4096, 14336}
(configs[3], Linear then element-wise multiply) in GB/s, timed over rotating weight copies (>= 512 MB) so that the 256 MB Infinity Cache
cannot serve the weight stream; C1, C2 and C5 in TFLOP/s; C3's shape in f16 (same post-ops) and as an s8 x s8 -> s32
GEMM (TOP/s against the 5.0 POP/s int8 peak); and the CPU baseline (the reference tests' portable naive loop, timed
on a bounded row sample of the same workload on this host's cores).

Before the W counted warmup steps, the step is also run untimed for --prewarm-ms of wall time (default 300 ms):
the GPU raises its clocks over the first ~100 ms of sustained load, and a timed region that starts on a cold GPU
reports the ramp rather than the kernel (10-15 % slower per step over the first tens of milliseconds).

For profiling, --only c3 runs just the C3 step (JSON line without decode or CPU baseline), --only decode just the
decode lines (--only decode-sweep: the decode step over M in 1..16 and N in 4096..28672, or the lists --sweep-m and
--sweep-n give, one JSON line each, the measurements behind the skinny dispatch rule), and --only copy runs an
elementwise copy-like kernel (y = -x, 512 MiB bf16 in, 512 MiB out) whose known traffic calibrates the
FETCH_SIZE / WRITE_SIZE counters against which the C3 kernel's HBM traffic is read. --only dispatch times a bf16
Linear + GELU(tanh) over prefill-like shapes under every kernel configuration (forced through KUDNN_HIP_FORCE_CFG and
KUDNN_HIP_FORCE_STREAMK, K slices by the planner's rule or none through KUDNN_HIP_FORCE_KSLICES) and under the
planner's own choice, one JSON line per shape, then an f32 Gemm over grids of
256-640 tiles of 128 x 128 under the 128 x 128 and 64 x 64 configurations: the measurements the dispatcher's rules are
drawn from. --only refperf times KuDNN::Gemm on the reference's own perf shape sets (the matmul gtest's freParas and
freParasMulti) in f32 and bf16, under the planner and under every forced configuration, one JSON line per shape and
type. --only torch times C3's shape through PyTorch's own ops (the bf16 GEMM alone, then GEMM + GELU + add unfused),
then C1, C2, C5 and the decode shapes the same way, for comparison. --only c1 prints the C1 line alone.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--prewarm-ms 300]
                       [--only c3|c1|copy|decode|decode-sweep|dispatch|refperf|torch]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "Linear+postop TFLOP/s (% MFMA peak) at 4096x4096x11008; M=1 GB/s (% HBM)"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_F32_TFLOPS = 157.3    # MI355X dense fp32 MFMA
PEAK_F16_TFLOPS = 2500.0   # MI355X dense f16 MFMA
PEAK_I8_TOPS = 5000.0      # MI355X dense int8 MFMA


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--prewarm-ms", type=float, default=300.0, help="untimed run time before warmup (clock ramp)")
    p.add_argument("--only", choices=["c3", "c1", "copy", "decode", "decode-sweep", "dispatch", "refperf", "torch"],
                   default=None,
                   help="profiling modes (see module docstring)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--no-others", action="store_true", help="skip the informational C1 / C2 / C5 lines")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU-baseline sample time")
    p.add_argument("--summarize-traffic", metavar="DIR", default=None,
                   help="read rocprofv3 FETCH_SIZE / WRITE_SIZE captures of --only c3 and --only copy from "
                        "DIR/{c3,copy}_{fetch,write}/run_counter_collection.csv and write profiles/traffic_c3.json "
                        "(no GPU needed; the digest is the built library's)")
    p.add_argument("--summarize-counters", metavar="CSV", default=None,
                   help="print per-dispatch means of every counter of the C3 kernel in a rocprofv3 "
                        "run_counter_collection.csv, with its duration, clock and MFMA busy fraction (no GPU needed)")
    p.add_argument("--counter-kernel", metavar="NAME", default=None,
                   help="with --summarize-counters: summarise the kernel whose name contains NAME instead of C3's")
    p.add_argument("--sweep-m", default="1,2,3,4,5,6,8,10,12,16", help="with --only decode-sweep: the values of M")
    p.add_argument("--sweep-n", default="4096,8192,14336,28672", help="with --only decode-sweep: the values of N")
    return p.parse_args()


# ---------------------------------------------------------------------------------------------------
# synthetic inputs: SplitMix64 (Vigna) per tensor, seed = config seed 0 + stream offset (X 0, W 1, bias 2,
# R / M2 3); uniform from the top 53 bits, normal by Box-Muller over two consecutive draws; a bf16 tensor is the
# RNE of the f32 sample. The k-th draw of a stream is mix(seed + k * golden gamma), so a whole tensor is generated on
# the device in one pass of int64 arithmetic (wrapping multiplication, masked shifts for the logical right shift).

_GAMMA = 0x9E3779B97F4A7C15
_MUL1 = 0xBF58476D1CE4E5B9
_MUL2 = 0x94D049BB133111EB


def _i64(c):
    return c - (1 << 64) if c >= (1 << 63) else c


def _u01(torch, first, n, seed, dev):
    k = torch.arange(first, first + n, device=dev, dtype=torch.int64)
    z = k * _i64(_GAMMA) + _i64(seed % (1 << 64))
    z = (z ^ ((z >> 30) & ((1 << 34) - 1))) * _i64(_MUL1)
    z = (z ^ ((z >> 27) & ((1 << 37) - 1))) * _i64(_MUL2)
    z = z ^ ((z >> 31) & ((1 << 33) - 1))
    return ((z >> 11) & ((1 << 53) - 1)).to(torch.float64) * (1.0 / 9007199254740992.0)


def synth(torch, shape, seed, dist, a, b, dtype, dev="cuda", chunk=1 << 24):
    """Tensor of `shape`: dist "uniform" on [a, b) or "normal" with mean a and standard deviation b. Generated in
    pieces of `chunk` elements, which bounds the int64 / float64 temporaries."""
    n = 1
    for d in shape:
        n *= d
    out = torch.empty(n, device=dev, dtype=torch.float32)
    for c0 in range(0, n, chunk):
        m = min(chunk, n - c0)
        if dist == "uniform":
            v = a + (b - a) * _u01(torch, c0 + 1, m, seed, dev)
        else:
            u = _u01(torch, 2 * c0 + 1, 2 * m, seed, dev).view(m, 2)
            u1 = torch.clamp(u[:, 0], min=1e-300)
            v = a + b * torch.sqrt(-2.0 * torch.log(u1)) * torch.cos(6.283185307179586 * u[:, 1])
        out[c0:c0 + m] = v.to(torch.float32)
    return out.view(*shape).to(dtype)


def time_launches(fn, steps, warmup, torch, stream, prewarm_ms=0.0):
    # the untimed calls rotate over the inputs as the timed ones do, so a profile of the run sees the same cache state
    t_end = time.perf_counter() + prewarm_ms * 1e-3
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn(i)
        i += 1
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall / steps * 1e3


def time_graph(run_on, n, replays, torch):
    """Milliseconds per step of n steps captured in one HIP graph and replayed `replays` times on a side stream (the
    device's time per step without the host's launch cost). run_on(stream, i) issues step i on `stream`; it is warmed
    on that stream first, so nothing is allocated during capture."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(n):
            run_on(s, i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                run_on(s, i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(replays):
            g.replay()
        e1.record(s)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (n * replays)


def bench_c3(args, torch, K):
    M, Kd, N = 4096, 4096, 11008
    dev = "cuda"
    bf = torch.bfloat16
    x = synth(torch, (M, Kd), 0, "normal", 0.0, 1.0, bf)
    w = synth(torch, (N, Kd), 1, "normal", 0.0, 0.02, bf)  # nn.Linear weight [N][K]
    bias = torch.zeros(1, N, device=dev, dtype=bf)
    r = synth(torch, (M, N), 3, "normal", 0.0, 1.0, bf)
    y = torch.empty(M, N, device=dev, dtype=bf)

    dx = K.desc([M, Kd], K.BF16, "AB")
    dw = K.desc([Kd, N], K.BF16, "BA")  # logical [K,N], physical [N][K]
    dy = K.desc([M, N], K.BF16, "AB")
    db = K.desc([1, N], K.BF16, "AB")
    plan = K.LinearPostOps(dx, dw, dy, db, act=K.ACT_GELU_TANH, binary=K.BIN_ADD, src=dy)
    stream = torch.cuda.current_stream()

    def step(i=0):
        plan.run(x, w, y, bias, r, stream=stream)

    ms_kernel, ms_wall = time_launches(step, args.steps, args.warmup, torch, stream, args.prewarm_ms)
    flops = 2.0 * M * N * Kd
    alg_bytes = 2 * (M * Kd + N * Kd + N + M * N + M * N)
    tflops = flops / (ms_kernel * 1e-3) / 1e12
    return {
        "plan": plan.describe(),
        "ms": ms_kernel,
        "ms_wall": ms_wall,
        "tflops": tflops,
        "flops": flops,
        "alg_bytes": alg_bytes,
    }


def bench_torch_c3(args, torch):
    """C3's shape through PyTorch's own ops, for comparison only (not this library): the bf16 GEMM alone
    (`torch.nn.functional.linear`, which ROCm's PyTorch hands to hipBLASLt), and the whole C3 step as that GEMM
    followed by separate GELU_tanh and add kernels. Same inputs and timing as the C3 line."""
    M, Kd, N = 4096, 4096, 11008
    bf = torch.bfloat16
    x = synth(torch, (M, Kd), 0, "normal", 0.0, 1.0, bf)
    w = synth(torch, (N, Kd), 1, "normal", 0.0, 0.02, bf)
    r = synth(torch, (M, N), 3, "normal", 0.0, 1.0, bf)
    y = torch.empty(M, N, device="cuda", dtype=bf)
    stream = torch.cuda.current_stream()
    F = torch.nn.functional
    flops = 2.0 * M * N * Kd
    for name, fn in (("torch linear (bf16 GEMM only)", lambda i=0: torch.matmul(x, w.t(), out=y)),
                     ("torch linear + gelu(tanh) + add (unfused)",
                      lambda i=0: torch.add(F.gelu(F.linear(x, w), approximate="tanh"), r, out=y))):
        ms, _ = time_launches(fn, args.steps, args.warmup, torch, stream, args.prewarm_ms)
        print(json.dumps({"op": name, "M": M, "K": Kd, "N": N, "ms": round(ms, 4),
                          "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}), flush=True)


def bench_torch_others(args, torch):
    """C1, C2, C5 and the decode shapes through PyTorch's own ops, for comparison only (not this library): the GEMM
    alone and the unfused Linear + post-op (hipBLASLt / rocBLAS on ROCm's PyTorch), with the inputs, the rotation over
    input copies and the timing of this library's lines for the same configurations."""
    F = torch.nn.functional
    torch.backends.cuda.matmul.allow_tf32 = False
    stream = torch.cuda.current_stream()

    def emit(op, cfg, M, Kd, N, ms, flops, alg_bytes=None):
        rec = {"op": op, "config": cfg, "M": M, "K": Kd, "N": N, "us": round(ms * 1e3, 2),
               "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2)}
        if alg_bytes is not None:
            rec["GB/s"] = round(alg_bytes / (ms * 1e-3) / 1e9, 1)
            rec["frac_hbm"] = round(alg_bytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
        print(json.dumps(rec), flush=True)

    for name in ("C1", "C2", "C5"):
        if name == "C1":
            M, Kd, N, dt, act, copies = 128, 1024, 1024, torch.float32, F.relu, 1
            xd, wd, bd = ("uniform", -1.0, 1.0), ("uniform", -1.0, 1.0), ("uniform", -0.1, 0.1)
        elif name == "C2":
            M, Kd, N, dt, act, copies = 2048, 4096, 4096, torch.float32, F.silu, 4
            xd, wd, bd = ("normal", 0.0, 1.0), ("normal", 0.0, 1.0 / 64), ("normal", 0.0, 0.02)
        else:
            M, Kd, N, dt, act, copies = 16384, 5120, 13824, torch.bfloat16, F.silu, 1
            xd, wd, bd = ("normal", 0.0, 1.0), ("normal", 0.0, 0.014), ("normal", 0.0, 0.02)
        xs = [synth(torch, (M, Kd), 0 + 16 * c, *xd, dt) for c in range(copies)]
        bias = synth(torch, (1, N), 2, *bd, dt).reshape(N)
        y = torch.empty(M, N, device="cuda", dtype=dt)
        if name == "C5":  # the weight stored [K][N], as in the C5 line
            w = synth(torch, (Kd, N), 1, *wd, dt)
            xb = xs[0].reshape(8, 2048, Kd)
            yb = y.reshape(8, 2048, N)
            fns = (("GEMM only", lambda i=0: torch.matmul(xb, w, out=yb)),
                   ("GEMM + bias + silu (unfused)", lambda i=0: act(torch.matmul(xb, w) + bias)))
        else:  # nn.Linear weight [N][K]
            ws = [synth(torch, (N, Kd), 1 + 16 * c, *wd, dt) for c in range(copies)]
            fns = (("GEMM only", lambda i=0: torch.matmul(xs[i % copies], ws[i % copies].t(), out=y)),
                   ("linear + bias + act (unfused)", lambda i=0: act(F.linear(xs[i % copies], ws[i % copies], bias))))
        for op, fn in fns:
            ms, _ = time_launches(fn, args.steps, max(args.warmup, copies), torch, stream, args.prewarm_ms)
            emit(f"torch {op}", name, M, Kd, N, ms, 2.0 * M * N * Kd)

    Kd = 4096
    for N in (4096, 14336):
        copies = max(2, -(-512 * 2**20 // (N * Kd * 2)))  # >= 512 MB of distinct weights, as in the decode lines
        ws = [synth(torch, (N, Kd), 1 + 16 * c, "normal", 0.0, 0.02, torch.bfloat16) for c in range(copies)]
        for M in (1, 4, 16):
            x = synth(torch, (M, Kd), 0, "normal", 0.0, 1.0, torch.bfloat16)
            m2 = synth(torch, (M, N), 3, "uniform", 0.5, 1.5, torch.bfloat16)
            y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
            alg = 2 * (N * Kd + M * Kd + 2 * M * N)
            for op, fn in (("linear only", lambda i=0: torch.matmul(x, ws[i % copies].t(), out=y)),
                           ("linear * M2 (unfused)", lambda i=0: torch.mul(F.linear(x, ws[i % copies]), m2, out=y))):
                steps = max(args.steps, 4 * copies)
                ms, _ = time_launches(fn, steps, max(args.warmup, copies), torch, stream, args.prewarm_ms)
                emit(f"torch {op}", "C4", M, Kd, N, ms, 2.0 * M * N * Kd, alg)


def bench_decode(args, torch, K, N, M=1):
    Kd = 4096
    dev = "cuda"
    wbytes = N * Kd * 2
    copies = max(2, -(-512 * 2**20 // wbytes))  # >= 512 MB of distinct weights
    bf = torch.bfloat16
    # copy c of the weight is stream 1 + 16 * c, so the copies differ and copy 0 is the config's W
    ws = [synth(torch, (N, Kd), 1 + 16 * c, "normal", 0.0, 0.02, bf) for c in range(copies)]
    x = synth(torch, (M, Kd), 0, "normal", 0.0, 1.0, bf)
    m2 = synth(torch, (M, N), 3, "uniform", 0.5, 1.5, bf)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    plan = K.LinearPostOps(K.desc([M, Kd], K.BF16), K.desc([Kd, N], K.BF16, "BA"), K.desc([M, N], K.BF16),
                           binary=K.BIN_MUL, src=K.desc([M, N], K.BF16))
    stream = torch.cuda.current_stream()

    def step(i=0):
        plan.run(x, ws[i % copies], y, None, m2, stream=stream)

    steps = max(args.steps, 4 * copies)
    ms, ms_wall = time_launches(step, steps, max(args.warmup, copies), torch, stream, args.prewarm_ms)
    ms_graph = time_graph(lambda s, i: plan.run(x, ws[i % copies], y, None, m2, stream=s), 4 * copies, 10, torch)
    alg_bytes = 2 * (N * Kd + M * Kd + 2 * M * N)
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    gbs_graph = alg_bytes / (ms_graph * 1e-3) / 1e9
    return {"N": N, "M": M, "K": Kd, "plan": plan.describe(), "us": ms * 1e3, "us_wall": ms_wall * 1e3,
            "GB/s": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "us_graph": ms_graph * 1e3, "frac_hbm_graph": gbs_graph / PEAK_HBM_GBS,
            "weight_copies": copies, "alg_bytes": alg_bytes}


def bench_config(args, torch, K, name):
    """The other configurations (informational, not `value`): C1, C2 (fp32) and C5 (bf16 3-D, K-major weight).

    C2's inputs are rotated over 4 copies (>= 512 MB) so that the Infinity Cache does not hold them; C1's 5 MB working
    set is cache-resident whatever is done, and C5's 760 MB footprint exceeds the cache by itself."""
    dev = "cuda"
    if name == "C1":
        M, Kd, N, dt, kind, alpha, copies = 128, 1024, 1024, torch.float32, K.ACT_RELU, 0.0, 1
        xd, wd, bd = ("uniform", -1.0, 1.0), ("uniform", -1.0, 1.0), ("uniform", -0.1, 0.1)
    elif name == "C2":
        M, Kd, N, dt, kind, alpha, copies = 2048, 4096, 4096, torch.float32, K.ACT_SWISH, 1.0, 4
        xd, wd, bd = ("normal", 0.0, 1.0), ("normal", 0.0, 1.0 / 64), ("normal", 0.0, 0.02)
    else:
        M, Kd, N, dt, kind, alpha, copies = 16384, 5120, 13824, torch.bfloat16, K.ACT_SWISH, 1.0, 1
        xd, wd, bd = ("normal", 0.0, 1.0), ("normal", 0.0, 0.014), ("normal", 0.0, 0.02)
    kdt = K.F32 if dt == torch.float32 else K.BF16
    # copy c of an input is its stream + 16 * c (copy 0 is the config's tensor)
    xs = [synth(torch, (M, Kd), 0 + 16 * c, *xd, dt) for c in range(copies)]
    if name == "C5":  # W{1,5120,13824} ABC: K-major [K][N], broadcast over the batch of 8
        ws = [synth(torch, (Kd, N), 1, *wd, dt)]
        da, db, dc = K.desc([8, 2048, Kd], kdt, "ABC"), K.desc([1, Kd, N], kdt, "ABC"), K.desc([8, 2048, N], kdt, "ABC")
        dbias = K.desc([1, 1, N], kdt, "ABC")
    else:  # nn.Linear weight [N][K] (logical [K,N], layout BA)
        ws = [synth(torch, (N, Kd), 1 + 16 * c, *wd, dt) for c in range(copies)]
        da, db, dc, dbias = K.desc([M, Kd], kdt), K.desc([Kd, N], kdt, "BA"), K.desc([M, N], kdt), K.desc([1, N], kdt)
    bias = synth(torch, (1, N), 2, *bd, dt)
    y = torch.empty(M, N, device=dev, dtype=dt)
    plan = K.LinearActivation(da, db, dc, dbias, alpha, 0.0, kind)
    stream = torch.cuda.current_stream()

    def step(i=0):
        plan.run(xs[i % copies], ws[i % copies], y, bias, stream=stream)

    ms, _ = time_launches(step, args.steps, max(args.warmup, copies), torch, stream, args.prewarm_ms)
    flops = 2.0 * M * N * Kd
    tflops = flops / (ms * 1e-3) / 1e12
    peak = PEAK_F32_TFLOPS if dt == torch.float32 else PEAK_BF16_TFLOPS
    out = {"config": name, "M": M, "K": Kd, "N": N, "plan": plan.describe(), "us": ms * 1e3, "TFLOP/s": tflops,
           "frac_peak": tflops / peak, "input_copies": copies}
    if name == "C1":  # a latency-bound call: also its time per step with the launches captured in a graph
        out["us_graph"] = time_graph(lambda s, i: plan.run(xs[0], ws[0], y, bias, stream=s), 50, 20, torch) * 1e3
    return out


def bench_c3_dtype(args, torch, K, name):
    """Informational: C3's shape in the other operand types of the primitive. "C3-f16": the same Linear + GELU_tanh +
    residual add with f16 tensors; "C3-s8": the s8 x s8 -> s32 GEMM (W8A8; the integer path has no post-ops), inputs
    uniform integers in [-128, 127] rounded from the same generator."""
    M, Kd, N = 4096, 4096, 11008
    stream = torch.cuda.current_stream()
    if name == "C3-f16":
        f16 = torch.float16
        x = synth(torch, (M, Kd), 0, "normal", 0.0, 1.0, f16)
        w = synth(torch, (N, Kd), 1, "normal", 0.0, 0.02, f16)
        r = synth(torch, (M, N), 3, "normal", 0.0, 1.0, f16)
        y = torch.empty(M, N, device="cuda", dtype=f16)
        dy = K.desc([M, N], K.F16)
        plan = K.LinearPostOps(K.desc([M, Kd], K.F16), K.desc([Kd, N], K.F16, "BA"), dy, None, act=K.ACT_GELU_TANH,
                               binary=K.BIN_ADD, src=dy)

        def step(i=0):
            plan.run(x, w, y, None, r, stream=stream)
        peak, unit = PEAK_F16_TFLOPS, "TFLOP/s"
    else:
        def s8(shape, seed):
            return torch.clamp(torch.round(synth(torch, shape, seed, "uniform", -128.5, 127.5, torch.float32)),
                               -128, 127).to(torch.int8)
        x, w = s8((M, Kd), 0), s8((N, Kd), 1)
        y = torch.empty(M, N, device="cuda", dtype=torch.int32)
        plan = K.Gemm(K.desc([M, Kd], K.S8), K.desc([Kd, N], K.S8, "BA"), K.desc([M, N], K.S32))

        def step(i=0):
            plan.run(x, w, y, stream=stream)
        peak, unit = PEAK_I8_TOPS, "TOP/s"
    ms, _ = time_launches(step, args.steps, args.warmup, torch, stream, args.prewarm_ms)
    rate = 2.0 * M * N * Kd / (ms * 1e-3) / 1e12
    return {"config": name, "M": M, "K": Kd, "N": N, "plan": plan.describe(), "us": ms * 1e3, unit: rate,
            "frac_peak": rate / peak}


C3_KERNEL = "gemm_pingpong_kernel<3, 20, 0, false, false>"  # bf16 operands, GELU_tanh, all-bf16 epilogue form


def counter_dispatches(csv_path, kernel_sub):
    """{dispatch id: {"counters": {name: value summed over the dispatch's rows}, "ns": duration}} for the dispatches
    of a rocprofv3 run_counter_collection.csv whose kernel name contains kernel_sub."""
    import csv

    out = {}
    with open(csv_path, newline="") as f:
        for row in csv.DictReader(f):
            if kernel_sub not in row["Kernel_Name"]:
                continue
            d = out.setdefault(row["Dispatch_Id"], {"counters": {}, "ns": 0})
            c = d["counters"]
            c[row["Counter_Name"]] = c.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
            d["ns"] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    return out


def _mean(xs):
    xs = list(xs)
    return sum(xs) / len(xs) if xs else float("nan")


def summarize_counters(path, kernel=C3_KERNEL):
    """Per-dispatch means of one kernel's counters in one capture (the C3 kernel unless another kernel-name substring
    is given), with the clock that GRBM_GUI_ACTIVE gives over the dispatch time (the counter is summed over the 8 XCCs)
    and the MFMA busy fraction of the 1024 SIMDs."""
    ds = counter_dispatches(path, kernel)
    names = sorted({n for d in ds.values() for n in d["counters"]})
    res = {"kernel": kernel, "dispatches": len(ds), "mean_us": _mean(d["ns"] / 1e3 for d in ds.values())}
    for n in names:
        res[n] = _mean(d["counters"][n] for d in ds.values() if n in d["counters"])
    if "GRBM_GUI_ACTIVE" in res:
        clocks = [d["counters"]["GRBM_GUI_ACTIVE"] / 8 / d["ns"] for _, d in sorted(ds.items(), key=lambda kv: int(kv[0]))]
        res["clock_ghz"] = _mean(clocks)
        res["clock_ghz_min_max"] = [min(clocks), max(clocks)]
        res["clock_ghz_last_half"] = _mean(clocks[len(clocks) // 2:])
        if "SQ_VALU_MFMA_BUSY_CYCLES" in res:
            res["mfma_busy"] = _mean(d["counters"]["SQ_VALU_MFMA_BUSY_CYCLES"] /
                                     (d["counters"]["GRBM_GUI_ACTIVE"] / 8 * 1024) for d in ds.values())
    print(json.dumps(res, indent=1))
    return res


def summarize_traffic(d):
    """profiles/traffic_c3.json from FETCH_SIZE / WRITE_SIZE captures of the C3 kernel and of the copy-like calibration
    kernel (torch.neg over 512 MiB bf16: its known bytes give each counter's scale on this part)."""
    import kudnn_amd as K

    d = Path(d)
    cap = {k: d / k / "run_counter_collection.csv" for k in ("c3_fetch", "c3_write", "copy_fetch", "copy_write")}
    c3f = counter_dispatches(cap["c3_fetch"], C3_KERNEL)
    c3w = counter_dispatches(cap["c3_write"], C3_KERNEL)
    cpf = counter_dispatches(cap["copy_fetch"], "neg_kernel")
    cpw = counter_dispatches(cap["copy_write"], "neg_kernel")
    fetch = _mean(x["counters"]["FETCH_SIZE"] for x in c3f.values())
    write = _mean(x["counters"]["WRITE_SIZE"] for x in c3w.values())
    cfetch = _mean(x["counters"]["FETCH_SIZE"] for x in cpf.values())
    cwrite = _mean(x["counters"]["WRITE_SIZE"] for x in cpw.values())
    copy_bytes = 512 << 20
    fs, ws = copy_bytes / (cfetch * 1024), copy_bytes / (cwrite * 1024)
    rd, wr = fetch * 1024 * fs, write * 1024 * ws
    alg = 2 * (4096 * 4096 + 11008 * 4096 + 2 * 4096 * 11008)
    rec = {"kernel": C3_KERNEL, "workload": "C3 4096x4096x11008 bf16 Linear+GELU_tanh+residual add",
           "source_digest": K.lib().kudnn_pingpong_source_digest().decode(),
           "dispatches": {"fetch": len(c3f), "write": len(c3w)},
           "fetch_kib_per_dispatch": round(fetch, 1), "write_kib_per_dispatch": round(write, 1),
           "copy_fetch_kib_per_dispatch": round(cfetch, 1), "copy_write_kib_per_dispatch": round(cwrite, 1),
           "copy_bytes_each_way": copy_bytes, "fetch_scale": round(fs, 5), "write_scale": round(ws, 5),
           "hbm_read_bytes_per_launch": int(rd), "hbm_write_bytes_per_launch": int(wr),
           "hbm_bytes_per_launch": int(rd + wr), "algorithmic_bytes_per_launch": alg,
           "traffic_over_algorithmic": round((rd + wr) / alg, 3)}
    (ROOT / "profiles" / "traffic_c3.json").write_text(json.dumps(rec, indent=1) + "\n")
    print(json.dumps(rec, indent=1))


def cpu_model():
    """The host CPU's model name (as lscpu prints it), from /proc/cpuinfo."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_rate(np, O, dt, M, N, Kd, act, act_alpha, threads, seconds, resid=None, bias_scale=0.0, w_scale=0.02):
    """TFLOP/s of the reference tests' naive Linear loop (f32 accumulation, OpenMP over rows) on a row sample of an
    M x K x N problem, grown until it takes about `seconds`; resid "mul" multiplies a [rows, N] operand in (C4).
    O is the oracle module (the timed CPU loop lives there). Returns (TFLOP/s, rows, seconds)."""
    rng = np.random.default_rng(0)
    f32 = dt == O.F32
    conv = (lambda a: a.astype(np.float32)) if f32 else (lambda a: O.from_f32_rne(a.astype(np.float32), O.BF16))
    w = conv(rng.standard_normal((N, Kd), dtype=np.float32) * w_scale)
    bias = conv(rng.standard_normal(N, dtype=np.float32) * bias_scale)

    def run(rows):
        x = conv(rng.standard_normal((rows, Kd), dtype=np.float32))
        r = conv(rng.uniform(0.5, 1.5, (rows, N)).astype(np.float32)) if resid else None
        y = np.zeros(rows * N, dtype=np.float32 if f32 else np.uint16)
        t0 = time.perf_counter()
        O.cpu_baseline(dt, rows, N, Kd, x, w, bias, r, y, act, act_alpha, threads, r_mul=resid == "mul")
        return time.perf_counter() - t0

    rows = min(M, 8)
    t = run(rows)
    if t < seconds and rows < M:  # cost is linear in rows
        rows = int(min(M, max(rows, rows * seconds / max(t, 1e-3))))
        t = run(rows)
    reps = 1
    if t < seconds / 2:  # the whole problem is short: repeat it
        reps = int(min(10000, seconds / max(t, 1e-4)))
        t = sum(run(rows) for _ in range(reps)) / reps
    return 2.0 * rows * N * Kd / t / 1e12, rows, t, reps


def cpu_baseline(args, np):
    """The reference tests' naive Linear loop (f32 accumulation, OpenMP over rows) on a row sample of C3, and the same
    loop on every other configuration (C1 also on one thread)."""
    import oracle as O

    M, Kd, N = 4096, 4096, 11008
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    rng = np.random.default_rng(0)
    w = O.from_f32_rne((rng.standard_normal((N, Kd), dtype=np.float32) * 0.02), O.BF16)
    bias = np.zeros(N, dtype=np.uint16)

    def run(rows):
        x = O.from_f32_rne(rng.standard_normal((rows, Kd), dtype=np.float32), O.BF16)
        r = O.from_f32_rne(rng.standard_normal((rows, N), dtype=np.float32), O.BF16)
        y = np.zeros(rows * N, dtype=np.uint16)
        t0 = time.perf_counter()
        O.cpu_baseline(O.BF16, rows, N, Kd, x, w, bias, r, y, O.ACT_GELU_TANH, 0.0, threads)
        return time.perf_counter() - t0

    rows = 8
    dt = run(rows)
    if dt < args.cpu_seconds:  # scale the sample to about cpu_seconds of work (cost is linear in rows)
        rows = int(min(M, max(rows, rows * args.cpu_seconds / max(dt, 1e-3))))
        dt = run(rows)
    tflops = 2.0 * rows * N * Kd / dt / 1e12

    # the other configurations, each on a sample of about a quarter of cpu_seconds
    share = args.cpu_seconds / 4
    per = []
    for name, dtp, m, n, k, act, alpha, resid, bs, ws, thr in (
            ("C1", O.F32, 128, 1024, 1024, O.ACT_RELU, 0.0, None, 0.1, 1.0, threads),
            ("C1 (1 thread)", O.F32, 128, 1024, 1024, O.ACT_RELU, 0.0, None, 0.1, 1.0, 1),
            ("C2", O.F32, 2048, 4096, 4096, O.ACT_SWISH, 1.0, None, 0.02, 1.0 / 64, threads),
            ("C4 M=1 N=4096", O.BF16, 1, 4096, 4096, O.ACT_NONE, 0.0, "mul", 0.0, 0.02, threads),
            ("C4 M=16 N=14336", O.BF16, 16, 14336, 4096, O.ACT_NONE, 0.0, "mul", 0.0, 0.02, threads),
            ("C5 (one batch of 8)", O.BF16, 2048, 13824, 5120, O.ACT_SWISH, 1.0, None, 0.02, 0.014, threads)):
        rate, r, t, reps = cpu_rate(np, O, dtp, m, n, k, act, alpha, thr, share, resid, bs, ws)
        e = {"config": name, "TFLOP/s": round(rate, 6), "threads": thr, "rows": r, "of_rows": m,
             "seconds_per_run": round(t, 4), "runs": reps}
        if resid == "mul":  # decode: the bandwidth metric (bf16 weight, X, M2 and Y bytes of the sampled rows)
            e["GB/s"] = round(2.0 * (n * k + r * k + 2 * r * n) / t / 1e9, 3)
        per.append(e)
    return {"value": tflops, "unit": "TFLOP/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "cflags": O.build_flags(),
            "sample": f"{rows} of {M} rows of C3 (bf16 Linear+GELU_tanh+residual, K={Kd}, N={N}); naive f32-accumulate "
                      f"loop of the reference gtest oracle, OpenMP over rows, {dt:.1f} s; the aarch64 SVE/KML path "
                      f"cannot build on this x86 host",
            "seconds": dt, "per_config": per,
            "per_config_note": "the same loop on a row sample of each configuration (C4: whole problem, times the "
                               "multiplier M2; C5: one batch, weight read as [N][K])"}


def _time_calls(fn, steps, warmup, torch, prewarm_ms=30.0):
    """Microseconds per call of fn() over `steps` back-to-back calls, after `prewarm_ms` of wall time and `warmup`
    calls untimed (the first configuration of a shape otherwise pays for the clock ramp and first touches)."""
    t_end = time.perf_counter() + prewarm_ms * 1e-3
    while time.perf_counter() < t_end:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps * 1e3


def _with_env(settings):
    """Sets (name, value) pairs in the environment (value None: unset) and returns the previous values."""
    saved = {}
    for key, val in settings:
        saved[key] = os.environ.get(key)
        if val is None:
            os.environ.pop(key, None)
        else:
            os.environ[key] = val
    return saved


def bench_dispatch(args, torch, K):
    """Every bf16 kernel configuration against the planner's choice over prefill-like shapes (microseconds per call;
    CUDA events around `--steps` back-to-back calls after 30 ms and `--warmup` calls untimed)."""
    configs = [("pingpong", "4", "0", "0"), ("pingpong_split", "4", "1", "0"), ("pingpong_kslices", "4", "0", None),
               ("4wave_256x128", "2", "0", None), ("4wave_128x128", "3", "0", None), ("4wave_256x256", "1", "0", None),
               ("planner", None, None, None)]
    g = torch.Generator(device="cuda").manual_seed(0)
    for M in (256, 512, 1024, 2048, 3072):
        for N, Kd in ((4096, 4096), (11008, 4096), (4096, 11008), (14336, 4096), (4096, 14336), (2048, 2048),
                      (8192, 8192)):
            x = torch.randn(M, Kd, device="cuda", generator=g).to(torch.bfloat16)
            w = (torch.randn(N, Kd, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
            y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
            line = {"M": M, "N": N, "K": Kd}
            for name, cfg, split, slices in configs:
                saved = _with_env((("KUDNN_HIP_FORCE_CFG", cfg), ("KUDNN_HIP_FORCE_STREAMK", split),
                                   ("KUDNN_HIP_FORCE_KSLICES", slices)))
                plan = K.LinearPostOps(K.desc([M, Kd], K.BF16), K.desc([Kd, N], K.BF16, "BA"), K.desc([M, N], K.BF16),
                                       None, act=K.ACT_GELU_TANH)
                line[name] = round(_time_calls(lambda: plan.run(x, w, y), args.steps, args.warmup, torch), 1)
                _with_env(saved.items())
                if cfg is None:
                    line["planner_plan"] = plan.describe()
                del plan
            print(json.dumps(line), flush=True)
            del x, w, y


# The reference's perf shape sets: freParas and freParasMulti of test/dnn/llt/gtest/src/matmul_gtest.cpp:550 and :697-705,
# as (M, N, K), run in its Matmul mode (src [M, K], wei [K, N] in layout AB, bias [1, N]).
REF_PERF_SHAPES = [(4096, 3072, 5120), (4096, 32768, 512), (4096, 1536, 5120), (4096, 5120, 1536), (4096, 5120, 3072),
                   (4096, 4096, 1152), (4096, 4608, 1152), (4096, 1152, 3256), (4096, 1152, 4608)]


def bench_refperf(args, torch, K):
    """KuDNN::Gemm on the reference's perf shapes, f32 and bf16, with the weight [K][N] as the reference's Matmul mode
    stores it: the planner's choice and every forced configuration (microseconds per call; CUDA events around
    `--steps` back-to-back calls after 30 ms and `--warmup` calls untimed)."""
    bf16_cfgs = [("ping-pong", "4", "0", "0"), ("ping-pong + K-split", "4", "1", "0"), ("ping-pong + K slices", "4", "0", None),
                 ("4-wave 256x128", "2", "0", None), ("4-wave 128x128", "3", "0", None), ("4-wave 256x256", "1", "0", None)]
    f32_cfgs = [("128x128", "10", None, None), ("64x64", "11", None, None)]
    g = torch.Generator(device="cuda").manual_seed(0)
    out = []
    for M, N, Kd in REF_PERF_SHAPES:
        for name, kdt, tdt, peak, cfgs in (("f32", K.F32, torch.float32, PEAK_F32_TFLOPS, f32_cfgs),
                                            ("bf16", K.BF16, torch.bfloat16, PEAK_BF16_TFLOPS, bf16_cfgs)):
            x = torch.randn(M, Kd, device="cuda", generator=g).to(tdt)
            w = (torch.randn(Kd, N, device="cuda", generator=g) * 0.02).to(tdt)
            b = (torch.randn(1, N, device="cuda", generator=g) * 0.02).to(tdt)
            y = torch.empty(M, N, device="cuda", dtype=tdt)
            line = {"M": M, "N": N, "K": Kd, "dtype": name}
            for cname, cfg, split, slices in [("planner", None, None, None)] + cfgs:
                saved = _with_env((("KUDNN_HIP_FORCE_CFG", cfg), ("KUDNN_HIP_FORCE_STREAMK", split),
                                   ("KUDNN_HIP_FORCE_KSLICES", slices)))
                plan = K.Gemm(K.desc([M, Kd], kdt), K.desc([Kd, N], kdt), K.desc([M, N], kdt), K.desc([1, N], kdt))
                us = _time_calls(lambda: plan.run(x, w, y, b), args.steps, args.warmup, torch)
                _with_env(saved.items())
                if cname == "planner":
                    tf = 2.0 * M * N * Kd / (us * 1e-6) / 1e12
                    line.update({"us": round(us, 1), "TFLOP/s": round(tf, 1), "frac_peak": round(tf / peak, 3),
                                 "plan": plan.describe()})
                else:
                    line[cname] = round(us, 1)
                del plan
            out.append(line)
            print(json.dumps(line), flush=True)
            del x, w, b, y
    return out


# f32 grids of 256 to 640 tiles of 128 x 128 (and two larger), weight [N][K]: where the 128 x 128 and 64 x 64 kernels
# trade places (the planner's f32 rule)
F32_TILE_SHAPES = [(2048, 2048, 4096), (2304, 2048, 2048), (2048, 2560, 2048), (2048, 3072, 4096), (1536, 4096, 2048),
                   (2560, 2560, 2048), (2048, 3584, 2048), (3072, 2560, 1024), (4096, 2304, 2048), (3072, 3072, 2048),
                   (2560, 4096, 2048), (4096, 1152, 4096), (4096, 1536, 5120), (2048, 4096, 4096)]


def bench_dispatch_f32(args, torch, K):
    """f32 Gemm under the 128 x 128 and 64 x 64 configurations and the planner's choice (microseconds per call)."""
    g = torch.Generator(device="cuda").manual_seed(0)
    for M, N, Kd in F32_TILE_SHAPES:
        x = torch.randn(M, Kd, device="cuda", generator=g)
        w = torch.randn(N, Kd, device="cuda", generator=g) * 0.02
        b = torch.randn(1, N, device="cuda", generator=g) * 0.02
        y = torch.empty(M, N, device="cuda")
        line = {"M": M, "N": N, "K": Kd, "tiles_128x128": ((M + 127) // 128) * ((N + 127) // 128)}
        for cname, cfg in (("128x128", "10"), ("64x64", "11"), ("planner", None)):
            saved = _with_env((("KUDNN_HIP_FORCE_CFG", cfg),))
            plan = K.Gemm(K.desc([M, Kd], K.F32), K.desc([Kd, N], K.F32, "BA"), K.desc([M, N], K.F32),
                          K.desc([1, N], K.F32))
            line[cname] = round(_time_calls(lambda: plan.run(x, w, y, b), args.steps, args.warmup, torch), 1)
            _with_env(saved.items())
            if cfg is None:
                line["planner_plan"] = plan.describe()
            del plan
        print(json.dumps(line), flush=True)
        del x, w, b, y


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is a design note "
                                   "(N-split of the weight), not an implemented path", "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch

    import kudnn_amd as K

    K.lib()  # no fallback: fail if the HIP library is missing
    if args.summarize_traffic:
        summarize_traffic(args.summarize_traffic)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters, args.counter_kernel or C3_KERNEL)
        return
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)

    if args.only == "copy":
        n = 256 << 20  # bf16 elements: 512 MiB read + 512 MiB written per launch
        x = torch.ones(n, device="cuda", dtype=torch.bfloat16)
        y = torch.empty_like(x)
        stream = torch.cuda.current_stream()
        ms, _ = time_launches(lambda i=0: torch.neg(x, out=y), args.steps, args.warmup, torch, stream, 0.0)
        print(json.dumps({"kernel": "copy-like elementwise (torch.neg, bf16)", "bytes_read": 2 * n,
                          "bytes_written": 2 * n, "ms": round(ms, 4), "GB/s": round(4 * n / (ms * 1e-3) / 1e9, 1)}))
        return

    if args.only == "dispatch":
        bench_dispatch(args, torch, K)
        bench_dispatch_f32(args, torch, K)
        return

    if args.only == "refperf":
        bench_refperf(args, torch, K)
        return

    if args.only == "torch":
        bench_torch_c3(args, torch)
        bench_torch_others(args, torch)
        return

    if args.only == "c1":
        d = bench_config(args, torch, K, "C1")
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}))
        return

    if args.only == "decode-sweep":
        # the decode step (Linear then element-wise multiply, K = 4096) over M and N, under the planner's choice or
        # the configuration KUDNN_HIP_FORCE_CFG names: the measurements the skinny dispatch rule is drawn from
        for m in (int(v) for v in args.sweep_m.split(",")):
            for n in (int(v) for v in args.sweep_n.split(",")):
                d = bench_decode(args, torch, K, n, m)
                print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}), flush=True)
        return

    if args.only == "decode":
        decode = [bench_decode(args, torch, K, n, m) for n in (4096, 14336) for m in (1, 4, 16)]
        print(json.dumps({"decode": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}
                                     for d in decode]}))
        return

    c3 = bench_c3(args, torch, K)
    only = args.only == "c3"
    decode = [] if (args.no_decode or only) else [bench_decode(args, torch, K, n, m) for n in (4096, 14336)
                                                  for m in (1, 4, 16)]
    others = [] if (args.no_others or only) else ([bench_config(args, torch, K, c) for c in ("C1", "C2", "C5")] +
                                                   [bench_c3_dtype(args, torch, K, c) for c in ("C3-f16", "C3-s8")])
    cpu = None if (args.no_cpu_baseline or only) else cpu_baseline(args, np)

    # the calibrated counter bytes of the C3 kernel, reported only when they were captured from a library built from
    # the same kernel sources as the one benched (the digest compiled into libkudnn_hip.so)
    traffic, traffic_note = None, "no counter capture (profiles/traffic_c3.json) for this build"
    tf = ROOT / "profiles" / "traffic_c3.json"
    built = K.lib().kudnn_pingpong_source_digest().decode()
    if tf.exists():
        try:
            rec = json.loads(tf.read_text())
            if rec.get("source_digest") == built:
                traffic, traffic_note = rec.get("hbm_bytes_per_launch"), f"captured from kernel sources {built}"
            else:
                traffic_note = (f"profiles/traffic_c3.json was captured from kernel sources {rec.get('source_digest')}, "
                                f"the library was built from {built}")
        except Exception as e:
            traffic_note = f"profiles/traffic_c3.json unreadable: {e}"

    out = {
        "metric": METRIC,
        "value": round(c3["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_ms": args.prewarm_ms,
        "ms_per_step": round(c3["ms_wall"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: SplitMix64 seed 0 + stream offset (X 0, W 1, R 3), Box-Muller normals, RNE to bf16; "
                "X~N(0,1), W~N(0,0.02), R~N(0,1), zero bias",
        "config": {"workload": "C3 bf16 Linear+GELU_tanh+residual add", "M": 4096, "K": 4096, "N": 11008,
                   "weight_layout": "BA ([N][K], nn.Linear)", "plan": c3["plan"]},
        "roofline": {"bound": "mfma", "achieved": round(c3["tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(c3["tflops"] / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "traffic_note": traffic_note,
                     "kernel_ms": round(c3["ms"], 4), "alg_flops": c3["flops"], "alg_bytes": c3["alg_bytes"]},
        "cpu_baseline": cpu,
        "decode": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()} for d in decode],
        "other_configs": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()} for d in others],
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark of the cooperative-matrix path on one MI355X.

Headline metric: the bf16 GEMM at M=N=K=8192 (A row-major,
B column-major, fp32 C) -- `value` is its TFLOP/s -- and the causal
flash-attention forward at B=4, H=32, S=4096, D=128 (fp16), reported beside it
in the same JSON line with its own roofline.  Inputs are the seeded synthetic
tensors of the parity tests, generated on the device and resident in HBM
before timing starts.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
                  [--workload headline|gemm_bf16|attn|gemm_i8|w8a16|gemm_f16_256|gemm_bf16_4096|gemm_ex_bf16|vendor_bf16|
                              gemm_bf16_ragged|gemm_cm2_f16|gemm_bf16_nn|gemm_shapes|attn_d64|attn_d96|attn_d256|w8a16_wrow|w8a16_julia|copy|
                              hbm_read|gemm_u8|mfma_loop|gemm_bf16_pad64|w8a16_m64|gemm_mid]

A step is one kernel launch over the whole problem (for the W8A16 and 256^3
workloads, whose kernels take microseconds, 10 back-to-back launches:
`launches_per_step`).  Kernel time is the median over the K steps of the
per-launch time that HIP events recorded on the launch stream give (`kernel_ms`;
the mean is `kernel_ms_mean`); wall time comes from a synchronised host clock
around the same region.  `vendor_bf16` times the vendor library (hipBLASLt,
through torch) on the headline product, for comparison only.

Clock settling: an idle MI355X holds a low engine clock (rocm-smi shows sclk at
114-811 MHz) and needs about half a second of sustained load to reach its
steady loaded clock (~1.9 GHz under these kernels).  So that the K steps are not
timed during that ramp, each workload first runs untimed for --settle seconds
(default 1.0, reported as `clock_settle_s`), then the W warmup steps, then the
K timed steps.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "lava.jl_amd"))

METRIC = "GEMM TFLOP/s at 8192³ bf16 + causal attn fwd TFLOP/s; % of MFMA peak"

# MI355X published dense peaks
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP16_TFLOPS = 2516.6
PEAK_INT8_TOPS = 5033.2
PEAK_HBM_GBS = 8000.0


def timed(lh, launch, steps: int, warmup: int, stream, group: int = 1):
    """Settle the clock, warm up, then time exactly `steps` steps of `group` back-to-back
    launches each.  The workload runs untimed for SETTLE_S[0] seconds first (the engine
    clock's ramp from idle).  An event recorded on `stream` after every step splits the
    region into per-step kernel times; the median of (step time / group) is the kernel time
    per launch (the mean is returned beside it).  group > 1 is for kernels of a few tens of
    microseconds, whose time per launch an event after every launch would inflate by the
    event's own cost.  A synchronised host clock around the same region gives the wall
    time per launch."""
    t_end = time.perf_counter() + SETTLE_S[0]
    while time.perf_counter() < t_end:
        for _ in range(4):
            launch()
        lh.synchronize()
    for _ in range(warmup * group):
        launch()
    lh.synchronize()
    ev = [lh.Event() for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(steps):
        for _ in range(group):
            launch()
        ev[i + 1].record(stream)
    lh.synchronize()
    wall = time.perf_counter() - t0
    per = [ev[i].elapsed_ms(ev[i + 1]) / group for i in range(steps)]
    TIMED_MEAN_MS[0] = sum(per) / steps
    return statistics.median(per), wall * 1e3 / (steps * group)


# mean of the per-launch kernel times of the last timed() call (reported beside the median)
TIMED_MEAN_MS = [0.0]
# the two operand arrays of the last GEMM or attention workload (for the MFMA-loop ceiling)
LAST_INPUTS = []
# seconds of untimed load before each workload's warmup (--settle)
SETTLE_S = [1.0]
# launches per timed step for the kernels of a few tens of microseconds (W8A16, the 256^3 GEMM)
SHORT_GROUP = 10
# (M, N, K, B row-major) of the gemm_shapes workload
GEMM_SHAPES = [(8192, 8192, 8192, False), (4096, 4096, 4096, False), (2048, 2048, 2048, False),
               (1024, 1024, 1024, False), (8192, 14336, 4096, False), (8192, 4096, 14336, False),
               (8192, 12288, 4096, False), (8192, 4096, 4096, False), (5000, 3000, 2000, False),
               (16384, 16384, 2048, False), (256, 4096, 4096, False), (64, 14336, 4096, False),
               (2048, 4096, 4096, False), (1536, 1536, 8192, False), (128, 28672, 8192, False),
               (2048, 2048, 8192, False), (8192, 14336, 4096, True), (4096, 4096, 4096, True),
               (512, 512, 4096, False), (1024, 1024, 8192, False)]


def load_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), committed under profiles/."""
    p = REPO / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(name, {}).get("bytes_per_launch")
    except Exception:
        return None


def roofline(bound, achieved, peak, unit, traffic):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# lava_hip_mfma_loop forms: (id, depth K of one MFMA, name)
MFMA_FORMS = {"f16_16x16x32": (0, 32), "bf16_16x16x32": (1, 32), "i8_16x16x64": (2, 64),
              "f16_32x32x16": (3, 16), "bf16_32x32x16": (4, 16), "i8_32x32x32": (5, 32)}


def mfma_loop_rate(lh, form, a, b, waves, stream, iters=4096, steps=5, warmup=2):
    """T(FL)OP/s of a loop of MFMAs of `form` with no memory access, its operands read once from
    the device arrays a and b (the workload's own inputs), 256 workgroups (one per CU) of
    `waves` waves per SIMD: what the matrix cores sustain on that data at the clock the power
    budget allows."""
    op, depth = MFMA_FORMS[form]
    nbytes = min(a.nbytes, b.nbytes) // 16 * 16
    sink = lh.HIPDeviceArray("f32", (256 * 256 * waves,))
    kms, _ = timed(lh, lambda: lh._lib.call("lava_hip_mfma_loop", op, a.ptr, b.ptr, nbytes, 256, waves, iters,
                                            sink.ptr, stream), steps, warmup, stream)
    return 256 * 4 * waves * iters * 8192.0 * depth / (kms * 1e-3) / 1e12


def with_loop_ceiling(roof, rate, what):
    """Adds the MFMA-loop ceiling (mfma_loop_rate) beside the published peak of a roofline."""
    roof["loop_ceiling"] = {"value": round(rate, 1), "frac": round(roof["achieved"] / rate, 4), "what": what}
    return roof


# ---------------------------------------------------------------- workloads
def bench_gemm(lh, dt, n, steps, warmup, stream, cfg, shape=None):
    M, N, Kd = shape if shape is not None else (n, n, n)
    A = lh.HIPDeviceArray(dt, (M, Kd), order="C")
    B = lh.HIPDeviceArray(dt, (Kd, N), order="F")
    acc = "i32" if dt == "i8" else "f32"
    C = lh.HIPDeviceArray(acc, (M, N), order="C")
    if dt == "i8":
        lh.fill_i8(A, lh.seed(cfg, 0))
        lh.fill_i8(B, lh.seed(cfg, 1))
    else:
        lh.fill_uniform(A, lh.seed(cfg, 0), -1.0, 1.0)
        lh.fill_uniform(B, lh.seed(cfg, 1), -1.0, 1.0)
    lh.synchronize()
    kern_ms, wall_ms = timed(lh, lambda: lh.gemm(C, A, B, stream=stream), steps, warmup, stream)
    flop = 2.0 * M * N * Kd
    LAST_INPUTS[:] = [A, B]
    return flop, kern_ms, wall_ms


def bench_gemm_ex(lh, n, steps, warmup, stream, cfg):
    """The fused epilogue at the headline shape: D (bf16) = gelu_tanh(A*B + bias + residual),
    bias one fp32 value per row, residual fp32 M x N."""
    A = lh.HIPDeviceArray("bf16", (n, n), order="C")
    B = lh.HIPDeviceArray("bf16", (n, n), order="F")
    D = lh.HIPDeviceArray("bf16", (n, n), order="C")
    bias = lh.HIPDeviceArray("f32", (n,))
    res = lh.HIPDeviceArray("f32", (n, n), order="C")
    lh.fill_uniform(A, lh.seed(cfg, 0), -1.0, 1.0)
    lh.fill_uniform(B, lh.seed(cfg, 1), -1.0, 1.0)
    lh.fill_uniform(bias, lh.seed(cfg, 2), -1.0, 1.0)
    lh.fill_uniform(res, lh.seed(cfg, 3), -1.0, 1.0)
    lh.synchronize()
    kern_ms, wall_ms = timed(lh, lambda: lh.gemm_ex(D, A, B, bias=bias, residual=res, act="gelu_tanh",
                                                    stream=stream), steps, warmup, stream)
    return 2.0 * n ** 3, kern_ms, wall_ms


def bench_gemm_cm2(lh, n, steps, warmup, stream, cfg, vocabulary=False):
    """The coopmat2 GEMM: fp16 A, B row-major, fp16 C (the tile kernel, or the
    tensor-vocabulary form)."""
    A = lh.HIPDeviceArray("f16", (n, n), order="C")
    B = lh.HIPDeviceArray("f16", (n, n), order="C")
    Cm = lh.HIPDeviceArray("f16", (n, n), order="C")
    lh.fill_uniform(A, lh.seed(cfg, 0), -1.0, 1.0)
    lh.fill_uniform(B, lh.seed(cfg, 1), -1.0, 1.0)
    lh.synchronize()
    kern_ms, wall_ms = timed(lh, lambda: lh.gemm_cm2(Cm, A, B, vocabulary=vocabulary, stream=stream), steps, warmup, stream)
    return 2.0 * n ** 3, kern_ms, wall_ms


def bench_gemm_layout(lh, dt, n, layout, steps, warmup, stream, cfg, group=1):
    A = lh.HIPDeviceArray(dt, (n, n), order="C" if layout & 1 else "F")
    B = lh.HIPDeviceArray(dt, (n, n), order="C" if layout & 2 else "F")
    C = lh.HIPDeviceArray("f32", (n, n), order="C" if layout & 4 else "F")
    lh.fill_uniform(A, lh.seed(cfg, 0), -1.0, 1.0)
    lh.fill_uniform(B, lh.seed(cfg, 1), -1.0, 1.0)
    lh.synchronize()
    kern_ms, wall_ms = timed(lh, lambda: lh.gemm(C, A, B, stream=stream), steps, warmup, stream, group=group)
    return 2.0 * n ** 3, kern_ms, wall_ms


def bench_attn(lh, steps, warmup, stream, B=4, H=32, S=4096, D=128):
    Q, K, V = (lh.HIPDeviceArray("f16", (D, S, H, B)) for _ in range(3))
    O = lh.HIPDeviceArray("f16", (D, S, H, B))
    for t, a in enumerate((Q, K, V)):
        lh.fill_normal(a, lh.seed(4, t))
    lh.synchronize()
    sc = 1.0 / math.sqrt(D)
    kern_ms, wall_ms = timed(lh, lambda: lh.flash_attn_fwd(O, Q, K, V, scale=sc, causal=True, stream=stream),
                             steps, warmup, stream)
    flop = 0.5 * 4.0 * B * H * S * S * D   # causal: half of 4*B*H*S^2*D
    LAST_INPUTS[:] = [Q, K]
    return flop, kern_ms, wall_ms


def bench_w8a16(lh, steps, warmup, stream, M=16, N=14336, K=4096, copies=6, x_order="C", w_order="F",
                y_order="C"):
    """Rotates `copies` weight/scale sets (> the 256 MB Infinity Cache) so that
    every launch streams its weights from HBM.  Orders: "C" row-major, "F" column-major
    (W "F": K contiguous per output column)."""
    X = lh.HIPDeviceArray("f16", (M, K), order=x_order)
    lh.fill_normal(X, lh.seed(3, 0))
    Ws, Ss = [], []
    for c in range(copies):
        W = lh.HIPDeviceArray("i8", (K, N), order=w_order)
        s = lh.HIPDeviceArray("f16", (N,))
        lh.fill_i8(W, lh.seed(3, 1) + 1000 * c, symmetric=True)
        lh.fill_uniform(s, lh.seed(3, 2) + 1000 * c, 0.001, 0.02)
        Ws.append(W)
        Ss.append(s)
    Y = lh.HIPDeviceArray("f32", (M, N), order=y_order)
    lh.synchronize()
    state = {"i": 0}

    def launch():
        i = state["i"] % copies
        state["i"] += 1
        lh.w8a16(Y, X, Ws[i], Ss[i], stream=stream)

    kern_ms, wall_ms = timed(lh, launch, steps, warmup, stream, group=SHORT_GROUP)
    nbytes = K * N + 2 * N + 2 * M * K + 4 * M * N
    return nbytes, kern_ms, wall_ms


# W8A16 workloads: (X, W, Y orders, description, traffic.json key).  The headline follows the
# GEMM configs' operand convention (A row-major, B column-major: both K-contiguous).
W8A16_WORKLOADS = {
    "w8a16": ("C", "F", "C", "X row-major, W column-major (K-contiguous operands), Y row-major", "w8a16"),
    "w8a16_wrow": ("C", "C", "C", "X, W and Y row-major (N-contiguous weights)", "w8a16_wrow"),
    "w8a16_julia": ("F", "F", "F", "X, W and Y column-major (Julia's default layout)", None),
}


def bench_vendor_bf16(steps, warmup, n=8192):
    """The vendor library on the headline product, for the counter comparison: hipBLASLt
    through torch.mm(A, B, out_dtype=float32), A row-major, B column-major (the transposed
    view of a row-major B^T), bf16 inputs, fp32 C."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(1)
    A = (torch.rand(n, n, device="cuda", generator=g) * 2 - 1).to(torch.bfloat16)
    Bt = (torch.rand(n, n, device="cuda", generator=g) * 2 - 1).to(torch.bfloat16)
    B = Bt.t()
    C = torch.empty(n, n, device="cuda", dtype=torch.float32)

    def launch():
        torch.mm(A, B, out_dtype=torch.float32, out=C)

    t_end = time.perf_counter() + SETTLE_S[0]
    while time.perf_counter() < t_end:
        launch()
        torch.cuda.synchronize()
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        launch()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    TIMED_MEAN_MS[0] = sum(per) / steps
    return 2.0 * n ** 3, statistics.median(per)


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline_gemm(n=8192, budget_s=20.0):
    """The oracle's fp32-accumulate GEMM (a port of the tile loop, not the Lava
    path: Julia/Mantle/lavapipe are not on the GPU box) on all host threads, over
    as many rows of the same 8192^3 bf16 problem as fit the time budget (all of
    them on a 16-core host)."""
    sys.path.insert(0, str(REPO))
    from oracle import oracle as o
    max_rows = n
    A = o.fill_uniform(max_rows * n, "bf16", 0x4C415641 + 256, -1.0, 1.0)   # the first rows of A
    B = o.fill_uniform(n * n, "bf16", 0x4C415641 + 257, -1.0, 1.0)    # B column-major, n x n
    t0 = time.perf_counter()
    o.gemm_f32acc(A, "bf16", B, "bf16", n, n, n, n, 1, 0)          # decoding B alone
    t_decode = time.perf_counter() - t0
    t0 = time.perf_counter()
    o.gemm_f32acc(A, "bf16", B, "bf16", n, n, n, n, 1, 64)
    per_row = max(time.perf_counter() - t0 - t_decode, 1e-4) / 64
    rows = int(max(16, min(max_rows, (budget_s - t_decode) / per_row)))
    t0 = time.perf_counter()
    o.gemm_f32acc(A, "bf16", B, "bf16", n, n, n, n, 1, rows)
    dt = time.perf_counter() - t0
    tflops = 2.0 * rows * n * n / dt / 1e12
    return {"value": round(tflops, 5), "unit": "TFLOP/s", "cores": o.num_threads(), "kind": "port",
            "note": CPU_NOTE,
            "sample": f"{rows} rows of C of the bf16 8192^3 GEMM (2*{rows}*8192*8192 FLOP, fp32 accumulate, "
                      f"includes decoding B), oracle/lava_oracle.c oracle_gemm_f32acc, {dt:.1f} s"}


# what the CPU figures are: the reference's own CPU path (Lava on lavapipe) cannot run on the box
CPU_NOTE = ("lavapipe baseline unavailable (no Julia, Mantle or Lavapipe_jll on the GPU box); not the Lava path: "
            "the build's own CPU restatement (oracle/lava_oracle.c, OpenMP over all host threads)")


def cpu_baseline_attn(B=4, H=32, S=4096, D=128, budget_s=10.0):
    """The oracle's causal attention (fp64 softmax(q K^T s) V per query row, a restatement, not the
    Lava path) on all host threads, over as many heads of the headline problem as fit the time
    budget (at least one), all S query rows of each.  FLOP by the GPU figure's convention: a
    head is 0.5 * 4 * S^2 * D."""
    sys.path.insert(0, str(REPO))
    import numpy as np
    from oracle import oracle as o
    n = D * S
    st = (1, D, D * S, D * S * H)
    rows = np.arange(S)
    heads, dt = 0, 0.0
    while heads == 0 or (dt / heads) * (heads + 1) <= budget_s:
        h = heads % H
        q, k, v = (o.fill_normal(n, "f16", 0x4C415641 + 4 * 256 + t + 16 * h) for t in range(3))
        t0 = time.perf_counter()
        o.attn_rows(q, k, v, S, D, (1, D, D * S, D * S), 1.0 / math.sqrt(D), True, 0, 0, rows)
        dt += time.perf_counter() - t0
        heads += 1
        if heads >= B * H:
            break
    flop = heads * 0.5 * 4.0 * S * S * D
    return {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": o.num_threads(), "kind": "port",
            "note": CPU_NOTE,
            "sample": f"{heads} head(s) of the causal B=4 H=32 S=4096 D=128 problem, all {S} query rows each "
                      f"({flop:.3g} FLOP by the 0.5*4*S^2*D convention; fp64 arithmetic), "
                      f"oracle/lava_oracle.c oracle_attn_rows, {dt:.1f} s"}


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="headline",
                    choices=["headline", "gemm_bf16", "attn", "gemm_i8", "w8a16", "gemm_f16_256", "gemm_bf16_4096",
                             "gemm_ex_bf16", "gemm_bf16_ragged", "gemm_cm2_f16", "gemm_bf16_nn", "attn_d64", "attn_d96", "attn_d256",
                             "copy", "hbm_read", "vendor_bf16", "w8a16_wrow", "w8a16_julia", "gemm_shapes", "gemm_u8",
                             "mfma_loop", "gemm_bf16_pad64", "w8a16_m64", "gemm_mid"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--settle", type=float, default=1.0,
                    help="seconds of untimed load before the warmup, for the clock to leave its idle state")
    args = ap.parse_args()
    SETTLE_S[0] = max(0.0, args.settle)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the cooperative-matrix path has no multi-GPU form in this build "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE={world}). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    K, W = args.steps, args.warmup
    out = {"metric": METRIC, "n_gpus": 1, "steps": K, "warmup": W, "clock_settle_s": SETTLE_S[0],
           "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "data": "synthetic (seeded: uniform[-1,1] GEMM inputs, normal(0,1) Q/K/V), "
                                         "generated on the device before timing"}
    if args.workload == "vendor_bf16":
        # torch brings its own HIP runtime: it runs in a process that has not loaded liblava_hip.so
        flop, kms = bench_vendor_bf16(K, W)
        out.update({"value": round(flop / (kms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(kms, 4),
                    "dtype": "bf16", "config": {"workload": "vendor reference: hipBLASLt (torch.mm, out_dtype fp32) on "
                                                            "the headline product, bf16 8192^3, A row-major, B column-major"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
        print(json.dumps(out), flush=True)
        return

    import lava_hip as lh
    lh.init()
    s = lh.Stream()
    stream = s.handle

    if args.workload in ("headline", "gemm_bf16"):
        flop, kms, wms = bench_gemm(lh, "bf16", 8192, K, W, stream, 1)
        gemm_mean = TIMED_MEAN_MS[0]
        achieved = flop / (kms * 1e-3) / 1e12
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16",
                    "config": {"workload": "bf16 GEMM M=N=K=8192, A row-major, B column-major, fp32 accumulate "
                                           "and output (BASELINE configs[1])", "M": 8192, "N": 8192, "K": 8192},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(gemm_mean, 4),
                    "roofline": roofline("mfma", achieved, PEAK_BF16_TFLOPS, "TFLOP/s", load_traffic("gemm_bf16_8192"))})
        with_loop_ceiling(out["roofline"], mfma_loop_rate(lh, "bf16_16x16x32", *LAST_INPUTS, 1, stream),
                          "bf16 16x16x32 MFMAs alone on the GEMM's A and B, 1 wave per SIMD as in the kernel")
        if args.workload == "headline":
            aflop, akms, awms = bench_attn(lh, K, W, stream)
            a_ach = aflop / (akms * 1e-3) / 1e12
            out["attn_fwd"] = {"value": round(aflop / (awms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                               "ms_per_step": round(awms, 4), "kernel_ms": round(akms, 4),
                               "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4), "dtype": "f16",
                               "config": {"workload": "causal flash-attention forward B=4 H=32 S=4096 D=128 fp16, "
                                                      "fp32 softmax state (BASELINE configs[4]); FLOP = "
                                                      "0.5*4*B*H*S^2*D"},
                               "roofline": with_loop_ceiling(
                                   roofline("mfma", a_ach, PEAK_FP16_TFLOPS, "TFLOP/s", load_traffic("flash_fwd_causal")),
                                   mfma_loop_rate(lh, "f16_32x32x16", *LAST_INPUTS, 2, stream),
                                   "f16 32x32x16 MFMAs alone on the attention's Q and K, 2 waves per SIMD as in "
                                   "the kernel")}
    elif args.workload == "gemm_bf16_4096":
        flop, kms, wms = bench_gemm(lh, "bf16", 4096, K, W, stream, 1)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16", "config": {"workload": "bf16 GEMM 4096^3 A row-major B column-major"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_mid":
        # a mid-size product: 256 tiles of 128 x 128 (64 of 256 x 256), the 128 x 128 kernel's share
        flop, kms, wms = bench_gemm(lh, "bf16", 0, K, W, stream, 1, shape=(2048, 4096, 4096))
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16", "config": {"workload": "bf16 GEMM M=2048 N=4096 K=4096, A row-major, B "
                                                            "column-major (the mid-size kernel)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_bf16_ragged":
        flop, kms, wms = bench_gemm(lh, "bf16", 0, K, W, stream, 1, shape=(8000, 8000, 8000))
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16", "config": {"workload": "bf16 GEMM M=N=K=8000 (not a tile multiple: "
                                                            "zero-clamped loads, bounds-checked store)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_bf16_pad64":
        # the headline product with A's and B's rows 8192 + 64 elements apart (not 16 KiB): the
        # L2-set aliasing check for the tile kernel's LDS-DMA row pattern
        n, ld = 8192, 8192 + 64
        A = lh.HIPDeviceArray("bf16", (n, ld), order="C")
        B = lh.HIPDeviceArray("bf16", (ld, n), order="F")
        C = lh.HIPDeviceArray("f32", (n, n), order="C")
        lh.fill_uniform(A, lh.seed(1, 0), -1.0, 1.0)
        lh.fill_uniform(B, lh.seed(1, 1), -1.0, 1.0)
        lh.synchronize()
        kms, wms = timed(lh, lambda: lh.gemm_raw("bf16", "f32", A.ptr, B.ptr, C.ptr, n, n, n, ld, ld, n, 1 | 4, stream),
                         K, W, stream)
        flop = 2.0 * n ** 3
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16", "config": {"workload": "bf16 GEMM 8192^3 as the headline, lda = ldb = 8256"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_shapes":
        # bf16 products off the square configs: language-model projections (8192 tokens), a
        # ragged non-square product, few-row (decode-like) products; A row-major, B column-major
        # (K-contiguous, the headline convention) and, for two shapes, B row-major
        rows = []
        for (M, N, Kd, brow) in GEMM_SHAPES:
            if brow:
                A = lh.HIPDeviceArray("bf16", (M, Kd), order="C")
                B = lh.HIPDeviceArray("bf16", (Kd, N), order="C")
                C = lh.HIPDeviceArray("f32", (M, N), order="C")
                lh.fill_uniform(A, lh.seed(1, 0), -1.0, 1.0)
                lh.fill_uniform(B, lh.seed(1, 1), -1.0, 1.0)
                lh.synchronize()
                kms, _ = timed(lh, lambda: lh.gemm(C, A, B, stream=stream), K, W, stream)
                flop = 2.0 * M * N * Kd
                del A, B, C
            else:
                flop, kms, _ = bench_gemm(lh, "bf16", 0, K, W, stream, 1, shape=(M, N, Kd))
            t = flop / (kms * 1e-3) / 1e12
            rows.append({"M": M, "N": N, "K": Kd, "B": "row" if brow else "col", "kernel_ms": round(kms, 4),
                         "TFLOP/s": round(t, 1), "frac": round(t / PEAK_BF16_TFLOPS, 3)})
        gm = math.exp(sum(math.log(r["TFLOP/s"]) for r in rows) / len(rows))
        out.update({"value": round(gm, 2), "unit": "TFLOP/s", "ms_per_step": None, "dtype": "bf16",
                    "config": {"workload": "bf16 GEMM over a list of shapes (geometric mean of the per-shape "
                                           "kernel TFLOP/s), fp32 C row-major, A row-major", "shapes": rows},
                    "roofline": roofline("mfma", gm, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "attn_d64":
        flop, kms, wms = bench_attn(lh, K, W, stream, D=64)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "f16", "config": {"workload": "causal flash-attention forward B=4 H=32 S=4096 D=64"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "attn_d96":
        flop, kms, wms = bench_attn(lh, K, W, stream, D=96)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "f16", "config": {"workload": "causal flash-attention forward B=4 H=32 S=4096 D=96 "
                                                           "(score/output kernel, rows staged 128 wide, MFMAs over 96 columns; FLOP at D=96)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "attn_d256":
        flop, kms, wms = bench_attn(lh, K, W, stream, D=256)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "f16", "config": {"workload": "causal flash-attention forward B=4 H=32 S=4096 D=256 "
                                                           "(two launches per call, one per half of V and O; FLOP at D=256)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_bf16_nn":
        flop, kms, wms = bench_gemm_layout(lh, "bf16", 8192, 1 | 2 | 4, K, W, stream, 1)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16", "config": {"workload": "bf16 GEMM 8192^3, A and B row-major (B read through "
                                                            "transposing LDS reads)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_cm2_f16":
        flop, kms, wms = bench_gemm_cm2(lh, 4096, K, W, stream, 1)
        tile_mean = TIMED_MEAN_MS[0]
        _, vkms, _ = bench_gemm_cm2(lh, 4096, K, W, stream, 1, vocabulary=True)
        TIMED_MEAN_MS[0] = tile_mean
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "f16", "config": {"workload": "coopmat2 GEMM 4096^3 fp16 -> fp16, A and B row-major"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "vocabulary_form_tflops": round(flop / (vkms * 1e-3) / 1e12, 2),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_ex_bf16":
        flop, kms, wms = bench_gemm_ex(lh, 8192, K, W, stream, 1)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "bf16", "config": {"workload": "bf16 GEMM 8192^3 with the fused epilogue: D bf16 = "
                                                            "gelu_tanh(A*B + bias[row] + residual), bias and residual fp32"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "attn":
        flop, kms, wms = bench_attn(lh, K, W, stream)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "f16", "config": {"workload": "causal flash-attention forward B=4 H=32 S=4096 D=128"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s",
                                         load_traffic("flash_fwd_causal"))})
    elif args.workload == "gemm_i8":
        flop, kms, wms = bench_gemm(lh, "i8", 4096, K, W, stream, 2)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "int8", "config": {"workload": "int8 GEMM 4096^3 -> int32 (BASELINE configs[2])"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_INT8_TOPS, "TOP/s",
                                         load_traffic("gemm_i8_4096"))})
    elif args.workload == "gemm_u8":
        n = 4096
        A = lh.HIPDeviceArray("u8", (n, n), order="C")
        B = lh.HIPDeviceArray("u8", (n, n), order="F")
        C = lh.HIPDeviceArray("u32", (n, n), order="C")
        lh.fill_i8(A, lh.seed(2, 0))
        lh.fill_i8(B, lh.seed(2, 1))
        lh.synchronize()
        kms, wms = timed(lh, lambda: lh.gemm(C, A, B, stream=stream), K, W, stream)
        flop = 2.0 * n ** 3
        out.update({"value": round(flop / (kms * 1e-3) / 1e12, 2), "unit": "TOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "u8", "config": {"workload": "uint8 GEMM 4096^3 -> uint32, A row-major, B column-major "
                                                          "(signed MFMA on bytes flipped by 128, row/column-sum "
                                                          "correction)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_INT8_TOPS, "TOP/s", load_traffic("gemm_u8_4096"))})
    elif args.workload in W8A16_WORKLOADS:
        xo, wo, yo, what, traffic_key = W8A16_WORKLOADS[args.workload]
        nbytes, kms, wms = bench_w8a16(lh, K, W, stream, x_order=xo, w_order=wo, y_order=yo)
        out.update({"value": round(nbytes / (wms * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(wms, 5),
                    "dtype": "f16", "launches_per_step": SHORT_GROUP,
                    "config": {"workload": "W8A16 16x4096 . 4096x14336, per-column fp16 scale, "
                                           "6 rotating weight copies (BASELINE configs[3]); " + what},
                    "kernel_ms": round(kms, 5), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 5),
                    "roofline": roofline("hbm", nbytes / (kms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s",
                                         load_traffic(traffic_key) if traffic_key else None)})
    elif args.workload == "w8a16_m64":
        # batched decode: 64 rows of X, W column-major (each workgroup multiplies 4 row blocks with
        # every dequantized weight fragment); past the weight stream the kernel is MFMA / L2 work,
        # so the figure is TFLOP/s, with the HBM rate beside it
        M = 64
        nbytes, kms, wms = bench_w8a16(lh, K, W, stream, M=M, x_order="C", w_order="F", y_order="C")
        flop = 2.0 * M * 4096 * 14336
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(wms, 5),
                    "dtype": "f16", "launches_per_step": SHORT_GROUP,
                    "config": {"workload": "W8A16 64x4096 . 4096x14336 (batched decode), per-column fp16 scale, "
                                           "6 rotating weight copies; X row-major, W column-major, Y row-major"},
                    "kernel_ms": round(kms, 5), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 5),
                    "hbm_GBs": round(nbytes / (kms * 1e-3) / 1e9, 1),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "gemm_f16_256":
        flop, kms, wms = bench_gemm_layout(lh, "f16", 256, 3 | 4, K, W, stream, 0, group=SHORT_GROUP)
        out.update({"value": round(flop / (wms * 1e-3) / 1e12, 3), "unit": "TFLOP/s", "ms_per_step": round(wms, 4),
                    "dtype": "f16", "launches_per_step": SHORT_GROUP, "config": {"workload": "fp16 GEMM 256^3, A and B row-major (BASELINE configs[0])"},
                    "kernel_ms": round(kms, 5), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 5),
                    "roofline": roofline("mfma", flop / (kms * 1e-3) / 1e12, PEAK_FP16_TFLOPS, "TFLOP/s", None)})

    elif args.workload == "hbm_read":
        # the HBM read ceiling: a tuned read-only stream (16-byte nontemporal loads, 8 in flight
        # per thread; the launch shapes a sweep of 4 / 8 / 16 loads in flight and 448 to 16384
        # workgroups found best), over 4 GiB, and over the W8A16 weight size (58.7 MB, 6 rotating
        # copies: 352 MB > the 256 MB MALL)
        nbytes = 1 << 32
        src = lh.HIPDeviceArray("u8", (nbytes,))
        sink = lh.HIPDeviceArray("u32", (8192 * 256,))
        src.fill_bytes(3)
        lh.synchronize()
        kms, wms = timed(lh, lambda: lh._lib.call("lava_hip_read_stream", src.ptr, nbytes, sink.ptr, 8192, 8, stream),
                         K, W, stream)
        del src
        wb = 4096 * 14336
        bufs = [lh.HIPDeviceArray("u8", (wb,)) for _ in range(6)]
        for b_ in bufs:
            b_.fill_bytes(5)
        lh.synchronize()
        it = [0]

        def launch_w():
            lh._lib.call("lava_hip_read_stream", bufs[it[0] % 6].ptr, wb, sink.ptr, 448, 8, stream)
            it[0] += 1

        wms_k, _ = timed(lh, launch_w, K, W, stream, group=SHORT_GROUP)
        out.update({"value": round(nbytes / (kms * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(wms, 4),
                    "dtype": "u8", "config": {"workload": "HBM read stream of 4 GiB (read bytes; 16-byte "
                                                          "nontemporal loads, 8 per thread in flight, 8192 x 256 threads)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "w8a16_size": {"bytes": wb, "copies": 6, "us": round(wms_k * 1e3, 2),
                                   "GBs": round(wb / (wms_k * 1e-3) / 1e9, 1), "launch": "448 x 256 threads"},
                    "roofline": roofline("hbm", nbytes / (kms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s", load_traffic("hbm_read_4g"))})
    elif args.workload == "mfma_loop":
        # the matrix cores alone: MFMA loops with no memory access, on each workload's own data
        # (the GEMM's uniform[-1,1] bf16, the attention's normal(0,1) fp16, the int8 GEMM's bytes)
        # and on constant data (every fp16 operand the same), at 1, 2 and 4 waves per SIMD
        n = 4096
        A = lh.HIPDeviceArray("bf16", (n, n))
        B = lh.HIPDeviceArray("bf16", (n, n))
        lh.fill_uniform(A, lh.seed(1, 0), -1.0, 1.0)
        lh.fill_uniform(B, lh.seed(1, 1), -1.0, 1.0)
        Q = lh.HIPDeviceArray("f16", (n, n))
        Kt = lh.HIPDeviceArray("f16", (n, n))
        lh.fill_normal(Q, lh.seed(4, 0))
        lh.fill_normal(Kt, lh.seed(4, 1))
        Ai = lh.HIPDeviceArray("i8", (n, n))
        Bi = lh.HIPDeviceArray("i8", (n, n))
        lh.fill_i8(Ai, lh.seed(2, 0))
        lh.fill_i8(Bi, lh.seed(2, 1))
        ones = lh.HIPDeviceArray("f16", (n, n))
        ones.fill_bytes(0x3C)   # every operand 0x3C3C = 1.0586
        lh.synchronize()
        rates = {}
        for form, a, b in (("bf16_16x16x32", A, B), ("bf16_32x32x16", A, B), ("f16_16x16x32", Q, Kt),
                           ("f16_32x32x16", Q, Kt), ("i8_16x16x64", Ai, Bi), ("i8_32x32x32", Ai, Bi),
                           ("f16_16x16x32 constant", ones, ones)):
            for waves in (1, 2, 4):
                rates[f"{form}, {waves} wave(s)/SIMD"] = round(
                    mfma_loop_rate(lh, form.split()[0], a, b, waves, stream, steps=K, warmup=W), 1)
        top = rates["bf16_16x16x32, 1 wave(s)/SIMD"]
        out.update({"value": top, "unit": "TFLOP/s", "ms_per_step": None, "dtype": "bf16",
                    "config": {"workload": "MFMA loops without memory access, 256 workgroups (one per CU), "
                                           "4096 rounds; value: bf16 16x16x32 at 1 wave/SIMD on uniform[-1,1]"},
                    "rates": rates, "roofline": roofline("mfma", top, PEAK_BF16_TFLOPS, "TFLOP/s", None)})
    elif args.workload == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain 1 GiB device copy
        nbytes = 1 << 30
        src = lh.HIPDeviceArray("u8", (nbytes,))
        dst = lh.HIPDeviceArray("u8", (nbytes,))
        src.fill_bytes(1)
        lh.synchronize()
        kms, wms = timed(lh, lambda: lh._lib.call("lava_hip_memcpy_d2d", dst.ptr, src.ptr, nbytes, stream), K, W,
                         stream)
        # the device as it reports itself: the dense fp16/bf16 peak re-derived as
        # CUs x max clock x 4096 FLOP per clock per CU, beside the vendor figure
        dp = lh.vocabulary.device_properties()
        out.update({"value": round(2 * nbytes / (kms * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(wms, 4),
                    "dtype": "u8", "config": {"workload": "device copy of 1 GiB (read + write bytes)"},
                    "kernel_ms": round(kms, 4), "kernel_ms_mean": round(TIMED_MEAN_MS[0], 4),
                    "device": {"cus": dp["cores"], "max_clock_mhz": dp["clock_khz"] / 1000.0,
                               "hbm_gib": round(dp["hbm_bytes"] / 2**30, 1), "l2_mib": round(dp["l2_bytes"] / 2**20, 1),
                               "derived_peak_bf16_tflops": round(dp["cores"] * dp["clock_khz"] * 1e3 * 4096 / 1e12, 1),
                               "vendor_peak_bf16_tflops": PEAK_BF16_TFLOPS},
                    "roofline": roofline("hbm", 2 * nbytes / (kms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s", 2 * nbytes)})

    if args.workload in ("headline", "gemm_bf16") and not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_gemm()
    if args.workload in ("headline", "attn") and not args.no_cpu_baseline:
        (out["attn_fwd"] if args.workload == "headline" else out)["cpu_baseline"] = cpu_baseline_attn()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

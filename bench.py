#!/usr/bin/env python3
"""Benchmark of the contract matrix-multiply path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--sections dense,decode,moe]

A step is one pass of the Llama-3.1-8B-shaped MLP contract GEMMs at M=2048 prefill rows:
w8a8_matmul (row quant + exact int8 GEMM + v2.1 epilogue, bf16 out) of the gate+up projection
(N=28672, K=4096) and of the down projection (N=4096, K=14336), synthetic inputs resident in HBM.
`value` is int8 TOPS (2 ops per multiply-accumulate) of the whole step.  One JSON line is printed.

The `roofline` object prices the dominant kernel (the int8 MFMA GEMM) from HIP events recorded on
the stream it is launched on; `cpu_baseline` times the reference's own CPU op sequence
(oracle/cpu_baseline.py) on a bounded row sample on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, 5.0 POPS
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
METRIC = "bit-exact contract GEMM int8 TOPS + MoE tokens/s, 1×MI355X, % of roofline"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _events_time(torch, fn, reps):
    """Average milliseconds of fn() over reps launches, HIP events on the current stream."""
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        fn()
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def dense_section(torch, args):
    from lockstep_amd import _lib as L
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
    from lockstep_amd import workloads as WL

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    M = 2048
    shapes = [("gate_up",) + WL.LLAMA8B["gate_up"], ("down",) + WL.LLAMA8B["down"]]
    data = []
    for name, N, K in shapes:
        x = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
        mask = torch.rand((M, K), generator=g, device=dev) < 0.001
        x = torch.where(mask, 20.0 * torch.sign(torch.randn((M, K), generator=g, device=dev)), x)
        W8 = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        ws = torch.empty(N, device=dev).uniform_(1e-3, 1e-2, generator=g)
        data.append((name, N, K, x, W8, ws))
    ops_step = sum(2 * M * N * K for _, N, K, *_ in data)

    def step():
        for _, N, K, x, W8, ws in data:
            FS.w8a8_matmul(x, W8, ws, out_dtype=torch.bfloat16)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = _events_time(torch, step, args.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    tops = ops_step / (ms * 1e-3) / 1e12

    # dominant kernel alone: the exact GEMM with the fused epilogue on pre-quantised rows
    gemm_ms, gemm_ops = [], []
    for name, N, K, x, W8, ws in data:
        q, asc = ops.rowquant(x)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        fn = lambda: ops.gemm(q, W8, L.EPI_V21, L.LSK_BF16, asc=asc, ws=ws, out=out)  # noqa: E731
        for _ in range(3):
            fn()
        gemm_ms.append(_events_time(torch, fn, max(args.steps, 10)))
        gemm_ops.append(2 * M * N * K)
    achieved = sum(gemm_ops) / (sum(gemm_ms) * 1e-3) / 1e12
    per_shape = {name: {"ms": round(t, 4), "TOPS": round(o / (t * 1e-3) / 1e12, 1)}
                 for (name, *_), t, o in zip(data, gemm_ms, gemm_ops)}
    return {
        "ms_per_step": ms, "value": tops, "wall_s": wall, "ops_step": ops_step,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": None,
                     "kernel": "gemm_i8_mfma_kernel", "per_shape": per_shape,
                     "note": "int8 ops (2 per MAC) per launch / average launch time, HIP events"},
    }


def decode_section(torch, args):
    """Batch-1/8/32 decode rows through w8a8_matmul; weights rotated over > 512 MB of copies so
    the 256 MB Infinity Cache cannot serve them.  GB/s counts the algorithmic bytes
    N*K + 4N + 4MK + 2MN of one call."""
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import workloads as WL

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    res = {}
    for name in ("gate_up", "down"):
        N, K = WL.LLAMA8B[name]
        copies = max(2, int((768 << 20) // (N * K)) + 1)
        Ws = [torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8) for _ in range(copies)]
        ws = torch.empty(N, device=dev).uniform_(1e-3, 1e-2, generator=g)
        for M in (1, 8, 32):
            x = torch.randn((M, K), generator=g, device=dev)
            it = [0]

            def fn():
                FS.w8a8_matmul(x, Ws[it[0] % copies], ws, out_dtype=torch.bfloat16)
                it[0] += 1
            for _ in range(copies):
                fn()
            ms = _events_time(torch, fn, 6 * copies)
            nbytes = N * K + 4 * N + 4 * M * K + 2 * M * N
            gbs = nbytes / (ms * 1e-3) / 1e9
            res["%s_M%d" % (name, M)] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                         "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        del Ws
    return res


def cpu_baseline_dense(args):
    """The reference's CPU op sequence for w8a8_matmul on a row sample of both step shapes."""
    import numpy as np
    import torch

    from lockstep_amd import workloads as WL
    from oracle import cpu_baseline as B

    rows = 64
    g = np.random.Generator(np.random.PCG64(7))
    total_ops, total_t = 0, 0.0
    for name in ("gate_up", "down"):
        N, K = WL.LLAMA8B[name]
        x = torch.from_numpy(g.standard_normal((rows, K), dtype=np.float64).astype(np.float32))
        W8 = torch.from_numpy(g.integers(-127, 128, (N, K), dtype=np.int8))
        ws = torch.from_numpy(g.uniform(1e-3, 1e-2, N).astype(np.float32))
        B.dense_w8a8(x[:17], W8, ws)                  # warm the allocator
        t0 = time.perf_counter()
        B.dense_w8a8(x, W8, ws)
        total_t += time.perf_counter() - t0
        total_ops += 2 * rows * N * K
    return {"value": round(total_ops / total_t / 1e12, 4), "unit": "TOPS", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": "%d of the 2048 rows of both step shapes (gate_up 28672x4096, down 4096x14336); "
                      "rows are independent so TOPS extrapolates linearly; torch CPU op sequence of "
                      "lockstep_fullstack.w8a8_matmul (torch._int_mm, rows padded to 17); host os.cpu_count()=%s"
                      % (rows, os.cpu_count())}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sections", default="dense,decode,moe")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (N=%d requested)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    from lockstep_amd import _lib
    _lib.load()
    sections = set(args.sections.split(","))

    log("bench: dense prefill step (M=2048, gate_up 28672x4096 + down 4096x14336)")
    d = dense_section(torch, args)
    out = {
        "metric": METRIC, "value": round(d["value"], 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(d["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Llama-3.1-8B MLP contract GEMMs, w8a8_matmul v2.1, M=2048 prefill rows",
                   "M": 2048, "gate_up": [28672, 4096], "down": [4096, 14336], "x": "f32 N(0,1), 0.1% +-20",
                   "out": "bf16", "parallelism": "single GPU"},
        "roofline": d["roofline"],
    }
    if "decode" in sections:
        log("bench: decode rows M in {1, 8, 32}")
        out["decode"] = decode_section(torch, args)
    if "moe" in sections:
        try:
            from bench_moe import moe_section
        except ImportError:
            moe_section = None
        if moe_section is not None:
            log("bench: MoE layers")
            out["moe"] = moe_section(torch, args)
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (reference op sequence, row sample)")
        out["cpu_baseline"] = cpu_baseline_dense(args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

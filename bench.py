#!/usr/bin/env python3
"""Benchmark of the contract matrix-multiply path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                    [--sections block,dense,decode,moe[,vendor,copy]] [--block-rows T]
                    [--moe-cases NAME,...] [--eager] [--mx-variant V] [--moe-variant V]

A step (the headline `value`) is one Qwen2.5-7B-shaped decoder block's four GEMMs through
ref_block_v1 at T=8192 prefill rows: per GEMM site quant8_dyn of the binary32 activation, the exact
int8 GEMM and the pow2 dequant (binary32 out); qkv 4608x3584, o 3584x3584, gate+up 37888x3584,
down 3584x18944; synthetic inputs resident in HBM.  `value` is int8 TOPS (2 ops per
multiply-accumulate) of the whole step.  Extra keys: the Llama-3.1-8B MLP step (w8a8_matmul v2.1 at
M=2048), decode rows, the MoE layers and their grouped-GEMM stages.  One JSON line is printed.

The `roofline` object prices the dominant kernel (the int8 MFMA GEMM) from HIP events recorded on
the stream it is launched on; `cpu_baseline` times the reference's own CPU op sequence on a
bounded row sample on this host's cores.
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

    # the Qwen2.5-7B block GEMMs at 8192 rows, the shapes whose H100 times the reference publishes
    # (int8 GEMM with the fused v2.1 epilogue on pre-quantised rows)
    ref_shapes = {}
    Mq = 8192
    aq = torch.randint(-127, 128, (Mq, 18944), generator=g, device=dev, dtype=torch.int8)
    ascq = torch.empty(Mq, device=dev).uniform_(1e-3, 1e-2, generator=g)
    for name, N, K in (("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)):
        a = aq[:, :K]
        W8 = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        ws = torch.empty(N, device=dev).uniform_(1e-3, 1e-2, generator=g)
        out = torch.empty((Mq, N), dtype=torch.bfloat16, device=dev)
        fn = lambda: ops.gemm(a, W8, L.EPI_V21, L.LSK_BF16, asc=ascq, ws=ws, out=out)  # noqa: E731
        for _ in range(3):
            fn()
        t = _events_time(torch, fn, 10)
        ref_shapes["qwen2.5_7b_%s_M8192" % name] = {"us": round(t * 1e3, 1), "TOPS": round(2 * Mq * N * K / (t * 1e-3) / 1e12, 1)}
        del W8, out
    torch.cuda.empty_cache()
    return {
        "ms_per_step": ms, "value": tops, "wall_s": wall, "ops_step": ops_step,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": None,
                     "kernel": "gemm_i8_pp_kernel", "per_shape": per_shape,
                     "note": "int8 ops (2 per MAC) per launch / average launch time, HIP events"},
        "qwen2_5_7b_m8192": dict(ref_shapes, note="int8 GEMM + fused v2.1 epilogue (bf16 out) on pre-quantised "
                                                   "rows, HIP events; the shapes the reference times on H100"),
    }


QWEN25_7B_BLOCK = (("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944))
BLOCK_EW = 7   # quant8_dyn of the float weight W8 / 128 gives back (W8, 7)


def block_section(torch, args):
    """The headline step: one Qwen2.5-7B-shaped decoder block's GEMMs through ref_block_v1 at T=8192
    prefill rows (hidden 3584; qkv 4608 = 28 query + 2 x 4 KV heads of 128; o 3584; gate+up 37888 =
    2 x 18944; down K = 18944).  Each GEMM site (ref_block_v1.py:166-167, 191-193, 196-198, 216-218)
    is ref_block_v1.linear_dyn: quant8_dyn of the binary32 activation (two launches) and the exact
    int8 GEMM with the pow2 dequant fused into its epilogue, binary32 out.  Activations N(0,1) and
    int8 weights uniform on [-127, 127] (exponent 7), resident in HBM.  HIP events recorded on the
    launch stream around every launch of the timed steps give the GEMM kernel's and the quantiser's
    own times."""
    from lockstep_amd import ref_block_v1 as RB

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    T = args.block_rows
    sites = []
    for name, N, K in QWEN25_7B_BLOCK:
        x = torch.randn((T, K), generator=g, device=dev, dtype=torch.float32)
        W8 = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        sites.append((name, N, K, x, W8))
    ops_site = [2 * T * N * K for _, N, K, _, _ in sites]
    ops_step = sum(ops_site)
    s = torch.cuda.current_stream()

    def step(marks=None):
        for i, (_, N, K, x, W8) in enumerate(sites):
            RB.linear_dyn(x, W8.t(), BLOCK_EW)
            if marks is not None:
                marks[i + 1].record(s)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    # events on the launch stream at every site boundary of every timed step (recording an event
    # costs the GPU nothing), so the site split comes from the timed steps themselves
    marks = [[ev() for _ in range(len(sites) + 1)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for k in range(args.steps):
        marks[k][0].record(s)
        step(marks[k])
    marks[-1][-1].synchronize()
    wall = time.perf_counter() - t0
    ms = marks[0][0].elapsed_time(marks[-1][-1]) / args.steps
    site_ms = [sum(mk[i].elapsed_time(mk[i + 1]) for mk in marks) / args.steps for i in range(len(sites))]
    # each site's GEMM alone on its quantised operands (the site's own quant left in its work
    # buffer, in the layout the site's GEMM reads): the dominant kernel's launch time
    gemm_ms = []
    for _, N, K, x, W8 in sites:
        from lockstep_amd import _lib as L
        from lockstep_amd import ops
        work = torch.empty((L.load().lsk_linear_dyn_workspace(T, K),), dtype=torch.uint8, device=dev)
        out = torch.empty((T, N), dtype=torch.float32, device=dev)
        ex = torch.empty((1,), dtype=torch.int32, device=dev)
        wp = RB.row_pairs_of(W8, T)
        ops.linear_dyn(x, W8, BLOCK_EW, stages=1, work=work, y=out, ex=ex, w_pairs=wp)
        fn = lambda: ops.linear_dyn(x, W8, BLOCK_EW, stages=2, work=work, y=out, ex=ex, w_pairs=wp)  # noqa: E731
        for _ in range(2):
            fn()
        gemm_ms.append(_events_time(torch, fn, max(args.steps, 5)))
        del work, out, ex, wp
    achieved = ops_step / (sum(gemm_ms) * 1e-3) / 1e12
    per_site = {name: {"site_us": round(t * 1e3, 1), "gemm_us": round(gk * 1e3, 1),
                       "quant8_dyn_us": round((t - gk) * 1e3, 1), "TOPS": round(o / (t * 1e-3) / 1e12, 1),
                       "gemm_TOPS": round(o / (gk * 1e-3) / 1e12, 1)}
                for (name, *_), t, gk, o in zip(sites, site_ms, gemm_ms, ops_site)}
    del sites
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "value": ops_step / (ms * 1e-3) / 1e12, "wall_s": wall, "ops_step": ops_step,
            "T": T, "per_site": per_site,
            "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": None,
                         "kernel": "gemm_i8_pp_pow2_persist_kernel (row-pair operands, POW2 epilogue, binary32 "
                                   "out) with its 256x128 column tails",
                         "note": "2*T*N*K int8 ops of the four GEMMs / the sum of their average launch times "
                                 "(HIP events on the launch stream, each site's GEMM alone on its quantised "
                                 "operands: lsk_linear_dyn stage 2)"}}


def cpu_baseline_block(args):
    """The reference's own CPU op sequence of one block GEMM site, ref_block_v1.py:122-133 and
    :167 (numpy quant8_dyn, int64 `a @ b`, the pow2 dequant), restated in the oracle, on a row
    sample of each of the four Qwen2.5-7B GEMMs.  numpy's int64 matmul runs on one core."""
    import numpy as np

    from oracle import contract as C

    rows = 6
    g = np.random.Generator(np.random.PCG64(13))
    total_ops, total_t = 0, 0.0
    for name, N, K in QWEN25_7B_BLOCK:
        x = g.standard_normal((rows, K), dtype=np.float32)
        W = g.integers(-127, 128, (K, N), dtype=np.int64)    # the reference's quantised weights are int64
        t0 = time.perf_counter()
        q, e = C.quant8_dyn(x)
        C.dequant_pow2(C.gemm_int(q, W), e + BLOCK_EW)
        total_t += time.perf_counter() - t0
        total_ops += 2 * rows * N * K
    return {"value": round(total_ops / total_t / 1e12, 6), "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": "%d rows of each of the four Qwen2.5-7B block GEMMs (qkv 4608x3584, o 3584x3584, gate_up "
                      "37888x3584, down 3584x18944): numpy quant8_dyn, int64 matmul and pow2 dequant as in "
                      "ref_block_v1.py:122-133,167 (rows are independent, so TOPS extrapolates linearly to T=%d); "
                      "host os.cpu_count()=%s" % (rows, args.block_rows, os.cpu_count())}


def vendor_section(torch, args):
    """Reference points for the dominant kernel on the step shapes (random int8 operands, warm
    part, best of 6 interleaved rounds): hipBLASLt's int8 GEMM through torch._int_mm (int32
    output, W as a column-major operand) and this library's exact GEMM with the bf16 v2.1
    epilogue on forced tiles (1: 256x256, 3: 256x128, 16: four-wave 256x256, 18: 256x128 with
    128-byte K stages)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import ops
    from lockstep_amd import workloads as WL

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    M = 2048
    res = {}
    for name, (N, K) in (("gate_up", WL.LLAMA8B["gate_up"]), ("down", WL.LLAMA8B["down"])):
        a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
        w = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        asc = torch.empty(M, device=dev).uniform_(1e-3, 1e-2, generator=g)
        ws = torch.empty(N, device=dev).uniform_(1e-3, 1e-2, generator=g)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        wt = w.t()
        cases = {"hipblaslt_int_mm_i32": (-1, lambda: torch._int_mm(a, wt))}
        for tile in (-1, 1, 3, 17, 18):
            cases["lockstep_bf16_tile%d" % tile] = (
                tile, lambda: ops.gemm(a, w, L.EPI_V21, L.LSK_BF16, asc=asc, ws=ws, out=out))
        for _ in range(100):
            cases["lockstep_bf16_tile-1"][1]()
        best = {}
        for _ in range(6):
            for key, (tile, fn) in cases.items():
                L.call("lsk_gemm_select", tile)
                best[key] = min(best.get(key, 1e9), _events_time(torch, fn, 10))
        L.call("lsk_gemm_select", -1)
        res[name] = {k: {"ms": round(v, 4), "TOPS": round(2 * M * N * K / (v * 1e-3) / 1e12, 1)} for k, v in best.items()}
        log("bench: vendor %s: %s" % (name, ", ".join("%s %.4f ms" % (k, v) for k, v in best.items())))
    return res


EAGER = False  # --eager: time the decode and MoE calls as plain launches (no HIP graph)


def _graph_time(torch, calls, reps):
    """Average milliseconds per call of the callables in `calls`, captured once into a HIP graph
    (so host overhead between launches is not timed) and replayed `reps` times; HIP events on
    the replay stream.  With --eager the calls are launched directly `reps` times instead."""
    if EAGER:
        for fn in calls:
            fn()
        return _events_time(torch, lambda: [fn() for fn in calls], reps) / len(calls)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in calls:          # first calls outside capture (one-time setup, allocator warm-up)
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in calls:
            fn()
    g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        g.replay()
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) / (reps * len(calls))


def decode_section(torch, args):
    """Batch-1/8/32 decode rows through w8a8_matmul (row quant + GEMV) and the GEMV alone on
    pre-quantised rows.  Each is timed as HIP-graph replays of one call per weight copy, the
    copies totalling > 768 MB so the 256 MB Infinity Cache cannot serve the weights.  GB/s counts
    the algorithmic bytes N*K + 4N + 4MK + 2MN of one call (int8 weights, f32 scales and
    activations, bf16 out)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
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
            q, asc = ops.rowquant(x)
            out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            full = [(lambda W=W: FS.w8a8_matmul(x, W, ws, out_dtype=torch.bfloat16)) for W in Ws]
            gemv = [(lambda W=W: ops.gemm(q, W, L.EPI_V21, L.LSK_BF16, asc=asc, ws=ws, out=out)) for W in Ws]
            ms = _graph_time(torch, full, 8)
            ms_k = _graph_time(torch, gemv, 8)
            nbytes = N * K + 4 * N + 4 * M * K + 2 * M * N
            gbs, gbs_k = nbytes / (ms * 1e-3) / 1e9, nbytes / (ms_k * 1e-3) / 1e9
            res["%s_M%d" % (name, M)] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                         "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                         "gemv_us": round(ms_k * 1e3, 2), "gemv_GB/s": round(gbs_k, 1),
                                         "gemv_frac_hbm": round(gbs_k / PEAK_HBM_GBS, 4)}
        del Ws
    # the single contract GEMM of the CPU-runnable case: M=16 rows of the Qwen2.5-7B o_proj shape
    # (N = K = 3584), x N(0,1) from seed 0, int8 weights, per-channel scales, bf16 out
    x, W8, ws = WL.dense_inputs(16, 3584, 3584, seed=0)
    xd, wsd = torch.from_numpy(x).to(dev), torch.from_numpy(ws).to(dev)
    W0 = torch.from_numpy(W8).to(dev)
    N, K, M = 3584, 3584, 16
    Ws = [W0.clone() for _ in range(int((768 << 20) // (N * K)) + 1)]
    q, asc = ops.rowquant(xd)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    full = [(lambda W=W: FS.w8a8_matmul(xd, W, wsd, out_dtype=torch.bfloat16)) for W in Ws]
    gemv = [(lambda W=W: ops.gemm(q, W, L.EPI_V21, L.LSK_BF16, asc=asc, ws=wsd, out=out)) for W in Ws]
    ms, ms_k = _graph_time(torch, full, 8), _graph_time(torch, gemv, 8)
    nbytes = N * K + 4 * N + 4 * M * K + 2 * M * N
    res["qwen25_7b_o_M16_seed0"] = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                    "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                    "gemv_us": round(ms_k * 1e3, 2),
                                    "gemv_frac_hbm": round(nbytes / (ms_k * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    del Ws
    res["note"] = ("us / GB/s: one w8a8_matmul call (row quant + GEMV kernels); gemv_*: the GEMV kernel alone on "
                   "pre-quantised rows; both from HIP-graph replays over > 768 MB of weight copies")
    return res


def ceiling_section(torch, args):
    """The part's int8 MFMA ceiling (lsk_mfma_probe: register-only v_mfma_i32_32x32x32_i8, 8 waves per
    SIMD) on all-zero, constant and uniformly random int8 operands: what the power budget leaves the
    GEMM kernels on the contract's random operands."""
    from lockstep_amd import _lib as L

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(23)
    blocks, iters = 2048, 2000
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    nops = 1 << 16
    cases = {"zero": torch.zeros(nops * 16, dtype=torch.int8, device=dev),
             "constant_0x55": torch.full((nops * 16,), 0x55, dtype=torch.int8, device=dev),
             "uniform_random": torch.randint(-127, 128, (nops * 16,), generator=g, device=dev, dtype=torch.int8)}
    ops_launch = blocks * 4 * iters * 16 * 65536
    res = {}
    for name, buf in cases.items():
        fn = lambda: L.call("lsk_mfma_probe", L.ptr(buf), nops, blocks, iters, L.ptr(sink), L.stream_of(buf))  # noqa
        for _ in range(3):
            fn()
        ms = _events_time(torch, fn, 5)
        res[name] = {"TOPS": round(ops_launch / (ms * 1e-3) / 1e12, 1), "ms": round(ms, 3)}
        log("bench: MFMA ceiling, %s operands: %.0f TOPS" % (name, res[name]["TOPS"]))
    res["note"] = ("register-only int8 MFMA loop, 2048 x 256 threads, 65536 ops per v_mfma_i32_32x32x32_i8; "
                   "HIP events")
    return res


def copy_section(torch, args):
    """A plain device copy of 1 GiB (read 1 GiB + write 1 GiB per launch): the calibration
    kernel for the FETCH_SIZE / WRITE_SIZE counters (rocprofv3 --pmc) behind `traffic`."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(7)
    dst = torch.empty_like(src)
    for _ in range(max(args.steps, 1)):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"bytes_per_launch": n}


TRAFFIC_FILES = {"qwen25_7b_block": "block_qwen25_7b_t8192_pmc.md", "llama8b": "dense_prefill_llama8b_pmc.md"}


def measured_traffic(workload):
    """HBM bytes per launch of the dominant kernel for each GEMM of a workload, from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, scaled by the 1 GiB copy's reading), or None."""
    path = os.path.join(ROOT, "profiles", TRAFFIC_FILES[workload])
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    kv = dict(t.split("=") for t in line.split(":", 1)[1].split())
                    return {k2: int(v) for k2, v in kv.items()}
    except (OSError, ValueError):
        return None
    return None


def _int8_expert_tables(torch, MR, g, dev, E, H, I):
    experts = []
    for _ in range(E):
        w13 = torch.randint(-127, 128, (2 * I, H), generator=g, device=dev, dtype=torch.int8)
        w2 = torch.randint(-127, 128, (H, I), generator=g, device=dev, dtype=torch.int8)
        ws13 = torch.empty(2 * I, device=dev).uniform_(1e-3, 1e-2, generator=g)
        ws2 = torch.empty(H, device=dev).uniform_(1e-3, 1e-2, generator=g)
        experts.append((w13.t(), ws13, w2.t(), ws2))
    return MR.ExpertTables(experts)


def _mx_expert_tables(torch, MR, g, dev, E, H, I):
    experts = []
    for _ in range(E):
        p13 = torch.randint(0, 256, (2 * I, H // 2), generator=g, device=dev, dtype=torch.uint8)
        s13 = 127 + torch.randint(-8, 3, (2 * I, H // 32), generator=g, device=dev, dtype=torch.int16)
        p2 = torch.randint(0, 256, (H, I // 2), generator=g, device=dev, dtype=torch.uint8)
        s2 = 127 + torch.randint(-8, 3, (H, I // 32), generator=g, device=dev, dtype=torch.int16)
        experts.append(((p13, s13.to(torch.uint8)), (p2, s2.to(torch.uint8)), None, None))
    return MR.ExpertTablesMX(experts, packed=True)


def moe_section(torch, args):
    """Config 4 (Qwen3-30B-A3B int8 experts, E=128, k=8, H=2048, I=768) and config 5 (GPT-OSS-20B
    MXFP4 experts, E=32, k=4, H=I=2880) at T in {1, 32, 4096}: one step = the router from the given
    logits (N(0,1), plus a Zipf(1.1) popularity bias for config 4) and the fused layer.  Two weight
    copies alternate so a step's experts were evicted from the Infinity Cache by the other copy;
    timed as HIP-graph replays (the layer has no host synchronisation), so host launch overhead
    is not counted."""
    from lockstep_amd import contract_common as CC
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    tab = CC.table_on(dev)
    res = {}
    cases = [("qwen3_30b_a3b_int8", WL.QWEN3_30B_A3B, 0, 75497472, 4718592 + 4 * (2 * 768 + 2048)),
             ("gpt_oss_20b_mxfp4", WL.GPT_OSS_20B, 1, 199065600, 13219200),
             ("gpt_oss_20b_mxfp4_mx2", WL.GPT_OSS_20B, 2, 199065600, 13219200)]
    copies = None
    for name, c, kind, ops_tok, bytes_expert in cases:
        E, k, H, I = c["E"], c["k"], c["H"], c["I"]
        mx = kind > 0
        # Qwen3-30B-A3B also at the token counts the reference publishes its fused-layer H100 times for
        # (8, 256, 2048)
        counts = (1, 8, 32, 256, 2048, 4096) if kind == 0 else (1, 32, 4096)
        wanted = [T for T in counts if not args.moe_cases or "%s_T%d" % (name, T) in args.moe_cases.split(",")]
        if not wanted:
            continue
        if kind != 2 or copies is None:  # the block-scaled case reuses the MXFP4 experts
            mk = _mx_expert_tables if mx else _int8_expert_tables
            copies = [mk(torch, MR, g, dev, E, H, I) for _ in range(2)]
        act = MR.act_swigluoai if mx else MR.act_silu
        fwd = (MR.moe_forward, MR.moe_forward_mx, MR.moe_forward_mx2)[kind]
        for T in wanted:
            x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
            logits = torch.randn((T, E), generator=g, device=dev)
            if not mx:
                rank = torch.randperm(E, generator=g, device=dev).to(torch.float32)
                logits = logits - 1.1 * torch.log1p(rank)[None, :]
            logits = logits.to(torch.bfloat16)
            def step(cp):
                # the router from the logits inside the layer (moe_ref's logits= form: the same
                # routing as router_from_logits, in fewer launches)
                fwd(x, None, cp, k, True, tab, 0, act, logits=logits)
            reps = 20 if T < 4096 else 5
            ms = _graph_time(torch, [(lambda cp=cp: step(cp)) for cp in copies], reps)
            idx, _, _ = MR.router_from_logits(logits, k, True, tab)
            active = int(torch.unique(idx).numel())
            gbs = active * bytes_expert / (ms * 1e-3) / 1e9
            tops = ops_tok * T / (ms * 1e-3) / 1e12
            peak_t = 2500.0 if mx else PEAK_INT8_TOPS
            res["%s_T%d" % (name, T)] = {
                "us": round(ms * 1e3, 2), "tokens_per_s": round(T / (ms * 1e-3), 1), "active_experts": active,
                "weight_GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "TOPS": round(tops, 2),
                "frac_mfma": round(tops / peak_t, 4)}
            log("bench: %s T=%d: %.1f us, %.0f tokens/s" % (name, T, ms * 1e3, T / (ms * 1e-3)))
        if kind == 0:
            copies = None
            torch.cuda.empty_cache()
    copies = None
    torch.cuda.empty_cache()
    res["note"] = ("tokens/s of one MoE layer (router from logits + fused layer); weight_GB/s counts the active "
                   "experts' weight bytes (int8 + f32 scales, or 4-bit codes + E8M0 bytes); TOPS counts "
                   "2 * k * (2I*H + I*H) ops per token; MXFP4 fractions are of the bf16 MFMA peak (2.5 PF) the "
                   "exact block contraction runs on; _mx2: the same layer with block-scaled activations "
                   "(moe_forward_mx2)")
    return res


# The reference's published grouped-GEMM times on H100 (ms) for the same shapes, with their source.
REF_GROUPED_H100 = {
    "qwen3_gate_up_R16384": (0.2378, "results/s3/logs/s21_m1g90b_h100.log:3"),
    "qwen3_down_R16384": (0.1508, "results/s3/logs/s21_m1g90b_h100.log:8"),
    "gptoss_int8_gate_up_R8192": (0.4620, "results/s3/logs/s21_m2x8_h100.log:11"),
    "gptoss_int8_gate_up_R256": (0.2012, "results/s3/logs/s21_m2x13_h100.log:11"),
    "gptoss_int8_down_R256": (0.1042, "results/s3/logs/s21_m2x13_h100.log:24"),
    "gptoss_mx_gate_up_R8192": (2.2807, "results/s3/logs/s21_m2x11_h100.log:4"),
    "gptoss_mx_down_R8192": (1.1408, "results/s3/logs/s21_m2x11_h100.log:22"),
    "gptoss_mx_gate_up_R256": (0.2693, "results/s3/logs/s21_m2x16_h100.log:5"),
    "gptoss_mx_down_R256": (0.1656, "results/s3/logs/s21_m2x16_h100.log:21"),
}


def grouped_section(torch, args):
    """The grouped expert GEMM stage alone (lsk_grouped_gemm_w8a8 / lsk_grouped_gemm_mx: expert-sorted
    rows through each expert's projection with the contract epilogue, bf16 out) at the shapes the
    reference publishes H100 times for: Qwen3-30B-A3B gate_up (N=1536, K=2048) and down (N=2048,
    K=768) over the 16384 rows of 2048 tokens x top-8; GPT-OSS-20B gate_up (N=5760) and down
    (N=2880) at K=2880 over 8192 rows (2048 tokens x top-4) and 256 rows (64 tokens), int8 and
    MXFP4.  Rows per expert come from the router on synthetic logits (Zipf-biased for Qwen3).
    HIP events over repeated launches on the launch stream."""
    from lockstep_amd import contract_common as CC
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    tab = CC.table_on(dev)
    res = {}

    def rows_of(T, E, k, zipf):
        logits = torch.randn((T, E), generator=g, device=dev)
        if zipf:
            rank = torch.randperm(E, generator=g, device=dev).to(torch.float32)
            logits = logits - 1.1 * torch.log1p(rank)[None, :]
        idx, _, _ = MR.router_from_logits(logits.to(torch.bfloat16), k, True, tab)
        cnt = torch.bincount(idx.reshape(-1), minlength=E)
        offs = torch.zeros(E + 1, dtype=torch.int32, device=dev)
        offs[1:] = torch.cumsum(cnt, 0).to(torch.int32)
        return offs, int(cnt.sum().item())

    def run(name, fn, R, N, K):
        for _ in range(3):
            fn()
        ms = _events_time(torch, fn, 20)
        ref_ms, src = REF_GROUPED_H100[name]
        res[name] = {"us": round(ms * 1e3, 1), "TOPS": round(2 * R * N * K / (ms * 1e-3) / 1e12, 1), "rows": R,
                     "N": N, "K": K, "reference_h100_us": round(ref_ms * 1e3, 1), "reference_source": src}
        log("bench: grouped %s: %.1f us (reference H100 %.1f us)" % (name, ms * 1e3, ref_ms * 1e3))

    # Qwen3-30B-A3B, int8
    c = WL.QWEN3_30B_A3B
    tables = _int8_expert_tables(torch, MR, g, dev, c["E"], c["H"], c["I"])
    offs, R = rows_of(2048, c["E"], c["k"], True)
    a8 = torch.randint(-127, 128, (R, c["H"]), generator=g, device=dev, dtype=torch.int8)
    asc = torch.empty(R, device=dev).uniform_(1e-3, 1e-2, generator=g)
    run("qwen3_gate_up_R16384", lambda: MR.grouped_linear(tables, "w13", a8, asc, offs), R, 2 * c["I"], c["H"])
    a8 = torch.randint(-127, 128, (R, c["I"]), generator=g, device=dev, dtype=torch.int8)
    run("qwen3_down_R16384", lambda: MR.grouped_linear(tables, "w2", a8, asc, offs), R, c["H"], c["I"])
    del tables, a8
    # GPT-OSS-20B shapes, int8 then MXFP4
    c = WL.GPT_OSS_20B
    for kind in ("int8", "mx"):
        mk = _int8_expert_tables if kind == "int8" else _mx_expert_tables
        tables = mk(torch, MR, g, dev, c["E"], c["H"], c["I"])
        fwd = MR.grouped_linear if kind == "int8" else MR.grouped_linear_mx
        for T in (2048, 64):
            offs, R = rows_of(T, c["E"], c["k"], False)
            asc = torch.empty(R, device=dev).uniform_(1e-3, 1e-2, generator=g)
            a8 = torch.randint(-127, 128, (R, c["H"]), generator=g, device=dev, dtype=torch.int8)
            if "gptoss_%s_gate_up_R%d" % (kind, R) in REF_GROUPED_H100:
                run("gptoss_%s_gate_up_R%d" % (kind, R), lambda: fwd(tables, "w13", a8, asc, offs), R, 2 * c["I"],
                    c["H"])
            if "gptoss_%s_down_R%d" % (kind, R) in REF_GROUPED_H100:
                a8 = torch.randint(-127, 128, (R, c["I"]), generator=g, device=dev, dtype=torch.int8)
                run("gptoss_%s_down_R%d" % (kind, R), lambda: fwd(tables, "w2", a8, asc, offs), R, c["H"], c["I"])
        del tables
        torch.cuda.empty_cache()
    res["note"] = ("grouped expert GEMM stage alone (rows already sorted by expert, contract epilogue, bf16 out), "
                   "HIP events; reference_h100_us: the reference's published time for the same shape on H100")
    return res


def cpu_baseline_moe(args):
    """The reference's moe_forward op sequence on the host (per-expert loop, int64 matmuls), on a
    token sample of the config-4 layer."""
    import numpy as np
    import torch

    from lockstep_amd import workloads as WL
    from oracle import contract as C
    from oracle import cpu_baseline as B

    c = WL.QWEN3_30B_A3B
    T = 16
    x, experts, logits = WL.moe_inputs(T, c["E"], c["k"], c["H"], c["I"], seed=9)
    idx, w, _ = C.router_from_logits(logits, c["k"], True)
    ex = [(torch.from_numpy(w13).t(), torch.from_numpy(ws13), torch.from_numpy(w2).t(), torch.from_numpy(ws2))
          for (w13, ws13, w2, ws2, _, _) in experts]
    xt = torch.from_numpy(x).to(torch.bfloat16)
    wt = torch.from_numpy(C.bf16_to_f32(w)).to(torch.bfloat16)
    t0 = time.perf_counter()
    B.moe_int8(xt, ex, torch.from_numpy(idx), wt)
    dt = time.perf_counter() - t0
    return {"value": round(T / dt, 2), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": "%d tokens of the Qwen3-30B-A3B layer (E=128, k=8, H=2048, I=768) through the torch CPU op "
                      "sequence of moe_ref.moe_forward (per-expert loop, int64 matmuls)" % T}


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
    ap.add_argument("--sections", default="block,dense,decode,moe,grouped,ceiling",
                    help="comma list of block (the headline), dense, decode, moe, grouped, ceiling, vendor, copy; the "
                         "JSON line's "
                         "value is the block step when block runs, else the dense step")
    ap.add_argument("--block-rows", type=int, default=8192, help="prefill rows T of the block step (8192 or 2048)")
    ap.add_argument("--moe-cases", default="", help="comma list of MoE cases to run, e.g. gpt_oss_20b_mxfp4_T4096 "
                                                     "(default: all)")
    ap.add_argument("--eager", action="store_true", help="time decode / MoE calls as plain launches, no HIP graphs "
                                                         "(for profilers that count per dispatch)")
    ap.add_argument("--mx-variant", type=int, default=0, help="main loop of the grouped MXFP4 GEMMs "
                                                              "(lsk_moe_mx_select; 0 is the default)")
    ap.add_argument("--moe-variant", type=int, default=-1, help="int8 grouped GEMM kernel "
                                                                "(lsk_moe_select; -1, by size, is the default)")
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
    global EAGER
    EAGER = args.eager
    _lib.call("lsk_moe_mx_select", args.mx_variant)
    _lib.call("lsk_moe_select", args.moe_variant)

    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic"}
    if "block" in sections:
        log("bench: Qwen2.5-7B block GEMMs through ref_block_v1, T=%d" % args.block_rows)
        b = block_section(torch, args)
        out.update({
            "value": round(b["value"], 2), "unit": "TOPS", "ms_per_step": round(b["ms_per_step"], 4),
            "config": {"workload": "Qwen2.5-7B decoder block GEMMs through ref_block_v1 (quant8_dyn + exact int8 "
                                   "GEMM + pow2 dequant, binary32 out), T=%d prefill rows" % b["T"],
                       "T": b["T"], "qkv": [4608, 3584], "o": [3584, 3584], "gate_up": [37888, 3584],
                       "down": [3584, 18944], "x": "f32 N(0,1)", "weights": "int8 U[-127,127], exponent 7",
                       "parallelism": "single GPU"},
            "roofline": b["roofline"], "per_site": b["per_site"]})
        tr = measured_traffic("qwen25_7b_block")
        if tr:
            out["roofline"]["traffic"] = sum(tr.values()) // len(tr)
            out["roofline"]["traffic_per_site"] = tr
            out["roofline"]["traffic_note"] = ("HBM bytes per launch (mean of the four GEMMs) from rocprofv3 "
                                               "FETCH_SIZE + WRITE_SIZE, profiles/block_qwen25_7b_t8192_pmc.md")
    if "dense" in sections:
        log("bench: Llama-3.1-8B MLP step (M=2048, gate_up 28672x4096 + down 4096x14336)")
        d = dense_section(torch, args)
        dense = {"workload": "Llama-3.1-8B MLP contract GEMMs, w8a8_matmul v2.1, M=2048 prefill rows, x f32 N(0,1) "
                             "with 0.1% +-20 outliers, bf16 out",
                 "TOPS": round(d["value"], 2), "ms_per_step": round(d["ms_per_step"], 4), "roofline": d["roofline"]}
        tr = measured_traffic("llama8b")
        if tr:
            dense["roofline"]["traffic"] = sum(tr.values()) // len(tr)
            dense["roofline"]["traffic_per_shape"] = tr
        out["llama3_1_8b_mlp_m2048"] = dense
        out["qwen2_5_7b_m8192_v21"] = d["qwen2_5_7b_m8192"]
        if "value" not in out:
            out.update({"value": dense["TOPS"], "unit": "TOPS", "ms_per_step": dense["ms_per_step"],
                        "config": {"workload": dense["workload"], "parallelism": "single GPU"},
                        "roofline": d["roofline"]})
    if "copy" in sections:
        out["copy"] = copy_section(torch, args)
    if "ceiling" in sections:
        out["mfma_ceiling"] = ceiling_section(torch, args)
    if "vendor" in sections:
        out["vendor"] = vendor_section(torch, args)
    if "decode" in sections:
        log("bench: decode rows M in {1, 8, 32}")
        out["decode"] = decode_section(torch, args)
    if "moe" in sections:
        log("bench: MoE layers")
        out["moe"] = moe_section(torch, args)
    if "grouped" in sections:
        log("bench: grouped expert GEMM stage")
        out["grouped"] = grouped_section(torch, args)
    if not args.no_cpu_baseline:
        log("bench: CPU baselines (reference op sequences, row samples)")
        if "block" in sections:
            out["cpu_baseline"] = cpu_baseline_block(args)
        if "dense" in sections:
            cb = cpu_baseline_dense(args)
            out["llama3_1_8b_mlp_m2048"]["cpu_baseline"] = cb
            out.setdefault("cpu_baseline", cb)
        if "moe" in sections:
            out["moe"]["cpu_baseline"] = cpu_baseline_moe(args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

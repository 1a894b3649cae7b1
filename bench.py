"""HiMuon optimizer-step benchmark on one MI355X.

Metric: HiMuon step latency (ms) on one MI355X, with NS5
TFLOP/s and its fraction of the bf16 dense MFMA peak.

Default workload: the Qwen3-4B-shaped parameter set (36 layers x {q 4096x2560,
k/v 1024x2560, o 2560x4096, gate/up 9728x2560, down 2560x9728}), bf16 params,
fp32 grads ~N(0, 1e-3^2), tile_size=512 (13,860 tiles), the whole step
captured in a hipGraph. Inputs are synthetic and resident in HBM before the
timed region.

A "step" is one ``optimizer.step()``: the write of the groups' (1 - lr*wd,
-lr) into the device table the graph reads (LR schedules need no recapture,
as with the reference's outside-graph WD/LR), then graph replay (momentum +
gather -> normaliser -> NS5 -> untile applying WD/LR to the parameters), then
the outside-graph WD/LR pass for anything the untile did not take (nothing in
the default workload). Defaults: 20 warm-up steps, 50 timed steps.

    python bench.py [--steps K] [--warmup W] [--config NAME] [--no-cpu-baseline] [--no-adamw]
                   [--reconfigure T]

Prints one JSON line. ``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (256 CU x 4096 FLOP/clk x 2.4 GHz)

# NS stage kernels per kernel family, per NS iteration.
NS_KERNELS = {
    "fused": "ns5 stage: ns_st_kernel<0> (X X^T) + ns_ba_kernel (c A A^T + b A, then B X + a X with B kept in LDS) per iteration",
    "stream": "ns5 stage: ns_st_kernel<0> (X X^T), <1> (c A A^T + b A), <2> (B X + a X) per iteration",
    "lds": "ns5 stage: ns5_lds_kernel (all 5 iterations of a 128-row tile resident in LDS)",
    "small": "ns5 stage: ns_gram_kernel x2 + ns_apply_kernel per iteration",
    "few_rows": "ns5 stage: ns5_small_kernel (all 5 iterations of a tile's 16, 32 or 64 rows resident in LDS)",
}


def ns_family(mp: int, np_: int, family: str = "auto", rows: int = 0) -> str:
    """The NS kernel family the library runs for an (mp, np) tile buffer
    (himuon_ns5_ex dispatch): with family "block128" the 128-blocks
    everywhere; with "stream3" the three streamed 256-block products wherever
    both edges are multiples of 256; with "auto", the operand's own 16, 32 or
    64 rows in LDS when it has rows <= 32 real rows, or <= 64 at np = 128
    ("few_rows"), LDS-resident
    for mp == 128 and np in {128, 256, 512}, the Gram kernel plus the fused
    GramB/Apply kernel for 512 x 512 tiles, streamed 256-blocks for other
    multiples of 256, else 128-blocks."""
    if family == "block128":
        return "small"
    if family == "auto" and rows and 0 < rows <= 64 and mp == 128 and (
            (rows > 32 and np_ == 128) or (rows <= 32 and np_ in (128, 256, 384, 512, 768, 1024))
            or (rows <= 16 and np_ in (1536, 2048))):
        return "few_rows"
    if mp == 128 and np_ in (128, 256, 512):
        return "lds"
    if mp % 256 == 0 and np_ % 256 == 0:
        return "fused" if (family == "auto" and mp == 512 and np_ == 512) else "stream"
    return "small"


PEAK_HBM_GBS = 8000.0

# HBM bytes per launch of the dominant kernel, from rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE (one pass each) over `bench.py --kernel-only`,
# each scaled by what the counter reads for the 256 MiB device copy this
# script runs first (a copy reads and writes exactly 256 MiB). Keyed by
# (config, kernel) with the sha256 (first 16 hex digits) of the kernel's
# source files: a figure measured on other sources is not reported.
KERNEL_TRAFFIC = {
    # 4096 tiles: FETCH_SIZE 2,389,747 KiB x 1.99968, WRITE_SIZE 2,097,152 KiB x 1.0
    ("qwen3-4b", "ns_ba_kernel"): (7.0409e+09, "3a8e3e6cc89a4157"),
    # 65,536 tiles of 128 x 128, the whole step (fp32 grads, momentum and params):
    # FETCH_SIZE 6,291,820 KiB x 1.99966, WRITE_SIZE 8,388,635 KiB x 1.0
    ("llama3-8b-t128", "lds_step_kernel"): (2.1473e+10, "d874cb37e2f82c2e"),
}
KERNEL_SOURCES = {
    "ns_ba_kernel": ["ns5_ba.hip", "ns5_kernels.h", "common.h"],
    "ns5_lds_kernel": ["ns5_lds.hip", "ns5_kernels.h", "common.h", "elem_ops.h"],
    "lds_step_kernel": ["ns5_lds.hip", "ns5_kernels.h", "common.h", "elem_ops.h"],
    "ns_st_kernel": ["ns5_stream.hip", "ns5_kernels.h", "common.h"],
}


def sources_digest(kernel: str) -> str:
    h = hashlib.sha256()
    for f in KERNEL_SOURCES[kernel]:
        with open(os.path.join(ROOT, "himuon_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


CONFIGS = {
    # name: (layers, [(h, w) per layer], tile_size, param dtype, description)
    "qwen3-4b": (36, [(4096, 2560), (1024, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (9728, 2560), (2560, 9728)],
                 512, torch.bfloat16, "Qwen3-4B-shaped param set (252 matrices), tile 512, hipGraph step"),
    "qwen3-0.6b": (28, [(2048, 1024), (1024, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (3072, 1024), (1024, 3072)],
                   512, torch.bfloat16, "Qwen3-0.6B-shaped param set (196 matrices), tile 512, hipGraph step"),
    "qwen3-0.6b-full": (28, [(2048, 1024), (1024, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (3072, 1024), (1024, 3072)],
                        1_000_000_000, torch.bfloat16, "Qwen3-0.6B-shaped set, full-matrix NS (Muon mode), hipGraph step"),
    "llama3-8b-t128": (32, [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336)],
                       128, torch.float32, "Llama-3-8B-shaped param set (224 matrices), tile 128, hipGraph step"),
    "cfg1": (1, [(1024, 1024)], 256, torch.float32, "single 1024x1024 fp32 matrix, tile 256"),
}


def ns_flops(m: int, n: int) -> float:
    """Algorithmic NS5 FLOPs of one m x n operand (m <= n): 5 (4 m^2 n + 2 m^3)."""
    return 5.0 * (4.0 * m * m * n + 2.0 * m**3)


def build_params(layers, shapes, dtype, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    params = []
    for _ in range(layers):
        for h, w in shapes:
            p = torch.nn.Parameter(torch.empty(h, w, device="cuda", dtype=dtype))
            p.data.normal_(0.0, 0.02, generator=g)
            if dtype != torch.float32:
                p.grad_dtype = torch.float32  # fp32 grads on bf16 params (the configs' setting)
            p.grad = torch.empty(h, w, device="cuda", dtype=torch.float32)
            p.grad.normal_(0.0, 1e-3, generator=g)
            params.append(p)
    return params


def algorithmic_flops(opt) -> float:
    total = 0.0
    for grp in opt._groups:
        t = grp["tiles"]
        total += ns_flops(t.m, t.n) * t.n_tiles
    return total


def time_ns_stage(opt, reps: int) -> float:
    """Average ms of the NS5 stage of one step (all chunks of all groups),
    HIP events on the stream the kernels are launched on. Each rep first
    re-gathers the tiles (untimed), so NS always starts from normalised
    momentum tiles as in a step, not from the previous rep's output."""
    s = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]

    def gather():
        for g in opt._groups:
            g["tiles"].gather()

    def run():
        for g in opt._groups:
            ofs = 0
            for c in g["chunks"]:
                g["tiles"].ns(ofs, c, g["steps"], opt._workspace, g["sub_batch"])
                ofs += c

    gather()
    run()
    torch.cuda.synchronize()
    for e0, e1 in evs:
        gather()
        e0.record(s)
        run()
        e1.record(s)
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in evs) / reps


def time_lds_step_stage(opt, reps: int) -> float | None:
    """Average ms of the step's LDS-resident launches (himuon_lds_step, one
    per chunk: momentum to WD/LR) over every group that runs them; None when
    no group does."""
    groups = [g for g in opt._groups if opt._fuse_lds_step and g["tiles"].lds_step_ok()]
    if not groups:
        return None

    def run():
        for g in groups:
            ofs = 0
            for c in g["chunks"]:
                g["tiles"].lds_step(ofs, c, g["steps"], opt._lrwd)
                ofs += c

    return _event_loop(run, reps)


def _event_loop(fn, reps: int, prep=None) -> float:
    """Average ms of fn() over reps runs, HIP events around each run on the
    current stream (the stream the library launches on); prep() runs
    untimed before each."""
    s = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    if prep:
        prep()
    fn()
    torch.cuda.synchronize()
    for e0, e1 in evs:
        if prep:
            prep()
        e0.record(s)
        fn()
        e1.record(s)
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in evs) / reps


def time_dominant_kernel(opt, reps: int) -> dict:
    """Per-launch time of the kernel that dominates the NS stage, on one
    sub-batch of the first group's tiles, from freshly gathered momentum:
    - 512 x 512 tiles: ns_ba_kernel (himuon_ba_bmm_add: c A A^T + b A and
      B X + a X fused) on X0 = bf16(x inv) and A = bf16(X0 X0^T); the first
      product (ns_st_kernel<0>, himuon_xxt) is timed beside it;
    - other geometries: one himuon_ns5 call on the sub-batch (ns5_lds_kernel
      for 128-row tiles: all iterations in one launch).
    Algorithmic FLOPs per launch: 4 m^3 per tile for ns_ba_kernel (2 m^3 for
    c A A^T, 2 m^2 n for B X with m = n), 2 m^2 n for the Gram kernel, the
    normative 5 (4 m^2 n + 2 m^3) per tile for a whole NS call."""
    from himuon_amd import _native as nat

    g = opt._groups[0]
    grp = g["tiles"]
    fam = ns_family(grp.mp, grp.np)
    n = min(g["sub_batch"], grp.n_tiles)
    if opt._fuse_lds_step and grp.lds_step_ok():
        # the whole step of n tiles in one launch (himuon_lds_step): the
        # momentum buffers and parameters of those tiles are read and written
        # once each, the grads read once
        ms = _event_loop(lambda: grp.lds_step(0, n, g["steps"], opt._lrwd), reps)
        gb = torch.empty(0, dtype=grp.dtype).element_size()
        pb = torch.empty(0, dtype=grp.upd_dtype).element_size()
        return {"kernel": "lds_step_kernel", "family": "lds_step", "launch_tiles": n, "launch_ms": ms,
                "flops_per_launch": float(ns_flops(grp.m, grp.n)) * n,
                "bytes_per_launch": float(_tile_elements(grp, n)) * (3 * gb + 2 * pb)}
    m, nn = grp.mp, grp.np
    x, y, inv = grp.tiles[:n], grp.alt[:n], grp.inv[:n]
    if fam == "fused":
        grp.gather()
        nat.ns5(x, y, inv, n, m, nn, 0, opt._workspace, n)  # X0 = bf16(x inv) in place
        A = opt._workspace[: n * m * m * 2].view(torch.bfloat16).view(n, m, m)
        gram_ms = _event_loop(lambda: nat.xxt(x, A, n, m, nn), reps)
        ba_ms = _event_loop(lambda: nat.ba_bmm_add(A, x, y, n, nat.NS_C, nat.NS_B, nat.NS_A), reps)
        flops = 4.0 * m**3 * n
        return {"kernel": "ns_ba_kernel", "family": fam, "launch_tiles": n, "launch_ms": ba_ms,
                "flops_per_launch": flops, "gram_kernel_launch_ms": gram_ms,
                "gram_kernel_tflops": 2.0 * m * m * nn * n / (gram_ms * 1e-3) / 1e12}
    steps = g["steps"]
    ms = _event_loop(lambda: nat.ns5(x, y, inv, n, m, nn, steps, opt._workspace, n, round_once=grp.round_once),
                     reps, prep=grp.gather)
    name = {"lds": "ns5_lds_kernel", "stream": "ns_st_kernel", "small": "ns_gram_kernel/ns_apply_kernel"}[fam]
    return {"kernel": name, "family": fam, "launch_tiles": n, "launch_ms": ms,
            "flops_per_launch": float(ns_flops(grp.m, grp.n)) * n}


def _tile_elements(grp, n: int) -> int:
    """Parameter elements covered by the group's first n bucket tiles."""
    total = 0
    for p, t0, cnt in zip(grp.params, grp.tile0, grp.tile_counts):
        h, w = p.shape
        C = -(-w // grp.tile_w)
        for lt in range(max(0, min(cnt, n - t0))):
            r, c = divmod(lt, C)
            total += min(grp.tile_h, h - r * grp.tile_h) * min(grp.tile_w, w - c * grp.tile_w)
    return total


def kernel_roofline(config: str, dk: dict) -> dict:
    tflops = dk["flops_per_launch"] / (dk["launch_ms"] * 1e-3) / 1e12
    entry = KERNEL_TRAFFIC.get((config, dk["kernel"]))
    traffic = None
    if entry is not None and dk["kernel"] in KERNEL_SOURCES and entry[1] == sources_digest(dk["kernel"]):
        traffic = entry[0]
    if "bytes_per_launch" in dk:
        # both bounds apply; the roofline's binding one is the lower ceiling:
        # HBM when the algorithmic intensity is below the ridge point
        gbs = dk["bytes_per_launch"] / (dk["launch_ms"] * 1e-3) / 1e9
        hbm = dk["flops_per_launch"] / dk["bytes_per_launch"] < PEAK_BF16_TFLOPS * 1e3 / PEAK_HBM_GBS
        out = {
            "kernel": f"{dk['kernel']} ({dk['launch_tiles']} tiles per launch)",
            "bound": "hbm" if hbm else "mfma",
            "achieved": round(gbs, 1) if hbm else round(tflops, 1),
            "peak": PEAK_HBM_GBS if hbm else PEAK_BF16_TFLOPS,
            "unit": "GB/s" if hbm else "TFLOP/s",
            "frac": round(gbs / PEAK_HBM_GBS if hbm else tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "launch_ms": round(dk["launch_ms"], 4),
            "flops_per_launch": dk["flops_per_launch"],
            "bytes_per_launch": dk["bytes_per_launch"],
            "tflops": round(tflops, 1),
            "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
            "hbm_gbs": round(gbs, 1),
            "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
        }
        if traffic:
            out["traffic_gbs"] = round(traffic / (dk["launch_ms"] * 1e-3) / 1e9, 1)
        return out
    out = {
        "kernel": f"{dk['kernel']} ({dk['launch_tiles']} tiles per launch)",
        "bound": "mfma",
        "achieved": round(tflops, 1),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
        "traffic": traffic,
        "launch_ms": round(dk["launch_ms"], 4),
        "flops_per_launch": dk["flops_per_launch"],
    }
    if traffic:
        out["traffic_gbs"] = round(traffic / (dk["launch_ms"] * 1e-3) / 1e9, 1)
        out["intensity_flop_per_byte"] = round(dk["flops_per_launch"] / traffic, 1)
    if "gram_kernel_launch_ms" in dk:
        out["gram_kernel_launch_ms"] = round(dk["gram_kernel_launch_ms"], 4)
        out["gram_kernel_tflops"] = round(dk["gram_kernel_tflops"], 1)
    return out


def time_ns_untile_stage(opt, reps: int) -> float | None:
    """Average ms of NS5 + untile (with WD/LR) as the step runs them: one
    launch per chunk where the untile is fused into the last NS iteration,
    else the NS launches and then the untile. HIP events on the launch
    stream; each rep re-gathers first (untimed). None when no group takes
    the fused path (ns5_ms + untile_ms then cover the same work)."""
    groups = [g for g in opt._groups
              if not (opt._fuse_lds_step and g["tiles"].lds_step_ok())]
    if not any(opt._fuse_ns_untile and g["tiles"].ns_untile_ok(g["steps"]) for g in groups):
        return None
    s = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]

    def run():
        for g in groups:
            grp = g["tiles"]
            nsu = opt._fuse_ns_untile and grp.ns_untile_ok(g["steps"])
            ofs = 0
            for c in g["chunks"]:
                if nsu:
                    grp.ns_untile(ofs, c, g["steps"], opt._workspace, g["sub_batch"], opt._lrwd)
                else:
                    grp.ns(ofs, c, g["steps"], opt._workspace, g["sub_batch"])
                ofs += c
            if not nsu and grp.fused:
                grp.untile(g["steps"], opt._lrwd)
            elif not nsu:
                grp.untile(g["steps"])

    for g in groups:
        g["tiles"].gather()
    run()
    torch.cuda.synchronize()
    for e0, e1 in evs:
        for g in groups:
            g["tiles"].gather()
        e0.record(s)
        run()
        e1.record(s)
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in evs) / reps


def time_io_stage(opt, reps: int) -> tuple[float, float]:
    """Average ms of gather (+normaliser) and of untile for one step (for a
    fused group, the untile that applies WD/LR to the parameters in place)."""
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    torch.cuda.synchronize()
    ev[0].record(s)
    for _ in range(reps):
        for g in opt._groups:
            g["tiles"].gather()
    ev[1].record(s)
    for _ in range(reps):
        for g in opt._groups:
            g["tiles"].untile(g["steps"], opt._lrwd)
    ev[2].record(s)
    ev[2].synchronize()
    return ev[0].elapsed_time(ev[1]) / reps, ev[1].elapsed_time(ev[2]) / reps


def time_apply(opt, reps: int) -> float:
    """Average ms of the outside-graph WD + LR application of one step (the
    multi-tensor HIP launch), HIP events on the current stream."""
    s = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    opt._apply_pending_updates()
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(reps):
        opt._apply_pending_updates()
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def time_adamw(reps: int, rows: int = 151936, cols: int = 2560) -> dict:
    """The AdamW fallback of one step (himuon.py:359-372) for a Qwen3-4B-shaped
    embedding (151,936 x 2,560, fp32 grads and moments): the fused HIP pass
    (himuon_adamw_step: read g, m, v, write m, v, update = 24 B per element)
    against the reference's torch op chain on the same tensors. HIP events on
    the current stream, the stream both run on."""
    from himuon_amd.engine import AdamwTables

    gen = torch.Generator(device="cuda").manual_seed(1)
    g = torch.randn(rows, cols, device="cuda", generator=gen) * 1e-3
    m, v, u = torch.zeros_like(g), torch.zeros_like(g), torch.empty_like(g)
    st = torch.zeros((), device="cuda")
    tables = AdamwTables([(g, m, v, u, st, 0)])

    def fused():
        tables.run([0.95], [0.95], [1e-8])

    def torch_ops():
        st.add_(1)
        m.lerp_(g, 1 - 0.95)
        v.lerp_(g.square(), 1 - 0.95)
        bc1 = 1 - 0.95**st
        bc2 = 1 - 0.95**st
        return (m / bc1) / (v.sqrt() / bc2**0.5 + 1e-8)

    def timeit(fn) -> float:
        s = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        fn()
        torch.cuda.synchronize()
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps

    fused_ms = timeit(fused)
    torch_ms = timeit(torch_ops)
    n = g.numel()
    del g, m, v, u, st, tables
    torch.cuda.empty_cache()
    return {
        "workload": f"Qwen3-4B embed_tokens {rows}x{cols}, fp32 grads and moments",
        "elements": n,
        "fused_ms": round(fused_ms, 3),
        "fused_gbs": round(24.0 * n / (fused_ms * 1e-3) / 1e9, 1),
        "torch_ops_ms": round(torch_ms, 3),
        "speedup": round(torch_ms / fused_ms, 2),
    }


def time_reconfigure(opt, tile: int, steps: int) -> dict:
    """reconfigure(tile_size=tile) mid-run: the plan, buffers and graph are
    dropped; time each of the eager warm-up steps, the step that recaptures
    the graph, and the replays that follow (wall clock around each step with
    device synchronisation)."""

    def timed_step() -> float:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        opt.step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    opt.reconfigure(tile_size=tile)
    eager = [round(timed_step(), 3) for _ in range(opt._cuda_graph_warmup)]
    capture = round(timed_step(), 3)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step()
    torch.cuda.synchronize()
    replay = (time.perf_counter() - t0) * 1e3 / steps
    ns_ms = time_ns_stage(opt, reps=max(3, steps // 2))
    flops = algorithmic_flops(opt)
    return {
        "tile_size": tile,
        "tiles": sum(g["tiles"].n_tiles for g in opt._groups),
        "eager_steps_ms": eager,
        "capture_step_ms": capture,
        "replay_step_ms": round(replay, 3),
        "ns5_ms": round(ns_ms, 3),
        "ns5_tflops": round(flops / (ns_ms * 1e-3) / 1e12, 1),
        "ns5_frac_peak": round(flops / (ns_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
    }


# The reference's NS microbenchmark points (microbench/experiments/
# exp_ns_kernel_microbench.py:50,279: T = 128, B = 32 / 128 / 512 / 2048; its
# fused ns5_smem kernel's times read off microbench/plots/ns_kernel_microbench.png,
# unstated NVIDIA hardware) and its rectangular sweep
# (exp_ns5_rect_bench.py:83-103,171: M <= N from DIMS, M N + 2 M^2 <= 49152,
# B = 2^21 // (M N)).
# (ns-t128-b65536: the cfg5 sub-batch size, beyond the reference's published points)
NS_MICRO_B = {"ns-t128-b32": 32, "ns-t128-b128": 128, "ns-t128-b512": 512, "ns-t128-b2048": 2048,
              "ns-t128-b65536": 65536}
NS_MICRO_REF_MS = {32: 0.14, 128: 0.20, 512: 0.46, 2048: 1.55}
RECT_DIMS = [16, 32, 64, 128, 256, 512, 1024, 2048]


def rect_shapes() -> list[tuple[int, int]]:
    return [(m, n) for m in RECT_DIMS for n in RECT_DIMS if n >= m and m * n + 2 * m * m <= 49152]


def ns_micro(B: int, reps: int, warmup: int, T: int = 128) -> dict:
    """NS5 on B random T x T tiles per call, as the reference's microbenchmark
    measures it: input torch.randn(B, T, T) bf16 with seed 42
    (exp_ns_kernel_microbench.py:121-123), a call = the Frobenius normaliser
    (himuon_tile_scale's formula, 1 / (||x|| + eps), here one torch reduction)
    + himuon_ns5 (all 5 iterations); median of `reps` calls with HIP events
    around each, after `warmup` calls. Each call starts from the same input
    (the NS runs from x into the ping-pong buffer; the input buffer is
    refreshed untimed)."""
    from himuon_amd import _native as nat

    torch.manual_seed(42)
    x0 = torch.randn(B, T, T, device="cuda", dtype=torch.bfloat16)
    x = x0.clone()
    y = torch.empty_like(x)
    inv = torch.empty(B, device="cuda", dtype=torch.float32)
    ws = torch.empty(max(1, nat.ns5_workspace_bytes(B, T, T)), device="cuda", dtype=torch.uint8)

    def norm():
        torch.reciprocal(x.float().flatten(1).norm(dim=1).add_(1e-7), out=inv)

    def ns():
        nat.ns5(x, y, inv, B, T, T, 5, ws, B)

    s = torch.cuda.current_stream()
    t_call, t_ns = [], []
    for k in range(warmup + reps):
        x.copy_(x0)
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(s)
        norm()
        e[1].record(s)
        ns()
        e[2].record(s)
        e[2].synchronize()
        if k >= warmup:
            t_call.append(e[0].elapsed_time(e[2]))
            t_ns.append(e[1].elapsed_time(e[2]))
    ms, ns_ms = float(np.median(t_call)), float(np.median(t_ns))
    flops = 30.0 * T**3 * B
    return {"B": B, "T": T, "ms": ms, "ns5_ms": ns_ms, "tflops": flops / (ms * 1e-3) / 1e12,
            "ns5_tflops": flops / (ns_ms * 1e-3) / 1e12, "family": ns_family(T, T)}


def ns_rect(reps: int, warmup: int, total_elements: int = 1 << 21) -> list[dict]:
    """The reference's rectangular sweep: for each admitted (M, N), B =
    total // (M N) random tiles zero-padded into the library's (mp, np)
    buffer (multiples of 128), the NS5 call timed as in ns_micro (normaliser
    untimed here: the reference's throughput column counts the NS call).
    Reported: median ms, the reference's bytes metric (B M N 2 bytes / time)
    and algorithmic TFLOP/s on the unpadded shape, 5 (4 M^2 N + 2 M^3)."""
    from himuon_amd import _native as nat

    out = []
    for m, n in rect_shapes():
        B = max(1, total_elements // (m * n))
        mp, np_ = -(-m // 128) * 128, -(-n // 128) * 128
        torch.manual_seed(42)
        x0 = torch.zeros(B, mp, np_, device="cuda", dtype=torch.bfloat16)
        x0[:, :m, :n] = torch.randn(B, m, n, device="cuda", dtype=torch.bfloat16)
        inv = torch.reciprocal(x0.float().flatten(1).norm(dim=1).add_(1e-7))
        x, y = x0.clone(), torch.empty_like(x0)
        ws = torch.empty(max(1, nat.ns5_workspace_bytes(B, mp, np_)), device="cuda", dtype=torch.uint8)
        s = torch.cuda.current_stream()
        ts = []
        for k in range(warmup + reps):
            x.copy_(x0)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            nat.ns5(x, y, inv, B, mp, np_, 5, ws, B, rows=m)
            e1.record(s)
            e1.synchronize()
            if k >= warmup:
                ts.append(e0.elapsed_time(e1))
        ms = float(np.median(ts))
        out.append({"M": m, "N": n, "B": B, "mp": mp, "np": np_, "family": ns_family(mp, np_, rows=m),
                    "ms": round(ms, 4),
                    "GBps": round(B * m * n * 2 / (ms * 1e-3) / 1e9, 1),
                    "tflops": round(ns_flops(m, n) * B / (ms * 1e-3) / 1e12, 2)})
        del x0, x, y, ws
    return out


# The reference's optimizer step microbenchmark
# (microbench/experiments/exp_optimizer_step_microbench.py:58-86,123-164):
# 8 x Linear(H, H) bf16 parameters with bf16 grads ~N(0, 1) refilled before
# every step, HiMuon at tile 512 with graph capture (warm-up 3) against Muon
# (full-matrix NS); median of 50 steps after 20, HIP events around each step;
# peak memory over 5 steps after 5. Its figure (a) reports Muon / HiMuon
# step-time ratios of 2.3 / 3.7 / 5.4 at H = 1024 / 2048 / 4096 on unstated
# NVIDIA hardware (read off microbench/plots/optimizer_step_microbench.png).
# Muon here is this library's full-matrix mode (tile_size above the matrix:
# NS on each whole matrix, same-shape matrices batched), the reference's
# Muon update on the same kernels.
STEP_MICRO_H = {"step-8xh1024": 1024, "step-8xh2048": 2048, "step-8xh4096": 4096}
STEP_MICRO_REF_RATIO = {1024: 2.3, 2048: 3.7, 4096: 5.4}


def step_micro(H: int, reps: int, warmup: int, K: int = 8) -> dict:
    from himuon_amd.optimizers.himuon import HiMuon

    res = {}
    for label, tile in (("himuon_tile512", 512), ("muon_full_matrix", 1_000_000_000)):
        torch.cuda.empty_cache()
        torch.manual_seed(7)
        params = []
        for _ in range(K):
            p = torch.nn.Parameter(torch.empty(H, H, device="cuda", dtype=torch.bfloat16))
            torch.nn.init.kaiming_uniform_(p, a=5 ** 0.5)  # nn.Linear's init
            params.append(p)
        opt = HiMuon([{"params": params, "weight_decay": 0.0, "use_muon": True}], lr=0.02, momentum=0.95,
                     nesterov=True, weight_decay=0.1, tile_size=tile, ns_steps=5, cuda_graph=True,
                     cuda_graph_warmup=3)
        gen = torch.Generator(device="cuda")

        def fill(seed):
            gen.manual_seed(seed)
            for p in params:
                if p.grad is None:
                    p.grad = torch.empty_like(p)
                p.grad.normal_(generator=gen)

        for i in range(warmup):
            fill(5000 + i)
            opt.step()
        torch.cuda.synchronize()
        times = []
        for i in range(reps):
            fill(5000 + warmup + i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            opt.step()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        for i in range(5):
            fill(9000 + i)
            opt.step()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        for i in range(5):
            fill(9100 + i)
            opt.step()
        torch.cuda.synchronize()
        res[label] = {"ms_median": round(float(np.median(times)), 4),
                      "ms_p25_p75": [round(float(np.percentile(times, q)), 4) for q in (25, 75)],
                      "peak_mem_bytes": int(torch.cuda.max_memory_allocated())}
        del opt, params
    ratio = res["muon_full_matrix"]["ms_median"] / res["himuon_tile512"]["ms_median"]
    mem = res["himuon_tile512"]["peak_mem_bytes"] / res["muon_full_matrix"]["peak_mem_bytes"] - 1.0
    return {"H": H, "K": K, **res, "speedup_vs_muon": round(ratio, 3), "peak_mem_vs_muon": round(mem, 4),
            "reference_speedup_vs_muon": STEP_MICRO_REF_RATIO.get(H)}


# The reference's per-layer tile-NS vs full-NS benchmark
# (microbench/experiments/exp_real_shapes_bench.py:43-50,125-160): for each
# Muon-eligible weight shape of a Qwen3 transformer block, G ~ randn bf16;
# tile NS = HiMuon._tile -> newton_schulz on the (R C, T, T) batch ->
# HiMuon._untile (the torch tiling copies included, as there), full NS =
# NS of the whole matrix (there Muon's zeropower_via_newtonschulz5, here this
# library's 2-D newton_schulz); median of 30 calls after 3, HIP events. Its
# figure reports tile/full speed-ups of 1.4-1.6x (Qwen3-0.6B) and 1.3x (k/v)
# to 2.9x (q) (Qwen3-4B) on unstated NVIDIA hardware
# (microbench/plots/real_shapes_bench.png).
REAL_SHAPES = {
    "real-shapes-qwen3-0.6b": [("q_proj", (2048, 1024)), ("k_proj", (1024, 1024)), ("v_proj", (1024, 1024)),
                               ("o_proj", (1024, 2048)), ("gate_proj", (3072, 1024)), ("up_proj", (3072, 1024)),
                               ("down_proj", (1024, 3072))],
    "real-shapes-qwen3-4b": [("q_proj", (4096, 2560)), ("k_proj", (1024, 2560)), ("v_proj", (1024, 2560)),
                             ("o_proj", (2560, 4096)), ("gate_proj", (9728, 2560)), ("up_proj", (9728, 2560)),
                             ("down_proj", (2560, 9728))],
}


def real_shapes(config: str, reps: int, warmup: int, tile: int = 512) -> list[dict]:
    from himuon_amd.optimizers.himuon import HiMuon

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        return float(np.median(ts))

    rows = []
    for name, (h, w) in REAL_SHAPES[config]:
        torch.manual_seed(0)
        G = torch.randn(h, w, device="cuda", dtype=torch.bfloat16)

        def tile_ns():
            tiled, info = HiMuon._tile(G, (tile, tile))
            R, C, Th, Tw = tiled.shape
            orth = HiMuon.newton_schulz(tiled.view(-1, Th, Tw), steps=5).view(R, C, Th, Tw)
            return HiMuon._untile(orth, info)

        def full_ns():
            return HiMuon.newton_schulz(G.clone(), steps=5)

        t_tile, t_full = timed(tile_ns), timed(full_ns)
        m, n = min(h, w), max(h, w)
        R, C = -(-h // tile), -(-w // tile)
        rows.append({"layer": name, "shape": [h, w], "tiles": R * C, "tile_ms": round(t_tile, 4),
                     "full_ms": round(t_full, 4), "speedup": round(t_full / t_tile, 3),
                     "full_ns_tflops": round(ns_flops(m, n) / (t_full * 1e-3) / 1e12, 1),
                     "tile_ns_tflops": round(R * C * ns_flops(tile, tile) / (t_tile * 1e-3) / 1e12, 1)})
    return rows


def ns_micro_line(args) -> dict:
    """The JSON line of an NS microbenchmark config."""
    warmup = max(args.warmup, 2)
    if args.config in STEP_MICRO_H:
        r = step_micro(STEP_MICRO_H[args.config], args.steps, args.warmup)
        return {"metric": "HiMuon step time (ms), 8 x Linear(H, H) bf16, tile 512, against full-matrix NS (Muon)",
                "value": r["himuon_tile512"]["ms_median"], "unit": "ms", "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": r["himuon_tile512"]["ms_median"], "higher_is_better": False,
                "scaling": "strong", "vs_baseline": None, "dtype": "bf16",
                "data": "synthetic: nn.Linear init, bf16 grads ~N(0, 1) refilled per step",
                "config": {"workload": args.config, "H": r["H"], "K": r["K"]}, "result": r}
    if args.config in REAL_SHAPES:
        rows = real_shapes(args.config, args.steps, warmup)
        return {"metric": "NS5 time per call (ms), tile 512 vs full matrix, per layer shape",
                "value": round(sum(r["tile_ms"] for r in rows), 4), "unit": "ms (sum of tile-NS over layers)",
                "n_gpus": 1, "steps": args.steps, "warmup": warmup, "higher_is_better": False,
                "scaling": "strong", "vs_baseline": None, "dtype": "bf16", "data": "synthetic: torch.randn bf16",
                "config": {"workload": args.config, "tile": 512}, "layers": rows}
    if args.config == "ns-rect":
        rows = ns_rect(args.steps, warmup)
        return {"metric": "NS5 time per call (ms) over the reference's (M, N) tile-shape sweep",
                "value": round(sum(r["ms"] for r in rows), 4), "unit": "ms (sum over shapes)", "n_gpus": 1,
                "steps": args.steps, "warmup": warmup, "higher_is_better": False, "scaling": "strong",
                "vs_baseline": None, "dtype": "bf16",
                "data": "synthetic: torch.randn tiles, seed 42, zero-padded to multiples of 128",
                "config": {"workload": "ns-rect", "total_elements": 1 << 21, "shapes": len(rows)}, "shapes": rows}
    B = NS_MICRO_B[args.config]
    r = ns_micro(B, args.steps, warmup)
    ref = NS_MICRO_REF_MS.get(B)  # a figure exists for the reference's published points only
    return {"metric": "NS5 time per call (ms), T = 128, B tiles (normaliser + 5 iterations)",
            "value": round(r["ms"], 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": warmup,
            "ms_per_step": round(r["ms"], 4), "higher_is_better": False, "scaling": "strong",
            "vs_baseline": round(r["ms"] / ref, 4) if ref else None, "dtype": "bf16",
            "data": "synthetic: torch.randn(B, 128, 128) bf16, seed 42 (exp_ns_kernel_microbench.py:121-123)",
            "config": {"workload": args.config, "T": 128, "B": B, "kernel_family": r["family"]},
            "tflops": round(r["tflops"], 1), "frac_peak": round(r["tflops"] / PEAK_BF16_TFLOPS, 4),
            "ns5_only_ms": round(r["ns5_ms"], 4), "ns5_only_tflops": round(r["ns5_tflops"], 1),
            "reference_figure_ms": ref,
            "reference_figure_note": "the reference's fused ns5_smem kernel, read off ns_kernel_microbench.png "
                                     "(log axis, unstated NVIDIA GPU); vs_baseline = value / that time"}


def _cpu_model() -> tuple[str, bool]:
    """Full CPU model string (lscpu's, else /proc/cpuinfo's) and whether the
    host has native bf16 (AVX512-BF16 or AMX-BF16)."""
    model, bf16 = platform.processor() or platform.machine(), False
    try:
        with open("/proc/cpuinfo") as f:
            info = f.read()
        names = [ln.split(":", 1)[1].strip() for ln in info.splitlines() if ln.startswith("model name")]
        model = names[0] if names else model
        bf16 = " avx512_bf16" in info or " amx_bf16" in info
    except OSError:
        pass
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = dict(ln.split(":", 1) for ln in out.splitlines() if ":" in ln)
        name = fields.get("Model name", "").strip()
        if len(name) > len(model):
            model = name
        extra = [f"{k.strip()} {fields[k].strip()}" for k in ("Vendor ID", "CPU family", "Model", "Stepping")
                 if k in fields]
        if extra:
            model = f"{model} ({', '.join(extra)})"
    except Exception:  # lscpu missing or unreadable: keep /proc/cpuinfo's name
        pass
    return model, bf16


def cpu_baseline(layers, shapes, tile, pdtype, budget_s: float = 20.0):
    """The reference's eager step restated in torch on the host CPU
    (oracle/torch_cpu_step.py: bf16 GEMMs on the host's native bf16 units,
    fp32 momentum, WD/LR in the parameter dtype) on full layers of the config
    (every matrix of a layer: momentum, tiling, NS5, untiling, WD/LR), after
    one untimed pass: the layer is stepped again until about half the time
    budget is spent (at least once), and the step is the mean layer time x the
    number of layers. If one layer does not fit the budget, only the matrices
    that fit are timed and scaled by their share of the layer's NS tiles.
    Threads: OMP_NUM_THREADS (the GPU box's CPU share), else all cores."""
    from oracle import torch_cpu_step as TC

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    cpu_model, bf16 = _cpu_model()
    gen = torch.Generator().manual_seed(0)
    layer = []
    for h, w in shapes:
        g = torch.randn(h, w, generator=gen) * 1e-3
        p = (torch.randn(h, w, generator=gen) * 0.02).to(pdtype)
        layer.append((p, g, torch.zeros(h, w)))

    def ntiles(h, w):
        return (-(-h // tile)) * (-(-w // tile)) if h * w > tile * tile else 1

    tiles_layer = sum(ntiles(h, w) for h, w in shapes)
    # untimed pass (oneDNN kernel selection, page faults), then the timed one
    t_warm = time.perf_counter()
    for p, g, buf in layer:
        TC.step_param(p, g, buf, 1e-2, 0.1, tile)
        if time.perf_counter() - t_warm > budget_s / 2:
            break
    done_tiles, t_spent, passes = 0, 0.0, 0
    while t_spent < budget_s / 2:
        for (p, g, buf), (h, w) in zip(layer, shapes):
            if t_spent > budget_s / 2:
                break
            t0 = time.perf_counter()
            TC.step_param(p, g, buf, 1e-2, 0.1, tile)
            t_spent += time.perf_counter() - t0
            done_tiles += ntiles(h, w)
        passes += 1
    torch.set_num_threads(prev_threads)
    layer_ms = t_spent * 1e3 * tiles_layer / done_tiles
    whole = done_tiles >= tiles_layer
    return {
        "value": round(layer_ms * layers, 1),
        "unit": "ms/step (mean layer time, x%d extrapolated)" % layers,
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/torch_cpu_step.py (the reference's eager step in torch on the CPU: bf16 bmm/baddbmm on "
                   f"native bf16, fp32 momentum, WD/LR) on {'full layers' if whole else 'part of one layer'}: "
                   f"{done_tiles} NS tiles ({done_tiles / tiles_layer:.2f} layers of {tiles_layer} tiles, "
                   f"{len(shapes)} matrices each) in {t_spent:.1f} s, after one untimed pass"),
        "layer_ms": round(layer_ms, 1),
        "cpu": cpu_model,
        "cpu_native_bf16": bf16,
        "torch_threads": threads,
    }


def _smi_sample() -> tuple[float, float] | None:
    """(socket power W, mean gfx clock MHz over the XCDs) from amd-smi."""
    import subprocess

    try:
        out = subprocess.run(["amd-smi", "metric", "--power", "--clock", "--json"], capture_output=True,
                             text=True, timeout=10).stdout
        d = json.loads(out)
        g = d["gpu_data"][0] if isinstance(d, dict) else d[0]
        clks = [v["clk"]["value"] for k, v in g["clock"].items()
                if k.startswith("gfx_") and isinstance(v.get("clk", {}).get("value"), (int, float))]
        return float(g["power"]["socket_power"]["value"]), float(np.mean(clks))
    except Exception:
        return None


def power_probe(opt, seconds: float = 12.0) -> dict:
    """Board power and shader clock (amd-smi, sampled from a thread every
    0.3 s) while the NS5 stage runs back to back, and for comparison while a
    16384^3 bf16 torch.matmul (hipBLASLt) runs: both sit at the board's power
    limit, which is why the MFMA clock under NS is below the 2.4 GHz behind
    the published peak."""
    import threading

    samples, phase, stop = [], ["idle"], threading.Event()

    def sampler():
        while not stop.is_set():
            v = _smi_sample()
            if v is not None:
                samples.append((phase[0], *v))
            time.sleep(0.3)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    time.sleep(2.0)
    phase[0] = "ns5_stage"
    t0 = time.time()
    while time.time() - t0 < seconds:
        time_ns_stage(opt, 3)
    phase[0] = "gemm_16384"
    a = torch.randn(16384, 16384, device="cuda", dtype=torch.bfloat16)
    b = torch.randn_like(a)
    t0 = time.time()
    while time.time() - t0 < seconds * 0.75:
        for _ in range(8):
            a @ b
        torch.cuda.synchronize()
    phase[0] = "end"
    stop.set()
    th.join()
    out = {}
    for ph in ("idle", "ns5_stage", "gemm_16384"):
        v = [(p, c) for q, p, c in samples if q == ph]
        if v:
            out[ph] = {"samples": len(v), "power_w_mean": round(float(np.mean([p for p, _ in v])), 1),
                       "power_w_max": max(p for p, _ in v),
                       "gfx_clock_mhz_mean": round(float(np.mean([c for _, c in v])), 1)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="qwen3-4b",
                    choices=sorted(CONFIGS) + sorted(NS_MICRO_B) + ["ns-rect"] + sorted(STEP_MICRO_H)
                    + sorted(REAL_SHAPES),
                    help="a parameter-set config (the HiMuon step), or a microbenchmark of the reference's: "
                         "ns-t128-b{32,128,512,2048} (NS5 per call on B tiles of 128x128; also b65536), ns-rect "
                         "(its rectangular tile-shape sweep), step-8xh{1024,2048,4096} (8 x Linear(H, H) step, "
                         "tile 512 against full-matrix NS) or real-shapes-qwen3-{0.6b,4b} (per-layer tile-NS "
                         "against full-NS)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-adamw", action="store_true",
                    help="skip the AdamW fallback timing (Qwen3-4B embedding, fused vs torch ops)")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--kernel-only", action="store_true",
                    help="after the warm-up steps, only time the dominant NS kernel (the command the "
                         "rocprofv3 counter passes run) and print its roofline")
    ap.add_argument("--power", action="store_true",
                    help="after the warm-up steps, sample board power and shader clock (amd-smi) while "
                         "the NS5 stage runs, and while a large hipBLASLt GEMM runs, and print them")
    ap.add_argument("--reconfigure", type=int, default=None, metavar="T",
                    help="after the timed steps, reconfigure(tile_size=T) and time the eager "
                         "warm-up steps, the recapture step and the replays of the new regime")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build runs the HiMuon step on one GPU only; --gpus N > 1 is not "
                                   "supported (multi-GPU would shard the tiles and all-gather the updated "
                                   "parameter rows; not built)"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm device"}))
        sys.exit(2)

    from himuon_amd._native import load
    from himuon_amd.optimizers.himuon import HiMuon

    load()
    if args.config in NS_MICRO_B or args.config in STEP_MICRO_H or args.config in REAL_SHAPES \
            or args.config == "ns-rect":
        print(json.dumps(ns_micro_line(args)), flush=True)
        return
    # A 256 MiB device copy of known size: under `rocprofv3 --pmc` its
    # FETCH_SIZE / WRITE_SIZE readings calibrate those counters (a plain copy
    # reads and writes exactly 256 MiB), so kernel traffic can be scaled.
    cal = torch.empty(64 << 20, device="cuda", dtype=torch.float32)
    torch.empty_like(cal).copy_(cal)
    del cal
    layers, shapes, tile, pdtype, desc = CONFIGS[args.config]
    params = build_params(layers, shapes, pdtype)
    opt = HiMuon([{"params": params, "use_muon": True}], lr=1e-2, weight_decay=0.1, tile_size=tile,
                 cuda_graph=True, cuda_graph_warmup=3)
    warmup = max(args.warmup, 4)  # 3 eager steps + capture
    for _ in range(warmup):
        opt.step()
    torch.cuda.synchronize()
    if args.power:
        print(json.dumps({"config": args.config, "power": power_probe(opt)}), flush=True)
        return
    if args.kernel_only:
        dk = time_dominant_kernel(opt, reps=max(3, args.steps))
        print(json.dumps({"config": args.config, "roofline": kernel_roofline(args.config, dk),
                          "sources_digest": sources_digest(dk["kernel"]) if dk["kernel"] in KERNEL_SOURCES
                          else None}), flush=True)
        return

    s = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(s)
    for _ in range(args.steps):
        opt.step()
    e1.record(s)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ev_ms = e0.elapsed_time(e1) / args.steps
    # per-step distribution (HIP events around each step), after the timed loop
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    marks[0].record(s)
    for k in range(args.steps):
        opt.step()
        marks[k + 1].record(s)
    torch.cuda.synchronize()
    per_step = np.array([marks[k].elapsed_time(marks[k + 1]) for k in range(args.steps)])

    ns_ms = time_ns_stage(opt, reps=max(3, args.steps // 2))
    dk = time_dominant_kernel(opt, reps=max(3, args.steps // 2))
    gather_ms, untile_ms = time_io_stage(opt, reps=max(3, args.steps // 2))
    nsu_ms = time_ns_untile_stage(opt, reps=max(3, args.steps // 2))
    lds_step_ms = time_lds_step_stage(opt, reps=max(3, args.steps // 2))
    apply_ms = time_apply(opt, reps=max(3, args.steps // 2))
    flops = algorithmic_flops(opt)
    n_tiles = sum(g["tiles"].n_tiles for g in opt._groups)
    fams = sorted({ns_family(g["tiles"].mp, g["tiles"].np, rows=g["tiles"].m) for g in opt._groups})
    n_el = sum(p.numel() for p in params)
    # bytes per element: update (untile writes it, the WD/LR pass reads it), parameter;
    # fused: the untile reads the NS tile and reads and writes the parameter
    fused = all(g["tiles"].fused for g in opt._groups)
    ub = torch.empty(0, dtype=opt._groups[0]["tiles"].upd_dtype).element_size()
    pb = params[0].element_size()
    ns_tflops = flops / (ns_ms * 1e-3) / 1e12

    out = {
        "metric": "HiMuon step latency (ms) on one MI355X; NS5 TFLOP/s and % of bf16 MFMA peak",
        "value": round(wall_ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup,
        "ms_per_step": round(wall_ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": desc,
            "config": args.config,
            "matrices": len(params),
            "elements": n_el,
            "tiles": n_tiles,
            "tile_size": tile,
            "grad_dtype": "fp32",
            "param_dtype": str(pdtype).replace("torch.", ""),
        },
        "step_ms_events": round(ev_ms, 3),
        "step_ms_p25_p50_p75": [round(float(v), 3) for v in np.percentile(per_step, [25, 50, 75])],
        "ns5_ms": round(ns_ms, 3),
        "ns5_tflops": round(ns_tflops, 1),
        "ns5_frac_peak": round(ns_tflops / PEAK_BF16_TFLOPS, 4),
        "gather_ms": round(gather_ms, 3),
        "gather_gbs": round(14.0 * n_el / (gather_ms * 1e-3) / 1e9, 1),
        "untile_ms": round(untile_ms, 3),
        "untile_gbs": round(((2 + 2 * pb) if fused else (2 + ub)) * n_el / (untile_ms * 1e-3) / 1e9, 1),
        "untile_applies_wd_lr": fused,
        # NS5 + untile as the step runs them, the untile fused into the last
        # NS iteration of 512 x 512 buckets (ns5_ms and untile_ms above time
        # the two launches that this replaces)
        "ns5_untile_fused_ms": None if nsu_ms is None else round(nsu_ms, 3),
        # 128 x 128-tile buckets run the whole step as one LDS-resident launch
        # per chunk; ns5/gather/untile above then time the launches it replaces
        "lds_step_ms": None if lds_step_ms is None else round(lds_step_ms, 3),
        "apply_ms": round(apply_ms, 3),
        "apply_gbs": None if fused else round((2 * pb + ub) * n_el / (apply_ms * 1e-3) / 1e9, 1),
        "update_dtype": None if fused else str(opt._groups[0]["tiles"].upd_dtype).replace("torch.", ""),
        "ns5_stage_kernels": ("step: lds_step_kernel (momentum, gather, normaliser, NS5 and untile with "
                              "WD/LR of 128x128 tiles in one launch per chunk)" if lds_step_ms is not None
                              else "; ".join(NS_KERNELS[f] for f in fams)),
        # the dominant kernel, one launch on one sub-batch (HIP events)
        "roofline": kernel_roofline(args.config, dk),
    }
    if args.reconfigure:
        out["reconfigure"] = time_reconfigure(opt, args.reconfigure, args.steps)
    if not args.no_adamw:
        out["adamw"] = time_adamw(reps=max(3, args.steps // 2))
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(layers, shapes, tile, pdtype, args.cpu_budget)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

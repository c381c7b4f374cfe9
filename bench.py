"""Benchmark of the chunked FP16 GEMM on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A step is one f16acc_amd.mm call on inputs already resident in HBM.  Each
timed op first runs back to back for 0.2 s so the GPU clock has settled, then
W warm-up steps, then exactly K timed steps.  The
default workload is the headline one: M = N = K = 4096, A and B ~ N(0, 1)
cast to fp16, B row-major [K, N] (as the reference's bench/gemm_bench.py
passes it), fp16 output, chunk-32 with FP32 chunk sum and FP32 redo of
overflowing tiles (at this shape by a second launch that leaves at once when
no tile overflowed).  Prints one JSON line:
  value       TFLOPS of the timed steps (2 M N K per step)
  roofline    the GEMM kernel's achieved TFLOP/s (the kernel launched alone
              through f16acc_gemm, HIP events over its timed region on the
              launch stream) against the MI355X dense fp16 MFMA peak;
              traffic = HBM bytes per launch from the rocprofv3 FETCH_SIZE /
              WRITE_SIZE summary in profiles/, when present; call_us = per
              mm call, both launches
  cpu_baseline the reference algorithm (the CPU oracle) on this host's cores
  hipblaslt   torch.mm (hipBLASLt) on the same inputs and GPU
  max_rel_err_vs_fp64 / max_rel_err_vs_oracle  the reference's error metric
Other workloads (--workload) are sweeps for the design record, not bench lines;
--workload shapes reports every configured shape against hipBLASLt;
--workload redo_overhead times the shipped kernels against a build without the
overflow flag and redo on data that never overflows; --workload persistent_ab
times multi-round shapes on the persistent kernel against a build that runs
them one tile per workgroup; --workload
overflow_split_redo times the overflow stress workload against a build that
redoes flagged tiles in a split-K pass instead of in the same workgroup;
--workload table_check times the per-shape table against every forced tile on
llama-2-7B, llama-3-8B and Qwen2.5-7B layer shapes; --workload small_grid_check
times its small-grid picks (K-group tiles, 64x64) against the other candidates,
--workload large_grid_check its picks on grids of a round or more, --workload
estimate_ab the picks its partial-round estimates changed against the picks
before them; --tile-calls runs every tile
untimed for rocprofv3 counter passes.
"""

import argparse
import json
import os
import re
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = 2516.6  # MI355X dense fp16 MFMA: 256 CU x 2.4 GHz x 4096 flop/clk
METRIC = "TFLOPS at 4096³ fp16 GEMM (1 GPU, % of fp16 MFMA peak); max rel err vs FP64"
REF_TFLOPS = 65.7  # reference README.md:29, RTX 4060 Ti, same GEMM (fp16 out)
PREHEAT_S = 0.2  # seconds of back-to-back calls before the warm-up steps
# rocprofv3 HBM-counter summaries of the workloads that have one
TRAFFIC_PROFILES = {w: os.path.join(ROOT, "profiles", f"{f}_fp16out_rowmajorB_traffic.txt")
                    for w, f in (("gemm4096", "gemm_4096"), ("gemm8192", "gemm_8192"))}

WORKLOADS = {
    # name: (M, N, K, b_layout, out_dtype)
    "gemm1024_f32": (1024, 1024, 1024, "row", torch.float32),
    "gemm4096": (4096, 4096, 4096, "row", torch.float16),
    "gemm4096_bt": (4096, 4096, 4096, "t", torch.float16),
    "gemm4096_f32": (4096, 4096, 4096, "row", torch.float32),
    "gemm8192": (8192, 8192, 8192, "row", torch.float16),
    "gemm8192_bt": (8192, 8192, 8192, "t", torch.float16),
    "gemm8192_f32": (8192, 8192, 8192, "row", torch.float32),
    "qwen_qo": (2048, 1536, 1536, "t", torch.float16),
    "qwen_kv": (2048, 256, 1536, "t", torch.float16),
    "qwen_gateup": (2048, 8960, 1536, "t", torch.float16),
    "qwen_down": (2048, 1536, 8960, "t", torch.float16),
    "odd": (2049, 1537, 8961, "t", torch.float16),
    "qwen_lm_head": (2048, 151936, 1536, "t", torch.float16),
}


def make_inputs(M, N, K, layout, seed=0, device="cuda"):
    """Seeded CPU inputs (the oracle sees the same bits), copied to the GPU.
    layout "row": b is [K, N] row-major; "t": b is the w.t() view of [N, K]."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).half()
    if layout == "row":
        b = torch.randn(K, N, generator=g).half()
        gb = b.to(device)
    else:
        w = torch.randn(N, K, generator=g).half()
        b = w.t()
        gb = w.to(device).t()
    return a, b, a.to(device), gb


def preheat(op, seconds=None):
    """Run `op` back to back for about `seconds` of wall time.  From idle the
    MI355X's shader clock dips a few milliseconds into a load and takes
    ~15 ms to settle again (a 4096^3 GEMM: ~152 us per call, ~205 us in the
    dip): a window timed straight after a short warm-up measures that
    transient, for this kernel and hipBLASLt alike.  One call completes
    before the clock starts: torch.mm's first call sets hipBLASLt up for
    longer than the whole pre-heat."""
    seconds = PREHEAT_S if seconds is None else seconds
    op()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            op()
        torch.cuda.synchronize()


def time_steps(op, steps, warmup):
    """Pre-heat the clock, warm up, then time exactly `steps` calls between two
    synchronisations.  Returns (total seconds, event seconds on the current
    stream)."""
    preheat(op)
    for _ in range(warmup):
        op()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        op()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(stop) / 1e3


def read_traffic(workload):
    """HBM bytes per launch from the workload's committed rocprofv3 counter
    summary (None for a workload without one)."""
    if workload not in TRAFFIC_PROFILES:
        return None
    try:
        with open(TRAFFIC_PROFILES[workload]) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


# Host threads the CPU baseline uses: a one-GPU job on an eight-GPU MI355X
# node gets a 16-core share of its host, whatever os.cpu_count() reports.
CPU_SHARE = 16


def cpu_model():
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            m = re.search(r"^model name\s*:\s*(.+)$", f.read(), re.M)
        return m.group(1).strip() if m else None
    except OSError:
        return None


def cpu_baseline(a, b, out_dtype, budget_s=20.0):
    """The reference algorithm (oracle.chunk32, PyTorch on the CPU) on this
    host's cores: the full GEMM on the bench's own inputs, repeated (at most
    3 runs) while within budget, plus the median of 5 at 1024^3 fp32 out
    (the reference's CPU-runnable config).  Returns the baseline record and
    the oracle's result for the bench inputs."""
    from oracle import chunk32

    host = os.cpu_count() or 1
    threads = max(1, min(CPU_SHARE, host))
    torch.set_num_threads(threads)
    M, K = a.shape
    N = b.shape[1]
    times, ref = [], None
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start + times[-1] < budget_s and len(times) < 3):
        t0 = time.perf_counter()
        ref = chunk32.mm(a, b, out_dtype)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    g = torch.Generator().manual_seed(0)
    a1, b1 = torch.randn(1024, 1024, generator=g).half(), torch.randn(1024, 1024, generator=g).half()
    t1 = []
    for _ in range(5):
        t0 = time.perf_counter()
        chunk32.mm(a1, b1, torch.float32)
        t1.append(time.perf_counter() - t0)
    t1 = statistics.median(t1)
    info = {"value": 2.0 * M * N * K / t / 1e12, "unit": "TFLOPS", "cores": threads, "kind": "port",
            "host_cpus": host, "cpu_model": cpu_model(),
            "thread_cap": f"{CPU_SHARE}: one GPU's share of the node's host CPUs",
            "sample": f"the full {M}x{N}x{K} GEMM (oracle/chunk32.py, torch CPU, {threads} threads), "
                      f"median of {len(times)} run(s), {t:.2f} s each",
            "gemm1024_f32": {"value": round(2.0 * 1024 ** 3 / t1 / 1e12, 4), "unit": "TFLOPS",
                             "ms": round(t1 * 1e3, 2), "runs": 5, "stat": "median"}}
    return info, ref


def sweep_tiles(names, rounds=5):
    """Time every tile configuration (forced) on the given workloads, chunked,
    next to the op as shipped (table choice, packing included) and hipBLASLt:
    the evidence behind the per-shape table, as the reference's autotuner
    times its CONFIGS (f16acc/kernel.py:16-19).  The candidates are timed in
    interleaved rounds (3 warm-up + 5 timed calls each, median over rounds)
    so the GPU's power-state drift falls on all of them alike."""
    import f16acc_amd
    from f16acc_amd import _lib
    from f16acc_amd.kernel import mm_tile, tile_config

    for name in names:
        M, N, K, layout, out_dtype = WORKLOADS[name]
        _, _, a, b = make_inputs(M, N, K, layout)
        flops = 2.0 * M * N * K
        ops = {tile: (lambda t=tile: mm_tile(a, b, t, out_dtype)) for tile in _lib.TILES
               if tile_config(a, b, tile)["tile"] == tile}  # tiles the operands allow
        ops["mm"] = lambda: f16acc_amd.mm(a, b, out_dtype)
        ops["hipblaslt"] = lambda: torch.mm(a, b)
        times = {k: [] for k in ops}
        for r in range(rounds):
            for k in round_order(list(ops), r):
                times[k].append(burst_time(ops[k]))
        row = {"workload": name, "M": M, "N": N, "K": K, "b": layout, "table": tile_config(a, b)["tile"]}
        row.update({k: round(flops / statistics.median(v) / 1e12, 1) for k, v in times.items()})
        print(json.dumps(row), flush=True)
        del a, b
        torch.cuda.empty_cache()


def tile_calls(names, calls):
    """`calls` calls of every tile configuration the operands allow (forced),
    of mm as shipped and of hipBLASLt on each workload, one after another with
    a synchronisation between them and no timing: a run for rocprofv3 --pmc,
    which reads each kernel's counters (MFMA busy cycles, LDS instructions,
    HBM bytes) per dispatch."""
    import f16acc_amd
    from f16acc_amd import _lib
    from f16acc_amd.kernel import mm_tile, tile_config

    for name in names:
        M, N, K, layout, out_dtype = WORKLOADS[name]
        _, _, a, b = make_inputs(M, N, K, layout)
        ops = {tile: (lambda t=tile: mm_tile(a, b, t, out_dtype)) for tile in _lib.TILES
               if tile_config(a, b, tile)["tile"] == tile}
        ops["mm"] = lambda: f16acc_amd.mm(a, b, out_dtype)
        ops["hipblaslt"] = lambda: torch.mm(a, b)
        for op in ops.values():
            for _ in range(calls):
                op()
            torch.cuda.synchronize()
        print(json.dumps({"workload": name, "M": M, "N": N, "K": K, "b": layout, "table": tile_config(a, b)["tile"],
                          "ops": list(ops), "calls": calls}), flush=True)
        del a, b
        torch.cuda.empty_cache()


# Transformer layer shapes the per-shape table was checked on (the Qwen2.5-1.5B
# ones are WORKLOADS): (model, hidden size, k/v width, MLP width)
LLM_MODELS = (("llama2-7b", 4096, 4096, 11008), ("llama3-8b", 4096, 1024, 14336), ("qwen2.5-7b", 3584, 512, 18944))


def table_check(tokens=(256, 1024, 4096), rounds=4):
    """The per-shape table against every forced tile on the layer GEMMs of
    LLM_MODELS at several token counts (x [M, K] @ w.t(), w [N, K] ~ N(0, 0.02),
    fp16 out, chunked): per-call times in settled bursts (median of interleaved
    rounds), the table's pick
    (split along K and ragged-round cuts included) next to each tile alone.
    Prints one JSON line per shape and a summary line."""
    import f16acc_amd
    from f16acc_amd import _lib
    from f16acc_amd.kernel import mm_tile, tile_config

    tiles = [t for t in _lib.TILES if t != "generic"]
    ratios = []
    for model, d, kv, ffn in LLM_MODELS:
        for M in tokens:
            for layer, N, K in (("q/o", d, d), ("k/v", kv, d), ("gate/up", ffn, d), ("down", d, ffn)):
                g = torch.Generator().manual_seed(0)
                a = torch.randn(M, K, generator=g).half().cuda()
                b = (torch.randn(N, K, generator=g) * 0.02).half().cuda().t()
                ops = {"table": lambda: f16acc_amd.mm(a, b)}
                ops.update({tile: (lambda x=tile: mm_tile(a, b, x)) for tile in tiles})
                runs = {k: [] for k in ops}
                names = list(ops)
                for r in range(rounds):  # interleaved, so clock drift falls on all alike
                    for k in round_order(names, r):
                        runs[k].append(settled_time(ops[k]))
                t = {k: statistics.median(v) for k, v in runs.items()}
                best = min(tiles, key=lambda k: t[k])
                ratios.append(t[best] / t["table"])
                print(json.dumps({"model": model, "layer": layer, "M": M, "N": N, "K": K,
                                  "pick": tile_config(a, b)["tile"], "table_us": round(t["table"] * 1e6, 1),
                                  "best_forced": best, "best_forced_us": round(t[best] * 1e6, 1),
                                  "best_forced_over_table": round(ratios[-1], 3),
                                  **{k: round(v * 1e6, 1) for k, v in t.items() if k != "table"}}), flush=True)
                del a, b
    print(json.dumps({"shapes": len(ratios), "table_at_least_as_fast": sum(r >= 0.999 for r in ratios),
                      "within_5pct_of_best_forced": sum(r >= 0.95 for r in ratios),
                      "worst_best_forced_over_table": round(min(ratios), 3)}), flush=True)


def large_grid_check(rounds=3):
    """The table's pick against every fast tile (forced) on grids of at
    least one round: x [M, K] @ w.t() over M 1024..8192, N 1024..16384,
    K 1024 and 4096, wherever the table picks a 256-row or 128x128 tile.
    mm as shipped is timed too ("table": with the ragged-round cut and the
    deferred redo launch where it plans them).  Per-call times in settled
    bursts, median of rounds whose order rotates; one JSON line per shape
    and a summary."""
    import itertools

    import f16acc_amd
    from f16acc_amd import _lib
    from f16acc_amd.kernel import mm_tile, tile_config

    cands = [t for t in _lib.TILES if t not in ("generic", "128x96k2", "64x32k4")]
    ratios = []
    for M, N, K in itertools.product((1024, 2048, 3072, 4096, 6144, 8192), (1024, 3072, 5120, 9216, 16384),
                                     (1024, 4096)):
        g = torch.Generator().manual_seed(0)
        a = torch.randn(M, K, generator=g).half().cuda()
        b = (torch.randn(N, K, generator=g) * 0.02).half().cuda().t()
        pick = tile_config(a, b)["tile"]
        if pick not in ("256x256", "256x288", "256x128", "128x256", "128x128"):
            continue
        ops = {"table": lambda: f16acc_amd.mm(a, b)}
        ops.update({t: (lambda x=t: mm_tile(a, b, x)) for t in cands})
        names = list(ops)
        runs = {k: [] for k in ops}
        for r in range(rounds):
            for k in round_order(names, r):
                runs[k].append(settled_time(ops[k], burst_ms=25.0))
        t = {k: statistics.median(v) for k, v in runs.items()}
        best = min(cands, key=lambda k: t[k])
        ratios.append(t[best] / t["table"])
        print(json.dumps({"M": M, "N": N, "K": K, "pick": pick, "table_us": round(t["table"] * 1e6, 1),
                          "best_forced": best, "best_forced_over_table": round(ratios[-1], 3),
                          **{k: round(v * 1e6, 1) for k, v in t.items() if k != "table"}}), flush=True)
        del a, b
    print(json.dumps({"shapes": len(ratios), "table_at_least_as_fast": sum(r >= 0.999 for r in ratios),
                      "within_5pct": sum(r >= 0.95 for r in ratios), "within_10pct": sum(r >= 0.90 for r in ratios),
                      "worst_best_forced_over_table": round(min(ratios), 3)}), flush=True)


def small_grid_check(rounds=3):
    """The table's pick against 128x96 in two K groups, 64x32 in four, 64x64
    and 128x128 (each forced) on grids that leave CUs idle: x [M, K] @ w.t()
    over M 256..4096, N 256..5120, K 1024..8192 and a second grid of other
    extents, wherever the table picks a K-group tile or 64x64 (the region of
    its small-grid rules).  Per-call times in settled bursts, median of
    rounds whose order rotates; one JSON line per shape and a summary."""
    import itertools

    import f16acc_amd
    from f16acc_amd.kernel import mm_tile, tile_config

    cands = ["128x96k2", "64x32k4", "64x64", "128x128"]
    grid = list(itertools.product((256, 512, 1024, 1536, 2048, 3072, 4096), (256, 512, 1024, 1536, 2816, 5120),
                                  (1024, 1536, 4096, 8192)))
    grid += list(itertools.product((384, 768, 1280, 2560), (384, 768, 1280, 2048), (1280, 2048, 2816, 5120)))
    ratios = []
    for M, N, K in grid:
        g = torch.Generator().manual_seed(0)
        a = torch.randn(M, K, generator=g).half().cuda()
        b = (torch.randn(N, K, generator=g) * 0.02).half().cuda().t()
        pick = tile_config(a, b)["tile"]
        if pick not in ("128x96k2", "64x32k4", "64x64"):
            continue
        ops = {"table": lambda: f16acc_amd.mm(a, b)}
        ops.update({t: (lambda x=t: mm_tile(a, b, x)) for t in cands})
        names = list(ops)
        runs = {k: [] for k in ops}
        for r in range(rounds):
            for k in round_order(names, r):
                runs[k].append(settled_time(ops[k], burst_ms=20.0))
        t = {k: statistics.median(v) for k, v in runs.items()}
        best = min(cands, key=lambda k: t[k])
        ratios.append(t[best] / t[pick])
        print(json.dumps({"M": M, "N": N, "K": K, "pick": pick, "pick_forced_us": round(t[pick] * 1e6, 2),
                          "best_forced": best, "best_forced_over_pick": round(ratios[-1], 3),
                          **{k: round(v * 1e6, 2) for k, v in t.items()}}), flush=True)
        del a, b
    print(json.dumps({"shapes": len(ratios), "pick_is_best": sum(r >= 0.999 for r in ratios),
                      "within_5pct": sum(r >= 0.95 for r in ratios), "within_10pct": sum(r >= 0.90 for r in ratios),
                      "worst_best_forced_over_pick": round(min(ratios), 3)}), flush=True)


def round_order(names, r):
    """The order ops are timed in round r: the list rotated by r, and
    reversed in every other pass through the rotations, so over the rounds
    each op is timed first as often as any other, within one (the op timed
    first after another one runs ~2-5 % slow: kernel times keep falling for
    tens of ms after a switch, and a fixed order charges that to one op)."""
    n = len(names)
    shift = r % n
    order = list(names[shift:]) + list(names[:shift])
    return order[::-1] if (r // n) % 2 else order


def settled_time(op, burst_ms=40.0):
    """Seconds per call in the second half of a ~burst_ms back-to-back burst
    (HIP events): the first half lets the clock settle after the previous op."""
    op()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    op()
    e.record()
    torch.cuda.synchronize()
    n = max(10, int(burst_ms / max(s.elapsed_time(e), 0.01)))
    for _ in range(n // 2):
        op()
    s.record()
    for _ in range(n - n // 2):
        op()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / 1e3 / (n - n // 2)


def shapes_report(names, rounds=4):
    """TFLOPS at every configured shape, as absolute numbers and as a fraction
    of the MI355X dense fp16 MFMA peak: mm as shipped (chunked, the per-shape
    table, packing and split-K included), its FP32-accumulate mode, and
    hipBLASLt (torch.mm, fp16 out) on the same inputs, timed in interleaved
    ~40 ms bursts (median over rounds of each burst's settled second half),
    plus mm's max relative error against an FP64 GEMM of the same inputs."""
    import f16acc_amd
    from f16acc_amd.kernel import tile_config

    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    rows = []
    for name in names:
        M, N, K, layout, out_dtype = WORKLOADS[name]
        _, _, a, b = make_inputs(M, N, K, layout)
        flops = 2.0 * M * N * K
        ops = {"mm": lambda: f16acc_amd.mm(a, b, out_dtype),
               "fp32acc": lambda: f16acc_amd.mm(a, b, out_dtype, chunked=False),
               "hipblaslt": lambda: torch.mm(a, b)}
        times = {k: [] for k in ops}
        for r in range(rounds):
            for k in round_order(list(ops), r):
                times[k].append(settled_time(ops[k]))
        c = f16acc_amd.mm(a, b, out_dtype)
        ref = a.double() @ b.double()
        err = ((c.double() - ref).abs().max() / ref.abs().max()).item()
        del c, ref
        import ctypes

        from f16acc_amd import _lib

        nsplit = ctypes.c_int64()
        _lib.check(_lib.tail_split(M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), a.data_ptr(),
                                   b.data_ptr(), ctypes.byref(nsplit)))
        table = tile_config(a, b)["tile"]
        if nsplit.value > 0:
            table = f"256x256 for n < {nsplit.value}, then {tile_config(a, b[:, nsplit.value:])['tile']}"
        elif nsplit.value < 0:
            table = f"256x256 for m < {-nsplit.value}, then {tile_config(a[-nsplit.value:], b)['tile']}"
        row = {"workload": name, "M": M, "N": N, "K": K, "b": "row-major [K,N]" if layout == "row" else "w.t()",
               "out": "fp16" if out_dtype == torch.float16 else "fp32", "table": table,
               "max_rel_err_vs_fp64": float(f"{err:.3g}")}
        for k, v in times.items():
            t = statistics.median(v)
            row[k] = {"us": round(t * 1e6, 1), "tflops": round(flops / t / 1e12, 1),
                      "frac_of_peak": round(flops / t / 1e12 / PEAK_TFLOPS, 3)}
        row["mm_vs_hipblaslt"] = round(row["hipblaslt"]["us"] / row["mm"]["us"], 3)
        print(json.dumps(row), flush=True)
        rows.append(row)
        del a, b
        torch.cuda.empty_cache()
    print("\n| shape | out | B | table tile | mm us | mm TFLOPS | frac of peak | FP32-acc TFLOPS | hipBLASLt TFLOPS |"
          " mm / hipBLASLt | max rel err vs FP64 |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for r in rows:
        print(f"| {r['M']}x{r['N']}x{r['K']} | {r['out']} | {r['b']} | {r['table']} | {r['mm']['us']} | "
              f"{r['mm']['tflops']} | {r['mm']['frac_of_peak']} | {r['fp32acc']['tflops']} | "
              f"{r['hipblaslt']['tflops']} | {r['mm_vs_hipblaslt']} | {r['max_rel_err_vs_fp64']:.2e} |")


def burst_time(op, warmup=3, calls=5):
    """Seconds per call over a short back-to-back burst (HIP events)."""
    for _ in range(warmup):
        op()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(calls):
        op()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / 1e3 / calls


def overflow_inputs(n=4096, blocks=7, block=128, seed=0):
    """Overflow stress GEMM: a, b ~ N(0, 1) fp16 (b row-major [K, N]) with
    `blocks` of the n/block row-blocks of a and column-blocks of b set to
    U(200, 255), chosen from the seed.  Their intersection tiles (7 x 7 of
    32 x 32 = 4.8 % of 128 x 128 tiles) have 32-term chunk sums near
    32 * 227^2 = 1.65e6 > 65504, inf in fp16, so they are flagged and redone
    in FP32; row-only or column-only blocks stay near 1.3e3."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(n, n, generator=g)
    b = torch.randn(n, n, generator=g)
    nb = n // block
    rows = torch.randperm(nb, generator=g)[:blocks].tolist()
    cols = torch.randperm(nb, generator=g)[:blocks].tolist()
    for r in rows:
        a[r * block:(r + 1) * block] = 200.0 + 55.0 * torch.rand(block, n, generator=g)
    for c in cols:
        b[:, c * block:(c + 1) * block] = 200.0 + 55.0 * torch.rand(n, block, generator=g)
    return a.half(), b.half(), sorted(rows), sorted(cols)


def overflow_bench(steps, warmup):
    """Overflow stress workload: chunked time with ~5 % of tiles redone in
    FP32, the same call on the no-overflow data, flagged tiles, and the check
    that every redone tile equals the FP32-accumulate mode (same tile, K not
    split) bit for bit."""
    import f16acc_amd
    from f16acc_amd.kernel import mm_flags, mm_tile, tile_config

    a_cpu, b_cpu, rows, cols = overflow_inputs()
    a, b = a_cpu.cuda(), b_cpu.cuda()
    M, K = a.shape
    N = b.shape[1]
    flops = 2.0 * M * N * K
    cfg = tile_config(a, b)
    _, ev = time_steps(lambda: f16acc_amd.mm(a, b, torch.float32), steps, warmup)
    t_over = ev / steps
    c, flags = mm_flags(a, b, torch.float32)
    c32 = mm_tile(a, b, cfg["tile"], torch.float32, chunked=False)  # unsplit: the redo's summation order
    _, _, ca, cb = make_inputs(M, N, K, "row")
    _, ev = time_steps(lambda: f16acc_amd.mm(ca, cb, torch.float32), steps, warmup)
    t_clean = ev / steps
    bm, bn = cfg["bm"], cfg["bn"]
    fl = flags.cpu().bool()
    # the tiles an overflowing 128-row block meets on this tile grid
    want = {(r * 128 // bm + i, q * 128 // bn + j) for r in rows for q in cols
            for i in range(max(1, 128 // bm)) for j in range(max(1, 128 // bn))}
    mask = fl.repeat_interleave(bm, 0).repeat_interleave(bn, 1)[:M, :N].cuda()
    redone_exact = bool(torch.equal(c[mask], c32[mask]))
    ref = a.double() @ b.double()
    keep = ~mask
    err_other = ((c.double() - ref).abs()[keep].max() / ref.abs()[keep].max()).item()
    line = {"workload": "overflow stress 4096^3, fp32 out, B row-major", "tile": cfg["tile"],
            "tiles": cfg["tiles_m"] * cfg["tiles_n"], "flagged_tiles": int(fl.sum()),
            "flagged_are_the_block_intersections": {tuple(t) for t in fl.nonzero().tolist()} == want,
            "us_with_overflow": round(t_over * 1e6, 2), "us_without_overflow": round(t_clean * 1e6, 2),
            "tflops_with_overflow": round(flops / t_over / 1e12, 1),
            "tflops_without_overflow": round(flops / t_clean / 1e12, 1),
            "redone_tiles_equal_fp32_mode": redone_exact, "max_rel_err_other_tiles_vs_fp64": err_other,
            "rows": rows, "cols": cols}
    print(json.dumps(line), flush=True)


def overflow_split_redo(rounds=5):
    """The overflow stress workload through three redo schemes, on the stress
    data and on its no-overflow twin, with the same inputs, timed in
    interleaved settled bursts (median over rounds):
      in_place  f16acc_gemm (no workspace): each flagged tile redone in FP32 by
                its own workgroup, a straggler on its CU;
      deferred  f16acc_gemm_ws (the entry mm uses): flagged tiles listed in the
                workspace header and redone by a second launch as 128x128
                quarters, one workgroup each;
      split     libf16acc_amd_splitredo.so (-DF16ACC_SPLIT_REDO=1, loaded
                here only): the chunked launch only flags; flagged tiles are
                recomputed as 128x128 tiles split three ways along K, plus a
                finishing launch.
    Checks: the same flags; unflagged tiles bit-equal; redone tiles against
    the FP32-accumulate mode (the split sums its three K ranges after)."""
    import ctypes

    from f16acc_amd import _lib, build
    from f16acc_amd.kernel import mm_tile, tile_config

    split = ctypes.CDLL(build.LIB_SPLITREDO)
    g_split = split.f16acc_gemm
    g_split.argtypes, g_split.restype = _lib.gemm.argtypes, _lib.gemm.restype
    a_cpu, b_cpu, rows, cols = overflow_inputs()
    data = {"overflow": (a_cpu.cuda(), b_cpu.cuda())}
    _, _, ca, cb = make_inputs(a_cpu.shape[0], b_cpu.shape[1], a_cpu.shape[1], "row")
    data["clean"] = (ca, cb)
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(_lib.WS_HEADER, dtype=torch.uint8, device="cuda")
    ws.zero_()
    out = {}
    times = {}
    for dname, (a, b) in data.items():
        M, K = a.shape
        N = b.shape[1]
        cfg = tile_config(a, b)
        for lname, fn in (("in_place", _lib.gemm), ("deferred", None), ("split", g_split)):
            c = torch.empty(M, N, device="cuda", dtype=torch.float32)
            fl = torch.zeros(cfg["tiles_m"] * cfg["tiles_n"], device="cuda", dtype=torch.uint8)

            def call(c=c, fl=None, fn=fn, a=a, b=b):
                args = (M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1),
                        _lib.OUT_F32, 1, st)
                if fn is None:
                    _lib.check(_lib.gemm_ws(a.data_ptr(), b.data_ptr(), None, c.data_ptr(), fl, *args, ws.data_ptr(),
                                            ws.numel()))
                else:
                    _lib.check(fn(a.data_ptr(), b.data_ptr(), c.data_ptr(), fl, *args))

            call(fl=fl.data_ptr())
            torch.cuda.synchronize()
            out[(dname, lname)] = (c.clone(), fl.clone())
            times[(dname, lname)] = (call, [])
    for _ in range(rounds):  # interleaved, so clock drift falls on all alike
        for key, (call, ts) in times.items():
            ts.append(settled_time(call))
    a, b = data["overflow"]
    cfg = tile_config(a, b)
    c_in, f_in = out[("overflow", "in_place")]
    c32 = mm_tile(a, b, cfg["tile"], torch.float32, chunked=False)
    bm, bn = cfg["bm"], cfg["bn"]
    M, N = c_in.shape
    mask = f_in.view(cfg["tiles_m"], cfg["tiles_n"]).bool().repeat_interleave(bm, 0).repeat_interleave(bn, 1)[:M, :N]
    ref = c32[mask].double()
    us = {f"{d}_{l}_us": round(statistics.median(ts) * 1e6, 2) for (d, l), (_, ts) in times.items()}
    clean = us["clean_in_place_us"]
    line = {"workload": "overflow stress 4096^3, fp32 out, B row-major: redo in place vs deferred list vs split",
            "tile": cfg["tile"], "flagged_tiles": int(f_in.sum()),
            "same_flags": all(torch.equal(out[("overflow", k)][1], f_in) for k in ("deferred", "split")), **us,
            **{f"overflow_cost_{k}_pct": round((us[f"overflow_{k}_us"] / clean - 1) * 100, 1)
               for k in ("in_place", "deferred", "split")},
            **{f"clean_cost_{k}_pct": round((us[f"clean_{k}_us"] / clean - 1) * 100, 1) for k in ("deferred", "split")},
            "unflagged_bit_equal": all(torch.equal(out[("overflow", k)][0][~mask], c_in[~mask])
                                       for k in ("deferred", "split")),
            "in_place_and_deferred_redone_equal_fp32_mode": bool(torch.equal(c_in[mask], c32[mask]) and
                                                                 torch.equal(out[("overflow", "deferred")][0][mask],
                                                                             c32[mask])),
            "split_redone_max_rel_diff_vs_fp32_mode": ((out[("overflow", "split")][0][mask].double() - ref).abs().max()
                                                       / ref.abs().max()).item(),
            "clean_outputs_bit_equal": all(torch.equal(out[("clean", k)][0], out[("clean", "in_place")][0])
                                           for k in ("deferred", "split"))}
    print(json.dumps(line), flush=True)


# Shapes of the redo-overhead A/B: the overflow stress config's no-overflow
# twin (4096^3, A and B ~ N(0, 1), fp32 out), the 8192^3 square GEMM and the
# Qwen2.5-1.5B layers at 2048 tokens (the K-group tiles, 256x288).
REDO_SHAPES = (("gemm4096_f32", 4096, 4096, 4096, "row", torch.float32),
               ("gemm8192", 8192, 8192, 8192, "row", torch.float16),
               ("qwen_qo", 2048, 1536, 1536, "t", torch.float16),
               ("qwen_kv", 2048, 256, 1536, "t", torch.float16),
               ("qwen_gateup", 2048, 8960, 1536, "t", torch.float16),
               ("qwen_down", 2048, 1536, 8960, "t", torch.float16))


def twin_ab(lib_path, shapes, rounds, shipped="shipped", twin="twin"):
    """f16acc_gemm_ws (the entry mm uses: split-K where the table splits) of
    the shipped library against the same source built with a -D switch
    (lib_path, loaded here only), through the C ABI on the same inputs, timed
    in interleaved settled bursts (median over rounds, the two taking turns at
    going first); both return the same bits on these inputs.  Yields one
    record per shape."""
    import ctypes

    from f16acc_amd import _lib

    other = ctypes.CDLL(lib_path)
    gemm_other = other.f16acc_gemm_ws
    gemm_other.argtypes, gemm_other.restype = _lib.gemm_ws.argtypes, _lib.gemm_ws.restype
    # every split on 256 CUs fits; the header (deferred redo list) starts empty
    ws = torch.empty((32 << 20) + _lib.WS_HEADER, dtype=torch.uint8, device="cuda")
    ws[:_lib.WS_HEADER].zero_()
    for name, M, N, K, layout, out_dtype in shapes:
        _, _, a, b = make_inputs(M, N, K, layout)
        outs = {k: torch.empty(M, N, device="cuda", dtype=out_dtype) for k in (shipped, twin)}
        stream = torch.cuda.current_stream().cuda_stream
        code = _lib.OUT_F32 if out_dtype == torch.float32 else _lib.OUT_F16

        def call(fn, c):
            return lambda: _lib.check(fn(a.data_ptr(), b.data_ptr(), None, c.data_ptr(), None, M, N, K, a.stride(0),
                                         a.stride(1), b.stride(0), b.stride(1), c.stride(0), c.stride(1), code, 1,
                                         stream, ws.data_ptr(), ws.numel()))

        ops = {shipped: call(_lib.gemm_ws, outs[shipped]), twin: call(gemm_other, outs[twin])}
        for op in ops.values():
            op()
        torch.cuda.synchronize()
        same = bool(torch.equal(outs[shipped], outs[twin]))
        times = {k: [] for k in ops}
        for r in range(rounds):
            for k in round_order(list(ops), r):
                times[k].append(settled_time(ops[k]))
        t = {k: statistics.median(v) for k, v in times.items()}
        yield {"workload": name, "M": M, "N": N, "K": K, "b": "row-major [K,N]" if layout == "row" else "w.t()",
               "out": "fp32" if out_dtype == torch.float32 else "fp16",
               f"us_{shipped}": round(t[shipped] * 1e6, 2), f"us_{twin}": round(t[twin] * 1e6, 2),
               "tflops": round(2 * M * N * K / t[shipped] / 1e12, 1),
               "pct": round((t[shipped] / t[twin] - 1) * 100, 2),
               "per_round_pct": [round((x / y - 1) * 100, 2) for x, y in zip(times[shipped], times[twin])],
               "same_bits": same, "rounds": rounds}
        del a, b, outs
        torch.cuda.empty_cache()


def redo_overhead(rounds=7):
    """What the overflow flag and the in-kernel FP32 redo cost when no tile
    overflows: the shipped library against the same source built with both
    compiled out (libf16acc_amd_noredo.so, -DF16ACC_NO_REDO=1).  Both must
    return the same bits on this data (no tile overflows).  The reference
    calls an in-kernel redo 8 % slower and a separate one "nearly free"
    (f16acc/kernel.py:6-9, README.md:20)."""
    from f16acc_amd import build

    for rec in twin_ab(build.LIB_NOREDO, REDO_SHAPES, rounds, twin="no_redo"):
        rec["redo_overhead_pct"] = rec.pop("pct")
        print(json.dumps(rec), flush=True)


PERSISTENT_SHAPES = (("qwen_lm_head", 2048, 151936, 1536, "t", torch.float16),
                     ("gemm8192", 8192, 8192, 8192, "row", torch.float16),
                     ("gemm8192_bt", 8192, 8192, 8192, "t", torch.float16),
                     ("gemm8192_f32", 8192, 8192, 8192, "row", torch.float32),
                     ("llama3_gateup_4096tok", 4096, 14336, 4096, "t", torch.float16),
                     ("llama2_lm_head_4096tok", 4096, 32000, 4096, "t", torch.float16))


# Shapes whose plan the partial-round estimates of the tile table changed,
# with the tile the table picked before them (M, N, K, b layout, old pick).
ESTIMATE_SHAPES = ((4096, 3072, 4096, "row", "128x128"), (4096, 3072, 4096, "t", "128x128"),
                   (8192, 1536, 1536, "row", "128x128"), (5888, 9216, 4096, "row", "128x128"),
                   (256, 1024, 2048, "row", "128x128"), (1024, 1024, 2048, "row", "128x128"),
                   (4096, 512, 2048, "row", "128x128"), (256, 4096, 2560, "row", "128x128"),
                   (3072, 1024, 4096, "row", "128x128"), (3072, 1024, 4096, "t", "128x128"),
                   (2048, 1536, 3072, "row", "128x128"), (768, 4096, 3072, "t", "128x128"),
                   (256, 11008, 8192, "row", "128x128"), (512, 6144, 14336, "row", "128x128"))


def estimate_ab(rounds=4):
    """mm as shipped against the plan the table made before it priced
    partial rounds of 128x128 (a lone last round) and 64x64 (a single round
    of three or fewer workgroups per CU): that pick forced through
    f16acc_gemm_tile_ws, which plans its K split as before and makes no
    ragged-round cut.  Per-call times in settled bursts, median of rounds
    whose order alternates; fp16 out.  pct < 0: the new plan is faster."""
    import ctypes

    import f16acc_amd
    from f16acc_amd import _lib
    from f16acc_amd.kernel import tile_config

    ws = torch.empty((32 << 20) + _lib.WS_HEADER, dtype=torch.uint8, device="cuda")
    ws[:_lib.WS_HEADER].zero_()
    for M, N, K, layout, old in ESTIMATE_SHAPES:
        _, _, a, b = make_inputs(M, N, K, layout)
        c_old = torch.empty(M, N, device="cuda", dtype=torch.float16)
        stream = torch.cuda.current_stream().cuda_stream
        args = (a.data_ptr(), b.data_ptr(), c_old.data_ptr(), None, M, N, K, a.stride(0), a.stride(1), b.stride(0),
                b.stride(1), c_old.stride(0), c_old.stride(1), _lib.OUT_F16, 1, stream, _lib.TILES.index(old),
                ws.data_ptr(), ws.numel())
        ops = {"new": lambda: f16acc_amd.mm(a, b), "old": lambda: _lib.check(_lib.gemm_tile_ws(*args))}
        times = {k: [] for k in ops}
        for r in range(rounds):
            for k in round_order(list(ops), r):
                times[k].append(settled_time(ops[k]))
        t = {k: statistics.median(v) * 1e6 for k, v in times.items()}
        print(json.dumps({"M": M, "N": N, "K": K, "b": layout, "pick_new": tile_config(a, b)["tile"], "pick_old": old,
                          "us_new": round(t["new"], 2), "us_old": round(t["old"], 2),
                          "pct": round((t["new"] / t["old"] - 1) * 100, 2)}), flush=True)
        del a, b, c_old
        torch.cuda.empty_cache()


def persistent_ab(rounds=5):
    """Multi-round shapes on the persistent 256x256 kernel (the shipped
    library) against the one-tile-per-workgroup grid
    (libf16acc_amd_nopersist.so, -DF16ACC_NO_PERSISTENT=1): pct < 0 means the
    persistent kernel is faster."""
    from f16acc_amd import build

    for rec in twin_ab(build.LIB_NOPERSIST, PERSISTENT_SHAPES, rounds, twin="grid"):
        print(json.dumps(rec), flush=True)


def qwen2_model(layers=28, seed=0, dtype=torch.float16):
    """Random-init Qwen2.5-1.5B architecture on the GPU: hidden 1536, SwiGLU
    8960, 12 query / 2 KV heads (head_dim 128), RMSNorm eps 1e-6, RoPE theta
    1e6, vocab 151936, tied embeddings, weights N(0, 0.02) (the library's
    initializer; biases start at 0).  No checkpoint is read."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(hidden_size=1536, intermediate_size=8960, num_hidden_layers=layers, num_attention_heads=12,
                      num_key_value_heads=2, rms_norm_eps=1e-6,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6}, vocab_size=151936,
                      tie_word_embeddings=True, initializer_range=0.02, max_position_embeddings=32768)
    torch.manual_seed(seed)
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg)
    return model.to(dtype).eval()


def qwen2_prefill_ab(layers=28, tokens=2048, seed=0, reps=5):
    """Prefill A/B on the random-init model, batch 1, seeded random tokens:
    logits of the unpatched FP16 model (hipBLASLt) and of the patched one
    (every nn.Linear through f16acc_amd.mm), each against an FP32 run of the
    same weights.  Returns top-1 agreement, mean next-token cross-entropy and
    prefill time; the analogue of the reference's bench/llm.py:33-64 without
    the checkpoint download."""
    import torch.nn.functional as F

    import f16acc_amd
    from f16acc_amd import patch

    ids = torch.randint(0, 151936, (1, tokens), generator=torch.Generator().manual_seed(seed)).cuda()
    model = qwen2_model(layers, seed, torch.float32)

    def run():
        with torch.no_grad():
            return model(ids).logits[0].float()

    def timed():
        """Median wall time of a forward, and of its host part alone (the
        launches, until the forward returns before the sync): the forward
        is GPU-bound when the host part is the shorter."""
        ts, hs = [], []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            run()
            hs.append(time.perf_counter() - t0)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), statistics.median(hs)

    ref = run()
    model.half()
    base = run()
    t_base, h_base = timed()
    for k in patch.calls:
        patch.calls[k] = 0
    f16acc_amd.enable()
    try:
        ours = run()
        n_calls = dict(patch.calls)
        t_ours, h_ours = timed()
    finally:
        f16acc_amd.disable()
    tgt = ids[0, 1:]

    def ce(lg):
        return F.cross_entropy(lg[:-1], tgt).item()

    top = {n: lg.argmax(-1) for n, lg in (("ref", ref), ("base", base), ("ours", ours))}
    return {"layers": layers, "tokens": tokens,
            "top1_patched_vs_unpatched": (top["ours"] == top["base"]).float().mean().item(),
            "top1_unpatched_vs_fp32": (top["base"] == top["ref"]).float().mean().item(),
            "top1_patched_vs_fp32": (top["ours"] == top["ref"]).float().mean().item(),
            "mean_ce_fp32": ce(ref), "mean_ce_unpatched": ce(base), "mean_ce_patched": ce(ours),
            "max_abs_logit_diff_patched_vs_fp32": (ours - ref).abs().max().item(),
            "max_abs_logit_diff_unpatched_vs_fp32": (base - ref).abs().max().item(),
            "calls_in_one_forward": n_calls,
            "prefill_ms_unpatched": round(t_base * 1e3, 2), "prefill_ms_patched": round(t_ours * 1e3, 2),
            "host_launch_ms_unpatched": round(h_base * 1e3, 2), "host_launch_ms_patched": round(h_ours * 1e3, 2),
            "tokens_per_s_unpatched": round(tokens / t_base, 1), "tokens_per_s_patched": round(tokens / t_ours, 1)}


def copy_reference(steps, warmup, nbytes=1 << 30):
    """A plain device copy of known size (1 GiB read + 1 GiB written per step):
    the calibration for rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.ones(nbytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    wall, ev = time_steps(lambda: dst.copy_(src), steps, warmup)
    print(json.dumps({"workload": "copy", "bytes_read_per_step": nbytes, "bytes_written_per_step": nbytes,
                      "GB_per_s": round(2 * nbytes * steps / ev / 1e9, 1), "steps": steps}), flush=True)


def _gemm_kernel_op(a, b, out_dtype):
    """One f16acc_gemm launch on HBM-resident a, b into a preallocated c, for
    a problem whose mm call is that launch plus the deferred redo launch (its
    workspace is the redo list alone); None for any other problem."""
    import ctypes

    from f16acc_amd import _lib

    M, K = a.shape
    N = b.shape[1]
    n = ctypes.c_size_t()
    _lib.check(_lib.workspace_size(M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), a.data_ptr(),
                                   b.data_ptr(), ctypes.byref(n)))
    if n.value != _lib.WS_HEADER:
        return None
    c = torch.empty(M, N, device=a.device, dtype=out_dtype)
    code = _lib.OUT_F32 if out_dtype == torch.float32 else _lib.OUT_F16
    stream = torch.cuda.current_stream().cuda_stream
    args = (a.data_ptr(), b.data_ptr(), c.data_ptr(), None, M, N, K, a.stride(0), a.stride(1), b.stride(0),
            b.stride(1), c.stride(0), c.stride(1), code, 1, stream)
    return lambda: _lib.check(_lib.gemm(*args))


def main():
    global PREHEAT_S
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="gemm4096",
                    choices=sorted(WORKLOADS) + ["copy", "overflow", "overflow_split_redo", "qwen2_prefill",
                                                 "redo_overhead", "persistent_ab", "shapes",
                                                 "table_check", "small_grid_check", "large_grid_check",
                                                 "estimate_ab"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and oracle comparison")
    ap.add_argument("--preheat", type=float, default=PREHEAT_S,
                    help="seconds of back-to-back calls before the warm-up steps (0 for counter runs)")
    ap.add_argument("--sweep-tiles", nargs="*", metavar="WORKLOAD",
                    help="time every tile configuration on these workloads (all if none given) and exit")
    ap.add_argument("--tile-calls", nargs="+", metavar="WORKLOAD",
                    help="run every tile configuration, mm and hipBLASLt --steps times each on these workloads, "
                         "untimed (for rocprofv3 --pmc), and exit")
    args = ap.parse_args()
    PREHEAT_S = args.preheat
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: there is no multi-GPU path (a GEMM would shard by M or N "
              "tiles with no exchange, or by K in multiples of 32 with one FP32 all-reduce); "
              "run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.workload == "copy":
        return copy_reference(args.steps, args.warmup)
    if args.workload == "table_check":
        return table_check()
    if args.workload == "small_grid_check":
        return small_grid_check()
    if args.workload == "large_grid_check":
        return large_grid_check()
    if args.workload == "estimate_ab":
        return estimate_ab()
    if args.workload == "shapes":
        return shapes_report(list(WORKLOADS))
    if args.workload == "overflow":
        return overflow_bench(args.steps, args.warmup)
    if args.workload == "overflow_split_redo":
        return overflow_split_redo()
    if args.workload == "redo_overhead":
        return redo_overhead()
    if args.workload == "persistent_ab":
        return persistent_ab()
    if args.workload == "qwen2_prefill":
        line = {"workload": "random-init Qwen2.5-1.5B FP16 prefill, batch 1, 2048 seeded tokens",
                **qwen2_prefill_ab()}
        return print(json.dumps(line), flush=True)
    if args.sweep_tiles is not None:
        return sweep_tiles(args.sweep_tiles or sorted(WORKLOADS))
    if args.tile_calls:
        return tile_calls(args.tile_calls, args.steps)

    import f16acc_amd
    from f16acc_amd.kernel import tile_config

    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    M, N, K, layout, out_dtype = WORKLOADS[args.workload]
    a_cpu, b_cpu, a, b = make_inputs(M, N, K, layout)
    flops = 2.0 * M * N * K
    cfg = tile_config(a, b)

    op = lambda: f16acc_amd.mm(a, b, out_dtype)  # noqa: E731
    wall, ev = time_steps(op, args.steps, args.warmup)
    value = flops * args.steps / wall / 1e12
    call_s = ev / args.steps  # per mm call (the GEMM kernel, and the redo launch where mm defers it)
    # The dominant kernel alone: where mm follows the GEMM with the deferred
    # redo launch, f16acc_gemm (no workspace) launches exactly that GEMM
    # kernel, once per call; elsewhere the mm call is its kernels.
    kernel_op = _gemm_kernel_op(a, b, out_dtype) or op
    kernel_s = time_steps(kernel_op, args.steps, args.warmup)[1] / args.steps
    achieved = flops / kernel_s / 1e12

    c = op()
    torch.cuda.synchronize()
    ref64 = a.double() @ b.double()
    err_fp64 = ((c.double() - ref64).abs().max() / ref64.abs().max()).item()
    del ref64

    # the comparisons run like the measured op: pre-heated, back to back
    blas_op = (lambda: torch.mm(a, b)) if out_dtype == torch.float16 else (lambda: torch.mm(a, b).float())
    blas_t = time_steps(blas_op, args.steps, args.warmup)[1] / args.steps
    fp32acc_t = time_steps(lambda: f16acc_amd.mm(a, b, out_dtype, chunked=False), args.steps, args.warmup)[1] / args.steps

    line = {
        "metric": METRIC if args.workload == "gemm4096" else
        f"TFLOPS at {M}x{N}x{K} fp16 GEMM ({'fp16' if out_dtype == torch.float16 else 'fp32'} out, 1 GPU)",
        "value": round(value, 2), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": round(value / REF_TFLOPS, 2) if args.workload == "gemm4096" else None,
        "baseline_note": "vs_baseline divides by the reference's 65.7 TFLOPS on an RTX 4060 Ti (README.md:29)",
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"fp16 GEMM M={M} N={N} K={K}, A,B~N(0,1) seeded, B "
                               f"{'row-major [K,N]' if layout == 'row' else 'w.t() of [N,K]'}, "
                               f"{'fp16' if out_dtype == torch.float16 else 'fp32'} out, chunk-32 + FP32 sum "
                               f"+ FP32 redo of overflowing tiles", "name": args.workload,
                   "tile": f"{cfg['bm']}x{cfg['bn']}", "tiles": cfg["tiles_m"] * cfg["tiles_n"],
                   "kernel_family": cfg["family"]},
        "frac_of_peak": round(value / PEAK_TFLOPS, 4),
        "max_rel_err_vs_fp64": err_fp64,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS, 4), "traffic": read_traffic(args.workload),
                     "kernel_us": round(kernel_s * 1e6, 2), "call_us": round(call_s * 1e6, 2),
                     "kernel": "the GEMM kernel alone (f16acc_gemm, one launch) where mm adds the deferred redo "
                               "launch, else the mm call; call_us: per mm call"},
        "hipblaslt": {"value": round(flops / blas_t / 1e12, 2), "unit": "TFLOPS",
                      "op": "torch.mm (hipBLASLt), same inputs", "us": round(blas_t * 1e6, 2)},
        "fp32_accumulate": {"value": round(flops / fp32acc_t / 1e12, 2), "unit": "TFLOPS",
                            "op": "f16acc_amd.mm(chunked=False)", "us": round(fp32acc_t * 1e6, 2)},
    }
    if not args.no_cpu:
        info, ref = cpu_baseline(a_cpu, b_cpu, out_dtype)
        line["cpu_baseline"] = info
        from oracle.chunk32 import rel

        line["max_rel_err_vs_oracle"] = rel(c.cpu(), ref)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

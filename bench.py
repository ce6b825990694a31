"""Benchmark of the tropical GEMM hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config P|C1|...|I2|E1]

A step is one call of the C ABI entry point ``tg_gemm_ws`` on the config's
synthetic inputs (already resident in HBM): for argmax configs that is the
B^T staging kernel and the tiled GEMM kernel (whose epilogue resolves the
argmax).  Steps are timed with HIP events on the stream the kernels run on
(torch's current stream), bracketed by device synchronisation.  ``value`` is
tropical GOP/s = 2*M*N*K / t_step, the reference's own "GFLOPS-equivalent"
count (crates/tropical-gemm/examples/bench_rust.rs:121).  ``roofline`` is
for the GEMM kernel alone, timed by the library's event hook
(tg_kernel_timing_*) on the same stream.

The CPU baseline is the single-thread restatement of the reference's CPU
argmax path (oracle/tg_oracle.c, ``tgo_portable_argmax_f32``) timed on a row
slab of the same workload on this host.

Prints one JSON line.  Only one GPU is supported: ``--gpus`` > 1 exits.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tropical-gemm_amd"))

METRIC = ("tropical GOP/s (2·M·N·K) MaxPlus f32 4096³ +argmax, 1 GPU; "
          "% VALU peak")
PEAK_FP32_TFLOPS = 157.3      # MI355X published FP32 vector (and dense) peak
# Tropical roofline: (x) and (+) have no fused form. The densest exact mix is
# one v_add_f32 per product plus half a v_max3_f32 (2 tropical ops per 1.5 VALU
# instructions), and v_max3_f32 issues at the same rate as v_add_f32 and
# v_fma_f32. At the FP32 instruction peak (157.3 TFLOP/s = 78.6e12 FMA
# lane-instructions/s) that is 157.3 * 2/3 = 104.9e12 tropical ops/s.
TROP_PEAK_TOPS = PEAK_FP32_TFLOPS * 2 / 3
PEAK_HBM_GBS = 8000.0         # MI355X published HBM3E bandwidth
PEAK_FP64_TFLOPS = 78.6       # MI355X published FP64 vector peak
# f64 has no three-input max: one v_add_f64 and one v_max_f64 per product
# (2 tropical ops per 2 instructions) at the FP64 instruction peak (78.6
# TFLOP/s = 39.3e12 FMA lane-instructions/s): 39.3e12 tropical ops/s.
TROP_PEAK_F64_TOPS = PEAK_FP64_TFLOPS / 2
# i64: one v_lshl_add_u64 (the wrapping add) and a max written as
# v_cmp_gt_i64 + two v_cndmask_b32 per product, 4 instructions for 2
# tropical ops.  MI355X publishes no 64-bit integer vector peak; at the
# 64-bit (FP64) instruction rate, 39.3e12 lane-instructions/s, that is
# 19.65e12 tropical ops/s (a register-only probe of the mix sustains 18.2e12).
TROP_PEAK_I64_TOPS = PEAK_FP64_TFLOPS / 4
DTYPE_NAME = {"f32": "f32", "f64": "f64", "i32": "i32", "i64": "i64"}
WORKLOAD_NAMES = {
    "P": "P: MaxPlus f32 4096^3 +argmax (BASELINE configs[4] forward)",
    "C1": "C1: MaxPlus f32 1024^3 +argmax",
    "C2": "C2: MinPlus f32 4096^3 +argmax, 10% +inf, zero diagonal",
    "C3": "C3: MaxMul f32 8192x2048x4096 value-only",
    "C4": "C4: MaxPlus i32 262144x128x128 +argmax",
    "C5": "C5: MaxPlus f32 4096^3 +argmax forward, then grad_A and grad_B backward",
    "M1": "M1: MaxPlus f32 65536x2048x8 +argmax (short K, HBM-bound)",
    "F1": "F1: MaxPlus f64 4096^3 +argmax",
    "F2": "F2: MaxPlus f64 4096^3 value-only",
    "I1": "I1: MaxPlus i64 4096^3 +argmax",
    "I2": "I2: MaxPlus i64 4096^3 value-only",
}
KERNEL_NAMES = {
    "P": "tg_gemm_dl<MaxPlus, f32, argmax>",
    "C1": "tg_gemm_dl<MaxPlus, f32, argmax> 4 K slices in one 1024-thread workgroup per 64x64 tile",
    "C2": "tg_gemm_dl<MinPlus, f32, argmax>",
    "C3": "tg_gemm_dl<MaxMul, f32, value-only>",
    "C4": "tg_gemm_kresw<MaxPlus, K=128> (wave-private 16x128 tiles, f32 keys)",
    "C5": "tg_gemm_dl<MaxPlus, f32, argmax>",
    "M1": "tg_gemm_shortk<MaxPlus, f32, argmax> (32x256 tiles, per-product index)",
    "F1": "tg_gemm_dl64<MaxPlus> (f64, 64x128 tiles, argmax)",
    "F2": "tg_gemm_dl64<MaxPlus, value-only> (f64, 64x128 tiles)",
    "I1": "tg_gemm_tiles<MaxPlus, i64, chunked argmax, 16-k chunks> (64x64 tiles)",
    "I2": "tg_gemm_tiles<MaxPlus, i64, value-only> (64x64 tiles)",
}
# HBM bytes per launch of the dominant kernel from rocprofv3 --pmc FETCH_SIZE
# and WRITE_SIZE, scaled by the same counters on a copy kernel of known size
# (profiles/tg_gemm_dl_maxplus_f32_4096_argmax.md, profiles/tg_gemm_kresw_*.md,
# profiles/tg_gemm_shortk_*.md, profiles/hbm_traffic_c2_c3_e1.md,
# profiles/tg_gemm_dl_split_*.md, profiles/tg_gemm_dl64_*.md,
# profiles/tg_gemm_tiles_maxplus_i64_4096.md).  E1: per GEMM launch.

TRAFFIC = {"P": 1.924e9, "C5": 1.924e9, "C4": 0.418e9, "M1": 1.108e9, "C1": 0.034e9,
           "C2": 1.771e9, "C3": 0.704e9, "F1": 3.439e9, "F2": 2.266e9, "E1": 0.1177e9,
           "I1": 4.881e9, "I2": 3.356e9}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# Rows of each configuration's CPU-baseline sample outside P (P: --cpu-rows):
# about 0.5-4 s of single-core work.  C1 and C4 run whole; M1's short K makes
# the reference's blocked loops slow (0.07 GOP/s), hence its small slab.
CPU_ROWS = {"C1": 1024, "C2": 512, "C3": 1024, "C4": 262144, "C5": 512, "M1": 4096, "F1": 256,
            "F2": 4096, "I1": 768, "I2": 768}
# Configurations without a CPU restatement of the reference path they would
# take, with the reason (none at present: every configuration has one).
NO_CPU_BASELINE: dict = {}


def run_cpu_baseline(cfg: dict, a, b, rows: int, value_only: bool = False) -> dict:
    """Single-thread restatement of the reference CPU algorithm for this
    configuration, timed on the first ``rows`` rows of the same inputs:
    argmax configurations run the reference's argmax path (BLIS PORTABLE
    tiling, 4x4 scalar microkernel); value-only f32 ones (and C1's
    value-only line) its AVX2 path (F32_AVX2 tiling, 8x8 microkernel);
    value-only MaxPlus f64 its AVX2 f64 path (F64_AVX2 tiling, 4x4
    microkernel)."""
    import numpy as np

    from oracle import oracle

    m, k = a.shape
    n = b.shape[1]
    rows = max(1, min(rows, m))
    ha = a[:rows].cpu().numpy()
    hb = b.cpu().numpy()
    sr = cfg["semiring"]
    if cfg["argmax"] and not value_only:
        fn, algo = oracle.portable_argmax, ("argmax algorithm (BLIS PORTABLE tiling, 4x4 scalar "
                                            "microkernel)")
    elif ha.dtype == np.float32:
        fn, algo = oracle.avx2_gemm_f32, ("value-only algorithm (BLIS F32_AVX2 tiling, AVX2 8x8 "
                                          "microkernel)")
    elif ha.dtype in (np.int32, np.int64):
        fn, algo = oracle.portable_gemm, ("value-only algorithm (BLIS PORTABLE tiling, 4x4 scalar "
                                          "microkernel)")
    elif ha.dtype == np.float64 and sr == "maxplus":
        fn, algo = oracle.avx2_gemm_maxplus_f64, ("value-only algorithm (BLIS F64_AVX2 tiling, AVX2 "
                                                  "4x4 f64 microkernel)")
    else:
        raise ValueError("no CPU baseline restated for this configuration")
    t0 = time.perf_counter()
    fn(sr, ha, hb)
    dt = time.perf_counter() - t0
    what = "the whole product" if rows == m else f"a {rows}-row slab"
    return {
        "value": round(2.0 * rows * n * k / dt / 1e9, 3),
        "unit": "GOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{what} ({rows}x{k}x{n}, {sr} {ha.dtype}) of this configuration's inputs, "
                   f"reference CPU {algo} restated in C, 1 thread, {dt:.1f} s on {cpu_model()}"),
    }


# Untimed warm-up.  With --warmup W given: exactly W steps.  By default:
# DEFAULT_WARMUP steps, repeated until at least WARMUP_MIN_S has passed, so
# that short steps (C4, M1: ~0.15 ms) also run on the settled engine clock
# (it ramps over the first ~15 ms of sustained load).  Returns the steps run.
DEFAULT_WARMUP = 25
WARMUP_MIN_S = 0.2


def warm_up(step, steps, dev) -> int:
    import torch

    if steps is not None:
        for _ in range(steps):
            step()
        torch.cuda.synchronize(dev)
        return steps
    t0 = time.perf_counter()
    done = 0
    while done == 0 or time.perf_counter() - t0 < WARMUP_MIN_S:
        for _ in range(DEFAULT_WARMUP):
            step()
        done += DEFAULT_WARMUP
        torch.cuda.synchronize(dev)
    return done


def cpu_rows_for(name: str, p_rows: int) -> int:
    """P uses --cpu-rows; the others their CPU_ROWS sample."""
    return p_rows if name == "P" else CPU_ROWS[name]


def run_einsum(args, lib, dev) -> int:
    """Einsum workload: a step is one ``tropical_gemm.einsum`` call on operands
    resident in HBM (contraction order, permutation copies and the GEMMs).
    The roofline is for the GEMM kernels, timed by the library's hook; their
    share of the step shows what the permutations and host planning cost."""
    import torch

    import workloads
    from tropical_gemm import _native as nat
    from tropical_gemm import einsum as E

    cfg = workloads.EINSUM[args.config]
    ops_ = workloads.make_einsum_operands(args.config, dev)
    code, sr = cfg["code"], cfg["semiring"]
    ixs, iy = E.parse(code)
    sizes = cfg["sizes"]
    path = E.einsum_path(ixs, iy, sizes, "greedy")
    # Tropical ops of the contraction tree: 2 per term of every pairwise GEMM.
    labs = [list(x) for x in ixs]
    ops = 0.0
    gemms = []
    for i, j in path:
        keep = set(iy)
        for o, lab in enumerate(labs):
            if o not in (i, j):
                keep.update(lab)
        union = list(dict.fromkeys(labs[i] + labs[j]))
        res = [x for x in union if x in keep]
        terms = 1
        for x in union:
            terms *= sizes[x]
        ops += 2.0 * terms
        gemms.append("".join(labs[i]) + "," + "".join(labs[j]) + "->" + "".join(res))
        labs = [lab for o, lab in enumerate(labs) if o not in (i, j)] + [res]

    def step():
        return E.einsum(code, *ops_, semiring=sr)

    warmup_run = warm_up(step, args.warmup, dev)
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps

    tot = ctypes.c_double(0.0)
    nl = ctypes.c_int64(0)
    nat.check(lib.tg_kernel_timing_read(ctypes.byref(tot), ctypes.byref(nl)))  # clear
    nat.check(lib.tg_kernel_timing_enable(1))
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize(dev)
    nat.check(lib.tg_kernel_timing_enable(0))
    nat.check(lib.tg_kernel_timing_read(ctypes.byref(tot), ctypes.byref(nl)))
    ms_gemms = tot.value / args.steps  # every GEMM kernel of one step
    gops = ops / (ms_step / 1e3) / 1e9
    kernel_tops = ops / (ms_gemms / 1e3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(gops, 2),
        "unit": "GOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup_run,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded torch Philox on device; workloads.py)",
        "config": {"workload": f"{args.config}: tropical einsum {code} ({sr}, value-only)",
                   "sizes": sizes, "contraction_path": gemms,
                   "parallelism": "none (1 GPU)"},
        "roofline": {
            "bound": "valu",
            "achieved": round(kernel_tops, 3),
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(kernel_tops / PEAK_FP32_TFLOPS, 4),
            "traffic": TRAFFIC.get(args.config),  # per GEMM launch
            "kernel": "tg_gemm_dl<MaxPlus, f32, value-only> (every GEMM of the contraction)",
            "kernel_ms": round(ms_gemms, 4),
            "kernel_launches_timed": int(nl.value),
            "ops_per_launch": ops / max(len(gemms), 1),
            "trop_peak": TROP_PEAK_TOPS,
            "frac_of_trop_peak": round(kernel_tops / TROP_PEAK_TOPS, 4),
        },
        "gemm_share_of_step": round(ms_gemms / ms_step, 4),
        "step_frac_of_trop_peak": round(gops / 1e3 / TROP_PEAK_TOPS, 4),
        "wall_s_timed_region": round(wall, 4),
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The engine clock ramps from ~2.1 to ~2.35 GHz over the first ~15 ms of
    # sustained VALU load.  Default: 25-step rounds until 0.2 s have passed.
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", default="P",
                    choices=["P", "C1", "C2", "C3", "C4", "C5", "M1", "F1", "F2", "I1", "I2",
                             "E1"])
    ap.add_argument("--cpu-rows", type=int, default=3072,
                    help="rows of P's CPU-baseline slab (0 skips the CPU baseline of every "
                         "configuration)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after timing, copy this many MiB once (a known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path.  Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import workloads
    from tropical_gemm import _native as nat

    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    lib = nat.load()
    dev = torch.device("cuda", 0)
    if args.config in workloads.EINSUM:
        return run_einsum(args, lib, dev)
    cfg = workloads.CONFIGS[args.config]
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    a, b = workloads.make_inputs(args.config, dev)
    tdt = a.dtype
    c = torch.empty((m, n), dtype=tdt, device=dev)
    am = torch.empty((m, n), dtype=torch.int32, device=dev) if cfg["argmax"] else None
    dt = nat.DTYPE[cfg["dtype"]]
    ws_bytes = lib.tg_gemm_workspace_size(dt, 1, m, n, k, 1 if cfg["argmax"] else 0)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    s_ptr = ctypes.c_void_p(stream.cuda_stream)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sr = nat.SEMIRING[cfg["semiring"]]

    backward = cfg.get("backward", False)
    if backward:
        g = workloads.make_grad(args.config, m, n, dev, tdt)
        ga = torch.empty((m, k), dtype=tdt, device=dev)
        gb = torch.empty((k, n), dtype=tdt, device=dev)

    def forward():
        rc = lib.tg_gemm_ws(0, sr, dt, 0, p(a), p(b), p(c), p(am), m, n, k, p(ws), ws_bytes, s_ptr)
        if rc != 0:
            raise nat.HipError(rc, nat.last_error())

    def backward_only():
        nat.check(lib.tg_backward_a(0, dt, 0, p(g), p(am), p(ga), m, n, k, s_ptr))
        nat.check(lib.tg_backward_b(0, dt, 0, p(g), p(am), p(gb), m, n, k, s_ptr))

    def step():
        forward()
        if backward:
            backward_only()

    warmup_run = warm_up(step, args.warmup, dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    # Step timing: events on the stream every kernel of the step runs on.
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / args.steps

    # Dominant-kernel timing: the library records a HIP event pair on the same
    # stream around its main GEMM kernel (B^T staging excluded).  Separate
    # pass over the same number of steps, so the step timing above carries no
    # event overhead.
    tot = ctypes.c_double(0.0)
    nl = ctypes.c_int64(0)
    nat.check(lib.tg_kernel_timing_read(ctypes.byref(tot), ctypes.byref(nl)))  # clear
    nat.check(lib.tg_kernel_timing_enable(1))
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize(dev)
    nat.check(lib.tg_kernel_timing_enable(0))
    nat.check(lib.tg_kernel_timing_read(ctypes.byref(tot), ctypes.byref(nl)))
    ms_kernel = tot.value / max(nl.value, 1)

    # C5: the backward pair alone (grad_A, grad_B), timed like the step.
    ms_backward = None
    if backward:
        torch.cuda.synchronize(dev)
        ev0.record(stream)
        for _ in range(args.steps):
            backward_only()
        ev1.record(stream)
        torch.cuda.synchronize(dev)
        ms_backward = ev0.elapsed_time(ev1) / args.steps

    # Post-timing sanity check (outside the timed region): every output equals
    # the product at its argmax, bit-exactly.
    check = None
    if am is not None:
        kk = am.long()
        aw = torch.gather(a, 1, kk)
        bw = torch.gather(b, 0, kk)
        prod = aw * bw if cfg["semiring"] == "maxmul" else aw + bw
        check = bool(torch.equal(prod, c))

    ops = 2.0 * m * n * k
    gops = ops / (ms_step / 1e3) / 1e9
    kernel_tops = ops / (ms_kernel / 1e3) / 1e12
    esize = a.element_size()
    algo_bytes = esize * (m * k + k * n + m * n) + (4 * m * n if am is not None else 0)
    if cfg.get("bound") == "hbm":
        # Short K: the output (and argmax) writes dominate; the roofline is
        # HBM bandwidth, achieved = algorithmic bytes / kernel time.
        kernel_gbs = algo_bytes / (ms_kernel / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(kernel_gbs, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(kernel_gbs / PEAK_HBM_GBS, 4)}
    else:
        # Tropical (+)/(x) has no MFMA form: the kernel is bound by the
        # vector ALU.  peak = MI355X published vector peak of the dtype.
        peak = PEAK_FP64_TFLOPS if cfg["dtype"] in ("f64", "i64") else PEAK_FP32_TFLOPS
        roofline = {"bound": "valu", "achieved": round(kernel_tops, 3), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(kernel_tops / peak, 4)}
    trop_peak = {"f64": TROP_PEAK_F64_TOPS, "i64": TROP_PEAK_I64_TOPS}.get(cfg["dtype"],
                                                                          TROP_PEAK_TOPS)
    roofline.update({
        "traffic": TRAFFIC.get(args.config),
        "kernel": KERNEL_NAMES[args.config],
        "kernel_ms": round(ms_kernel, 4),
        "kernel_launches_timed": int(nl.value),
        "ops_per_launch": ops,
        "trop_peak": trop_peak,
        "frac_of_trop_peak": round(kernel_tops / trop_peak, 4),
        "algorithmic_bytes": algo_bytes,
    })
    out = {
        "metric": METRIC,
        "value": round(gops, 2),
        "unit": "GOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup_run,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAME[cfg["dtype"]],
        "data": "synthetic (seeded torch Philox on device; workloads.py)",
        "config": {"workload": WORKLOAD_NAMES[args.config],
                   "semiring": cfg["semiring"], "m": m, "n": n, "k": k,
                   "argmax": cfg["argmax"], "layout": "row-major", "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "step_frac_of_trop_peak": round(gops / 1e3 / trop_peak, 4),
        "wall_s_timed_region": round(wall, 4),
        "argmax_consistency_check": check,
        "device": torch.cuda.get_device_name(dev),
    }
    if backward:
        # Backward bytes: read dC and argmax (4 B each per output), write
        # grad_A and grad_B once.
        bwd_bytes = 8 * m * n + esize * (m * k + k * n)
        out["backward"] = {"ms": round(ms_backward, 4), "algorithmic_bytes": bwd_bytes,
                           "GB_per_s": round(bwd_bytes / (ms_backward / 1e3) / 1e9, 1),
                           "frac_of_hbm_peak": round(bwd_bytes / (ms_backward / 1e3) / 8e12, 4)}
    if args.copy_mib > 0:
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize(dev)
        dst.copy_(src)
        torch.cuda.synchronize(dev)
        out["copy_calibration_bytes"] = args.copy_mib << 20
    if args.cpu_rows > 0 and args.config in NO_CPU_BASELINE:
        out["cpu_baseline_note"] = NO_CPU_BASELINE[args.config]
    elif args.cpu_rows > 0:
        rows = cpu_rows_for(args.config, args.cpu_rows)
        out["cpu_baseline"] = run_cpu_baseline(cfg, a, b, rows)
        out["gpu_vs_cpu_baseline"] = round(gops / out["cpu_baseline"]["value"], 1)
        if args.config == "C1":
            # The reference's value-only CPU path on the same product (its
            # headline CPU number is this path at n = 1024).
            out["cpu_baseline_value_only"] = run_cpu_baseline(cfg, a, b, rows, value_only=True)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark of the SC matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2|cfg3|cfg4|cfg5]
                    [--impl auto|fp4|int8|valu] [--no-cpu]

Default workload (BASELINE.json's metric, configuration 2): one
``sc_matmul(a, b, "per_row", sc_prec=8, stoc_len=256, smooth_scales=s)`` with
a (4096, 4096) ~ N(0,1) with 1% of channels x20, b (11008, 4096) ~ N(0, 0.02^2),
s = compute_smooth_scales(accumulate_act_scales(a), b, 0.5). Inputs are generated on the
host with numpy's seeded PCG64 and are resident in HBM before timing. A step is one full
sc_matmul call (quantize a, quantize b, SC GEMM, epilogue).

Printed: one JSON line. ``value`` is SC bit-ops/s = N*M*D*stoc_len / step time (the
reference's unit of work; the MFMA kernel executes its own, smaller op count, reported in
``roofline``). After the timed steps the same number of steps runs again with HIP events
recorded on the launch stream around every library call (the library's launch observer):
``roofline`` is the SC GEMM launches of a step (FP4 e2m1 MFMA by default, int8 MFMA or VALU
popcount with --impl), ``quantizers`` the quantizer launches. ``cpu_baseline`` times the
CPU oracle on a sample of the same workload and checks those outputs bit-exactly against
the GPU result; ``reference_cpu`` is the reference's own cfg1 call timed under
TRITON_INTERPRET=1 in the build container (the reference does not exist on the GPU box).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
MFMA_FP4_PEAK_TFLOPS = 10100.0  # MI355X dense fp4 MFMA, 10.1 PFLOP/s
VALU_PEAK_TOPS = 256 * 4 * 16 * 2.4e9 / 1e12 * 1.0  # 64 lane-ops/clk/CU at 2.4 GHz


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_cfg2(seed_a=1, seed_b=2, seed_ch=3):
    N, M, D = 4096, 11008, 4096
    ra = np.random.default_rng(seed_a)
    a = ra.standard_normal((N, D), dtype=np.float32)
    ch = np.random.default_rng(seed_ch).choice(D, size=D // 100, replace=False)
    a[:, ch] *= 20.0
    b = (np.random.default_rng(seed_b).standard_normal((M, D), dtype=np.float32) * 0.02)
    return a, b.astype(np.float32)


def make_cfg3(seed_a=4, seed_b=5):
    """ViT-B MLP: a = GELU(N(0,1)) (12608, 3072) = 64 images x 197 tokens, b ~ N(0, 0.02^2)
    (768, 3072); GELU with erf, computed in float64 on the host then rounded to fp32."""
    from math import sqrt
    from scipy.special import erf
    z = np.random.default_rng(seed_a).standard_normal((12608, 3072))
    a = (0.5 * z * (1.0 + erf(z / sqrt(2.0)))).astype(np.float32)
    b = (np.random.default_rng(seed_b).standard_normal((768, 3072)) * 0.02).astype(np.float32)
    return a, b


def make_cfg4(seed_q=6, seed_k=7, seed_p=8, seed_v=9, bh=768):
    """ViT-B attention at batch 64 (BH = 768): q, k (BH, 197, 64) ~ N(0,1); P = row-softmax
    of N(0,1) logits (BH, 197, 197); V^T (BH, 64, 197) ~ N(0,1)."""
    q = np.random.default_rng(seed_q).standard_normal((bh, 197, 64), dtype=np.float32)
    k = np.random.default_rng(seed_k).standard_normal((bh, 197, 64), dtype=np.float32)
    z = np.random.default_rng(seed_p).standard_normal((bh, 197, 197))
    z = np.exp(z - z.max(axis=-1, keepdims=True))
    p = (z / z.sum(axis=-1, keepdims=True)).astype(np.float32)
    vt = np.random.default_rng(seed_v).standard_normal((bh, 64, 197), dtype=np.float32)
    return q, k, p, vt


def make_cfg5(seed_a=10, seed_b=11, seed_rows=12):
    """Mixed-precision unipolar: a (4096, 4096) ~ N(0,1) with 205 rows (5%, seeded choice)
    replaced by Student-t (df = 3) rows; b (4096, 4096) ~ N(0, 0.02^2)."""
    a = np.random.default_rng(seed_a).standard_normal((4096, 4096), dtype=np.float32)
    rr = np.random.default_rng(seed_rows)
    rows = rr.choice(4096, size=205, replace=False)
    a[rows] = rr.standard_t(3, size=(205, 4096)).astype(np.float32)
    b = (np.random.default_rng(seed_b).standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    return a, b


CFG5_LEVELS = [256, 64, 16]


def time_steps(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps, out


# arithmetic the SC GEMM computes in: every kernel counts integers exactly
DTYPE = {0: "int8 MFMA (exact int32 counts)", 1: "u32 popcount (exact int32 counts)",
         2: "e2m1 MFMA (exact integer counts in fp32)"}


def kernel_roofline(impl, N, M, D, JP, batch=1):
    """(ops per launch, peak in 1e12/s, unit, bound, kernel name) for the SC GEMM kernel on
    an N x M x D problem (times batch): the algorithmic work of the interval formulation
    over the useful (unpadded) outputs. FP4 MFMA: one multiply-add per (n, m, d, interval)
    over JPF = max(JP, 16) intervals; int8 MFMA: over JP intervals; VALU: an AND and a
    popcount per 32-interval word and bit plane."""
    units = float(N) * M * D * batch
    if impl == 2:
        return (2.0 * units * max(JP, 16), MFMA_FP4_PEAK_TFLOPS, "TFLOP/s", "mfma",
                "sc_gemm_fp4_kernel")
    if impl == 0:
        return (2.0 * units * JP, MFMA_INT8_PEAK_TOPS, "TOP/s", "mfma",
                "sc_gemm_mfma_kernel")
    return (units * max(1, JP // 32) * 2 * 2, VALU_PEAK_TOPS, "TOP/s", "valu",
            "sc_gemm_valu_kernel")


class LaunchTimer:
    """HIP events recorded on the launch stream (torch's current stream, which the library
    launches on) right before and after every scmp_quantize / scmp_sc_gemm call, through
    the library's launch observer. An FP4 GEMM call also launches a counter clear of a few
    hundred bytes before the GEMM kernel; its time is inside the bracket."""

    def __init__(self):
        self.recs, self.pending = [], None

    def __call__(self, stage, kind, info):
        import torch
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(torch.cuda.current_stream())
        if stage == "pre":
            self.pending = (kind, info, ev)
        else:
            k, i, e0 = self.pending
            self.recs.append((k, dict(i), e0, ev))

    def durations(self):
        import torch
        torch.cuda.synchronize()
        return [(k, i, e0.elapsed_time(e1)) for k, i, e0, e1 in self.recs]


def observe_steps(fn, steps):
    """Run `steps` more steps with the launch observer on; per-launch (kind, info, ms)."""
    from scmp_kernels_amd.sc import kernels as K
    timer = LaunchTimer()
    K.launch_observer = timer
    try:
        for _ in range(steps):
            fn()
    finally:
        K.launch_observer = None
    return timer.durations()


def launch_roofline(launches, steps, traffic_file=None):
    """roofline object for the GEMM launches of the observed steps: algorithmic work of
    all GEMM launches of a step over their summed event time (one launch per step at cfg2,
    cfg4 two GEMMs, cfg3 a main and a tail launch, cfg5 one per level), plus one entry per
    distinct launch; and the quantizer launches' HBM rate."""
    gem = [(i, ms) for k, i, ms in launches if k == "sc_gemm"]
    per = {}
    for i, ms in gem:
        key = (i["N"], i["M"], i["D"], i["batch"], i["JP"], i["impl"], i["chunk"])
        per.setdefault(key, []).append(ms)
    entries, ops_step, ms_step = [], 0.0, 0.0
    peak = unit = bound = None
    kernels = set()
    for (N, M, D, batch, JP, impl, chunk), ms in per.items():
        ops, peak, unit, bound, kname = kernel_roofline(impl, N, M, D, JP, batch)
        kernels.add(kname)
        avg = float(np.mean(ms))
        ops_step += ops * len(ms) / steps
        ms_step += float(np.sum(ms)) / steps
        entries.append({"kernel": kname, "N": N, "M": M, "D": D, "batch": batch, "JP": JP,
                        "chunk": chunk, "launches": len(ms), "avg_ms": round(avg, 4),
                        "ops_per_launch": ops,
                        "frac": round(ops / (avg * 1e-3) / 1e12 / peak, 4)})
    achieved = ops_step / (ms_step * 1e-3) / 1e12
    roof = {"bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": None,
            "kernel": "+".join(sorted(kernels)), "avg_ms": round(ms_step, 4),
            "ops_per_launch": ops_step, "launches": entries,
            "timing": f"HIP events around every SC GEMM call of {steps} steps"}
    if traffic_file and len(kernels) == 1:
        tp = os.path.join(ROOT, "profiles", traffic_file)
        if os.path.exists(tp):
            with open(tp) as f:
                roof["traffic"] = json.load(f).get(next(iter(kernels)), {}).get(
                    "traffic_bytes")
    quants = []
    qper = {}
    for k, i, ms in launches:
        if k == "quantize":
            key = (i["rows"], i["cols"], i["code_bytes"], i["variant"])
            qper.setdefault(key, []).append(ms)
    for (rows, cols, cbytes, var), ms in qper.items():
        avg = float(np.mean(ms))
        nbytes = 4 * rows * cols + cbytes
        quants.append({"rows": rows, "cols": cols, "launches": len(ms),
                       "avg_us": round(avg * 1e3, 2), "bytes": nbytes,
                       "GB/s": round(nbytes / (avg * 1e-3) / 1e9, 1),
                       "frac_of_8TB/s": round(nbytes / (avg * 1e-3) / 8e12, 3)})
    return roof, {"bound": "hbm", "peak_GB/s": 8000.0,
                  "bytes": "fp32 input read once + GEMM code bytes written", "launches": quants}


def bench_cfg2(args):
    import torch
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.quant import accumulate_act_scales, compute_smooth_scales

    dev = torch.device("cuda", 0)
    t0 = time.perf_counter()
    a_h, b_h = make_cfg2()
    a = torch.from_numpy(a_h).to(dev)
    b = torch.from_numpy(b_h).to(dev)
    s = compute_smooth_scales(accumulate_act_scales(a), b, alpha=0.5)
    log(f"inputs ready in {time.perf_counter() - t0:.1f}s")
    N, D = a.shape
    M = b.shape[0]
    L = 256
    if args.impl != "auto":
        os.environ["SCMP_GEMM_IMPL"] = args.impl

    def step():
        return sc_matmul(a, b, "per_row", sc_prec=8, stoc_len=L, smooth_scales=s)

    t_step, y = time_steps(step, args.steps, args.warmup)
    log(f"sc_matmul step: {t_step * 1e3:.3f} ms")
    # the same steps again with events around each launch: the GEMM launch the step runs
    # (fused fp32 row/column epilogue) and the two quantizer launches
    launches = observe_steps(step, max(3, args.steps))
    roof, quants = launch_roofline(launches, max(3, args.steps), "cfg2_gemm_traffic.json")
    B = N * M * D * L
    roof["effective_sc_bitops_per_s"] = B / (roof["avg_ms"] * 1e-3)
    log(f"SC GEMM: {roof['avg_ms']:.3f} ms per launch, {roof['frac']:.3f} of peak; "
        f"quantizers {[q['avg_us'] for q in quants['launches']]} us")
    impl = next(i["impl"] for k, i, _ in launches if k == "sc_gemm")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(a_h, b_h, s.cpu().numpy(), y, rows=args.cpu_rows)
    return {
        "metric": "ms & SC bit-ops/s per sc_matmul (M=4096,N=11008,D=4096, per_row, sc_prec=8)",
        "value": B / t_step,
        "unit": "SC bit-ops/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": DTYPE[impl], "data": "synthetic (numpy PCG64 seeds 1,2,3)",
        "config": {"workload": "cfg2: LLM linear per_row bipolar + SmoothQuant",
                   "a": [N, D], "b": [M, D], "sc_prec": 8, "stoc_len": L,
                   "granularity": "per_row", "gemm_kernel": roof["kernel"]},
        "roofline": roof,
        "quantizers": quants,
        "cpu_baseline": cpu,
        "reference_cpu": reference_cpu_record(),
    }


def reference_cpu_record():
    """The reference's own cfg1 call timed under TRITON_INTERPRET=1 in the build container
    (tests/golden/gen_golden.py --time-cfg1; the reference is not present on the GPU box),
    read from the committed record."""
    p = os.path.join(ROOT, "tests", "golden", "ref_cpu_timing.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        r = json.load(f)
    return {"value": r["warm_sc_bitops_per_s"], "unit": "SC bit-ops/s", "cores": r["cores"],
            "kind": "reference", "sample": r["what"] + f"; warm median {r['warm_median_s']} s"
            f", cold {r['cold_s']} s; {r['host']['cpu']}, measured in the build container"}


def bench_other(args):
    """The other BASELINE configurations, timed as whole calls (inputs resident in HBM,
    tables cached after the warmup), with the GEMM launches' roofline and a CPU oracle
    sample checked bit-exactly against the GPU result."""
    import torch
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.mp import classify_rows_by_metric
    dev = torch.device("cuda", 0)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    if args.config == "cfg3":
        a_h, b_h = make_cfg3()
        a, b = T(a_h), T(b_h)
        N, D = a.shape
        M = b.shape[0]
        B = N * M * D * 256
        desc = "ViT-B MLP per_row bipolar chunk_d=72, 12608x768x3072"

        def step():
            return sc_matmul(a, b, "per_row", sc_prec=8, chunk_d=72)

        def cpu(y):
            rows = np.linspace(0, N - 1, min(N, 4 * args.cpu_rows)).astype(np.int64)
            return _cpu_sample(
                lambda O, ctx: O.sc_matmul(a_h[rows], b_h, "per_row", sc_prec=8, chunk_d=72,
                                           ctx=ctx),
                lambda: y[torch.from_numpy(rows).to(dev)], len(rows) * M * D * 256,
                f"{len(rows)} of {N} rows of a (evenly spaced) x all {M} rows of b, D={D}")
    elif args.config == "cfg4":
        q_h, k_h, p_h, vt_h = make_cfg4()
        q, k, p, vt = T(q_h), T(k_h), T(p_h), T(vt_h)
        B = 2 * 768 * 197 * 197 * 64 * 256
        desc = "attention per_head bipolar BH=768: QK^T (197x197x64) + P.V (197x64x197)"

        def step():
            y1 = sc_matmul(q, k, "per_head", sc_prec=8)
            return y1, sc_matmul(p, vt, "per_head", sc_prec=8)

        def cpu(y):
            hd = np.linspace(0, 767, 384).astype(np.int64)
            hi = torch.from_numpy(hd).to(dev)

            def run(O, ctx):
                return np.concatenate([
                    O.sc_matmul(q_h[hd], k_h[hd], "per_head", sc_prec=8, ctx=ctx).ravel(),
                    O.sc_matmul(p_h[hd], vt_h[hd], "per_head", sc_prec=8, ctx=ctx).ravel()])
            return _cpu_sample(run, lambda: torch.cat([y[0][hi].ravel(), y[1][hi].ravel()]),
                               2 * len(hd) * 197 * 197 * 64 * 256,
                               f"{len(hd)} of 768 heads (evenly spaced), QK^T and P.V")
    elif args.config == "cfg5":
        a_h, b_h = make_cfg5()
        a, b = T(a_h), T(b_h)
        metric = a.amax(dim=1) - a.amin(dim=1)
        ra = classify_rows_by_metric(metric, CFG5_LEVELS, [1 / 3] * 3)
        B = sum(len(ra.level_row_indices[L]) * 4096 * 4096 * L for L in CFG5_LEVELS)
        desc = "mixed-level unipolar grouped (G=4), 4096x4096x4096, levels {256,64,16}"
        from scmp_kernels_amd.mp import sc_matmul_mixed

        def step():
            # Y[rows_L] = sc_matmul(a[rows_L], b, stoc_len=L, rng_levels=L) for every level,
            # in one call (b quantized once per call, rows read and written in place)
            return sc_matmul_mixed(a, b, ra, mode="unipolar", group_a=4, group_b=4)

        def cpu(y):
            sel, work = [], 0
            for L in CFG5_LEVELS:
                rows = ra.level_row_indices[L].cpu().numpy()
                g = np.linspace(0, len(rows) // 4 - 1, 16).astype(np.int64)
                for gi in g:
                    sel.append((L, rows[4 * gi:4 * gi + 4]))
                    work += 4 * 4096 * 4096 * L

            def run(O, ctx):
                return np.concatenate([
                    O.sc_matmul(a_h[r], b_h, "per_row", mode="unipolar", group_a=4,
                                group_b=4, stoc_len=L, rng_levels=L, ctx=ctx).ravel()
                    for L, r in sel])

            def got():
                return torch.cat([y[torch.from_numpy(r).to(dev)].ravel() for _, r in sel])
            return _cpu_sample(run, got, work, "16 groups of 4 rows per level (evenly "
                               "spaced in each level's row order) x all 4096 rows of b")
    else:
        raise SystemExit(f"unknown --config {args.config}")
    t, y = time_steps(step, args.steps, args.warmup)
    log(f"{args.config}: {t * 1e3:.3f} ms per call")
    launches = observe_steps(step, max(3, args.steps))
    roof, quants = launch_roofline(launches, max(3, args.steps),
                                   f"{args.config}_gemm_traffic.json")
    log(f"{args.config} GEMMs: {roof['avg_ms']:.3f} ms per step, {roof['frac']:.3f} of peak")
    impl = next(i["impl"] for k, i, _ in launches if k == "sc_gemm")
    return {"metric": f"ms & SC bit-ops/s per call ({desc})", "value": B / t,
            "unit": "SC bit-ops/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(t * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": DTYPE[impl],
            "data": "synthetic (numpy PCG64, bench.py generators)",
            "config": {"workload": args.config, "sc_bit_ops": B},
            "roofline": roof, "quantizers": quants,
            "cpu_baseline": None if args.no_cpu else cpu(y)}


def _cpu_sample(run, got, work, sample):
    """Time the CPU oracle on a sample (run(O, ctx) -> flat array) and compare it bit for
    bit with the GPU's values for the same outputs (got() -> flat device tensor)."""
    from oracle import sc_oracle as O
    nthreads = min(16, os.cpu_count() or 1)
    O.lib()
    t0 = time.perf_counter()
    ref = run(O, O.Ctx(nthreads=nthreads))
    dt = time.perf_counter() - t0
    g = got().cpu().numpy()
    exact = bool(np.array_equal(g.view(np.uint32), ref.view(np.uint32)))
    log(f"cpu oracle: {dt:.1f}s on {nthreads} threads; bit-exact={exact}")
    return {"value": work / dt, "unit": "SC bit-ops/s", "cores": nthreads, "kind": "port",
            "sample": f"{sample}; {dt:.1f} s", "sample_bit_exact_vs_gpu": exact}


def profile_gemm(args):
    """Two cfg2 steps (the first builds the tables), then one device copy of a known size
    (2^28 int32 each way) whose FETCH_SIZE / WRITE_SIZE counter values scale the second
    step's GEMM counters to bytes. Used under rocprofv3 --pmc."""
    import torch
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.quant import accumulate_act_scales, compute_smooth_scales
    dev = torch.device("cuda", 0)
    a_h, b_h = make_cfg2()
    a = torch.from_numpy(a_h).to(dev)
    b = torch.from_numpy(b_h).to(dev)
    s = compute_smooth_scales(accumulate_act_scales(a), b, alpha=0.5)
    if args.impl != "auto":
        os.environ["SCMP_GEMM_IMPL"] = args.impl
    for _ in range(2):
        sc_matmul(a, b, "per_row", sc_prec=8, stoc_len=256, smooth_scales=s)
        torch.cuda.synchronize()
    src = torch.ones(2 ** 28, dtype=torch.int32, device=dev)     # 1 GiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log("profile_gemm: two sc_matmul steps, then a 1 GiB device copy")


def cpu_baseline(a_h, b_h, s_h, y_gpu, rows):
    """The CPU oracle (C, OpenMP) on `rows` rows of a against all of b: same per-row work
    as the GPU step, scaled to bit-ops/s. Also a bit-exact check of those rows."""
    import torch
    from oracle import sc_oracle as O
    nthreads = min(16, os.cpu_count() or 1)
    idx = np.linspace(0, a_h.shape[0] - 1, rows).astype(np.int64)
    a_s = a_h[idx]
    O.lib()
    t0 = time.perf_counter()
    y_ref = O.sc_matmul(a_s, b_h, "per_row", sc_prec=8, stoc_len=256, smooth_scales=s_h,
                        ctx=O.Ctx(nthreads=nthreads))
    dt = time.perf_counter() - t0
    got = y_gpu[torch.from_numpy(idx).to(y_gpu.device)].cpu().numpy()
    exact = bool(np.array_equal(got.view(np.uint32), y_ref.view(np.uint32)))
    B = rows * b_h.shape[0] * a_h.shape[1] * 256
    log(f"cpu oracle: {rows} rows in {dt:.1f}s on {nthreads} threads; bit-exact={exact}")
    return {"value": B / dt, "unit": "SC bit-ops/s", "cores": nthreads, "kind": "port",
            "sample": f"{rows} of 4096 rows of a (evenly spaced) x all 11008 rows of b, "
                      f"D=4096, full pipeline (smoothing, quantizers, table accumulator, "
                      f"epilogue); {dt:.1f} s",
            "sample_bit_exact_vs_gpu": exact}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--impl", default="auto", choices=["auto", "fp4", "int8", "valu"],
                    help="SC GEMM kernel; auto = the library default (FP4 MFMA when the "
                         "stream table fits e2m1, else int8 MFMA)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--mode", default="step", choices=["step", "gemm"],
                    help="step: the benchmark (default); gemm: two cfg2 steps plus a 1 GiB "
                         "copy, for counter collection")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build runs the SC matmul on a single "
              f"MI355X); --gpus {args.gpus} is not supported.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.config in ("cfg3", "cfg4", "cfg5"):
        print(json.dumps(bench_other(args)), flush=True)
        return
    if args.config != "cfg2":
        print(f"unknown --config {args.config}", file=sys.stderr)
        sys.exit(2)
    if args.mode == "gemm":
        profile_gemm(args)
        return
    res = bench_cfg2(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

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
``roofline``). ``roofline`` times the dominant kernel (the SC GEMM: FP4 e2m1 MFMA by
default, int8 MFMA or VALU popcount with --impl) with HIP events on the stream it runs on. ``cpu_baseline`` times the CPU oracle on a row sample of the same
workload and checks those rows bit-exactly against the GPU result.
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


def gemm_event_time(run, reps):
    """Average duration of one launch of the dominant kernel, HIP events on the current
    stream (the stream the library launches on)."""
    import torch
    s = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    run()
    torch.cuda.synchronize()
    for e0, e1 in ev:
        e0.record(s)
        run()
        e1.record(s)
    torch.cuda.synchronize()
    ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    return float(np.mean(ms)), float(np.min(ms))


# arithmetic the SC GEMM computes in: every kernel counts integers exactly
DTYPE = {0: "int8 MFMA (exact int32 counts)", 1: "u32 popcount (exact int32 counts)",
         2: "e2m1 MFMA (exact integer counts in fp32)"}


def resolve_impl(name, tabs):
    """The kernel id the library runs for --impl `name` (auto follows sc/kernels.py)."""
    from scmp_kernels_amd import _lib
    if name == "valu":
        return _lib.GEMM_VALU
    if name == "int8":
        return _lib.GEMM_MFMA
    has4 = tabs.lut4(_lib.stream_of(tabs.lut.device)) is not None
    if name == "fp4" and not has4:
        raise SystemExit("--impl fp4: the stream table has counts e2m1 cannot represent")
    return _lib.GEMM_MFMA_FP4 if has4 else _lib.GEMM_MFMA


def kernel_roofline(impl, N, M, D, JP):
    """(ops per launch, peak in 1e12/s, unit, bound, kernel name) for the SC GEMM kernel.
    The MFMA kernels issue one multiply-add per (n, m, d, interval) over the padded interval
    extent (JP for int8, max(JP, 32) for FP4); the VALU kernel an AND and a popcount per
    32-interval word and bit plane."""
    if impl == 2:
        return (2.0 * N * M * D * max(JP, 32), MFMA_FP4_PEAK_TFLOPS, "TFLOP/s", "mfma",
                "sc_gemm_fp4_kernel")
    if impl == 0:
        return (2.0 * N * M * D * JP, MFMA_INT8_PEAK_TOPS, "TOP/s", "mfma",
                "sc_gemm_mfma_kernel")
    return (float(N * M * D * max(1, JP // 32) * 2 * 2), VALU_PEAK_TOPS, "TOP/s", "valu",
            "sc_gemm_valu_kernel")


def bench_cfg2(args):
    import torch
    from scmp_kernels_amd import sc_matmul, _lib
    from scmp_kernels_amd.sc import kernels as K
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

    # dominant kernel alone: the SC GEMM on pre-quantized codes, int32 output
    tabs = K._get_tables(None, 8, L, 256, True, D, dev)
    ca, cb = K._codes(N, D, dev), K._codes(M, D, dev)
    K.quantize(a, _lib.Q_GROUP_SYM, 127, 256, smooth=s, smooth_mode=_lib.SMOOTH_DIV, code=ca,
               code_kind=_lib.CODE_THERMO, jtab=tabs.jtab)
    K.quantize(b, _lib.Q_GROUP_SYM, 127, 256, smooth=s, smooth_mode=_lib.SMOOTH_MUL, code=cb,
               code_kind=_lib.CODE_Q)
    I = torch.empty((N, M), dtype=torch.int32, device=dev)
    epi = _lib.Epilogue()
    epi.kind = _lib.EPI_INT
    impl = resolve_impl(args.impl, tabs)

    def gemm():
        K.sc_gemm(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, iout=I, impl=impl)

    g_avg, g_min = gemm_event_time(gemm, max(3, args.steps))

    # the two quantizer launches of a step, each timed alone: algorithmic HBM bytes =
    # fp32 input read once + GEMM code bytes written (padded rows) + the smoothing vector
    def quant_a():
        K.quantize(a, _lib.Q_GROUP_SYM, 127, 256, smooth=s, smooth_mode=_lib.SMOOTH_DIV,
                   code=ca, code_kind=_lib.CODE_THERMO, jtab=tabs.jtab)

    def quant_b():
        K.quantize(b, _lib.Q_GROUP_SYM, 127, 256, smooth=s, smooth_mode=_lib.SMOOTH_MUL,
                   code=cb, code_kind=_lib.CODE_Q)

    quants = {}
    for name, fn, x, c in (("a", quant_a, a, ca), ("b", quant_b, b, cb)):
        q_avg, _ = gemm_event_time(fn, max(5, args.steps))
        nbytes = 4 * x.numel() + c.numel() + 4 * D
        quants[name] = {"shape": list(x.shape), "avg_us": round(q_avg * 1e3, 2),
                        "bytes": nbytes, "GB/s": round(nbytes / (q_avg * 1e-3) / 1e9, 1),
                        "frac_of_8TB/s": round(nbytes / (q_avg * 1e-3) / 8e12, 3)}
    log(f"quantizers: {quants}")
    log(f"SC GEMM kernel: avg {g_avg:.3f} ms, min {g_min:.3f} ms (JP={tabs.JP})")
    B = N * M * D * L
    ops, peak, unit, bound, kname = kernel_roofline(impl, N, M, D, tabs.JP)
    achieved = ops / (g_avg * 1e-3) / 1e12
    roof = {
        "bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
        "frac": round(achieved / peak, 4), "traffic": None,
        "kernel": kname, "avg_ms": round(g_avg, 4), "ops_per_launch": ops,
        "effective_sc_bitops_per_s": B / (g_avg * 1e-3),
    }
    tp = os.path.join(ROOT, "profiles", "cfg2_gemm_traffic.json")
    if os.path.exists(tp):
        with open(tp) as f:
            roof["traffic"] = json.load(f).get(kname, {}).get("traffic_bytes")

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
                   "granularity": "per_row", "gemm_kernel": kname},
        "roofline": roof,
        "quantizers": {"bound": "hbm", "peak_GB/s": 8000.0, **quants},
        "cpu_baseline": cpu,
    }


def bench_other(args):
    """The other BASELINE configurations, timed as whole calls (inputs resident in HBM,
    tables cached after the warmup); not the driver's headline metric."""
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
    elif args.config == "cfg4":
        q_h, k_h, p_h, vt_h = make_cfg4()
        q, k, p, vt = T(q_h), T(k_h), T(p_h), T(vt_h)
        B = 2 * 768 * 197 * 197 * 64 * 256
        desc = "attention per_head bipolar BH=768: QK^T (197x197x64) + P.V (197x64x197)"

        def step():
            sc_matmul(q, k, "per_head", sc_prec=8)
            return sc_matmul(p, vt, "per_head", sc_prec=8)
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
    else:
        raise SystemExit(f"unknown --config {args.config}")
    t, _ = time_steps(step, args.steps, args.warmup)
    log(f"{args.config}: {t * 1e3:.3f} ms per call")
    return {"metric": f"ms & SC bit-ops/s per call ({desc})", "value": B / t,
            "unit": "SC bit-ops/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(t * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "data": "synthetic (numpy PCG64, bench.py generators)",
            "config": {"workload": args.config, "sc_bit_ops": B}}


def profile_gemm(args):
    """One launch of the dominant kernel on the cfg2 operands, then one device copy of a
    known size (8 * 2^27 bytes each way) whose FETCH_SIZE / WRITE_SIZE counter values scale
    the GEMM's counters to bytes. Used under rocprofv3 --pmc."""
    import torch
    from scmp_kernels_amd import _lib
    from scmp_kernels_amd.sc import kernels as K
    from scmp_kernels_amd.quant import accumulate_act_scales, compute_smooth_scales
    dev = torch.device("cuda", 0)
    a_h, b_h = make_cfg2()
    a = torch.from_numpy(a_h).to(dev)
    b = torch.from_numpy(b_h).to(dev)
    s = compute_smooth_scales(accumulate_act_scales(a), b, alpha=0.5)
    N, D = a.shape
    M = b.shape[0]
    tabs = K._get_tables(None, 8, 256, 256, True, D, dev)
    ca, cb = K._codes(N, D, dev), K._codes(M, D, dev)
    K.quantize(a, _lib.Q_GROUP_SYM, 127, 256, smooth=s, smooth_mode=_lib.SMOOTH_DIV, code=ca,
               code_kind=_lib.CODE_THERMO, jtab=tabs.jtab)
    K.quantize(b, _lib.Q_GROUP_SYM, 127, 256, smooth=s, smooth_mode=_lib.SMOOTH_MUL, code=cb,
               code_kind=_lib.CODE_Q)
    I = torch.empty((N, M), dtype=torch.int32, device=dev)
    epi = _lib.Epilogue()
    epi.kind = _lib.EPI_INT
    impl = resolve_impl(args.impl, tabs)
    torch.cuda.synchronize()
    K.sc_gemm(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, iout=I, impl=impl,
              tile=args.tile)
    torch.cuda.synchronize()
    src = torch.ones(2 ** 28, dtype=torch.int32, device=dev)     # 1 GiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log("profile_gemm: one GEMM launch, then a 1 GiB device copy")


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
                    help="step: the benchmark (default); gemm: one dominant-kernel launch "
                         "plus a 1 GiB copy, for counter collection")
    ap.add_argument("--tile", type=int, default=0)
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

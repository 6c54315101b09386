"""Write golden vectors for the SC matmul path by running the reference implementation
(swalther06/scmp_kernels at /root/reference) under TRITON_INTERPRET=1 on the CPU.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/gen_golden.py [--ref /root/reference] [--out tests/golden]

What is run and why: the reference's fused Triton quantizers, its float64 host scale path
and the per-path fp32 epilogue order are pinned by no closed form; these vectors pin the
oracle's restatement of them. Two harness adaptations are needed for a GPU-less
interpreter run:

* ``libdevice.nearbyint`` is not implemented by this Triton's interpreter; it is replaced
  by a round-half-to-even written in ``tl`` ops (same function on every input);
* ``Tensor.cuda`` returns the tensor itself, so the reference's "move CPU inputs to the
  GPU" step (scmp_kernels/sc/kernels.py:1115-1117) is a no-op.

Inputs come from numpy's seeded PCG64 generator so the fixtures do not depend on torch's
RNG. Each case is written to ``<name>.npz`` (numeric arrays only, no pickles) with its
call arguments in ``cases.json``.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

os.environ["TRITON_INTERPRET"] = "1"

import triton  # noqa: E402  (after TRITON_INTERPRET is set)
import triton.language as tl  # noqa: E402


@triton.jit
def _rne(x):
    """Round half to even from floor and parity (stand-in for libdevice.nearbyint)."""
    f = tl.floor(x)
    d = x - f
    half_up = tl.where((f - 2.0 * tl.floor(f * 0.5)) == 0.0, f, f + 1.0)
    return tl.where(d > 0.5, f + 1.0, tl.where(d < 0.5, f, half_up))


def _install_shims(ref_root: str):
    sys.path.insert(0, ref_root)
    import torch

    class _LibdeviceShim:
        nearbyint = _rne

    torch.Tensor.cuda = lambda self, *a, **k: self  # noqa: E731
    import scmp_kernels.quant.fused as fused
    fused.libdevice = _LibdeviceShim()
    import scmp_kernels.sc.kernels as kernels
    kernels.libdevice = _LibdeviceShim()
    return torch


def _normal(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def _time_cfg1(out_dir, sc_matmul, clear_rng_cache, a, b, torch):
    """Time the reference's own cfg1 call (per_tensor bipolar, (32,256) x (64,256), L=256)
    under the interpreter: one cold call (sequences and tables built) and five warm calls
    (cached), wall clock. Written to ref_cpu_timing.json with the host description."""
    import platform
    import time
    import triton as _triton
    kw = {"granularity": "per_tensor", "sc_prec": 8, "stoc_len": 256}
    clear_rng_cache()
    t0 = time.perf_counter()
    sc_matmul(a, b, **kw)
    cold = time.perf_counter() - t0
    warm = []
    for _ in range(5):
        t0 = time.perf_counter()
        sc_matmul(a, b, **kw)
        warm.append(time.perf_counter() - t0)
    clear_rng_cache()
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    warm_s = sorted(warm)[len(warm) // 2]
    rec = {
        "what": "reference sc_matmul, BASELINE cfg1: per_tensor bipolar a(32,256) x b(64,256), "
                "sc_prec=8, stoc_len=256, under TRITON_INTERPRET=1 on the CPU",
        "sc_bitops_per_call": 32 * 64 * 256 * 256,
        "cold_s": round(cold, 4), "warm_median_s": round(warm_s, 4),
        "warm_sc_bitops_per_s": 32 * 64 * 256 * 256 / warm_s,
        "warm_s": [round(w, 4) for w in warm],
        "cores": 1,
        "cores_note": "the Triton interpreter runs each program instance in one Python "
                      "thread; torch.get_num_threads()=%d for the torch ops around it"
                      % torch.get_num_threads(),
        "host": {"cpu": cpu, "os_cpu_count": os.cpu_count(), "python": platform.python_version(),
                 "torch": torch.__version__, "triton": _triton.__version__,
                 "numpy": np.__version__},
    }
    with open(os.path.join(out_dir, "ref_cpu_timing.json"), "w") as f:
        json.dump(rec, f, indent=1)
    print(f"cfg1 reference timing: cold {cold:.3f} s, warm median {warm_s:.3f} s", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=os.path.dirname(os.path.abspath(__file__)))
    ap.add_argument("--only", default="",
                    help="comma-separated case names to (re)write; the others keep their "
                         "files and cases.json entries")
    ap.add_argument("--time-cfg1", action="store_true",
                    help="also time the reference's cfg1 sc_matmul (ref_cpu_timing.json)")
    args = ap.parse_args()
    only = set(filter(None, args.only.split(",")))
    torch = _install_shims(args.ref)
    from scmp_kernels import sc_matmul
    from scmp_kernels.sc import clear_rng_cache
    from scmp_kernels.sc import kernels as K
    from scmp_kernels import quant as Qm
    from scmp_kernels.sc.config_helpers import make_sobol_simple_config

    cases = {}
    cases_path = os.path.join(args.out, "cases.json")
    if only and os.path.exists(cases_path):
        with open(cases_path) as f:
            cases = json.load(f)

    def T(x):
        return torch.from_numpy(np.ascontiguousarray(x))

    def save(name, meta, **arrs):
        if only and name not in only:
            return
        path = os.path.join(args.out, f"{name}.npz")
        np.savez_compressed(path, **{k: np.asarray(v) for k, v in arrs.items()})
        cases[name] = meta
        print(f"wrote {name}: " + ", ".join(f"{k}{tuple(np.asarray(v).shape)}"
                                            for k, v in arrs.items()), flush=True)

    def run_matmul(name, a, b, kwargs, env=None, smooth=None):
        if only and name not in only:
            return
        env = env or {}
        old = {k: os.environ.get(k) for k in env}
        os.environ.update(env)
        clear_rng_cache()
        try:
            kw = dict(kwargs)
            if smooth is not None:
                kw["smooth_scales"] = T(smooth)
            y = sc_matmul(T(a), T(b), **kw)
        finally:
            for k, v in old.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
            clear_rng_cache()
        arrs = dict(a=a, b=b, y=y.numpy())
        if smooth is not None:
            arrs["smooth"] = smooth
        save(name, {"kind": "sc_matmul", "kwargs": kwargs, "env": env}, **arrs)

    # --- configuration 1 of BASELINE.json: per_tensor bipolar (32,256) x (64,256) -------
    rng = np.random.default_rng(0)
    a = _normal(rng, (32, 256))
    b = _normal(rng, (64, 256))
    run_matmul("cfg1_per_tensor_bipolar", a, b,
               {"granularity": "per_tensor", "sc_prec": 8, "stoc_len": 256})

    if args.time_cfg1:
        _time_cfg1(args.out, sc_matmul, clear_rng_cache, T(a), T(b), torch)

    rng = np.random.default_rng(101)
    run_matmul("per_tensor_unipolar", _normal(rng, (8, 64)), _normal(rng, (16, 64), 0.5),
               {"granularity": "per_tensor", "mode": "unipolar", "sc_prec": 8})

    rng = np.random.default_rng(102)
    a = _normal(rng, (8, 64))
    a[:, 7] *= 30.0
    b = _normal(rng, (16, 64), 0.5)
    s = (np.abs(a).max(axis=0) ** 0.5 / np.maximum(np.abs(b).max(axis=0), 1e-5) ** 0.5)
    s = np.maximum(s, 1e-5).astype(np.float32)
    run_matmul("per_row_bipolar_smooth", a, b, {"granularity": "per_row", "sc_prec": 8},
               smooth=s)

    rng = np.random.default_rng(103)
    run_matmul("per_row_bipolar_g3", _normal(rng, (10, 48)), _normal(rng, (7, 48)),
               {"granularity": "per_row", "sc_prec": 8, "group_a": 3, "group_b": 2})

    rng = np.random.default_rng(104)
    a = _normal(rng, (9, 64))
    a[2] = rng.standard_t(3, 64).astype(np.float32)
    b = _normal(rng, (10, 64), 0.02)
    for L in (256, 64, 16):
        run_matmul(f"per_row_unipolar_g4_L{L}", a, b,
                   {"granularity": "per_row", "mode": "unipolar", "sc_prec": 8,
                    "group_a": 4, "group_b": 4, "stoc_len": L, "rng_levels": L})

    rng = np.random.default_rng(105)
    a, b = _normal(rng, (6, 40)), _normal(rng, (5, 40))
    run_matmul("per_row_bipolar_halve", a, b,
               {"granularity": "per_row", "sc_prec": 8, "halve_bipolar_stoc_len": True})
    run_matmul("per_row_bipolar_prefix64", a, b,
               {"granularity": "per_row", "sc_prec": 8, "stoc_len": 64})
    run_matmul("per_row_bipolar_L64_counter", a, b,
               {"granularity": "per_row", "sc_prec": 8, "stoc_len": 64, "rng_levels": 64},
               env={"SC_OWEN_MODE": "counter"})
    run_matmul("per_row_bipolar_L32_norescale", a, b,
               {"granularity": "per_row", "sc_prec": 8, "stoc_len": 32, "rng_levels": 32},
               env={"SC_SCRAMBLE_RESCALE": "0"})
    run_matmul("per_row_bipolar_p6", a, b, {"granularity": "per_row", "sc_prec": 6})

    rng = np.random.default_rng(106)
    run_matmul("chunk_d_bipolar", _normal(rng, (8, 100)), _normal(rng, (12, 100), 0.02),
               {"granularity": "per_row", "sc_prec": 8, "chunk_d": 24})

    rng = np.random.default_rng(107)
    q = _normal(rng, (3, 10, 16))
    k = _normal(rng, (3, 12, 16))
    run_matmul("per_head_qk", q, k, {"granularity": "per_head", "sc_prec": 8})
    logits = _normal(rng, (2, 9, 11))
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p = (p / p.sum(-1, keepdims=True)).astype(np.float32)
    vt = _normal(rng, (2, 6, 11))
    run_matmul("per_head_pv", p, vt, {"granularity": "per_head", "sc_prec": 8})

    rng = np.random.default_rng(108)
    run_matmul("per_row_3d_bipolar", _normal(rng, (2, 6, 32)), _normal(rng, (2, 5, 32)),
               {"granularity": "per_row", "sc_prec": 8})
    run_matmul("per_row_3d_unipolar", _normal(rng, (2, 4, 32)), _normal(rng, (2, 3, 32)),
               {"granularity": "per_row", "mode": "unipolar", "sc_prec": 8})

    # --- RNG configurations other than the default Sobol (sc/sng.py:15-53, 187-230;
    #     sc/rng.py:32-113; Owen 'random', sc/kernels.py:664-668) ---------------------------
    import random as _random
    pr = _random.Random(2024)

    def perm8():
        p = list(range(8))
        pr.shuffle(p)
        return p

    D = 24
    q_s = [perm8() if i % 3 else None for i in range(D)]
    k_s = [perm8() if i % 2 else None for i in range(D)]
    cfg_shared = {"rng_pool": [{"type": "lfsr", "seed": 45, "taps": [7, 5, 4, 3]}],
                  "sng": {"q": [{"rng_id": 0, "scramble": s} for s in q_s],
                          "k": [{"rng_id": 0, "scramble": s} for s in k_s]}}
    cfg_multi = {"rng_pool": [{"type": "lfsr", "seed": 45, "taps": [7, 5, 4, 3]},
                              {"type": "lfsr", "seed": 3, "taps": [7, 6, 5, 0]},
                              {"type": "sobol", "seed_type": "k"}],
                 "sng": {"q": [{"rng_id": i % 2, "scramble": q_s[i]} for i in range(D)],
                         "k": [{"rng_id": 1 + i % 2, "scramble": k_s[i]} for i in range(D)]}}
    cfg_true = {"rng_pool": [{"type": "true_random", "seed": 7},
                             {"type": "true_random", "seed": 8}],
                "sng": {"q": [{"rng_id": 0, "scramble": None} for _ in range(D)],
                        "k": [{"rng_id": 1, "scramble": None} for _ in range(D)]}}
    rng = np.random.default_rng(111)
    a, b = _normal(rng, (6, D)), _normal(rng, (5, D))
    run_matmul("per_row_bipolar_lfsr_shared_scrambled", a, b,
               {"granularity": "per_row", "sc_prec": 8, "config": cfg_shared})
    run_matmul("per_row_bipolar_multi_rng_scrambled", a, b,
               {"granularity": "per_row", "sc_prec": 8, "config": cfg_multi})
    run_matmul("per_row_unipolar_multi_rng_L64", a, b,
               {"granularity": "per_row", "mode": "unipolar", "sc_prec": 8, "group_a": 2,
                "group_b": 2, "stoc_len": 64, "rng_levels": 64, "config": cfg_multi})
    run_matmul("per_row_bipolar_true_random", a, b,
               {"granularity": "per_row", "sc_prec": 8, "config": cfg_true})
    rng = np.random.default_rng(112)
    a, b = _normal(rng, (7, 40)), _normal(rng, (6, 40))
    run_matmul("per_row_bipolar_L64_owen_random", a, b,
               {"granularity": "per_row", "sc_prec": 8, "stoc_len": 64, "rng_levels": 64},
               env={"SC_OWEN_MODE": "random"})
    run_matmul("per_row_bipolar_prefix64_owen_random", a, b,
               {"granularity": "per_row", "sc_prec": 8, "stoc_len": 64},
               env={"SC_OWEN_MODE": "random"})

    # --- integer accumulator straight from the tiled kernel (q_max_sq = stoc_len) --------
    rng = np.random.default_rng(109)
    for (L, R, mode) in ((256, 256, "bipolar"), (64, 64, "unipolar"), (128, 128, "bipolar")):
        N, M, D = 5, 7, 40
        clear_rng_cache()
        cfg = make_sobol_simple_config(D, D, 8)
        ra, rb = K._get_cached_sequences(cfg, 8, torch.device("cpu"))
        cum, ktab = K._get_cached_enable_tables(cfg, 8, torch.device("cpu"), ra, rb, L,
                                                rng_levels=R)
        hi = R + 1
        ba = rng.integers(0, hi, (N, D)).astype(np.int16)
        bb = rng.integers(0, hi, (M, D)).astype(np.int16)
        if mode == "bipolar":
            sa = rng.choice(np.array([-1, 1], np.int8), (N, D))
            sb = rng.choice(np.array([-1, 1], np.int8), (M, D))
            I = K.enable_matmul_triton(cum, ktab, T(ba), T(bb), T(sa), T(sb), N, M, D, L,
                                       float(L), True)
        else:
            sa = np.zeros((N, D), np.int8)
            sb = np.zeros((M, D), np.int8)
            I = K.enable_matmul_triton(cum, ktab, T(ba), T(bb), None, None, N, M, D, L,
                                       float(L), False)
        save(f"accum_{mode}_L{L}_R{R}", {"kind": "accum", "L": L, "R": R, "mode": mode,
                                         "D": D},
             beta_a=ba, beta_b=bb, sign_a=sa, sign_b=sb, I=I.numpy(),
             ktab=ktab.numpy(), cum=cum.numpy())
        clear_rng_cache()

    # --- quantizer API outputs -----------------------------------------------------------
    rng = np.random.default_rng(110)
    x = _normal(rng, (6, 50))
    x[0, :5] = [0.0, 0.5, -0.5, 1.5, -2.5]       # exact halves and zero
    x[1] = 0.0                                   # all-zero row -> 1e-5 floor
    x[2, 3] = 1e-7
    bta, sg, sc = Qm.fused_quantize_bipolar_perrow(T(x), 8)
    save("q_fused_perrow", {"kind": "quant", "fn": "fused_quantize_bipolar_perrow",
                            "sc_prec": 8},
         x=x, beta=bta.numpy(), sign=sg.numpy(), scale=sc.numpy())
    absmax = float(np.abs(x).max())
    bta, sg, sc = Qm.fused_quantize_bipolar(T(x), absmax, 8)
    save("q_fused_tensor", {"kind": "quant", "fn": "fused_quantize_bipolar", "sc_prec": 8,
                            "abs_max": absmax},
         x=x, beta=bta.numpy(), sign=sg.numpy(), scale=np.float64(sc))
    for cs in (True, False):
        bta, sc, zp, rs = Qm.fused_quantize_unipolar(T(x), float(x.max()), float(x.min()), 8,
                                                     compute_sum=cs, rng_levels=64)
        arrs = dict(x=x, beta=bta.numpy(), scale=np.float64(sc), zp=np.float64(zp))
        if rs is not None:
            arrs["row_sum"] = rs.numpy()
        save(f"q_fused_unipolar_sum{int(cs)}", {"kind": "quant", "fn": "fused_quantize_unipolar",
                                               "sc_prec": 8, "rng_levels": 64,
                                               "compute_sum": cs}, **arrs)
    for G in (1, 4, 100):
        s_, xi, sg = Qm._grouped_symmetric_quant(T(x), G, 127)
        save(f"q_grouped_sym_G{G}", {"kind": "quant", "fn": "_grouped_symmetric_quant",
                                     "G": G, "q_max": 127},
             x=x, scale=s_.numpy(), x_int=xi.numpy(), sign=sg.numpy())
        s_, z_, xi = Qm._grouped_asymmetric_quant(T(x), G, 255)
        save(f"q_grouped_asym_G{G}", {"kind": "quant", "fn": "_grouped_asymmetric_quant",
                                      "G": G, "q_max": 255},
             x=x, scale=s_.numpy(), zp=z_.numpy(), x_int=xi.numpy())
    x3 = _normal(rng, (2, 5, 12))
    for G in (1, 5):
        s_, xi, sg = Qm._grouped_symmetric_quant_batched(T(x3), G, 127)
        save(f"q_grouped_sym_batched_G{G}", {"kind": "quant",
                                             "fn": "_grouped_symmetric_quant_batched",
                                             "G": G, "q_max": 127},
             x=x3, scale=s_.numpy(), x_int=xi.numpy(), sign=sg.numpy())

    with open(cases_path, "w") as f:
        json.dump(cases, f, indent=1, sort_keys=True)
    print(f"{len(cases)} cases", flush=True)


if __name__ == "__main__":
    main()

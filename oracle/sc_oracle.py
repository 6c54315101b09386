"""CPU oracle for the SC matmul path of swalther06/scmp_kernels.

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product (``scmp_kernels_amd``) never
does. It restates the reference's algorithm on the CPU:

* integer / byte work (RNG sequences, tables, the SC accumulator) in plain C
  (``oracle/sc_oracle.c``, built by ``oracle/Makefile``);
* fp32 quantizer and epilogue arithmetic with one IEEE rounding per operation, in C or
  numpy float32 (numpy performs no FMA contraction), in the reference's order.

Each function cites the reference file:line it follows (paths relative to the reference
repo root). What pins each function is listed in ``oracle/README.md``.
"""
from __future__ import annotations

import ctypes
import hashlib
import math
import os
import random
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libscoracle.so")
_lib = None

f32 = np.float32


def build() -> str:
    """Compile the C oracle (``make -C oracle``); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if os.path.exists(os.path.join(_HERE, "Makefile")) and os.access(_HERE, os.W_OK):
            build()                     # incremental: rebuilds only when the C file changed
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_bitrev.restype = ctypes.c_int32
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# -------------------------------------------------------------------------------------
# RNG sequences: scmp_kernels/sc/rng.py, scmp_kernels/sc/sng.py
# -------------------------------------------------------------------------------------

def sobol_default_seed(length: int, seed_type: str) -> list:
    """scmp_kernels/sc/rng.py:156-171."""
    if seed_type == "k":
        if length == 8:
            return [1, 1, 1, 1, 9, 1, 41, 255]
        seed = [1] * length
        if length >= 5:
            seed[4] = 9
        if length >= 7:
            seed[6] = 41
        return seed
    return [1] * length


def sobol_sequence(length: int, seed: list, n: int) -> np.ndarray:
    """scmp_kernels/sc/rng.py:173-225 (direction vectors + Gray-code stepping)."""
    s = np.asarray(seed, dtype=np.int64)
    V = np.zeros(length, dtype=np.int64)
    lib().orc_sobol_dirvec(ctypes.c_int(length), _p(s), _p(V))
    out = np.zeros(n, dtype=np.int32)
    lib().orc_sobol(ctypes.c_int(length), _p(V), ctypes.c_int64(n), _p(out))
    return out


def lfsr_sequence(length: int, seed: int, taps: list, n: int) -> np.ndarray:
    """scmp_kernels/sc/rng.py:32-77."""
    if seed == 0:
        raise ValueError("LFSR seed must be non-zero")
    t = np.asarray(taps, dtype=np.int32)
    out = np.zeros(n, dtype=np.int32)
    lib().orc_lfsr(ctypes.c_int(length), ctypes.c_int64(seed), _p(t), ctypes.c_int(len(t)),
                   ctypes.c_int64(n), _p(out))
    return out


def lfsr_distinct_states(taps: list, n: int) -> int:
    """Distinct register values from seed 1 before the first repeat, capped at 2^n
    (scmp_kernels/sc/lfsr_taps.py:99-111); a tap set is maximal when this is 2^n - 1."""
    t = np.asarray(taps, dtype=np.int32)
    f = lib().orc_lfsr_distinct
    f.restype = ctypes.c_int64
    return int(f(ctypes.c_int(n), _p(t), ctypes.c_int(len(t))))


def lfsr_search(n: int) -> list:
    """search_taps, scmp_kernels/sc/lfsr_taps.py:35-96: every maximal tap set, MSB plus an
    odd number of lower positions, in itertools.combinations order by tap count."""
    from itertools import combinations
    out = []
    for n_taps in range(2, n + 1, 2):
        for combo in combinations(range(n - 1), n_taps - 1):
            taps = sorted([n - 1] + list(combo), reverse=True)
            if lfsr_distinct_states(taps, n) == 2 ** n - 1:
                out.append(taps)
    return out


def true_random_sequence(length: int, seed: int, n: int) -> np.ndarray:
    """scmp_kernels/sc/rng.py:80-113 (Python's Mersenne Twister, randint(0, 2^len - 1))."""
    r = random.Random(seed)
    mx = 2 ** length - 1
    return np.array([r.randint(0, mx) for _ in range(n)], dtype=np.int32)


def rng_sequence(cfg: dict, sc_prec: int, n: int) -> np.ndarray:
    """scmp_kernels/sc/rng.py:242-268 (create_rng) + RNGPool defaults (sng.py:92-97)."""
    typ = cfg.get("type", "lfsr")
    if typ == "sobol":
        seed = cfg.get("seed")
        if seed is None:
            seed = sobol_default_seed(sc_prec, cfg.get("seed_type", "q"))
        return sobol_sequence(sc_prec, list(seed), n)
    if typ == "lfsr":
        return lfsr_sequence(sc_prec, cfg["seed"], cfg["taps"], n)
    if typ == "true_random":
        return true_random_sequence(sc_prec, cfg["seed"], n)
    raise ValueError(f"Unknown RNG type: {typ}")


def scramble(seq: np.ndarray, perm: list) -> np.ndarray:
    """scmp_kernels/sc/sng.py:15-29."""
    seq = np.ascontiguousarray(seq, dtype=np.int32)
    p = np.asarray(perm, dtype=np.int32)
    out = np.zeros_like(seq)
    lib().orc_scramble(_p(seq), ctypes.c_int64(seq.size), _p(p), ctypes.c_int(len(p)), _p(out))
    return out


def sng_sequences(config: dict, side: str, sc_prec: int) -> np.ndarray:
    """SNGBank.get_all_sequences, scmp_kernels/sc/sng.py:187-230, for side 'q' or 'k'.
    Sequences have length 2^sc_prec (scmp_kernels/sc/kernels.py:78-85)."""
    n = 2 ** sc_prec
    sngs = config["sng"][side]
    pool = config["rng_pool"]
    cache = {}

    def seq_of(rid):
        if rid not in cache:
            cache[rid] = rng_sequence(pool[rid], sc_prec, n)
        return cache[rid]

    ids = [s["rng_id"] for s in sngs]
    for rid in ids:
        seq_of(rid)
    if len(set(ids)) == 1:
        base = seq_of(ids[0])
        scr = [s.get("scramble") for s in sngs]
        if all(s is None for s in scr):
            return np.broadcast_to(base, (len(sngs), n)).copy()
        # apply_scramble_batch (sng.py:32-53): None -> identity over sc_prec bits
        out = np.zeros((len(sngs), n), dtype=np.int32)
        for i, s in enumerate(scr):
            out[i] = scramble(base, s if s is not None else list(range(sc_prec)))
        return out
    out = np.zeros((len(sngs), n), dtype=np.int32)
    for i, s in enumerate(sngs):
        base = seq_of(s["rng_id"])
        sc = s.get("scramble")
        out[i] = scramble(base, sc) if sc is not None else base
    return out


def make_sobol_simple_config(q_e: int, k_e: int, sc_prec: int = 8) -> dict:
    """scmp_kernels/sc/config_helpers.py:583-607."""
    return {
        "rng_pool": [{"type": "sobol", "seed_type": "q"}, {"type": "sobol", "seed_type": "k"}],
        "sng": {
            "q": [{"rng_id": 0, "scramble": None} for _ in range(q_e)],
            "k": [{"rng_id": 1, "scramble": None} for _ in range(k_e)],
        },
    }


# -------------------------------------------------------------------------------------
# Prefix / Owen / rescale and tables: scmp_kernels/sc/kernels.py:596-759
# -------------------------------------------------------------------------------------

OWEN_SEED = 0x5A5A5A5A  # scmp_kernels/sc/kernels.py:635


def owen_masks(D: int, base: int, mode: str = "bitrev", device="cpu") -> Optional[np.ndarray]:
    """scmp_kernels/sc/kernels.py:646-670. Returns per-d XOR masks or None (off).
    'random' is torch.randint(0, base, (D, 1)) from torch.Generator(device) seeded with
    0x5A5A5A5A, the generator of the device the sequences live on (kernels.py:664-668):
    "cpu" is the reference's draw for CPU tensors (pinned by a reference-run golden vector);
    a GPU device gives torch's device generator, which the product uses for device tensors
    (the values of that generator are torch's, not restated here)."""
    mode = mode.lower()
    if mode == "off":
        return None
    idx = np.arange(D, dtype=np.int64) % base
    if mode == "counter":
        return idx.astype(np.int32)
    if mode == "bitrev":
        nbits = int(round(math.log2(base)))
        return np.array([lib().orc_bitrev(int(i), nbits) for i in idx], dtype=np.int32)
    import torch
    g = torch.Generator(device=device).manual_seed(OWEN_SEED)
    m = torch.randint(0, base, (D, 1), generator=g, device=device)
    return m.reshape(D).cpu().numpy().astype(np.int32)


def prepare_prefix(r: np.ndarray, sc_prec: int, L: int, R: int, owen_mode: str = "bitrev",
                   scramble_rescale: bool = True, owen_device="cpu") -> np.ndarray:
    """_prepare_rng_prefix, scmp_kernels/sc/kernels.py:673-704. r: (D, 2^p) int32."""
    r = np.ascontiguousarray(r, dtype=np.int32)
    D, full = r.shape
    needs_mask = (L < full) if R == 2 ** sc_prec else scramble_rescale
    masks = owen_masks(D, 2 ** sc_prec, owen_mode, owen_device) if needs_mask else None
    out = np.zeros((D, L), dtype=np.int32)
    lib().orc_prepare_prefix(_p(r), ctypes.c_int(D), ctypes.c_int(full), ctypes.c_int(sc_prec),
                             ctypes.c_int(L), ctypes.c_int(R),
                             _p(masks) if masks is not None else None,
                             ctypes.c_int(1 if scramble_rescale else 0), _p(out))
    return out


def next_pow2(x: int) -> int:
    return 1 << (int(x) - 1).bit_length() if x > 1 else 1


def dedupe_rows(*arrs):
    """Map each row index d to the first row with identical content in every array."""
    D = arrs[0].shape[0]
    seen = {}
    tab_of = np.zeros(D, dtype=np.int32)
    uniq = []
    for d in range(D):
        h = hashlib.sha1(b"".join(a[d].tobytes() for a in arrs)).digest()
        if h not in seen:
            seen[h] = len(uniq)
            uniq.append(d)
        tab_of[d] = seen[h]
    return tab_of, np.asarray(uniq, dtype=np.int64)


def k_table(r: np.ndarray, V: int) -> np.ndarray:
    """compute_k_table_kernel, scmp_kernels/sc/kernels.py:140-169."""
    r = np.ascontiguousarray(r, dtype=np.int32)
    D, L = r.shape
    K = np.zeros((D, V), dtype=np.int16)
    lib().orc_k_table(_p(r), ctypes.c_int(D), ctypes.c_int(L), ctypes.c_int(V), _p(K))
    return K


def c_table(r: np.ndarray, V: int) -> np.ndarray:
    """build_cum_indicator_kernel, scmp_kernels/sc/kernels.py:102-137."""
    r = np.ascontiguousarray(r, dtype=np.int32)
    D, L = r.shape
    C = np.zeros((D, L + 1, V), dtype=np.int16)
    lib().orc_c_table(_p(r), ctypes.c_int(D), ctypes.c_int(L), ctypes.c_int(V), _p(C))
    return C


class Tables:
    """K / C tables for one (config, sc_prec, L, R) with identical per-d rows stored once
    (the reference stores D copies; values are the same)."""

    def __init__(self, config: dict, sc_prec: int, L: int, R: int,
                 owen_mode: str = "bitrev", scramble_rescale: bool = True,
                 owen_device="cpu"):
        ra_full = sng_sequences(config, "q", sc_prec)
        rb_full = sng_sequences(config, "k", sc_prec)
        self.ra = prepare_prefix(ra_full, sc_prec, L, R, owen_mode, scramble_rescale,
                                 owen_device)
        self.rb = prepare_prefix(rb_full, sc_prec, L, R, owen_mode, scramble_rescale,
                                 owen_device)
        self.L, self.R = L, R
        self.V = next_pow2(R + 1)  # scmp_kernels/sc/kernels.py:737-739
        self.tab_of, uniq = dedupe_rows(self.ra, self.rb)
        self.K = k_table(self.ra[uniq], self.V)
        self.C = c_table(self.rb[uniq], self.V)
        self.D = self.ra.shape[0]

    def sub(self, d0: int, d1: int):
        """Tables for dimensions [d0, d1) (chunked path uses rows 0..d_len-1)."""
        t = Tables.__new__(Tables)
        t.ra, t.rb = self.ra[d0:d1], self.rb[d0:d1]
        t.L, t.R, t.V, t.K, t.C, t.D = self.L, self.R, self.V, self.K, self.C, d1 - d0
        t.tab_of = np.ascontiguousarray(self.tab_of[d0:d1])
        return t


def sc_accum(beta_a, s_a, beta_b, s_b, tabs: Tables, nthreads: int = 1) -> np.ndarray:
    """Integer accumulator I[n,m] (scmp_kernels/sc/kernels.py:216-245), int32."""
    beta_a = np.ascontiguousarray(beta_a, dtype=np.int16)
    beta_b = np.ascontiguousarray(beta_b, dtype=np.int16)
    N, D = beta_a.shape
    M = beta_b.shape[0]
    assert D == tabs.D, (D, tabs.D)
    sa = np.ascontiguousarray(s_a, dtype=np.int8) if s_a is not None else None
    sb = np.ascontiguousarray(s_b, dtype=np.int8) if s_b is not None else None
    I = np.zeros((N, M), dtype=np.int32)
    lib().orc_sc_accum(_p(beta_a), _p(sa) if sa is not None else None, _p(beta_b),
                       _p(sb) if sb is not None else None, ctypes.c_int(N), ctypes.c_int(M),
                       ctypes.c_int(D), _p(tabs.K), _p(tabs.C), _p(tabs.tab_of),
                       ctypes.c_int(tabs.L), ctypes.c_int(tabs.V), _p(I),
                       ctypes.c_int(nthreads))
    return I


def sc_accum_stream(beta_a, s_a, beta_b, s_b, ra, rb) -> np.ndarray:
    """I[n,m] evaluated straight from the streams (no tables), for tiny inputs."""
    beta_a = np.ascontiguousarray(beta_a, dtype=np.int16)
    beta_b = np.ascontiguousarray(beta_b, dtype=np.int16)
    ra = np.ascontiguousarray(ra, dtype=np.int32)
    rb = np.ascontiguousarray(rb, dtype=np.int32)
    N, D = beta_a.shape
    M = beta_b.shape[0]
    sa = np.ascontiguousarray(s_a, dtype=np.int8) if s_a is not None else None
    sb = np.ascontiguousarray(s_b, dtype=np.int8) if s_b is not None else None
    I = np.zeros((N, M), dtype=np.int32)
    lib().orc_sc_accum_stream(_p(beta_a), _p(sa) if sa is not None else None, _p(beta_b),
                              _p(sb) if sb is not None else None, ctypes.c_int(N),
                              ctypes.c_int(M), ctypes.c_int(D), _p(ra), _p(rb),
                              ctypes.c_int(ra.shape[1]), _p(I))
    return I


# -------------------------------------------------------------------------------------
# Quantizers: scmp_kernels/quant/fused.py, scmp_kernels/quant/grouped.py
# -------------------------------------------------------------------------------------

def _c32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def quant_fused_perrow_bipolar(x, sc_prec: int, R: int):
    """fused_quantize_bipolar_perrow, scmp_kernels/quant/fused.py:134-159."""
    x = _c32(x)
    rows, cols = x.shape
    Q = 2 ** (sc_prec - 1) - 1
    beta = np.zeros((rows, cols), np.int16)
    sign = np.zeros((rows, cols), np.int8)
    scale = np.zeros(rows, np.float32)
    lib().orc_quant_fused_perrow_bipolar(_p(x), ctypes.c_int(rows), ctypes.c_int(cols),
                                         ctypes.c_int(Q), ctypes.c_int(R), _p(beta), _p(sign),
                                         _p(scale))
    return beta, sign, scale


def quant_fused_bipolar(x, abs_max: float, sc_prec: int, R: int):
    """fused_quantize_bipolar (per-tensor), scmp_kernels/quant/fused.py:162-189: host
    float64 scale, its reciprocal passed to the kernel as fp32."""
    x = _c32(x)
    Q = 2 ** (sc_prec - 1) - 1
    abs_max = max(abs_max, 1e-5)
    scale = abs_max / Q
    inv = 1.0 / scale
    beta = np.zeros(x.shape, np.int16)
    sign = np.zeros(x.shape, np.int8)
    lib().orc_quant_fused_flat_bipolar(_p(x), ctypes.c_int64(x.size), ctypes.c_float(inv),
                                       ctypes.c_int(Q), ctypes.c_int(R), _p(beta), _p(sign))
    return beta, sign, scale


def quant_fused_unipolar(x, fp_max: float, fp_min: float, sc_prec: int, R: int,
                         compute_sum: bool = True):
    """fused_quantize_unipolar, scmp_kernels/quant/fused.py:192-234."""
    x = _c32(x)
    rows, cols = x.shape
    Q = 2 ** sc_prec - 1
    range_fp = max(fp_max - fp_min, 1e-5)
    scale = range_fp / Q
    inv = 1.0 / scale
    zp = round(-fp_min / scale)
    zp = max(0, min(Q, zp))
    zp_f = float(zp)
    beta = np.zeros((rows, cols), np.int32)
    rowsum = np.zeros(rows, np.float32) if compute_sum else None
    lib().orc_quant_fused_unipolar(_p(x), ctypes.c_int(rows), ctypes.c_int(cols),
                                   ctypes.c_float(inv), ctypes.c_float(zp_f), ctypes.c_int(Q),
                                   ctypes.c_int(R), _p(beta),
                                   _p(rowsum) if rowsum is not None else None)
    return beta, scale, zp_f, rowsum


def quant_batched_bipolar(x, inv: np.ndarray, sc_prec: int, R: int):
    """fused_quant_bipolar_batched_kernel, scmp_kernels/quant/fused.py:237-283:
    returns boundary/sign in the transposed (BH, cols, rows) layout."""
    x = _c32(x)
    BH, rows, cols = x.shape
    Q = 2 ** (sc_prec - 1) - 1
    inv = _c32(inv)
    beta = np.zeros((BH, cols, rows), np.int16)
    sign = np.zeros((BH, cols, rows), np.int8)
    lib().orc_quant_batched_bipolar(_p(x), ctypes.c_int(BH), ctypes.c_int(rows),
                                    ctypes.c_int(cols), _p(inv), ctypes.c_int(Q),
                                    ctypes.c_int(R), _p(beta), _p(sign))
    return beta, sign


def grouped_sym(x, G: int, Q: int):
    """_grouped_symmetric_quant, scmp_kernels/quant/grouped.py:13-75."""
    x = _c32(x)
    rows, cols = x.shape
    scale = np.zeros(rows, np.float32)
    xi = np.zeros((rows, cols), np.float32)
    sign = np.zeros((rows, cols), np.int8)
    lib().orc_grouped_sym(_p(x), ctypes.c_int(rows), ctypes.c_int(cols), ctypes.c_int(G),
                          ctypes.c_int(Q), _p(scale), _p(xi), _p(sign))
    return scale, xi, sign


def grouped_asym(x, G: int, Q: int):
    """_grouped_asymmetric_quant, scmp_kernels/quant/grouped.py:78-133."""
    x = _c32(x)
    rows, cols = x.shape
    scale = np.zeros(rows, np.float32)
    zp = np.zeros(rows, np.float32)
    xi = np.zeros((rows, cols), np.float32)
    lib().orc_grouped_asym(_p(x), ctypes.c_int(rows), ctypes.c_int(cols), ctypes.c_int(G),
                           ctypes.c_int(Q), _p(scale), _p(zp), _p(xi))
    return scale, zp, xi


def grouped_sym_batched(x, G: int, Q: int):
    """_grouped_symmetric_quant_batched, scmp_kernels/quant/grouped.py:136-163."""
    x = _c32(x)
    BH, rows, cols = x.shape
    if G >= rows:
        sc, xi, sg = zip(*[grouped_sym(x[b], rows, Q) for b in range(BH)])
    elif G == 1:
        sc, xi, sg = zip(*[grouped_sym(x[b], 1, Q) for b in range(BH)])
    else:
        raise NotImplementedError(
            f"_grouped_symmetric_quant_batched: G={G} not supported (use G=1 or G>=rows)")
    return np.stack(sc), np.stack(xi), np.stack(sg)


def beta_div(q: np.ndarray, Q: int, R: int, absval: bool = True) -> np.ndarray:
    """(|q| * R / Q).round().short(), scmp_kernels/sc/kernels.py:1679-1686."""
    q = _c32(q)
    out = np.zeros(q.shape, np.int16)
    lib().orc_beta_from_q_div(_p(q), ctypes.c_int64(q.size), ctypes.c_int(Q), ctypes.c_int(R),
                              ctypes.c_int(1 if absval else 0), _p(out))
    return out


def beta_mul(q: np.ndarray, Q: int, R: int) -> np.ndarray:
    """(|q| * (R / Q)).round().short(), scmp_kernels/sc/kernels.py:1864-1865."""
    q = _c32(q)
    out = np.zeros(q.shape, np.int16)
    lib().orc_beta_from_q_mul(_p(q), ctypes.c_int64(q.size), ctypes.c_int(Q), ctypes.c_int(R),
                              _p(out))
    return out


# -------------------------------------------------------------------------------------
# SmoothQuant helpers (scmp_kernels/quant/smoothquant.py:97-126)
# -------------------------------------------------------------------------------------

def apply_smoothing(a, b, s):
    """(a / s, b * s) in fp32, scmp_kernels/quant/smoothquant.py:124-126."""
    s = _c32(s)
    return (_c32(a) / s).astype(f32), (_c32(b) * s).astype(f32)


# -------------------------------------------------------------------------------------
# sc_matmul dispatch (scmp_kernels/sc/matmul.py:81-279) with the per-path epilogues
# -------------------------------------------------------------------------------------

def _inner_scale(Q: int, L: int) -> np.float32:
    """q_max_sq / stoc_len in fp32 (scmp_kernels/sc/kernels.py:212, 397)."""
    return f32(f32(Q * Q) / f32(L))


def _row_epilogue(I, c, sa, sb):
    """fl(fl(I*c) * fl(sa*sb)) (kernels.py:248 then :1707 / :1271 / :1894)."""
    raw = (I.astype(f32) * c).astype(f32)
    return (raw * (sa[:, None] * sb[None, :]).astype(f32)).astype(f32)


def _grouped_zp_epilogue(I, c, sa, za, suma, sb, zb, sumb, D):
    """Zero-point correction then scale, scmp_kernels/sc/kernels.py:1699-1707."""
    raw = (I.astype(f32) * c).astype(f32)
    t1 = ((-zb)[None, :] * suma[:, None]).astype(f32)
    t2 = (za[:, None] * sumb[None, :]).astype(f32)
    t3 = ((f32(D) * za)[:, None] * zb[None, :]).astype(f32)
    corr = ((t1 - t2).astype(f32) + t3).astype(f32)
    raw = (raw + corr).astype(f32)
    return (raw * (sa[:, None] * sb[None, :]).astype(f32)).astype(f32)


class Ctx:
    """Options that the reference reads from the environment per call
    (scmp_kernels/sc/kernels.py:648-701)."""

    def __init__(self, owen_mode="bitrev", scramble_rescale=True, nthreads=1,
                 owen_device="cpu"):
        self.owen_mode = owen_mode
        self.scramble_rescale = scramble_rescale
        self.nthreads = nthreads
        self.owen_device = owen_device   # device whose generator draws 'random' masks


def _tables(config, sc_prec, L, R, ctx):
    return Tables(config, sc_prec, L, R, ctx.owen_mode, ctx.scramble_rescale,
                  ctx.owen_device)


def sc_matmul(a, b, granularity="per_row", *, mode="bipolar", sc_prec=8, stoc_len=None,
              chunk_d=0, group_a=1, group_b=1, rng_levels=None, config=None,
              halve_bipolar_stoc_len=False, smooth_scales=None, ctx: Ctx = None,
              return_parts=False):
    """Oracle of scmp_kernels.sc_matmul (scmp_kernels/sc/matmul.py:81-279). Inputs are
    numpy arrays (float32). Returns Y (float32) or (Y, parts) with the integer
    accumulator(s) and quantized operands when return_parts."""
    ctx = ctx or Ctx()
    a = _c32(a)
    b = _c32(b)
    if granularity not in ("per_tensor", "per_row", "per_head"):
        raise ValueError(f"sc_matmul: unknown granularity '{granularity}'.")
    if mode not in ("bipolar", "unipolar"):
        raise ValueError(f"sc_matmul: unknown mode '{mode}'.")
    if halve_bipolar_stoc_len and mode == "bipolar":
        halved = 2 ** (sc_prec - 1)
        if stoc_len is None:
            stoc_len = halved
        if rng_levels is None:
            rng_levels = halved
    if smooth_scales is not None:
        a, b = apply_smoothing(a, b, smooth_scales)
    L = stoc_len if stoc_len is not None else 2 ** sc_prec
    R = rng_levels if rng_levels is not None else 2 ** sc_prec
    parts = {}

    if granularity == "per_tensor":
        amax, amin = float(a.max()), float(a.min())
        bmax, bmin = float(b.max()), float(b.min())
        if a.ndim == 3:
            ys = [_per_tensor_2d(a[i], b[i], amax, amin, bmax, bmin, mode, sc_prec, L, R,
                                 config, ctx, {}) for i in range(a.shape[0])]
            Y = np.stack(ys)
        else:
            Y = _per_tensor_2d(a, b, amax, amin, bmax, bmin, mode, sc_prec, L, R, config,
                               ctx, parts)
    elif granularity == "per_row":
        if chunk_d > 0 and a.ndim == 2 and mode == "bipolar" and a.shape[1] > chunk_d:
            Y = _per_row_chunked(a, b, sc_prec, L, R, chunk_d, config, ctx, parts)
        elif a.ndim == 3:
            Y = _per_row_batched(a, b, group_a, group_b, mode, sc_prec, L, R, config, ctx,
                                 parts)
        else:
            Y = _per_row_2d(a, b, group_a, group_b, mode, sc_prec, L, R, config, ctx, parts)
    else:
        Y = _per_head(a, b, sc_prec, L, R, config, ctx, parts)
    return (Y, parts) if return_parts else Y


def _per_tensor_2d(a, b, amax, amin, bmax, bmin, mode, sc_prec, L, R, config, ctx, parts):
    """_sc_matmul_per_tensor + _sc_matmul_enable_triton,
    scmp_kernels/sc/kernels.py:1054-1204."""
    N, D = a.shape
    M = b.shape[0]
    if config is None:
        config = make_sobol_simple_config(D, D, sc_prec)
    tabs = _tables(config, sc_prec, L, R, ctx)
    if mode == "bipolar":
        Q = 2 ** (sc_prec - 1) - 1
        abs_a = max(abs(amax), abs(amin), 1e-5)
        abs_b = max(abs(bmax), abs(bmin), 1e-5)
        ba, sga, sa = quant_fused_bipolar(a, abs_a, sc_prec, R)
        bb, sgb, sb = quant_fused_bipolar(b, abs_b, sc_prec, R)
        I = sc_accum(ba, sga, bb, sgb, tabs, ctx.nthreads)
        raw = (I.astype(f32) * _inner_scale(Q, L)).astype(f32)
        Y = (raw * f32(sa * sb)).astype(f32)
        parts.update(I=I, beta_a=ba, sign_a=sga, beta_b=bb, sign_b=sgb, scale_a=sa, scale_b=sb)
        return Y
    Q = 2 ** sc_prec - 1
    ba, sa, za, suma = quant_fused_unipolar(a, amax, amin, sc_prec, R, True)
    bb, sb, zb, sumb = quant_fused_unipolar(b, bmax, bmin, sc_prec, R, True)
    I = sc_accum(ba.astype(np.int16), None, bb.astype(np.int16), None, tabs, ctx.nthreads)
    raw = (I.astype(f32) * _inner_scale(Q, L)).astype(f32)
    t1 = (f32(-zb) * suma[:, None]).astype(f32)
    t2 = (f32(za) * sumb[None, :]).astype(f32)
    corr = ((t1 - t2).astype(f32) + f32(D * za * zb)).astype(f32)
    raw = (raw + corr).astype(f32)
    parts.update(I=I, beta_a=ba, beta_b=bb, scale_a=sa, scale_b=sb, zp_a=za, zp_b=zb)
    return (raw * f32(sa * sb)).astype(f32)


def _per_row_2d(a, b, group_a, group_b, mode, sc_prec, L, R, config, ctx, parts):
    """_sc_matmul_per_row + _sc_matmul_grouped_enable, scmp_kernels/sc/kernels.py:1574-1707
    (also the D <= chunk_d fallback of _sc_matmul_per_row_mlp, :1522-1566, whose bipolar
    arithmetic is the same)."""
    N, D = a.shape
    M = b.shape[0]
    if config is None:
        config = make_sobol_simple_config(D, D, sc_prec)
    tabs = _tables(config, sc_prec, L, R, ctx)
    if mode == "bipolar":
        Q = 2 ** (sc_prec - 1) - 1
        sa, qa, sga = grouped_sym(a, group_a, Q)
        sb, qb, sgb = grouped_sym(b, group_b, Q)
        ba, bb = beta_div(qa, Q, R), beta_div(qb, Q, R)
        I = sc_accum(ba, sga, bb, sgb, tabs, ctx.nthreads)
        parts.update(I=I, q_a=qa, q_b=qb, beta_a=ba, beta_b=bb, sign_a=sga, sign_b=sgb,
                     scale_a=sa, scale_b=sb)
        return _row_epilogue(I, _inner_scale(Q, L), sa, sb)
    Q = 2 ** sc_prec - 1
    sa, za, qa = grouped_asym(a, group_a, Q)
    sb, zb, qb = grouped_asym(b, group_b, Q)
    ba, bb = beta_div(qa, Q, R, False), beta_div(qb, Q, R, False)
    I = sc_accum(ba, None, bb, None, tabs, ctx.nthreads)
    suma = qa.sum(axis=1, dtype=np.float64).astype(f32)
    sumb = qb.sum(axis=1, dtype=np.float64).astype(f32)
    parts.update(I=I, q_a=qa, q_b=qb, beta_a=ba, beta_b=bb, scale_a=sa, scale_b=sb, zp_a=za,
                 zp_b=zb)
    return _grouped_zp_epilogue(I, _inner_scale(Q, L), sa, za, suma, sb, zb, sumb, D)


def _per_row_batched(a, b, group_a, group_b, mode, sc_prec, L, R, config, ctx, parts):
    """_sc_matmul_per_row_batched, scmp_kernels/sc/kernels.py:1779-1895."""
    BH, Ma, D = a.shape
    if config is None:
        config = make_sobol_simple_config(D, D, sc_prec)
    if mode == "unipolar":
        return np.stack([_per_row_2d(a[i], b[i], group_a, group_b, mode, sc_prec, L, R,
                                     config, ctx, {}) for i in range(BH)])
    Q = 2 ** (sc_prec - 1) - 1
    tabs = _tables(config, sc_prec, L, R, ctx)
    sa, qa, sga = grouped_sym_batched(a, group_a, Q)
    sb, qb, sgb = grouped_sym_batched(b, group_b, Q)
    ba, bb = beta_mul(qa, Q, R), beta_mul(qb, Q, R)
    c = _inner_scale(Q, L)
    out, Is = [], []
    for i in range(BH):
        I = sc_accum(ba[i], sga[i], bb[i], sgb[i], tabs, ctx.nthreads)
        Is.append(I)
        out.append(_row_epilogue(I, f32(c * f32(1.0)), sa[i], sb[i]))
    parts.update(I=np.stack(Is))
    return np.stack(out)


def _per_row_chunked(a, b, sc_prec, L, R, chunk_d, config, ctx, parts):
    """_sc_matmul_per_row_mlp fast path + _sc_matmul_bipolar_mlp_chunked,
    scmp_kernels/sc/kernels.py:1499-1520, 1274-1383."""
    N, D = a.shape
    M = b.shape[0]
    Q = 2 ** (sc_prec - 1) - 1
    if config is None:
        config = make_sobol_simple_config(chunk_d, chunk_d, sc_prec)
    tabs = _tables(config, sc_prec, L, R, ctx)
    c = _inner_scale(Q, L)
    out = np.zeros((N, M), np.float32)
    Is = []
    for d0 in range(0, D, chunk_d):
        d1 = min(d0 + chunk_d, D)
        ba, sga, sa = quant_fused_perrow_bipolar(a[:, d0:d1], sc_prec, R)
        bb, sgb, sb = quant_fused_perrow_bipolar(b[:, d0:d1], sc_prec, R)
        I = sc_accum(ba, sga, bb, sgb, tabs.sub(0, d1 - d0), ctx.nthreads)
        Is.append(I)
        partial = (I.astype(f32) * c).astype(f32)
        out = (out + (partial * (sa[:, None] * sb[None, :]).astype(f32)).astype(f32)).astype(f32)
    parts.update(I_chunks=Is)
    return out


def _per_head(a, b, sc_prec, L, R, config, ctx, parts, ranges=None):
    """per_head dispatch (scmp_kernels/sc/matmul.py:264-279) + _sc_matmul_per_head_bipolar
    (scmp_kernels/sc/kernels.py:440-585). ranges: the caller's per-head (q_maxs, q_mins,
    k_maxs, k_mins), float32 (BH,) each; None: the heads' own max / min (matmul.py:271-274)."""
    BH, N, D = a.shape
    M = b.shape[1]
    if config is None:
        config = make_sobol_simple_config(D, D, sc_prec)
    Q = 2 ** (sc_prec - 1) - 1
    if ranges is None:
        amax = a.reshape(BH, -1).max(axis=1)
        amin = a.reshape(BH, -1).min(axis=1)
        bmax = b.reshape(BH, -1).max(axis=1)
        bmin = b.reshape(BH, -1).min(axis=1)
    else:
        amax, amin, bmax, bmin = (np.asarray(r, dtype=f32).reshape(BH) for r in ranges)
    eps = f32(1e-5)
    Aq = np.maximum(np.maximum(np.abs(amax), np.abs(amin)), eps).astype(f32)
    Ak = np.maximum(np.maximum(np.abs(bmax), np.abs(bmin)), eps).astype(f32)
    sq = (Aq / f32(Q)).astype(f32)
    sk = (Ak / f32(Q)).astype(f32)
    iq = (f32(1.0) / sq).astype(f32)
    ik = (f32(1.0) / sk).astype(f32)
    bq_t, sgq_t = quant_batched_bipolar(a, iq, sc_prec, R)
    bk_t, sgk_t = quant_batched_bipolar(b, ik, sc_prec, R)
    tabs = _tables(config, sc_prec, L, R, ctx)
    hs = (sq * sk).astype(f32)
    c = _inner_scale(Q, L)
    out, Is = [], []
    for h in range(BH):
        I = sc_accum(bq_t[h].T, sgq_t[h].T, bk_t[h].T, sgk_t[h].T, tabs, ctx.nthreads)
        Is.append(I)
        out.append((I.astype(f32) * f32(c * hs[h])).astype(f32))
    parts.update(I=np.stack(Is), scale_q=sq, scale_k=sk)
    return np.stack(out)


# -------------------------------------------------------------------------------------
# Mixed-precision row classifier (scmp_kernels/mp/config.py:154-191)
# -------------------------------------------------------------------------------------

def sc_matmul_per_tensor(a, b, max_fp_a, min_fp_a, max_fp_b=None, min_fp_b=None,
                         mode="bipolar", sc_prec=8, config=None, stoc_len=None,
                         rng_levels=None, ctx: Ctx = None):
    """_sc_matmul_per_tensor with the caller's ranges, scmp_kernels/sc/kernels.py:1054-1153
    (b's range defaults to a's, :1090-1093; 3-D runs every batch with the same ranges,
    :1207-1226)."""
    ctx = ctx or Ctx()
    a, b = _c32(a), _c32(b)
    L = stoc_len if stoc_len is not None else 2 ** sc_prec
    R = rng_levels if rng_levels is not None else 2 ** sc_prec
    if max_fp_b is None:
        max_fp_b = max_fp_a
    if min_fp_b is None:
        min_fp_b = min_fp_a
    rng = (float(max_fp_a), float(min_fp_a), float(max_fp_b), float(min_fp_b))
    if a.ndim == 3:
        return np.stack([_per_tensor_2d(a[i], b[i], *rng, mode, sc_prec, L, R, config, ctx,
                                        {}) for i in range(a.shape[0])])
    return _per_tensor_2d(a, b, *rng, mode, sc_prec, L, R, config, ctx, {})


def sc_matmul_per_head_bipolar(q, k, q_maxs, q_mins, k_maxs, k_mins, sc_prec, config,
                               stoc_len=None, rng_levels=None, ctx: Ctx = None):
    """_sc_matmul_per_head_bipolar with the caller's per-head ranges,
    scmp_kernels/sc/kernels.py:440-585."""
    ctx = ctx or Ctx()
    L = stoc_len if stoc_len is not None else 2 ** sc_prec
    R = rng_levels if rng_levels is not None else 2 ** sc_prec
    return _per_head(_c32(q), _c32(k), sc_prec, L, R, config, ctx, {},
                     ranges=(q_maxs, q_mins, k_maxs, k_mins))


def sc_matmul_per_row_mlp(a, b, max_fp_a=0.0, min_fp_a=0.0, max_fp_b=None, min_fp_b=None,
                          mode="bipolar", sc_prec=8, config=None, group_a=1, group_b=1,
                          chunk_d=0, stoc_len=None, rng_levels=None, ctx: Ctx = None):
    """_sc_matmul_per_row_mlp, scmp_kernels/sc/kernels.py:1444-1566: bipolar with
    chunk_d < D takes the chunked path (:1499-1521); other bipolar calls the row-group path
    (:1548-1553, = _sc_matmul_per_row's, :1683-1686, :1718); unipolar quantizes per tensor
    with the caller's ranges (:1555-1559, 1386-1418, = _sc_matmul_per_tensor's). 3-D runs
    each batch with the ranges and without groups or chunks (:1421-1441)."""
    ctx = ctx or Ctx()
    a, b = _c32(a), _c32(b)
    L = stoc_len if stoc_len is not None else 2 ** sc_prec
    R = rng_levels if rng_levels is not None else 2 ** sc_prec
    if max_fp_b is None:
        max_fp_b = max_fp_a
    if min_fp_b is None:
        min_fp_b = min_fp_a
    if a.ndim == 3:
        return np.stack([sc_matmul_per_row_mlp(a[i], b[i], max_fp_a, min_fp_a, max_fp_b,
                                               min_fp_b, mode, sc_prec, config,
                                               stoc_len=stoc_len, rng_levels=rng_levels,
                                               ctx=ctx) for i in range(a.shape[0])])
    D = a.shape[1]
    if mode == "bipolar" and chunk_d > 0 and D > chunk_d:
        return _per_row_chunked(a, b, sc_prec, L, R, chunk_d, config, ctx, {})
    if mode == "bipolar":
        return _per_row_2d(a, b, max(group_a, 1), max(group_b, 1), mode, sc_prec, L, R,
                           config, ctx, {})
    if mode != "unipolar":
        raise ValueError(f"Unknown mode: {mode}")
    return _per_tensor_2d(a, b, float(max_fp_a), float(min_fp_a), float(max_fp_b),
                          float(min_fp_b), mode, sc_prec, L, R, config, ctx, {})


def classify_rows_by_metric(metric: np.ndarray, levels: list, fractions: list):
    """Rank rows by metric (descending, stable like torch's argsort on CPU is NOT
    guaranteed; ties are rare for float metrics), bucket by rounded fractions."""
    N = metric.shape[0]
    order = np.argsort(-metric, kind="stable")
    row_levels = np.zeros(N, dtype=np.int64)
    rows_of = {}
    off = 0
    for i, (sl, fr) in enumerate(zip(levels, fractions)):
        cnt = round(fr * N) if i < len(levels) - 1 else N - off
        cnt = max(0, min(cnt, N - off))
        rows = order[off:off + cnt]
        row_levels[rows] = i
        rows_of[sl] = rows
        off += cnt
    return row_levels, rows_of

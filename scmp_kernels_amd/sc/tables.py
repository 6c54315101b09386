"""RNG sequences and SC GEMM stream tables, built on the GPU and cached per configuration.

Replaces the reference's sequence/table pipeline:
  RNGPool / SNGBank (scmp_kernels/sc/sng.py:69-230) + Sobol / LFSR / TrueRandom
  (scmp_kernels/sc/rng.py:32-268)            -> scmp_rng_sobol / scmp_rng_lfsr / scmp_rng_expand
  _owen_scramble / _prepare_rng_prefix (scmp_kernels/sc/kernels.py:646-704) -> scmp_rng_prepare
  build_enable_tables / k & cum tables (kernels.py:102-169, 712-795) -> scmp_build_stream_tables

A "table class" is a set of inner dimensions d whose prepared A and B sequences are equal;
the default Sobol config at full stream length has one class, Owen-scrambled prefixes have
one class per distinct XOR mask. The cache key follows the reference: the configuration,
sc_prec, stoc_len and rng_levels, but not the Owen environment variables (call
clear_rng_cache() after changing them, as with the reference).
"""
from __future__ import annotations

import json
import math
import os
import random
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .. import _lib
from .rng import sobol_direction_vectors, sobol_default_seed

_table_cache: dict = {}


def clear():
    _table_cache.clear()


def config_key(config: Optional[dict], default_desc: tuple) -> str:
    """Cache key of a configuration. The implicit default config is keyed by its
    parameters; an explicit dict by its JSON text, like the reference
    (scmp_kernels/sc/kernels.py:62-64)."""
    if config is None:
        return "default:" + ",".join(map(str, default_desc))
    return json.dumps(config, sort_keys=True)


def owen_mode_from_env() -> str:
    """scmp_kernels/sc/kernels.py:648-652."""
    if os.environ.get("SC_DISABLE_OWEN", "0") == "1":
        return "off"
    return os.environ.get("SC_OWEN_MODE", "bitrev").lower()


def scramble_rescale_from_env() -> bool:
    """scmp_kernels/sc/kernels.py:700."""
    return os.environ.get("SC_SCRAMBLE_RESCALE", "1") == "1"


_OWEN_SEED = 0x5A5A5A5A  # scmp_kernels/sc/kernels.py:635


def owen_masks(D: int, base: int, mode: str, device="cpu") -> Optional[np.ndarray]:
    """Per-dimension XOR masks, scmp_kernels/sc/kernels.py:655-670. 'random' draws
    randint(0, base, (D, 1)) from a generator of the device the sequences live on, seeded
    with the reference's seed (kernels.py:664-668: torch.Generator(device=prefix.device))."""
    if mode == "off":
        return None
    idx = np.arange(D, dtype=np.int64) % base
    if mode == "counter":
        return idx.astype(np.int32)
    if mode == "bitrev":
        nbits = int(round(math.log2(base)))
        out = np.zeros(D, dtype=np.int64)
        for i in range(nbits):
            out |= ((idx >> i) & 1) << (nbits - 1 - i)
        return out.astype(np.int32)
    g = torch.Generator(device=device).manual_seed(_OWEN_SEED)
    m = torch.randint(0, base, (D, 1), generator=g, device=device)
    return m.reshape(D).cpu().numpy().astype(np.int32)


def beta_of_q(q: np.ndarray, Q: int, R: int) -> np.ndarray:
    """rne(fl(fl(q * R) / Q)) in fp32 (scmp_kernels/sc/kernels.py:1679-1686)."""
    t = (q.astype(np.float32) * np.float32(R)).astype(np.float32)
    return np.rint((t / np.float32(Q)).astype(np.float32)).astype(np.int64)


def interval_width(sc_prec: int, L: int, R: int, bipolar: bool) -> int:
    """JP: the K extent per inner dimension of the SC GEMM, a power of two >= 16 that
    bounds the number of distinct attainable thermometer lengths."""
    Q = 2 ** (sc_prec - 1) - 1 if bipolar else 2 ** sc_prec - 1
    qmax = Q + 1 if bipolar else Q
    nb = len(set(int(v) for v in beta_of_q(np.arange(qmax + 1), Q, R)) - {0})
    J = max(1, min(L, nb))
    JP = 16
    while JP < J:
        JP *= 2
    return JP


@dataclass
class StreamTables:
    JP: int
    nclass: int
    D: int
    L: int
    R: int
    sc_prec: int
    bipolar: bool
    lut: torch.Tensor            # (nclass, 256, JP) int8
    jtab: torch.Tensor           # (nclass, 256) uint8
    kappa: torch.Tensor          # (nclass, JP+1) int16
    d_class: Optional[torch.Tensor]  # (D,) int32 or None (one class)
    class_of: np.ndarray         # host copy of the class of each d
    ra: torch.Tensor             # prepared A-side sequences (D, L) int32
    rb: torch.Tensor             # prepared B-side sequences (D, L) int32
    _bitlut: Optional[torch.Tensor] = None
    _lut4: Optional[torch.Tensor] = None
    _fp4_ok: Optional[bool] = None
    _runs: Optional[tuple] = None

    def class_runs(self):
        """The inner dimensions laid out in runs of one class, each run padded to whole
        groups of 8: (src, group_class, Dp) with src[p] the d at position p (-1: padding),
        an int32 device tensor of Dp entries, and group_class the class of each group of 8
        positions (Dp / 8 entries). Built on first use."""
        if self._runs is None:
            cls = self.class_of.astype(np.int64)
            counts = np.bincount(cls, minlength=self.nclass)
            padded = (counts + 7) // 8 * 8
            start = np.concatenate([[0], np.cumsum(padded)[:-1]])     # run start per class
            first = np.concatenate([[0], np.cumsum(counts)[:-1]])     # in the sorted order
            order = np.argsort(cls, kind="stable")
            pos = start[cls[order]] + (np.arange(len(order)) - first[cls[order]])
            Dp = int(padded.sum())
            src = np.full(Dp, -1, dtype=np.int32)
            src[pos] = order
            gcls = np.repeat(np.arange(self.nclass, dtype=np.int32), padded // 8)
            dev = self.lut.device
            self._runs = (torch.from_numpy(src).to(dev), torch.from_numpy(gcls).to(dev), Dp)
        return self._runs

    def lut4(self, stream) -> Optional[torch.Tensor]:
        """FP4 (e2m1) form of the table, or None when some count is not representable
        (then only the int8 kernel applies). Built on first use."""
        if self._fp4_ok is None:
            JPF = max(self.JP, 32)
            l4 = torch.empty((self.nclass, 256, JPF // 2), dtype=torch.uint8,
                             device=self.lut.device)
            bad = torch.zeros(1, dtype=torch.int32, device=self.lut.device)
            _lib.check(_lib.load().scmp_build_fp4_lut(
                self.lut.data_ptr(), self.nclass, self.JP, l4.data_ptr(), bad.data_ptr(),
                stream), "scmp_build_fp4_lut")
            self._fp4_ok = int(bad.item()) == 0
            self._lut4 = l4 if self._fp4_ok else None
        return self._lut4

    def bitlut(self, stream) -> torch.Tensor:
        """Bit planes for the VALU comparison kernel (built on first use)."""
        if self._bitlut is None:
            W = max(1, self.JP // 32)
            bl = torch.empty((self.nclass, 256, 2, W), dtype=torch.int32, device=self.lut.device)
            _lib.check(_lib.load().scmp_build_bitlut(
                self.lut.data_ptr(), self.nclass, self.JP, bl.data_ptr(), stream),
                "scmp_build_bitlut")
            self._bitlut = bl
        return self._bitlut


def _base_sequence(cfg: dict, p: int, device) -> torch.Tensor:
    """One RNG of the pool as a length-2^p int32 device sequence (create_rng,
    scmp_kernels/sc/rng.py:242-268)."""
    n = 2 ** p
    lib = _lib.load()
    stream = _lib.stream_of(device)
    typ = cfg.get("type", "lfsr")
    out = torch.empty(n, dtype=torch.int32, device=device)
    if typ == "sobol":
        seed = cfg.get("seed")
        if seed is None:
            seed = sobol_default_seed(p, cfg.get("seed_type", "q"))
        V = np.asarray(sobol_direction_vectors(p, list(seed)), dtype=np.int64)
        _lib.check(lib.scmp_rng_sobol(p, V.ctypes.data, n, out.data_ptr(), stream),
                   "scmp_rng_sobol")
    elif typ == "lfsr":
        mask = 0
        for t in cfg["taps"]:
            mask |= 1 << int(t)
        _lib.check(lib.scmp_rng_lfsr(p, int(cfg["seed"]), mask, n, out.data_ptr(), stream),
                   "scmp_rng_lfsr")
    elif typ == "true_random":
        # Python's Mersenne Twister, as TrueRandom.simulate (rng.py:99-113)
        r = random.Random(cfg["seed"])
        mx = 2 ** p - 1
        host = torch.tensor([r.randint(0, mx) for _ in range(n)], dtype=torch.int32)
        out.copy_(host)
    else:
        raise ValueError(f"Unknown RNG type: {typ}")
    return out


def _validate_pool(config: dict):
    """RNGPool constructs every pool entry (sng.py:92-98); mirror its construction errors."""
    for cfg in config["rng_pool"]:
        typ = cfg.get("type", "lfsr")
        if typ == "lfsr" and cfg.get("seed", 0) == 0:
            raise ValueError("LFSR seed must be non-zero")
        if typ not in ("lfsr", "true_random", "sobol"):
            raise ValueError(f"Unknown RNG type: {typ}")


def side_sequences(config: dict, side: str, p: int, D: int, device) -> torch.Tensor:
    """SNGBank.get_all_sequences (scmp_kernels/sc/sng.py:187-230) for the first D
    elements of side 'q' or 'k': (D, 2^p) int32 on the device."""
    sngs = config["sng"][side]
    if len(sngs) < D:
        raise ValueError(
            f"sc_matmul: config has {len(sngs)} '{side}' SNG entries, need at least {D}")
    ids_all = [s["rng_id"] for s in sngs]
    single = len(set(ids_all)) == 1
    sngs = sngs[:D]
    uniq = sorted(set(s["rng_id"] for s in sngs))
    pos = {rid: i for i, rid in enumerate(uniq)}
    base = torch.stack([_base_sequence(config["rng_pool"][rid], p, device) for rid in uniq])
    src = torch.tensor([pos[s["rng_id"]] for s in sngs], dtype=torch.int32, device=device)
    scr = [s.get("scramble") for s in sngs]
    any_scr = any(s is not None for s in (x.get("scramble") for x in config["sng"][side]))
    perm = None
    if any_scr:
        rows = []
        for s in scr:
            if s is None:
                # apply_scramble_batch treats None as the identity over sc_prec bits
                rows.append(list(range(p)) if single else [-1] * p)
            else:
                if len(s) != p:
                    raise ValueError(f"sc_matmul: scramble of length {len(s)} != sc_prec {p}")
                rows.append([int(v) for v in s])
        perm = torch.tensor(rows, dtype=torch.int32, device=device)
    out = torch.empty((D, 2 ** p), dtype=torch.int32, device=device)
    _lib.check(_lib.load().scmp_rng_expand(
        base.data_ptr(), 2 ** p, src.data_ptr(), _lib.ptr(perm), p, D, out.data_ptr(),
        _lib.stream_of(device)), "scmp_rng_expand")
    return out


def prepare(r: torch.Tensor, p: int, L: int, R: int, masks: Optional[np.ndarray],
            scramble_rescale: bool) -> torch.Tensor:
    D, full = r.shape
    out = torch.empty((D, L), dtype=torch.int32, device=r.device)
    m = torch.from_numpy(masks).to(r.device) if masks is not None else None
    _lib.check(_lib.load().scmp_rng_prepare(
        r.data_ptr(), D, full, p, L, R, _lib.ptr(m), 1 if scramble_rescale else 0,
        out.data_ptr(), _lib.stream_of(r.device)), "scmp_rng_prepare")
    return out


def get_tables(config: Optional[dict], default_desc: tuple, make_config, sc_prec: int,
               L: int, R: int, bipolar: bool, D: int, device,
               min_jp: int = 16) -> StreamTables:
    """Cached stream tables for inner dimensions 0..D-1 of `config` (built with
    make_config() when config is None). min_jp: table width of at least this many intervals
    (a power of two; intervals past the attainable ones are empty, so every sum is the
    same)."""
    key = (config_key(config, default_desc), sc_prec, L, R, bipolar, D, str(device), min_jp)
    t = _table_cache.get(key)
    if t is not None:
        return t
    if config is None:
        config = make_config()
    if sc_prec < 1 or sc_prec > 8:
        raise NotImplementedError(
            f"sc_matmul: sc_prec={sc_prec} is not supported by the gfx950 kernels "
            f"(8-bit operand codes need 1 <= sc_prec <= 8)")
    if L > 2 ** sc_prec:
        raise ValueError(
            f"sc_matmul: stoc_len={L} exceeds the 2**sc_prec={2 ** sc_prec} RNG period")
    _validate_pool(config)
    ra_full = side_sequences(config, "q", sc_prec, D, device)
    rb_full = side_sequences(config, "k", sc_prec, D, device)
    base = 2 ** sc_prec
    needs_mask = (L < base) if R == base else True
    masks = owen_masks(D, base, owen_mode_from_env(), device) if needs_mask else None
    srs = scramble_rescale_from_env()
    ra = prepare(ra_full, sc_prec, L, R, masks, srs)
    rb = prepare(rb_full, sc_prec, L, R, masks, srs)
    both = torch.cat([ra, rb], dim=1).cpu().numpy()
    _, rep, class_of = np.unique(both, axis=0, return_index=True, return_inverse=True)
    class_of = class_of.reshape(-1).astype(np.int32)
    nclass = len(rep)
    JP = max(interval_width(sc_prec, L, R, bipolar), min_jp)
    lib = _lib.load()
    stream = _lib.stream_of(device)
    jtab = torch.empty((nclass, 256), dtype=torch.uint8, device=device)
    lut = torch.empty((nclass, 256, JP), dtype=torch.int8, device=device)
    kappa = torch.empty((nclass, JP + 1), dtype=torch.int16, device=device)
    jmax = torch.zeros(1, dtype=torch.int32, device=device)
    rep_t = torch.from_numpy(rep.astype(np.int32)).to(device)
    _lib.check(lib.scmp_build_stream_tables(
        ra.data_ptr(), rb.data_ptr(), rep_t.data_ptr(), nclass, L, sc_prec, R,
        1 if bipolar else 0, JP, jtab.data_ptr(), lut.data_ptr(), kappa.data_ptr(),
        jmax.data_ptr(), stream), "scmp_build_stream_tables")
    J = int(jmax.item())
    if J > JP or (bipolar and J > 127):
        raise ValueError(
            f"sc_matmul: RNG configuration yields {J} distinct enable lengths, more than "
            f"the {JP if J > JP else 127} the 8-bit operand codes can address")
    d_class = torch.from_numpy(class_of).to(device) if nclass > 1 else None
    t = StreamTables(JP=JP, nclass=nclass, D=D, L=L, R=R, sc_prec=sc_prec, bipolar=bipolar,
                     lut=lut, jtab=jtab, kappa=kappa, d_class=d_class, class_of=class_of,
                     ra=ra, rb=rb)
    _table_cache[key] = t
    return t

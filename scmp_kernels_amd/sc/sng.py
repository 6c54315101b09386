"""Stochastic number generators: RNG pool, per-element SNGs and bit scrambles
(scmp_kernels/sc/sng.py).

The classes keep the reference's interface and return numpy arrays. The sequences come from
the GPU generators (scmp_rng_sobol / scmp_rng_lfsr via the RNG classes of ``.rng``) and the
per-element bit permutations from one scmp_rng_expand launch per bank; TrueRandom stays on
the host because its stream is Python's Mersenne Twister by definition (rng.py:80-113).
"""
from __future__ import annotations

import random
from typing import Optional

import numpy as np

from .rng import RNG, create_rng


def _expand(base: np.ndarray, src: np.ndarray, perm: Optional[np.ndarray], p: int) -> np.ndarray:
    """out[d] = scramble(base[src[d]], perm[d]) on the GPU (scmp_rng_expand)."""
    import torch
    from .. import _lib
    if not torch.cuda.is_available():
        raise RuntimeError("scmp_kernels_amd: SNG sequences are built on the GPU; none "
                           "available")
    dev = torch.device("cuda", torch.cuda.current_device())
    b = torch.from_numpy(np.ascontiguousarray(base, dtype=np.int32)).to(dev)
    s = torch.from_numpy(np.ascontiguousarray(src, dtype=np.int32)).to(dev)
    pm = None if perm is None else torch.from_numpy(np.ascontiguousarray(perm, np.int32)).to(dev)
    D, n = len(src), base.shape[1]
    out = torch.empty((D, n), dtype=torch.int32, device=dev)
    if D and n:
        _lib.check(_lib.load().scmp_rng_expand(b.data_ptr(), n, s.data_ptr(), _lib.ptr(pm), p,
                                               D, out.data_ptr(), _lib.stream_of(dev)),
                   "scmp_rng_expand")
    return out.cpu().numpy()


def _perm_row(scramble, p: int) -> list:
    if len(scramble) != p:
        raise ValueError(f"scramble of length {len(scramble)} for {p}-bit values")
    return [int(v) for v in scramble]


def apply_scramble(sequence: np.ndarray, scramble: list) -> np.ndarray:
    """Output bit i = input bit scramble[i], for i < len(scramble) (sng.py:15-29)."""
    seq = np.asarray(sequence)
    p = len(scramble)
    if p == 0:
        return np.zeros_like(seq)
    flat = seq.reshape(1, -1).astype(np.int32)
    out = _expand(flat, np.zeros(1, np.int32), np.array([_perm_row(scramble, p)]), p)
    return out.reshape(seq.shape).astype(seq.dtype)


def apply_scramble_batch(sequences: np.ndarray, scrambles: list, sc_prec: int) -> np.ndarray:
    """Row d gets scrambles[d] (None: the identity over sc_prec bits), sng.py:32-53."""
    seqs = np.asarray(sequences)
    n_el = seqs.shape[0]
    perm = np.array([_perm_row(s, sc_prec) if s is not None else list(range(sc_prec))
                     for s in scrambles], dtype=np.int32).reshape(n_el, sc_prec)
    out = _expand(seqs.astype(np.int32), np.arange(n_el, dtype=np.int32), perm, sc_prec)
    return out.astype(seqs.dtype)


def reverse_permutation(n_bits: int) -> list:
    """Bit reversal, sng.py:56-58."""
    return list(range(n_bits - 1, -1, -1))


def generate_random_permutation(n_bits: int) -> list:
    """A random bit permutation from Python's ``random`` (sng.py:61-66)."""
    perm = list(range(n_bits))
    random.shuffle(perm)
    return perm


class RNGPool:
    """RNG instances built from config entries, with one cached sequence per RNG
    (sng.py:69-120). As in the reference, the cache is keyed by rng_id only: the first
    requested length is the one kept."""

    def __init__(self, rng_configs: list, sc_prec: int):
        self.sc_prec = sc_prec
        self.rngs: list = []
        self._sequence_cache: dict = {}
        for cfg in rng_configs:
            self.rngs.append(create_rng(rng_type=cfg.get("type", "lfsr"), length=sc_prec,
                                        **{k: v for k, v in cfg.items() if k != "type"}))

    def __len__(self):
        return len(self.rngs)

    def get_sequence(self, rng_id: int, stoc_len: int) -> np.ndarray:
        if rng_id not in self._sequence_cache:
            self._sequence_cache[rng_id] = np.asarray(
                self.rngs[rng_id].simulate(stoc_len), dtype=np.int32)
        return self._sequence_cache[rng_id]

    def clear_cache(self):
        self._sequence_cache.clear()


class SNG:
    """One element's generator: a pool RNG and an optional bit scramble (sng.py:123-157)."""

    def __init__(self, rng_pool: RNGPool, rng_id: int, scramble: Optional[list] = None):
        self.rng_pool = rng_pool
        self.rng_id = rng_id
        self.scramble = scramble

    def get_sequence(self, stoc_len: int) -> np.ndarray:
        seq = self.rng_pool.get_sequence(self.rng_id, stoc_len)
        if self.scramble is not None:
            return apply_scramble(seq, self.scramble)
        return seq.copy()


class SNGBank:
    """The SNGs of one operand side (sng.py:160-230); ``get_all_sequences`` builds every
    element's sequence in one GPU launch."""

    def __init__(self, rng_pool: RNGPool, sng_configs: list):
        self.rng_pool = rng_pool
        self.sng_configs = sng_configs
        self.sngs = [SNG(rng_pool, cfg["rng_id"], cfg.get("scramble")) for cfg in sng_configs]

    def __len__(self):
        return len(self.sngs)

    def get_all_sequences(self, stoc_len: int) -> np.ndarray:
        """(n_elements, stoc_len) int32. One shared RNG: scrambles act over sc_prec bits
        (None = identity), as apply_scramble_batch; several RNGs: each element's own
        SNG.get_sequence (None = unchanged)."""
        n_el = len(self.sngs)
        if n_el == 0:
            return np.zeros((0, stoc_len), dtype=np.int32)
        ids = []
        for sng in self.sngs:
            if sng.rng_id not in ids:
                ids.append(sng.rng_id)
        base = np.stack([self.rng_pool.get_sequence(r, stoc_len) for r in ids])
        src = np.array([ids.index(s.rng_id) for s in self.sngs], dtype=np.int32)
        p = self.rng_pool.sc_prec
        scr = [s.scramble for s in self.sngs]
        if all(s is None for s in scr):
            perm = None
        elif len(ids) == 1:
            perm = np.array([_perm_row(s, p) if s is not None else list(range(p))
                             for s in scr], dtype=np.int32)
        else:
            perm = np.array([_perm_row(s, p) if s is not None else [-1] * p for s in scr],
                            dtype=np.int32)
        return _expand(base, src, perm, p)


__all__ = ["RNG", "RNGPool", "SNG", "SNGBank", "apply_scramble", "apply_scramble_batch",
           "reverse_permutation", "generate_random_permutation"]

"""RNG / SNG configuration dictionaries.

The schema is the reference's (scmp_kernels/sc/config_helpers.py:74-82):
``{"rng_pool": [{"type", "seed" | "seed_type", "taps"}, ...],
   "sng": {"q": [{"rng_id", "scramble"[, "complement"]}, ...], "k": [...]}}``.
``make_sobol_simple_config`` is the default of every sc_matmul path.
"""
from __future__ import annotations

import random
from typing import Optional


def make_sobol_simple_config(q_e: int, k_e: int, sc_prec: int = 8) -> dict:
    """Q: Sobol seed [1,1,...]; K: Sobol seed [1,1,1,1,9,1,41,255] (no scrambles)
    (scmp_kernels/sc/config_helpers.py:583-607)."""
    return {
        "rng_pool": [
            {"type": "sobol", "seed_type": "q"},
            {"type": "sobol", "seed_type": "k"},
        ],
        "sng": {
            "q": [{"rng_id": 0, "scramble": None} for _ in range(q_e)],
            "k": [{"rng_id": 1, "scramble": None} for _ in range(k_e)],
        },
    }


def make_sobol_antithetic_config(q_e: int, k_e: int, sc_prec: int = 8) -> dict:
    """As make_sobol_simple_config with ``"complement": True`` on the K side; the SNG
    ignores the flag (scmp_kernels/sc/config_helpers.py:610-634, sng.py:179-182), so the
    streams are the simple config's; only the cache key differs."""
    cfg = make_sobol_simple_config(q_e, k_e, sc_prec)
    for s in cfg["sng"]["k"]:
        s["complement"] = True
    return cfg


def make_sobol_altseed_config(q_e: int, k_e: int, sc_prec: int = 8,
                              k_seed: Optional[list] = None) -> dict:
    """K side uses another valid Sobol seed (scmp_kernels/sc/config_helpers.py:637-672)."""
    if k_seed is None:
        k_seed = [(1 << (i + 1)) - 1 for i in range(sc_prec)]
    return {
        "rng_pool": [{"type": "sobol", "seed_type": "q"}, {"type": "sobol", "seed": list(k_seed)}],
        "sng": {
            "q": [{"rng_id": 0, "scramble": None} for _ in range(q_e)],
            "k": [{"rng_id": 1, "scramble": None} for _ in range(k_e)],
        },
    }


def make_sobol_custom_seed_config(q_e: int, k_e: int, sc_prec: int, q_seed: list = None,
                                  k_seed: list = None, use_scrambling: bool = False) -> dict:
    """Custom Sobol seeds, optional random per-element scrambles
    (scmp_kernels/sc/config_helpers.py:724-763)."""
    def scr():
        return generate_random_permutation(sc_prec) if use_scrambling else None
    return {
        "rng_pool": [{"type": "sobol", "seed": q_seed, "seed_type": "q"},
                     {"type": "sobol", "seed": k_seed, "seed_type": "k"}],
        "sng": {
            "q": [{"rng_id": 0, "scramble": scr()} for _ in range(q_e)],
            "k": [{"rng_id": 1, "scramble": scr()} for _ in range(k_e)],
        },
    }


def make_independent_config(q_e: int, k_e: int, sc_prec: int, q_taps: list, k_taps: list,
                            q_seed: int, k_seed: int, q_scramble: Optional[list] = None,
                            k_scramble: Optional[list] = None) -> dict:
    """Two LFSRs, one per side (scmp_kernels/sc/config_helpers.py:85-117)."""
    return {
        "rng_pool": [{"type": "lfsr", "seed": q_seed, "taps": q_taps},
                     {"type": "lfsr", "seed": k_seed, "taps": k_taps}],
        "sng": {
            "q": [{"rng_id": 0, "scramble": q_scramble} for _ in range(q_e)],
            "k": [{"rng_id": 1, "scramble": k_scramble} for _ in range(k_e)],
        },
    }


def make_default_config(q_e: int, k_e: int, sc_prec: int, taps: list, seed: int = 125) -> dict:
    """Shared LFSR, K side bit-reversed (scmp_kernels/sc/config_helpers.py:51-82). The
    reference reads default taps from a data file it does not ship, so taps are required."""
    return {
        "rng_pool": [{"type": "lfsr", "seed": seed, "taps": taps}],
        "sng": {
            "q": [{"rng_id": 0, "scramble": None} for _ in range(q_e)],
            "k": [{"rng_id": 0, "scramble": reverse_permutation(sc_prec)} for _ in range(k_e)],
        },
    }


def reverse_permutation(n_bits: int) -> list:
    """scmp_kernels/sc/sng.py:56-58."""
    return list(range(n_bits - 1, -1, -1))


def generate_random_permutation(n_bits: int) -> list:
    """scmp_kernels/sc/sng.py:61-66."""
    perm = list(range(n_bits))
    random.shuffle(perm)
    return perm

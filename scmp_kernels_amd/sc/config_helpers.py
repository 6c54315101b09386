"""RNG / SNG configuration dictionaries, their makers and the JSON config registry.

The schema is the reference's (scmp_kernels/sc/config_helpers.py:74-82):
``{"rng_pool": [{"type", "seed" | "seed_type", "taps"}, ...],
   "sng": {"q": [{"rng_id", "scramble"[, "complement"]}, ...], "k": [...]}}``.
``make_sobol_simple_config`` is the default of every sc_matmul path. The random makers draw
from Python's ``random`` in the reference's order (same draws for the same seed), so a
seeded caller gets the configuration the reference would build. The LFSR makers take their
default taps from the tap store of ``.lfsr_taps`` (shipped for 2..16 bits).
"""
from __future__ import annotations

import json
import os
import random
from datetime import datetime
from pathlib import Path
from typing import Optional

from .lfsr_taps import get_taps
from .rng import Sobol
from .sng import generate_random_permutation, reverse_permutation

CONFIG_DIR = Path(__file__).parent / "configs"
CONFIG_REGISTRY_FILE = CONFIG_DIR / "config_registry.json"


def get_taps_choices(sc_prec: int) -> list:
    """Every stored maximal-length tap set of sc_prec bits; ValueError when the store has
    none (config_helpers.py:20-42)."""
    taps = get_taps(sc_prec)
    if not taps:
        raise ValueError(
            f"No pre-computed taps for sc_prec={sc_prec}. "
            f"Run `python -m scmp_kernels_amd.sc.lfsr_taps {sc_prec}` to generate.")
    return taps


def get_default_taps(sc_prec: int) -> list:
    """The first stored tap set (config_helpers.py:45-48)."""
    return get_taps_choices(sc_prec)[0]


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


def make_sobol_dse_config(q_e: int, k_e: int, sc_prec: int,
                          use_scrambling: bool = True) -> dict:
    """Random valid Sobol seeds for Q and K and random per-element scrambles, for design
    space exploration (config_helpers.py:675-721; the reference's ``from rng import Sobol``
    cannot import, this one uses the package's Sobol)."""
    q_seed = Sobol.random_seed(sc_prec)
    k_seed = Sobol.random_seed(sc_prec)
    sq = _random_scrambles(q_e, sc_prec, use_scrambling)
    sk = _random_scrambles(k_e, sc_prec, use_scrambling)
    return {
        "rng_pool": [{"type": "sobol", "seed": q_seed}, {"type": "sobol", "seed": k_seed}],
        "sng": {"q": [{"rng_id": 0, "scramble": s} for s in sq],
                "k": [{"rng_id": 1, "scramble": s} for s in sk]},
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


def make_default_config(q_e: int, k_e: int, sc_prec: int, taps: Optional[list] = None,
                        seed: int = 125) -> dict:
    """One shared LFSR, K side bit-reversed (config_helpers.py:51-82)."""
    if taps is None:
        taps = get_default_taps(sc_prec)
    return {
        "rng_pool": [{"type": "lfsr", "seed": seed, "taps": taps}],
        "sng": {
            "q": [{"rng_id": 0, "scramble": None} for _ in range(q_e)],
            "k": [{"rng_id": 0, "scramble": reverse_permutation(sc_prec)} for _ in range(k_e)],
        },
    }


def make_per_element_scramble_config(q_e: int, k_e: int, sc_prec: int,
                                     taps: Optional[list] = None, seed: int = 125,
                                     k_reverse_of_q: bool = True) -> dict:
    """One shared LFSR; every element its own random scramble, K's the reverse of Q's
    (config_helpers.py:119-163)."""
    if taps is None:
        taps = get_default_taps(sc_prec)
    assert q_e == k_e, "Q and K must have same embedding size for paired scrambling"
    sng_q, sng_k = [], []
    for _ in range(q_e):
        sq = generate_random_permutation(sc_prec)
        sk = list(reversed(sq)) if k_reverse_of_q else generate_random_permutation(sc_prec)
        sng_q.append({"rng_id": 0, "scramble": sq})
        sng_k.append({"rng_id": 0, "scramble": sk})
    return {"rng_pool": [{"type": "lfsr", "seed": seed, "taps": taps}],
            "sng": {"q": sng_q, "k": sng_k}}


def make_fully_independent_config(q_e: int, k_e: int, sc_prec: int,
                                  taps_choices: Optional[list] = None) -> dict:
    """One LFSR per element with random taps and seed (config_helpers.py:166-209)."""
    if taps_choices is None:
        taps_choices = get_taps_choices(sc_prec)
    pool, ids = [], {"q": [], "k": []}
    for side, n in (("q", q_e), ("k", k_e)):
        for _ in range(n):
            taps = random.choice(taps_choices)
            seed = random.randint(1, 2 ** sc_prec - 1)
            pool.append({"type": "lfsr", "seed": seed, "taps": taps})
            ids[side].append(len(pool) - 1)
    return {"rng_pool": pool,
            "sng": {side: [{"rng_id": i, "scramble": None} for i in ids[side]]
                    for side in ("q", "k")}}


def make_separated_random_config(q_e: int, k_e: int, sc_prec: int,
                                 taps_choices: Optional[list] = None) -> dict:
    """Q on RNG 0, K on RNG 1, random taps and seeds, no scrambles
    (config_helpers.py:212-245)."""
    if taps_choices is None:
        taps_choices = get_taps_choices(sc_prec)
    q_taps = random.choice(taps_choices)
    k_taps = random.choice(taps_choices)
    q_seed = random.randint(1, 2 ** sc_prec - 1)
    k_seed = random.randint(1, 2 ** sc_prec - 1)
    return make_independent_config(q_e, k_e, sc_prec, q_taps, k_taps, q_seed, k_seed)


def _random_scrambles(n: int, sc_prec: int, use_scrambling: bool) -> list:
    """Per element: a random permutation with probability 1/2 (when enabled), else None;
    the draw order of config_helpers.py:285-291."""
    return [generate_random_permutation(sc_prec)
            if use_scrambling and random.random() > 0.5 else None for _ in range(n)]


def make_random_config(q_e: int, k_e: int, sc_prec: int,
                       taps_choices: Optional[list] = None,
                       use_scrambling: bool = True) -> dict:
    """Q on RNG 0, K on RNG 1 with random taps and seeds, random per-element scrambles
    (config_helpers.py:248-299)."""
    if taps_choices is None:
        taps_choices = get_taps_choices(sc_prec)
    q_taps = random.choice(taps_choices)
    k_taps = random.choice(taps_choices)
    q_seed = random.randint(1, 2 ** sc_prec - 1)
    k_seed = random.randint(1, 2 ** sc_prec - 1)
    sq = _random_scrambles(q_e, sc_prec, use_scrambling)
    sk = _random_scrambles(k_e, sc_prec, use_scrambling)
    return {
        "rng_pool": [{"type": "lfsr", "seed": q_seed, "taps": q_taps},
                     {"type": "lfsr", "seed": k_seed, "taps": k_taps}],
        "sng": {"q": [{"rng_id": 0, "scramble": s} for s in sq],
                "k": [{"rng_id": 1, "scramble": s} for s in sk]},
    }


def make_single_rng_reverse_config(q_e: int, k_e: int, sc_prec: int,
                                   taps_choices: Optional[list] = None,
                                   use_per_element_scrambling: bool = True) -> dict:
    """One random LFSR shared by Q and K; K's scramble is the reverse of Q's, per element or
    globally (config_helpers.py:302-355)."""
    if taps_choices is None:
        taps_choices = get_taps_choices(sc_prec)
    assert q_e == k_e, "Q and K must have same size for paired reverse scrambling"
    taps = random.choice(taps_choices)
    seed = random.randint(1, 2 ** sc_prec - 1)
    sng_q, sng_k = [], []
    if use_per_element_scrambling:
        for _ in range(q_e):
            sq = generate_random_permutation(sc_prec)
            sng_q.append({"rng_id": 0, "scramble": sq})
            sng_k.append({"rng_id": 0, "scramble": list(reversed(sq))})
    else:
        rev = reverse_permutation(sc_prec)
        for _ in range(q_e):
            sng_q.append({"rng_id": 0, "scramble": None})
            sng_k.append({"rng_id": 0, "scramble": rev})
    return {"rng_pool": [{"type": "lfsr", "seed": seed, "taps": taps}],
            "sng": {"q": sng_q, "k": sng_k}}


# -------------------------------------------------------------------------------------
# Saved configs and the best-config registry (config_helpers.py:362-577)
# -------------------------------------------------------------------------------------

def save_config(config: dict, filepath: Optional[Path] = None, operation: str = "matmul",
                sc_prec: int = 8, binary_prec: str = "fp8_e4m3",
                operand_sizes: Optional[dict] = None, error: Optional[float] = None,
                input_seed: Optional[int] = None, dse_params: Optional[dict] = None,
                notes: str = "") -> Path:
    """Write {"metadata": ..., "config": config} as JSON; the default path is
    CONFIG_DIR/<operation>_<sc_prec>bit_<timestamp>.json (config_helpers.py:362-430)."""
    CONFIG_DIR.mkdir(parents=True, exist_ok=True)
    if filepath is None:
        stamp = datetime.now().strftime("%Y%m%d_%H%M%S")
        filepath = CONFIG_DIR / f"{operation}_{sc_prec}bit_{stamp}.json"
    doc = {
        "metadata": {
            "operation": operation, "sc_prec": sc_prec, "binary_prec": binary_prec,
            "operand_sizes": operand_sizes or {}, "error": error, "input_seed": input_seed,
            "created_at": datetime.now().isoformat(), "dse_params": dse_params,
            "notes": notes,
        },
        "config": config,
    }
    with open(filepath, "w") as f:
        json.dump(doc, f, indent=2)
    return Path(filepath)


def load_config(filepath: Path) -> tuple:
    """(config, metadata) of a saved config (config_helpers.py:433-446)."""
    with open(filepath) as f:
        doc = json.load(f)
    return doc["config"], doc["metadata"]


def _registry_key(operation: str, sc_prec: int, binary_prec: str) -> str:
    return f"{operation}_{sc_prec}bit_{binary_prec}"


def save_best_config(config: dict, error: float, operation: str = "matmul", sc_prec: int = 8,
                     binary_prec: str = "fp8_e4m3", operand_sizes: Optional[dict] = None,
                     input_seed: Optional[int] = None, dse_params: Optional[dict] = None,
                     notes: str = "") -> Path:
    """Save the config; record it as the best of its (operation, sc_prec, binary_prec)
    unless the registry already holds one with an error at most as large
    (config_helpers.py:449-517)."""
    filepath = save_config(config=config, operation=operation, sc_prec=sc_prec,
                           binary_prec=binary_prec, operand_sizes=operand_sizes, error=error,
                           input_seed=input_seed, dse_params=dse_params, notes=notes)
    registry = _load_registry()
    key = _registry_key(operation, sc_prec, binary_prec)
    if key in registry:
        existing = registry[key].get("error")
        if existing is not None and error >= existing:
            return filepath
    registry[key] = {
        "filepath": str(filepath), "error": error, "operation": operation,
        "sc_prec": sc_prec, "binary_prec": binary_prec, "operand_sizes": operand_sizes,
        "input_seed": input_seed, "updated_at": datetime.now().isoformat(),
    }
    _save_registry(registry)
    return filepath


def load_best_config(operation: str = "matmul", sc_prec: int = 8,
                     binary_prec: str = "fp8_e4m3") -> tuple:
    """(config, metadata) of the registered best, (None, None) when there is none or its
    file is gone (config_helpers.py:520-546)."""
    entry = _load_registry().get(_registry_key(operation, sc_prec, binary_prec))
    if entry is None or not os.path.exists(entry["filepath"]):
        return None, None
    return load_config(entry["filepath"])


def list_saved_configs() -> list:
    """The registry entries (config_helpers.py:549-557)."""
    return list(_load_registry().values())


def _load_registry() -> dict:
    CONFIG_DIR.mkdir(parents=True, exist_ok=True)
    if not CONFIG_REGISTRY_FILE.exists():
        return {}
    with open(CONFIG_REGISTRY_FILE) as f:
        return json.load(f)


def _save_registry(registry: dict):
    CONFIG_DIR.mkdir(parents=True, exist_ok=True)
    with open(CONFIG_REGISTRY_FILE, "w") as f:
        json.dump(registry, f, indent=2)

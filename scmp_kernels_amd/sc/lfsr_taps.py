"""LFSR tap search and the tap-set store (scmp_kernels/sc/lfsr_taps.py).

A tap set of an n-bit right-shift LFSR (scmp_kernels/sc/rng.py:55-77) is maximal-length
when the register, started from 1, visits 2^n - 1 distinct states before its first repeat
(lfsr_taps.py:99-111). The candidates are the reference's: the MSB n-1 plus an odd number
of further positions, in itertools.combinations order by tap count (lfsr_taps.py:58-90).
Every candidate is tested on the GPU, one device thread per tap set
(scmp_lfsr_search: Brent cycle detection with O(1) state), so a 16-bit search takes a
fraction of a second instead of the reference's hours.

The store is the reference's JSON format: {"<n_bits>": [[taps...], ...]}. This package
ships ``lfsr_taps_data.json`` for 2..16 bits, written by ``search_and_save_all_taps``
(``python -m scmp_kernels_amd.sc.lfsr_taps 2 3 ... 16``), so the default LFSR config makers
work out of the box; the reference ships no store and its makers raise until one is made.
"""
from __future__ import annotations

import json
import os
from itertools import combinations
from pathlib import Path
from typing import Optional

import numpy as np

TAPS_FILE = Path(__file__).parent / "lfsr_taps_data.json"


def _candidates(n_bits: int) -> list:
    """Tap sets in the reference's enumeration order (lfsr_taps.py:74-83)."""
    out = []
    for n_taps in range(2, n_bits + 1, 2):
        for combo in combinations(range(n_bits - 1), n_taps - 1):
            out.append(sorted([n_bits - 1] + list(combo), reverse=True))
    return out


def _distinct_states(n_bits: int, tap_sets: list) -> np.ndarray:
    """Distinct states before the first repeat, from seed 1, per tap set (GPU)."""
    import torch
    from .. import _lib
    if not 2 <= n_bits <= _lib.LFSR_SEARCH_MAX_BITS:
        raise ValueError(f"LFSR search supports 2..{_lib.LFSR_SEARCH_MAX_BITS} bits, "
                         f"got {n_bits}")
    if not torch.cuda.is_available():
        raise RuntimeError("scmp_kernels_amd: the LFSR tap search runs on the GPU; none "
                           "available")
    masks = np.zeros(len(tap_sets), dtype=np.uint32)
    for i, taps in enumerate(tap_sets):
        m = 0
        for t in taps:
            t = int(t)
            if not 0 <= t < n_bits:
                raise ValueError(f"tap position {t} outside a {n_bits}-bit register")
            m |= 1 << t
        masks[i] = m
    if len(masks) == 0:
        return np.zeros(0, dtype=np.int64)
    dev = torch.device("cuda", torch.cuda.current_device())
    dm = torch.from_numpy(masks.view(np.int32)).to(dev)
    out = torch.empty(len(masks), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().scmp_lfsr_search(n_bits, dm.data_ptr(), len(masks),
                                            out.data_ptr(), _lib.stream_of(dev)),
               "scmp_lfsr_search")
    return out.cpu().numpy().view(np.uint32).astype(np.int64)


def search_taps(n_bits: int, verbose: bool = True) -> list:
    """All maximal-length tap configurations of an n-bit LFSR, each sorted descending
    (lfsr_taps.py:35-96)."""
    cands = _candidates(n_bits)
    if verbose:
        print(f"Searching {n_bits}-bit LFSR taps ({len(cands)} combinations)...")
    distinct = _distinct_states(n_bits, cands)
    valid = [t for t, k in zip(cands, distinct) if k == 2 ** n_bits - 1]
    if verbose:
        print(f"  Found {len(valid)} valid tap configurations for {n_bits} bits")
    return valid


def _is_maximal_length(taps: list, n_bits: int, expected_period: int) -> bool:
    """True when the LFSR from seed 1 visits exactly expected_period distinct states before
    its first repeat (lfsr_taps.py:99-111; construction errors count as False)."""
    try:
        return int(_distinct_states(n_bits, [list(taps)])[0]) == expected_period
    except ValueError:
        return False


def save_taps(taps_dict: dict, filepath: Optional[Path] = None):
    """Write {n_bits: [taps, ...]} as JSON with string keys (lfsr_taps.py:114-131)."""
    if filepath is None:
        filepath = TAPS_FILE
    with open(filepath, "w") as f:
        json.dump({str(k): v for k, v in taps_dict.items()}, f, indent=2)
    print(f"Saved tap configurations to {filepath}")


def load_taps(filepath: Optional[Path] = None) -> dict:
    """{n_bits: [taps, ...]} from the JSON store, {} when absent (lfsr_taps.py:134-154)."""
    if filepath is None:
        filepath = TAPS_FILE
    if not os.path.exists(filepath):
        return {}
    with open(filepath) as f:
        return {int(k): v for k, v in json.load(f).items()}


def get_taps(n_bits: int, filepath: Optional[Path] = None) -> list:
    """The stored tap configurations of one width, [] when none (lfsr_taps.py:157-172)."""
    return load_taps(filepath).get(n_bits, [])


def search_and_save_all_taps(bit_widths: list = None, filepath: Optional[Path] = None,
                             verbose: bool = True):
    """Search the widths missing from the store and save it (lfsr_taps.py:175-210)."""
    if bit_widths is None:
        bit_widths = [4, 5, 6, 7, 8, 10, 12]
    if filepath is None:
        filepath = TAPS_FILE
    taps_dict = load_taps(filepath)
    for n_bits in bit_widths:
        if n_bits in taps_dict:
            if verbose:
                print(f"Skipping {n_bits} bits (already have {len(taps_dict[n_bits])} configs)")
            continue
        taps_dict[n_bits] = search_taps(n_bits, verbose=verbose)
    save_taps(dict(sorted(taps_dict.items())), filepath)


if __name__ == "__main__":
    import sys
    widths = [int(x) for x in sys.argv[1:]] or [4, 5, 6, 7, 8, 9]
    print(f"Searching for valid LFSR taps for bit widths: {widths}")
    search_and_save_all_taps(widths)
    print("\nSummary:")
    for n, t in sorted(load_taps().items()):
        print(f"  {n} bits: {len(t)} valid tap configurations")

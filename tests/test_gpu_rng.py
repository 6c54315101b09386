"""GPU parity of the RNG configuration surface: the LFSR tap search (scmp_lfsr_search), the
SNG classes (scmp_rng_expand) and sc_matmul under LFSR / scrambled / independent configs,
each against the CPU oracle."""
import random

import numpy as np
import pytest
import torch

from oracle import sc_oracle as O

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda", 0)


@pytest.mark.parametrize("n", range(2, 15))
def test_search_taps_matches_oracle(n):
    from scmp_kernels_amd.sc.lfsr_taps import search_taps
    _dev()
    assert search_taps(n, verbose=False) == O.lfsr_search(n)


def test_is_maximal_length():
    from scmp_kernels_amd.sc.lfsr_taps import _is_maximal_length, _distinct_states
    _dev()
    assert _is_maximal_length([7, 2, 1, 0], 8, 255)
    assert not _is_maximal_length([7, 0], 8, 255)
    assert not _is_maximal_length([9, 0], 8, 255)           # tap outside the register
    cands = [[7, 3, 2, 1], [7, 0], [5, 4, 2, 1], [11, 10, 2, 0], [3, 1]]
    widths = [8, 8, 6, 12, 4]
    for taps, n in zip(cands, widths):
        assert int(_distinct_states(n, [taps])[0]) == O.lfsr_distinct_states(taps, n)


def test_search_limits():
    from scmp_kernels_amd.sc.lfsr_taps import search_taps
    _dev()
    with pytest.raises(ValueError, match="LFSR search supports"):
        search_taps(21, verbose=False)


def test_scramble_functions():
    from scmp_kernels_amd.sc.sng import apply_scramble, apply_scramble_batch
    _dev()
    rng = np.random.default_rng(0)
    seq = rng.integers(0, 256, 300).astype(np.int32)
    perm = [3, 0, 7, 1, 6, 2, 5, 4]
    np.testing.assert_array_equal(apply_scramble(seq, perm), O.scramble(seq, perm))
    np.testing.assert_array_equal(apply_scramble(seq, perm[:5]), O.scramble(seq, perm[:5]))
    seqs = rng.integers(0, 1024, (5, 64)).astype(np.int32)     # bits above sc_prec drop
    scr = [perm, None, perm[::-1], None, list(range(8))]
    ref = np.stack([O.scramble(s, p if p is not None else list(range(8)))
                    for s, p in zip(seqs, scr)])
    np.testing.assert_array_equal(apply_scramble_batch(seqs, scr, 8), ref)


@pytest.mark.parametrize("maker", ["per_element", "fully_independent", "random",
                                   "single_reverse", "default", "sobol_dse"])
def test_sng_bank_matches_oracle(maker):
    from scmp_kernels_amd.sc import config_helpers as C
    from scmp_kernels_amd.sc.sng import RNGPool, SNGBank, SNG
    _dev()
    random.seed(21)
    cfg = {
        "per_element": lambda: C.make_per_element_scramble_config(24, 24, 8),
        "fully_independent": lambda: C.make_fully_independent_config(12, 9, 8),
        "random": lambda: C.make_random_config(20, 20, 8),
        "single_reverse": lambda: C.make_single_rng_reverse_config(16, 16, 8),
        "default": lambda: C.make_default_config(10, 10, 8),
        "sobol_dse": lambda: C.make_sobol_dse_config(16, 16, 8),
    }[maker]()
    pool = RNGPool(cfg["rng_pool"], 8)
    assert len(pool) == len(cfg["rng_pool"])
    for side in ("q", "k"):
        bank = SNGBank(pool, cfg["sng"][side])
        assert len(bank) == len(cfg["sng"][side])
        np.testing.assert_array_equal(bank.get_all_sequences(256), O.sng_sequences(cfg, side, 8))
    s0 = cfg["sng"]["q"][0]
    one = SNG(pool, s0["rng_id"], s0.get("scramble")).get_sequence(256)
    ref = O.rng_sequence(cfg["rng_pool"][s0["rng_id"]], 8, 256)
    if s0.get("scramble") is not None:
        ref = O.scramble(ref, s0["scramble"])
    np.testing.assert_array_equal(one, ref)


@pytest.mark.parametrize("maker,granularity", [("per_element", "per_row"),
                                               ("fully_independent", "per_row"),
                                               ("default", "per_tensor"),
                                               ("random", "per_row")])
def test_sc_matmul_lfsr_configs_vs_oracle(maker, granularity):
    """sc_matmul under the LFSR makers' configs: bit-exact fp32 output against the oracle."""
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.sc import config_helpers as C
    from scmp_kernels_amd.sc.kernels import clear_rng_cache
    dev = _dev()
    D = 48
    random.seed(33)
    cfg = {
        "per_element": lambda: C.make_per_element_scramble_config(D, D, 8),
        "fully_independent": lambda: C.make_fully_independent_config(D, D, 8),
        "default": lambda: C.make_default_config(D, D, 8),
        "random": lambda: C.make_random_config(D, D, 8),
    }[maker]()
    rng = np.random.default_rng(9)
    a = rng.standard_normal((37, D)).astype(np.float32)
    b = rng.standard_normal((29, D)).astype(np.float32)
    clear_rng_cache()
    got = sc_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), granularity,
                    sc_prec=8, config=cfg).cpu().numpy()
    ref = O.sc_matmul(a, b, granularity, sc_prec=8, config=cfg)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))

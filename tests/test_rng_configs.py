"""RNG configuration surface on the CPU: the LFSR tap oracle (pinned by GF(2) algebra), the
shipped tap store, the config makers (scmp_kernels/sc/config_helpers.py) and the JSON config
registry. GPU parity of the tap search and of SNG sequences is in test_gpu_rng.py."""
import json
import random

import pytest

from oracle import sc_oracle as O
from scmp_kernels_amd.sc import config_helpers as C
from scmp_kernels_amd.sc import lfsr_taps as LT


# -------------------------------------------------------------------------------------
# the oracle's brute-force maximal-length test, against primitivity of the characteristic
# polynomial x^n + sum_{t in taps} x^t over GF(2) (the register's bit 0 at time k is b_k,
# and the feedback makes b_{k+n} = xor of b_{k+t}); a different method, so a wrong shift
# direction, tap index or period count fails here
# -------------------------------------------------------------------------------------

def _mulmod(a: int, b: int, p: int, n: int) -> int:
    r = 0
    while b:
        if b & 1:
            r ^= a
        b >>= 1
        a <<= 1
        if a >> n & 1:
            a ^= p
    return r


def _powmod(e: int, p: int, n: int) -> int:
    r, base = 1, 2                               # the polynomial x
    while e:
        if e & 1:
            r = _mulmod(r, base, p, n)
        base = _mulmod(base, base, p, n)
        e >>= 1
    return r


def _prime_factors(m: int) -> list:
    out, d = [], 2
    while d * d <= m:
        while m % d == 0:
            if d not in out:
                out.append(d)
            m //= d
        d += 1
    if m > 1:
        out.append(m)
    return out


def _primitive(taps: list, n: int) -> bool:
    p = 1 << n
    for t in taps:
        p ^= 1 << t
    if not p & 1:
        return False
    order = 2 ** n - 1
    if _powmod(order, p, n) != 1:
        return False
    return all(_powmod(order // q, p, n) != 1 for q in _prime_factors(order))


@pytest.mark.parametrize("n", range(2, 13))
def test_oracle_lfsr_search_equals_primitive_polynomials(n):
    cands = LT._candidates(n)
    assert O.lfsr_search(n) == [t for t in cands if _primitive(t, n)]


def test_oracle_lfsr_known_answers():
    # x^8 + x^7 + x^2 + x + 1 is primitive; x^8 + x^7 + 1 is not (no primitive trinomial
    # of degree 8), and a tap set without bit 0 makes the register map non-invertible
    assert O.lfsr_distinct_states([7, 2, 1, 0], 8) == 255
    assert O.lfsr_distinct_states([7, 0], 8) < 255
    assert O.lfsr_distinct_states([7, 3, 2, 1], 8) < 255


def test_candidate_order_matches_reference_enumeration():
    # lfsr_taps.py:74-83: tap counts 2, 4, ...; combinations of the lower positions in
    # lexicographic order; each set sorted descending with the MSB first
    c = LT._candidates(5)
    assert c[:4] == [[4, 0], [4, 1], [4, 2], [4, 3]]
    assert c[4] == [4, 2, 1, 0]
    assert len(c) == sum(1 for k in range(1, 5, 2) for _ in __import__("itertools")
                         .combinations(range(4), k))


def test_shipped_tap_store_matches_oracle():
    store = LT.load_taps()
    assert sorted(store) == list(range(2, 17))
    for n, taps in store.items():
        assert taps == O.lfsr_search(n), n


def test_tap_store_roundtrip(tmp_path, capsys):
    f = tmp_path / "taps.json"
    LT.save_taps({5: [[4, 2, 1, 0]], 3: [[2, 0]]}, f)
    assert "Saved tap configurations" in capsys.readouterr().out
    assert json.loads(f.read_text()) == {"5": [[4, 2, 1, 0]], "3": [[2, 0]]}
    assert LT.load_taps(f) == {5: [[4, 2, 1, 0]], 3: [[2, 0]]}
    assert LT.get_taps(5, f) == [[4, 2, 1, 0]]
    assert LT.get_taps(7, f) == []
    assert LT.load_taps(tmp_path / "absent.json") == {}


# -------------------------------------------------------------------------------------
# config makers
# -------------------------------------------------------------------------------------

def _is_perm(s, p):
    return sorted(s) == list(range(p))


def test_default_taps_and_default_config():
    assert C.get_default_taps(8) == LT.get_taps(8)[0]
    cfg = C.make_default_config(3, 2, 8)
    assert cfg["rng_pool"] == [{"type": "lfsr", "seed": 125, "taps": C.get_default_taps(8)}]
    assert [s["scramble"] for s in cfg["sng"]["q"]] == [None] * 3
    assert [s["scramble"] for s in cfg["sng"]["k"]] == [list(range(7, -1, -1))] * 2
    with pytest.raises(ValueError, match="No pre-computed taps"):
        C.get_taps_choices(30)


def test_per_element_scramble_config():
    random.seed(3)
    cfg = C.make_per_element_scramble_config(6, 6, 8)
    for q, k in zip(cfg["sng"]["q"], cfg["sng"]["k"]):
        assert _is_perm(q["scramble"], 8) and k["scramble"] == q["scramble"][::-1]
    random.seed(3)
    assert C.make_per_element_scramble_config(6, 6, 8) == cfg
    cfg2 = C.make_per_element_scramble_config(4, 4, 8, k_reverse_of_q=False)
    assert all(_is_perm(s["scramble"], 8) for s in cfg2["sng"]["k"])
    with pytest.raises(AssertionError):
        C.make_per_element_scramble_config(3, 4, 8)


def test_fully_independent_config():
    random.seed(11)
    choices = LT.get_taps(8)
    cfg = C.make_fully_independent_config(5, 3, 8)
    pool = cfg["rng_pool"]
    assert len(pool) == 8
    assert [s["rng_id"] for s in cfg["sng"]["q"]] == [0, 1, 2, 3, 4]
    assert [s["rng_id"] for s in cfg["sng"]["k"]] == [5, 6, 7]
    assert all(e["taps"] in choices and 1 <= e["seed"] <= 255 for e in pool)
    # the reference's draw order: per element a choice of taps, then a seed
    random.seed(11)
    draws = []
    for _ in range(8):
        draws.append((random.choice(choices), random.randint(1, 255)))
    assert [(e["taps"], e["seed"]) for e in pool] == draws


def test_separated_and_random_configs():
    random.seed(2)
    sep = C.make_separated_random_config(4, 5, 8)
    assert [e["type"] for e in sep["rng_pool"]] == ["lfsr", "lfsr"]
    assert {s["rng_id"] for s in sep["sng"]["q"]} == {0}
    assert {s["rng_id"] for s in sep["sng"]["k"]} == {1}
    random.seed(2)
    rc = C.make_random_config(50, 50, 8)
    assert rc["rng_pool"] == sep["rng_pool"]          # same four leading draws
    scr = [s["scramble"] for s in rc["sng"]["q"] + rc["sng"]["k"]]
    assert any(s is None for s in scr) and any(s is not None for s in scr)
    assert all(s is None or _is_perm(s, 8) for s in scr)
    assert all(s["scramble"] is None
               for s in C.make_random_config(9, 9, 8, use_scrambling=False)["sng"]["q"])


def test_single_rng_reverse_config():
    random.seed(8)
    cfg = C.make_single_rng_reverse_config(5, 5, 8)
    assert len(cfg["rng_pool"]) == 1
    for q, k in zip(cfg["sng"]["q"], cfg["sng"]["k"]):
        assert k["scramble"] == q["scramble"][::-1]
    g = C.make_single_rng_reverse_config(3, 3, 8, use_per_element_scrambling=False)
    assert [s["scramble"] for s in g["sng"]["k"]] == [list(range(7, -1, -1))] * 3


def test_sobol_dse_config_builds():
    # the reference's maker fails on a broken import (config_helpers.py:692); this one works
    random.seed(4)
    cfg = C.make_sobol_dse_config(6, 6, 8)
    for e in cfg["rng_pool"]:
        seed = e["seed"]
        assert e["type"] == "sobol" and seed[0] == 1
        assert all(v % 2 == 1 and v < 2 ** (i + 1) for i, v in enumerate(seed))


# -------------------------------------------------------------------------------------
# saved configs and the best-config registry
# -------------------------------------------------------------------------------------

@pytest.fixture
def config_dir(tmp_path, monkeypatch):
    d = tmp_path / "configs"
    monkeypatch.setattr(C, "CONFIG_DIR", d)
    monkeypatch.setattr(C, "CONFIG_REGISTRY_FILE", d / "config_registry.json")

    # saved-config file names carry a timestamp to the second (as in the reference): a
    # clock that advances one second per call keeps the files of one test apart
    import datetime as _dt

    class _Clock(_dt.datetime):
        t = _dt.datetime(2026, 1, 1)

        @classmethod
        def now(cls, tz=None):
            cls.t += _dt.timedelta(seconds=1)
            return cls.t

    monkeypatch.setattr(C, "datetime", _Clock)
    return d


def test_save_and_load_config(config_dir):
    cfg = C.make_sobol_simple_config(2, 2)
    path = C.save_config(cfg, operation="matmul", sc_prec=8, error=0.5, notes="x")
    assert path.parent == config_dir and path.name.startswith("matmul_8bit_")
    got, meta = C.load_config(path)
    assert got == cfg
    assert meta["error"] == 0.5 and meta["notes"] == "x" and meta["operand_sizes"] == {}
    explicit = C.save_config(cfg, filepath=config_dir / "mine.json")
    assert C.load_config(explicit)[0] == cfg


def test_best_config_registry(config_dir):
    a = C.make_sobol_simple_config(1, 1)
    b = C.make_sobol_altseed_config(1, 1)
    assert C.load_best_config() == (None, None)
    C.save_best_config(a, error=0.3)
    assert C.load_best_config()[0] == a
    C.save_best_config(b, error=0.3)          # not better: registry keeps a
    assert C.load_best_config()[0] == a
    C.save_best_config(b, error=0.1)
    assert C.load_best_config()[0] == b
    C.save_best_config(a, error=0.2, sc_prec=6)
    keys = sorted((e["sc_prec"], e["error"]) for e in C.list_saved_configs())
    assert keys == [(6, 0.2), (8, 0.1)]
    # a registered file that has been deleted reads as no best config
    reg = json.loads(C.CONFIG_REGISTRY_FILE.read_text())
    __import__("os").remove(reg["matmul_8bit_fp8_e4m3"]["filepath"])
    assert C.load_best_config() == (None, None)

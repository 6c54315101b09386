"""Pins of the CPU oracle by closed forms, invariants, textbook special cases and brute
force: independent of the golden vectors, and chosen so that a plausible slip (a wrong
shift direction, tap index, off-by-one in a prefix, a transposed table, a dropped term)
fails at least one of them."""
import numpy as np
import pytest

from oracle import sc_oracle as O

FIRST16 = [0, 128, 192, 64, 96, 224, 160, 32, 48, 176, 240, 112, 80, 208, 144, 16]


# ---------------------------------------------------------------------------- Sobol

def _gray_closed_form(V, n):
    """x_t = XOR of V[k] over the set bits k of gray(t) = t ^ (t >> 1)."""
    out = []
    for t in range(n):
        g, x, k = t ^ (t >> 1), 0, 0
        while g:
            if g & 1:
                x ^= V[k]
            g >>= 1
            k += 1
        out.append(x)
    return np.array(out, dtype=np.int32)


@pytest.mark.parametrize("side,V", [("q", [128, 64, 32, 16, 8, 4, 2, 1]),
                                    ("k", [128, 64, 32, 16, 72, 4, 82, 255])])
def test_sobol_default_sequences(side, V):
    seq = O.sobol_sequence(8, O.sobol_default_seed(8, side), 256)
    assert seq[:16].tolist() == FIRST16                     # shared prefix (both seeds)
    assert sorted(seq.tolist()) == list(range(256))         # a permutation of [0, 2^p)
    np.testing.assert_array_equal(seq, _gray_closed_form(V, 256))


def test_sobol_q_is_bit_reversal_order():
    """With V = 2^(p-1-i) the Gray-code Sobol sequence is the bit-reversed Gray code."""
    seq = O.sobol_sequence(6, [1] * 6, 64)
    brev = [int(f"{t ^ (t >> 1):06b}"[::-1], 2) for t in range(64)]
    assert seq.tolist() == brev


# ----------------------------------------------------------------------------- LFSR

def test_lfsr_primitive_polynomial_has_full_period():
    """Right-shift Fibonacci LFSR, feedback into bit n-1 from the tapped bits: the output
    recurrence has characteristic polynomial x^n + sum_t x^t. Taps {0,2,3,4} give the
    primitive x^8+x^4+x^3+x^2+1, so every non-zero state appears once per 255 steps."""
    seq = O.lfsr_sequence(8, 1, [0, 2, 3, 4], 510)
    assert sorted(seq[:255].tolist()) == list(range(1, 256))
    np.testing.assert_array_equal(seq[:255], seq[255:])
    assert seq[0] == 1 and seq[1] == 128          # 1 -> (1 >> 1) | (1 << 7)


def test_lfsr_reducible_polynomial_has_short_period():
    seq = O.lfsr_sequence(8, 1, [0, 4], 256)      # x^8 + x^4 + 1 = (x^4 + x^2 + 1)^2
    period = 1 + seq[1:].tolist().index(1)
    assert period < 255


def test_lfsr_rejects_zero_seed():
    with pytest.raises(ValueError):
        O.lfsr_sequence(8, 0, [0, 2, 3, 4], 8)


# ------------------------------------------------------------------ SNG scrambles

def _bits(v, n):
    return [(int(v) >> i) & 1 for i in range(n)]


def test_scramble_identity_and_reversal():
    """The identity permutation leaves p-bit values unchanged; reverse_permutation(p) of
    scmp_kernels/sc/sng.py:56-58, [p-1, ..., 0], is p-bit reversal."""
    vals = np.arange(256, dtype=np.int32)
    np.testing.assert_array_equal(O.scramble(vals, list(range(8))), vals)
    rev = [int(f"{v:08b}"[::-1], 2) for v in range(256)]
    assert O.scramble(vals, list(range(7, -1, -1))).tolist() == rev
    rev5 = [int(f"{v:05b}"[::-1], 2) for v in range(32)]
    assert O.scramble(np.arange(32, dtype=np.int32), [4, 3, 2, 1, 0]).tolist() == rev5


def test_scramble_direction_known_answer():
    """Output bit i takes source bit perm[i] (sng.py:21-28). perm = [1, 2, 0]: value 1
    (bit 0 set) lands on output bit 2 (perm[2] = 0), so 1 -> 4; the opposite direction
    (output bit perm[i] <- source bit i) would give 1 -> 2."""
    got = O.scramble(np.array([1, 2, 4, 3, 6, 5, 7, 0], dtype=np.int32), [1, 2, 0])
    assert got.tolist() == [4, 1, 2, 5, 3, 6, 7, 0]


def test_scramble_inverse_round_trip_and_transposition():
    rng = np.random.default_rng(17)
    vals = rng.integers(0, 256, 500).astype(np.int32)
    for _ in range(5):
        perm = rng.permutation(8).tolist()
        inv = np.argsort(perm).tolist()            # perm[inv[i]] == i
        np.testing.assert_array_equal(O.scramble(O.scramble(vals, perm), inv), vals)
        # popcount is invariant under any bit permutation
        assert [bin(v).count("1") for v in O.scramble(vals, perm)] == \
            [bin(v).count("1") for v in vals]
    # a single transposition (2 5) swaps exactly bits 2 and 5
    perm = [0, 1, 5, 3, 4, 2, 6, 7]
    out = O.scramble(vals, perm)
    for v, w in zip(vals, out):
        bv, bw = _bits(v, 8), _bits(w, 8)
        assert bw[2] == bv[5] and bw[5] == bv[2]
        assert all(bw[i] == bv[i] for i in range(8) if i not in (2, 5))


def _lfsr_cfg(n, rng_ids, scrambles, pool):
    return {"rng_pool": pool,
            "sng": {"q": [{"rng_id": r, "scramble": s} for r, s in zip(rng_ids, scrambles)],
                    "k": [{"rng_id": rng_ids[0], "scramble": None}] * n}}


def test_sng_shared_rng_branch():
    """SNGBank.get_all_sequences with one shared RNG (sng.py:205-222): no scrambles ->
    the base sequence in every row; some scrambles -> apply_scramble_batch, where None is
    the identity over sc_prec bits, i.e. the base sequence again."""
    pool = [{"type": "lfsr", "seed": 45, "taps": [7, 5, 4, 3]}]
    base = O.lfsr_sequence(8, 45, [7, 5, 4, 3], 256)
    rev = list(range(7, -1, -1))
    cfg = _lfsr_cfg(3, [0, 0, 0], [None, None, None], pool)
    np.testing.assert_array_equal(O.sng_sequences(cfg, "q", 8), np.stack([base] * 3))
    cfg = _lfsr_cfg(3, [0, 0, 0], [None, rev, None], pool)
    seqs = O.sng_sequences(cfg, "q", 8)
    np.testing.assert_array_equal(seqs[0], base)
    np.testing.assert_array_equal(seqs[2], base)
    assert seqs[1].tolist() == [int(f"{v:08b}"[::-1], 2) for v in base]


def test_sng_multi_rng_branch():
    """Several RNG ids (sng.py:223-230): each row is its own RNG's sequence, scrambled by
    its own permutation where one is given and raw otherwise."""
    pool = [{"type": "lfsr", "seed": 45, "taps": [7, 5, 4, 3]},
            {"type": "lfsr", "seed": 3, "taps": [7, 6, 5, 0]}]
    b0 = O.lfsr_sequence(8, 45, [7, 5, 4, 3], 256)
    b1 = O.lfsr_sequence(8, 3, [7, 6, 5, 0], 256)
    assert not np.array_equal(b0, b1)
    rev = list(range(7, -1, -1))
    cfg = _lfsr_cfg(4, [0, 1, 1, 0], [None, None, rev, rev], pool)
    seqs = O.sng_sequences(cfg, "q", 8)
    np.testing.assert_array_equal(seqs[0], b0)
    np.testing.assert_array_equal(seqs[1], b1)
    assert seqs[2].tolist() == [int(f"{v:08b}"[::-1], 2) for v in b1]
    assert seqs[3].tolist() == [int(f"{v:08b}"[::-1], 2) for v in b0]


# ------------------------------------------------------------ prefix / Owen / rescale

def test_owen_bitrev_masks():
    m = O.owen_masks(300, 256, "bitrev")
    want = [int(f"{d % 256:08b}"[::-1], 2) for d in range(300)]
    assert m.tolist() == want
    assert O.owen_masks(5, 256, "off") is None
    assert O.owen_masks(300, 256, "counter").tolist() == [d % 256 for d in range(300)]


@pytest.mark.parametrize("L,R", [(256, 256), (64, 256), (64, 64), (16, 16), (128, 32)])
def test_prepare_prefix_closed_form(L, R):
    D = 40
    cfg = O.make_sobol_simple_config(D, D, 8)
    full = O.sng_sequences(cfg, "k", 8)
    got = O.prepare_prefix(full, 8, L, R, "bitrev", True)
    mask = np.array([int(f"{d:08b}"[::-1], 2) for d in range(D)])[:, None]
    if R == 256:
        want = full[:, :L] ^ mask if L < 256 else full
    else:
        want = ((full[:, :L] ^ mask) * R) // 256
    np.testing.assert_array_equal(got, want)
    if R < 256:   # rescaled values cover [0, R)
        assert got.min() >= 0 and got.max() < R


# --------------------------------------------------------------------------- tables

def test_k_and_c_tables_invariants():
    cfg = O.make_sobol_simple_config(3, 3, 8)
    ra = O.sng_sequences(cfg, "q", 8)
    rb = O.sng_sequences(cfg, "k", 8)
    K = O.k_table(ra, 512)
    C = O.c_table(rb, 512)
    v = np.arange(512)
    # full-length Sobol is a permutation of [0, 256): K[d, v] = min(v, 256)
    np.testing.assert_array_equal(K[0], np.minimum(v, 256))
    assert (C[:, 0, :] == 0).all()                          # empty prefix
    np.testing.assert_array_equal(C[0, 256], np.minimum(v, 256))  # whole stream
    assert (np.diff(C[0].astype(int), axis=0) >= 0).all()   # monotone in k
    assert (np.diff(C[0].astype(int), axis=1) >= 0).all()   # monotone in v
    # each prefix step adds exactly the indicator of the new element
    step = np.diff(C[0].astype(int), axis=0)
    np.testing.assert_array_equal(step, (rb[0][:, None] < v[None, :]).astype(int))


# ---------------------------------------------------------------------- accumulator

@pytest.mark.parametrize("L,R", [(256, 256), (64, 64), (32, 256)])
def test_accumulator_table_form_equals_stream_form(L, R):
    """The reference's table lookup against the bitstream AND + popcount definition."""
    rng = np.random.default_rng(L + R)
    N, M, D = 7, 9, 21
    tabs = O.Tables(O.make_sobol_simple_config(D, D, 8), 8, L, R)
    ba = rng.integers(0, R + 1, (N, D)).astype(np.int16)
    bb = rng.integers(0, R + 1, (M, D)).astype(np.int16)
    sa = rng.choice([-1, 1], (N, D)).astype(np.int8)
    sb = rng.choice([-1, 1], (M, D)).astype(np.int8)
    I_tab = O.sc_accum(ba, sa, bb, sb, tabs)
    I_str = O.sc_accum_stream(ba, sa, bb, sb, tabs.ra, tabs.rb)
    np.testing.assert_array_equal(I_tab, I_str)
    # dropping the signs changes the result (the sign product is not a no-op)
    assert not np.array_equal(O.sc_accum(ba, None, bb, None, tabs), I_tab)


def test_accumulator_special_cases():
    D = 10
    tabs = O.Tables(O.make_sobol_simple_config(D, D, 8), 8, 256, 256)
    one = np.ones((1, D), np.int8)
    full = np.full((1, D), 256, np.int16)
    zero = np.zeros((1, D), np.int16)
    vals = np.arange(D, dtype=np.int16)[None, :] * 25
    # beta_b = 256 counts K_a = beta_a (full-length Sobol) per d
    assert O.sc_accum(vals, one, full, one, tabs)[0, 0] == int(vals.sum())
    # beta_a = 256 counts every position below beta_b
    assert O.sc_accum(full, one, vals, one, tabs)[0, 0] == int(vals.sum())
    # any zero boundary contributes nothing; saturation gives L per d
    assert O.sc_accum(zero, one, full, one, tabs)[0, 0] == 0
    assert O.sc_accum(full, one, full, -one, tabs)[0, 0] == -256 * D


def test_accumulator_expectation():
    """E[count] ~ beta_a * beta_b / 2^p for the low-discrepancy streams."""
    D = 64
    tabs = O.Tables(O.make_sobol_simple_config(D, D, 8), 8, 256, 256)
    rng = np.random.default_rng(3)
    ba = rng.integers(0, 257, (16, D)).astype(np.int16)
    bb = rng.integers(0, 257, (16, D)).astype(np.int16)
    I = O.sc_accum(ba, None, bb, None, tabs).astype(np.float64)
    exact = ba.astype(np.float64) @ bb.T.astype(np.float64) / 256.0
    assert np.abs(I - exact).max() / np.abs(exact).max() < 0.02


# ------------------------------------------------------------------------ boundary

@pytest.mark.parametrize("Q", [127, 255])
@pytest.mark.parametrize("R", [16, 32, 64, 128, 256])
def test_boundary_closed_form(Q, R):
    """beta = rne(m*R/Q) has no ties (R a power of two, Q odd), so it equals
    floor((2mR + Q) / (2Q)) exactly, for both fp32 formulas of the reference."""
    m = np.arange(0, Q + 2, dtype=np.float32)
    want = (2 * m.astype(np.int64) * R + Q) // (2 * Q)
    np.testing.assert_array_equal(O.beta_div(m, Q, R), want)
    np.testing.assert_array_equal(O.beta_mul(m, Q, R), want)
    np.testing.assert_array_equal(O.beta_div(-m, Q, R), want)   # magnitude of negatives

"""GPU parity: every HIP kernel (through the C ABI) against the CPU oracle on the same
seeded inputs, and sc_matmul against the reference's golden vectors. Bit-exact: integer
sequences, tables, quantized codes and accumulators; fp32 outputs compared bitwise."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import sc_oracle as O

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _dev():
    return torch.device("cuda", 0)


def T(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(_dev())


def bits_equal(got: torch.Tensor, ref: np.ndarray):
    g = got.detach().cpu().numpy()
    assert g.shape == ref.shape, (g.shape, ref.shape)
    if g.dtype.kind == "f":
        g = g.astype(ref.dtype)
        bad = g.view(np.uint8 if g.itemsize == 1 else np.uint32 if g.itemsize == 4 else np.uint64) \
            != ref.view(np.uint8 if ref.itemsize == 1 else np.uint32 if ref.itemsize == 4 else np.uint64)
    else:
        bad = g != ref
    n = int(np.count_nonzero(bad))
    assert n == 0, f"{n} of {bad.size} elements differ; first at {np.argwhere(bad)[0].tolist()}"


# -------------------------------------------------------------------------------------
# RNG sequences, prefix/Owen/rescale, stream tables
# -------------------------------------------------------------------------------------

@pytest.mark.parametrize("p", [4, 6, 8])
@pytest.mark.parametrize("seed_type", ["q", "k"])
def test_sobol_sequence(p, seed_type):
    from scmp_kernels_amd.sc.rng import Sobol
    got = Sobol(p, seed_type=seed_type).simulate()
    ref = O.sobol_sequence(p, O.sobol_default_seed(p, seed_type), 2 ** p)
    np.testing.assert_array_equal(got, ref)


def test_sobol_custom_seed_and_lfsr():
    from scmp_kernels_amd.sc.rng import Sobol, LFSR
    seed = [1, 3, 7, 15, 31, 63, 127, 255]
    np.testing.assert_array_equal(Sobol(8, seed=seed).simulate(),
                                  O.sobol_sequence(8, seed, 256))
    for taps in ([7, 5, 4, 3], [7, 6, 5, 0], [7, 3, 2, 1]):
        np.testing.assert_array_equal(LFSR(125, 8, taps).simulate(),
                                      O.lfsr_sequence(8, 125, taps, 256))


@pytest.mark.parametrize("L,R,mode,srs", [(256, 256, "bitrev", True), (64, 256, "bitrev", True),
                                          (64, 64, "bitrev", True), (16, 16, "counter", True),
                                          (128, 128, "random", True), (32, 32, "bitrev", False),
                                          (64, 64, "off", True)])
def test_prepare_prefix(L, R, mode, srs):
    from scmp_kernels_amd.sc import tables as TB
    D = 300
    cfg = O.make_sobol_simple_config(D, D, 8)
    ref_full = O.sng_sequences(cfg, "k", 8)
    got_full = TB.side_sequences(cfg, "k", 8, D, _dev())
    bits_equal(got_full, ref_full)
    masks = TB.owen_masks(D, 256, mode, _dev())
    ref_masks = O.owen_masks(D, 256, mode, _dev())
    if masks is None:
        assert ref_masks is None
    else:
        np.testing.assert_array_equal(masks, ref_masks)
    got = TB.prepare(got_full, 8, L, R, masks, srs)
    bits_equal(got, O.prepare_prefix(ref_full, 8, L, R, mode, srs, owen_device=_dev()))


def test_scrambled_config_sequences():
    from scmp_kernels_amd.sc import tables as TB
    from scmp_kernels_amd.sc.config_helpers import make_sobol_custom_seed_config
    import random
    random.seed(5)
    cfg = make_sobol_custom_seed_config(40, 40, 8, use_scrambling=True)
    for side in ("q", "k"):
        bits_equal(TB.side_sequences(cfg, side, 8, 40, _dev()), O.sng_sequences(cfg, side, 8))
    # shared RNG with some elements unscrambled -> identity over sc_prec bits
    cfg["rng_pool"] = [{"type": "lfsr", "seed": 77, "taps": [7, 5, 4, 3]}]
    for s in cfg["sng"]["q"] + cfg["sng"]["k"]:
        s["rng_id"] = 0
    cfg["sng"]["q"][3]["scramble"] = None
    for side in ("q", "k"):
        bits_equal(TB.side_sequences(cfg, side, 8, 40, _dev()), O.sng_sequences(cfg, side, 8))


def _lut_counts(tabs, c, L):
    """count[qa_row, qb_row] = sum_{j' < jtab[|qa|]} lut[qb_row][j'] from the HIP tables."""
    JP = tabs.JP
    lut = tabs.lut[c].cpu().numpy().astype(np.int64)        # (256, JP) interleaved bytes
    U = JP // 4
    jp = np.arange(JP)
    byte_of = 4 * (jp % U) + jp // U                          # logical j' -> byte offset
    logical = lut[:, byte_of]                                 # (256, JP) in j' order
    cum = np.concatenate([np.zeros((256, 1), np.int64), np.cumsum(logical, axis=1)], axis=1)
    return cum, tabs.jtab[c].cpu().numpy().astype(np.int64)


@pytest.mark.parametrize("L,R,bipolar,p", [(256, 256, True, 8), (128, 128, True, 8),
                                           (64, 64, False, 8), (16, 16, False, 8),
                                           (256, 256, False, 8), (64, 256, True, 8),
                                           (64, 64, True, 6), (32, 32, True, 8)])
def test_stream_tables_match_reference_tables(L, R, bipolar, p):
    """sum_{j'<j(q_a)} lut[q_b][j'] == C[K[beta(q_a)], beta(q_b)] for every class, q_a, q_b."""
    from scmp_kernels_amd.sc import tables as TB
    from scmp_kernels_amd.sc.config_helpers import make_sobol_simple_config
    D = 260
    TB.clear()
    tabs = TB.get_tables(None, ("t", D, p), lambda: make_sobol_simple_config(D, D, p), p, L, R,
                         bipolar, D, _dev())
    ref = O.Tables(O.make_sobol_simple_config(D, D, p), p, L, R)
    Q = 2 ** (p - 1) - 1 if bipolar else 2 ** p - 1
    qmax = Q + 1 if bipolar else Q
    beta = TB.beta_of_q(np.arange(qmax + 1), Q, R)
    reps = {}
    for d in range(D):
        reps.setdefault(int(tabs.class_of[d]), d)
    for c, d in reps.items():
        cum, jtab = _lut_counts(tabs, c, L)
        td = ref.tab_of[d]
        K, C = ref.K[td], ref.C[td]
        for qa in range(qmax + 1):
            ka = K[beta[qa]]
            j = jtab[qa]
            for qb in range(-(Q + 1) if bipolar else 0, Q + 1):
                row = qb & 0xff
                want = C[ka, beta[abs(qb)]] * (-1 if qb < 0 else 1)
                assert cum[row, j] == want, (c, qa, qb, cum[row, j], want)


# -------------------------------------------------------------------------------------
# quantizers
# -------------------------------------------------------------------------------------

def _qx(seed=0, rows=37, cols=131):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0, :6] = [0.0, 0.5, -0.5, 1.5, -2.5, 1e-7]
    x[1] = 0.0
    x[2] *= 1e-6
    return x


def test_quant_fused_perrow():
    from scmp_kernels_amd.quant import fused_quantize_bipolar_perrow
    x = _qx(1)
    for R in (256, 64, 16):
        b, s, sc = fused_quantize_bipolar_perrow(T(x), 8, rng_levels=R)
        rb, rs, rsc = O.quant_fused_perrow_bipolar(x, 8, R)
        bits_equal(b, rb); bits_equal(s, rs); bits_equal(sc, rsc)


def test_quant_fused_tensor_and_unipolar():
    from scmp_kernels_amd.quant import fused_quantize_bipolar, fused_quantize_unipolar
    x = _qx(2)
    am = float(np.abs(x).max())
    b, s, sc = fused_quantize_bipolar(T(x), am, 8)
    rb, rs, rsc = O.quant_fused_bipolar(x, am, 8, 256)
    bits_equal(b, rb); bits_equal(s, rs); assert sc == rsc
    for R in (256, 64):
        b, sc, zp, rsum = fused_quantize_unipolar(T(x), float(x.max()), float(x.min()), 8,
                                                  compute_sum=True, rng_levels=R)
        rb, rsc, rzp, rrs = O.quant_fused_unipolar(x, float(x.max()), float(x.min()), 8, R)
        bits_equal(b, rb); bits_equal(rsum, rrs); assert (sc, zp) == (rsc, rzp)


@pytest.mark.parametrize("G", [1, 4, 5, 100])
def test_quant_grouped(G):
    from scmp_kernels_amd.quant import _grouped_symmetric_quant, _grouped_asymmetric_quant
    x = _qx(3)
    s, xi, sg = _grouped_symmetric_quant(T(x), G, 127)
    rs, rxi, rsg = O.grouped_sym(x, G, 127)
    bits_equal(s, rs); bits_equal(xi, rxi); bits_equal(sg, rsg)
    s, zp, xi = _grouped_asymmetric_quant(T(x), G, 255)
    rs, rzp, rxi = O.grouped_asym(x, G, 255)
    bits_equal(s, rs); bits_equal(zp, rzp); bits_equal(xi, rxi)


@pytest.mark.parametrize("rows,cols,G", [(301, 4096, 4), (97, 3000, 4), (50, 2100, 2),
                                         (9, 1030, 4)])
def test_quant_grouped_wide(rows, cols, G):
    """Few groups of 1025-4096 four-column chunks: 1024-thread workgroups (a ragged last
    group, rows not a multiple of 4 columns, one to four chunks per thread)."""
    from scmp_kernels_amd.quant import _grouped_symmetric_quant, _grouped_asymmetric_quant
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[rng.integers(0, rows, 5)] *= 30.0
    s, xi, sg = _grouped_symmetric_quant(T(x), G, 127)
    rs, rxi, rsg = O.grouped_sym(x, G, 127)
    bits_equal(s, rs); bits_equal(xi, rxi); bits_equal(sg, rsg)
    s, zp, xi = _grouped_asymmetric_quant(T(x), G, 255)
    rs, rzp, rxi = O.grouped_asym(x, G, 255)
    bits_equal(s, rs); bits_equal(zp, rzp); bits_equal(xi, rxi)


def test_quant_grouped_batched():
    from scmp_kernels_amd.quant import _grouped_symmetric_quant_batched
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 7, 19)).astype(np.float32)
    for G in (1, 7, 10):
        s, xi, sg = _grouped_symmetric_quant_batched(T(x), G, 127)
        rs, rxi, rsg = O.grouped_sym_batched(x, G, 127)
        bits_equal(s, rs); bits_equal(xi, rxi); bits_equal(sg, rsg)
    with pytest.raises(NotImplementedError):
        _grouped_symmetric_quant_batched(T(x), 3, 127)


def _near_half(seed, rows, cols, Q, asym):
    """Rows whose quotients x / s sit at (or within 1e-4 of) half-integers, where the
    quantizer's multiply-by-reciprocal shortcut must hand over to the exact division, plus
    exact multiples of s and values at the clamp."""
    rng = np.random.default_rng(seed)
    A = (rng.uniform(0.5, 2.0, rows) * 10.0 ** rng.integers(-3, 3, rows)).astype(np.float32)
    if asym:
        lo = (-A * rng.uniform(0.0, 1.0, rows)).astype(np.float32)
        s = (np.maximum(A - lo, np.float32(1e-5)) / np.float32(Q)).astype(np.float32)
        zp = np.clip(np.rint((-lo / s).astype(np.float32)), 0, Q).astype(np.float32)
        k = rng.integers(0, Q, (rows, cols)).astype(np.float32)
        base = (-zp * s)[:, None]                # x / s + zp lands on k + frac + d
    else:
        s = (np.maximum(A, np.float32(1e-5)) / np.float32(Q)).astype(np.float32)
        k = rng.integers(-Q, Q, (rows, cols)).astype(np.float32)
        base = np.zeros((rows, 1), np.float32)
    d = rng.choice(np.array([0.0, 1e-7, -1e-7, 3e-5, -3e-5, 1e-4, -1e-4, 0.25], np.float32),
                   (rows, cols))
    frac = np.where(rng.random((rows, cols)) < 0.8, np.float32(0.5), np.float32(0.0))
    x = (base + (k + frac + d) * s[:, None]).astype(np.float32)
    x = np.clip(x, (lo if asym else -A)[:, None], A[:, None]).astype(np.float32)
    x[:, 0] = A                                  # pins the statistic of every row
    if asym:
        x[:, 1] = lo
    return x


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("smooth_mode", [0, 1, 2])
def test_quant_codes_near_half_integers(asym, smooth_mode):
    """GEMM code bytes of the row quantizers (codes-only path, full 4-column chunks) on
    quotients placed at half-integers, against the oracle's exact-division quantizer."""
    from scmp_kernels_amd import _lib
    from scmp_kernels_amd.sc import kernels as K
    rows, cols = 64, 256
    Q = 255 if asym else 127
    x = _near_half(7 + smooth_mode + 3 * asym, rows, cols, Q, asym)
    sm = None
    xs = x
    if smooth_mode:
        sm = np.random.default_rng(11).uniform(0.25, 4.0, cols).astype(np.float32)
        xs = (x / sm if smooth_mode == 1 else x * sm).astype(np.float32)
    if asym:
        _, _, ref_q = O.grouped_asym(xs, 1, Q)
    else:
        _, ref_q, _ = O.grouped_sym(xs, 1, Q)
    ref = (ref_q.astype(np.int32) & 0xff).astype(np.uint8)
    code = torch.full((256, cols), 0x5A, dtype=torch.uint8, device=_dev())
    ws = K.quantize(T(x), _lib.Q_GROUP_ASYM if asym else _lib.Q_GROUP_SYM, Q, 256,
                    smooth=None if sm is None else T(sm), smooth_mode=smooth_mode,
                    code=code, code_kind=_lib.CODE_Q)
    got = code.cpu().numpy()
    del ws
    np.testing.assert_array_equal(got[:rows], ref)
    assert not got[rows:].any()                  # padding rows are zero


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("cols,rows,G,cbr", [(197, 39, 5, 13), (198, 39, 5, 13),
                                             (199, 39, 13, 13), (197, 200, 100, 200)])
def test_quant_codes_ragged_columns_and_padding(asym, cols, rows, G, cbr):
    """Row-group quantizer codes when the row length is not a multiple of 4 (the last
    4-column chunk is partial), in batches of cbr rows, with the padding rows of every batch
    and the columns past the row end pre-filled with garbage: codes equal the oracle's,
    padding is zero, row sums count only real columns. The (197, 200, 100) case holds more
    chunks per group than the registers do (the re-reading path)."""
    from scmp_kernels_amd import _lib
    from scmp_kernels_amd.sc import kernels as K
    Q = 255 if asym else 127
    x = np.random.default_rng(cols + rows + G).standard_normal((rows, cols)).astype(np.float32)
    if asym:
        _, _, ref_q = O.grouped_asym(x, G, Q)
    else:
        _, ref_q, _ = O.grouped_sym(x, G, Q)
    ref = (ref_q.astype(np.int32) & 0xff).astype(np.uint8)
    nb = rows // cbr
    ld = (cols + 15) // 16 * 16
    code = torch.full((nb, cbr + 19, ld), 0x5A, dtype=torch.uint8, device=_dev())
    rs = torch.full((rows,), -1.0, dtype=torch.float32, device=_dev()) if asym else None
    ws = K.quantize(T(x), _lib.Q_GROUP_ASYM if asym else _lib.Q_GROUP_SYM, Q, 256, group=G,
                    code=code, code_kind=_lib.CODE_Q, code_batch_rows=cbr, rowsum=rs)
    got = code.cpu().numpy()
    del ws
    np.testing.assert_array_equal(got[:, :cbr, :cols].reshape(rows, cols), ref)
    assert not got[:, :cbr, cols:].any()          # columns past the row end
    assert not got[:, cbr:, :].any()              # padding rows of every batch
    if asym:
        np.testing.assert_array_equal(rs.cpu().numpy(),
                                      ref_q.astype(np.float64).sum(axis=1).astype(np.float32))


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("rows", [1368, 1000])
def test_quant_codes_wide_groups(asym, rows):
    """Row groups of 4 x 4096 (4096 four-column chunks), more groups than compute units
    (1368 rows: 342 groups, 512-thread workgroups two per compute unit) and fewer (1000
    rows: 250 groups, 1024-thread workgroups): code bytes and row sums against the
    oracle."""
    from scmp_kernels_amd import _lib
    from scmp_kernels_amd.sc import kernels as K
    G, cols = 4, 4096
    Q = 255 if asym else 127
    x = np.random.default_rng(rows + asym).standard_normal((rows, cols)).astype(np.float32)
    if asym:
        _, _, ref_q = O.grouped_asym(x, G, Q)
    else:
        _, ref_q, _ = O.grouped_sym(x, G, Q)
    ref = (ref_q.astype(np.int32) & 0xff).astype(np.uint8)
    code = torch.full((rows, cols), 0x5A, dtype=torch.uint8, device=_dev())
    rs = torch.full((rows,), -1.0, dtype=torch.float32, device=_dev()) if asym else None
    ws = K.quantize(T(x), _lib.Q_GROUP_ASYM if asym else _lib.Q_GROUP_SYM, Q, 256, group=G,
                    code=code, code_kind=_lib.CODE_Q, rowsum=rs)
    got = code.cpu().numpy()
    del ws
    np.testing.assert_array_equal(got, ref)
    if asym:
        np.testing.assert_array_equal(rs.cpu().numpy(),
                                      ref_q.astype(np.float64).sum(axis=1).astype(np.float32))


# -------------------------------------------------------------------------------------
# the SC GEMM: integer accumulator against the oracle
# -------------------------------------------------------------------------------------

def _int_accum_gpu(a, b, *, L, R, bipolar, group=1, impl=0, tile=0, D=None):
    """I[n, m] through the product kernels (quantizer codes + scmp_sc_gemm EPI_INT)."""
    from scmp_kernels_amd import _lib
    from scmp_kernels_amd.sc import kernels as K
    dev = _dev()
    A, B = T(a), T(b)
    N, D = a.shape
    M = b.shape[0]
    tabs = K._get_tables(None, 8, L, R, bipolar, D, dev)
    ca, cb = K._codes(N, D, dev), K._codes(M, D, dev)
    var = _lib.Q_GROUP_SYM if bipolar else _lib.Q_GROUP_ASYM
    Q = 127 if bipolar else 255
    w1 = K.quantize(A, var, Q, R, group=group, code=ca, code_kind=_lib.CODE_THERMO,
                    jtab=tabs.jtab, col_class=tabs.d_class)
    w2 = K.quantize(B, var, Q, R, group=group, code=cb, code_kind=_lib.CODE_Q)
    I = torch.empty((N, M), dtype=torch.int32, device=dev)
    epi = _lib.Epilogue()
    epi.kind = _lib.EPI_INT
    K.sc_gemm(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, iout=I, impl=impl, tile=tile)
    torch.cuda.synchronize()
    del w1, w2
    return I.cpu().numpy()


def _int_accum_ref(a, b, *, L, R, bipolar, group=1):
    D = a.shape[1]
    tabs = O.Tables(O.make_sobol_simple_config(D, D, 8), 8, L, R)
    if bipolar:
        sa, qa, sga = O.grouped_sym(a, group, 127)
        sb, qb, sgb = O.grouped_sym(b, group, 127)
        return O.sc_accum(O.beta_div(qa, 127, R), sga, O.beta_div(qb, 127, R), sgb, tabs)
    sa, za, qa = O.grouped_asym(a, group, 255)
    sb, zb, qb = O.grouped_asym(b, group, 255)
    return O.sc_accum(O.beta_div(qa, 255, R, False), None, O.beta_div(qb, 255, R, False), None,
                      tabs)


GEMM_CASES = [
    # (N, M, D, L, R, bipolar)    JP: 128 / 128 / 64 / 16 / 256 / 32
    (70, 45, 96, 256, 256, True),
    (257, 300, 200, 128, 128, True),
    (33, 97, 77, 64, 64, False),
    (40, 31, 50, 16, 16, False),
    (65, 66, 129, 256, 256, False),
    (31, 129, 64, 32, 32, True),
    # D >= 512: the FP4 kernel shares tiles between workgroups (split inner dimension,
    # exact partial sums combined by the last contributor)
    (300, 500, 1024, 256, 256, True),
    (260, 270, 600, 128, 128, True),
    (257, 300, 777, 64, 64, False),
    # outputs 193 to 224 wide take 256 x 224 FP4 tiles (whole, and shared at D >= 512)
    (300, 210, 96, 256, 256, True),
    (300, 197, 1024, 128, 128, False),
]


# (impl, tile): int8 MFMA presets 0-4, VALU popcount, FP4 MFMA
KERNELS = [(0, 0), (0, 1), (0, 2), (0, 3), (0, 4), (1, 0), (2, 0)]


@pytest.mark.parametrize("case", GEMM_CASES)
@pytest.mark.parametrize("impl,tile", KERNELS)
def test_gemm_int_accumulator(case, impl, tile):
    N, M, D, L, R, bip = case
    rng = np.random.default_rng(N * 7 + M)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = rng.standard_normal((M, D)).astype(np.float32)
    a[3] = 0.0                                     # an all-zero row
    got = _int_accum_gpu(a, b, L=L, R=R, bipolar=bip, impl=impl, tile=tile)
    ref = _int_accum_ref(a, b, L=L, R=R, bipolar=bip)
    np.testing.assert_array_equal(got, ref)


def _random_gemm_shapes(n):
    rng = np.random.default_rng(2024)
    modes = [(256, 256, True), (128, 128, True), (64, 64, False), (16, 16, False)]
    out = []
    for k in range(n):
        N = int(rng.integers(1, 420))
        M = int(rng.integers(1, 420))
        # inner dimensions around the split threshold (512) and off multiples of 8 / 16
        D = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(500, 1100))]))
        out.append((N, M, D) + modes[k % len(modes)])
    return out


def test_gemm_wide_tile_padding_rule():
    """Few rows and M = 2300 (M rounded up to 512 passes the 256-row padding of the code
    buffers): 128 x 512 tiles would read B rows past the buffer, so the plan keeps 256 x 256
    tiles; and M = 2560, where 128 x 512 tiles are taken."""
    for N, M, D in ((100, 2300, 96), (100, 2560, 64)):
        rng = np.random.default_rng(N + M)
        a = rng.standard_normal((N, D)).astype(np.float32)
        b = rng.standard_normal((M, D)).astype(np.float32)
        got = _int_accum_gpu(a, b, L=64, R=64, bipolar=True, impl=2)
        np.testing.assert_array_equal(got, _int_accum_ref(a, b, L=64, R=64, bipolar=True))


@pytest.mark.parametrize("case", _random_gemm_shapes(12))
def test_gemm_random_shapes_fp4(case):
    """Seeded random shapes through the default (FP4) kernel: whole and split tiles,
    narrow outputs, lone last groups, inner dimensions off multiples of 8."""
    N, M, D, L, R, bip = case
    rng = np.random.default_rng(N + 1000 * M + D)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = rng.standard_normal((M, D)).astype(np.float32)
    got = _int_accum_gpu(a, b, L=L, R=R, bipolar=bip, impl=2)
    ref = _int_accum_ref(a, b, L=L, R=R, bipolar=bip)
    np.testing.assert_array_equal(got, ref)


def test_gemm_extremes():
    """Saturated operands: every code at +-Q (full-length Sobol: count = L per d)."""
    N, M, D = 64, 64, 48
    a = np.ones((N, D), np.float32)
    a[::2] *= -1
    b = np.ones((M, D), np.float32)
    ref = _int_accum_ref(a, b, L=256, R=256, bipolar=True)
    for impl, tile in KERNELS:
        got = _int_accum_gpu(a, b, L=256, R=256, bipolar=True, impl=impl, tile=tile)
        np.testing.assert_array_equal(got, ref)
        assert abs(int(got[0, 0])) == 256 * D


# -------------------------------------------------------------------------------------
# sc_matmul end to end
# -------------------------------------------------------------------------------------

with open(os.path.join(GOLD, "cases.json")) as f:
    _CASES = json.load(f)
GOLDEN_MATMUL = sorted(k for k, v in _CASES.items() if v["kind"] == "sc_matmul")


@pytest.mark.parametrize("name", GOLDEN_MATMUL)
def test_sc_matmul_golden(name, monkeypatch):
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.sc import clear_rng_cache
    meta = _CASES[name]
    with np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False) as z:
        z = {k: z[k] for k in z.files}
    for k, v in meta["env"].items():
        monkeypatch.setenv(k, v)
    clear_rng_cache()
    kw = dict(meta["kwargs"])
    if "smooth" in z:
        kw["smooth_scales"] = T(z["smooth"])
    y = sc_matmul(T(z["a"]), T(z["b"]), **kw)
    clear_rng_cache()
    if meta["env"].get("SC_OWEN_MODE") == "random":
        # The reference draws 'random' Owen masks from the generator of the device its
        # sequences live on (sc/kernels.py:664-668): the vector, written on the CPU, pins
        # the oracle with the CPU generator; on the GPU both sides use the device's.
        kw.pop("smooth_scales", None)
        gran = kw.pop("granularity")
        ref = O.sc_matmul(z["a"], z["b"], gran, smooth_scales=z.get("smooth"),
                          ctx=O.Ctx(owen_mode="random", owen_device=_dev()), **kw)
        bits_equal(y, ref)
        return
    bits_equal(y, z["y"])


def test_owen_random_masks_use_the_device_generator():
    """The product's 'random' masks are torch.randint on the sequences' device with the
    reference's seed (sc/kernels.py:664-668), and differ from the CPU generator's."""
    from scmp_kernels_amd.sc import tables as TB
    g = torch.Generator(device=_dev()).manual_seed(0x5A5A5A5A)
    want = torch.randint(0, 256, (300, 1), generator=g, device=_dev()).reshape(-1)
    got = TB.owen_masks(300, 256, "random", _dev())
    np.testing.assert_array_equal(got, want.cpu().numpy())
    assert not np.array_equal(got, TB.owen_masks(300, 256, "random", "cpu"))


RANDOM_CASES = [
    ("per_row", dict(mode="bipolar"), (129, 67, 300)),
    ("per_row", dict(mode="unipolar", group_a=4, group_b=4), (130, 70, 96)),
    ("per_row", dict(mode="unipolar", group_a=4, group_b=4, stoc_len=64, rng_levels=64),
     (97, 61, 200)),
    ("per_row", dict(mode="unipolar", group_a=4, group_b=3, stoc_len=16, rng_levels=16),
     (50, 40, 64)),
    ("per_row", dict(mode="bipolar", chunk_d=72), (300, 65, 3 * 72 + 48)),
    # 16-interval tables through the chunk_d kernel (stored in 32-interval rows)
    ("per_row", dict(mode="bipolar", chunk_d=24, stoc_len=16), (90, 70, 5 * 24 + 10)),
    ("per_row", dict(mode="bipolar", chunk_d=26, stoc_len=16, rng_levels=16), (70, 90, 4 * 26)),
    # odd chunks with 16- and 32-interval tables (widened to 64 intervals, one d per k-step)
    ("per_row", dict(mode="bipolar", chunk_d=25, stoc_len=16), (80, 66, 4 * 25 + 7)),
    ("per_row", dict(mode="bipolar", chunk_d=9, stoc_len=8, rng_levels=16), (40, 30, 5 * 9)),
    ("per_row", dict(mode="bipolar", chunk_d=27, stoc_len=32), (70, 45, 3 * 27 + 11)),
    ("per_row", dict(mode="bipolar", halve_bipolar_stoc_len=True), (64, 64, 128)),
    ("per_tensor", dict(mode="bipolar"), (32, 64, 256)),
    ("per_tensor", dict(mode="unipolar"), (40, 33, 100)),
    # outputs at most 64 wide: 256 x 64 tiles, shared between workgroups (split partial
    # sums) at these inner dimensions
    ("per_row", dict(mode="bipolar"), (1000, 64, 1024)),
    ("per_row", dict(mode="bipolar"), (700, 40, 2048)),
]


@pytest.mark.parametrize("gran,kw,shape", RANDOM_CASES)
def test_sc_matmul_vs_oracle(gran, kw, shape):
    from scmp_kernels_amd import sc_matmul
    N, M, D = shape
    rng = np.random.default_rng(N + M + D)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = (rng.standard_normal((M, D)) * 0.05).astype(np.float32)
    y = sc_matmul(T(a), T(b), gran, **kw)
    bits_equal(y, O.sc_matmul(a, b, gran, **kw))


@pytest.mark.parametrize("shape", [(6, 197, 64, 197), (4, 197, 197, 64), (3, 300, 20, 33)])
def test_per_head_vs_oracle(shape):
    from scmp_kernels_amd import sc_matmul
    BH, N, D, M = shape
    rng = np.random.default_rng(sum(shape))
    q = rng.standard_normal((BH, N, D)).astype(np.float32)
    k = rng.standard_normal((BH, M, D)).astype(np.float32)
    y = sc_matmul(T(q), T(k), "per_head")
    bits_equal(y, O.sc_matmul(q, k, "per_head"))


@pytest.mark.parametrize("D", [64, 66])
def test_quantize_pair_equals_two_calls(D):
    """scmp_quantize_pair against two scmp_quantize calls, bitwise (codes with their padding
    rows, per-row scales): per-head q (thermometer codes) and k (byte codes) of 600 heads of
    197 rows; D = 64 runs as one launch, D = 66 (rows not 16-byte aligned) as two calls."""
    from scmp_kernels_amd import _lib
    from scmp_kernels_amd.sc import kernels as K
    BH, N = 600, 197
    rng = np.random.default_rng(D)
    q = T(rng.standard_normal((BH * N, D)).astype(np.float32))
    k = T(rng.standard_normal((BH * N, D)).astype(np.float32) * 3)
    tabs = K._get_tables(None, 8, 256, 128, True, D, _dev())
    outs = []
    for paired in (False, True):
        ca, cb = K._codes(N, D, _dev(), batch=BH), K._codes(N, D, _dev(), batch=BH)
        ca.fill_(0x5A)
        cb.fill_(0xA5)
        sq = torch.full((BH * N,), -1.0, device=_dev())
        sk = torch.full((BH * N,), -1.0, device=_dev())
        first = (q, _lib.Q_HEAD_SYM, 127, 128,
                 dict(group=N, code=ca, code_kind=_lib.CODE_THERMO, code_batch_rows=N,
                      jtab=tabs.jtab, col_class=tabs.d_class, scale=sq))
        second = (k, _lib.Q_HEAD_SYM, 127, 128,
                  dict(group=N, code=cb, code_kind=_lib.CODE_Q, code_batch_rows=N, scale=sk))
        if paired:
            ws = K.quantize_pair(first, second)
        else:
            ws = (K.quantize(*first[:4], **first[4]), K.quantize(*second[:4], **second[4]))
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in (ca, cb, sq, sk)])
        del ws
    for x, y in zip(*outs):
        np.testing.assert_array_equal(x.view(np.uint8), y.view(np.uint8))


@pytest.mark.parametrize("shape", [(600, 197, 197, 64), (300, 96, 384, 96), (260, 40, 900, 40)])
def test_per_head_many_large_heads(shape):
    """More heads than compute units, heads of 64 to 155 KB of fp32 (P-like 197 x 197;
    rows of 96 or 225 four-column chunks; 4-aligned and ragged rows): sampled heads (first,
    last, middle, and those past the first 256 and 512) against the oracle."""
    from scmp_kernels_amd import sc_matmul
    BH, N, D, M = shape
    rng = np.random.default_rng(BH + N + D)
    q = rng.standard_normal((BH, N, D)).astype(np.float32)
    k = rng.standard_normal((BH, M, D)).astype(np.float32)
    y = sc_matmul(T(q), T(k), "per_head")
    heads = sorted({0, 1, BH // 2, BH - 2, BH - 1, 256, 257, 511 % BH})
    bits_equal(y[heads], O.sc_matmul(q[heads], k[heads], "per_head"))


@pytest.mark.parametrize("mode", ["bipolar", "unipolar"])
@pytest.mark.parametrize("N,M,D", [(65600, 48, 96), (66000, 17, 20)])
def test_narrow_tiles_more_than_compute_units(mode, N, M, D):
    """Outputs at most 64 wide in more 256 x 64 tiles than compute units (whole tiles per
    workgroup; D = 20 is three 8-d groups, the last one partial). Sampled rows of the first
    and last tiles and random rows against the oracle."""
    from scmp_kernels_amd import sc_matmul
    rng = np.random.default_rng(N + M + D)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = rng.standard_normal((M, D)).astype(np.float32)
    y = sc_matmul(T(a), T(b), "per_row", mode=mode)
    rows = np.unique(np.concatenate([np.arange(0, 256, 37), np.arange(N - 300, N, 41),
                                     rng.integers(0, N, 40)]))
    bits_equal(y[torch.from_numpy(rows).cuda()], O.sc_matmul(a[rows], b, "per_row", mode=mode))


def test_per_row_3d_wide_tiles_vs_oracle():
    """Batched operands whose per-batch output (300 x 500) takes 128 x 512 tiles."""
    from scmp_kernels_amd import sc_matmul
    rng = np.random.default_rng(12)
    a = rng.standard_normal((3, 300, 96)).astype(np.float32)
    b = rng.standard_normal((3, 500, 96)).astype(np.float32)
    for kw in (dict(mode="bipolar"), dict(mode="unipolar", stoc_len=64, rng_levels=64)):
        bits_equal(sc_matmul(T(a), T(b), "per_row", **kw), O.sc_matmul(a, b, "per_row", **kw))


def test_per_row_3d_vs_oracle():
    from scmp_kernels_amd import sc_matmul
    rng = np.random.default_rng(11)
    a = rng.standard_normal((5, 40, 64)).astype(np.float32)
    b = rng.standard_normal((5, 33, 64)).astype(np.float32)
    bits_equal(sc_matmul(T(a), T(b), "per_row"), O.sc_matmul(a, b, "per_row"))
    bits_equal(sc_matmul(T(a), T(b), "per_tensor"), O.sc_matmul(a, b, "per_tensor"))


# -------------------------------------------------------------------------------------
# per-d table classes in runs: both code buffers' columns rearranged class by class, one
# class table in LDS at a time (SCMP_FP4_RUNS=1 forces the layout where the padding rule
# would not choose it)
# -------------------------------------------------------------------------------------

RUNS_CASES = [
    # (N, M, D, L, R, bipolar)
    (257, 300, 777, 64, 64, False),      # split tiles, runs padded to whole groups
    (260, 270, 600, 128, 128, True),
    (70, 45, 96, 32, 32, True),
    (40, 31, 50, 16, 16, False),         # 16-interval tables (four d per k-step)
    (300, 200, 2048, 64, 64, True),
    (33, 97, 77, 64, 64, False),         # fewer d than classes
]


def _nclass(L, R, bipolar, D):
    from scmp_kernels_amd.sc import kernels as K
    return K._get_tables(None, 8, L, R, bipolar, D, _dev()).nclass


@pytest.mark.parametrize("case", RUNS_CASES)
def test_gemm_class_runs(case, monkeypatch):
    N, M, D, L, R, bip = case
    monkeypatch.setenv("SCMP_FP4_RUNS", "1")
    assert _nclass(L, R, bip, D) > 1
    rng = np.random.default_rng(N * 5 + M + D)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = rng.standard_normal((M, D)).astype(np.float32)
    a[1] = 0.0
    got = _int_accum_gpu(a, b, L=L, R=R, bipolar=bip, impl=2)
    np.testing.assert_array_equal(got, _int_accum_ref(a, b, L=L, R=R, bipolar=bip))


@pytest.mark.parametrize("kw,shape", [
    (dict(mode="unipolar", group_a=4, group_b=4, stoc_len=64, rng_levels=64), (300, 200, 1024)),
    (dict(mode="bipolar", stoc_len=64, rng_levels=64), (129, 260, 2048)),
])
def test_sc_matmul_class_runs_chosen(kw, shape, monkeypatch):
    """Shapes where the run layout is chosen by itself (64 classes of 64-interval tables,
    D a multiple of 512: no padding), against the oracle."""
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.sc import kernels as K
    monkeypatch.delenv("SCMP_FP4_RUNS", raising=False)
    N, M, D = shape
    tabs = K._get_tables(None, 8, 64, 64, kw["mode"] == "bipolar", D, _dev())
    assert K._fp4_class_runs(tabs, D) is not None
    rng = np.random.default_rng(N + 2 * M + D)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = (rng.standard_normal((M, D)) * 0.05).astype(np.float32)
    bits_equal(sc_matmul(T(a), T(b), "per_row", **kw), O.sc_matmul(a, b, "per_row", **kw))


@pytest.mark.parametrize("gran,kw,shape", [
    ("per_tensor", dict(mode="unipolar", stoc_len=64, rng_levels=64), (70, 90, 1024)),
    ("per_tensor", dict(mode="bipolar", stoc_len=64, rng_levels=64), (65, 40, 512)),
    ("per_row", dict(mode="unipolar", stoc_len=32, rng_levels=32, smooth=True), (50, 70, 520)),
])
def test_sc_matmul_class_runs_other_epilogues(gran, kw, shape, monkeypatch):
    """The run layout (forced) under the scalar and zero-point epilogues, whose correction
    terms use the true inner dimension, not the padded one the GEMM runs over."""
    from scmp_kernels_amd import sc_matmul
    monkeypatch.setenv("SCMP_FP4_RUNS", "1")
    N, M, D = shape
    rng = np.random.default_rng(N + M + D + 7)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = (rng.standard_normal((M, D)) * 0.05).astype(np.float32)
    kw = dict(kw)
    if kw.pop("smooth", False):
        kw["smooth_scales"] = rng.uniform(0.5, 2.0, D).astype(np.float32)
        y = sc_matmul(T(a), T(b), gran, **dict(kw, smooth_scales=T(kw["smooth_scales"])))
    else:
        y = sc_matmul(T(a), T(b), gran, **kw)
    bits_equal(y, O.sc_matmul(a, b, gran, **kw))


def test_class_runs_equal_global_tables_full_size(monkeypatch):
    """cfg5's L=64 level shape (1365 x 4096 x 4096, unipolar, groups of 4): the run layout
    and the per-d global-table path give the same bits."""
    from scmp_kernels_amd import sc_matmul
    dev = _dev()
    g = torch.Generator(device=dev).manual_seed(5)
    a = torch.randn((1365, 4096), device=dev, generator=g)
    b = torch.randn((4096, 4096), device=dev, generator=g) * 0.02
    kw = dict(mode="unipolar", group_a=4, group_b=4, stoc_len=64, rng_levels=64)
    monkeypatch.setenv("SCMP_FP4_RUNS", "0")
    ref = sc_matmul(a, b, "per_row", **kw)
    monkeypatch.delenv("SCMP_FP4_RUNS")
    got = sc_matmul(a, b, "per_row", **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32),
                                  ref.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("shape", [(6, 197, 64, 197), (3, 300, 136, 33)])
def test_per_head_class_runs_vs_oracle(shape, monkeypatch):
    """Batched codes (one buffer per head) through the run layout."""
    from scmp_kernels_amd import sc_matmul
    monkeypatch.setenv("SCMP_FP4_RUNS", "1")
    BH, N, D, M = shape
    rng = np.random.default_rng(sum(shape) + 1)
    q = rng.standard_normal((BH, N, D)).astype(np.float32)
    k = rng.standard_normal((BH, M, D)).astype(np.float32)
    kw = dict(stoc_len=64, rng_levels=64)
    bits_equal(sc_matmul(T(q), T(k), "per_head", **kw), O.sc_matmul(q, k, "per_head", **kw))


@pytest.mark.parametrize("rows,ld_in,ncols,ld_out", [(7, 4096, 4096, 4096), (1, 48, 40, 48),
                                                     (300, 20000, 19999, 20000),
                                                     (9, 100, 117, 128), (513, 16384, 16000,
                                                                          16016)])
def test_permute_code_columns(rows, ld_in, ncols, ld_out):
    """scmp_permute_code_columns against numpy: gathered columns, -1 entries and the columns
    past ncols zero (the three launch forms: 4 rows or 1 row per workgroup through LDS, and
    a row stride that is not a multiple of 16)."""
    from scmp_kernels_amd import _lib
    dev = _dev()
    rng = np.random.default_rng(rows + ld_in)
    x = rng.integers(0, 256, (rows, ld_in), dtype=np.uint8)
    src = rng.integers(0, ld_in, ncols).astype(np.int32)
    src[rng.random(ncols) < 0.1] = -1
    xin, s = T(x), torch.from_numpy(src).to(dev)
    out = torch.full((rows, ld_out), 0xAB, dtype=torch.uint8, device=dev)
    _lib.check(_lib.load().scmp_permute_code_columns(
        xin.data_ptr(), rows, ld_in, s.data_ptr(), ncols, out.data_ptr(), ld_out,
        _lib.stream_of(dev)), "scmp_permute_code_columns")
    ref = np.zeros((rows, ld_out), np.uint8)
    ref[:, :ncols] = np.where(src >= 0, x[:, np.clip(src, 0, None)], 0)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def test_chunk_d_full_rounds_and_tail():
    """chunk_d where 128 x 128 tiles fill the compute units 1.1 times (284 tiles on 256 CUs):
    rows of the full round (128 x 128 tiles) and of the tail (64 x 128 tiles, rows 8192 on)
    against the oracle, including the rows at the boundary and the last rows."""
    from scmp_kernels_amd import sc_matmul
    N, M, D = 9000, 500, 200
    rng = np.random.default_rng(9000)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = (rng.standard_normal((M, D)) * 0.05).astype(np.float32)
    y = sc_matmul(T(a), T(b), "per_row", mode="bipolar", chunk_d=48)
    rows = np.r_[0:40, 8150:8260, 8960:9000]
    ref = O.sc_matmul(a[rows], b, "per_row", mode="bipolar", chunk_d=48)
    bits_equal(y[torch.from_numpy(rows).to(y.device)], ref)


@pytest.mark.parametrize("N,L", [(18000, 256), (22384, 256), (18000, 32), (18000, 64)])
def test_chunk_d_tall_tiles_and_tail(N, L):
    """chunk_d with 256 x 128 tiles (128 x 64 per wave) in the full round: 64 of them per
    round at M = 500 cover rows 0-16383, and the rest run as 64 x 128 tiles (N = 18000) or
    128 x 128 tiles (N = 22384, whose 6000 remaining rows would take two rounds of 64-row
    tiles). L = 64: one table class per d of a chunk, read from global memory. Rows at the
    start, around the boundary and at the end against the oracle."""
    from scmp_kernels_amd import sc_matmul
    M, D = 500, 200
    rng = np.random.default_rng(N + L)
    a = rng.standard_normal((N, D)).astype(np.float32)
    b = (rng.standard_normal((M, D)) * 0.05).astype(np.float32)
    kw = dict(mode="bipolar", chunk_d=48, stoc_len=L, rng_levels=L)
    y = sc_matmul(T(a), T(b), "per_row", **kw)
    rows = np.r_[0:40, 16300:16460, N - 40:N]
    ref = O.sc_matmul(a[rows], b, "per_row", **kw)
    bits_equal(y[torch.from_numpy(rows).to(y.device)], ref)

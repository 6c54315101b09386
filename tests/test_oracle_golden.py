"""The CPU oracle against the golden vectors written by running the reference itself
(tests/golden/gen_golden.py, TRITON_INTERPRET=1). Bit-exact on every array."""
import json
import os

import numpy as np
import pytest

from oracle import sc_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLD, "cases.json")) as f:
    CASES = json.load(f)


def _load(name):
    with np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _ctx(env):
    return O.Ctx(owen_mode=env.get("SC_OWEN_MODE", "bitrev"),
                 scramble_rescale=env.get("SC_SCRAMBLE_RESCALE", "1") == "1")


MATMUL = sorted(k for k, v in CASES.items() if v["kind"] == "sc_matmul")
ACCUM = sorted(k for k, v in CASES.items() if v["kind"] == "accum")
QUANT = sorted(k for k, v in CASES.items() if v["kind"] == "quant")


@pytest.mark.parametrize("name", MATMUL)
def test_sc_matmul_golden(name):
    meta = CASES[name]
    z = _load(name)
    kw = dict(meta["kwargs"])
    gran = kw.pop("granularity")
    y = O.sc_matmul(z["a"], z["b"], gran, smooth_scales=z.get("smooth"), ctx=_ctx(meta["env"]),
                    **kw)
    assert y.dtype == np.float32 and y.shape == z["y"].shape
    np.testing.assert_array_equal(y.view(np.uint32), z["y"].view(np.uint32))


@pytest.mark.parametrize("name", ACCUM)
def test_accumulator_golden(name):
    meta = CASES[name]
    z = _load(name)
    L, R, D = meta["L"], meta["R"], meta["D"]
    cfg = O.make_sobol_simple_config(D, D, 8)
    tabs = O.Tables(cfg, 8, L, R)
    # tables: the oracle's (deduplicated) K / C rows equal every reference row
    K = tabs.K[tabs.tab_of]
    C = tabs.C[tabs.tab_of]
    np.testing.assert_array_equal(K, z["ktab"])
    np.testing.assert_array_equal(C, z["cum"])
    bip = meta["mode"] == "bipolar"
    I = O.sc_accum(z["beta_a"], z["sign_a"] if bip else None, z["beta_b"],
                   z["sign_b"] if bip else None, tabs)
    np.testing.assert_array_equal(I, z["I"].astype(np.int32))
    # and the table-free evaluation from the streams
    I2 = O.sc_accum_stream(z["beta_a"], z["sign_a"] if bip else None, z["beta_b"],
                           z["sign_b"] if bip else None, tabs.ra, tabs.rb)
    np.testing.assert_array_equal(I2, I)


def _eq(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype.kind == "f":
        np.testing.assert_array_equal(a.astype(b.dtype).view(np.uint8), b.view(np.uint8))
    else:
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("name", QUANT)
def test_quantizer_golden(name):
    meta = CASES[name]
    z = _load(name)
    fn = meta["fn"]
    x = z["x"]
    if fn == "fused_quantize_bipolar_perrow":
        beta, sign, scale = O.quant_fused_perrow_bipolar(x, 8, 256)
        _eq(beta, z["beta"]); _eq(sign, z["sign"]); _eq(scale, z["scale"])
    elif fn == "fused_quantize_bipolar":
        beta, sign, scale = O.quant_fused_bipolar(x, meta["abs_max"], 8, 256)
        _eq(beta, z["beta"]); _eq(sign, z["sign"]); assert scale == float(z["scale"])
    elif fn == "fused_quantize_unipolar":
        beta, scale, zp, rs = O.quant_fused_unipolar(x, float(x.max()), float(x.min()), 8,
                                                      meta["rng_levels"], meta["compute_sum"])
        _eq(beta, z["beta"])
        assert scale == float(z["scale"]) and zp == float(z["zp"])
        if meta["compute_sum"]:
            _eq(rs, z["row_sum"])
    elif fn == "_grouped_symmetric_quant":
        s, xi, sg = O.grouped_sym(x, meta["G"], meta["q_max"])
        _eq(s, z["scale"]); _eq(xi, z["x_int"]); _eq(sg, z["sign"])
    elif fn == "_grouped_asymmetric_quant":
        s, zp, xi = O.grouped_asym(x, meta["G"], meta["q_max"])
        _eq(s, z["scale"]); _eq(zp, z["zp"]); _eq(xi, z["x_int"])
    elif fn == "_grouped_symmetric_quant_batched":
        s, xi, sg = O.grouped_sym_batched(x, meta["G"], meta["q_max"])
        _eq(s, z["scale"]); _eq(xi, z["x_int"]); _eq(sg, z["sign"])
    else:
        raise AssertionError(fn)

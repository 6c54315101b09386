"""Parity at the BASELINE configurations' full sizes. The whole product call runs on the
GPU at full shape; the oracle recomputes a seeded sample of independent pieces (rows of
a for the row-local paths, whole quantization groups for grouped paths, whole heads for
per_head), which it finishes in seconds. Every sampled value must match bit for bit;
repeated calls must be identical.

Inputs come from bench.py's seeded generators, so these are the benchmark's own
operands."""
import numpy as np
import pytest
import torch

import bench
from oracle import sc_oracle as O

pytestmark = pytest.mark.gpu

CTX = O.Ctx(nthreads=8)


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _bits_equal(got: np.ndarray, ref: np.ndarray, what: str):
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    bad = got.view(np.uint32) != ref.view(np.uint32)
    n = int(bad.sum())
    assert n == 0, f"{what}: {n} of {bad.size} values differ, first at {np.argwhere(bad)[0]}"


def _sample_rows(n, k, seed):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, n - 1], rng.choice(n, size=k - 2, replace=False)]))
    return rows


def test_cfg2_llm_per_row_smoothquant():
    """4096 x 11008 x 4096 per_row bipolar with SmoothQuant (the benchmark call)."""
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.quant import accumulate_act_scales, compute_smooth_scales
    a_h, b_h = bench.make_cfg2()
    a, b = _dev(a_h), _dev(b_h)
    s = compute_smooth_scales(accumulate_act_scales(a), b, alpha=0.5)
    y = sc_matmul(a, b, "per_row", sc_prec=8, stoc_len=256, smooth_scales=s)
    y2 = sc_matmul(a, b, "per_row", sc_prec=8, stoc_len=256, smooth_scales=s)
    assert torch.equal(y, y2)
    rows = _sample_rows(4096, 48, 20)
    ref = O.sc_matmul(a_h[rows], b_h, "per_row", sc_prec=8, stoc_len=256,
                      smooth_scales=s.cpu().numpy(), ctx=CTX)
    _bits_equal(y[torch.from_numpy(rows).cuda()].cpu().numpy(), ref, "cfg2 rows")


def test_cfg3_vit_mlp_chunk_d():
    """12608 x 768 x 3072 per_row bipolar, chunk_d = 72 (42 chunks of 72 + one of 48)."""
    from scmp_kernels_amd import sc_matmul
    a_h, b_h = bench.make_cfg3()
    a, b = _dev(a_h), _dev(b_h)
    y = sc_matmul(a, b, "per_row", sc_prec=8, chunk_d=72, group_a=1, group_b=1)
    rows = _sample_rows(a_h.shape[0], 64, 21)
    ref = O.sc_matmul(a_h[rows], b_h, "per_row", sc_prec=8, chunk_d=72, ctx=CTX)
    _bits_equal(y[torch.from_numpy(rows).cuda()].cpu().numpy(), ref, "cfg3 rows")


def test_cfg4_attention_per_head():
    """ViT-B attention at BH = 768: QK^T (197 x 197 x 64) and P.V (197 x 64 x 197)."""
    from scmp_kernels_amd import sc_matmul
    q_h, k_h, p_h, vt_h = bench.make_cfg4()
    heads = _sample_rows(768, 6, 22)
    hd = torch.from_numpy(heads).cuda()
    y_qk = sc_matmul(_dev(q_h), _dev(k_h), "per_head", sc_prec=8)
    assert tuple(y_qk.shape) == (768, 197, 197)
    ref = O.sc_matmul(q_h[heads], k_h[heads], "per_head", sc_prec=8, ctx=CTX)
    _bits_equal(y_qk[hd].cpu().numpy(), ref, "cfg4 QK heads")
    y_pv = sc_matmul(_dev(p_h), _dev(vt_h), "per_head", sc_prec=8)
    assert tuple(y_pv.shape) == (768, 197, 64)
    ref = O.sc_matmul(p_h[heads], vt_h[heads], "per_head", sc_prec=8, ctx=CTX)
    _bits_equal(y_pv[hd].cpu().numpy(), ref, "cfg4 PV heads")


def test_cfg5_mixed_level_unipolar_grouped():
    """4096 x 4096 x 4096 unipolar, groups of 4 rows, per-row levels {256, 64, 16} from
    classify_rows_by_metric on the row range (equal fractions, descending-metric order
    inside a level), through the benchmarked call sc_matmul_mixed. Sampled: whole groups of
    4 rows at the start, middle and end of every level (a level's row groups follow its row
    order), checked against the oracle's sc_matmul of those rows at the level's length."""
    from scmp_kernels_amd.mp import classify_rows_by_metric, sc_matmul_mixed
    a_h, b_h = bench.make_cfg5()
    a, b = _dev(a_h), _dev(b_h)
    metric = (a.amax(dim=1) - a.amin(dim=1))
    ra = classify_rows_by_metric(metric, bench.CFG5_LEVELS, [1 / 3] * 3)
    Y = sc_matmul_mixed(a, b, ra, mode="unipolar", group_a=4, group_b=4)
    assert torch.equal(Y, sc_matmul_mixed(a, b, ra, mode="unipolar", group_a=4, group_b=4))
    for L in bench.CFG5_LEVELS:
        rows_h = ra.level_row_indices[L].cpu().numpy()
        ngroups = (len(rows_h) + 3) // 4
        for g in (0, ngroups // 2, ngroups - 1):
            sel = rows_h[4 * g:4 * g + 4]
            ref = O.sc_matmul(a_h[sel], b_h, "per_row", mode="unipolar", group_a=4, group_b=4,
                              stoc_len=L, rng_levels=L, ctx=CTX)
            _bits_equal(Y[torch.from_numpy(sel).cuda()].cpu().numpy(), ref,
                        f"cfg5 level {L} group {g}")


def test_cfg2_prepared_weight_smoothquant():
    """The weight-side cache at cfg2: prepare_weight(b, smooth_scales=s) once, then
    sc_matmul(a, w, ...) on sampled rows against the oracle's plain call (b * s folded into
    the weight quantizer's load, a / s into the activation quantizer's)."""
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.quant import accumulate_act_scales, compute_smooth_scales
    from scmp_kernels_amd.sc import prepare_weight
    a_h, b_h = bench.make_cfg2()
    a, b = _dev(a_h), _dev(b_h)
    s = compute_smooth_scales(accumulate_act_scales(a), b, alpha=0.5)
    w = prepare_weight(b, mode="bipolar", sc_prec=8, smooth_scales=s)
    del b
    y = sc_matmul(a, w, "per_row", sc_prec=8, stoc_len=256, smooth_scales=s)
    rows = _sample_rows(4096, 24, 23)
    ref = O.sc_matmul(a_h[rows], b_h, "per_row", sc_prec=8, stoc_len=256,
                      smooth_scales=s.cpu().numpy(), ctx=CTX)
    _bits_equal(y[torch.from_numpy(rows).cuda()].cpu().numpy(), ref, "cfg2 prepared rows")

"""Prepared weights and the mixed-level per_row dispatch on the GPU: bit-identical to the
plain sc_matmul calls they replace (which are themselves checked against the oracle in
test_gpu_parity.py), and against the oracle directly for one mixed case."""
import os

import numpy as np
import pytest
import torch

from oracle import sc_oracle as O

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda", 0)


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def _data(N, M, D, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((N, D)).astype(np.float32)
    a[rng.choice(N, max(1, N // 20), replace=False)] *= 6.0
    b = (rng.standard_normal((M, D)) * 0.02).astype(np.float32)
    s = rng.uniform(0.5, 2.0, D).astype(np.float32)
    return a, b, s


@pytest.mark.parametrize("mode,group_b,smooth", [("bipolar", 1, False), ("bipolar", 1, True),
                                                 ("unipolar", 4, False), ("unipolar", 1, True)])
def test_prepared_weight_equals_plain_call(mode, group_b, smooth):
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.sc import prepare_weight
    dev = _dev()
    a_h, b_h, s_h = _data(300, 200, 256, 1)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    s = torch.from_numpy(s_h).to(dev) if smooth else None
    w = prepare_weight(b, mode=mode, sc_prec=8, group_b=group_b, smooth_scales=s)
    for L in (256, 64, 16):
        kw = dict(mode=mode, sc_prec=8, group_a=2, group_b=group_b, stoc_len=L, rng_levels=L,
                  smooth_scales=s)
        ref = sc_matmul(a, b, "per_row", **kw)
        got = sc_matmul(a, w, "per_row", **kw)
        np.testing.assert_array_equal(_bits(got), _bits(ref))


def test_prepared_weight_rejects_mismatch():
    from scmp_kernels_amd import sc_matmul
    from scmp_kernels_amd.sc import prepare_weight
    dev = _dev()
    a_h, b_h, s_h = _data(40, 30, 64, 2)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    s = torch.from_numpy(s_h).to(dev)
    w = prepare_weight(b, mode="bipolar", smooth_scales=s)
    with pytest.raises(ValueError, match="prepared"):
        sc_matmul(a, w, "per_row", mode="unipolar", smooth_scales=s)
    with pytest.raises(ValueError, match="smooth_scales"):
        sc_matmul(a, w, "per_row")
    with pytest.raises(ValueError, match="smooth_scales differ"):
        sc_matmul(a, w, "per_row", smooth_scales=s * 2)
    with pytest.raises(ValueError, match="per_row"):
        sc_matmul(a, w, "per_tensor", smooth_scales=s)
    with pytest.raises(ValueError, match="per_row"):
        sc_matmul(a, w, "per_row", chunk_d=32, smooth_scales=s)
    # the same values in another tensor are accepted
    np.testing.assert_array_equal(_bits(sc_matmul(a, w, "per_row", smooth_scales=s.clone())),
                                  _bits(sc_matmul(a, b, "per_row", smooth_scales=s)))


def _loop(a, b, ra, **kw):
    """The reference caller's loop: one sc_matmul per level on the gathered rows."""
    from scmp_kernels_amd import sc_matmul
    y = torch.zeros((a.shape[0], b.shape[0]), dtype=torch.float32, device=a.device)
    for L, rows in ra.level_row_indices.items():
        if rows.numel() and L > 0:
            y[rows] = sc_matmul(a[rows], b, "per_row", stoc_len=L, rng_levels=L, **kw)
    return y


@pytest.mark.parametrize("mode,ga,gb", [("unipolar", 4, 4), ("bipolar", 1, 1),
                                        ("bipolar", 3, 2)])
def test_mixed_equals_per_level_loop(mode, ga, gb):
    from scmp_kernels_amd.mp import classify_rows_by_metric, sc_matmul_mixed
    from scmp_kernels_amd.sc import prepare_weight
    dev = _dev()
    a_h, b_h, _ = _data(517, 260, 192, 3)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    metric = a.amax(dim=1) - a.amin(dim=1)
    ra = classify_rows_by_metric(metric, [256, 64, 16], [1 / 3] * 3)
    kw = dict(mode=mode, sc_prec=8, group_a=ga, group_b=gb)
    ref = _loop(a, b, ra, **kw)
    got = sc_matmul_mixed(a, b, ra, **kw)
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    w = prepare_weight(b, mode=mode, group_b=gb)
    np.testing.assert_array_equal(_bits(sc_matmul_mixed(a, w, ra, **kw)), _bits(ref))


@pytest.mark.parametrize("impl", ["int8", "valu"])
def test_mixed_row_map_other_kernels(impl, monkeypatch):
    """The row map of the int8 MFMA and VALU kernels (and the int8 in-place epilogue)."""
    from scmp_kernels_amd.mp import classify_rows_by_metric, sc_matmul_mixed
    dev = _dev()
    a_h, b_h, _ = _data(300, 130, 96, 4)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    ra = classify_rows_by_metric(a.abs().amax(dim=1), [256, 64], [0.5, 0.5])
    kw = dict(mode="bipolar", sc_prec=8)
    monkeypatch.setenv("SCMP_GEMM_IMPL", impl)
    ref = _loop(a, b, ra, **kw)
    got = sc_matmul_mixed(a, b, ra, **kw)
    np.testing.assert_array_equal(_bits(got), _bits(ref))


def test_mixed_pruned_level_and_oracle():
    from scmp_kernels_amd.mp import AdaptiveMPConfig, adaptive_classify_rows, sc_matmul_mixed
    dev = _dev()
    a_h, b_h, _ = _data(120, 70, 64, 5)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    cfg = AdaptiveMPConfig([256, 64, 0], target_fractions=[0.5, 0.3, 0.2])
    ra = adaptive_classify_rows(a.abs().amax(dim=1), cfg)
    got = sc_matmul_mixed(a, b, ra, mode="unipolar", group_a=1, group_b=1)
    pruned = ra.level_row_indices[0].cpu().numpy()
    assert len(pruned) > 0 and not got[ra.level_row_indices[0]].any()
    for L in (256, 64):
        rows = ra.level_row_indices[L].cpu().numpy()
        ref = O.sc_matmul(a_h[rows], b_h, "per_row", mode="unipolar", sc_prec=8, stoc_len=L,
                          rng_levels=L)
        np.testing.assert_array_equal(got.cpu().numpy()[rows].view(np.uint32),
                                      ref.view(np.uint32))


def test_mixed_rejects_bad_rows():
    from scmp_kernels_amd.mp import RowAssignment, sc_matmul_mixed
    dev = _dev()
    a_h, b_h, _ = _data(10, 8, 32, 6)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    ra = RowAssignment(row_levels=torch.zeros(10, dtype=torch.long),
                       level_row_indices={256: torch.tensor([0, 3, 10])})
    with pytest.raises(ValueError, match="row indices"):
        sc_matmul_mixed(a, b, ra)


def test_mixed_rejects_repeated_rows_and_zero_fills_missing():
    """A row in two places is rejected (it would be written twice with different values);
    rows that no level names are zero, also when the index count equals N."""
    from scmp_kernels_amd.mp import RowAssignment, sc_matmul_mixed
    dev = _dev()
    a_h, b_h, _ = _data(12, 9, 64, 7)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    lv = torch.zeros(12, dtype=torch.long)
    dup = RowAssignment(row_levels=lv, level_row_indices={
        256: torch.tensor([0, 1, 2, 3, 4, 5]), 64: torch.tensor([6, 7, 8, 9, 10, 5])})
    with pytest.raises(ValueError, match="more than once"):
        sc_matmul_mixed(a, b, dup, mode="bipolar")
    dup1 = RowAssignment(row_levels=lv, level_row_indices={
        256: torch.tensor([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 10])})
    with pytest.raises(ValueError, match="more than once"):
        sc_matmul_mixed(a, b, dup1, mode="bipolar")
    part = RowAssignment(row_levels=lv, level_row_indices={
        256: torch.tensor([0, 2, 4, 6]), 64: torch.tensor([1, 3, 5])})
    y = sc_matmul_mixed(a, b, part, mode="bipolar")
    assert not y[7:].any()
    for L, rows in part.level_row_indices.items():
        r = rows.numpy()
        ref = O.sc_matmul(a_h[r], b_h, "per_row", mode="bipolar", sc_prec=8, stoc_len=L,
                          rng_levels=L)
        np.testing.assert_array_equal(y.cpu().numpy()[r].view(np.uint32), ref.view(np.uint32))


def test_mixed_row_check_syncs_once_per_assignment():
    """The row validation's host sync runs on the first call with an assignment; a second
    call with the same index tensors issues no synchronizing operation, and an in-place
    change of an index tensor makes the next call check (and sync) again."""
    from scmp_kernels_amd.mp import classify_rows_by_metric, sc_matmul_mixed
    dev = _dev()
    a_h, b_h, _ = _data(260, 130, 96, 8)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    ra = classify_rows_by_metric(a.abs().amax(dim=1), [256, 64], [0.5, 0.5])
    y1 = sc_matmul_mixed(a, b, ra, mode="bipolar")
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        y2 = sc_matmul_mixed(a, b, ra, mode="bipolar")
    finally:
        torch.cuda.set_sync_debug_mode(0)
    np.testing.assert_array_equal(_bits(y2), _bits(y1))
    rows = ra.level_row_indices[64]
    rows.copy_(rows.flip(0))                     # same rows, new order: version bumped
    torch.cuda.set_sync_debug_mode("error")
    try:
        with pytest.raises(RuntimeError):
            sc_matmul_mixed(a, b, ra, mode="bipolar")
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    y3 = sc_matmul_mixed(a, b, ra, mode="bipolar")
    ref = _loop(a, b, ra, mode="bipolar", sc_prec=8)
    np.testing.assert_array_equal(_bits(y3), _bits(ref))

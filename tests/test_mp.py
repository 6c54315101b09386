"""Mixed-precision row assignment (scmp_kernels/mp/config.py:42-191): slice sizes,
descending-metric order inside each level, clamping, and MPConfig validation; the
product classifier is checked against the oracle's restatement and a brute-force
definition."""
import numpy as np
import pytest
import torch

from oracle import sc_oracle as O
from scmp_kernels_amd.mp import MPConfig, classify_rows_by_metric


@pytest.mark.parametrize("N,levels,fracs", [
    (4096, [256, 64, 16], [1 / 3] * 3),
    (10, [256, 128, 64, 32], [0.25] * 4),
    (7, [256, 64], [0.9, 0.1]),
    (3, [256, 128, 64, 32, 16], [0.3, 0.3, 0.3, 0.05, 0.05]),
    (1, [256, 16], [0.5, 0.5]),
])
def test_classify_matches_oracle_and_definition(N, levels, fracs):
    metric = np.random.default_rng(N).standard_normal(N).astype(np.float32)
    ra = classify_rows_by_metric(torch.from_numpy(metric), levels, fracs)
    lv_ref, rows_ref = O.classify_rows_by_metric(metric, levels, fracs)
    np.testing.assert_array_equal(ra.row_levels.numpy(), lv_ref)
    order = np.argsort(-metric, kind="stable")
    seen = 0
    for i, L in enumerate(levels):
        rows = ra.level_row_indices[L].numpy()
        np.testing.assert_array_equal(rows, rows_ref[L])
        # consecutive slice of the descending ranking
        np.testing.assert_array_equal(rows, order[seen:seen + len(rows)])
        want = N - seen if i == len(levels) - 1 else min(max(round(fracs[i] * N), 0), N - seen)
        assert len(rows) == want
        seen += len(rows)
    assert seen == N


def test_mpconfig_defaults_and_errors():
    cfg = MPConfig([256, 64, 16])
    assert cfg.level_fractions == [1 / 3] * 3
    with pytest.raises(ValueError, match="length"):
        MPConfig([256, 64], [1.0])
    with pytest.raises(ValueError, match="sum to 1.0"):
        MPConfig([256, 64], [0.5, 0.6])


# -------------------------------------------------------------------------------------
# adaptive / free-boundary / range classifiers (scmp_kernels/mp/config.py:199-1007):
# known answers worked out by hand on small metrics
# -------------------------------------------------------------------------------------

from scmp_kernels_amd.mp import (AdaptiveMPConfig, FreeBoundaryMPConfig, RangeMPConfig,  # noqa: E402
                                 adaptive_classify_rows, classify_groups_by_range,
                                 get_current_block_idx, set_current_block_idx)
import json  # noqa: E402

# metric normalized: (m - 1) / 8 -> [0, 0.125, 0.25, 0.375, 0.5, 0.625, 0.75, 0.875, 1.0]
_M = torch.tensor([5.0, 1.0, 9.0, 3.0, 7.0, 2.0, 8.0, 4.0, 6.0])


def _levels(ra, levels):
    return {L: ra.level_row_indices[L].tolist() for L in levels}


def test_adaptive_calibrated_thresholds(tmp_path):
    table = {"stoc_len_levels": [256, 64, 16], "timestep_buckets": 2, "layer_buckets": 2,
             "operator_defaults": {"qk": [0.7, 0.3]},
             "buckets": {"qk:t1:l0": {"thresholds": [0.9, 0.1]}}}
    p = tmp_path / "table.json"
    p.write_text(json.dumps(table))
    cfg = AdaptiveMPConfig([256, 64, 16], threshold_table_path=str(p))
    # operator default: >= 0.7 -> 256; [0.3, 0.7) -> 64; below -> 16
    ra = adaptive_classify_rows(_M, cfg, operator="qk")
    assert _levels(ra, [256, 64, 16]) == {256: [2, 4, 6], 64: [0, 7, 8], 16: [1, 3, 5]}
    assert ra.row_levels.tolist() == [1, 2, 0, 2, 0, 2, 0, 1, 1]
    # bucket (t=1, l=0): timestep 9 of 10 -> bucket 1; block 0 of 4 -> bucket 0
    ra = adaptive_classify_rows(_M, cfg, operator="qk", block_idx=0, total_blocks=4,
                                timestep=9, total_timesteps=10)
    assert _levels(ra, [256, 64, 16]) == {256: [2], 64: [0, 3, 4, 5, 6, 7, 8], 16: [1]}
    with pytest.raises(ValueError, match="no classification path"):
        adaptive_classify_rows(_M, cfg, operator="mlp")
    # constant metric: every row at the first level
    ra = adaptive_classify_rows(torch.ones(4), cfg, operator="qk")
    assert _levels(ra, [256, 64, 16]) == {256: [0, 1, 2, 3], 64: [], 16: []}


def test_adaptive_table_validation(tmp_path):
    def load(payload):
        p = tmp_path / "t.json"
        p.write_text(json.dumps(payload))
        return AdaptiveMPConfig([256, 64], threshold_table_path=str(p))
    with pytest.raises(ValueError, match="do not match"):
        load({"stoc_len_levels": [256, 32]})
    with pytest.raises(ValueError, match="length 2, expected 1"):
        load({"stoc_len_levels": [256, 64], "operator_defaults": {"qk": [0.5, 0.2]}})
    with pytest.raises(ValueError, match="outside"):
        load({"stoc_len_levels": [256, 64], "operator_defaults": {"qk": [1.5]}})
    with pytest.raises(ValueError, match="Invalid adaptive MP bucket key"):
        load({"stoc_len_levels": [256, 64], "buckets": {"qk:3:l0": [0.5]}})
    with pytest.raises(ValueError, match="non-increasing"):
        AdaptiveMPConfig([256, 64, 16], operator_default_thresholds={})  # valid
        p = tmp_path / "u.json"
        p.write_text(json.dumps({"stoc_len_levels": [256, 64, 16],
                                 "operator_defaults": {"qk": [0.3, 0.6]}}))
        AdaptiveMPConfig([256, 64, 16], threshold_table_path=str(p))
    with pytest.raises(AssertionError):
        AdaptiveMPConfig([64, 256])
    assert AdaptiveMPConfig([256, 64, 0], enable_pruning=False).stoc_len_levels == [256, 64]


def test_adaptive_quantile_path():
    cfg = AdaptiveMPConfig([256, 64, 16], target_fractions=[1 / 3, 1 / 3, 1 / 3])
    ra = adaptive_classify_rows(_M, cfg)
    # descending metric order: rows 2, 6, 4 | 8, 0, 7 | 3, 5, 1
    assert _levels(ra, [256, 64, 16]) == {256: [2, 6, 4], 64: [8, 0, 7], 16: [3, 5, 1]}


def test_free_boundaries_and_fixed_levels():
    cfg = FreeBoundaryMPConfig([256, 64, 16])
    set_current_block_idx(3)
    assert get_current_block_idx() == 3
    # default boundaries (2/3, 1/3): >= 2/3 -> 256, [1/3, 2/3) -> 64, below -> 16
    ra = adaptive_classify_rows(_M, cfg, operator="proj")
    assert _levels(ra, [256, 64, 16]) == {256: [2, 4, 6], 64: [0, 7, 8], 16: [1, 3, 5]}
    cfg.set_boundaries("proj", 3, torch.tensor([0.2, 0.8]))      # re-sorted descending
    ra = adaptive_classify_rows(_M, cfg, operator="proj")
    assert _levels(ra, [256, 64, 16]) == {256: [2, 6], 64: [0, 3, 4, 7, 8], 16: [1, 5]}
    cfg.set_fixed_level("proj", 3, 1)
    ra = adaptive_classify_rows(_M, cfg, operator="proj")
    assert _levels(ra, [256, 64, 16]) == {256: [], 64: list(range(9)), 16: []}
    cfg.clear_fixed_level("proj", 3)          # set_fixed_level dropped the boundaries
    assert adaptive_classify_rows(_M, cfg, operator="proj").row_levels.tolist() == \
        [1, 2, 0, 2, 0, 2, 0, 1, 1]
    set_current_block_idx(0)
    with pytest.raises(AssertionError):
        FreeBoundaryMPConfig([256, 64], boundaries={(0, "qk"): [0.5, 0.2]})


def test_classify_groups_by_range(capsys):
    # 4 groups of 2 rows; ranges 1, 4, 7, 10 -> normalized 0, 1/3, 2/3, 1
    w = torch.zeros(8, 3)
    for g, r in enumerate([1.0, 4.0, 7.0, 10.0]):
        w[2 * g, 0] = r
    cfg = RangeMPConfig([256, 64, 16], base_threshold=0.5)
    # boundaries 0.5 and 0.25: >= 0.5 -> 256, [0.25, 0.5) -> 64, below -> 16
    assert classify_groups_by_range(w, 2, cfg, operator="fc1") == [16, 64, 256, 256]
    assert "[RangeMP] fc1: groups=4" in capsys.readouterr().out
    cfg.operator_thresholds["fc2"] = 0.99                      # capped at 0.95
    assert classify_groups_by_range(w, 2, cfg, operator="fc2") == [16, 16, 64, 256]
    # one per-tensor group: its normalized range is 0, the lowest level
    assert classify_groups_by_range(w, 0, cfg) == [16]


def test_mixed_row_check():
    """sc_matmul_mixed's row validation (host logic on index tensors): bounds, repeats,
    exact coverage."""
    from scmp_kernels_amd.mp.dispatch import _check_rows
    t = torch.tensor
    assert _check_rows([t([0, 2, 4]), t([1, 3])], 5) is True
    assert _check_rows([t([0, 2, 4]), t([1])], 5) is False
    assert _check_rows([], 0) is True and _check_rows([], 3) is False
    with pytest.raises(ValueError, match="more than once"):
        _check_rows([t([0, 1, 2, 3]), t([3])], 5)      # duplicated 3 and missing 4
    with pytest.raises(ValueError, match="more than once"):
        _check_rows([t([0, 0])], 1)
    with pytest.raises(ValueError, match=r"\[0, 5\)"):
        _check_rows([t([0, 5])], 5)
    with pytest.raises(ValueError, match=r"\[0, 5\)"):
        _check_rows([t([-1, 2])], 5)

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

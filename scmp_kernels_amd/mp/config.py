"""Per-row stoc_len level assignment (scmp_kernels/mp/config.py:42-191).

Rows are ranked by an importance metric; the top fraction gets the longest stream.
Callers then run one ``sc_matmul(a[rows_L], b, ..., stoc_len=L, rng_levels=L)`` per
level and scatter the results back (the reference's mixed-precision harness).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class MPConfig:
    """Configuration for per-token-row mixed-precision SC (mp/config.py:42-62)."""
    stoc_len_levels: list
    level_fractions: Optional[list] = None
    qk_metric: str = "q_row_max"
    av_metric: str = "attn_row_max"
    mlp_metric: str = "x_row_max"

    def __post_init__(self):
        if self.level_fractions is None:
            n = len(self.stoc_len_levels)
            self.level_fractions = [1.0 / n] * n
        if len(self.level_fractions) != len(self.stoc_len_levels):
            raise ValueError(
                f"level_fractions length ({len(self.level_fractions)}) must match "
                f"stoc_len_levels length ({len(self.stoc_len_levels)})")
        if abs(sum(self.level_fractions) - 1.0) >= 1e-6:
            raise ValueError(
                f"level_fractions must sum to 1.0, got {sum(self.level_fractions)}")


@dataclass
class RowAssignment:
    """Row-to-level assignment (mp/config.py:66-69)."""
    row_levels: torch.Tensor
    level_row_indices: dict


def classify_rows_by_metric(metric: torch.Tensor, stoc_len_levels: list,
                            level_fractions: list) -> RowAssignment:
    """Rank rows by metric (descending); level i takes round(frac_i * N) rows, the last
    level the rest, clamped to the rows left (mp/config.py:154-191). Rows of each level
    are returned in descending-metric order."""
    N = metric.shape[0]
    sorted_indices = metric.argsort(descending=True)
    row_levels = torch.empty(N, dtype=torch.long, device=metric.device)
    level_row_indices = {}
    offset = 0
    for i, (sl, frac) in enumerate(zip(stoc_len_levels, level_fractions)):
        if i < len(stoc_len_levels) - 1:
            count = round(frac * N)
        else:
            count = N - offset
        count = max(0, min(count, N - offset))
        rows = sorted_indices[offset:offset + count]
        row_levels[rows] = i
        level_row_indices[sl] = rows
        offset += count
    return RowAssignment(row_levels=row_levels, level_row_indices=level_row_indices)

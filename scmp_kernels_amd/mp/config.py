"""Per-row stream-length level assignment (the call surface of the reference's
scmp_kernels/mp/config.py:42-191).

Rows are ranked by an importance metric and cut into consecutive slices, the most
important slice getting the longest stream. A caller then runs one
``sc_matmul(a[rows_L], b, ..., stoc_len=L, rng_levels=L)`` per level and scatters the
results back into ``Y[rows_L]``.
"""
from __future__ import annotations

from dataclasses import dataclass
from itertools import accumulate
from typing import Optional

import torch


@dataclass
class MPConfig:
    """Stream-length levels (longest first) and the fraction of rows each receives;
    equal fractions when omitted (scmp_kernels/mp/config.py:42-62)."""
    stoc_len_levels: list
    level_fractions: Optional[list] = None
    qk_metric: str = "q_row_max"
    av_metric: str = "attn_row_max"
    mlp_metric: str = "x_row_max"

    def __post_init__(self):
        levels = len(self.stoc_len_levels)
        if self.level_fractions is None:
            self.level_fractions = [1.0 / levels for _ in range(levels)]
        nfrac = len(self.level_fractions)
        if nfrac != levels:
            raise ValueError(
                f"level_fractions length ({nfrac}) must match "
                f"stoc_len_levels length ({levels})")
        total = sum(self.level_fractions)
        if not abs(total - 1.0) < 1e-6:
            raise ValueError(f"level_fractions must sum to 1.0, got {total}")


@dataclass
class RowAssignment:
    """``row_levels[n]``: level index of row n; ``level_row_indices[L]``: the rows at
    stream length L, most important first (scmp_kernels/mp/config.py:66-69)."""
    row_levels: torch.Tensor
    level_row_indices: dict


def _slice_sizes(nrows: int, nlevels: int, fractions: list) -> list:
    """Rows per level: round(fraction * nrows) for every level but the last, which takes
    what is left; each size is clamped to the rows still unassigned."""
    sizes = []
    left = nrows
    for i, frac in enumerate(fractions[:nlevels]):
        want = left if i == nlevels - 1 else round(frac * nrows)
        take = min(max(want, 0), left)
        sizes.append(take)
        left -= take
    return sizes


def classify_rows_by_metric(metric: torch.Tensor, stoc_len_levels: list,
                            level_fractions: list) -> RowAssignment:
    """Rank rows by ``metric`` (descending) and hand consecutive slices of the ranking to
    the levels in order (scmp_kernels/mp/config.py:154-191)."""
    nrows = metric.shape[0]
    ranking = metric.argsort(descending=True)
    sizes = _slice_sizes(nrows, len(stoc_len_levels), list(level_fractions))
    edges = [0, *accumulate(sizes)]
    row_levels = torch.empty(nrows, dtype=torch.long, device=metric.device)
    level_row_indices = {}
    for lvl, (stoc_len, lo, hi) in enumerate(zip(stoc_len_levels, edges[:-1], edges[1:])):
        rows = ranking[lo:hi]
        row_levels[rows] = lvl
        level_row_indices[stoc_len] = rows
    return RowAssignment(row_levels=row_levels, level_row_indices=level_row_indices)

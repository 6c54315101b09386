"""Per-row stream-length level assignment (the call surface of the reference's
scmp_kernels/mp/config.py: fixed-fraction, adaptive / calibrated-threshold, free-boundary
and weight-range classifiers; the loggers and the auto-calibrator are not part of it).

Rows are ranked by an importance metric and cut into consecutive slices, the most
important slice getting the longest stream. A caller then runs one
``sc_matmul(a[rows_L], b, ..., stoc_len=L, rng_levels=L)`` per level and scatters the
results back into ``Y[rows_L]``.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from itertools import accumulate
from pathlib import Path
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


# -------------------------------------------------------------------------------------
# Current block (scmp_kernels/mp/config.py:28-39): classifiers keyed by (block, operator)
# read it when the caller gives no block index.
# -------------------------------------------------------------------------------------

_CURRENT_BLOCK_IDX: int = 0


def set_current_block_idx(i: int) -> None:
    global _CURRENT_BLOCK_IDX
    _CURRENT_BLOCK_IDX = int(i)


def get_current_block_idx() -> int:
    return _CURRENT_BLOCK_IDX


def _bucket_index(value: int, total: int, num_buckets: int) -> int:
    """Calibration bucket of a timestep / block index (mp/config.py:72-77)."""
    if num_buckets <= 1 or total <= 1:
        return 0
    return min(num_buckets - 1, int(value / max(total - 1, 1) * num_buckets))


def _parse_bucket_key(bucket_key: str) -> tuple:
    """'<operator>:t<int>:l<int>' -> (operator, t, l) (mp/config.py:80-91)."""
    parts = bucket_key.split(":")
    if (len(parts) != 3 or not parts[1].startswith("t") or not parts[2].startswith("l")
            or not parts[1][1:].lstrip("-").isdigit() or not parts[2][1:].lstrip("-").isdigit()):
        raise ValueError(f"Invalid adaptive MP bucket key '{bucket_key}'. "
                         "Expected format '<operator>:t<int>:l<int>'.")
    return parts[0], int(parts[1][1:]), int(parts[2][1:])


def _extract_thresholds(payload, n_levels: int, source: str) -> list:
    """A validated, non-increasing threshold list of length n_levels - 1 in [0, 1]
    (mp/config.py:94-116)."""
    raw = payload.get("thresholds") if isinstance(payload, dict) else payload
    if raw is None:
        raise ValueError(f"Missing 'thresholds' in adaptive MP payload for {source}.")
    th = [float(x) for x in raw]
    want = max(n_levels - 1, 0)
    if len(th) != want:
        raise ValueError(f"Adaptive MP thresholds for {source} have length {len(th)}, "
                         f"expected {want} for {n_levels} stoc_len levels.")
    for i, t in enumerate(th):
        if not 0.0 <= t <= 1.0:
            raise ValueError(f"Adaptive MP threshold {t} for {source} is outside [0, 1].")
        if i > 0 and t > th[i - 1] + 1e-6:
            raise ValueError(f"Adaptive MP thresholds for {source} must be non-increasing, "
                             f"got {th}.")
    return th


def _assignment_from_levels(row_levels: torch.Tensor, stoc_len_levels: list) -> RowAssignment:
    """Rows of each level in ascending row order (torch.where)."""
    return RowAssignment(row_levels=row_levels, level_row_indices={
        sl: torch.where(row_levels == i)[0] for i, sl in enumerate(stoc_len_levels)})


def _all_rows_to_level(n: int, device, stoc_len_levels: list, level: int) -> RowAssignment:
    """Every row at one level (mp/config.py:500-517, and the degenerate-metric case)."""
    row_levels = torch.full((n,), int(level), dtype=torch.long, device=device)
    return RowAssignment(row_levels=row_levels, level_row_indices={
        sl: (torch.arange(n, device=device) if i == int(level)
             else torch.empty(0, dtype=torch.long, device=device))
        for i, sl in enumerate(stoc_len_levels)})


def _normalized(metric: torch.Tensor):
    """(metric - min) / (max - min), or None when the range is below 1e-8."""
    lo, hi = metric.min(), metric.max()
    if (hi - lo).item() < 1e-8:
        return None
    return (metric - lo) / (hi - lo)


def _classify_rows_by_thresholds(metric_norm: torch.Tensor, stoc_len_levels: list,
                                 thresholds: list) -> RowAssignment:
    """Level i takes the rows with thresholds[i] <= metric_norm < thresholds[i-1]; the rows
    below every threshold go to the last level (mp/config.py:119-151)."""
    n_levels = len(stoc_len_levels)
    if len(thresholds) != max(n_levels - 1, 0):
        raise ValueError(f"Expected {max(n_levels - 1, 0)} thresholds for {n_levels} levels, "
                         f"got {len(thresholds)}.")
    row_levels = torch.full((metric_norm.shape[0],), n_levels - 1, dtype=torch.long,
                            device=metric_norm.device)
    for i, t in enumerate(thresholds):
        mask = metric_norm >= metric_norm.new_tensor(t)
        if i > 0:
            mask &= metric_norm < metric_norm.new_tensor(thresholds[i - 1])
        row_levels[mask] = i
    return _assignment_from_levels(row_levels, stoc_len_levels)


@dataclass
class AdaptiveMPConfig:
    """Levels assigned by one of three data-driven paths, checked in this order by
    ``adaptive_classify_rows``: free boundaries (``FreeBoundaryMPConfig``), quantile
    fractions (``target_fractions``), calibrated thresholds per (operator, timestep bucket,
    layer bucket) (``threshold_table_path``) (mp/config.py:199-305). A stream length of 0
    as the last level means pruned rows (the mixed dispatch writes zeros for them)."""
    stoc_len_levels: list
    enable_pruning: bool = True
    threshold_table_path: Optional[str] = None
    timestep_buckets: int = 1
    layer_buckets: int = 1
    operator_default_thresholds: dict = field(default_factory=dict)
    bucket_thresholds: dict = field(default_factory=dict)
    target_fractions: Optional[list] = None

    def __post_init__(self):
        lv = self.stoc_len_levels
        assert len(lv) >= 2, "Need at least 2 levels (high + low or high + skip)"
        for i in range(len(lv) - 1):
            assert lv[i] > lv[i + 1], f"stoc_len_levels must be sorted descending, got {lv}"
        if not self.enable_pruning and 0 in lv:
            self.stoc_len_levels = [x for x in lv if x > 0]
        if self.threshold_table_path:
            self.load_threshold_table(self.threshold_table_path)
        if self.target_fractions is not None:
            assert len(self.target_fractions) == len(self.stoc_len_levels), (
                f"target_fractions length {len(self.target_fractions)} "
                f"must match stoc_len_levels length {len(self.stoc_len_levels)}")
            total = sum(self.target_fractions)
            assert abs(total - 1.0) < 1e-6, f"target_fractions must sum to 1.0, got {total}"

    def load_threshold_table(self, path: str):
        """Thresholds exported by a calibration run: {"stoc_len_levels", "timestep_buckets",
        "layer_buckets", "operator_defaults": {op: thresholds}, "buckets":
        {"op:t<i>:l<j>": thresholds}} (mp/config.py:255-286)."""
        with open(Path(path)) as f:
            payload = json.load(f)
        table_levels = [int(x) for x in payload["stoc_len_levels"]]
        if table_levels != self.stoc_len_levels:
            raise ValueError(f"Adaptive MP table levels {table_levels} do not match runtime "
                             f"levels {self.stoc_len_levels}.")
        n = len(self.stoc_len_levels)
        self.timestep_buckets = int(payload.get("timestep_buckets", 1))
        self.layer_buckets = int(payload.get("layer_buckets", 1))
        self.operator_default_thresholds = {
            op: _extract_thresholds(v, n, f"operator_default:{op}")
            for op, v in payload.get("operator_defaults", {}).items()}
        self.bucket_thresholds = {}
        for key, v in payload.get("buckets", {}).items():
            self.bucket_thresholds[_parse_bucket_key(key)] = _extract_thresholds(v, n, key)

    def get_thresholds(self, timestep: int, total_timesteps: int,
                       operator: Optional[str] = None, block_idx: Optional[int] = None,
                       total_blocks: Optional[int] = None) -> Optional[list]:
        """The bucket's thresholds, else the operator default, else None
        (mp/config.py:288-305)."""
        if (self.bucket_thresholds and operator and block_idx is not None
                and total_blocks is not None):
            key = (operator, _bucket_index(timestep, total_timesteps, self.timestep_buckets),
                   _bucket_index(block_idx, total_blocks, self.layer_buckets))
            if key in self.bucket_thresholds:
                return self.bucket_thresholds[key]
        if operator and operator in self.operator_default_thresholds:
            return self.operator_default_thresholds[operator]
        return None


@dataclass
class FreeBoundaryMPConfig(AdaptiveMPConfig):
    """k-1 free boundaries on the normalized metric per (block, operator), or a fixed level
    per (block, operator); missing entries use equal spacing (mp/config.py:415-497)."""
    boundaries: dict = field(default_factory=dict)
    fixed_levels: dict = field(default_factory=dict)

    def __post_init__(self):
        super().__post_init__()
        k = len(self.stoc_len_levels)
        for key, b in self.boundaries.items():
            assert isinstance(key, tuple) and len(key) == 2, (
                f"boundaries key must be (block_idx, op_name), got {key!r}")
            n = (b if isinstance(b, torch.Tensor) else torch.as_tensor(b)).numel()
            assert n == k - 1, f"boundaries[{key!r}] must have length {k - 1}, got {n}"
        for key, li in self.fixed_levels.items():
            assert isinstance(key, tuple) and len(key) == 2, (
                f"fixed_levels key must be (block_idx, op_name), got {key!r}")
            assert 0 <= int(li) < k, f"fixed_levels[{key!r}] must be in [0, {k}), got {int(li)}"

    def default_boundaries(self) -> torch.Tensor:
        k = len(self.stoc_len_levels)
        return torch.tensor([(k - 1 - i) / k for i in range(k - 1)], dtype=torch.float32)

    def _key(self, operator: str, block_idx: Optional[int]) -> tuple:
        return (int(_CURRENT_BLOCK_IDX if block_idx is None else block_idx), operator)

    def get_boundaries(self, operator: str, block_idx: Optional[int] = None) -> torch.Tensor:
        b = self.boundaries.get(self._key(operator, block_idx))
        if b is None:
            return self.default_boundaries()
        return b if isinstance(b, torch.Tensor) else torch.as_tensor(b)

    def set_boundaries(self, operator: str, block_idx: int, boundaries) -> None:
        bt = (boundaries.detach().cpu().float() if isinstance(boundaries, torch.Tensor)
              else torch.as_tensor(boundaries, dtype=torch.float32))
        k = len(self.stoc_len_levels)
        assert bt.numel() == k - 1, f"expected {k - 1} boundaries, got {bt.numel()}"
        key = self._key(operator, block_idx)
        self.fixed_levels.pop(key, None)
        self.boundaries[key] = bt

    def get_fixed_level(self, operator: str, block_idx: Optional[int] = None) -> Optional[int]:
        li = self.fixed_levels.get(self._key(operator, block_idx))
        return None if li is None else int(li)

    def set_fixed_level(self, operator: str, block_idx: int, level_idx: int) -> None:
        k = len(self.stoc_len_levels)
        assert 0 <= int(level_idx) < k, f"level_idx must be in [0, {k}), got {int(level_idx)}"
        key = self._key(operator, block_idx)
        self.boundaries.pop(key, None)
        self.fixed_levels[key] = int(level_idx)

    def clear_fixed_level(self, operator: str, block_idx: int) -> None:
        self.fixed_levels.pop(self._key(operator, block_idx), None)


def _classify_with_free_boundaries(metric: torch.Tensor, boundaries: torch.Tensor,
                                   stoc_len_levels: list) -> RowAssignment:
    """Level k+1 for rows whose normalized metric lies below the k-th largest boundary
    (mp/config.py:520-565)."""
    norm = _normalized(metric)
    if norm is None:
        return _all_rows_to_level(metric.shape[0], metric.device, stoc_len_levels, 0)
    b, _ = torch.sort(boundaries.to(metric.device).float(), descending=True)
    row_levels = torch.zeros(metric.shape[0], dtype=torch.long, device=metric.device)
    for k in range(len(stoc_len_levels) - 1):
        row_levels[norm < b[k]] = k + 1
    return _assignment_from_levels(row_levels, stoc_len_levels)


def adaptive_classify_rows(metric: torch.Tensor, config: AdaptiveMPConfig,
                           operator: Optional[str] = None, block_idx: Optional[int] = None,
                           total_blocks: Optional[int] = None, timestep: int = 0,
                           total_timesteps: int = 1) -> RowAssignment:
    """Row levels by the config's path: free boundaries, quantile fractions or calibrated
    thresholds; ValueError when none applies (mp/config.py:308-412)."""
    n = metric.shape[0]
    levels = config.stoc_len_levels
    if isinstance(config, FreeBoundaryMPConfig):
        fixed = config.get_fixed_level(operator or "")
        if fixed is not None:
            return _all_rows_to_level(n, metric.device, levels, fixed)
        return _classify_with_free_boundaries(metric, config.get_boundaries(operator or ""),
                                              levels)
    if config.target_fractions is not None:
        order = metric.argsort(descending=True)
        row_levels = torch.empty(n, dtype=torch.long, device=metric.device)
        rows_of = {}
        offset = 0
        for i, (sl, frac) in enumerate(zip(levels, config.target_fractions)):
            count = round(frac * n) if i < len(levels) - 1 else n - offset
            rows = order[offset:offset + count]
            row_levels[rows] = i
            rows_of[sl] = rows
            offset += count
        return RowAssignment(row_levels=row_levels, level_row_indices=rows_of)
    norm = _normalized(metric)
    if norm is None:
        return _all_rows_to_level(n, metric.device, levels, 0)
    th = config.get_thresholds(timestep=timestep, total_timesteps=total_timesteps,
                               operator=operator, block_idx=block_idx,
                               total_blocks=total_blocks)
    if th is not None:
        return _classify_rows_by_thresholds(norm, levels, th)
    raise ValueError(
        f"AdaptiveMPConfig: no classification path for operator={operator!r} "
        f"block_idx={block_idx} (not a FreeBoundaryMPConfig, target_fractions unset, and no "
        f"calibrated thresholds - bucket miss and no operator_default). Re-run calibration "
        f"covering this operator/layer, or set target_fractions.")


@dataclass
class RangeMPConfig:
    """Levels per weight-row group from the group's (max - min) range
    (mp/config.py:885-921)."""
    stoc_len_levels: list
    base_threshold: float = 0.3
    operator_thresholds: dict = field(default_factory=dict)

    def __post_init__(self):
        lv = self.stoc_len_levels
        assert len(lv) >= 2, "Need at least 2 levels (high + low)"
        for i in range(len(lv) - 1):
            assert lv[i] > lv[i + 1], f"stoc_len_levels must be sorted descending, got {lv}"

    def get_threshold(self, operator: Optional[str] = None) -> float:
        if operator and operator in self.operator_thresholds:
            return self.operator_thresholds[operator]
        return self.base_threshold


def classify_groups_by_range(weight: torch.Tensor, group_size: int, config: RangeMPConfig,
                             operator: Optional[str] = None) -> list:
    """One stream length per group of group_size weight rows: normalized range >= the
    operator threshold (at most 0.95) -> the longest; below it, evenly spaced boundaries
    pick the shorter levels. Prints the distribution line (mp/config.py:924-1007)."""
    out_features = weight.shape[0]
    if group_size <= 0 or group_size >= out_features:
        group_size = out_features
    groups = out_features // group_size
    levels = config.stoc_len_levels
    n_levels = len(levels)
    threshold = min(config.get_threshold(operator), 0.95)
    w = weight.reshape(groups, -1).float()
    rng = w.amax(dim=-1) - w.amin(dim=-1)
    norm = (rng - rng.min()) / (rng.max() - rng.min() + 1e-8)
    glevel = torch.zeros(groups, dtype=torch.long, device=weight.device)
    for k in range(n_levels - 1):
        glevel[norm < threshold * (n_levels - 1 - k) / (n_levels - 1)] = k + 1
    result = [levels[i] for i in glevel.tolist()]
    dist = {sl: result.count(sl) for sl in levels}
    print(f"  [RangeMP] {operator or 'unknown'}: groups={groups}, threshold={threshold:.2f}, "
          f"distribution={dist}, range_stats: min={rng.min().item():.4f}, "
          f"max={rng.max().item():.4f}, mean={rng.mean().item():.4f}")
    return result

"""Mixed-precision dispatch of the per_row SC matmul over a row-to-level assignment.

A mixed-precision caller of the reference runs, for every level L of a RowAssignment
(scmp_kernels/mp/config.py:154-191, 308-412),

    Y[rows_L] = sc_matmul(a[rows_L], b, "per_row", ..., stoc_len=L, rng_levels=L)

which gathers a's rows, quantizes b once per level and scatters each result into Y.
``sc_matmul_mixed`` computes the same Y in one call: b is quantized once (or comes from
``prepare_weight``), each level's quantizer reads its rows of a in place through a row index,
and each level's GEMM writes its rows of Y in place through a row map. Rows at stream length
0 (pruned by an adaptive config) are zero.
"""
from __future__ import annotations

from typing import Optional

import torch

from ..sc import kernels as _k
from ..sc.matmul import _VALID_MODES
from ..quant.smoothquant import _check_smoothing_vector
from .config import RowAssignment


def _check_rows(row_lists, N: int) -> bool:
    """Validate the row indices the kernels will read and write, with one host sync: every
    index in [0, N) and no row in two places (a repeated row would be written twice, by two
    levels or by two row groups of one level, with different values). Returns whether the
    rows cover all N rows exactly once (then the output needs no zero fill)."""
    if not row_lists:
        return N == 0
    idx = torch.cat(row_lists)
    lo, hi = torch.aminmax(idx)
    cnt = torch.bincount(idx.clamp(0, max(N - 1, 0)), minlength=max(N, 1))
    lo, hi, most, seen = (int(v) for v in torch.stack(
        [lo, hi, cnt.max(), (cnt > 0).sum()]).cpu())
    if lo < 0 or hi >= N:
        raise ValueError(f"sc_matmul_mixed: row indices must lie in [0, {N}), got "
                         f"[{lo}, {hi}]")
    if most > 1:
        raise ValueError("sc_matmul_mixed: a row appears more than once in the assignment "
                         "(each row belongs to one level, once)")
    return seen == N


def _checked_rows(assignment, originals, row_lists, N: int) -> bool:
    """_check_rows with its host sync taken once per assignment: the result is kept on the
    assignment together with the index tensors it checked, and holds for a later call
    with the same N whose level tensors are the same objects at the same version (torch
    bumps a tensor's version on every in-place change). Index tensors on the CPU are
    checked there, with no device sync."""
    if all(not t.is_cuda for t in originals):
        return _check_rows([t.to(torch.int64) for t in originals], N)
    key = (N, tuple((id(t), t._version) for t in originals))
    seen = getattr(assignment, "_scmp_rows_checked", None)
    if seen is not None and seen[0] == key and all(a is b for a, b in zip(seen[1], originals)):
        return seen[2]
    exact = _check_rows(row_lists, N)
    try:
        assignment._scmp_rows_checked = (key, list(originals), exact)
    except AttributeError:
        pass
    return exact


@torch.no_grad()
def sc_matmul_mixed(a: torch.Tensor, b, assignment: RowAssignment, *, mode: str = "unipolar",
                    sc_prec: int = 8, group_a: int = 1, group_b: int = 1,
                    rng_levels: Optional[int] = None, config: Optional[dict] = None,
                    smooth_scales: Optional[torch.Tensor] = None) -> torch.Tensor:
    """(N, M) float32: rows ``assignment.level_row_indices[L]`` hold
    ``sc_matmul(a[rows], b, "per_row", mode=mode, sc_prec=sc_prec, group_a=group_a,
    group_b=group_b, stoc_len=L, rng_levels=R, config=config, smooth_scales=...)`` with
    R = L (``rng_levels=None``, the mixed-precision convention) or the given rng_levels.
    The row groups of group_a follow each level's row order. ``b`` is an (M, D) weight or a
    PreparedWeight of the same mode / sc_prec / group_b / smoothing. The row indices are
    validated (in range, no row twice) once per assignment: the first call with device
    index tensors syncs with the host, later calls with the same unmodified tensors do not.
    Rows that no level names are zero."""
    if mode not in _VALID_MODES:
        raise ValueError(f"sc_matmul: unknown mode '{mode}'. Expected one of {_VALID_MODES}.")
    if not 1 <= sc_prec <= 8:
        raise ValueError(f"sc_matmul: sc_prec={sc_prec} outside [1, 8]")
    if a.dim() != 2:
        raise ValueError(f"sc_matmul_mixed: a must be 2-D, got {a.dim()}-D")
    prepared = isinstance(b, _k.PreparedWeight)
    if not prepared and b.dim() != 2:
        raise ValueError(f"sc_matmul_mixed: b must be 2-D, got {b.dim()}-D")
    if a.shape[1] != b.shape[1]:
        raise ValueError(f"sc_matmul_mixed: inner dims differ: {a.shape[1]} vs {b.shape[1]}")
    dev = b.device if prepared else (a.device if a.is_cuda else None)
    home = None
    if dev is None or not a.is_cuda:
        if not torch.cuda.is_available():
            raise RuntimeError("scmp_kernels_amd: the SC kernels run on the GPU; got CPU "
                               "tensors and no GPU is available")
        home = a.device
        dev = dev if dev is not None else torch.device("cuda", torch.cuda.current_device())
    if a.is_cuda and a.device != dev:
        raise ValueError(f"sc_matmul_mixed: a is on {a.device}, b on {dev}")
    if not prepared and b.device != dev:
        b = b.to(dev)
    a = _k._rows2d(a.to(dev))
    N, D = a.shape
    smooth = None
    if smooth_scales is not None:
        if a.dtype != torch.float32:
            raise ValueError("sc_matmul_mixed: smooth_scales need float32 activations")
        _check_smoothing_vector(smooth_scales, D, names=("a",))
        smooth = smooth_scales.to(device=dev, dtype=torch.float32).contiguous()

    levels, pruned, originals = [], [], []
    for L, rows in assignment.level_row_indices.items():
        if rows.numel():
            originals.append(rows)
        rows = rows.to(device=dev, dtype=torch.int64).contiguous()
        L = int(L)
        if rows.numel() == 0:
            continue
        if L <= 0:
            pruned.append(rows)
            continue
        if L > 2 ** sc_prec:
            raise ValueError(f"sc_matmul: stoc_len={L} exceeds 2**sc_prec={2 ** sc_prec}; the "
                             f"RNG sequences are 2**sc_prec long.")
        levels.append((L, L if rng_levels is None else int(rng_levels), rows))
    exact = _checked_rows(assignment, originals, [r for _, _, r in levels] + pruned, N)
    M = b.M if prepared else b.shape[0]
    with torch.cuda.device(dev):
        if prepared:
            b.check(D, mode, sc_prec, group_b, smooth_scales)
        y = (torch.empty if exact else torch.zeros)((N, M), dtype=torch.float32, device=dev)
        for rows in pruned:
            y.index_fill_(0, rows, 0.0)
        _k._per_row_levels(a, b, levels, y, group_a=group_a, group_b=group_b, mode=mode,
                           sc_prec=sc_prec, config=config, smooth_scales=smooth)
    return y.to(home) if home is not None else y

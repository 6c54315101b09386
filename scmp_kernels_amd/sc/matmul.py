"""``sc_matmul``: the public SC matmul entry point, with the call surface of the
reference's scmp_kernels/sc/matmul.py:61-279.

The function checks its arguments (same ValueError messages as the reference), applies
the ``halve_bipolar_stoc_len`` defaults, and hands the call to one host path of
:mod:`.kernels` according to granularity, operand rank and ``chunk_d``. All work runs on
the operands' GPU: the current device is switched to ``a.device`` for the call and
restored afterwards. ``smooth_scales`` on fp32 operands is passed down to the quantizers,
which divide / multiply as they load; other dtypes are smoothed up front.
"""
from __future__ import annotations

import contextlib
from typing import Optional

import torch

from . import kernels as _paths
# the per-path entry points, reachable from this module as in the reference
# (scmp_kernels/sc/matmul.py:23-29); each takes the reference's parameter list
from .kernels import (_sc_matmul_per_head_bipolar, _sc_matmul_per_row,  # noqa: F401
                      _sc_matmul_per_row_batched, _sc_matmul_per_row_mlp,
                      _sc_matmul_per_tensor)
from ..quant.smoothquant import apply_smoothing, _check_smoothing_vector

_VALID_GRANULARITIES = ("per_tensor", "per_row", "per_head")
_VALID_MODES = ("bipolar", "unipolar")


def _device_scope(a: torch.Tensor, b: torch.Tensor):
    """The context every launch of one call runs in: a's GPU as the current device (the
    reference's device guard, scmp_kernels/sc/matmul.py:37-78). Operands on two devices
    are rejected."""
    if a.device != b.device:
        raise ValueError(
            f"sc_matmul: a and b must be on the same device, got a.device={a.device}, "
            f"b.device={b.device}.")
    return torch.cuda.device(a.device) if a.is_cuda else contextlib.nullcontext()


def _check_combination(a, b, granularity: str, mode: str, chunk_d: int) -> None:
    """Reject unsupported argument combinations (scmp_kernels/sc/matmul.py:164-221)."""
    if granularity not in _VALID_GRANULARITIES:
        raise ValueError(f"sc_matmul: unknown granularity '{granularity}'. "
                         f"Expected one of {_VALID_GRANULARITIES}.")
    if mode not in _VALID_MODES:
        raise ValueError(f"sc_matmul: unknown mode '{mode}'. Expected one of {_VALID_MODES}.")
    ranks = f"a.dim()={a.dim()}, b.dim()={b.dim()}"
    if chunk_d > 0:
        why = None
        if granularity != "per_row":
            why = (f"requires granularity='per_row', got '{granularity}'. D-chunking is only "
                   f"implemented in the per-row MLP fast path.")
        elif mode != "bipolar":
            why = (f"requires mode='bipolar', got '{mode}'. D-chunking is not implemented for "
                   f"unipolar quantization.")
        elif a.dim() != 2 or b.dim() != 2:
            why = f"requires 2D inputs (the per-row MLP fast path is 2D only), got {ranks}."
        if why:
            raise ValueError(f"sc_matmul: chunk_d > 0 {why}")
    if granularity == "per_head":
        if a.dim() != 3 or b.dim() != 3:
            raise ValueError(f"sc_matmul: granularity='per_head' requires 3D inputs "
                             f"(BH, *, D), got {ranks}.")
        if mode != "bipolar":
            raise ValueError(f"sc_matmul: granularity='per_head' currently only supports "
                             f"mode='bipolar', got '{mode}'.")


def _smoothing_for_kernels(a, b, smooth_scales):
    """(a, b, s): ``s`` for the quantizers to apply while loading fp32 operands, or
    (a / s, b * s, None) for other dtypes."""
    if smooth_scales is None:
        return a, b, None
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        a, b = apply_smoothing(a, b, smooth_scales)
        return a, b, None
    _check_smoothing_vector(smooth_scales, a.shape[-1], b.shape[-1], names=("a", "b"))
    dev = a.device if a.is_cuda else torch.device("cuda")
    return a, b, smooth_scales.to(device=dev, dtype=torch.float32).contiguous()


@torch.no_grad()
def sc_matmul(
    a: torch.Tensor,
    b: torch.Tensor,
    granularity: str = "per_row",
    *,
    mode: str = "bipolar",
    sc_prec: int = 8,
    stoc_len: Optional[int] = None,
    chunk_d: int = 0,
    group_a: int = 1,
    group_b: int = 1,
    rng_levels: Optional[int] = None,
    config: Optional[dict] = None,
    halve_bipolar_stoc_len: bool = False,
    smooth_scales: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Stochastic-computing ``a @ b.T``: ``(N, D) x (M, D) -> (N, M)`` or
    ``(BH, N, D) x (BH, M, D) -> (BH, N, M)``, float32 (scmp_kernels/sc/matmul.py:61-163).

    granularity: "per_tensor" | "per_row" | "per_head"; mode: "bipolar" | "unipolar";
    stoc_len: stream length (default 2**sc_prec, at most 2**sc_prec); chunk_d: per-row
    bipolar 2-D inner-dimension chunks with their own scales; group_a / group_b: rows per
    quantization group; rng_levels: RNG grid size (default 2**sc_prec); config: RNG/SNG
    dict (default: one Sobol sequence per side); halve_bipolar_stoc_len: default
    stoc_len and rng_levels to 2**(sc_prec-1) in bipolar mode; smooth_scales: (D,)
    SmoothQuant vector, ``sc_matmul(a, b, smooth_scales=s) == sc_matmul(a / s, b * s)``.
    sc_prec must lie in [1, 8] (byte operand codes).
    """
    if isinstance(b, _paths.PreparedWeight):
        return _sc_matmul_prepared(a, b, granularity, mode=mode, sc_prec=sc_prec,
                                   stoc_len=stoc_len, chunk_d=chunk_d, group_a=group_a,
                                   group_b=group_b, rng_levels=rng_levels, config=config,
                                   halve_bipolar_stoc_len=halve_bipolar_stoc_len,
                                   smooth_scales=smooth_scales)
    with _device_scope(a, b):
        _check_combination(a, b, granularity, mode, chunk_d)
        if halve_bipolar_stoc_len and mode == "bipolar":
            half = 2 ** (sc_prec - 1)
            stoc_len = half if stoc_len is None else stoc_len
            rng_levels = half if rng_levels is None else rng_levels
        if stoc_len is not None and stoc_len > 2 ** sc_prec:
            raise ValueError(
                f"sc_matmul: stoc_len={stoc_len} exceeds 2**sc_prec={2 ** sc_prec}; the RNG "
                f"sequences are 2**sc_prec long.")
        if a.shape[-2] == 0 or b.shape[-2] == 0:
            # no rows on one side: an empty product, nothing to launch
            lead = a.shape[:-2] if a.dim() == 3 else ()
            return torch.empty((*lead, a.shape[-2], b.shape[-2]), dtype=torch.float32,
                               device=a.device)
        if a.shape[-1] == 0:
            raise ValueError("sc_matmul: the inner dimension D must be positive")
        a, b, smooth = _smoothing_for_kernels(a, b, smooth_scales)
        common = dict(mode=mode, sc_prec=sc_prec, config=config, stoc_len=stoc_len,
                      rng_levels=rng_levels, smooth_scales=smooth)
        if granularity == "per_tensor":
            return _paths._sc_matmul_per_tensor(a, b, **common)
        if granularity == "per_head":
            del common["mode"]
            return _paths._sc_matmul_per_head_bipolar(a, b, **common)
        groups = dict(group_a=group_a, group_b=group_b)
        if chunk_d > 0:
            return _paths._sc_matmul_per_row_mlp(a, b, chunk_d=chunk_d, **groups, **common)
        if a.dim() == 3:
            return _paths._sc_matmul_per_row_batched(a, b, **groups, **common)
        return _paths._sc_matmul_per_row(a, b, **groups, **common)


def _sc_matmul_prepared(a, w, granularity, *, mode, sc_prec, stoc_len, chunk_d, group_a,
                        group_b, rng_levels, config, halve_bipolar_stoc_len, smooth_scales):
    """sc_matmul with a weight from ``prepare_weight``: the 2-D per_row path without the
    weight's quantizer. Results equal sc_matmul(a, b, ...) with the original weight."""
    if granularity != "per_row" or chunk_d > 0 or a.dim() != 2:
        raise ValueError("sc_matmul: a prepared weight supports granularity='per_row' with "
                         f"2-D a and chunk_d=0, got granularity='{granularity}', "
                         f"chunk_d={chunk_d}, a.dim()={a.dim()}.")
    if mode not in _VALID_MODES:
        raise ValueError(f"sc_matmul: unknown mode '{mode}'. Expected one of {_VALID_MODES}.")
    if halve_bipolar_stoc_len and mode == "bipolar":
        half = 2 ** (sc_prec - 1)
        stoc_len = half if stoc_len is None else stoc_len
        rng_levels = half if rng_levels is None else rng_levels
    if stoc_len is not None and stoc_len > 2 ** sc_prec:
        raise ValueError(
            f"sc_matmul: stoc_len={stoc_len} exceeds 2**sc_prec={2 ** sc_prec}; the RNG "
            f"sequences are 2**sc_prec long.")
    smooth = None
    if smooth_scales is not None:
        if a.dtype != torch.float32:
            raise ValueError("sc_matmul: a prepared weight with smooth_scales needs float32 "
                             "activations")
        _check_smoothing_vector(smooth_scales, a.shape[-1], names=("a",))
        smooth = smooth_scales.to(device=w.device, dtype=torch.float32).contiguous()
        # the weight was prepared with this vector (compared by PreparedWeight.check)
        if smooth_scales is w.smooth_scales:
            smooth = w.smooth_scales.to(device=w.device, dtype=torch.float32).contiguous()
    with torch.cuda.device(w.device):
        w.check(a.shape[-1], mode, sc_prec, group_b, smooth_scales)
        return _paths._sc_matmul_per_row(a, w, group_a=group_a, group_b=group_b, mode=mode,
                                         sc_prec=sc_prec, config=config, stoc_len=stoc_len,
                                         rng_levels=rng_levels, smooth_scales=smooth)


_sc_matmul_impl = sc_matmul

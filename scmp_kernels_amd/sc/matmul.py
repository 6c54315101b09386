"""Unified public SC matmul entry point (the reference's scmp_kernels/sc/matmul.py:61-279).

``sc_matmul`` validates its arguments with the reference's messages, applies the
halve_bipolar_stoc_len override, and dispatches by granularity / dimensionality /
chunk_d to the host paths in :mod:`.kernels`. SmoothQuant's ``(a / s, b * s)``
(matmul.py:189-190) is folded into the quantizer loads rather than materialized.
"""
from __future__ import annotations

import contextlib
import functools
from typing import Optional

import torch

from .kernels import (
    _sc_matmul_per_tensor,
    _sc_matmul_per_row,
    _sc_matmul_per_row_mlp,
    _sc_matmul_per_row_batched,
    _sc_matmul_per_head_bipolar,
)
from ..quant.smoothquant import apply_smoothing

_VALID_GRANULARITIES = ("per_tensor", "per_row", "per_head")
_VALID_MODES = ("bipolar", "unipolar")


def _pin_to_operand_device(fn):
    """Run on the operands' GPU; the previous current device is restored on exit
    (scmp_kernels/sc/matmul.py:37-58)."""
    @functools.wraps(fn)
    def wrapper(a, b, *args, **kwargs):
        if a.device != b.device:
            raise ValueError(
                f"sc_matmul: a and b must be on the same device, got a.device={a.device}, "
                f"b.device={b.device}.")
        if a.is_cuda:
            with torch.cuda.device(a.device):
                return fn(a, b, *args, **kwargs)
        return fn(a, b, *args, **kwargs)
    return wrapper


@_pin_to_operand_device
@torch.no_grad()
def sc_matmul(a: torch.Tensor, b: torch.Tensor, *args, **kwargs) -> torch.Tensor:
    """Device-guarded public entry point; see :func:`_sc_matmul_impl`."""
    guard = torch.cuda.device(a.device) if a.is_cuda else contextlib.nullcontext()
    with guard:
        return _sc_matmul_impl(a, b, *args, **kwargs)


@torch.no_grad()
def _sc_matmul_impl(
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
    """Stochastic-computing matmul ``a @ b.T`` (2-D ``(N, D) x (M, D) -> (N, M)`` or 3-D
    ``(BH, N, D) x (BH, M, D) -> (BH, N, M)``), float32 output.

    Arguments and errors are those of the reference (scmp_kernels/sc/matmul.py:82-163):
    granularity in {"per_tensor", "per_row", "per_head"}, mode in {"bipolar",
    "unipolar"}, stoc_len (default 2**sc_prec; at most 2**sc_prec), chunk_d (per_row
    bipolar 2-D only), group_a / group_b row groups, rng_levels (default 2**sc_prec),
    config (Sobol/LFSR RNG/SNG dict), halve_bipolar_stoc_len, smooth_scales (D,).
    sc_prec must be in [1, 8] (8-bit operand codes).
    """
    if granularity not in _VALID_GRANULARITIES:
        raise ValueError(
            f"sc_matmul: unknown granularity '{granularity}'. "
            f"Expected one of {_VALID_GRANULARITIES}.")
    if mode not in _VALID_MODES:
        raise ValueError(
            f"sc_matmul: unknown mode '{mode}'. "
            f"Expected one of {_VALID_MODES}.")

    if halve_bipolar_stoc_len and mode == "bipolar":
        halved = 2 ** (sc_prec - 1)
        if stoc_len is None:
            stoc_len = halved
        if rng_levels is None:
            rng_levels = halved

    smooth = None
    if smooth_scales is not None:
        if a.dtype == torch.float32 and b.dtype == torch.float32:
            # validated here, applied inside the quantizers
            if smooth_scales.dim() != 1:
                raise ValueError(
                    f"smooth_scales must be 1D (D,), got shape {tuple(smooth_scales.shape)}")
            if a.shape[-1] != smooth_scales.shape[0] or b.shape[-1] != smooth_scales.shape[0]:
                raise ValueError(
                    f"D mismatch: a.shape[-1]={a.shape[-1]}, b.shape[-1]={b.shape[-1]}, "
                    f"smooth_scales.shape[0]={smooth_scales.shape[0]}")
            smooth = smooth_scales.to(device=a.device if a.is_cuda else "cuda",
                                      dtype=torch.float32).contiguous()
        else:
            a, b = apply_smoothing(a, b, smooth_scales)

    if chunk_d > 0:
        if granularity != "per_row":
            raise ValueError(
                f"sc_matmul: chunk_d > 0 requires granularity='per_row', "
                f"got '{granularity}'. D-chunking is only implemented in the "
                f"per-row MLP fast path.")
        if mode != "bipolar":
            raise ValueError(
                f"sc_matmul: chunk_d > 0 requires mode='bipolar', got '{mode}'. "
                f"D-chunking is not implemented for unipolar quantization.")
        if a.dim() != 2 or b.dim() != 2:
            raise ValueError(
                f"sc_matmul: chunk_d > 0 requires 2D inputs (the per-row MLP "
                f"fast path is 2D only), got a.dim()={a.dim()}, b.dim()={b.dim()}.")

    if granularity == "per_head":
        if a.dim() != 3 or b.dim() != 3:
            raise ValueError(
                f"sc_matmul: granularity='per_head' requires 3D inputs (BH, *, D), "
                f"got a.dim()={a.dim()}, b.dim()={b.dim()}.")
        if mode != "bipolar":
            raise ValueError(
                f"sc_matmul: granularity='per_head' currently only supports "
                f"mode='bipolar', got '{mode}'.")

    if stoc_len is not None and stoc_len > 2 ** sc_prec:
        raise ValueError(
            f"sc_matmul: stoc_len={stoc_len} exceeds 2**sc_prec={2 ** sc_prec}; the RNG "
            f"sequences are 2**sc_prec long.")

    if granularity == "per_tensor":
        return _sc_matmul_per_tensor(a, b, mode=mode, sc_prec=sc_prec, config=config,
                                     stoc_len=stoc_len, rng_levels=rng_levels,
                                     smooth_scales=smooth)
    if granularity == "per_row":
        if chunk_d > 0:
            return _sc_matmul_per_row_mlp(a, b, mode=mode, sc_prec=sc_prec, config=config,
                                          group_a=group_a, group_b=group_b, chunk_d=chunk_d,
                                          stoc_len=stoc_len, rng_levels=rng_levels,
                                          smooth_scales=smooth)
        if a.dim() == 3:
            return _sc_matmul_per_row_batched(a, b, group_a=group_a, group_b=group_b,
                                              mode=mode, sc_prec=sc_prec, config=config,
                                              stoc_len=stoc_len, rng_levels=rng_levels,
                                              smooth_scales=smooth)
        return _sc_matmul_per_row(a, b, group_a=group_a, group_b=group_b, mode=mode,
                                  sc_prec=sc_prec, config=config, stoc_len=stoc_len,
                                  rng_levels=rng_levels, smooth_scales=smooth)
    return _sc_matmul_per_head_bipolar(a, b, sc_prec=sc_prec, config=config,
                                       stoc_len=stoc_len, rng_levels=rng_levels,
                                       smooth_scales=smooth)

"""SmoothQuant helpers with the call surface of the reference's
scmp_kernels/quant/smoothquant.py.

The matmul is invariant under a per-channel rescaling of the contracted axis,
``A @ B.T == (A / s) @ (B * s).T``; choosing ``s_d = amax_d(A)^alpha / amax_d(B)^(1-alpha)``
moves activation outliers into the weights. These are calibration-time tensor utilities
that run on whatever device their inputs live on. Inside ``sc_matmul`` the two scalings
are never materialized: the HIP quantizers apply ``x / s[d]`` (activations) and
``x * s[d]`` (weights) as they load, with the same single fp32 rounding.
"""
from __future__ import annotations

from typing import Optional

import torch


def _check_smoothing_vector(s: torch.Tensor, *dims: int, names: tuple = ()) -> None:
    """Raise the reference's ValueErrors for a smoothing vector that is not 1-D or whose
    length differs from one of the operand widths."""
    if s.dim() != 1:
        raise ValueError(f"smooth_scales must be 1D (D,), got shape {tuple(s.shape)}")
    if any(d != s.shape[0] for d in dims):
        parts = ", ".join(f"{n}.shape[-1]={d}" for n, d in zip(names, dims))
        if len(dims) == 1:
            raise ValueError(f"D mismatch: {parts} vs smooth_scales.shape[0]={s.shape[0]}")
        raise ValueError(f"D mismatch: {parts}, smooth_scales.shape[0]={s.shape[0]}")


@torch.no_grad()
def accumulate_act_scales(x: torch.Tensor, running: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Running per-channel max of |x| over every leading axis of ``x (..., D)``; merged
    into ``running`` (D,) when given (scmp_kernels/quant/smoothquant.py:32-50)."""
    channel_max = x.detach().reshape(-1, x.shape[-1]).abs().amax(dim=0)
    if running is None:
        return channel_max
    prev = running.to(device=channel_max.device, dtype=channel_max.dtype)
    return torch.maximum(prev, channel_max)


@torch.no_grad()
def compute_smooth_scales(act_scales: torch.Tensor, weight: torch.Tensor, alpha: float = 0.5,
                          eps: float = 1e-5) -> torch.Tensor:
    """``s = max(act^alpha / w_max^(1-alpha), eps)`` with both maxima floored at ``eps``;
    ``w_max`` is the per-column max |weight| of ``weight (M, D)``. Returned on weight's
    device and dtype (scmp_kernels/quant/smoothquant.py:53-93)."""
    if not 0.0 <= alpha <= 1.0:
        raise ValueError(f"alpha must be in [0, 1], got {alpha}")
    if act_scales.dim() != 1:
        raise ValueError(f"act_scales must be 1D (D,), got shape {tuple(act_scales.shape)}")
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2D (M, D), got shape {tuple(weight.shape)}")
    if weight.shape[-1] != act_scales.shape[0]:
        raise ValueError(
            f"D mismatch: weight.shape[-1]={weight.shape[-1]} vs "
            f"act_scales.shape[0]={act_scales.shape[0]}")
    act = act_scales.to(device=weight.device, dtype=weight.dtype).clamp_min(eps)
    wmax = weight.abs().amax(dim=0).clamp_min(eps)
    return torch.clamp_min(torch.pow(act, alpha) / torch.pow(wmax, 1.0 - alpha), eps)


@torch.no_grad()
def apply_smoothing(a: torch.Tensor, b: torch.Tensor, smooth_scales: torch.Tensor):
    """Return ``(a / s, b * s)``, ``s`` broadcast along the last axis of both operands
    (scmp_kernels/quant/smoothquant.py:96-126)."""
    _check_smoothing_vector(smooth_scales, a.shape[-1], b.shape[-1], names=("a", "b"))
    return (a / smooth_scales.to(device=a.device, dtype=a.dtype),
            b * smooth_scales.to(device=b.device, dtype=b.dtype))


@torch.no_grad()
def apply_smoothing_offline(weight: torch.Tensor, smooth_scales: torch.Tensor) -> torch.Tensor:
    """``weight * s``, computed once at load time so that later calls only divide the
    activations (scmp_kernels/quant/smoothquant.py:129-147)."""
    _check_smoothing_vector(smooth_scales, weight.shape[-1], names=("weight",))
    return weight * smooth_scales.to(device=weight.device, dtype=weight.dtype)


__all__ = [
    "accumulate_act_scales",
    "compute_smooth_scales",
    "apply_smoothing",
    "apply_smoothing_offline",
]

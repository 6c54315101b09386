"""Fused FP -> SC-boundary quantizers (the reference's scmp_kernels/quant/fused.py API),
each one scmp_quantize call on the GPU.

* Bipolar  -> (boundary int16, sign int8, scale)
* Unipolar -> (boundary int32, scale, zp[, row_sum])

``boundary = rne(|q| * fl32(R / Q))`` with R = rng_levels (default 2**sc_prec).
The reference's Triton kernel objects ``fused_quant_kernel`` and
``fused_quant_bipolar_batched_kernel`` have no equivalent here (the quantizer is a HIP
kernel behind the C ABI); those names are kept and raise NotImplementedError when used.
"""
from __future__ import annotations

import functools
from typing import Optional

import torch

from .. import _lib


def _resolve_rng_levels(sc_prec: int, rng_levels: Optional[int]) -> int:
    return 2 ** sc_prec if rng_levels is None else int(rng_levels)


class _TritonKernelName:
    """Placeholder for a Triton kernel object of the reference."""

    def __init__(self, name: str, use: str):
        self.__name__ = name
        self._use = use

    def __getitem__(self, grid):
        raise NotImplementedError(
            f"{self.__name__} is a Triton kernel in the reference; the gfx950 build runs a "
            f"HIP quantizer instead: call {self._use}.")

    def __call__(self, *a, **k):
        return self[None]


fused_quant_kernel = _TritonKernelName(
    "fused_quant_kernel",
    "fused_quantize_bipolar / fused_quantize_bipolar_perrow / fused_quantize_unipolar")
fused_quant_bipolar_batched_kernel = _TritonKernelName(
    "fused_quant_bipolar_batched_kernel", "sc_matmul(..., granularity='per_head')")


@functools.lru_cache(maxsize=8)
def _quant_dummy(device: torch.device) -> torch.Tensor:
    """1-element int8 tensor per device (quant/fused.py:126-131)."""
    return torch.empty(1, dtype=torch.int8, device=device)


def _on_gpu(x: torch.Tensor):
    if x.is_cuda:
        return x, None
    if not torch.cuda.is_available():
        raise RuntimeError("scmp_kernels_amd: the quantizers run on the GPU; none available")
    return x.cuda(), x.device


def _back(t, home):
    if home is None or t is None:
        return t
    return t.to(home)


def fused_quantize_bipolar_perrow(fp_tensor: torch.Tensor, sc_prec: int,
                                  rng_levels: Optional[int] = None):
    """Per-row bipolar (quant/fused.py:134-159): A = max(max|x|, 1e-5), scale = A / Q,
    q = clamp(rne(x * fl(1 / scale)), +-Q). Returns (boundary int16, sign int8 with 0 for
    zeros, scale_row float32)."""
    from ..sc.kernels import quantize
    x, home = _on_gpu(fp_tensor)
    rows, cols = x.shape
    Q = 2 ** (sc_prec - 1) - 1
    R = _resolve_rng_levels(sc_prec, rng_levels)
    beta = torch.empty((rows, cols), dtype=torch.int16, device=x.device)
    sign = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    quantize(x, _lib.Q_ROW_SYM, Q, R, group=1, beta16=beta, sign=sign, scale=scale)
    return _back(beta, home), _back(sign, home), _back(scale, home)


def fused_quantize_bipolar(fp_tensor: torch.Tensor, abs_max: float, sc_prec: int,
                           rng_levels: Optional[int] = None):
    """Per-tensor bipolar with the caller's range (quant/fused.py:162-189): scale =
    max(abs_max, 1e-5) / Q in Python floats; returns (boundary, sign, scale)."""
    from ..sc.kernels import quantize
    x, home = _on_gpu(fp_tensor)
    rows, cols = x.shape
    Q = 2 ** (sc_prec - 1) - 1
    R = _resolve_rng_levels(sc_prec, rng_levels)
    abs_max = max(abs_max, 1e-5)
    scale = abs_max / Q
    inv_scale = 1.0 / scale
    beta = torch.empty((rows, cols), dtype=torch.int16, device=x.device)
    sign = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    quantize(x, _lib.Q_HOST_SYM, Q, R, host_inv=inv_scale, beta16=beta, sign=sign)
    return _back(beta, home), _back(sign, home), scale


def fused_quantize_unipolar(fp_tensor: torch.Tensor, fp_max: float, fp_min: float,
                            sc_prec: int, compute_sum: bool = False,
                            rng_levels: Optional[int] = None):
    """Unipolar with the caller's range (quant/fused.py:192-234): scale = max(max - min,
    1e-5) / Q, zp = clamp(round(-min / scale), 0, Q) in Python floats;
    q = clamp(rne(fl(x * inv) + zp), 0, Q). Returns (boundary int32, scale, zp,
    row_sum float32 | None)."""
    from ..sc.kernels import quantize
    x, home = _on_gpu(fp_tensor)
    rows, cols = x.shape
    Q = 2 ** sc_prec - 1
    R = _resolve_rng_levels(sc_prec, rng_levels)
    range_fp = max(fp_max - fp_min, 1e-5)
    scale = range_fp / Q
    inv_scale = 1.0 / scale
    zp = round(-fp_min / scale)
    zp = max(0, min(Q, zp))
    zp_f = float(zp)
    beta = torch.empty((rows, cols), dtype=torch.int32, device=x.device)
    row_sum = torch.empty(rows, dtype=torch.float32, device=x.device) if compute_sum else None
    quantize(x, _lib.Q_HOST_ASYM, Q, R, host_inv=inv_scale, host_zp=zp_f, beta32=beta,
             rowsum=row_sum)
    return _back(beta, home), scale, zp_f, _back(row_sum, home)


__all__ = [
    "fused_quant_kernel",
    "fused_quant_bipolar_batched_kernel",
    "fused_quantize_bipolar",
    "fused_quantize_bipolar_perrow",
    "fused_quantize_unipolar",
    "_quant_dummy",
]

"""Row-group quantizers (the reference's scmp_kernels/quant/grouped.py API, torch there),
each one scmp_quantize call on the GPU with the reference's fp32 operation order:
division by the scale (not a reciprocal multiply), round half to even, clamp.
"""
from __future__ import annotations

import torch

from .. import _lib
from .fused import _on_gpu, _back


def _grouped_symmetric_quant(x, G, q_max):
    """Groups of G consecutive rows (remainder rows form the last group):
    scale = max(max|x|, 1e-5) / q_max, x_int = clamp(rne(x / scale), +-q_max),
    sign = sgn(x_int) with 0 -> +1 (quant/grouped.py:13-75).
    Returns (scale_row (rows,), x_int float32, sign int8)."""
    from ..sc.kernels import quantize
    x, home = _on_gpu(x)
    rows, cols = x.shape
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    xint = torch.empty((rows, cols), dtype=torch.float32, device=x.device)
    sign = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    quantize(x, _lib.Q_GROUP_SYM, int(q_max), 1, group=G, xint=xint, sign=sign, scale=scale)
    return _back(scale, home), _back(xint, home), _back(sign, home)


def _grouped_asymmetric_quant(x, G, q_max):
    """scale = max(max - min, 1e-5) / q_max, zp = clamp(rne(-min / scale), 0, q_max),
    x_int = clamp(rne(fl(x / scale) + zp), 0, q_max) (quant/grouped.py:78-133).
    Returns (scale_row, zp_row, x_int)."""
    from ..sc.kernels import quantize
    x, home = _on_gpu(x)
    rows, cols = x.shape
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    zp = torch.empty(rows, dtype=torch.float32, device=x.device)
    xint = torch.empty((rows, cols), dtype=torch.float32, device=x.device)
    quantize(x, _lib.Q_GROUP_ASYM, int(q_max), 1, group=G, xint=xint, scale=scale, zp=zp)
    return _back(scale, home), _back(zp, home), _back(xint, home)


def _grouped_symmetric_quant_batched(x, G, q_max):
    """Batched (BH, rows, cols) symmetric quant for G == 1 (per row) or G >= rows (per
    batch) (quant/grouped.py:136-163). Returns (scale (BH, rows), x_int, sign)."""
    from ..sc.kernels import quantize
    assert x.dim() == 3, f"expected (BH, rows, cols), got {tuple(x.shape)}"
    BH, rows, cols = x.shape
    if G >= rows:
        g = rows
    elif G == 1:
        g = 1
    else:
        raise NotImplementedError(
            f"_grouped_symmetric_quant_batched: G={G} not supported "
            f"(use G=1 or G>=rows)")
    x, home = _on_gpu(x)
    scale = torch.empty((BH, rows), dtype=torch.float32, device=x.device)
    xint = torch.empty((BH, rows, cols), dtype=torch.float32, device=x.device)
    sign = torch.empty((BH, rows, cols), dtype=torch.int8, device=x.device)
    quantize(x.reshape(BH * rows, cols), _lib.Q_GROUP_SYM, int(q_max), 1, group=g,
             xint=xint, sign=sign, scale=scale)
    return _back(scale, home), _back(xint, home), _back(sign, home)


__all__ = [
    "_grouped_symmetric_quant",
    "_grouped_asymmetric_quant",
    "_grouped_symmetric_quant_batched",
]

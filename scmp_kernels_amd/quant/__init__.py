"""FP -> SC-domain quantization (the reference's scmp_kernels.quant surface,
scmp_kernels/quant/__init__.py:17-51).

* Bipolar  -> (boundary int16, sign int8, scale)
* Unipolar -> (boundary int32, scale, zp[, row_sum])
"""
from .fused import (
    fused_quant_kernel,
    fused_quant_bipolar_batched_kernel,
    fused_quantize_bipolar,
    fused_quantize_bipolar_perrow,
    fused_quantize_unipolar,
    _quant_dummy,
)
from .grouped import (
    _grouped_symmetric_quant,
    _grouped_asymmetric_quant,
    _grouped_symmetric_quant_batched,
)
from .smoothquant import (
    accumulate_act_scales,
    compute_smooth_scales,
    apply_smoothing,
    apply_smoothing_offline,
)

__all__ = [
    "fused_quant_kernel",
    "fused_quant_bipolar_batched_kernel",
    "fused_quantize_bipolar",
    "fused_quantize_bipolar_perrow",
    "fused_quantize_unipolar",
    "_quant_dummy",
    "_grouped_symmetric_quant",
    "_grouped_asymmetric_quant",
    "_grouped_symmetric_quant_batched",
    "accumulate_act_scales",
    "compute_smooth_scales",
    "apply_smoothing",
    "apply_smoothing_offline",
]

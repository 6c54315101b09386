"""scmp_kernels_amd: the stochastic-computing matmul of swalther06/scmp_kernels, built for
AMD Instinct MI355X (gfx950) with hand-written HIP kernels behind a C ABI
(include/scmp_hip.h, libscmp_hip.so).

Drop-in surface (same names, arguments and errors as the reference):
    scmp_kernels_amd.sc_matmul
    scmp_kernels_amd.sc.{sc_matmul, clear_rng_cache, det_kernel_tuning}
    scmp_kernels_amd.quant.{fused_quantize_*, _grouped_*_quant, SmoothQuant helpers}
    scmp_kernels_amd.mp.{MPConfig, RowAssignment, classify_rows_by_metric}
"""
from .sc import sc_matmul

__all__ = ["sc_matmul"]

"""Stochastic-computing matmul on MI355X (the reference's scmp_kernels.sc surface,
scmp_kernels/sc/__init__.py:20-27).

* ``sc_matmul`` — unified granularity dispatcher.
* ``clear_rng_cache`` — drop cached RNG sequences and stream tables.
* ``det_kernel_tuning`` — re-entrant context manager (API compatibility).
* ``prepare_weight`` / ``PreparedWeight`` — the per_row weight quantized once (no
  counterpart in the reference, which re-quantizes the weight on every call).
"""
from .matmul import sc_matmul
from .kernels import PreparedWeight, clear_rng_cache, det_kernel_tuning, prepare_weight

__all__ = ["sc_matmul", "clear_rng_cache", "det_kernel_tuning", "prepare_weight",
           "PreparedWeight"]

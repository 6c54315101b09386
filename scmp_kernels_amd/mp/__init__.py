"""Mixed precision: per-row stream-length assignment (the reference's scmp_kernels.mp
classifiers, scmp_kernels/mp/config.py) and the mixed-level per_row dispatch
``sc_matmul_mixed``. The reference's loggers and auto-calibrator are not provided."""
from .config import (
    AdaptiveMPConfig,
    FreeBoundaryMPConfig,
    MPConfig,
    RangeMPConfig,
    RowAssignment,
    adaptive_classify_rows,
    classify_groups_by_range,
    classify_rows_by_metric,
    get_current_block_idx,
    set_current_block_idx,
)
from .dispatch import sc_matmul_mixed

__all__ = [
    "MPConfig", "AdaptiveMPConfig", "FreeBoundaryMPConfig", "RangeMPConfig", "RowAssignment",
    "classify_rows_by_metric", "adaptive_classify_rows", "classify_groups_by_range",
    "set_current_block_idx", "get_current_block_idx", "sc_matmul_mixed",
]

"""Mixed-precision row assignment used by the mixed-length (rng_levels) SC path
(the reference's scmp_kernels/mp/config.py:42-191 subset on the hot path)."""
from .config import MPConfig, RowAssignment, classify_rows_by_metric

__all__ = ["MPConfig", "RowAssignment", "classify_rows_by_metric"]

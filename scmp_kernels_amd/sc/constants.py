"""Numeric range constants of the reference's quantization bookkeeping
(scmp_kernels/sc/constants.py): the largest finite values of the binary formats."""

FP8_E4M3_MAX = 448      # FP8 E4M3 (OCP)
FP8_E5M2_MAX = 57344    # FP8 E5M2
INT8_MAX = 127          # signed 8-bit, symmetric

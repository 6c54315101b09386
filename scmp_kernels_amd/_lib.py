"""ctypes binding of libscmp_hip.so (declared in include/scmp_hip.h).

The library is built in-tree by ``python -m scmp_kernels_amd.build`` (or
``__graft_entry__.build()``). There is no fallback: every SC entry point raises
``RuntimeError`` if the library is missing or cannot be loaded.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libscmp_hip.so")

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_float = ctypes.c_float
c_vp = ctypes.c_void_p

SCMP_OK = 0
SCMP_E_ARG = -1

# quantizer variants / modes (scmp_hip.h)
(Q_GROUP_SYM, Q_ROW_SYM, Q_TENSOR_SYM, Q_HEAD_SYM, Q_GROUP_ASYM, Q_TENSOR_ASYM, Q_HOST_SYM,
 Q_HOST_ASYM) = range(8)
SMOOTH_NONE, SMOOTH_DIV, SMOOTH_MUL = 0, 1, 2
CODE_NONE, CODE_THERMO, CODE_Q = 0, 1, 2
EPI_INT, EPI_ROWCOL, EPI_SCALAR, EPI_HEAD, EPI_ZP_ROWCOL, EPI_ZP_SCALAR = range(6)
GEMM_MFMA, GEMM_VALU, GEMM_MFMA_FP4 = 0, 1, 2
LFSR_SEARCH_MAX_BITS = 20          # SCMP_LFSR_SEARCH_MAX_BITS


class QuantArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_vp), ("rows", c_i64), ("cols", c_i64), ("ld", c_i64),
        ("smooth", c_vp), ("smooth_mode", c_int), ("variant", c_int),
        ("group", c_i64), ("seg", c_i64), ("q_max", c_int), ("rng_levels", c_int),
        ("host_inv", c_float), ("host_zp", c_float),
        ("code_kind", c_int), ("code", c_vp), ("code_ld", c_i64), ("code_rows", c_i64),
        ("code_batch_rows", c_i64),
        ("jtab", c_vp), ("col_class", c_vp),
        ("beta16", c_vp), ("beta32", c_vp), ("beta_formula", c_int), ("sign", c_vp),
        ("xint", c_vp), ("out_ld", c_i64), ("scale", c_vp), ("scale64", c_vp), ("inv", c_vp),
        ("zp", c_vp), ("zp64", c_vp), ("rowsum", c_vp), ("workspace", c_vp),
        ("row_index", c_vp), ("given_absmax", c_vp),
    ]


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("kind", c_int), ("c", c_float), ("sa", c_vp), ("sb", c_vp),
        ("sa_chunk_stride", c_i64), ("sb_chunk_stride", c_i64),
        ("sa_batch_stride", c_i64), ("sb_batch_stride", c_i64),
        ("s", c_vp), ("za", c_vp), ("zb", c_vp), ("suma", c_vp), ("sumb", c_vp),
        ("t3", c_vp), ("dfloat", c_float),
    ]


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("ca", c_vp), ("lda", c_i64), ("bsa", c_i64), ("cb", c_vp), ("ldb", c_i64),
        ("bsb", c_i64), ("N", c_i64), ("M", c_i64), ("D", c_i64), ("batch", c_i64),
        ("bipolar", c_int), ("JP", c_int), ("lut", c_vp), ("d_class", c_vp), ("chunk", c_i64),
        ("epi", Epilogue), ("y", c_vp), ("iout", c_vp), ("ldy", c_i64), ("bsy", c_i64),
        ("impl", c_int), ("bitlut", c_vp), ("tile", c_int), ("nclass", c_int),
        ("workspace", c_vp), ("workspace_bytes", c_i64), ("row_map", c_vp),
        ("group_class", c_vp),
    ]


EXPORTS = [
    "scmp_abi_version", "scmp_last_error", "scmp_rng_sobol", "scmp_rng_lfsr",
    "scmp_rng_expand", "scmp_rng_prepare", "scmp_lfsr_search", "scmp_build_stream_tables",
    "scmp_quant_workspace_bytes", "scmp_quantize", "scmp_quantize_pair", "scmp_sc_gemm",
    "scmp_build_bitlut",
    "scmp_build_fp4_lut", "scmp_sc_gemm_workspace_bytes", "scmp_permute_code_columns",
    "scmp_sc_gemm_noalloc",
]

SC_GEMM_NOALLOC_SCRATCH_BYTES = 129 << 20   # SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH):
    """Load (once) and return the library handle with argument types set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"scmp_kernels_amd: HIP library not found at {path}; build it with "
                f"`python -m scmp_kernels_amd.build` (gfx950).")
        lib = ctypes.CDLL(path)
        lib.scmp_abi_version.restype = c_int
        lib.scmp_last_error.restype = ctypes.c_char_p
        lib.scmp_rng_sobol.argtypes = [c_int, c_vp, c_i64, c_vp, c_vp]
        lib.scmp_rng_lfsr.argtypes = [c_int, c_i64, ctypes.c_uint64, c_i64, c_vp, c_vp]
        lib.scmp_rng_expand.argtypes = [c_vp, c_i64, c_vp, c_vp, c_int, c_int, c_vp, c_vp]
        lib.scmp_lfsr_search.argtypes = [c_int, c_vp, c_i64, c_vp, c_vp]
        lib.scmp_rng_prepare.argtypes = [c_vp, c_int, c_int, c_int, c_int, c_int, c_vp, c_int,
                                         c_vp, c_vp]
        lib.scmp_build_stream_tables.argtypes = [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int,
                                                 c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp]
        lib.scmp_quant_workspace_bytes.argtypes = [c_i64, c_i64, c_i64, c_i64]
        lib.scmp_quant_workspace_bytes.restype = c_i64
        lib.scmp_quantize.argtypes = [ctypes.POINTER(QuantArgs), c_vp]
        lib.scmp_quantize_pair.argtypes = [ctypes.POINTER(QuantArgs), ctypes.POINTER(QuantArgs),
                                           c_vp]
        lib.scmp_sc_gemm.argtypes = [ctypes.POINTER(GemmArgs), c_vp]
        lib.scmp_sc_gemm_noalloc.argtypes = [ctypes.POINTER(GemmArgs), c_vp]
        lib.scmp_sc_gemm_workspace_bytes.argtypes = [ctypes.POINTER(GemmArgs)]
        lib.scmp_sc_gemm_workspace_bytes.restype = c_i64
        lib.scmp_build_bitlut.argtypes = [c_vp, c_int, c_int, c_vp, c_vp]
        lib.scmp_build_fp4_lut.argtypes = [c_vp, c_int, c_int, c_vp, c_vp, c_vp]
        lib.scmp_permute_code_columns.argtypes = [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64,
                                                  c_vp]
        for name in EXPORTS:
            getattr(lib, name).restype = getattr(lib, name).restype or c_int
        lib.scmp_last_error.restype = ctypes.c_char_p
        lib.scmp_quant_workspace_bytes.restype = c_i64
        lib.scmp_sc_gemm_workspace_bytes.restype = c_i64
        _lib = lib
        return lib


def check(rc: int, what: str):
    """Map a negative return code to ValueError (bad arguments) or RuntimeError."""
    if rc == SCMP_OK:
        return
    msg = load().scmp_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def ptr(t) -> int:
    """Device pointer of a tensor (0 for None)."""
    return 0 if t is None else t.data_ptr()


def stream_of(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream

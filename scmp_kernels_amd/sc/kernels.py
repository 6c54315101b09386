"""Host orchestration of the SC matmul on gfx950 (PyTorch tensors for memory and streams,
libscmp_hip.so for every kernel).

Each path mirrors one host function of the reference (scmp_kernels/sc/kernels.py) and
keeps its numerics: the same quantizer variant, boundary grid, stream tables and fp32
epilogue order. The pipeline per call is

    quantize(a) -> A codes (thermometer lengths), quantize(b) -> B codes (q bytes)
    SC GEMM (int8 MFMA, exact int32 accumulator) -> fp32 epilogue

with SmoothQuant's a/s, b*s folded into the quantizer loads. Per-tensor ranges are
reduced on the device (no host synchronization); the scale products that the reference
forms in Python floats are formed in float64 on the device.

The FP->int quantizer API of the reference is re-exported here under its original names
(scmp_kernels/sc/kernels.py:42-52).
"""
from __future__ import annotations

import os
from typing import Optional

import numpy as np
import torch

from .. import _lib
from ..quant import (  # noqa: F401  (re-exports, scmp_kernels/sc/kernels.py:42-52)
    fused_quant_kernel,
    fused_quant_bipolar_batched_kernel,
    fused_quantize_bipolar,
    fused_quantize_bipolar_perrow,
    fused_quantize_unipolar,
    _quant_dummy,
    _grouped_symmetric_quant,
    _grouped_asymmetric_quant,
    _grouped_symmetric_quant_batched,
)
from . import tables as _tables
from .config_helpers import make_sobol_simple_config

ROW_PAD = 256      # GEMM workgroup tile rows: code buffers are padded to this


def clear_rng_cache():
    """Clear the cached RNG sequences and stream tables (kernels.py:90-94)."""
    _tables.clear()


def _resolve_rng_levels(sc_prec: int, rng_levels: Optional[int]) -> int:
    """scmp_kernels/sc/kernels.py:596-606."""
    if rng_levels is None:
        return 2 ** sc_prec
    return int(rng_levels)


# -------------------------------------------------------------------------------------
# det kernel tuning (scmp_kernels/sc/kernels.py:1728-1745): a re-entrant context manager
# that the reference never consults when choosing tiles; kept for API compatibility.
# -------------------------------------------------------------------------------------

_DET_KERNEL_TUNING_DEPTH = 0


class det_kernel_tuning:
    """Re-entrant context manager opting in to det-tuned tile selection (no effect on the
    results; tiles here are chosen by problem shape)."""

    def __enter__(self):
        global _DET_KERNEL_TUNING_DEPTH
        _DET_KERNEL_TUNING_DEPTH += 1
        return self

    def __exit__(self, *_):
        global _DET_KERNEL_TUNING_DEPTH
        _DET_KERNEL_TUNING_DEPTH -= 1


def _det_kernel_tuning_active() -> bool:
    return _DET_KERNEL_TUNING_DEPTH > 0


# -------------------------------------------------------------------------------------
# low-level launch helpers
# -------------------------------------------------------------------------------------

def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def _rows2d(x: torch.Tensor) -> torch.Tensor:
    """fp32 2-D view with unit column stride (copies only when needed)."""
    if x.dtype != torch.float32:
        x = x.float()
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    if x.stride(-1) != 1 or x.stride(0) < x.shape[1]:
        x = x.contiguous()
    return x


def _workspace(rows, cols, group, seg, device):
    nbytes = int(_lib.load().scmp_quant_workspace_bytes(rows, cols, group, seg))
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _quant_args(x: torch.Tensor, variant: int, q_max: int, rng_levels: int, *, group: int = 1,
                seg: int = 0, smooth: Optional[torch.Tensor] = None, smooth_mode: int = 0,
                code: Optional[torch.Tensor] = None, code_kind: int = 0,
                code_batch_rows: int = 0, jtab=None, col_class=None, beta16=None, beta32=None,
                beta_formula: int = 0, sign=None, xint=None, scale=None, scale64=None,
                inv=None, zp=None, zp64=None, rowsum=None, host_inv: float = 0.0,
                host_zp: float = 0.0, row_index=None, given_absmax=None):
    """The scmp_quant_args of one quantizer call, its workspace and its observer info."""
    x = _rows2d(x)
    rows, cols = x.shape
    if row_index is not None:
        rows = int(row_index.numel())
    G = rows if group <= 0 or group > rows else group
    a = _lib.QuantArgs()
    a.x, a.rows, a.cols, a.ld = x.data_ptr(), rows, cols, x.stride(0)
    a.smooth, a.smooth_mode = _lib.ptr(smooth), smooth_mode
    a.variant, a.group, a.seg = variant, G, seg
    a.q_max, a.rng_levels = q_max, rng_levels
    a.host_inv, a.host_zp = host_inv, host_zp
    a.code_kind, a.code = code_kind, _lib.ptr(code)
    if code is not None:
        a.code_ld, a.code_rows = code.shape[-1], code.shape[-2]
    a.code_batch_rows = code_batch_rows
    a.jtab, a.col_class = _lib.ptr(jtab), _lib.ptr(col_class)
    a.beta16, a.beta32, a.beta_formula = _lib.ptr(beta16), _lib.ptr(beta32), beta_formula
    a.sign, a.xint, a.out_ld = _lib.ptr(sign), _lib.ptr(xint), cols
    a.scale, a.scale64, a.inv = _lib.ptr(scale), _lib.ptr(scale64), _lib.ptr(inv)
    a.zp, a.zp64, a.rowsum = _lib.ptr(zp), _lib.ptr(zp64), _lib.ptr(rowsum)
    ws = _workspace(rows, cols, G, seg, x.device)
    a.workspace = ws.data_ptr()
    a.row_index = _lib.ptr(row_index)
    a.given_absmax = _lib.ptr(given_absmax)
    info = {"rows": rows, "cols": cols, "in_bytes": 4 * rows * cols,
            "code_bytes": 0 if code is None else code.numel(), "variant": variant}
    return a, ws, info, x.device


def quantize(x: torch.Tensor, variant: int, q_max: int, rng_levels: int, **kw):
    """One scmp_quantize call on the current stream; outputs are written in place (keywords
    as _quant_args). row_index (int64 device tensor): quantize rows x[row_index] in that
    order. given_absmax (float32 device tensor, one value per row group): the groups' max|x|
    from the caller instead of the reduction (symmetric variants)."""
    a, ws, info, dev = _quant_args(x, variant, q_max, rng_levels, **kw)
    if launch_observer is not None:
        _observe("pre", "quantize", info)
    _lib.check(_lib.load().scmp_quantize(a, _lib.stream_of(dev)), "scmp_quantize")
    if launch_observer is not None:
        _observe("post", "quantize", info)
    return ws  # keep the workspace alive until the stream has consumed it


def quantize_pair(first: tuple, second: tuple):
    """Two independent quantizer calls, each (x, variant, q_max, rng_levels, keywords), as
    one scmp_quantize_pair call: one launch when both are head-symmetric code-only calls of
    the dense shape (the first with thermometer codes, the second with byte codes), else
    the two calls in order (as two quantize calls when a row is not whole 4-column chunks,
    which the single launch never takes). Returns both workspaces."""
    if first[0].shape[-1] % 4 or second[0].shape[-1] % 4:
        return quantize(*first[:4], **first[4]), quantize(*second[:4], **second[4])
    a, ws1, i1, dev = _quant_args(*first[:4], **first[4])
    b, ws2, i2, _ = _quant_args(*second[:4], **second[4])
    info = None
    if launch_observer is not None:
        info = dict(i1)
        if i1["cols"] == i2["cols"]:
            info["rows"] = i1["rows"] + i2["rows"]
        info["in_bytes"] = i1["in_bytes"] + i2["in_bytes"]
        info["code_bytes"] = i1["code_bytes"] + i2["code_bytes"]
        _observe("pre", "quantize", info)
    _lib.check(_lib.load().scmp_quantize_pair(a, b, _lib.stream_of(dev)), "scmp_quantize_pair")
    if info is not None:
        _observe("post", "quantize", info)
    return ws1, ws2


def _gemm_impl() -> Optional[int]:
    """SCMP_GEMM_IMPL = fp4 | int8 | valu selects the SC GEMM kernel; unset: FP4 MFMA
    when the stream table fits e2m1, else int8 MFMA."""
    v = os.environ.get("SCMP_GEMM_IMPL", "").lower()
    return {"valu": _lib.GEMM_VALU, "int8": _lib.GEMM_MFMA, "mfma": _lib.GEMM_MFMA,
            "fp4": _lib.GEMM_MFMA_FP4}.get(v)


# LDS of one FP4 GEMM workgroup (gemm_fp4_kernel.h: kFp4MaxLds, kFactorFloats)
_FP4_MAX_LDS = 160 * 1024
_FP4_STAGE_BYTES = (5 * 128 + 3 * 512) * 4


def _fp4_class_runs(tabs: "_tables.StreamTables", D: int):
    """The class-run layout (StreamTables.class_runs) when the FP4 kernel should use it:
    several classes whose tables do not all fit in LDS, and runs padded by at most an
    eighth of D. SCMP_FP4_RUNS=0 keeps the per-d global-table path, =1 takes runs
    whenever they are legal."""
    env = os.environ.get("SCMP_FP4_RUNS", "")
    if env == "0" or tabs.nclass <= 1 or D != tabs.D:
        return None
    rowb = max(tabs.JP, 32) // 2
    tab = 256 * (8 if tabs.JP == 16 else 16 * ((rowb // 16) | 1))   # one table in LDS
    if env != "1" and tab * (1 + tabs.nclass) + _FP4_STAGE_BYTES <= _FP4_MAX_LDS:
        return None                              # every class table fits in LDS
    runs = tabs.class_runs()
    if runs[2] > 65536 or (env != "1" and runs[2] > D + D // 8):
        return None                              # the FP4 kernel's exact range: D <= 65536
    return runs


def _permute_codes(c: torch.Tensor, src: torch.Tensor, Dp: int, stream) -> torch.Tensor:
    """Code buffer with its columns in class-run order (scmp_permute_code_columns)."""
    shape = tuple(c.shape[:-1]) + (_round_up(Dp, 16),)
    out = torch.empty(shape, dtype=torch.uint8, device=c.device)
    rows = c.numel() // c.shape[-1]
    _lib.check(_lib.load().scmp_permute_code_columns(
        c.data_ptr(), rows, c.shape[-1], src.data_ptr(), Dp, out.data_ptr(), shape[-1],
        stream), "scmp_permute_code_columns")
    return out


# Observer of the library's launches: when set, called as observer(stage, kind, info) with
# stage "pre" / "post" right before and after each scmp_quantize / scmp_sc_gemm call
# (kind "quantize" / "sc_gemm"), on the thread that issues it, so that a profiler can
# record events on the launch stream around it. info holds the call's shape. None: off.
launch_observer = None


def _observe(stage, kind, info):
    obs = launch_observer
    if obs is not None:
        obs(stage, kind, info)


def sc_gemm(ca, cb, *, N, M, D, batch, tabs: "_tables.StreamTables", epi: "_lib.Epilogue",
            y=None, iout=None, ldy=None, bsy=0, chunk=0, d_class=None, impl=None, tile=None,
            row_map=None):
    """scmp_sc_gemm on the current stream. ca / cb are code buffers (batch, rows_pad, ld)
    or (rows_pad, ld)."""
    g, keep = sc_gemm_args(ca, cb, N=N, M=M, D=D, batch=batch, tabs=tabs, epi=epi, y=y,
                           iout=iout, ldy=ldy, bsy=bsy, chunk=chunk, d_class=d_class,
                           impl=impl, tile=tile, row_map=row_map)
    lib = _lib.load()
    ws = None
    nbytes = int(lib.scmp_sc_gemm_workspace_bytes(g))
    if nbytes > 0:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=ca.device)
        g.workspace, g.workspace_bytes = ws.data_ptr(), nbytes
    info = None
    if launch_observer is not None:
        info = {"N": N, "M": M, "D": D, "batch": max(batch, 1), "JP": tabs.JP,
                "impl": g.impl, "chunk": chunk, "epi": epi.kind}
        _observe("pre", "sc_gemm", info)
    _lib.check(lib.scmp_sc_gemm(g, _lib.stream_of(ca.device)), "scmp_sc_gemm")
    if info is not None:
        _observe("post", "sc_gemm", info)
    return ws, keep  # keep the buffers alive until the stream has consumed them


def sc_gemm_args(ca, cb, *, N, M, D, batch, tabs: "_tables.StreamTables",
                 epi: "_lib.Epilogue", y=None, iout=None, ldy=None, bsy=0, chunk=0,
                 d_class=None, impl=None, tile=None, row_map=None):
    """The scmp_gemm_args of one SC GEMM (workspace not yet attached) and the device
    buffers it points to, which must stay alive until the stream has consumed them.
    Chooses the kernel and, for the FP4 kernel with per-d classes, the class-run layout
    (launching the code permutation on the current stream)."""
    dev = ca.device
    stream = _lib.stream_of(dev)
    if impl is None:
        impl = _gemm_impl()
    if impl is None and D > 65536:
        impl = _lib.GEMM_MFMA  # the FP4 kernel's fp32 accumulator is exact up to 2^24
    if impl is None or impl == _lib.GEMM_MFMA_FP4:
        l4 = tabs.lut4(stream)
        if l4 is None and impl == _lib.GEMM_MFMA_FP4:
            raise ValueError("sc_matmul: the stream table has counts FP4 cannot represent")
        impl = _lib.GEMM_MFMA_FP4 if l4 is not None else _lib.GEMM_MFMA
    dc = d_class if d_class is not None else tabs.d_class
    gcls = None
    if impl == _lib.GEMM_MFMA_FP4 and d_class is None and not 0 < chunk < D:
        runs = _fp4_class_runs(tabs, D)
        if runs is not None:
            # every class's inner dimensions side by side (an exact integer sum in any
            # order), so the kernel holds one class table in LDS at a time
            src, gcls, D = runs
            ca = _permute_codes(ca, src, D, stream)
            cb = _permute_codes(cb, src, D, stream)
            dc = None
    g = _lib.GemmArgs()
    g.ca, g.lda = ca.data_ptr(), ca.shape[-1]
    g.bsa = ca.shape[-2] * ca.shape[-1] if ca.dim() == 3 else 0
    g.cb, g.ldb = cb.data_ptr(), cb.shape[-1]
    g.bsb = cb.shape[-2] * cb.shape[-1] if cb.dim() == 3 else 0
    g.N, g.M, g.D, g.batch = N, M, D, batch
    g.bipolar, g.JP = 1 if tabs.bipolar else 0, tabs.JP
    g.lut = tabs.lut4(stream).data_ptr() if impl == _lib.GEMM_MFMA_FP4 else tabs.lut.data_ptr()
    g.d_class = _lib.ptr(dc)
    g.group_class = _lib.ptr(gcls)
    g.nclass = tabs.nclass
    g.chunk = chunk
    g.epi = epi
    g.y, g.iout = _lib.ptr(y), _lib.ptr(iout)
    g.ldy = ldy if ldy is not None else M
    g.bsy = bsy
    g.impl = impl
    g.row_map = _lib.ptr(row_map)
    g.tile = int(os.environ.get("SCMP_GEMM_TILE", "0")) if tile is None else tile
    if g.impl == _lib.GEMM_VALU:
        g.bitlut = tabs.bitlut(stream).data_ptr()
    return g, (ca, cb)


def _codes(rows: int, D: int, device, batch: int = 0) -> torch.Tensor:
    """Uninitialized code buffer; the quantizer fills it including the zero padding."""
    shape = (_round_up(rows, ROW_PAD), _round_up(D, 16))
    if batch:
        shape = (batch,) + shape
    return torch.empty(shape, dtype=torch.uint8, device=device)


def _inner_scale(Q: int, L: int) -> float:
    """q_max_sq / stoc_len evaluated in fp32 (kernels.py:212)."""
    return float(np.float32(np.float32(Q * Q) / np.float32(L)))


def _get_tables(config, sc_prec, L, R, bipolar, D, device):
    return _tables.get_tables(config, ("sobol_simple", D, D, sc_prec),
                              lambda: make_sobol_simple_config(D, D, sc_prec),
                              sc_prec, L, R, bipolar, D, device)


def _smooth_args(smooth: Optional[torch.Tensor], side: str):
    if smooth is None:
        return None, _lib.SMOOTH_NONE
    return smooth, (_lib.SMOOTH_DIV if side == "a" else _lib.SMOOTH_MUL)


def _check_gpu(a: torch.Tensor):
    if not a.is_cuda:
        raise RuntimeError("scmp_kernels_amd: the SC kernels run on the GPU; got CPU tensors "
                           "and no GPU is available")


def _to_gpu(a: torch.Tensor, b: torch.Tensor):
    """CPU inputs are moved to the GPU and results back (kernels.py:1115-1117,
    1150-1151)."""
    if a.is_cuda:
        return a, b, None
    if not torch.cuda.is_available():
        raise RuntimeError("scmp_kernels_amd: the SC kernels run on the GPU; got CPU tensors "
                           "and no GPU is available")
    return a.cuda(), b.cuda(), a.device


# -------------------------------------------------------------------------------------
# Prepared weights: the B operand of the per_row path quantized once
# -------------------------------------------------------------------------------------

class PreparedWeight:
    """The B operand of the 2-D per_row path, quantized once: GEMM codes (the quantized
    integers as bytes), per-row scales and, for unipolar, zero-points and row sums. The
    codes do not depend on stoc_len, rng_levels or the RNG config, so one prepared weight
    serves every stream length (e.g. every level of a mixed-precision assignment).
    ``smooth_scales`` is the SmoothQuant vector baked in (b * s), or None."""

    def __init__(self, codes, scale, zp, rowsum, *, M, D, mode, sc_prec, group_b,
                 smooth_scales, device):
        self.codes, self.scale, self.zp, self.rowsum = codes, scale, zp, rowsum
        self.M, self.D, self.mode, self.sc_prec, self.group_b = M, D, mode, sc_prec, group_b
        self.smooth_scales = smooth_scales
        self.device = device

    @property
    def shape(self):
        return (self.M, self.D)

    def check(self, D: int, mode: str, sc_prec: int, group_b: int, smooth_scales):
        """ValueError unless this weight was prepared for these sc_matmul arguments."""
        if D != self.D:
            raise ValueError(f"sc_matmul: prepared weight has D={self.D}, a has D={D}")
        if (mode, sc_prec, group_b) != (self.mode, self.sc_prec, self.group_b):
            raise ValueError(
                f"sc_matmul: prepared weight was quantized for mode={self.mode!r}, "
                f"sc_prec={self.sc_prec}, group_b={self.group_b}; the call asks for "
                f"mode={mode!r}, sc_prec={sc_prec}, group_b={group_b}")
        mine = self.smooth_scales
        if (mine is None) != (smooth_scales is None):
            raise ValueError("sc_matmul: smooth_scales must be the vector the weight was "
                             "prepared with (or None for both)")
        if mine is not None and smooth_scales is not mine and not torch.equal(
                smooth_scales.to(device=mine.device, dtype=mine.dtype), mine):
            raise ValueError("sc_matmul: smooth_scales differ from the vector the weight "
                             "was prepared with")


@torch.no_grad()
def prepare_weight(b: torch.Tensor, *, mode: str = "bipolar", sc_prec: int = 8,
                   group_b: int = 1, smooth_scales: Optional[torch.Tensor] = None
                   ) -> PreparedWeight:
    """Quantize the weight ``b`` (M, D) of the per_row path once, with the grouped
    quantizer that _sc_matmul_per_row applies to b (scmp_kernels/sc/kernels.py:1661-1707),
    SmoothQuant's ``b * s`` folded into the load (scmp_kernels/quant/smoothquant.py:130-147).
    ``sc_matmul(a, w, "per_row", ...)`` then quantizes only ``a``."""
    if mode not in ("bipolar", "unipolar"):
        raise ValueError(f"Unknown mode: {mode}")
    if not 1 <= sc_prec <= 8:
        raise ValueError(f"sc_matmul: sc_prec={sc_prec} outside [1, 8]")
    if b.dim() != 2:
        raise ValueError(f"prepare_weight: expected a 2-D weight, got {b.dim()}-D")
    if not b.is_cuda:
        if not torch.cuda.is_available():
            raise RuntimeError("scmp_kernels_amd: the SC kernels run on the GPU; got a CPU "
                               "weight and no GPU is available")
        b = b.cuda()
    dev = b.device
    M, D = b.shape
    s = None
    if smooth_scales is not None:
        from ..quant.smoothquant import _check_smoothing_vector
        _check_smoothing_vector(smooth_scales, D, names=("b",))
        s = smooth_scales.to(device=dev, dtype=torch.float32).contiguous()
    cb = _codes(M, D, dev)
    sb = torch.empty(M, dtype=torch.float32, device=dev)
    zb = rb = None
    with torch.cuda.device(dev):
        if mode == "bipolar":
            Q = 2 ** (sc_prec - 1) - 1
            ws = quantize(b, _lib.Q_GROUP_SYM, Q, 2 ** sc_prec, group=group_b, smooth=s,
                          smooth_mode=_lib.SMOOTH_MUL if s is not None else 0, code=cb,
                          code_kind=_lib.CODE_Q, scale=sb)
        else:
            Q = 2 ** sc_prec - 1
            zb = torch.empty(M, dtype=torch.float32, device=dev)
            rb = torch.empty(M, dtype=torch.float32, device=dev)
            ws = quantize(b, _lib.Q_GROUP_ASYM, Q, 2 ** sc_prec, group=group_b, smooth=s,
                          smooth_mode=_lib.SMOOTH_MUL if s is not None else 0, code=cb,
                          code_kind=_lib.CODE_Q, scale=sb, zp=zb, rowsum=rb)
    del ws
    return PreparedWeight(cb, sb, zb, rb, M=M, D=D, mode=mode, sc_prec=sc_prec,
                          group_b=group_b, smooth_scales=smooth_scales, device=dev)


# -------------------------------------------------------------------------------------
# per_row, 2-D  (scmp_kernels/sc/kernels.py:1574-1707)
# -------------------------------------------------------------------------------------

@torch.no_grad()
def _sc_matmul_per_row(a, b, group_a=1, group_b=1, mode="unipolar", sc_prec=8, config=None,
                       stoc_len=None, rng_levels=None, smooth_scales=None):
    if stoc_len is None:
        stoc_len = 2 ** sc_prec
    prepared = isinstance(b, PreparedWeight)
    assert a.dim() == 2 and (prepared or b.dim() == 2), \
        f"Expected 2D, got a:{a.dim()}D b:{len(b.shape)}D"
    assert a.shape[1] == b.shape[1], f"Inner dim mismatch: {a.shape[1]} vs {b.shape[1]}"
    if mode not in ("bipolar", "unipolar"):
        raise ValueError(f"Unknown mode: {mode}")
    if prepared:
        a, home = _to_gpu_one(a, b.device)
        w = b
    else:
        a, b, home = _to_gpu(a, b)
        w = None
    R = _resolve_rng_levels(sc_prec, rng_levels)
    y = torch.empty((a.shape[0], b.shape[0]), dtype=torch.float32, device=a.device)
    _per_row_levels(a, b if w is None else w, [(stoc_len, R, None)], y, group_a=group_a,
                    group_b=group_b, mode=mode, sc_prec=sc_prec, config=config,
                    smooth_scales=smooth_scales)
    return y.to(home) if home is not None else y


def _to_gpu_one(a: torch.Tensor, device):
    """a on the prepared weight's device (CPU input: moved there, result moved back)."""
    home = None
    if not a.is_cuda:
        home = a.device
        a = a.to(device)
    elif a.device != device:
        raise ValueError(f"sc_matmul: a is on {a.device}, the prepared weight on {device}")
    return a, home


def _per_row_levels(a, b, levels, y, *, group_a, group_b, mode, sc_prec, config,
                    smooth_scales):
    """The 2-D per_row path (scmp_kernels/sc/kernels.py:1574-1707) for one or more stream
    lengths: ``levels`` is a list of (stoc_len, rng_levels, rows) with rows an int64 device
    tensor of rows of ``a`` (None: all rows). Each level quantizes a[rows] (read in place
    through the quantizer's row index, grouped in that order) at its own boundary grid and
    writes Y[rows] through the GEMM's row map; b (a tensor or a PreparedWeight) is quantized
    at most once."""
    dev = a.device
    D = a.shape[1]
    bip = mode == "bipolar"
    Q = 2 ** (sc_prec - 1) - 1 if bip else 2 ** sc_prec - 1
    s_a, m_a = _smooth_args(smooth_scales, "a")
    if isinstance(b, PreparedWeight):
        w = b
    else:
        w = prepare_weight(b, mode=mode, sc_prec=sc_prec, group_b=group_b,
                           smooth_scales=smooth_scales)
    M = w.M
    keep = []
    for stoc_len, R, rows in levels:
        N = a.shape[0] if rows is None else int(rows.numel())
        if N == 0:
            continue
        tabs = _get_tables(config, sc_prec, stoc_len, R, bip, D, dev)
        ca = _codes(N, D, dev)
        sa = torch.empty(N, dtype=torch.float32, device=dev)
        epi = _lib.Epilogue()
        epi.c = _inner_scale(Q, stoc_len)
        epi.sa, epi.sb = sa.data_ptr(), w.scale.data_ptr()
        if bip:
            wq = quantize(a, _lib.Q_GROUP_SYM, Q, R, group=group_a, smooth=s_a,
                          smooth_mode=m_a, code=ca, code_kind=_lib.CODE_THERMO,
                          jtab=tabs.jtab, col_class=tabs.d_class, scale=sa, row_index=rows)
            epi.kind = _lib.EPI_ROWCOL
            keep.append((ca, sa))
        else:
            za = torch.empty(N, dtype=torch.float32, device=dev)
            ra = torch.empty(N, dtype=torch.float32, device=dev)
            wq = quantize(a, _lib.Q_GROUP_ASYM, Q, R, group=group_a, smooth=s_a,
                          smooth_mode=m_a, code=ca, code_kind=_lib.CODE_THERMO,
                          jtab=tabs.jtab, col_class=tabs.d_class, scale=sa, zp=za,
                          rowsum=ra, row_index=rows)
            epi.kind = _lib.EPI_ZP_ROWCOL
            epi.za, epi.zb = za.data_ptr(), w.zp.data_ptr()
            epi.suma, epi.sumb = ra.data_ptr(), w.rowsum.data_ptr()
            epi.dfloat = float(np.float32(D))
            keep.append((ca, sa, za, ra))
        wg = sc_gemm(ca, w.codes, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, y=y,
                     ldy=y.stride(0), row_map=rows)
        keep.append((wq, wg))
    return keep


# -------------------------------------------------------------------------------------
# per_row + chunk_d (scmp_kernels/sc/kernels.py:1444-1566, 1274-1383)
# -------------------------------------------------------------------------------------

@torch.no_grad()
def _sc_matmul_per_row_mlp(a, b, max_fp_a=0.0, min_fp_a=0.0, max_fp_b=None, min_fp_b=None,
                           mode="bipolar", sc_prec=8, config=None, group_a=1, group_b=1,
                           chunk_d=0, stoc_len=None, rng_levels=None, *, smooth_scales=None):
    """scmp_kernels/sc/kernels.py:1444-1566, same parameters. Bipolar with chunk_d < D: the
    chunked path (one launch, per-chunk scales). Other bipolar calls: the row-group path of
    _sc_matmul_per_row (kernels.py:1548-1553; group sizes <= 0 mean 1). Unipolar: per-tensor
    quantization with the caller's ranges (max_fp_b / min_fp_b default to a's), which is
    _sc_matmul_per_tensor's (kernels.py:1386-1418). 3-D: each batch with the ranges and
    without groups or chunks (kernels.py:1421-1441)."""
    if stoc_len is None:
        stoc_len = 2 ** sc_prec
    if max_fp_b is None:
        max_fp_b = max_fp_a
    if min_fp_b is None:
        min_fp_b = min_fp_a
    if a.dim() == 3:
        out = torch.empty((a.shape[0], a.shape[1], b.shape[1]), dtype=torch.float32,
                          device=a.device)
        for i in range(a.shape[0]):
            out[i] = _sc_matmul_per_row_mlp(a[i], b[i], max_fp_a, min_fp_a, max_fp_b,
                                            min_fp_b, mode, sc_prec, config, stoc_len=stoc_len,
                                            rng_levels=rng_levels, smooth_scales=smooth_scales)
        return out
    assert a.dim() == 2 and b.dim() == 2, f"Expected 2D, got a:{a.dim()}D b:{b.dim()}D"
    assert a.shape[1] == b.shape[1], f"Dim mismatch: a={a.shape[1]}, b={b.shape[1]}"
    N, D = a.shape
    if mode == "unipolar":
        return _sc_matmul_per_tensor(a, b, max_fp_a, min_fp_a, max_fp_b, min_fp_b,
                                     mode=mode, sc_prec=sc_prec, config=config,
                                     stoc_len=stoc_len, rng_levels=rng_levels,
                                     smooth_scales=smooth_scales)
    if mode != "bipolar":
        raise ValueError(f"Unknown mode: {mode}")
    if not (chunk_d > 0 and D > chunk_d):
        # standard path: the grouped quantizer arithmetic of _sc_matmul_per_row
        return _sc_matmul_per_row(a, b, group_a=max(group_a, 1), group_b=max(group_b, 1),
                                  mode=mode, sc_prec=sc_prec, config=config,
                                  stoc_len=stoc_len, rng_levels=rng_levels,
                                  smooth_scales=smooth_scales)
    a, b, home = _to_gpu(a, b)
    M = b.shape[0]
    dev = a.device
    R = _resolve_rng_levels(sc_prec, rng_levels)
    Q = 2 ** (sc_prec - 1) - 1
    # Tables of at most 32 intervals put two inner dimensions in one MFMA k-step (both
    # kernels), so a chunk must end on an even d; for an odd chunk_d the table is widened
    # to 64 intervals (empty past the attainable ones: the same sums), one d per k-step.
    tabs = _tables.get_tables(config, ("sobol_simple", chunk_d, chunk_d, sc_prec),
                              lambda: make_sobol_simple_config(chunk_d, chunk_d, sc_prec),
                              sc_prec, stoc_len, R, True, chunk_d, dev,
                              min_jp=64 if chunk_d % 2 else 16)
    impl = _gemm_impl()
    if impl == _lib.GEMM_VALU:
        impl = None                    # the VALU kernel has no chunked accumulation
    # dimension d of every chunk uses the tables of local index d mod chunk_d
    d_class = None
    if tabs.nclass > 1:
        d_class = torch.from_numpy(tabs.class_of[np.arange(D) % chunk_d]).to(dev)
    nseg = (D + chunk_d - 1) // chunk_d
    ca, cb = _codes(N, D, dev), _codes(M, D, dev)
    sa = torch.empty((nseg, N), dtype=torch.float32, device=dev)
    sb = torch.empty((nseg, M), dtype=torch.float32, device=dev)
    s_a, m_a = _smooth_args(smooth_scales, "a")
    s_b, m_b = _smooth_args(smooth_scales, "b")
    w1 = quantize(a, _lib.Q_ROW_SYM, Q, R, group=1, seg=chunk_d, smooth=s_a, smooth_mode=m_a,
                  code=ca, code_kind=_lib.CODE_THERMO, jtab=tabs.jtab, col_class=d_class,
                  scale=sa)
    w2 = quantize(b, _lib.Q_ROW_SYM, Q, R, group=1, seg=chunk_d, smooth=s_b, smooth_mode=m_b,
                  code=cb, code_kind=_lib.CODE_Q, scale=sb)
    y = torch.empty((N, M), dtype=torch.float32, device=dev)
    epi = _lib.Epilogue()
    epi.kind, epi.c = _lib.EPI_ROWCOL, _inner_scale(Q, stoc_len)
    epi.sa, epi.sb = sa.data_ptr(), sb.data_ptr()
    epi.sa_chunk_stride, epi.sb_chunk_stride = N, M
    sc_gemm(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, y=y, chunk=chunk_d,
            d_class=d_class, impl=impl)
    del w1, w2
    return y.to(home) if home is not None else y


# -------------------------------------------------------------------------------------
# per_row, 3-D (scmp_kernels/sc/kernels.py:1779-1895)
# -------------------------------------------------------------------------------------

@torch.no_grad()
def _sc_matmul_per_row_batched(a, b, group_a=1, group_b=1, mode="bipolar", sc_prec=8,
                               config=None, stoc_len=None, rng_levels=None,
                               smooth_scales=None):
    assert a.dim() == 3 and b.dim() == 3, f"Expected 3D, got a:{a.dim()}D b:{b.dim()}D"
    BH, Ma, D = a.shape
    BH_b, Nb, D_b = b.shape
    assert BH == BH_b, f"batch mismatch: a BH={BH} vs b BH={BH_b}"
    assert D == D_b, f"inner-dim mismatch: a D={D} vs b D={D_b}"
    if stoc_len is None:
        stoc_len = 2 ** sc_prec
    a, b, home = _to_gpu(a, b)
    dev = a.device
    if mode == "unipolar":
        out = torch.empty((BH, Ma, Nb), dtype=torch.float32, device=dev)
        for i in range(BH):
            out[i] = _sc_matmul_per_row(a[i], b[i], group_a=group_a, group_b=group_b,
                                        mode=mode, sc_prec=sc_prec, config=config,
                                        stoc_len=stoc_len, rng_levels=rng_levels,
                                        smooth_scales=smooth_scales)
        return out.to(home) if home is not None else out
    if mode != "bipolar":
        raise ValueError(f"Unknown mode: {mode}")

    def group_of(G, rows):
        if G >= rows:
            return rows
        if G == 1:
            return 1
        raise NotImplementedError(
            f"_grouped_symmetric_quant_batched: G={G} not supported (use G=1 or G>=rows)")

    ga, gb = group_of(group_a, Ma), group_of(group_b, Nb)
    R = _resolve_rng_levels(sc_prec, rng_levels)
    Q = 2 ** (sc_prec - 1) - 1
    tabs = _get_tables(config, sc_prec, stoc_len, R, True, D, dev)
    ca, cb = _codes(Ma, D, dev, batch=BH), _codes(Nb, D, dev, batch=BH)
    sa = torch.empty(BH * Ma, dtype=torch.float32, device=dev)
    sb = torch.empty(BH * Nb, dtype=torch.float32, device=dev)
    s_a, m_a = _smooth_args(smooth_scales, "a")
    s_b, m_b = _smooth_args(smooth_scales, "b")
    w1 = quantize(a.reshape(BH * Ma, D), _lib.Q_GROUP_SYM, Q, R, group=ga, smooth=s_a,
                  smooth_mode=m_a, code=ca, code_kind=_lib.CODE_THERMO, code_batch_rows=Ma,
                  jtab=tabs.jtab, col_class=tabs.d_class, scale=sa)
    w2 = quantize(b.reshape(BH * Nb, D), _lib.Q_GROUP_SYM, Q, R, group=gb, smooth=s_b,
                  smooth_mode=m_b, code=cb, code_kind=_lib.CODE_Q, code_batch_rows=Nb,
                  scale=sb)
    y = torch.empty((BH, Ma, Nb), dtype=torch.float32, device=dev)
    epi = _lib.Epilogue()
    # acc *= inner_scale * 1.0 (head scale of ones, kernels.py:1877-1892) == fl(I * c)
    epi.kind, epi.c = _lib.EPI_ROWCOL, _inner_scale(Q, stoc_len)
    epi.sa, epi.sb = sa.data_ptr(), sb.data_ptr()
    epi.sa_batch_stride, epi.sb_batch_stride = Ma, Nb
    sc_gemm(ca, cb, N=Ma, M=Nb, D=D, batch=BH, tabs=tabs, epi=epi, y=y, bsy=Ma * Nb)
    del w1, w2
    return y.to(home) if home is not None else y


# -------------------------------------------------------------------------------------
# per_head bipolar (scmp_kernels/sc/kernels.py:440-585)
# -------------------------------------------------------------------------------------

def _head_absmax(maxs, mins, BH, dev, name):
    """max(|max|, |min|) per head (kernels.py:490-491; the 1e-5 clamp is the quantizer's)."""
    mx = torch.as_tensor(maxs, device=dev).reshape(-1).float()
    mn = torch.as_tensor(mins, device=dev).reshape(-1).float()
    if mx.numel() != BH or mn.numel() != BH:
        raise ValueError(f"_sc_matmul_per_head_bipolar: {name}_maxs / {name}_mins need one "
                         f"value per head ({BH}), got {mx.numel()} and {mn.numel()}")
    return torch.maximum(mx.abs(), mn.abs()).contiguous()


@torch.no_grad()
def _sc_matmul_per_head_bipolar(q_flat, k_flat, q_maxs=None, q_mins=None, k_maxs=None,
                                k_mins=None, sc_prec=8, config=None, stoc_len=None,
                                rng_levels=None, *, smooth_scales=None):
    """scmp_kernels/sc/kernels.py:440-585, same parameters: q_maxs / q_mins / k_maxs /
    k_mins are the (BH,) per-head ranges the quantizers scale by. None (this build's
    sc_matmul) takes each head's own max and min, reduced on the device, which is what the
    reference's sc_matmul passes (sc/matmul.py:271-274)."""
    if stoc_len is None:
        stoc_len = 2 ** sc_prec
    BH, N, D = q_flat.shape
    BH_k, M, D_k = k_flat.shape
    if BH_k != BH or D_k != D:
        raise ValueError(
            f"_sc_matmul_per_head_bipolar: shape mismatch — q is (BH={BH}, N={N}, D={D}), "
            f"k is (BH={BH_k}, M={M}, D={D_k}); require equal BH and D.")
    given = [r is not None for r in (q_maxs, q_mins, k_maxs, k_mins)]
    if any(given) and not all(given):
        raise ValueError("_sc_matmul_per_head_bipolar: give all four of q_maxs, q_mins, "
                         "k_maxs, k_mins, or none")
    q_flat, k_flat, home = _to_gpu(q_flat, k_flat)
    dev = q_flat.device
    gq = gk = None
    if all(given):
        gq = _head_absmax(q_maxs, q_mins, BH, dev, "q")
        gk = _head_absmax(k_maxs, k_mins, BH, dev, "k")
    Q = 2 ** (sc_prec - 1) - 1
    R = _resolve_rng_levels(sc_prec, rng_levels)
    tabs = _tables.get_tables(config, ("sobol_simple", D, D, sc_prec),
                              lambda: make_sobol_simple_config(D, D, sc_prec),
                              sc_prec, stoc_len, R, True, D, dev)
    ca, cb = _codes(N, D, dev, batch=BH), _codes(M, D, dev, batch=BH)
    sq = torch.empty(BH * N, dtype=torch.float32, device=dev)
    sk = torch.empty(BH * M, dtype=torch.float32, device=dev)
    s_a, m_a = _smooth_args(smooth_scales, "a")
    s_b, m_b = _smooth_args(smooth_scales, "b")
    # both quantizer calls in one launch when their shapes allow (the library checks)
    w1, w2 = quantize_pair(
        (q_flat.reshape(BH * N, D), _lib.Q_HEAD_SYM, Q, R,
         dict(group=N, smooth=s_a, smooth_mode=m_a, code=ca, code_kind=_lib.CODE_THERMO,
              code_batch_rows=N, jtab=tabs.jtab, col_class=tabs.d_class, scale=sq,
              given_absmax=gq)),
        (k_flat.reshape(BH * M, D), _lib.Q_HEAD_SYM, Q, R,
         dict(group=M, smooth=s_b, smooth_mode=m_b, code=cb, code_kind=_lib.CODE_Q,
              code_batch_rows=M, scale=sk, given_absmax=gk)))
    # out_scale = scale_q * scale_k (kernels.py:550), fp32: the kernel multiplies the
    # head's first row scales (every row of a head has the head's scale)
    y = torch.empty((BH, N, M), dtype=torch.float32, device=dev)
    epi = _lib.Epilogue()
    epi.kind, epi.c = _lib.EPI_HEAD, _inner_scale(Q, stoc_len)
    epi.sa, epi.sb = sq.data_ptr(), sk.data_ptr()
    epi.sa_batch_stride, epi.sb_batch_stride = N, M
    sc_gemm(ca, cb, N=N, M=M, D=D, batch=BH, tabs=tabs, epi=epi, y=y, bsy=N * M)
    del w1, w2
    return y.to(home) if home is not None else y


# -------------------------------------------------------------------------------------
# per_tensor (scmp_kernels/sc/kernels.py:1054-1226), ranges reduced on the device
# -------------------------------------------------------------------------------------

def _host_scales(max_fp, min_fp, mode, Q):
    """The reference's Python-float scale math for a caller's range: bipolar
    (scale, 1 / scale, 0) from max(|max|, |min|, 1e-5) (kernels.py:1173-1176,
    quant/fused.py:172-174); unipolar (scale, 1 / scale, zp) (quant/fused.py:204-209)."""
    max_fp, min_fp = float(max_fp), float(min_fp)
    if mode == "bipolar":
        scale = max(abs(max_fp), abs(min_fp), 1e-5) / Q
        return scale, 1.0 / scale, 0.0
    scale = max(max_fp - min_fp, 1e-5) / Q
    zp = float(max(0, min(Q, round(-min_fp / scale))))
    return scale, 1.0 / scale, zp


@torch.no_grad()
def _sc_matmul_per_tensor(a, b, max_fp_a=None, min_fp_a=None, max_fp_b=None, min_fp_b=None,
                          mode="bipolar", sc_prec=8, config=None, stoc_len=None,
                          rng_levels=None, *, smooth_scales=None):
    """scmp_kernels/sc/kernels.py:1054-1153, same parameters. Given ranges are used as the
    reference uses them (Python-float scales; b's default to a's; a 3-D call uses them for
    every batch). None (this build's sc_matmul) reduces the whole tensors' max and min on
    the device, which is what the reference's sc_matmul passes (sc/matmul.py:214-225), with
    the scale math in float64 on the device and no host sync."""
    if stoc_len is None:
        stoc_len = 2 ** sc_prec
    if (max_fp_a is None) != (min_fp_a is None):
        raise ValueError("_sc_matmul_per_tensor: give both max_fp_a and min_fp_a, or neither")
    if max_fp_a is None and (max_fp_b is not None or min_fp_b is not None):
        raise ValueError("_sc_matmul_per_tensor: b's range needs a's (max_fp_a, min_fp_a)")
    host = max_fp_a is not None
    if host:
        if max_fp_b is None:
            max_fp_b = max_fp_a
        if min_fp_b is None:
            min_fp_b = min_fp_a
    if a.dim() == 3:
        BH, N, D = a.shape
        M = b.shape[1]
        batch = BH
    else:
        assert a.dim() == 2 and b.dim() == 2, f"Expected 2D, got a:{a.dim()}D b:{b.dim()}D"
        assert a.shape[1] == b.shape[1], f"Dim mismatch: a={a.shape[1]}, b={b.shape[1]}"
        N, D = a.shape
        M = b.shape[0]
        batch = 0
    if mode not in ("bipolar", "unipolar"):
        raise ValueError(f"Unknown mode: {mode}")
    a, b, home = _to_gpu(a, b)
    dev = a.device
    R = _resolve_rng_levels(sc_prec, rng_levels)
    bip = mode == "bipolar"
    tabs = _get_tables(config, sc_prec, stoc_len, R, bip, D, dev)
    nb = max(batch, 1)
    ca, cb = _codes(N, D, dev, batch=batch), _codes(M, D, dev, batch=batch)
    a2, b2 = a.reshape(nb * N, D), b.reshape(nb * M, D)
    s_a, m_a = _smooth_args(smooth_scales, "a")
    s_b, m_b = _smooth_args(smooth_scales, "b")
    sa64 = torch.empty(1, dtype=torch.float64, device=dev)
    sb64 = torch.empty(1, dtype=torch.float64, device=dev)
    y = torch.empty((batch, N, M) if batch else (N, M), dtype=torch.float32, device=dev)
    epi = _lib.Epilogue()
    if host:
        Q = 2 ** (sc_prec - 1) - 1 if bip else 2 ** sc_prec - 1
        sca, inva, zpa = _host_scales(max_fp_a, min_fp_a, mode, Q)
        scb, invb, zpb = _host_scales(max_fp_b, min_fp_b, mode, Q)
        var = _lib.Q_HOST_SYM if bip else _lib.Q_HOST_ASYM
        za = zb = ra = rb = None
        if not bip:
            za = torch.empty(nb * N, dtype=torch.float32, device=dev)
            zb = torch.empty(nb * M, dtype=torch.float32, device=dev)
            ra = torch.empty(nb * N, dtype=torch.float32, device=dev)
            rb = torch.empty(nb * M, dtype=torch.float32, device=dev)
        w1 = quantize(a2, var, Q, R, smooth=s_a, smooth_mode=m_a, code=ca,
                      code_kind=_lib.CODE_THERMO, code_batch_rows=N if batch else 0,
                      jtab=tabs.jtab, col_class=tabs.d_class, host_inv=inva, host_zp=zpa,
                      zp=za, rowsum=ra)
        w2 = quantize(b2, var, Q, R, smooth=s_b, smooth_mode=m_b, code=cb,
                      code_kind=_lib.CODE_Q, code_batch_rows=M if batch else 0, host_inv=invb,
                      host_zp=zpb, zp=zb, rowsum=rb)
        # Python-float products, rounded to fp32 where torch multiplies (kernels.py:1202-1204)
        s = torch.tensor([sca * scb], dtype=torch.float32).to(dev)
        epi.c, epi.s = _inner_scale(Q, stoc_len), s.data_ptr()
        if bip:
            epi.kind = _lib.EPI_SCALAR
        else:
            t3 = torch.tensor([D * zpa * zpb], dtype=torch.float32).to(dev)
            epi.kind = _lib.EPI_ZP_SCALAR
            epi.za, epi.zb, epi.t3 = za.data_ptr(), zb.data_ptr(), t3.data_ptr()
            epi.suma, epi.sumb = ra.data_ptr(), rb.data_ptr()
            epi.sa_batch_stride, epi.sb_batch_stride = N, M
        sc_gemm(ca, cb, N=N, M=M, D=D, batch=nb, tabs=tabs, epi=epi, y=y, bsy=N * M)
    elif bip:
        Q = 2 ** (sc_prec - 1) - 1
        w1 = quantize(a2, _lib.Q_TENSOR_SYM, Q, R, smooth=s_a, smooth_mode=m_a, code=ca,
                      code_kind=_lib.CODE_THERMO, code_batch_rows=N if batch else 0,
                      jtab=tabs.jtab, col_class=tabs.d_class, scale64=sa64)
        w2 = quantize(b2, _lib.Q_TENSOR_SYM, Q, R, smooth=s_b, smooth_mode=m_b, code=cb,
                      code_kind=_lib.CODE_Q, code_batch_rows=M if batch else 0, scale64=sb64)
        s = (sa64 * sb64).float()          # Python-float product -> fp32 (kernels.py:1204)
        epi.kind, epi.c, epi.s = _lib.EPI_SCALAR, _inner_scale(Q, stoc_len), s.data_ptr()
        sc_gemm(ca, cb, N=N, M=M, D=D, batch=nb, tabs=tabs, epi=epi, y=y, bsy=N * M)
    else:
        Q = 2 ** sc_prec - 1
        za = torch.empty(nb * N, dtype=torch.float32, device=dev)
        zb = torch.empty(nb * M, dtype=torch.float32, device=dev)
        za64 = torch.empty(1, dtype=torch.float64, device=dev)
        zb64 = torch.empty(1, dtype=torch.float64, device=dev)
        ra = torch.empty(nb * N, dtype=torch.float32, device=dev)
        rb = torch.empty(nb * M, dtype=torch.float32, device=dev)
        w1 = quantize(a2, _lib.Q_TENSOR_ASYM, Q, R, smooth=s_a, smooth_mode=m_a, code=ca,
                      code_kind=_lib.CODE_THERMO, code_batch_rows=N if batch else 0,
                      jtab=tabs.jtab, col_class=tabs.d_class, scale64=sa64, zp=za,
                      zp64=za64, rowsum=ra)
        w2 = quantize(b2, _lib.Q_TENSOR_ASYM, Q, R, smooth=s_b, smooth_mode=m_b, code=cb,
                      code_kind=_lib.CODE_Q, code_batch_rows=M if batch else 0, scale64=sb64,
                      zp=zb, zp64=zb64, rowsum=rb)
        s = (sa64 * sb64).float()
        t3 = ((D * za64) * zb64).float()   # Python float D * zp_a * zp_b (kernels.py:1202)
        epi.kind, epi.c = _lib.EPI_ZP_SCALAR, _inner_scale(Q, stoc_len)
        epi.s, epi.za, epi.zb, epi.t3 = s.data_ptr(), za.data_ptr(), zb.data_ptr(), t3.data_ptr()
        epi.suma, epi.sumb = ra.data_ptr(), rb.data_ptr()
        epi.sa_batch_stride, epi.sb_batch_stride = N, M
        sc_gemm(ca, cb, N=N, M=M, D=D, batch=nb, tabs=tabs, epi=epi, y=y, bsy=N * M)
    del w1, w2
    return y.to(home) if home is not None else y

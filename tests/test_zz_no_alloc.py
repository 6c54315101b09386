"""scmp_sc_gemm_noalloc (the SC GEMM with the library's static scratch as its split-tile
workspace) against scmp_sc_gemm with a caller-allocated workspace: bit-identical outputs on
two calls in a row, the second on a smaller problem, both large enough that the FP4 kernel
shares tiles between workgroups (so the scratch is really used)."""
import ctypes

import numpy as np
import pytest
import torch

from scmp_kernels_amd import _lib


def _dev():
    return torch.device("cuda:0")


def _gemm_inputs(N, M, D, L, seed):
    """Codes, tables and epilogue of one per_row bipolar SC GEMM (the sc_matmul path)."""
    from scmp_kernels_amd.sc import kernels as K
    dev = _dev()
    rng = np.random.default_rng(seed)
    a = torch.from_numpy(rng.standard_normal((N, D)).astype(np.float32)).to(dev)
    b = torch.from_numpy((rng.standard_normal((M, D)) * 0.02).astype(np.float32)).to(dev)
    tabs = K._get_tables(None, 8, L, L, True, D, dev)
    ca, cb = K._codes(N, D, dev), K._codes(M, D, dev)
    sa = torch.empty(N, dtype=torch.float32, device=dev)
    sb = torch.empty(M, dtype=torch.float32, device=dev)
    keep = [K.quantize(a, _lib.Q_GROUP_SYM, 127, L, code=ca, code_kind=_lib.CODE_THERMO,
                       jtab=tabs.jtab, col_class=tabs.d_class, scale=sa),
            K.quantize(b, _lib.Q_GROUP_SYM, 127, L, code=cb, code_kind=_lib.CODE_Q, scale=sb),
            ca, cb, sa, sb]
    epi = _lib.Epilogue()
    epi.kind, epi.c = _lib.EPI_ROWCOL, K._inner_scale(127, L)
    epi.sa, epi.sb = sa.data_ptr(), sb.data_ptr()
    return ca, cb, tabs, epi, keep


def _run_both(N, M, D, L, seed):
    from scmp_kernels_amd.sc import kernels as K
    lib = _lib.load()
    dev = _dev()
    stream = _lib.stream_of(dev)
    ca, cb, tabs, epi, keep = _gemm_inputs(N, M, D, L, seed)
    y_ref = torch.full((N, M), float("nan"), dtype=torch.float32, device=dev)
    y_na = torch.full((N, M), float("nan"), dtype=torch.float32, device=dev)

    g, k1 = K.sc_gemm_args(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, y=y_ref)
    assert g.impl == _lib.GEMM_MFMA_FP4
    need = int(lib.scmp_sc_gemm_workspace_bytes(g))
    assert 0 < need <= _lib.SC_GEMM_NOALLOC_SCRATCH_BYTES, need   # tiles are shared
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    g.workspace, g.workspace_bytes = ws.data_ptr(), need
    _lib.check(lib.scmp_sc_gemm(g, stream), "scmp_sc_gemm")

    g2, k2 = K.sc_gemm_args(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, y=y_na)
    assert g2.workspace is None and g2.workspace_bytes == 0
    _lib.check(lib.scmp_sc_gemm_noalloc(g2, stream), "scmp_sc_gemm_noalloc")
    torch.cuda.synchronize()
    ref, got = y_ref.cpu().numpy(), y_na.cpu().numpy()
    del ws, keep, k1, k2
    assert np.isfinite(ref).all() and np.abs(ref).max() > 0
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    return need


@pytest.mark.gpu
def test_noalloc_gemm_equals_workspace_gemm_twice():
    print("noalloc: call 1, per_row bipolar 1000 x 1500 x 1024, L=256", flush=True)
    need1 = _run_both(1000, 1500, 1024, 256, seed=11)
    print("noalloc: call 2, per_row bipolar 300 x 700 x 640, L=64", flush=True)
    need2 = _run_both(300, 700, 640, 64, seed=12)
    assert need2 < need1


@pytest.mark.gpu
def test_noalloc_gemm_without_shared_tiles_and_rejections():
    """A problem that shares no tiles (no workspace needed) runs too; a caller-supplied
    workspace is refused before any device work."""
    print("noalloc: per_row bipolar 200 x 96 x 200 (whole tiles)", flush=True)
    from scmp_kernels_amd.sc import kernels as K
    lib = _lib.load()
    dev = _dev()
    stream = _lib.stream_of(dev)
    N, M, D, L = 200, 96, 200, 256
    ca, cb, tabs, epi, keep = _gemm_inputs(N, M, D, L, seed=13)
    y1 = torch.empty((N, M), dtype=torch.float32, device=dev)
    y2 = torch.empty((N, M), dtype=torch.float32, device=dev)
    g, k1 = K.sc_gemm_args(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, y=y1)
    assert int(lib.scmp_sc_gemm_workspace_bytes(g)) == 0
    _lib.check(lib.scmp_sc_gemm(g, stream), "scmp_sc_gemm")
    g2, k2 = K.sc_gemm_args(ca, cb, N=N, M=M, D=D, batch=1, tabs=tabs, epi=epi, y=y2)
    _lib.check(lib.scmp_sc_gemm_noalloc(g2, stream), "scmp_sc_gemm_noalloc")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y2.cpu().numpy().view(np.uint32),
                                  y1.cpu().numpy().view(np.uint32))
    g2.workspace, g2.workspace_bytes = ca.data_ptr(), 16
    assert lib.scmp_sc_gemm_noalloc(g2, stream) == _lib.SCMP_E_ARG
    assert b"workspace must be NULL" in lib.scmp_last_error()
    del keep, k1, k2


def test_noalloc_rejects_problems_beyond_the_scratch():
    """A problem whose split-tile workspace exceeds the static scratch is refused with
    SCMP_E_ARG before any device call (runs without a GPU: nothing is launched)."""
    lib = _lib.load()
    dummy = ctypes.c_void_p(256)          # never dereferenced: the size check rejects first
    g = _lib.GemmArgs()
    g.ca = g.cb = g.lut = g.y = dummy.value
    # 16 x 17 tiles per batch entry, 4001 entries: 1.09M tiles (4.4 MB of tile counters),
    # not a multiple of the workgroup count, so tiles are shared
    g.N, g.M, g.D, g.batch = 4096, 4352, 1024, 4001
    g.lda = g.ldb = 1024
    g.JP, g.ldy = 128, 4352
    g.epi.kind = _lib.EPI_ROWCOL
    g.impl = _lib.GEMM_MFMA_FP4
    assert int(lib.scmp_sc_gemm_workspace_bytes(g)) > _lib.SC_GEMM_NOALLOC_SCRATCH_BYTES
    assert lib.scmp_sc_gemm_noalloc(g, None) == _lib.SCMP_E_ARG
    assert b"static scratch" in lib.scmp_last_error()

"""The drop-in call surface, following the reference's tests/test_sc_smoke.py: imports,
output shape and dtype per granularity (GPU), the ValueError gates (CPU: they fire before
any kernel), the device guard, determinism across calls and cache clears, and the
loud failure when no GPU / HIP library is available."""
import numpy as np
import pytest
import torch

from scmp_kernels_amd import sc_matmul


def _have_gpu():
    return torch.cuda.is_available()


def test_import_surface():
    import scmp_kernels_amd
    from scmp_kernels_amd.sc import sc_matmul as s2, det_kernel_tuning, clear_rng_cache  # noqa
    from scmp_kernels_amd.sc import kernels as K
    from scmp_kernels_amd import quant as Qm
    from scmp_kernels_amd.mp import MPConfig, RowAssignment, classify_rows_by_metric  # noqa
    assert scmp_kernels_amd.sc_matmul is s2
    # the reference's re-exports from sc.kernels (scmp_kernels/sc/kernels.py:42-52)
    for name in ("fused_quantize_bipolar", "fused_quantize_bipolar_perrow",
                 "fused_quantize_unipolar", "_grouped_symmetric_quant",
                 "_grouped_asymmetric_quant", "_grouped_symmetric_quant_batched",
                 "fused_quant_kernel", "fused_quant_bipolar_batched_kernel", "_quant_dummy"):
        assert hasattr(K, name), name
    # the 13 names of scmp_kernels.quant (quant/__init__.py:17-51)
    for name in ("fused_quantize_bipolar", "fused_quantize_bipolar_perrow",
                 "fused_quantize_unipolar", "fused_quant_kernel",
                 "fused_quant_bipolar_batched_kernel", "_quant_dummy",
                 "_grouped_symmetric_quant", "_grouped_asymmetric_quant",
                 "_grouped_symmetric_quant_batched", "accumulate_act_scales",
                 "compute_smooth_scales", "apply_smoothing", "apply_smoothing_offline"):
        assert hasattr(Qm, name), name


def test_det_kernel_tuning_is_reentrant():
    from scmp_kernels_amd.sc import det_kernel_tuning
    from scmp_kernels_amd.sc import kernels as K
    assert not K._det_kernel_tuning_active()
    with det_kernel_tuning():
        with det_kernel_tuning():
            assert K._det_kernel_tuning_active()
        assert K._det_kernel_tuning_active()
    assert not K._det_kernel_tuning_active()


# ---- validation gates: raised before any kernel runs (CPU tensors are fine) ----------

def _t(*shape):
    return torch.zeros(*shape)


@pytest.mark.parametrize("kw,shapes,match", [
    (dict(granularity="per_tensor", chunk_d=72), ((64, 1024), (128, 1024)), "chunk_d"),
    (dict(granularity="per_row", mode="unipolar", chunk_d=72), ((64, 1024), (128, 1024)),
     "chunk_d"),
    (dict(granularity="per_row", chunk_d=72), ((4, 64, 1024), (4, 128, 1024)), "chunk_d"),
    (dict(granularity="per_head"), ((64, 1024), (128, 1024)), "per_head"),
    (dict(granularity="per_head", mode="unipolar"), ((4, 8, 64), (4, 8, 64)), "per_head"),
    (dict(granularity="per_block"), ((8, 64), (16, 64)), "granularity"),
    (dict(mode="ternary"), ((8, 64), (16, 64)), "mode"),
    (dict(stoc_len=512, sc_prec=8), ((8, 64), (16, 64)), "stoc_len"),
])
def test_validation_gates(kw, shapes, match):
    with pytest.raises(ValueError, match=match):
        sc_matmul(_t(*shapes[0]), _t(*shapes[1]), **kw)


def test_smooth_scales_validation():
    with pytest.raises(ValueError, match="1D"):
        sc_matmul(_t(4, 8), _t(5, 8), smooth_scales=_t(2, 8))
    with pytest.raises(ValueError, match="D mismatch"):
        sc_matmul(_t(4, 8), _t(5, 8), smooth_scales=_t(7))


@pytest.mark.skipif(_have_gpu(), reason="checks the behaviour without a GPU")
def test_no_gpu_fails_loudly():
    """Without a GPU there is no silent CPU fallback."""
    with pytest.raises(RuntimeError, match="GPU"):
        sc_matmul(torch.randn(4, 16), torch.randn(5, 16))


def test_missing_library_fails_loudly(tmp_path):
    from scmp_kernels_amd import _lib
    saved = _lib._lib
    try:
        _lib._lib = None
        with pytest.raises(RuntimeError, match="HIP library not found"):
            _lib.load(str(tmp_path / "libscmp_hip.so"))
    finally:
        _lib._lib = saved


# ---- GPU: shapes, dtype, device guard, determinism ------------------------------------

def _dev_randn(*shape, seed=0):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.standard_normal(shape).astype(np.float32)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("gran,sa,sb,kw,out", [
    ("per_tensor", (8, 64), (16, 64), {}, (8, 16)),
    ("per_row", (8, 64), (16, 64), {}, (8, 16)),
    ("per_row", (4, 8, 64), (4, 16, 64), {}, (4, 8, 16)),
    ("per_head", (16, 197, 64), (16, 197, 64), {}, (16, 197, 197)),
    ("per_row", (64, 1024), (128, 1024), dict(chunk_d=72), (64, 128)),
    ("per_row", (9, 40), (11, 40), dict(mode="unipolar", group_a=4, group_b=4), (9, 11)),
])
def test_output_shape_dtype(gran, sa, sb, kw, out):
    y = sc_matmul(_dev_randn(*sa, seed=1), _dev_randn(*sb, seed=2), granularity=gran,
                  sc_prec=8, **kw)
    assert tuple(y.shape) == out and y.dtype == torch.float32 and y.is_cuda
    assert torch.isfinite(y).all()


@pytest.mark.gpu
@pytest.mark.parametrize("gran,chunk_d,three_d", [
    ("per_tensor", 0, False), ("per_row", 0, False), ("per_row", 128, False),
    ("per_row", 0, True), ("per_head", 0, True)])
def test_deterministic_and_device_restored(gran, chunk_d, three_d):
    """Same inputs give identical outputs across calls and after clear_rng_cache; the
    current device is left as it was; inputs are not modified."""
    from scmp_kernels_amd.sc import clear_rng_cache
    if three_d:
        a, b = _dev_randn(4, 8, 64, seed=3), _dev_randn(4, 16, 64, seed=4)
    else:
        a, b = _dev_randn(8, 256, seed=3), _dev_randn(16, 256, seed=4)
    a0, b0 = a.clone(), b.clone()
    before = torch.cuda.current_device()
    y0 = sc_matmul(a, b, granularity=gran, chunk_d=chunk_d, sc_prec=8)
    y1 = sc_matmul(a, b, granularity=gran, chunk_d=chunk_d, sc_prec=8)
    clear_rng_cache()
    y2 = sc_matmul(a, b, granularity=gran, chunk_d=chunk_d, sc_prec=8)
    assert torch.cuda.current_device() == before
    assert torch.equal(y0, y1) and torch.equal(y0, y2)
    assert torch.equal(a, a0) and torch.equal(b, b0)


@pytest.mark.gpu
def test_cpu_inputs_round_trip():
    """CPU operands run on the GPU and the result comes back on the CPU
    (scmp_kernels/sc/kernels.py:1115-1117, 1150-1151)."""
    a, b = _dev_randn(8, 96, seed=5), _dev_randn(12, 96, seed=6)
    for gran in ("per_tensor", "per_row"):
        y_gpu = sc_matmul(a, b, granularity=gran)
        y_cpu = sc_matmul(a.cpu(), b.cpu(), granularity=gran)
        assert y_cpu.device.type == "cpu"
        assert torch.equal(y_cpu, y_gpu.cpu())


@pytest.mark.gpu
def test_operands_on_different_devices_rejected():
    a = _dev_randn(4, 16)
    with pytest.raises(ValueError, match="same device"):
        sc_matmul(a, a.cpu())


@pytest.mark.parametrize("gran,sa,sb,out", [
    ("per_row", (0, 64), (16, 64), (0, 16)),
    ("per_row", (8, 64), (0, 64), (8, 0)),
    ("per_tensor", (0, 32), (5, 32), (0, 5)),
    ("per_row", (3, 0, 64), (3, 16, 64), (3, 0, 16)),
])
def test_empty_operands_give_empty_output(gran, sa, sb, out):
    """No rows on one side: an empty float32 product on the operands' device, no launch
    (runs on the CPU too: nothing reaches the GPU)."""
    y = sc_matmul(torch.zeros(sa), torch.zeros(sb), granularity=gran)
    assert tuple(y.shape) == out and y.dtype == torch.float32 and y.device.type == "cpu"


def test_zero_inner_dimension_rejected():
    with pytest.raises(ValueError, match="inner dimension"):
        sc_matmul(torch.zeros(4, 0), torch.zeros(5, 0))


def _fake_tables(class_of, JP=64):
    from types import SimpleNamespace
    from scmp_kernels_amd.sc import tables as TB
    class_of = np.asarray(class_of, dtype=np.int32)
    t = SimpleNamespace(class_of=class_of, nclass=int(class_of.max()) + 1, JP=JP,
                        D=len(class_of), lut=torch.zeros(1), _runs=None)
    t.class_runs = lambda: TB.StreamTables.class_runs(t)
    return t


@pytest.mark.parametrize("D,nclass,seed", [(4096, 64, 0), (777, 64, 1), (100, 7, 2),
                                           (64, 1, 3), (513, 300, 4)])
def test_class_runs_layout(D, nclass, seed):
    """Every d appears once, in runs of its own class (increasing d inside a run), each
    run padded with -1 to whole groups of 8 whose class is the run's."""
    rng = np.random.default_rng(seed)
    class_of = rng.integers(0, nclass, D)
    class_of[:nclass] = np.arange(nclass)                  # every class occurs
    t = _fake_tables(class_of)
    src, gcls, Dp = t.class_runs()
    src, gcls = src.numpy(), gcls.numpy()
    assert Dp % 8 == 0 and len(src) == Dp and len(gcls) == Dp // 8
    assert sorted(src[src >= 0].tolist()) == list(range(D))
    counts = np.bincount(class_of, minlength=t.nclass)
    assert Dp == int(((counts + 7) // 8 * 8).sum())
    grp = np.repeat(gcls, 8)
    real = src >= 0
    np.testing.assert_array_equal(class_of[src[real]], grp[real])
    for c in range(t.nclass):
        pos = np.nonzero(grp == c)[0]
        if len(pos):
            assert pos[-1] - pos[0] + 1 == len(pos)            # one contiguous run
            run = src[pos]
            k = counts[c]
            assert (run[:k] >= 0).all() and (run[k:] == -1).all()
            assert (np.diff(run[:k]) > 0).all()


def test_class_runs_selection(monkeypatch):
    from scmp_kernels_amd.sc import kernels as K
    monkeypatch.delenv("SCMP_FP4_RUNS", raising=False)
    assert K._fp4_class_runs(_fake_tables(np.zeros(512, int)), 512) is None   # one class
    # 8 classes of 64-interval tables fit in LDS: all of them are staged, no runs
    assert K._fp4_class_runs(_fake_tables(np.arange(512) % 8), 512) is None
    # 64 classes do not fit: runs when the padding is small
    t = _fake_tables(np.arange(4096) % 64)
    src, gcls, Dp = K._fp4_class_runs(t, 4096)
    assert Dp == 4096
    # ... but not when the runs would grow D by more than an eighth
    assert K._fp4_class_runs(_fake_tables(np.arange(256) % 64), 256) is None
    monkeypatch.setenv("SCMP_FP4_RUNS", "1")
    assert K._fp4_class_runs(_fake_tables(np.arange(256) % 64), 256)[2] == 512
    monkeypatch.setenv("SCMP_FP4_RUNS", "0")
    assert K._fp4_class_runs(t, 4096) is None
    # not even when forced do runs pad D past the FP4 kernel's 65536 (here 5000 classes of
    # 13-14 d each: 65500 -> 80000)
    monkeypatch.setenv("SCMP_FP4_RUNS", "1")
    assert K._fp4_class_runs(_fake_tables(np.arange(65500) % 5000), 65500) is None

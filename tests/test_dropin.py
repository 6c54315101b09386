"""The package under the reference's import name (scmp_kernels_amd.compat.install): the
reference's own smoke expectations (tests/test_sc_smoke.py:25-129 of the reference: imports,
shape and dtype per granularity, the ValueError gates) through ``scmp_kernels.*`` names, and
the per-path entry points called with the reference's positional parameter lists
(scmp_kernels/sc/kernels.py:440, :1054, :1444), checked against the oracle."""
import inspect

import numpy as np
import pytest
import torch

from oracle import sc_oracle as O


@pytest.fixture
def sk():
    from scmp_kernels_amd import compat
    compat.install()
    import scmp_kernels
    yield scmp_kernels
    compat.uninstall()


def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return "cuda"


# ------------------------------------------------------------------ CPU: names, gates

def test_alias_imports(sk):
    from scmp_kernels import sc_matmul                                  # noqa: F401
    from scmp_kernels.sc import sc_matmul as s2, det_kernel_tuning, clear_rng_cache  # noqa
    from scmp_kernels.sc.kernels import fused_quantize_bipolar         # noqa: F401
    from scmp_kernels.quant import (accumulate_act_scales, compute_smooth_scales,  # noqa
                                    apply_smoothing, _grouped_symmetric_quant)
    from scmp_kernels.mp import MPConfig, RowAssignment, classify_rows_by_metric  # noqa
    from scmp_kernels.sc.config_helpers import make_sobol_simple_config  # noqa: F401
    import scmp_kernels.sc.kernels as K
    import scmp_kernels_amd
    assert sk.sc_matmul is scmp_kernels_amd.sc_matmul is s2
    assert K.__name__ == "scmp_kernels_amd.sc.kernels"


def test_alias_refuses_a_foreign_package(monkeypatch):
    import types
    from scmp_kernels_amd import compat
    monkeypatch.setitem(__import__("sys").modules, "scmp_kernels",
                        types.ModuleType("scmp_kernels"))
    with pytest.raises(ImportError, match="already imported"):
        compat.install()


def test_private_entry_points_take_the_reference_parameters(sk):
    """Parameter names and order of the reference's per-path functions."""
    from scmp_kernels.sc import matmul as Mm
    want = {
        "_sc_matmul_per_tensor": ["a", "b", "max_fp_a", "min_fp_a", "max_fp_b", "min_fp_b",
                                  "mode", "sc_prec", "config", "stoc_len", "rng_levels"],
        "_sc_matmul_per_head_bipolar": ["q_flat", "k_flat", "q_maxs", "q_mins", "k_maxs",
                                        "k_mins", "sc_prec", "config", "stoc_len",
                                        "rng_levels"],
        "_sc_matmul_per_row_mlp": ["a", "b", "max_fp_a", "min_fp_a", "max_fp_b", "min_fp_b",
                                   "mode", "sc_prec", "config", "group_a", "group_b",
                                   "chunk_d", "stoc_len", "rng_levels"],
    }
    for name, params in want.items():
        sig = inspect.signature(getattr(Mm, name))
        pos = [p.name for p in sig.parameters.values()
               if p.kind == inspect.Parameter.POSITIONAL_OR_KEYWORD]
        assert pos == params, name
    with pytest.raises(ValueError, match="max_fp_a and min_fp_a"):
        Mm._sc_matmul_per_tensor(torch.zeros(2, 4), torch.zeros(3, 4), 1.0)
    with pytest.raises(ValueError, match="all four"):
        Mm._sc_matmul_per_head_bipolar(torch.zeros(1, 2, 4), torch.zeros(1, 3, 4),
                                       torch.ones(1), torch.zeros(1), None, None, 8, None)


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
])
def test_reference_validation_gates(sk, kw, shapes, match):
    """tests/test_sc_smoke.py:81-129 of the reference, through scmp_kernels.sc_matmul."""
    with pytest.raises(ValueError, match=match):
        sk.sc_matmul(_t(*shapes[0]), _t(*shapes[1]), **kw)


# ------------------------------------------------------------------ GPU: smoke shapes

@pytest.mark.gpu
@pytest.mark.parametrize("gran,sa,sb,kw,out", [
    ("per_tensor", (8, 64), (16, 64), {}, (8, 16)),
    ("per_row", (8, 64), (16, 64), {}, (8, 16)),
    ("per_row", (4, 8, 64), (4, 16, 64), {}, (4, 8, 16)),
    ("per_head", (16, 197, 64), (16, 197, 64), {}, (16, 197, 197)),
    ("per_row", (64, 1024), (128, 1024), {"chunk_d": 72}, (64, 128)),
])
def test_reference_smoke_shapes(sk, gran, sa, sb, kw, out):
    """tests/test_sc_smoke.py:30-74 of the reference (shape and dtype), with the values
    checked against the oracle."""
    dev = _gpu()
    g = torch.Generator().manual_seed(sum(sa) + len(kw))
    a, b = torch.randn(*sa, generator=g), torch.randn(*sb, generator=g)
    y = sk.sc_matmul(a.to(dev), b.to(dev), granularity=gran, sc_prec=8, **kw)
    assert tuple(y.shape) == out and y.dtype == torch.float32
    ref = O.sc_matmul(a.numpy(), b.numpy(), gran, sc_prec=8, **kw)
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------ GPU: per-path entry points, positional

def _ab(shape_a, shape_b, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape_a).astype(np.float32),
            (rng.standard_normal(shape_b) * 0.5).astype(np.float32))


def _bits(y):
    return y.cpu().numpy().view(np.uint32)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["bipolar", "unipolar"])
@pytest.mark.parametrize("rank", [2, 3])
def test_per_tensor_with_the_callers_ranges(sk, mode, rank):
    from scmp_kernels.sc.matmul import _sc_matmul_per_tensor
    dev = _gpu()
    lead = (3,) if rank == 3 else ()
    a_h, b_h = _ab((*lead, 40, 96), (*lead, 30, 96), 31 + rank)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    # the ranges the reference's sc_matmul passes: the product's default path must agree
    rng = (float(a_h.max()), float(a_h.min()), float(b_h.max()), float(b_h.min()))
    y = _sc_matmul_per_tensor(a, b, *rng, mode, 8, None, 128)
    np.testing.assert_array_equal(_bits(y), _bits(sk.sc_matmul(a, b, "per_tensor", mode=mode,
                                                               stoc_len=128)))
    # ranges of the caller's own: narrower than the data (clamping), b's defaulting to a's
    for ranges in [(1.5, -0.75, 4.0, -3.0), (0.6, -1.2, None, None)]:
        y = _sc_matmul_per_tensor(a, b, *ranges, mode, 8, None, 128)
        ref = O.sc_matmul_per_tensor(a_h, b_h, *ranges, mode=mode, sc_prec=8, stoc_len=128)
        np.testing.assert_array_equal(_bits(y), ref.view(np.uint32))


@pytest.mark.gpu
def test_per_head_with_the_callers_ranges(sk):
    from scmp_kernels.sc.matmul import _sc_matmul_per_head_bipolar
    dev = _gpu()
    q_h, k_h = _ab((6, 37, 64), (6, 29, 64), 41)
    q, k = torch.from_numpy(q_h).to(dev), torch.from_numpy(k_h).to(dev)
    cfg = O.make_sobol_simple_config(64, 64, 8)
    qmx, qmn = q.amax(dim=(1, 2)), q.amin(dim=(1, 2))
    kmx, kmn = k.amax(dim=(1, 2)), k.amin(dim=(1, 2))
    y = _sc_matmul_per_head_bipolar(q, k, qmx, qmn, kmx, kmn, 8, cfg)
    np.testing.assert_array_equal(_bits(y), _bits(sk.sc_matmul(q, k, "per_head")))
    # narrower (clamps at [-128, 127]) and wider ranges of the caller's own
    for f in (0.5, 1.7):
        rq = (qmx * f, qmn * f * 0.8, kmx * f * 1.1, kmn * f)
        y = _sc_matmul_per_head_bipolar(q, k, *rq, 8, cfg, 64)
        ref = O.sc_matmul_per_head_bipolar(q_h, k_h, *(r.cpu().numpy() for r in rq), 8, cfg,
                                           stoc_len=64)
        np.testing.assert_array_equal(_bits(y), ref.view(np.uint32))


@pytest.mark.gpu
def test_per_row_mlp_reference_positions(sk):
    from scmp_kernels.sc.matmul import _sc_matmul_per_row_mlp
    dev = _gpu()
    a_h, b_h = _ab((33, 200), (21, 200), 51)
    a, b = torch.from_numpy(a_h).to(dev), torch.from_numpy(b_h).to(dev)
    # bipolar, chunked (ranges ignored, as in the reference)
    y = _sc_matmul_per_row_mlp(a, b, 0.0, 0.0, None, None, "bipolar", 8, None, 1, 1, 72)
    ref = O.sc_matmul_per_row_mlp(a_h, b_h, chunk_d=72)
    np.testing.assert_array_equal(_bits(y), ref.view(np.uint32))
    # bipolar, D <= chunk_d: the row-group path with the given groups
    y = _sc_matmul_per_row_mlp(a, b, 0.0, 0.0, None, None, "bipolar", 8, None, 3, 2, 256)
    ref = O.sc_matmul_per_row_mlp(a_h, b_h, group_a=3, group_b=2, chunk_d=256)
    np.testing.assert_array_equal(_bits(y), ref.view(np.uint32))
    # unipolar: per-tensor quantization with the caller's ranges
    y = _sc_matmul_per_row_mlp(a, b, 2.5, -2.0, 1.0, -1.5, "unipolar", 8, None)
    ref = O.sc_matmul_per_row_mlp(a_h, b_h, 2.5, -2.0, 1.0, -1.5, mode="unipolar")
    np.testing.assert_array_equal(_bits(y), ref.view(np.uint32))
    # 3-D: every batch with the ranges, no groups
    a3, b3 = _ab((2, 9, 64), (2, 7, 64), 52)
    y = _sc_matmul_per_row_mlp(torch.from_numpy(a3).to(dev), torch.from_numpy(b3).to(dev),
                               3.0, -3.0, None, None, "unipolar", 8, None, stoc_len=64)
    ref = O.sc_matmul_per_row_mlp(a3, b3, 3.0, -3.0, mode="unipolar", stoc_len=64)
    np.testing.assert_array_equal(_bits(y), ref.view(np.uint32))

"""SmoothQuant helpers (the reference's tests/test_smoothquant.py covers the same
behaviour): running max-abs, the alpha = 0 / 1 closed forms, the matmul identity in 2-D
and 3-D, the offline bake, argument errors, the outlier-MSE claim, and (GPU) that the
``smooth_scales`` kwarg equals smoothing by hand, bit for bit."""
import numpy as np
import pytest
import torch

from scmp_kernels_amd.quant import (
    accumulate_act_scales,
    apply_smoothing,
    apply_smoothing_offline,
    compute_smooth_scales,
)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def test_running_max_abs():
    g = _gen(11)
    parts = [torch.randn(5, 3, 12, generator=g) * k for k in (1.0, 4.0, 0.5)]
    run = None
    for p in parts:
        run = accumulate_act_scales(p, run)
    want = torch.stack([p.reshape(-1, 12).abs().amax(0) for p in parts]).amax(0)
    assert run.shape == (12,)
    assert torch.equal(run, want)


def test_smooth_scales_closed_forms():
    g = _gen(12)
    act = torch.rand(24, generator=g) * 3 + 0.05
    w = torch.randn(40, 24, generator=g)
    w[:, 5] = 0.0                                   # a dead column hits the eps floor
    wmax = w.abs().amax(0).clamp(min=1e-5)
    torch.testing.assert_close(compute_smooth_scales(act, w, alpha=0.0), 1.0 / wmax)
    torch.testing.assert_close(compute_smooth_scales(act, w, alpha=1.0), act)
    s = compute_smooth_scales(act, w, alpha=0.5)
    torch.testing.assert_close(s, (act / wmax).sqrt(), rtol=1e-6, atol=0)
    assert bool((s >= 1e-5).all())


@pytest.mark.parametrize("shape_a,shape_b", [((6, 48), (9, 48)), ((3, 6, 48), (3, 9, 48))])
def test_matmul_identity(shape_a, shape_b):
    g = _gen(13)
    a = torch.randn(*shape_a, generator=g, dtype=torch.float64)
    b = torch.randn(*shape_b, generator=g, dtype=torch.float64)
    s = torch.rand(48, generator=g, dtype=torch.float64) + 0.25
    a2, b2 = apply_smoothing(a, b, s)
    ref = a @ b.transpose(-1, -2)
    got = a2 @ b2.transpose(-1, -2)
    assert float((ref - got).abs().max()) < 1e-10
    # inputs are left alone
    assert not torch.equal(a2, a)


def test_offline_bake():
    g = _gen(14)
    a = torch.randn(5, 20, generator=g, dtype=torch.float64)
    w = torch.randn(7, 20, generator=g, dtype=torch.float64)
    s = torch.rand(20, generator=g, dtype=torch.float64) + 0.5
    wb = apply_smoothing_offline(w, s)
    assert float(((a / s) @ wb.T - a @ w.T).abs().max()) < 1e-10


def test_argument_errors():
    with pytest.raises(ValueError, match="alpha"):
        compute_smooth_scales(torch.ones(6), torch.ones(3, 6), alpha=-0.1)
    with pytest.raises(ValueError, match="D mismatch"):
        compute_smooth_scales(torch.ones(6), torch.ones(3, 7))
    with pytest.raises(ValueError, match="1D"):
        compute_smooth_scales(torch.ones(2, 6), torch.ones(3, 6))
    with pytest.raises(ValueError, match="2D"):
        compute_smooth_scales(torch.ones(6), torch.ones(6))
    with pytest.raises(ValueError, match="1D"):
        apply_smoothing(torch.zeros(2, 6), torch.zeros(3, 6), torch.zeros(2, 6))
    with pytest.raises(ValueError, match="D mismatch"):
        apply_smoothing(torch.zeros(2, 6), torch.zeros(3, 5), torch.zeros(6))
    with pytest.raises(ValueError, match="D mismatch"):
        apply_smoothing_offline(torch.zeros(3, 5), torch.zeros(6))


def _fake_int8(x, dims):
    """Symmetric absmax fake-quantization over ``dims`` (q_max = 127)."""
    scale = x.abs().amax(dim=dims, keepdim=True).clamp(min=1e-5) / 127
    return (x / scale).round().clamp(-127, 127) * scale


@pytest.mark.parametrize("dims", [(-1,), (0, 1)])
def test_outlier_mse_halved(dims):
    """Moving outlier channels into the weights at least halves the int8 error."""
    g = _gen(15)
    a = torch.randn(96, 192, generator=g) * 0.5
    a[:, [2, 31, 77, 140]] *= 50.0
    w = torch.randn(48, 192, generator=g) * 0.5
    ref = a @ w.T
    plain = (_fake_int8(a, dims) @ _fake_int8(w, dims).T - ref).pow(2).mean()
    s = compute_smooth_scales(accumulate_act_scales(a), w, alpha=0.5)
    a2, w2 = apply_smoothing(a, w, s)
    smooth = (_fake_int8(a2, dims) @ _fake_int8(w2, dims).T - ref).pow(2).mean()
    assert float(smooth) < 0.5 * float(plain)


@pytest.mark.gpu
@pytest.mark.parametrize("gran,kw", [("per_row", {}), ("per_row", dict(chunk_d=24)),
                                     ("per_tensor", {}),
                                     ("per_row", dict(mode="unipolar", group_a=2))])
def test_smooth_kwarg_equals_manual_smoothing(gran, kw):
    """sc_matmul(a, b, smooth_scales=s) == sc_matmul(a / s, b * s) bit for bit: the
    quantizers divide / multiply while loading with the same fp32 rounding."""
    from scmp_kernels_amd import sc_matmul
    rng = np.random.default_rng(16)
    a = torch.from_numpy((rng.standard_normal((20, 80)) * 0.5).astype(np.float32)).cuda()
    a[:, 9] *= 30.0
    b = torch.from_numpy((rng.standard_normal((18, 80)) * 0.5).astype(np.float32)).cuda()
    s = compute_smooth_scales(accumulate_act_scales(a), b, alpha=0.5)
    y_kw = sc_matmul(a, b, gran, smooth_scales=s, **kw)
    a2, b2 = apply_smoothing(a, b, s)
    y_manual = sc_matmul(a2, b2, gran, **kw)
    assert torch.equal(y_kw, y_manual)

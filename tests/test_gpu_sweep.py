"""Seeded random sweep of sc_matmul against the oracle: shapes around the FP4 kernel's
tile-shape choices (narrow, 256 x 256, 128 x 512), split-tile, chunk_d round/tail and
class-run thresholds, every stream length, both modes, row groups, per_row and
per_tensor, with the class-run layout forced on, off or left to its rule. per_row
results are checked on whole row groups sampled from the output (rows are independent
between groups)."""
import numpy as np
import pytest
import torch

from oracle import sc_oracle as O

pytestmark = pytest.mark.gpu


def _cases(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        N = int(rng.choice([rng.integers(1, 130), rng.integers(129, 700), rng.integers(1200, 1500)]))
        M = int(rng.choice([rng.integers(1, 65), rng.integers(65, 600), 512 * int(rng.integers(1, 4)),
                            rng.integers(900, 2400)]))
        D = int(rng.choice([rng.integers(8, 200), 512 * int(rng.integers(1, 3)), rng.integers(500, 1100)]))
        L = int(rng.choice([256, 128, 64, 32, 16]))
        mode = str(rng.choice(["bipolar", "unipolar"]))
        gran = str(rng.choice(["per_row", "per_row", "per_tensor"]))
        kw = dict(mode=mode, stoc_len=L, rng_levels=L)
        if gran == "per_row" and mode == "bipolar" and rng.random() < 0.3 and D > 40:
            kw["chunk_d"] = int(rng.integers(8, D // 2))        # odd or even
        if gran == "per_row" and mode == "unipolar" and rng.random() < 0.5:
            kw["group_a"], kw["group_b"] = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        if gran == "per_tensor":
            N, M = min(N, 500), min(M, 600)
        runs = str(rng.choice(["", "0", "1"]))
        out.append((N, M, D, gran, kw, runs, int(rng.integers(0, 2 ** 31))))
    return out


def test_random_sweep_vs_oracle(monkeypatch):
    from scmp_kernels_amd import sc_matmul
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    dev = torch.device("cuda", 0)
    failed = []
    for N, M, D, gran, kw, runs, seed in _cases(1, 70):
        if runs:
            monkeypatch.setenv("SCMP_FP4_RUNS", runs)
        else:
            monkeypatch.delenv("SCMP_FP4_RUNS", raising=False)
        rng = np.random.default_rng(seed)
        a = rng.standard_normal((N, D)).astype(np.float32)
        b = (rng.standard_normal((M, D)) * 0.05).astype(np.float32)
        y = sc_matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), gran, **kw)
        y = y.cpu().numpy()
        if gran == "per_row":
            ga = kw.get("group_a", 1)
            ng = -(-N // ga)
            gsel = np.unique(np.concatenate([[0, ng - 1], rng.integers(0, ng, 12)]))
            rows = np.concatenate([np.arange(g * ga, min((g + 1) * ga, N)) for g in gsel])
            ref = O.sc_matmul(a[rows], b, gran, **kw)
            got = y[rows]
        else:
            ref, got = O.sc_matmul(a, b, gran, **kw), y
        if not np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32)):
            failed.append((gran, N, M, D, kw, runs or "-"))
    assert not failed, f"{len(failed)} cases differ from the oracle: {failed}"

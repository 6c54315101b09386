"""RNG descriptions for stochastic computing (Sobol, LFSR, TrueRandom).

Mirrors the reference's scmp_kernels/sc/rng.py interface (classes, seeds, ``simulate``).
``simulate`` of Sobol and LFSR runs the generator kernels of libscmp_hip.so on the
current GPU (scmp_rng_sobol / scmp_rng_lfsr) and returns a numpy array; TrueRandom is
Python's Mersenne Twister by definition (rng.py:80-113) and stays on the host.
"""
from __future__ import annotations

import random
from typing import Optional

import numpy as np


def sobol_default_seed(length: int, seed_type: str) -> list:
    """Default direction-vector seeds, scmp_kernels/sc/rng.py:156-171."""
    if seed_type == "k":
        if length == 8:
            return [1, 1, 1, 1, 9, 1, 41, 255]
        seed = [1] * length
        if length >= 5:
            seed[4] = 9
        if length >= 7:
            seed[6] = 41
        return seed
    return [1] * length


def sobol_direction_vectors(length: int, seed: list) -> list:
    """V_i = int(seed_i / 2^(i+1) * 2^length) in float64, scmp_kernels/sc/rng.py:173-183."""
    return [int(seed[i] / (1 << (i + 1)) * (1 << length)) for i in range(length)]


def _device_sequence(kind: str, length: int, n: int, **kw) -> np.ndarray:
    import torch
    from .. import _lib
    if not torch.cuda.is_available():
        raise RuntimeError("scmp_kernels_amd: RNG generation runs on the GPU; none available")
    dev = torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(n, dtype=torch.int32, device=dev)
    lib = _lib.load()
    s = _lib.stream_of(dev)
    if kind == "sobol":
        V = np.asarray(kw["V"], dtype=np.int64)
        _lib.check(lib.scmp_rng_sobol(length, V.ctypes.data, n, out.data_ptr(), s),
                   "scmp_rng_sobol")
    else:
        mask = 0
        for t in kw["taps"]:
            mask |= 1 << int(t)
        _lib.check(lib.scmp_rng_lfsr(length, kw["seed"], mask, n, out.data_ptr(), s),
                   "scmp_rng_lfsr")
    return out.cpu().numpy()


class RNG:
    def simulate(self, num_cycles: int = None) -> np.ndarray:
        raise NotImplementedError

    def reset(self):
        pass


class LFSR(RNG):
    """Fibonacci right-shift LFSR (scmp_kernels/sc/rng.py:32-77)."""

    def __init__(self, seed: int, length: int, taps: list):
        if seed == 0:
            raise ValueError("LFSR seed must be non-zero")
        self.seed, self.length, self.taps = seed, length, list(taps)

    def simulate(self, num_cycles: int = None) -> np.ndarray:
        n = 2 ** self.length if num_cycles is None else num_cycles
        return _device_sequence("lfsr", self.length, n, seed=self.seed, taps=self.taps)


class TrueRandom(RNG):
    """Python ``random`` stream, randint(0, 2^length - 1) (scmp_kernels/sc/rng.py:80-113)."""

    def __init__(self, seed: int, length: int):
        self.seed, self.length, self.max_val = seed, length, 2 ** length - 1

    def reset(self):
        random.seed(self.seed)

    def simulate(self, num_cycles: int = None) -> np.ndarray:
        n = 2 ** self.length if num_cycles is None else num_cycles
        self.reset()
        return np.array([random.randint(0, self.max_val) for _ in range(n)], dtype=np.int32)


class Sobol(RNG):
    """Gray-code Sobol sequence, SCGen seeds (scmp_kernels/sc/rng.py:116-239)."""

    def __init__(self, length: int, seed: list = None, seed_type: str = "q"):
        self.length = length
        self.max_val = 2 ** length
        self.seed = list(seed) if seed is not None else sobol_default_seed(length, seed_type)
        self._direction_vectors = sobol_direction_vectors(length, self.seed)

    def simulate(self, num_cycles: int = None) -> np.ndarray:
        n = 2 ** self.length if num_cycles is None else num_cycles
        return _device_sequence("sobol", self.length, n, V=self._direction_vectors)

    @staticmethod
    def random_seed(length: int) -> list:
        """seed[0] = 1, seed[i] odd in [1, 2^(i+1)) (scmp_kernels/sc/rng.py:227-239)."""
        seed = [1]
        for i in range(1, length):
            max_val = 1 << (i + 1)
            seed.append(random.randint(0, max_val // 2 - 1) * 2 + 1)
        return seed


def create_rng(rng_type: str, length: int, **kwargs) -> RNG:
    """scmp_kernels/sc/rng.py:242-268."""
    if rng_type == "lfsr":
        return LFSR(seed=kwargs["seed"], length=length, taps=kwargs["taps"])
    if rng_type == "true_random":
        return TrueRandom(seed=kwargs["seed"], length=length)
    if rng_type == "sobol":
        return Sobol(length=length, seed=kwargs.get("seed"),
                     seed_type=kwargs.get("seed_type", "q"))
    raise ValueError(f"Unknown RNG type: {rng_type}")

"""bench.py's synthetic inputs come from the tests' seeded generator: its
device restatement of SplitMix64 + Box-Muller (bench.seeded_normal) against
the oracle's fill_normal -- bit-identical on the CPU, and on the GPU within
one float32 ulp (the device's float64 log / cos may round differently)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import bench

CASES = [(0x4E463457, 0.02, 100_003), (((0x4E463458 << 16) + 1), 1.0, 4096), (5, 0.1, 1), (2**64 - 3, 0.5, 777)]


@pytest.mark.parametrize("seed,sigma,n", CASES)
def test_seeded_normal_matches_oracle_on_cpu(oracle, seed, sigma, n):
    got = bench.seeded_normal(torch, seed, sigma, n, device="cpu").numpy()
    assert got.dtype == np.float32 and got.shape == (n,)
    assert np.array_equal(got, oracle.fill_normal(seed % 2**64, sigma, n))


def test_rng_draws_are_distinct_streams(oracle):
    # draw k of a workload seeded s is fill_normal((s << 16) + k): distinct streams, reproducible
    r = bench.Rng(torch, 0x4E463457, device="cpu")
    a, b = r.normal(3, 5), r.normal(15, sigma=0.02)
    assert a.shape == (3, 5) and not np.array_equal(a.numpy().ravel(), b.numpy() / 0.02)
    assert np.array_equal(a.numpy().ravel(), oracle.fill_normal((0x4E463457 << 16) + 1, 1.0, 15))
    assert np.array_equal(b.numpy(), oracle.fill_normal((0x4E463457 << 16) + 2, 0.02, 15))


@pytest.mark.gpu
@pytest.mark.parametrize("seed,sigma,n", CASES)
def test_seeded_normal_matches_oracle_on_gpu(device, oracle, seed, sigma, n):
    got = bench.seeded_normal(torch, seed, sigma, n, device=device).cpu().numpy()
    ref = oracle.fill_normal(seed % 2**64, sigma, n)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= ulp)

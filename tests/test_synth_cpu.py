"""The counter-based synthetic logits on the host (meshy_synth_bf16_rows_host):
the fp32 routines of the Box-Muller generator (csrc/synth_math.h, built here
with g++ as a separate program) against float64 numpy, the whole pair
against a float64 Box-Muller of the same hash, the library's rows against the
g++ build bit for bit, the N(0, scale^2) distribution (Kolmogorov-Smirnov on
the fp32 values, moments and tails of the bf16 rows) and row addressing."""

from __future__ import annotations

import math
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

from meshy_amd import workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "meshy_amd", "csrc")
M64 = 2**64 - 1


def _mix(x):
    x = (x + 0x9E3779B97F4A7C15) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def _mix_np(x):
    x = x + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def _box_muller64(h):
    """The documented pair of hash h in float64: u1 = (lo32 + 1) / 2^32,
    theta = 2 pi hi32 / 2^32, r = sqrt(-2 ln u1), (r cos theta, r sin theta)."""
    lo = (h & np.uint64(0xFFFFFFFF)).astype(np.float64) + 1.0
    hi = (h >> np.uint64(32)).astype(np.float64)
    r = np.sqrt(-2.0 * np.log(lo / 2.0**32))
    t = 2.0 * math.pi * hi / 2.0**32
    return r, np.stack([r * np.cos(t), r * np.sin(t)], axis=1)


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("needs g++")
    d = tmp_path_factory.mktemp("synth")
    exe = str(d / "synth_math_harness")
    cmd = ["g++", "-std=c++17", "-O2", "-ffp-contract=off", f"-I{CSRC}",
           os.path.join(ROOT, "tests", "native", "synth_math_harness.cpp"), "-o", exe]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]

    def run(mode, arr, out_dtype):
        src, dst = str(d / "in.bin"), str(d / "out.bin")
        np.ascontiguousarray(arr).tofile(src)
        subprocess.run([exe, mode, src, dst], check=True, timeout=120)
        return np.fromfile(dst, out_dtype)

    return run


def test_splitmix_finaliser_known_answer():
    # splitmix64 seeded with 0 starts 0xe220a8397b1dcdaf (Vigna's reference output)
    assert _mix(0) == 0xE220A8397B1DCDAF
    assert int(_mix_np(np.array([0], np.uint64))[0]) == 0xE220A8397B1DCDAF


def test_ln_against_float64(harness):
    """-2 ln(n / 2^32) over every decade of n, both sides of the u1 = 1/2 and
    m = sqrt 2 switches and the ends (n = 1 gives 64 ln 2, n = 2^32 gives 0)."""
    rng = np.random.default_rng(0)
    edges = [1, 2, 3, 2**24, 2**24 + 1, 2**31 - 1, 2**31, 2**31 + 1, int(math.sqrt(2) * 2**31),
             int(math.sqrt(2) * 2**31) + 1, int(2**32 * (1 - 0.29289322)), int(2**32 * (1 - 0.29289322)) + 1,
             2**32 - 2, 2**32 - 1, 2**32]
    n = np.concatenate([np.array(edges, np.uint64), rng.integers(1, 2**32 + 1, 200_000, dtype=np.uint64),
                        np.unique(np.logspace(0, 32, 50_000, base=2).astype(np.uint64)),
                        np.uint64(2**32) - np.unique(np.logspace(0, 31, 50_000, base=2).astype(np.uint64))])
    got = harness("ln", n, np.float32).astype(np.float64)
    c = 2.0**32 - n.astype(np.float64)
    ref = np.where(n > 2**31, -2.0 * np.log1p(-c / 2.0**32), -2.0 * (np.log(n.astype(np.float64)) - 32 * math.log(2)))
    assert got[len(edges) - 1] == 0.0 and abs(got[0] - 64 * math.log(2)) < 1e-5  # n = 2^32 and n = 1
    pos = ref > 0
    assert np.all(got[~pos] == 0.0)
    assert (np.abs(got - ref)[pos] / ref[pos]).max() < 5e-7


def test_sqrt_against_float64(harness):
    rng = np.random.default_rng(1)
    x = np.concatenate([np.array([0.0, 1e-9, 2.4e-7, 1.0, 2.0, 4.0, 44.36], np.float32),
                        rng.uniform(0, 45, 200_000).astype(np.float32),
                        (10.0 ** rng.uniform(-8, 1.7, 50_000)).astype(np.float32)])
    got = harness("sqrt", x, np.float32).astype(np.float64)
    ref = np.sqrt(x.astype(np.float64))
    assert got[0] == 0.0
    pos = ref > 0
    assert (np.abs(got - ref)[pos] / ref[pos]).max() <= 2.0**-23  # within an ulp


def test_cos_sin_against_float64(harness):
    """Every octant, both ends of each and its middle, and random angles."""
    rng = np.random.default_rng(2)
    base = np.arange(0, 2**32, 2**29, dtype=np.uint64)
    a = np.concatenate([base + d for d in (0, 1, 31, 32, 2**28, 2**29 - 32, 2**29 - 1)]).astype(np.uint32)
    a = np.concatenate([a, rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32)])
    got = harness("turn", a, np.float32).reshape(-1, 2).astype(np.float64)
    th = 2.0 * math.pi * a.astype(np.float64) / 2.0**32
    assert np.abs(got[:, 0] - np.cos(th)).max() < 2e-7
    assert np.abs(got[:, 1] - np.sin(th)).max() < 2e-7
    assert got[0].tolist() == [1.0, 0.0]  # a = 0: theta = 0


def test_pairs_are_the_box_muller_pair(harness):
    """The fp32 pair against the float64 Box-Muller of the same hash, with
    hashes whose u1 is 1/2^32, 1 and just below 1."""
    rng = np.random.default_rng(3)
    h = rng.integers(0, 2**63, 200_000, dtype=np.uint64) * np.uint64(2) + rng.integers(0, 2, 200_000, dtype=np.uint64)
    hi = rng.integers(0, 2**32, 300, dtype=np.uint64) << np.uint64(32)
    h = np.concatenate([h, hi, hi + np.uint64(2**32 - 1), hi + np.uint64(2**32 - 7)])
    got = harness("pair", h, np.float32).reshape(-1, 2).astype(np.float64)
    r, ref = _box_muller64(h)
    assert (np.abs(got - ref).max(axis=1) / np.maximum(r, 1e-30)).max() < 1e-6
    assert np.abs(got - ref).max() < 2e-6


def test_fp32_values_are_normal(harness):
    """Kolmogorov-Smirnov of 10^6 fp32 values (before the bf16 rounding)
    against N(0, 1): a bounded or skewed generator fails it."""
    stats = pytest.importorskip("scipy.stats")
    h = _mix_np(np.arange(500_000, dtype=np.uint64) ^ np.uint64(_mix(11)))
    z = harness("pair", h, np.float32).astype(np.float64)
    res = stats.kstest(z, "norm")
    assert res.pvalue > 1e-3, res
    # each half of the pair on its own, and the two halves uncorrelated
    zz = z.reshape(-1, 2)
    assert stats.kstest(zz[:, 0], "norm").pvalue > 1e-3 and stats.kstest(zz[:, 1], "norm").pvalue > 1e-3
    assert abs(np.corrcoef(zz[:, 0], zz[:, 1])[0, 1]) < 5e-3


def test_library_rows_equal_the_gxx_build(harness):
    """The library's host rows (compiled by hipcc) equal the header compiled
    by g++ bit for bit: element 2p and 2p + 1 are pair p.  Rows of an odd
    width start on either half of a pair."""
    cols = 777
    rows = [0, 1, 2, 5, 1000003]
    got = workloads.synth_logit_rows(rows, cols, seed=1, scale=2.0).view(torch.int16).numpy().view(np.uint16)
    k = (np.array(rows, np.uint64)[:, None] * np.uint64(cols) + np.arange(cols, dtype=np.uint64)[None, :]).ravel()
    pairs = harness("bf16", k >> np.uint64(1), np.uint16).reshape(-1, 2)
    want = np.where((k & np.uint64(1)) == 0, pairs[:, 0], pairs[:, 1]).reshape(len(rows), cols)
    assert np.array_equal(got, want)


def test_rows_are_the_float64_pair_rounded_to_bf16():
    """Element k of seed s is the k % 2 half of pair k // 2 of hash
    mix(mix(s) ^ (k // 2)), times the scale, in bf16 (within its rounding)."""
    cols = 1000
    for seed, scale in ((0, 2.0), (3, 1.0), (2**63 + 5, 0.5)):
        rows = [0, 3, 77777]
        got = workloads.synth_logit_rows(rows, cols, seed, scale).float().numpy().astype(np.float64)
        k = (np.array(rows, np.uint64)[:, None] * np.uint64(cols) + np.arange(cols, dtype=np.uint64)[None, :]).ravel()
        h = _mix_np(np.uint64(_mix(seed)) ^ (k >> np.uint64(1)))
        _, z = _box_muller64(h)
        ref = np.where((k & np.uint64(1)) == 0, z[:, 0], z[:, 1]).reshape(len(rows), cols) * scale
        assert (np.abs(got - ref) <= 2.0**-8 * np.abs(ref) + 1e-30).all(), (seed, scale)


def test_bf16_distribution_and_row_addressing():
    cols = 131072
    x = workloads.synth_logit_rows(range(64), cols, seed=1, scale=2.0).double()
    n = x.numel()
    mean, std = x.mean().item(), x.std().item()
    assert abs(mean) < 5 * 2.0 / math.sqrt(n) and abs(std - 2.0) < 0.002
    kurt = (((x - mean) / std) ** 4).mean().item()
    assert abs(kurt - 3.0) < 0.02
    # tails of a normal, beyond the old Irwin-Hall bound of 3.46 sd
    frac3 = (x.abs() > 6.0).double().mean().item()
    assert abs(frac3 - 0.0026998) < 0.0002
    assert x.abs().max().item() > 2.0 * 4.8
    # a row is the same whichever batch of rows regenerates it
    y = workloads.synth_logit_rows([7, 50, 7], cols, seed=1, scale=2.0)
    assert torch.equal(y[0], x[7].bfloat16()) and torch.equal(y[1], x[50].bfloat16()) and torch.equal(y[0], y[2])
    # seeds give different streams
    assert not torch.equal(workloads.synth_logit_rows([7], cols, seed=2), y[:1])

"""The counter-based synthetic logits on the host (meshy_synth_bf16_rows_host):
known answers from a pure-Python restatement of the documented generator, the
distribution it promises, and row addressing."""

from __future__ import annotations

import math
import struct

import numpy as np
import torch

from meshy_amd import workloads

M64 = 2**64 - 1


def _mix(x):
    x = (x + 0x9E3779B97F4A7C15) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def _f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def _element(seed, k, scale):
    """The generator as documented, in Python integers and numpy fp32."""
    h = _mix(_mix(seed) ^ k)
    s = (h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48)
    mult = np.float32(scale * math.sqrt(3.0) / 65536.0)
    x = (np.float32(s) - np.float32(131070.0)) * mult  # one fp32 rounding
    u = int(np.array([x], np.float32).view(np.uint32)[0])
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return u >> 16


def test_splitmix_finaliser_known_answer():
    # splitmix64 seeded with 0 starts 0xe220a8397b1dcdaf (Vigna's reference output)
    assert _mix(0) == 0xE220A8397B1DCDAF


def test_host_rows_equal_the_python_restatement():
    cols = 777
    for seed, scale in ((0, 2.0), (3, 1.0), (2**63 + 5, 0.5)):
        rows = [0, 1, 5, 1000003]
        got = workloads.synth_logit_rows(rows, cols, seed, scale).view(torch.int16).numpy().astype(np.uint16)
        for i, r in enumerate(rows):
            for c in (0, 1, 2, 7, 8, 500, cols - 1):
                assert got[i, c] == _element(seed, r * cols + c, scale), (seed, r, c)


def test_distribution_and_row_addressing():
    cols = 4096
    x = workloads.synth_logit_rows(range(256), cols, seed=1, scale=2.0).float()
    assert abs(x.mean().item()) < 0.01 and abs(x.std().item() - 2.0) < 0.01
    assert x.abs().max().item() <= 2 * math.sqrt(3) * 2.0 + 0.05
    # a row is the same whichever batch of rows regenerates it
    y = workloads.synth_logit_rows([7, 200, 7], cols, seed=1, scale=2.0)
    assert torch.equal(y[0], x[7].bfloat16()) and torch.equal(y[1], x[200].bfloat16()) and torch.equal(y[0], y[2])
    # seeds and scales give different streams
    assert not torch.equal(workloads.synth_logit_rows([7], cols, seed=2), y[:1])

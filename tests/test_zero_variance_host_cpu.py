"""The zero-variance filter over host tensors (meshy_zero_variance_groups_host,
no device needed): the reference's known answers (test_rollout_advantage.py:
90-93) and the oracle (rollout.py:100-115 restated with Python's max/min) on
ragged groups with NaN, +-inf, spreads at the tolerance and offsets past the
end; the flags stay on the host."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import grpo as ogrpo


def test_known_answers_on_the_host():
    from meshy_amd.advantage import zero_variance_groups

    groups = [[0.0, 0.0, 0.0], [1.0, 1.0], [0.0, 1.0], [], [1.0, 1.0 + 2e-8], [1.0, 1.0]]
    flat = torch.tensor([x for g in groups for x in g], dtype=torch.float64)
    off = torch.tensor(np.cumsum([0] + [len(g) for g in groups]))
    got = zero_variance_groups(flat, off)
    assert not got.is_cuda and got.dtype == torch.bool
    assert got.tolist() == [True, True, False, True, False, True]


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_host_filter_matches_oracle(seed):
    from meshy_amd.advantage import zero_variance_groups

    rng = np.random.default_rng(seed)
    sizes = [0, 1, 2, 8, 8, 8, 200, 3, 0, 64, 65, 8, 1, 2]
    vals, offs = [], [0]
    for i, n in enumerate(sizes):
        base = float(rng.choice([0.0, 1.0, -2.0, 1e6]))
        g = [base] * n
        kind = i % 7
        if n and kind == 1:
            g[int(rng.integers(0, n))] += 1e-8 * float(rng.choice([0.5, 1.0, 2.0]))
        elif n and kind == 2:
            g[int(rng.integers(0, n))] = math.nan
        elif n and kind == 3:
            g[0] = math.nan
        elif n and kind == 4:
            g[-1] = math.inf
        elif n and kind == 5:
            g = [float(x) for x in rng.random(n)]
        elif n and kind == 6:
            g = [-math.inf] * n  # inf - inf is NaN: not zero variance
        vals += g
        offs.append(len(vals))
    offs.append(len(vals) + 5)  # a last group that claims five more samples than there are
    for tol in (1e-8, 0.0, 2.0):
        got = zero_variance_groups(torch.tensor(vals, dtype=torch.float64), torch.tensor(offs), tol).tolist()
        clamped = offs[:-1] + [len(vals)]
        assert got == ogrpo.zero_variance_batched(vals, clamped, tol), tol
    # float32 rewards are widened to float64 first, as Python floats would be
    r32 = torch.tensor(vals, dtype=torch.float32)
    got = zero_variance_groups(r32, torch.tensor(offs)).tolist()
    assert got == ogrpo.zero_variance_batched([float(x) for x in r32.tolist()], offs[:-1] + [len(vals)])


def test_host_filter_edges():
    from meshy_amd.advantage import zero_variance_groups

    assert zero_variance_groups(torch.zeros(0, dtype=torch.float64), torch.zeros(3, dtype=torch.int64)).tolist() == [
        True, True]
    assert zero_variance_groups(torch.ones(4), torch.tensor([0])).tolist() == []
    with pytest.raises(ValueError, match="at least one entry"):
        zero_variance_groups(torch.ones(4), torch.zeros(0, dtype=torch.int64))

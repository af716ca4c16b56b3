"""GRPO advantages and the zero-variance filter over host data (the library's
host entry points, no device needed): the reference's known answers
(test_rollout_advantage.py:13-18, 90-93), the per-group plugin form on sample
objects as the rollout worker calls it, and the oracle (rollout.py:88-115
restated: torch's fp32 arithmetic for the advantages, Python's max/min for the
filter) on ragged groups with NaN, +-inf, spreads at the tolerance and offsets
past the end; results stay on the host."""

from __future__ import annotations

import math
from types import SimpleNamespace as NS

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


def test_grpo_known_answer_on_the_host():
    # test_rollout_advantage.py:13-18 (pins the unbiased std)
    from meshy_amd.advantage import grpo_advantage, grpo_advantages

    adv = grpo_advantages(torch.tensor([1.0, 2.0, 3.0]), torch.tensor([0, 3]))
    assert not adv.is_cuda and adv.tolist() == pytest.approx([-1.0, 0.0, 1.0], abs=1e-6)
    samples = [NS(reward=r, advantage=None) for r in (1.0, 2.0, 3.0)]
    grpo_advantage(samples)
    assert [s.advantage for s in samples] == pytest.approx([-1.0, 0.0, 1.0])
    assert all(type(s.advantage) is float for s in samples)
    one = [NS(reward=0.7, advantage=None)]
    grpo_advantage(one)
    assert one[0].advantage == 0.7  # a size-1 group keeps its reward
    grpo_advantage([])


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_grpo_host_matches_oracle(seed):
    """Ragged groups (size 1 to 64, all-equal groups, large and tiny spreads)
    batched and per group, against torch's fp32 arithmetic."""
    from meshy_amd.advantage import grpo_advantage, grpo_advantages

    rng = np.random.default_rng(seed)
    sizes = [1, 2, 8, 8, 3, 64, 8, 5, 1, 16]
    groups = []
    for i, n in enumerate(sizes):
        kind = i % 4
        if kind == 0:
            g = rng.integers(0, 2, n).astype(np.float32)
        elif kind == 1:
            g = np.full(n, float(rng.choice([0.0, 1.0, -3.5])), np.float32)
        elif kind == 2:
            g = (rng.standard_normal(n) * 100).astype(np.float32)
        else:
            g = (1.0 + rng.standard_normal(n) * 1e-4).astype(np.float32)
        groups.append(g)
    flat = np.concatenate(groups)
    off = np.cumsum([0] + sizes)
    got = grpo_advantages(torch.from_numpy(flat), torch.from_numpy(off))
    want = ogrpo.grpo_batched(torch.from_numpy(flat), off)

    def tol(g, ref):
        # fp32 results; a mean one rounding step away in either computation
        # moves every advantage by about that step over the spread
        spread = float(np.std(g.astype(np.float64), ddof=1)) if len(g) > 1 else 1.0
        return 1e-5 * max(max(map(abs, ref)), 1.0) + 2.0 ** -22 * float(np.abs(g).max()) / max(spread, 1e-8)

    for k, g in enumerate(groups):
        a, b = int(off[k]), int(off[k + 1])
        ref = want[a:b].tolist()
        assert (got[a:b] - want[a:b]).abs().max().item() <= tol(g, ref), k
        samples = [NS(reward=float(x), advantage=None) for x in g]
        grpo_advantage(samples)
        ref = ogrpo.grpo_group([float(x) for x in g])
        assert max(abs(s.advantage - r) for s, r in zip(samples, ref)) <= tol(g, ref), k

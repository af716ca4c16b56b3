"""The oracle's critic gauges (metrics.py:58-217, 278-328) pinned on the CPU:
the reference's own streaming-equals-window checks (test_critic_batching.py:
145-213), hand-computed answers, and independent numpy restatements of AUC,
Pearson and the variance ratio."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import critic as ocritic


def _window(rows=24, span=40, seed=0):
    # the shape of test_critic_batching.py:145-154
    g = torch.Generator().manual_seed(seed)
    mask = torch.zeros(rows, span)
    for j in range(rows):
        mask[j, 3 + j % 5:] = 1.0
    returns = torch.randn(rows, span, generator=g) * mask
    values = (returns + 0.3 * torch.randn(rows, span, generator=g)) * mask
    rewards = (torch.rand(rows, generator=g) > 0.5).float()
    groups = torch.arange(rows) // 4
    return values, returns, mask, rewards, groups


def test_streaming_equals_whole_window():
    values, returns, mask, rewards, groups = _window()
    want = ocritic.critic_diagnostics(values, returns, mask, rewards, groups)
    acc = ocritic.Accumulator()
    for lo in range(0, 24, 5):
        acc.update(values[lo:lo + 5], returns[lo:lo + 5], mask[lo:lo + 5], rewards[lo:lo + 5], groups[lo:lo + 5])
    assert ocritic.same_gauges(ocritic.diagnostics_from_states([acc.state]), want)


def test_interleaved_ranks_equal_whole_window():
    values, returns, mask, rewards, groups = _window(seed=1)
    want = ocritic.critic_diagnostics(values, returns, mask, rewards, groups)
    states = []
    for rank in range(2):
        sel = torch.arange(rank, 24, 2)
        acc = ocritic.Accumulator()
        acc.update(values[sel], returns[sel], mask[sel], rewards[sel], groups[sel])
        states.append(acc.state)
    assert ocritic.same_gauges(ocritic.diagnostics_from_states(states), want)


def test_auc_hand_computed():
    # one prompt: correct rows 0.9, 0.5; incorrect 0.5, 0.1 -> wins 1 + 1 + 0.5 + 1 of 4
    v = torch.tensor([0.9, 0.5, 0.5, 0.1])
    c = torch.tensor([True, True, False, False])
    g = torch.zeros(4, dtype=torch.long)
    assert ocritic.within_prompt_auc(v, c, g) == 0.875
    assert math.isnan(ocritic.within_prompt_auc(v, torch.ones(4, dtype=torch.bool), g))  # no incorrect row
    # a second prompt where the critic ranks backwards: 0 of 1 -> pooled 3.5 / 5
    v2 = torch.cat([v, torch.tensor([0.2, 0.8])])
    c2 = torch.cat([c, torch.tensor([True, False])])
    g2 = torch.cat([g, torch.ones(2, dtype=torch.long)])
    assert ocritic.within_prompt_auc(v2, c2, g2) == 3.5 / 5


def test_auc_and_pearson_against_numpy():
    rng = np.random.default_rng(4)
    for trial in range(20):
        n = int(rng.integers(2, 60))
        gids = rng.integers(0, max(1, n // 3), n) * 7 - 5  # arbitrary, unsorted ids
        vals = np.round(rng.normal(size=n), 1).astype(np.float32)  # ties
        rew = (rng.random(n) > 0.5).astype(np.float32)
        wins = pairs = 0.0
        for i in range(n):
            for j in range(n):
                if gids[i] == gids[j] and rew[i] >= 0.5 and rew[j] < 0.5:
                    pairs += 1
                    wins += 1.0 if vals[i] > vals[j] else (0.5 if vals[i] == vals[j] else 0.0)
        got = ocritic.within_prompt_auc(torch.from_numpy(vals), torch.from_numpy(rew >= 0.5), torch.from_numpy(gids))
        assert (math.isnan(got) and pairs == 0) or got == pytest.approx(wins / pairs, abs=1e-12)
        uniq = np.unique(gids)
        mv = np.array([vals[gids == u].astype(np.float64).mean() for u in uniq])
        mr = np.array([rew[gids == u].astype(np.float64).mean() for u in uniq])
        got = ocritic.prompt_pearson(torch.from_numpy(vals), torch.from_numpy(rew), torch.from_numpy(gids))
        if len(uniq) < 2 or mv.std() == 0 or mr.std() == 0:
            assert math.isnan(got)
        else:
            assert got == pytest.approx(np.corrcoef(mv, mr)[0, 1], abs=1e-5)


def test_variance_ratio_and_gap_closed_forms():
    values, returns, mask, _, _ = _window(seed=3)
    assert ocritic.variance_reduction(returns, returns, mask) == pytest.approx(1.0)  # V = r: nothing left
    assert ocritic.variance_reduction(torch.zeros_like(returns), returns, mask) == pytest.approx(0.0, abs=1e-6)
    assert math.isnan(ocritic.variance_reduction(values, torch.full_like(returns, 0.25), mask))  # constant r
    sel = mask.reshape(-1) > 0
    r = returns.reshape(-1)[sel].double().numpy()
    v = values.reshape(-1)[sel].double().numpy()
    assert ocritic.variance_reduction(values, returns, mask) == pytest.approx(1 - np.var(r - v) / np.var(r), rel=1e-5)
    assert ocritic.calibration_gap(returns + 0.125, returns, mask) == pytest.approx(0.125, rel=1e-6)
    # fractional mask: the gap and the loss weight by m, the ratio selects m > 0
    m = mask * 0.5
    assert ocritic.calibration_gap(returns + 0.125, returns, m) == pytest.approx(0.125, rel=1e-6)
    assert ocritic.variance_reduction(values, returns, m) == ocritic.variance_reduction(values, returns, mask)

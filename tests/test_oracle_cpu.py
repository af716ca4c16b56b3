"""Pins the CPU oracle (CPU only): the reference's known answers, closed forms,
brute force on tiny inputs and an independent float64 evaluation.  Each check
is chosen so that a plausible slip in the restatement (a dropped term, a wrong
sign or index, the biased instead of the unbiased std) fails it."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import batch as obatch
from oracle import gae as ogae
from oracle import grpo as ogrpo
from oracle import logprob as olp
from oracle import ppo as oppo
from oracle import vapo as ovapo

# ------------------------------------------------------------------ logprob


def test_logprob_oracle_against_float64_and_closed_forms():
    g = torch.Generator().manual_seed(0)
    z = (torch.randn(2, 37, 300, generator=g) * 3).to(torch.bfloat16)
    y = torch.randint(0, 300, (2, 37), generator=g)
    lp = olp.forward_logprobs(z, y, chunk=8, with_entropy=True, entropy_chunk_size=5)
    lp64, ent64, _ = olp.logprob_entropy_f64(z, y)
    assert (lp[0] - lp64).abs().max() < 1e-4
    assert (lp[1] - ent64).abs().max() < 1e-4
    # uniform logits: logp = -ln V, H = ln V
    V = 1000
    zu = torch.zeros(1, 3, V, dtype=torch.bfloat16)
    lpu, entu = olp.forward_logprobs(zu, torch.tensor([[0, 1, 999]]), with_entropy=True)
    assert torch.allclose(lpu, torch.full((1, 3), -math.log(V)), atol=1e-5)
    assert torch.allclose(entu, torch.full((1, 3), math.log(V)), atol=1e-5)
    # a two-point distribution with probabilities (p, 1-p): H = -p ln p - (1-p) ln(1-p)
    z2 = torch.full((1, 1, 2), 0.0)
    z2[0, 0, 1] = 1.0
    p = 1 / (1 + math.e)
    h = olp.chunk_entropy(z2.to(torch.bfloat16))
    assert abs(h.item() - (-p * math.log(p) - (1 - p) * math.log(1 - p))) < 1e-5
    # ignore_index
    y2 = y.clone()
    y2[0, 0] = -100
    assert olp.chunk_logprobs(z, y2)[0, 0].item() == 0.0


def test_logprob_grad_is_onehot_minus_softmax():
    g = torch.Generator().manual_seed(1)
    z = torch.randn(1, 4, 50, generator=g).to(torch.bfloat16)
    y = torch.randint(0, 50, (1, 4), generator=g)
    w = torch.randn(1, 4, generator=g)
    grad = olp.logprob_grad(z, y, w)
    p = torch.softmax(z.float(), -1)
    expect = w.unsqueeze(-1) * (torch.nn.functional.one_hot(y, 50).float() - p)
    assert torch.allclose(grad, expect, atol=1e-6)


# ------------------------------------------------------------------ GRPO


def test_grpo_oracle_known_answers():
    # test_rollout_advantage.py:13-18: [1,2,3] -> [-1,0,1] pins the unbiased std
    assert ogrpo.grpo_group([1.0, 2.0, 3.0]) == pytest.approx([-1.0, 0.0, 1.0])
    assert ogrpo.grpo_group([0.25]) == [0.25]
    assert ogrpo.grpo_group([1.0, 1.0, 1.0]) == [0.0, 0.0, 0.0]
    # one success in 8: mean 1/8, unbiased std sqrt(1/8) -> 0.875 / 0.35355
    adv = ogrpo.grpo_group([1.0] + [0.0] * 7)
    assert adv[0] == pytest.approx(0.875 / math.sqrt(1 / 8), rel=1e-6)


def test_zero_variance_oracle_known_answers():
    # test_rollout_advantage.py:90-93
    assert ogrpo.zero_variance_group([0.0, 0.0, 0.0])
    assert ogrpo.zero_variance_group([1.0, 1.0])
    assert not ogrpo.zero_variance_group([0.0, 1.0])
    assert ogrpo.zero_variance_group([])                        # rollout.py:109-110
    # the comparison is in float64: a spread of 2e-8 at 1.0 is not within 1e-8
    assert not ogrpo.zero_variance_group([1.0, 1.0 + 2e-8])
    assert ogrpo.zero_variance_group([1.0, 1.0 + 5e-9])
    assert not ogrpo.zero_variance_group([math.inf, math.inf])  # inf - inf is NaN


def test_zero_variance_oracle_against_brute_force():
    """For NaN-free groups the spread is the largest pairwise difference
    (rounding is monotone, so the pair (max, min) attains it); with NaN the
    builtins keep a NaN first element (never within) and skip later ones."""
    rng = np.random.default_rng(5)
    for _ in range(400):
        n = int(rng.integers(1, 9))
        base = float(rng.choice([0.0, 1.0, -3.5, 1e6]))
        r = [base + float(rng.choice([0.0, 0.0, 4e-9, -6e-9, 1e-8, 0.3])) for _ in range(n)]
        tol = float(rng.choice([1e-8, 0.0, 0.5]))
        want = max(a - b for a in r for b in r) <= tol
        assert ogrpo.zero_variance_group(r, tol) == want, (r, tol)
        if n > 1 and rng.random() < 0.5:
            k = int(rng.integers(0, n))
            r2 = list(r)
            r2[k] = math.nan
            rest = [x for x in r2 if not math.isnan(x)]
            want2 = k != 0 and max(a - b for a in rest for b in rest) <= tol
            assert ogrpo.zero_variance_group(r2, tol) == want2, (r2, tol)


# ------------------------------------------------------------------ PPO


class _NoCp:
    def all_reduce_sum(self, v):
        return v


def test_ppo_oracle_diagnostics_known_answers():
    # test_ppo_diagnostics.py:58-80
    rows, S = 2, 8
    mask = torch.ones(rows, S)
    mask[:, -1] = 0
    doc_ids = torch.arange(rows).unsqueeze(1).expand(rows, S).clone()
    old = -torch.ones(rows, S)
    new = (old + 0.1).requires_grad_()
    loss, sums = oppo.ppo_clip_loss(new, old, mask, doc_ids, torch.tensor([1.0, -1.0]), 2, n_docs_global=2,
                                    n_tokens_global=int(mask.sum()), clip_low=0.2, clip_high=0.28, use_tis=True,
                                    per_token_loss=True, rollout_lp=old.clone(),
                                    entropy=torch.full((rows, S), 2.0))
    red = oppo.reduce_mini_metrics(sums)
    assert red["ppo_kl"] == pytest.approx(-0.1)
    assert red["log_ratio_abs_mean"] == pytest.approx(0.1)
    assert red["ratio_mean"] == pytest.approx(math.exp(0.1))
    assert red["ess_ratio"] == pytest.approx(1.0)
    assert red["entropy"] == pytest.approx(2.0)
    assert red["train_rollout_kl"] == pytest.approx(math.exp(-0.1) + 0.1 - 1, rel=1e-4)
    assert red["train_rollout_logdiff_abs"] == pytest.approx(0.1)
    loss.backward()


def test_ppo_oracle_icepop_positive_lm_known_answers():
    # test_vapo_alignment.py:116-149
    old = torch.full((1, 3), -2.)
    new = old.clone().requires_grad_()
    roll = old - torch.tensor([[2., 6., .25]]).log()
    kw = dict(n_docs_global=1, n_tokens_global=3, clip_low=.2, clip_high=.28, use_tis=True, use_icepop=True,
              tis_min=.5, tis_max=5., positive_lm_coef=.1, positive_lm_weights=torch.tensor([.5]),
              train_lp_is_old=True)
    ids = torch.zeros(1, 3, dtype=torch.long)
    loss, sums = oppo.ppo_clip_loss(new, old, torch.ones(1, 3), ids, torch.ones(1), 1, per_token_loss=True,
                                    rollout_lp=roll, **kw)
    assert float(loss.detach()) == pytest.approx(-2 / 3 + .1, abs=1e-6)
    assert float(sums["tis_masked_sum"]) == 2. and float(sums["ratio_sum"]) == 3.
    loss.backward()
    torch.testing.assert_close(new.grad, torch.tensor([[-2.05 / 3, -.05 / 3, -.05 / 3]]))
    roll2 = old - torch.tensor([[.5, 5., 1.]]).log()
    loss, sums = oppo.ppo_clip_loss(old.clone().requires_grad_(), old, torch.ones(1, 3), ids, torch.ones(1), 1,
                                    per_token_loss=False, rollout_lp=roll2, **kw)
    assert float(sums["tis_masked_sum"]) == 0.
    assert float(loss.detach()) == pytest.approx(-6.5 / 3 + .1, abs=1e-6)


def test_ppo_oracle_clip_and_tie_gradient():
    # Hand-derived: A = 1, r in-range -> grad = -r / N; r above 1 + eps_h with A > 0 -> clipped, grad 0;
    # A < 0 and r below 1 - eps_l -> the clipped term is the min (-clamp*A larger), grad 0.
    old = torch.zeros(1, 4)
    lr = torch.tensor([[0.0, 0.5, -0.5, 0.1]])
    new = (old + lr).requires_grad_()
    adv = torch.tensor([[1.0, 1.0, -1.0, -1.0]])
    loss, _ = oppo.ppo_clip_loss(new, old, torch.ones(1, 4), torch.zeros(1, 4, dtype=torch.long), adv, 1,
                                 n_docs_global=1, n_tokens_global=4, clip_low=0.2, clip_high=0.28,
                                 per_token_loss=True)
    loss.backward()
    r = lr.exp()
    expect = torch.tensor([[-r[0, 0] / 4, 0.0, 0.0, r[0, 3] / 4]])
    assert torch.allclose(new.grad, expect, atol=1e-7)


# ------------------------------------------------------------------ GAE


def test_gae_oracle_closed_forms():
    S = 50
    mask = torch.ones(1, S)
    ids = torch.zeros(1, S, dtype=torch.long)
    R = 0.8
    rewards = torch.zeros(1, S)
    rewards[0, -1] = R
    # V = 0, terminal reward, constant lambda, gamma = 1: A_t = lambda^(S-1-t) R
    lengths = torch.full((1,), 1.0 / (1.0 - 0.9))
    adv, lam = ogae.compute_vapo_gae(rewards, torch.zeros(1, S), mask, ids, 1, lengths=lengths, gamma=1.0,
                                     alpha=1.0)
    lam_f = float(lam[0])
    assert lam_f == pytest.approx(0.9, abs=1e-6)
    assert torch.allclose(adv[0].double(), torch.tensor([lam_f ** (S - 1 - t) * R for t in range(S)],
                                                        dtype=torch.float64), atol=1e-6)
    # returns with gamma = 1: R broadcast over the run
    assert torch.allclose(ogae.compute_returns(rewards, mask, ids), torch.full((1, S), R))
    # lambda = 0 (alpha tiny): A = delta
    g = torch.Generator().manual_seed(0)
    v = torch.randn(1, S, generator=g)
    r = torch.randn(1, S, generator=g)
    adv0, _ = ogae.compute_vapo_gae(r, v, mask, ids, 1, gamma=0.7, alpha=1e-9)
    delta = r + 0.7 * torch.cat([v[:, 1:], torch.zeros(1, 1)], 1) - v
    assert torch.allclose(adv0, delta, atol=1e-6)
    # VAPO lambda from the masked length: 1 - 1/(1.5 * 50)
    _, lam2 = ogae.compute_vapo_gae(rewards, torch.zeros(1, S), mask, ids, 1)
    assert float(lam2[0]) == pytest.approx(1 - 1 / 75, abs=1e-6)


def test_gae_oracle_matches_brute_force_with_holes_and_docs():
    g = torch.Generator().manual_seed(3)
    rows, S = 3, 40
    ids = torch.tensor([[0] * 15 + [1] * 25, [2] * 40, [3] * 10 + [4] * 30])
    mask = (torch.rand(rows, S, generator=g) > 0.15).float()
    v = torch.randn(rows, S, generator=g)
    r = torch.randn(rows, S, generator=g)
    adv, lam = ogae.compute_vapo_gae(r, v, mask, ids, 5, gamma=0.95, alpha=0.2)
    bf = ogae.gae_brute_force(r, v, mask, ids, torch.cat([lam, torch.zeros(1)]), 0.95)
    assert (adv.double() - bf).abs().max() < 1e-4
    # cont is zero across a doc change and a mask hole: a reward after them never flows back
    assert ogae.continuation_mask(torch.ones(1, 4), torch.tensor([[0, 0, 1, 1]])).tolist() == [[1, 0, 1, 0]]
    assert ogae.continuation_mask(torch.tensor([[1., 0., 1., 1.]]), torch.zeros(1, 4, dtype=torch.long)).tolist() \
        == [[0, 0, 1, 0]]


def test_attach_gae_oracle_grid_shift_and_reward_placement():
    # prompt of 3 (mask 0) + response of 5; on the next-token grid the loss
    # mask is positions 2..6 and the reward sits at last - 1 = 6.
    lam, R = 0.9, 0.5
    s = {"tokens": torch.arange(8), "mask_assistant": torch.tensor([0, 0, 0, 1, 1, 1, 1, 1.]),
         "values": torch.zeros(8), "reward": torch.tensor(R)}
    empty = {"tokens": torch.arange(4), "mask_assistant": torch.zeros(4), "values": torch.ones(4),
             "reward": torch.tensor(1.0)}
    first_only = {"tokens": torch.arange(3), "mask_assistant": torch.tensor([1., 0, 0]), "values": torch.zeros(3),
                  "reward": torch.tensor(1.0)}
    adv, metrics = ogae.attach_gae_advantages([s, empty, first_only], seq_len=100, gae_lambda=lam)
    lam_f = float(1.0 - 1.0 / float(torch.tensor(1.0 / (1.0 - lam), dtype=torch.float32)))
    expect = torch.tensor([0, 0, lam_f ** 4 * R, lam_f ** 3 * R, lam_f ** 2 * R, lam_f * R, R, 0], dtype=torch.float64)
    assert torch.allclose(adv[0].double(), expect, atol=1e-6)
    assert adv[1].abs().sum() == 0 and adv[2].abs().sum() == 0  # no response / response at 0: no reward
    # 'empty' has values 1 but no loss tokens; first_only has none either: 5 loss tokens in all
    assert metrics["critic/value_mean"] == 0.0
    assert metrics["critic/advantage_mean"] == pytest.approx(float(expect.sum()) / 5, rel=1e-5)
    assert metrics["critic/advantage_seq_mean"] == pytest.approx(float(expect.sum()) / 5 / 3, rel=1e-5)
    assert metrics["critic/lambda_mean"] == pytest.approx(lam, abs=1e-6)
    # truncation to seq_len: the sample is cut to 6 tokens, its last response token is 5
    adv_t, _ = ogae.attach_gae_advantages([s], seq_len=6, gae_lambda=lam)
    assert adv_t[0].shape == (6,) and adv_t[0][4] == R


# ------------------------------------------------------------------ whitening


def test_whitening_oracle_known_answers():
    # test_vapo_alignment.py:39-46
    def row(vals):
        return {ovapo.ADVANTAGE_TOKENS: torch.tensor(vals, dtype=torch.float32),
                "mask_assistant": torch.tensor([0] + [1] * (len(vals) - 1))}

    s = row([2., 4., 1000.])
    ovapo.whiten_advantages([s], 3)
    torch.testing.assert_close(s[ovapo.ADVANTAGE_TOKENS], torch.tensor([-2 ** -.5, 2 ** -.5, 0.]))
    s = row([2., 2., 1000.])
    ovapo.whiten_advantages([s], 3)
    assert s[ovapo.ADVANTAGE_TOKENS].abs().sum() == 0
    # replication divides the statistics: two copies of [1,2] with replication 2 == [1,2] once
    a, b = row([1., 2., 9.]), row([1., 2., 9.])
    ovapo.whiten_advantages([a, b], 3, replication=2)
    c = row([1., 2., 9.])
    ovapo.whiten_advantages([c], 3)
    torch.testing.assert_close(a[ovapo.ADVANTAGE_TOKENS], c[ovapo.ADVANTAGE_TOKENS])


# ------------------------------------------------------------------ batch


def _sample(length, prompt=3, adv=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    mask = torch.ones(length)
    mask[:prompt] = 0
    return {"tokens": torch.randint(1, 1000, (length,), generator=g), "logprobs": torch.randn(length, generator=g),
            "mask_assistant": mask, "advantage": torch.tensor(adv)}


def test_batch_oracle_known_answers():
    # test_dynamic_batching.py:259-285, 288-294, 297-306, 309-316
    samples = [_sample(10, seed=1), _sample(6, seed=2, adv=2.0)]
    mb = obatch.build_micro_batch(samples, (0, 1), 32, (10, 6), layout="packed", need_rollout_lp=True)
    assert torch.equal(mb["cu_seqlens"], torch.tensor([0, 10, 16, 32], dtype=torch.int32))
    assert mb["max_seqlen"] == 16
    assert mb["mask"][0, 9] == 0 and mb["mask"][0, 15] == 0
    assert torch.equal(mb["positions"][0, 16:], torch.arange(16, dtype=torch.int32))
    assert (mb["doc_ids"][0, 16:] == 2).all()
    assert torch.allclose(mb["advantages"], torch.tensor([1.0, 2.0]))
    mb = obatch.build_micro_batch([_sample(8, seed=3)], (0,), 8, (8,), layout="packed", need_rollout_lp=False)
    assert torch.equal(mb["cu_seqlens"], torch.tensor([0, 8], dtype=torch.int32))
    for layout in ("padded", "packed"):
        mb = obatch.build_micro_batch([], (), 64, (), layout=layout, need_rollout_lp=True)
        assert mb["n_docs"] == 0 and (mb["doc_ids"] == 0).all() and mb["advantages"].numel() == 0
    mb = obatch.build_micro_batch([_sample(20, seed=4)], (0,), 16, (12,), layout="padded", need_rollout_lp=False)
    assert mb["labels"][0, 11] == 0 and mb["mask"][0, 11] == 0 and int(mb["lengths"][0]) == 12


# ------------------------------------------------------------------ the C ABI


def test_library_exports_every_header_symbol():
    import re

    from meshy_amd import _lib

    lib = _lib.load()
    with open(_lib.os.path.join(_lib.os.path.dirname(_lib.LIB_PATH), "..", "include", "meshy_amd.h")) as f:
        header = f.read()
    declared = set(re.findall(r"\b(meshy_[a-z0-9_]+)\s*\(", header))
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    assert lib.meshy_abi_version() == _lib.ABI_VERSION

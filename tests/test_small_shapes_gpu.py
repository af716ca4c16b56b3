"""The smallest non-empty shapes against the oracle: one token, one position
per row, one row, every token masked out."""

from __future__ import annotations

import pytest
import torch

from oracle import critic as ocritic
from oracle import gae as ogae
from oracle import ppo as oppo
from oracle import vapo as ovapo

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    return torch.device("cuda:0")


@pytest.mark.parametrize("per_token", [True, False])
def test_ppo_one_token_one_document(dev, per_token):
    from types import SimpleNamespace as NS

    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    new = torch.tensor([[-0.7]])
    old = torch.tensor([[-1.1]])
    mask = torch.ones(1, 1)
    ids = torch.zeros(1, 1, dtype=torch.long)
    adv = torch.tensor([0.8])
    z = torch.zeros(1, 1, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask.to(dev), ids.to(dev), adv.to(dev), None, torch.zeros(1, device=dev), 1)
    stub = NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, use_icepop=False,
              calculate_per_token_loss=per_token, old_logprobs_source="rollout", sharder=None, parallel_dims=NS(cp=1))
    nd = new.to(dev).requires_grad_(True)
    loss, sums = ppo_clip_loss(stub, nd, old.to(dev), mb, MiniPlan((), 1, 1, ()))
    loss.backward()
    nr = new.clone().requires_grad_(True)
    ref_loss, ref_sums = oppo.ppo_clip_loss(nr, old, mask, ids, adv, 1, n_docs_global=1, n_tokens_global=1,
                                            clip_low=0.2, clip_high=0.28, per_token_loss=per_token)
    ref_loss.backward()
    assert loss.item() == pytest.approx(ref_loss.item(), abs=1e-6)
    assert nd.grad.cpu().item() == pytest.approx(nr.grad.item(), abs=1e-6)
    for k, v in ref_sums.items():
        if k in sums:
            assert sums[k].item() == pytest.approx(float(v), abs=1e-6), k


def test_gae_rows_of_one_position(dev):
    """[rows, 1]: every position ends its row, so A = r - V and G = r where valid."""
    from meshy_amd.gae import compute_returns, compute_vapo_gae

    g = torch.Generator().manual_seed(3)
    rows = 7
    rewards = torch.randn(rows, 1, generator=g)
    values = torch.randn(rows, 1, generator=g)
    mask = (torch.rand(rows, 1, generator=g) > 0.3).float()
    ids = torch.arange(rows).reshape(rows, 1)
    ref_adv, ref_lam = ogae.compute_vapo_gae(rewards, values, mask, ids, rows, gamma=0.99, alpha=1.5)
    ref_ret = ogae.compute_returns(rewards, mask, ids, gamma=0.99)
    d = [t.to(dev) for t in (rewards, values, mask, ids)]
    adv, lam = compute_vapo_gae(*d, rows, gamma=0.99, alpha=1.5)
    ret = compute_returns(d[0], d[2], d[3], gamma=0.99)
    assert torch.allclose(adv.cpu(), ref_adv, atol=1e-6) and torch.allclose(ret.cpu(), ref_ret, atol=1e-6)
    assert torch.allclose(lam.cpu(), ref_lam, atol=1e-7)


def test_whitening_with_every_token_masked_out(dev):
    """No token selected: the reference's count clamp gives mean 0 and
    variance 0, and every advantage outside the mask becomes 0."""
    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.vapo import whiten_advantages

    vals = [3.0, -1.0, 7.5, 2.0]
    s = {ADVANTAGE_TOKENS: torch.tensor(vals), "mask_assistant": torch.zeros(4)}
    r = {ovapo.ADVANTAGE_TOKENS: torch.tensor(vals), "mask_assistant": torch.zeros(4)}
    whiten_advantages([s], 4, dev)
    ovapo.whiten_advantages([r], 4)
    assert torch.equal(s[ADVANTAGE_TOKENS].cpu(), r[ovapo.ADVANTAGE_TOKENS])


def test_critic_diagnostics_of_one_row_and_one_token(dev):
    from meshy_amd import critic

    v = torch.tensor([[0.4]])
    r = torch.tensor([[1.0]])
    m = torch.ones(1, 1)
    rew = torch.tensor([1.0])
    grp = torch.tensor([5])
    got = critic.critic_diagnostics(v.to(dev), r.to(dev), m.to(dev), rew.to(dev), grp.to(dev)).as_dict()
    want = ocritic.critic_diagnostics(v, r, m, rew, grp)
    assert ocritic.same_gauges(got, want, rel=1e-5, abs_=1e-6), (got, want)

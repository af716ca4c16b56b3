"""Zero-size inputs through every device entry point: no launch error, outputs
of the right (empty) shape, and the reference's values where it defines them
(an empty masked mean is 0, an empty group list gives no advantages)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    return torch.device("cuda:0")


def test_logprob_entropy_and_backward_of_no_tokens(dev):
    from meshy_amd import logprob

    z = torch.zeros(1, 0, 1000, dtype=torch.bfloat16, device=dev, requires_grad=True)
    y = torch.zeros(1, 0, dtype=torch.long, device=dev)
    lp, h = logprob.logprobs_and_entropy(z, y, with_entropy=True)
    assert lp.shape == (1, 0) and h.shape == (1, 0)
    lp.sum().backward()
    assert z.grad.shape == z.shape
    assert logprob.chunk_logprobs(z.detach(), y).shape == (1, 0)
    assert logprob.chunk_entropy(z.detach()).shape == (1, 0)


def test_topk_and_gather_of_no_tokens(dev):
    from meshy_amd import topk

    z = torch.zeros(1, 0, 1000, dtype=torch.bfloat16, device=dev)
    ids, lps = topk.teacher_topk(z, 8)
    assert ids.shape == (1, 0, 8) and lps.shape == (1, 0, 8)
    g = topk.gather_logprobs(z, torch.zeros(1, 0, 9, dtype=torch.long, device=dev))
    assert g.shape == (1, 0, 9)


def test_gae_of_no_tokens_and_no_documents(dev):
    from meshy_amd.gae import compute_returns, gae_and_returns

    e = torch.zeros(1, 0, device=dev)
    ids = torch.zeros(1, 0, dtype=torch.long, device=dev)
    adv, ret, lam = gae_and_returns(e, e, e, ids, 0)
    assert adv.shape == (1, 0) and ret.shape == (1, 0) and lam.numel() == 0
    assert compute_returns(e, e, ids).shape == (1, 0)
    # documents but no tokens: lambda of empty documents (length 0 -> max(L, 1) = 1)
    adv, ret, lam = gae_and_returns(e, e, e, ids, 3, alpha=2.0)
    assert lam.shape == (3,) and torch.allclose(lam.cpu(), torch.full((3,), 0.5))


def test_group_advantages_of_no_groups(dev):
    from meshy_amd.advantage import grpo_advantages, zero_variance_groups

    adv = grpo_advantages(torch.zeros(0, device=dev), torch.zeros(1, dtype=torch.long, device=dev))
    assert adv.numel() == 0
    flags = zero_variance_groups(torch.zeros(0, dtype=torch.float64, device=dev),
                                 torch.zeros(1, dtype=torch.long, device=dev))
    assert flags.numel() == 0


def test_whitening_and_critic_reductions_of_no_tokens(dev):
    from meshy_amd import critic, vapo

    e = torch.zeros(0, device=dev)
    assert vapo.whiten_flat(e, e).numel() == 0
    ids = torch.zeros(0, dtype=torch.long, device=dev)
    assert critic.advantages_to_per_sequence(e, e, ids, 0).numel() == 0
    v = torch.zeros(0, device=dev, requires_grad=True)
    err = critic.clipped_value_error(v, e, e, 0.2)
    err.sum().backward()
    assert err.numel() == 0 and v.grad.numel() == 0
    acc = critic.Accumulator()
    grid = torch.zeros(2, 0, device=dev)
    acc.update(grid, grid, grid, torch.ones(2, device=dev), torch.arange(2, device=dev))
    st = acc.state
    assert st.n_tokens == 0.0 and st.row_value == [0.0, 0.0] and st.row_group == [0, 1]


def test_ppo_loss_of_no_tokens(dev):
    """Two documents without tokens: loss and every sum 0, an empty gradient."""
    from types import SimpleNamespace as NS

    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    e = torch.zeros(1, 0, device=dev)
    ids = torch.zeros(1, 0, dtype=torch.long, device=dev)
    mb = Batch(ids, ids, ids.int(), e, ids, torch.zeros(2, device=dev), None, torch.zeros(2, device=dev), 2)
    stub = NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, use_icepop=False,
              calculate_per_token_loss=True, old_logprobs_source="rollout", sharder=None, parallel_dims=NS(cp=1))
    new = torch.zeros(1, 0, device=dev, requires_grad=True)
    loss, sums = ppo_clip_loss(stub, new, e, mb, MiniPlan((), 2, 0, ()))
    loss.backward()
    assert loss.item() == 0.0 and new.grad.shape == (1, 0)
    assert all(v.item() == 0.0 for v in sums.values())


def test_rollout_metrics_of_samples_without_tokens(dev):
    """Samples whose token, mask and log-prob columns are all empty: the
    oracle's statistics (zero response lengths, no kept log-probs)."""
    from oracle import rollout_metrics as orm

    from meshy_amd.rollout_metrics import rollout_metrics

    samples = [{"tokens": torch.zeros(0, dtype=torch.long), "logprobs": torch.zeros(0),
                "mask_assistant": torch.zeros(0), "reward": torch.tensor(float(i % 2))} for i in range(3)]
    m, hist = rollout_metrics(samples, seq_len=64)
    rm, rh = orm.rollout_metrics(samples, seq_len=64)
    assert set(m) == set(rm) and set(hist) == set(rh)
    for k, v in rm.items():
        assert m[k] == pytest.approx(v, abs=1e-6), k

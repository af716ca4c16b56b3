"""The composed path at T = 16384 against the oracle chain.

The 256 GRPO samples (32 groups of 8) are planned under a budget of 8192
tokens and packed with their GRPO advantages in one step; the first two
micros (8192 tokens each) then take logits rows [0, 8192) and [8192, 16384)
of one bf16 [16384, 151936] tensor through the fused log-prob + entropy, the
clipped PPO loss (token mean, eps 0.2 / 0.28, old = rollout log-probs) and its
backward into the logits.  Per micro, the loss and every diagnostic sum,
dLoss/dnew_lp and dLoss/dlogits are compared with the oracle's chain
(plan.py:211-288, batch.py:96-230, rollout.py:88-97, trainer.py:451-527,
705-848) on the same inputs.
"""

from __future__ import annotations

import math
from types import SimpleNamespace as NS

import pytest
import torch

from oracle import batch as obatch
from oracle import grpo as ogrpo
from oracle import logprob as olp
from oracle import plan as oplan
from oracle import ppo as oppo

pytestmark = pytest.mark.gpu

TOL = 1e-3
V = 151936
MICRO = 8192


class _NoCp:
    enabled = False

    def shard_seq(self, *tensors):
        return tensors


def _stub():
    return NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, use_icepop=False,
              tis_ratio_min=0.5, tis_ratio_max=5.0, calculate_per_token_loss=True,
              positive_lm_loss_coef=0.0, old_logprobs_source="rollout", sharder=_NoCp(),
              parallel_dims=NS(cp=1))


def _close(a: float, b: float) -> bool:
    """Within 1e-3 absolute (the bar; relative for sums over many tokens), and
    within 1e-3 relative, which is the binding test for the small values the
    chain produces (the loss is O(1e-1), per-token gradients O(1e-5))."""
    return math.isfinite(a) and abs(a - b) <= TOL * max(1.0, abs(b)) and abs(a - b) <= TOL * abs(b) + 1e-9


def test_composed_path_matches_the_oracle_chain(dev):
    from meshy_amd import logprob, workloads
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    cfg = PlannerConfig(layout="packed", mini_batch_size=256, seq_len=MICRO, align=2048,
                        max_tokens_per_micro=MICRO)
    res = pack_step(ragged, cfg, dev)
    mini = res.plan.per_rank[0][0]
    mbs = res.batches[:2]
    assert [mb.input_ids.shape[1] for mb in mbs] == [MICRO, MICRO]
    gen = torch.Generator(device=dev).manual_seed(5)
    logits = torch.randn(1, 2 * MICRO, V, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0
    stub = _stub()
    gpu = []
    for j, mb in enumerate(mbs):
        z = logits[:, j * MICRO:(j + 1) * MICRO].detach().requires_grad_(True)
        lp, ent = logprob.logprobs_and_entropy(z, mb.labels, with_entropy=True)
        lp.retain_grad()
        loss, sums = ppo_clip_loss(stub, lp, mb.rollout_logprobs, mb, mini, entropy=ent)
        loss.backward()
        gpu.append((loss.item(), {k: float(v) for k, v in sums.items()}, lp.grad.cpu(), z.grad.cpu()))

    # The oracle chain on the same samples and logits.
    samples = batch.sample_dicts(rewards=rewards)
    lengths, loss_t = oplan.sample_lengths(samples, MICRO)
    local, per_rank = oplan.build_plan(lengths, loss_t, 1, layout="packed", mini_batch_size=256, seq_len=MICRO,
                                       align=2048, max_tokens_per_micro=MICRO)
    adv = []
    for g in range(len(group_offsets) - 1):
        adv += ogrpo.grpo_group([float(rewards[i]) for i in range(group_offsets[g], group_offsets[g + 1])])
    loc = [dict(samples[i], advantage=torch.tensor(adv[i])) for i in local[0]]
    micros, n_docs_g, n_tok_g, _ = per_rank[0][0]
    assert (mini.n_docs_global, mini.n_tokens_global) == (n_docs_g, n_tok_g)
    for j in range(2):
        idx, seq_len, doc_lens = micros[j]
        ref = obatch.build_micro_batch(loc, idx, seq_len, doc_lens, layout="packed", need_rollout_lp=True)
        mb = mbs[j]
        for k in ("labels", "doc_ids", "mask", "rollout_logprobs"):
            assert torch.equal(getattr(mb, k).cpu(), ref[k]), k
        assert (mb.advantages.cpu() - ref["advantages"]).abs().max().item() <= TOL
        zc = logits[:, j * MICRO:(j + 1) * MICRO].cpu().float().requires_grad_(True)
        lp = olp.forward_logprobs(zc, ref["labels"])
        with torch.no_grad():
            ent = olp.chunk_entropy(zc.detach())
        lp.retain_grad()
        ref_loss, ref_sums = oppo.ppo_clip_loss(
            lp, ref["rollout_logprobs"], ref["mask"], ref["doc_ids"], ref["advantages"], ref["n_docs"],
            n_docs_global=n_docs_g, n_tokens_global=n_tok_g, clip_low=0.2, clip_high=0.28,
            per_token_loss=True, entropy=ent, rollout_lp=ref["rollout_logprobs"])
        ref_loss.backward()

        loss, sums, g_new, g_z = gpu[j]
        print(f"micro {j}: loss {loss:.6e} ref {ref_loss.item():.6e}", flush=True)
        assert _close(loss, ref_loss.item())
        assert set(sums) == set(ref_sums)
        for k, b in ref_sums.items():
            assert _close(sums[k], float(b)), (k, sums[k], float(b))
        rg = lp.grad
        assert (g_new - rg).abs().max().item() <= TOL * rg.abs().max().item()
        # dLoss/dlogits in bf16: each element within its rounding (2^-8 relative
        # to the row's |dLoss/dlp|, the largest any element of the row can reach).
        rz = zc.grad
        gmax = rg.abs().reshape(-1)
        for a in range(0, MICRO, 1024):
            got = g_z[0, a:a + 1024].float()
            assert torch.isfinite(got).all()
            assert ((got - rz[0, a:a + 1024]).abs() <= 4e-3 * gmax[a:a + 1024, None] + 1e-30).all(), a

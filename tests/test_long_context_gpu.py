"""Long context: 16 sequences with lengths U{8192..131072} (seed 3) packed
under a 131072-token budget (align 2048), then the fused log-prob + entropy
and its backward over the largest micro's bf16 logits [T, 131072].

* every micro the GPU pack materialises is bit-exact against the oracle's
  build_micro_batch (batch.py:142-178) for the native plan (plan.py:211-288,
  itself pinned by the golden plans);
* logp and entropy (trainer.py:414-449) on 8192 seeded rows of every micro
  (all rows of a shorter one), labels being that micro's packed labels, within
  1e-3 of the oracle.  The logits [T, 131072] are N(0, 2^2) from the
  counter-based Box-Muller generator on the device, and the host regenerates
  the checked rows instead of copying them;
* the logits gradient of the whole largest micro (trainer.py:504-517) on 1024
  seeded rows within the bf16 rounding of the oracle's fp32 autograd gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import batch as obatch
from oracle import logprob as olp

pytestmark = pytest.mark.gpu

V = 131072
BUDGET = 131072
TOL = 1e-3


class _NoCp:
    enabled = False

    def shard_seq(self, *tensors):
        return tensors


@pytest.fixture(scope="module")
def long_micros(dev):
    from meshy_amd import workloads
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import PlannerConfig, build_plan

    lengths = workloads.long_context_16_lengths(3)
    rng = np.random.default_rng(33)
    prompt = rng.integers(64, 257, len(lengths))
    batch = workloads.RaggedBatch(prompt, lengths - prompt, rng, vocab=V)
    samples = batch.sample_dicts()
    cfg = PlannerConfig(layout="packed", mini_batch_size=len(lengths), seq_len=BUDGET, align=2048,
                        max_tokens_per_micro=BUDGET)
    plan = build_plan(lengths.tolist(), batch.loss_tokens(BUDGET).tolist(), 1, cfg)
    micros = [m for mini in plan.per_rank[0] for m in mini.micros]
    samples = plan.local_samples(samples, 0)  # MicroPlan.sample_idx indexes the rank-local list
    mbs = build_micro_batches(samples, micros, layout="packed", device=dev, sharder=_NoCp(),
                              need_rollout_lp=True)
    return samples, micros, mbs


def test_every_long_micro_bit_exact(long_micros):
    samples, micros, mbs = long_micros
    assert len(mbs) == len(micros) and max(m.seq_len for m in micros) <= BUDGET
    for mb, m in zip(mbs, micros):
        ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout="packed",
                                       need_rollout_lp=True)
        for k in ("input_ids", "labels", "positions", "mask", "doc_ids", "rollout_logprobs"):
            got = getattr(mb, k).cpu()
            assert got.dtype == ref[k].dtype and torch.equal(got, ref[k]), k
        assert torch.equal(mb.attention_masks.cu_seq_q.cpu(), ref["cu_seqlens"])
        assert mb.attention_masks.max_q == ref["max_seqlen"]


N_MICROS = 7  # the plan of the 16 seeded lengths (asserted below)


@pytest.mark.parametrize("j", range(N_MICROS))
def test_logprob_on_every_long_micro(dev, long_micros, j):
    """Logits of micro j are N(0, 2^2) from the counter-based generator (seed 100 + j)
    on the device; the host regenerates 8192 seeded rows (all rows of a shorter
    micro) bit for bit and the oracle checks logp and entropy there."""
    from meshy_amd import logprob, workloads

    _, micros, mbs = long_micros
    assert len(micros) == N_MICROS
    labels = mbs[j].labels
    T = labels.shape[1]
    assert int(labels.max()) < V
    z = workloads.synth_logits(T, V, seed=100 + j, device=dev).unsqueeze(0)
    lp, ent = logprob.logprobs_and_entropy(z, labels, with_entropy=True)
    assert torch.isfinite(lp).all() and torch.isfinite(ent).all()
    n = min(T, 8192)
    rows = np.sort(np.random.default_rng(7 + j).choice(T, n, replace=False))
    zs = workloads.synth_logit_rows(rows, V, seed=100 + j)
    probe = torch.from_numpy(rows[[0, n // 2, n - 1]]).to(dev)
    assert torch.equal(z[0, probe].cpu(), zs[[0, n // 2, n - 1]])  # the host rows are the device's
    rows_t = torch.from_numpy(rows).to(dev)
    lp_s, ent_s, ys = lp[0, rows_t].cpu(), ent[0, rows_t].cpu(), labels[0, rows_t].cpu()
    worst_lp = worst_ent = 0.0
    for a in range(0, n, 1024):
        zc = zs[a:a + 1024].unsqueeze(0)
        worst_lp = max(worst_lp, (lp_s[a:a + 1024] - olp.chunk_logprobs(zc, ys[a:a + 1024].unsqueeze(0))[0])
                       .abs().max().item())
        worst_ent = max(worst_ent, (ent_s[a:a + 1024] - olp.chunk_entropy(zc)[0]).abs().max().item())
    print(f"micro {j}: T={T} V={V}, {n} seeded rows: max|dlogp|={worst_lp:.2e} max|dH|={worst_ent:.2e}", flush=True)
    assert worst_lp <= TOL and worst_ent <= TOL


def test_backward_on_the_largest_long_micro(dev, long_micros):
    """The logits gradient of the whole largest micro (trainer.py:504-517),
    checked on 1024 seeded rows regenerated on the host, within the bf16
    rounding of the oracle's fp32 autograd gradient."""
    from meshy_amd import logprob, workloads

    _, micros, mbs = long_micros
    j = max(range(len(micros)), key=lambda i: micros[i].seq_len)
    labels = mbs[j].labels
    T = labels.shape[1]
    print(f"largest long micro: T={T} V={V} ({T * V * 2 / 1e9:.1f} GB of logits)", flush=True)
    assert T >= 8192
    z = workloads.synth_logits(T, V, seed=100 + j, device=dev).unsqueeze(0)
    g = torch.randn(1, T, generator=torch.Generator().manual_seed(8)).to(dev)
    zg = z.requires_grad_(True)
    lpg = logprob.logprobs_and_entropy(zg, labels)
    (lpg * g).sum().backward()
    grad = zg.grad
    assert grad.shape == z.shape and grad.dtype == torch.bfloat16
    rows = np.sort(np.random.default_rng(9).choice(T, 1024, replace=False))
    rows_t = torch.from_numpy(rows).to(dev)
    got = grad[0, rows_t].float().cpu()
    ref = olp.logprob_grad(workloads.synth_logit_rows(rows, V, seed=100 + j).unsqueeze(0),
                           labels[0, rows_t].cpu().unsqueeze(0), g[0, rows_t].cpu().unsqueeze(0))[0]
    gr = g[0, rows_t].cpu().abs()
    assert torch.isfinite(got).all()
    assert ((got - ref).abs() <= 4e-3 * gr[:, None] + 1e-30).all()

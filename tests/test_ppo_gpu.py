"""Clipped PPO loss on the GPU: the reference's known answers
(tests/test_ppo_diagnostics.py:58-95, tests/test_vapo_alignment.py:116-149)
and the oracle (the reference's torch restatement, autograd for gradients).
Tolerance: 1e-3 absolute on loss, diagnostics and gradients."""

from __future__ import annotations

import math
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import ppo as oppo

pytestmark = pytest.mark.gpu
TOL = 1e-3


class _NoCp:
    enabled = False

    def all_reduce_sum(self, value):
        return value


def _stub(**kw):
    base = dict(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=True, tis_ratio_min=0.5,
                tis_ratio_max=5.0, calculate_per_token_loss=True, old_logprobs_source="rollout",
                sharder=_NoCp(), parallel_dims=NS(cp=1))
    base.update(kw)
    return NS(**base)


def _batch(dev, rows=2, S=8):
    from meshy_amd.batch import Batch

    mask = torch.ones(rows, S)
    mask[:, -1] = 0
    doc_ids = torch.arange(rows).unsqueeze(1).expand(rows, S).clone()
    return Batch(
        input_ids=torch.zeros(rows, S, dtype=torch.long, device=dev),
        labels=torch.zeros(rows, S, dtype=torch.long, device=dev),
        positions=torch.zeros(rows, S, dtype=torch.int32, device=dev),
        mask=mask.to(dev), doc_ids=doc_ids.to(dev), advantages=torch.tensor([1.0, -1.0], device=dev),
        rollout_logprobs=None, lengths=torch.tensor([S, S], dtype=torch.int32, device=dev), n_docs=rows,
    )


def test_reports_kl_and_ess(dev):
    # test_ppo_diagnostics.py:58-80
    from meshy_amd.loss import ppo_clip_loss, reduce_mini_metrics
    from meshy_amd.plan import MiniPlan

    mb = _batch(dev)
    mini = MiniPlan(micros=(), n_docs_global=2, n_tokens_global=int(mb.mask.sum()), tokens_per_rank=(16,))
    old = -torch.ones(2, 8, device=dev)
    new = (old + 0.1).requires_grad_()
    mb.rollout_logprobs = old.clone()
    loss, sums = ppo_clip_loss(_stub(), new, old, mb, mini, entropy=torch.full((2, 8), 2.0, device=dev))
    red = reduce_mini_metrics(NS(parallel_dims=NS(get_optional_mesh=lambda name: None)), sums)
    assert red["ppo_kl"] == pytest.approx(-0.1, abs=1e-6)
    assert red["log_ratio_abs_mean"] == pytest.approx(0.1, abs=1e-6)
    assert red["ratio_mean"] == pytest.approx(math.exp(0.1), rel=1e-6)
    assert red["ess_ratio"] == pytest.approx(1.0, rel=1e-6)
    assert red["entropy"] == pytest.approx(2.0, rel=1e-6)
    assert red["train_rollout_kl"] == pytest.approx(math.exp(-0.1) + 0.1 - 1, rel=1e-4)
    assert red["train_rollout_logdiff_abs"] == pytest.approx(0.1, rel=1e-5)
    assert sums["token_count"].item() == float(mb.mask.sum())
    loss.backward()


def test_ess_drops_with_uneven_weights(dev):
    # test_ppo_diagnostics.py:83-95
    from meshy_amd.loss import ppo_clip_loss, reduce_mini_metrics
    from meshy_amd.plan import MiniPlan

    mb = _batch(dev)
    mini = MiniPlan(micros=(), n_docs_global=2, n_tokens_global=int(mb.mask.sum()), tokens_per_rank=(16,))
    old = torch.zeros(2, 8, device=dev)
    new = torch.zeros(2, 8, device=dev)
    new[:, 0] = 1.5
    _, sums = ppo_clip_loss(_stub(), new, old, mb, mini)
    red = reduce_mini_metrics(NS(parallel_dims=NS(get_optional_mesh=lambda name: None)), sums)
    assert 0.0 < red["ess_ratio"] < 1.0
    assert "train_rollout_kl" not in red


def test_icepop_and_positive_lm_gradient(dev):
    # test_vapo_alignment.py:116-149
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    stub = NS(ppo_clip_eps_low=.2, ppo_clip_eps_high=.28, use_tis=True, use_icepop=True, tis_ratio_min=.5,
              tis_ratio_max=5., calculate_per_token_loss=True, positive_lm_loss_coef=.1,
              old_logprobs_source="train", sharder=NS(all_reduce_sum=lambda x: x), parallel_dims=NS(cp=1))
    old = torch.full((1, 3), -2., device=dev)
    new = old.clone().requires_grad_()
    z = torch.zeros(1, 3, dtype=torch.long, device=dev)
    batch = Batch(z, z, z.int(), torch.ones(1, 3, device=dev), z.clone(), torch.ones(1, device=dev),
                  old - torch.tensor([[2., 6., .25]], device=dev).log(), torch.tensor([3], device=dev), 1,
                  positive_lm_weights=torch.tensor([.5], device=dev))
    mini = MiniPlan(micros=(), n_docs_global=1, n_tokens_global=3, tokens_per_rank=(3,))
    loss, sums = ppo_clip_loss(stub, new, old, batch, mini)
    assert float(loss.detach()) == pytest.approx(-2 / 3 + .1, abs=1e-6)
    assert float(sums["tis_masked_sum"]) == 2.
    assert float(sums["ratio_sum"]) == 3.
    loss.backward()
    torch.testing.assert_close(new.grad.cpu(), torch.tensor([[-2.05 / 3, -.05 / 3, -.05 / 3]]))
    stub.calculate_per_token_loss = False
    batch.rollout_logprobs = old - torch.tensor([[.5, 5., 1.]], device=dev).log()
    loss, sums = ppo_clip_loss(stub, old.clone().requires_grad_(), old, batch, mini)
    assert float(sums["tis_masked_sum"]) == 0.
    assert float(loss.detach()) == pytest.approx(-6.5 / 3 + .1, abs=1e-6)
    stub.use_icepop = False
    stub.positive_lm_loss_coef = 0.
    loss, sums = ppo_clip_loss(stub, old, old, batch, mini)
    assert float(loss) == pytest.approx(-1., abs=1e-6)


def _compare(dev, new, old, mask, doc_ids, adv, n_docs, *, rollout=None, entropy=None, pos_w=None,
             nonfinite=False, **cfg):
    """Kernel vs oracle: loss, every sum, and d loss / d new."""
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    n_docs_global = cfg.pop("n_docs_global", n_docs)
    n_tokens_global = cfg.pop("n_tokens_global", int(mask.sum()))
    stub = NS(ppo_clip_eps_low=cfg.get("clip_low", 0.2), ppo_clip_eps_high=cfg.get("clip_high", 0.28),
              use_tis=cfg.get("use_tis", False), use_icepop=cfg.get("use_icepop", False),
              tis_ratio_min=cfg.get("tis_min", 0.5), tis_ratio_max=cfg.get("tis_max", 5.0),
              calculate_per_token_loss=cfg.get("per_token_loss", True),
              positive_lm_loss_coef=cfg.get("positive_lm_coef", 0.0),
              old_logprobs_source="train" if cfg.get("train_lp_is_old") else "rollout",
              sharder=_NoCp(), parallel_dims=NS(cp=1))
    rows, S = new.shape
    z = torch.zeros(rows, S, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask.to(dev), doc_ids.to(dev), adv.to(dev),
               None if rollout is None else rollout.to(dev), torch.zeros(max(n_docs, 1), device=dev), n_docs,
               positive_lm_weights=None if pos_w is None else pos_w.to(dev))
    mini = MiniPlan(micros=(), n_docs_global=n_docs_global, n_tokens_global=n_tokens_global, tokens_per_rank=())
    nd = new.to(dev).requires_grad_(True)
    loss, sums = ppo_clip_loss(stub, nd, old.to(dev), mb, mini, entropy=None if entropy is None else entropy.to(dev))
    loss.backward()
    nr = new.clone().requires_grad_(True)
    ref_loss, ref_sums = oppo.ppo_clip_loss(
        nr, old, mask, doc_ids, adv, n_docs, n_docs_global=n_docs_global, n_tokens_global=n_tokens_global,
        clip_low=stub.ppo_clip_eps_low, clip_high=stub.ppo_clip_eps_high, use_tis=stub.use_tis,
        use_icepop=stub.use_icepop, tis_min=stub.tis_ratio_min, tis_max=stub.tis_ratio_max,
        per_token_loss=stub.calculate_per_token_loss, positive_lm_coef=stub.positive_lm_loss_coef,
        positive_lm_weights=pos_w, rollout_lp=rollout, train_lp_is_old=cfg.get("train_lp_is_old", False),
        entropy=entropy)
    ref_loss.backward()
    assert set(sums) == set(ref_sums)

    def same(a, b, scale):
        # NaN where torch gives NaN, the same infinity where it gives one.
        if math.isnan(b):
            return math.isnan(a)
        if math.isinf(b):
            return a == b
        return abs(a - b) <= TOL * scale

    assert same(loss.item(), ref_loss.item(), 1.0), (loss.item(), ref_loss.item())
    for k in ref_sums:
        # 1e-3 absolute for O(1) values, 1e-3 relative for token sums over many tokens.
        a, b = float(sums[k]), float(ref_sums[k])
        assert same(a, b, max(1.0, abs(b)) if math.isfinite(b) else 1.0), (k, a, b)
    g, rg = nd.grad.cpu(), nr.grad
    finite = torch.isfinite(new) & torch.isfinite(old)  # gradients compared where the inputs are finite
    if nonfinite:
        g, rg = g[finite], rg[finite]
        assert torch.equal(torch.isnan(g), torch.isnan(rg))
        keep = ~torch.isnan(rg)
        g, rg = g[keep], rg[keep]
    assert (g - rg).abs().max().item() <= TOL * max(1e-6, rg.abs().max().item())
    return loss, sums


def _random_packed(n_docs, seed, max_len=300, pad=17):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_len, (n_docs,), generator=g).tolist()
    T = sum(lens) + pad
    doc_ids = torch.cat([torch.full((L,), j) for j, L in enumerate(lens)] + [torch.full((pad,), n_docs)])
    mask = (torch.rand(T, generator=g) > 0.3).float()
    mask[doc_ids == n_docs] = 0
    old = -torch.rand(T, generator=g) * 8
    new = old + torch.randn(T, generator=g) * 0.3
    roll = old + torch.randn(T, generator=g) * 0.2
    ent = torch.rand(T, generator=g) * 5
    adv = torch.randn(n_docs, generator=g)
    posw = torch.rand(n_docs, generator=g)
    return [x.reshape(1, -1) if x.numel() == T else x for x in (new, old, mask, doc_ids)] + [adv, roll.reshape(1, -1),
                                                                                            ent.reshape(1, -1), posw]


@pytest.mark.parametrize("variant", [
    dict(),
    dict(per_token_loss=False),
    dict(use_tis=True),
    dict(use_icepop=True, train_lp_is_old=True),
    dict(use_icepop=True, positive_lm_coef=0.1, per_token_loss=False),
    dict(positive_lm_coef=0.3),
])
def test_matches_oracle_packed(dev, variant):
    new, old, mask, doc_ids, adv, roll, ent, posw = _random_packed(37, seed=len(str(variant)))
    _compare(dev, new, old, mask, doc_ids, adv, 37, rollout=roll, entropy=ent, pos_w=posw, **variant)


def test_random_document_layouts(dev):
    """30 seeded batches whose document sizes run from 1 token to several
    2048-token tiles (tiles with one to many documents, both tile paths),
    empty document slots, padded rows or a packed row, a padding slot, and every
    variant of reduction, TIS, IcePop and positive-LM loss, against the oracle."""
    rng = np.random.default_rng(31)
    variants = [dict(), dict(per_token_loss=False), dict(use_tis=True), dict(use_icepop=True),
                dict(positive_lm_coef=0.2, per_token_loss=False)]
    for trial in range(30):
        sizes = rng.choice([1, 2, 5, 60, 700, 2047, 2049, 5000], size=int(rng.integers(1, 40)))
        ids = np.repeat(np.arange(len(sizes)), sizes) * int(rng.choice([1, 3]))
        n_docs = int(ids.max()) + 1
        pad = int(rng.integers(0, 50))
        ids = np.concatenate([ids, np.full(pad, n_docs)])
        n = len(ids)
        rows = 1
        for r in (2, 3, 4):
            if n % r == 0 and rng.random() < 0.3:
                rows = r
        t = lambda x: torch.from_numpy(x).reshape(rows, -1)  # noqa: E731
        old = -rng.random(n).astype(np.float32) * 8
        new = (old + rng.standard_normal(n).astype(np.float32) * 0.3).astype(np.float32)
        mask = (rng.random(n) > 0.2).astype(np.float32)
        mask[ids == n_docs] = 0
        roll = (old + rng.standard_normal(n).astype(np.float32) * 0.2).astype(np.float32)
        adv = torch.from_numpy(rng.standard_normal(n_docs).astype(np.float32))
        posw = torch.from_numpy(rng.random(n_docs).astype(np.float32))
        _compare(dev, t(new), t(old), t(mask), t(ids.astype(np.int64)), adv, n_docs, rollout=t(roll), pos_w=posw,
                 **variants[trial % len(variants)])


@pytest.mark.parametrize("case", ["nan_new_masked", "inf_ratio_pos_adv", "inf_ratio_neg_adv", "neg_inf_new_masked"])
@pytest.mark.parametrize("per_token_loss", [True, False])
def test_non_finite_inputs_propagate_like_torch(dev, case, per_token_loss):
    """IEEE semantics as torch has them: a NaN at a masked token still gives a
    NaN loss (NaN * 0), an infinite ratio is clipped to a finite term for a
    positive advantage and an infinite one for a negative advantage, and every
    diagnostic follows (inf * 0 = NaN in the masked sums, inf / inf in ESS)."""
    new, old, mask, doc_ids, adv, roll, ent, posw = _random_packed(9, seed=3)
    ids = doc_ids.reshape(-1)
    tok = int((ids == 4).nonzero()[3])
    if case == "nan_new_masked":
        mask[0, tok] = 0.0
        new[0, tok] = float("nan")
    elif case in ("inf_ratio_pos_adv", "inf_ratio_neg_adv"):
        mask[0, tok] = 1.0
        old[0, tok] = float("-inf")
        adv[4] = 0.7 if case == "inf_ratio_pos_adv" else -0.7
    else:
        mask[0, tok] = 0.0
        new[0, tok] = float("-inf")
    _compare(dev, new, old, mask, doc_ids, adv, 9, rollout=roll, entropy=ent, nonfinite=True,
             per_token_loss=per_token_loss)


@pytest.mark.parametrize("T", [1, 2, 1023, 1024, 1025, 2047, 2048, 2049, 4097])
@pytest.mark.parametrize("per_token_loss", [True, False])
def test_token_counts_around_workgroup_boundaries(dev, T, per_token_loss):
    """The backward takes 1024 tokens per workgroup and the forward 2048 per
    tile: counts on either side of both, with the last lanes past the end."""
    g = torch.Generator().manual_seed(T)
    n_docs = max(1, min(5, T // 3))
    cuts = sorted(torch.randperm(max(T - 1, 1), generator=g)[:n_docs - 1].add(1).tolist()) if T > 1 else []
    doc_ids = torch.zeros(T, dtype=torch.long)
    for c in cuts:
        doc_ids[c:] += 1
    mask = (torch.rand(T, generator=g) > 0.25).float()
    old = -torch.rand(T, generator=g) * 4
    new = old + torch.randn(T, generator=g) * 0.3
    adv = torch.randn(n_docs, generator=g)
    _compare(dev, new.reshape(1, -1), old.reshape(1, -1), mask.reshape(1, -1), doc_ids.reshape(1, -1), adv, n_docs,
             per_token_loss=per_token_loss)


@pytest.mark.parametrize("per_token_loss", [True, False])
def test_no_documents_gives_zero_loss_and_gradient(dev, per_token_loss):
    """Every token in the padding slot (n_docs = 0): loss, sums and gradient are 0."""
    T = 1500
    g = torch.Generator().manual_seed(2)
    old = -torch.rand(1, T, generator=g)
    new = old + torch.randn(1, T, generator=g) * 0.3
    loss, sums = _compare(dev, new, old, torch.zeros(1, T), torch.zeros(1, T, dtype=torch.long), torch.zeros(0), 0,
                          per_token_loss=per_token_loss, n_docs_global=0, n_tokens_global=0)
    assert loss.item() == 0.0


def test_per_token_advantages_padded_rows(dev):
    g = torch.Generator().manual_seed(5)
    rows, S = 6, 700
    doc_ids = torch.arange(rows).unsqueeze(1).expand(rows, S).clone()
    mask = (torch.rand(rows, S, generator=g) > 0.2).float()
    old = -torch.rand(rows, S, generator=g) * 3
    new = old + torch.randn(rows, S, generator=g) * 0.5
    adv = torch.randn(rows, S, generator=g)
    _compare(dev, new, old, mask, doc_ids, adv, rows, per_token_loss=False)


@pytest.mark.parametrize("n_docs", [3000, 5000])
def test_many_tiny_documents_and_empty_pad(dev, n_docs):
    """One- and two-token documents: many (tile, document) pairs per tile, and
    thousands of documents for the one-workgroup combine, under both
    reductions."""
    g = torch.Generator().manual_seed(9)
    lens = (torch.randint(1, 3, (n_docs,), generator=g)).tolist()
    doc_ids = torch.cat([torch.full((L,), j) for j, L in enumerate(lens)]).reshape(1, -1)
    T = doc_ids.numel()
    mask = torch.ones(1, T)
    old = -torch.rand(1, T, generator=g)
    new = old + torch.randn(1, T, generator=g) * 0.4
    adv = torch.randn(n_docs, generator=g)
    _compare(dev, new, old, mask, doc_ids, adv, n_docs, per_token_loss=False)
    _compare(dev, new, old, mask, doc_ids, adv, n_docs, per_token_loss=True)


@pytest.mark.parametrize("per_token_loss", [True, False])
def test_empty_document_slots_inside_tiles(dev, per_token_loss):
    """Documents without tokens between the ids a tile holds (ids 0, 2, 3, 7 ...):
    the tile's document range counts them, their sums stay zero and no other
    (tile, document) pair is disturbed; documents cross 2048-token tiles."""
    g = torch.Generator().manual_seed(21)
    n_docs = 40
    present = sorted(torch.randperm(n_docs, generator=g)[:18].tolist())
    lens = torch.randint(50, 1500, (len(present),), generator=g).tolist()
    doc_ids = torch.cat([torch.full((L,), d) for d, L in zip(present, lens)]).reshape(1, -1)
    T = doc_ids.numel()
    mask = (torch.rand(1, T, generator=g) > 0.2).float()
    old = -torch.rand(1, T, generator=g) * 4
    new = old + torch.randn(1, T, generator=g) * 0.3
    adv = torch.randn(n_docs, generator=g)
    _compare(dev, new, old, mask, doc_ids, adv, n_docs, per_token_loss=per_token_loss)


def test_size_mismatch_raises(dev):
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    stub = NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, calculate_per_token_loss=True,
              sharder=_NoCp(), parallel_dims=NS(cp=1))
    z = torch.zeros(1, 8, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), torch.ones(1, 8, device=dev), torch.zeros(1, 7, dtype=torch.long, device=dev),
               torch.ones(1, device=dev), None, torch.zeros(1, device=dev), 1)
    new = torch.zeros(1, 8, device=dev)
    with pytest.raises(ValueError, match="doc_ids"):
        ppo_clip_loss(stub, new, new, mb, MiniPlan((), 1, 8, ()))


def test_ppo_512_docs_full_size(dev):
    """~2M packed tokens, 512 docs, token-mean, eps 0.2/0.28, TIS off."""
    from meshy_amd import workloads

    batch, old, new, rewards, group_offsets = workloads.ppo_512_docs(2)
    from oracle.grpo import grpo_batched

    adv = grpo_batched(torch.from_numpy(rewards), torch.from_numpy(group_offsets))
    n = len(batch.lengths)
    doc_ids = torch.from_numpy(np.repeat(np.arange(n), batch.lengths)).reshape(1, -1)
    mask = torch.from_numpy(batch.mask).reshape(1, -1)
    loss, sums = _compare(dev, torch.from_numpy(new).reshape(1, -1), torch.from_numpy(old).reshape(1, -1),
                          mask, doc_ids, adv, n, clip_low=0.2, clip_high=0.28, per_token_loss=True)
    assert 0.0 <= float(sums["clip_sum"]) / float(sums["token_count"]) <= 1.0


def test_deterministic(dev):
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    new, old, mask, doc_ids, adv, roll, ent, posw = _random_packed(200, seed=3, max_len=5000)
    rows, S = new.shape
    z = torch.zeros(rows, S, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask.to(dev), doc_ids.to(dev), adv.to(dev), roll.to(dev),
               torch.zeros(200, device=dev), 200)
    mini = MiniPlan((), 200, int(mask.sum()), ())
    outs = []
    for _ in range(2):
        nd = new.to(dev).requires_grad_(True)
        loss, sums = ppo_clip_loss(_stub(use_tis=False), nd, old.to(dev), mb, mini)
        loss.backward()
        outs.append((loss.item(), torch.stack(list(sums.values())).cpu(), nd.grad.cpu()))
    assert outs[0][0] == outs[1][0]
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])


@pytest.mark.parametrize("n,n_slots,offset", [(0, 3, 0), (1, 1, 0), (7, 5, 0), (8, 4, 0), (9, 20, 1),
                                               (17, 3, 1), (100_003, 513, 0), (1_000_000, 4097, 1)])
def test_segment_offsets_match_searchsorted(dev, n, n_slots, offset):
    """off[d] = first position whose id is >= d (empty slots and slots past the
    last id included), off[n_slots] = n; lengths off a multiple of 8 and a
    misaligned view exercise the scalar path."""
    from meshy_amd.loss import segment_offsets

    rng = np.random.default_rng(n + n_slots)
    ids = np.sort(rng.integers(0, n_slots, n)).astype(np.int64)
    if n > 10:
        ids[ids == ids[n // 2]] = ids[n // 2] - 1 if ids[n // 2] > 0 else 0  # leave an empty slot
        ids.sort()
    base = torch.zeros(n + offset, dtype=torch.int64)
    base[offset:] = torch.from_numpy(ids)
    got = segment_offsets(base.to(dev)[offset:], n_slots).cpu().numpy()
    want = np.concatenate([np.searchsorted(ids, np.arange(n_slots), side="left"), [n]])
    assert np.array_equal(got, want)


def test_segment_offsets_detect_unsorted(dev):
    from meshy_amd.loss import segment_offsets

    ids = torch.arange(1000, dtype=torch.int64) // 10
    assert segment_offsets(ids.to(dev), 100, check_sorted=True).shape == (101,)
    ids[517] = 3
    with pytest.raises(ValueError):
        segment_offsets(ids.to(dev), 100, check_sorted=True)


@pytest.mark.parametrize("n,n_slots", [(1, 1), (7, 3), (1000, 2), (65536, 1024), (1_000_003, 1000), (300_000, 70_001)])
def test_doc_order_is_the_stable_sort(dev, n, n_slots):
    """meshy_doc_order's permutation is numpy's stable argsort of the ids
    (ties keep their positions) and its ids are the sorted ids, over slot
    counts on both sides of a power of two."""
    from meshy_amd.loss import doc_order

    rng = np.random.default_rng(n + n_slots)
    ids = rng.integers(0, n_slots, n)
    perm, sorted_ids = doc_order(torch.from_numpy(ids).to(dev), n_slots)
    want = np.argsort(ids, kind="stable")
    assert np.array_equal(perm.cpu().numpy(), want)
    assert np.array_equal(sorted_ids.cpu().numpy(), ids[want])


def test_loss_takes_doc_ids_out_of_order(dev):
    """doc_ids that decrease (a batch not built by the pack kernels) are
    accepted, as the reference's index_add_ accepts them: the loss runs on the
    tokens in document order and matches the oracle, call after call, and
    after an in-place edit of the ids."""
    g = torch.Generator().manual_seed(4)
    doc_ids = torch.tensor([[0, 0, 1, 1, 0, 1, 1, 1]])
    mask = torch.ones(1, 8)
    mask[0, -1] = 0
    old = -torch.rand(1, 8, generator=g) * 3
    new = old + 0.1 * torch.randn(1, 8, generator=g)
    adv = torch.tensor([1.0, -1.0])
    for _ in range(2):
        _compare(dev, new, old, mask, doc_ids, adv, 2, use_tis=True)
    doc_ids[0, 4] = 1
    _compare(dev, new, old, mask, doc_ids, adv, 2, use_tis=True)


@pytest.mark.parametrize("per_token_loss", [True, False])
@pytest.mark.parametrize("per_token_adv", [False, True])
@pytest.mark.parametrize("icepop", [False, True])
def test_doc_ids_in_any_order_match_oracle(dev, per_token_loss, per_token_adv, icepop):
    """Random document ids in random order (the padding slot among them) over
    a [3, 700] batch, with rollout log-probs, entropy and positive-LM
    weights: loss, every sum and d loss / d new_lp against the oracle's
    index_add_ over the same order."""
    g = torch.Generator().manual_seed(per_token_loss * 4 + per_token_adv * 2 + icepop)
    rows, S, n = 3, 700, 9
    doc_ids = torch.randint(0, n + 1, (rows, S), generator=g)
    mask = (torch.rand(rows, S, generator=g) > 0.2).float()
    old = -torch.rand(rows, S, generator=g) * 4
    new = old + 0.1 * torch.randn(rows, S, generator=g)
    adv = torch.randn(rows, S, generator=g) if per_token_adv else torch.randn(n, generator=g)
    rollout = old + 0.05 * torch.randn(rows, S, generator=g)
    entropy = torch.rand(rows, S, generator=g)
    pos_w = torch.rand(n, generator=g)
    _compare(dev, new, old, mask, doc_ids, adv, n, rollout=rollout, entropy=entropy, pos_w=pos_w,
             per_token_loss=per_token_loss, use_icepop=icepop, use_tis=not icepop, positive_lm_coef=0.1)


def test_doc_ids_in_any_order_are_deterministic(dev):
    """The document order is a function of the ids alone (a stable sort), so
    repeated calls give bitwise equal losses, sums and gradients."""
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    g = torch.Generator().manual_seed(8)
    rows, S, n = 2, 5000, 40
    doc_ids = torch.randint(0, n, (rows, S), generator=g).to(dev)
    mask = (torch.rand(rows, S, generator=g) > 0.1).float().to(dev)
    old = (-torch.rand(rows, S, generator=g) * 4).to(dev)
    z = torch.zeros(rows, S, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask, doc_ids, torch.randn(n, generator=g).to(dev), None,
               torch.zeros(n, device=dev), n)
    mini = MiniPlan(micros=(), n_docs_global=n, n_tokens_global=int(mask.sum()), tokens_per_rank=())
    outs = []
    for stub in (_stub(calculate_per_token_loss=False), _stub(calculate_per_token_loss=False)):
        new = (old + 0.05).requires_grad_(True)
        loss, sums = ppo_clip_loss(stub, new, old, mb, mini)
        loss.backward()
        outs.append((loss.detach().clone(), {k: v.clone() for k, v in sums.items()}, new.grad.clone()))
    (l0, s0, g0), (l1, s1, g1) = outs
    assert torch.equal(l0, l1) and torch.equal(g0, g1)
    assert all(torch.equal(s0[k], s1[k]) for k in s0)


@pytest.mark.parametrize("bad", [-1, 3, 7])
def test_loss_rejects_doc_ids_out_of_range(dev, bad):
    """Ids outside [0, n_docs] (n_docs = the padding slot) lie in no slot's
    token range, so the tile kernels would never visit them: the order check
    also rejects them, with ValueError, as the reference's index_add_ raises
    (trainer.py:787-791).  Sorted or not, the range error is the one raised."""
    from meshy_amd.loss import DocIdRangeError, ppo_clip_loss, segment_offsets
    from meshy_amd.plan import MiniPlan

    mb = _batch(dev, rows=1, S=8)
    ids = [0, 0, 1, 1, 1, 2, 2, 2]
    ids[0 if bad < 0 else 7] = bad
    mb.doc_ids = torch.tensor([ids], device=dev)
    mb.advantages = torch.tensor([1.0, -1.0], device=dev)
    mb.n_docs = 2
    mini = MiniPlan(micros=(), n_docs_global=2, n_tokens_global=int(mb.mask.sum()), tokens_per_rank=(8,))
    old = -torch.ones(1, 8, device=dev)
    new = (old + 0.05).requires_grad_()
    for _ in range(2):  # the cached verdict raises the same error
        with pytest.raises(DocIdRangeError, match=r"\[0, 2\]"):
            ppo_clip_loss(_stub(), new, old, mb, mini)
    with pytest.raises(DocIdRangeError):
        segment_offsets(torch.tensor([2, 1, bad], device=dev), 3, check_sorted=True)


def test_gae_rejects_doc_ids_out_of_range(dev):
    """compute_vapo_gae indexes lambda by doc id (gae.py:266-276): an id past
    the padding slot raises ValueError instead of falling back to the unsorted
    path; compute_returns, which only compares ids (gae.py:77-93), accepts it."""
    from meshy_amd import gae

    rows, S = 2, 16
    mask = torch.ones(rows, S, device=dev)
    ids = torch.zeros(rows, S, dtype=torch.int64, device=dev)
    ids[1] = 1
    ids[1, -1] = 5
    r = torch.zeros(rows, S, device=dev)
    with pytest.raises(ValueError, match="doc_ids must lie"):
        gae.compute_vapo_gae(r, torch.zeros(rows, S, device=dev), mask, ids, 2)
    assert torch.isfinite(gae.compute_returns(r, mask, ids)).all()


def test_inputs_cache_follows_edits(dev):
    """Later calls on one micro-batch reuse its flattened inputs (PPO epochs);
    an in-place edit of old_lp or the advantages, a new mini-batch denominator
    or a replaced tensor rebuilds them, so every call matches the oracle."""
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    g = torch.Generator().manual_seed(31)
    rows, S, n = 1, 5000, 3
    doc_ids = torch.repeat_interleave(torch.arange(n), torch.tensor([1200, 2600, 1200])).reshape(1, -1)
    mask = (torch.rand(rows, S, generator=g) > 0.1).float()
    old = -torch.rand(rows, S, generator=g) * 2
    new = old + torch.randn(rows, S, generator=g) * 0.3
    adv = torch.tensor([0.7, -1.2, 0.4])
    z = torch.zeros(rows, S, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask.to(dev), doc_ids.to(dev), adv.to(dev), None, torch.zeros(n, device=dev), n)
    stub = _stub(use_tis=False)

    def check(old_c, adv_c, n_tok):
        mini = MiniPlan(micros=(), n_docs_global=n, n_tokens_global=n_tok, tokens_per_rank=())
        nd = new.to(dev).requires_grad_(True)
        loss, sums = ppo_clip_loss(stub, nd, old_dev, mb, mini)
        loss.backward()
        nr = new.clone().requires_grad_(True)
        ref_loss, ref_sums = oppo.ppo_clip_loss(nr, old_c, mask, doc_ids, adv_c, n, n_docs_global=n,
                                                n_tokens_global=n_tok, clip_low=0.2, clip_high=0.28,
                                                per_token_loss=True)
        ref_loss.backward()
        assert abs(loss.item() - ref_loss.item()) <= TOL
        assert abs(sums["ppo_kl_sum"].item() - ref_sums["ppo_kl_sum"].item()) <= 1e-5 * max(1.0, abs(
            ref_sums["ppo_kl_sum"].item()))
        assert (nd.grad.cpu() - nr.grad).abs().max().item() <= 1e-6
        return mb.__dict__["_meshy_ppo_inputs"][1]

    n_tok = int(mask.sum())
    old_dev = old.to(dev)
    first = check(old, adv, n_tok)
    assert check(old, adv, n_tok) is first  # reused
    old_dev.mul_(0.5)  # in place: a new version
    again = check(old * 0.5, adv, n_tok)
    assert again is not first
    mb.advantages.neg_()
    again2 = check(old * 0.5, -adv, n_tok)
    assert again2 is not again
    assert check(old * 0.5, -adv, n_tok + 100) is not again2  # another denominator
    old_dev = (old * 0.25).to(dev)  # a replaced tensor
    check(old * 0.25, -adv, n_tok)


def test_segment_offsets_cache_follows_doc_ids(dev):
    """A batch caches its document offsets after the first loss call; replacing
    or editing doc_ids in place recomputes them."""
    from meshy_amd.loss import batch_segment_offsets, ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    mb = _batch(dev, rows=1, S=8)
    mb.doc_ids = torch.tensor([[0, 0, 0, 0, 0, 1, 1, 1]], device=dev)
    mb.advantages = torch.tensor([1.0], device=dev)
    mb.n_docs = 1
    a = batch_segment_offsets(mb)
    assert a.tolist() == [0, 5, 8]
    assert batch_segment_offsets(mb) is a  # cached
    mb.doc_ids[0, 5:] = 0  # in place: every token now in document 0, padding slot empty
    b = batch_segment_offsets(mb)
    assert b is not a and b.tolist() == [0, 8, 8]
    mini = MiniPlan(micros=(), n_docs_global=1, n_tokens_global=int(mb.mask.sum()), tokens_per_rank=(8,))
    old = -torch.ones(1, 8, device=dev)
    new = (old + 0.05).requires_grad_()
    loss, _ = ppo_clip_loss(_stub(), new, old, mb, mini)
    ref, _ = oppo.ppo_clip_loss(new.detach().cpu().requires_grad_(True), old.cpu(), mb.mask.cpu(),
                                mb.doc_ids.cpu(), mb.advantages.cpu(), 1, n_docs_global=1,
                                n_tokens_global=mini.n_tokens_global, clip_low=0.2, clip_high=0.28,
                                per_token_loss=True, use_tis=True, tis_min=0.5, tis_max=5.0)
    assert abs(float(loss.detach()) - float(ref.detach())) <= TOL

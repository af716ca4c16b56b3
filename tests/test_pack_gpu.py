"""Micro-batch packing and GRPO on the GPU against the oracle and the
reference's known answers (tests/test_dynamic_batching.py:240-316,
tests/test_rollout_advantage.py:13-18).  Indices and copies are bit-exact."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import batch as obatch
from oracle import grpo as ogrpo

pytestmark = pytest.mark.gpu


class _NoCp:
    enabled = False

    def shard_seq(self, *tensors):
        return tensors


def _sample(length, prompt=3, adv=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    mask = torch.ones(length)
    mask[:prompt] = 0
    return {
        "tokens": torch.randint(1, 1000, (length,), generator=g),
        "logprobs": torch.randn(length, generator=g),
        "mask_assistant": mask,
        "advantage": torch.tensor(adv),
    }


def _shift(x):
    return torch.cat([x[1:], x.new_zeros(1)])


def _assert_same(mb, ref, layout):
    for k in ("input_ids", "labels", "positions", "mask", "doc_ids"):
        got = getattr(mb, k).cpu()
        assert got.dtype == ref[k].dtype, k
        assert torch.equal(got, ref[k]), k
    if ref["rollout_logprobs"] is None:
        assert mb.rollout_logprobs is None
    else:
        assert torch.equal(mb.rollout_logprobs.cpu(), ref["rollout_logprobs"])
    assert torch.equal(mb.advantages.cpu(), ref["advantages"])
    assert torch.equal(mb.lengths.cpu(), ref["lengths"])
    assert mb.n_docs == ref["n_docs"]
    assert torch.equal(mb.positive_lm_weights.cpu(), ref["positive_lm_weights"])
    if layout == "packed":
        assert torch.equal(mb.attention_masks.cu_seq_q.cpu(), ref["cu_seqlens"])
        assert mb.attention_masks.max_q == ref["max_seqlen"] == mb.attention_masks.max_k
    else:
        assert mb.attention_masks is None


def test_packed_layout_and_metadata(dev):
    # test_dynamic_batching.py:259-285
    from meshy_amd.batch import build_micro_batch
    from meshy_amd.plan import MicroPlan

    samples = [_sample(10, seed=1), _sample(6, seed=2, adv=2.0)]
    mb = build_micro_batch(samples, MicroPlan((0, 1), 32, (10, 6)), layout="packed", device=dev,
                           sharder=_NoCp(), need_rollout_lp=True)
    assert mb.input_ids.shape == (1, 32)
    row = mb.input_ids[0].cpu()
    assert torch.equal(row[:10], samples[0]["tokens"]) and torch.equal(row[10:16], samples[1]["tokens"])
    assert (row[16:] == 0).all()
    assert torch.equal(mb.labels[0, :10].cpu(), _shift(samples[0]["tokens"]))
    assert mb.mask[0, 9] == 0 and mb.mask[0, 15] == 0
    assert torch.equal(mb.rollout_logprobs[0, 10:16].cpu(), _shift(samples[1]["logprobs"]))
    assert torch.equal(mb.positions[0, 16:].cpu(), torch.arange(16, dtype=torch.int32))
    assert (mb.doc_ids[0, 16:] == 2).all()
    assert torch.equal(mb.attention_masks.cu_seq_q.cpu(), torch.tensor([0, 10, 16, 32], dtype=torch.int32))
    assert mb.attention_masks.max_q == 16
    assert torch.allclose(mb.advantages.cpu(), torch.tensor([1.0, 2.0]))
    ref = obatch.build_micro_batch(samples, (0, 1), 32, (10, 6), layout="packed", need_rollout_lp=True)
    _assert_same(mb, ref, "packed")


def test_packed_without_padding_has_no_pad_doc(dev):
    from meshy_amd.batch import build_micro_batch
    from meshy_amd.plan import MicroPlan

    mb = build_micro_batch([_sample(8, seed=3)], MicroPlan((0,), 8, (8,)), layout="packed", device=dev,
                           sharder=_NoCp(), need_rollout_lp=False)
    assert torch.equal(mb.attention_masks.cu_seq_q.cpu(), torch.tensor([0, 8], dtype=torch.int32))
    assert mb.rollout_logprobs is None


@pytest.mark.parametrize("layout", ["padded", "packed"])
def test_filler_micro_is_all_padding(dev, layout):
    from meshy_amd.batch import build_micro_batch
    from meshy_amd.plan import MicroPlan

    mb = build_micro_batch([], MicroPlan((), 64, ()), layout=layout, device=dev, sharder=_NoCp(),
                           need_rollout_lp=True)
    assert mb.n_docs == 0 and mb.input_ids.shape == (1, 64)
    assert (mb.mask == 0).all() and (mb.doc_ids == 0).all() and mb.advantages.numel() == 0
    ref = obatch.build_micro_batch([], (), 64, (), layout=layout, need_rollout_lp=True)
    _assert_same(mb, ref, layout)


def test_padded_matches_per_sample_shift(dev):
    # test_dynamic_batching.py:240-256
    from meshy_amd.batch import build_micro_batch
    from meshy_amd.plan import MicroPlan

    samples = [_sample(10, seed=1), _sample(6, seed=2, adv=-0.5)]
    mb = build_micro_batch(samples, MicroPlan((0, 1), 16, (10, 6)), layout="padded", device=dev,
                           sharder=_NoCp(), need_rollout_lp=True)
    assert mb.input_ids.shape == (2, 16) and mb.n_slots == 3
    ref = obatch.build_micro_batch(samples, (0, 1), 16, (10, 6), layout="padded", need_rollout_lp=True)
    _assert_same(mb, ref, "padded")
    assert torch.allclose(mb.advantages.cpu(), torch.tensor([1.0, -0.5]))


def test_truncation_in_micro(dev):
    # test_dynamic_batching.py:309-316
    from meshy_amd.batch import build_micro_batch
    from meshy_amd.plan import MicroPlan

    samples = [_sample(20, seed=4)]
    mb = build_micro_batch(samples, MicroPlan((0,), 16, (12,)), layout="padded", device=dev,
                           sharder=_NoCp(), need_rollout_lp=False)
    assert torch.equal(mb.input_ids[0, :12].cpu(), samples[0]["tokens"][:12])
    assert mb.labels[0, 11] == 0 and mb.mask[0, 11] == 0 and int(mb.lengths[0]) == 12


def test_per_token_advantages_and_positive_weights(dev):
    from meshy_amd.batch import ADVANTAGE_TOKENS, build_micro_batches
    from meshy_amd.plan import MicroPlan

    samples = [_sample(9, seed=5), _sample(7, seed=6), _sample(12, seed=7)]
    for j, s in enumerate(samples):
        s[ADVANTAGE_TOKENS] = torch.randn(len(s["tokens"]), generator=torch.Generator().manual_seed(j))
        s["reward"] = torch.tensor([1.0, 0.0, 0.9][j])
        s["positive_lm_weight"] = torch.tensor(0.25 * (j + 1))
    micros = [MicroPlan((2, 0), 32, (12, 9)), MicroPlan((1,), 8, (7,))]
    for layout in ("packed", "padded"):
        mbs = build_micro_batches(samples, micros, layout=layout, device=dev, sharder=_NoCp(),
                                  need_rollout_lp=True)
        for mb, m in zip(mbs, micros):
            ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                           need_rollout_lp=True)
            _assert_same(mb, ref, layout)


@pytest.mark.parametrize("layout,align", [("packed", 2048), ("packed", 1), ("packed", 64), ("padded", 64)])
def test_grpo_256_samples_full_plan_bit_exact(dev, layout, align):
    """256 GRPO samples (budget 8192): every micro of the plan against the oracle."""
    from meshy_amd import workloads
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import PlannerConfig, build_plan

    batch, rewards, _ = workloads.grpo_256_samples(0)
    adv = np.linspace(-1, 1, len(rewards)).astype(np.float32)
    samples = batch.sample_dicts(rewards=rewards, advantages=adv)
    budget = 8192 if layout == "packed" else 16384
    cfg = PlannerConfig(layout=layout, mini_batch_size=256, seq_len=8192, align=align,
                        max_tokens_per_micro=budget)
    lt = batch.loss_tokens(8192)
    plan = build_plan(batch.lengths.tolist(), lt.tolist(), 1, cfg)
    local = plan.local_samples(samples, 0)
    micros = [m for mini in plan.per_rank[0] for m in mini.micros]
    mbs = build_micro_batches(local, micros, layout=layout, device=dev, sharder=_NoCp(),
                              need_rollout_lp=True)
    assert len(mbs) == len(micros)
    for mb, m in zip(mbs, micros):
        ref = obatch.build_micro_batch(local, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                       need_rollout_lp=True)
        _assert_same(mb, ref, layout)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_pack_writes_the_segment_offsets_of_every_micro(dev, layout):
    """The offsets the pack writes next to cu_seqlens equal those computed from
    doc_ids (searchsorted of the flattened ids), fillers and truncated
    documents included, and the losses take them without another pass."""
    from meshy_amd import workloads
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.loss import batch_segment_offsets
    from meshy_amd.plan import MicroPlan, PlannerConfig, build_plan

    batch, rewards, _ = workloads.grpo_256_samples(0)
    samples = batch.sample_dicts(rewards=rewards, advantages=rewards)
    cfg = PlannerConfig(layout=layout, mini_batch_size=64, seq_len=4096, align=64,
                        max_tokens_per_micro=8192 if layout == "packed" else 16384)
    plan = build_plan(np.minimum(batch.lengths, 4096).tolist(), batch.loss_tokens(4096).tolist(), 1, cfg)
    local = plan.local_samples(samples, 0)
    micros = [m for mini in plan.per_rank[0] for m in mini.micros] + [MicroPlan((), 64, ())]
    mbs = build_micro_batches(local, micros, layout=layout, device=dev, sharder=_NoCp(), need_rollout_lp=True)
    for mb in mbs:
        ids = mb.doc_ids.reshape(-1).cpu()
        want = torch.searchsorted(ids, torch.arange(mb.n_docs + 2), right=False)
        got = batch_segment_offsets(mb)
        assert got.dtype == torch.int64 and torch.equal(got.cpu(), want), (mb.n_docs, got, want)
        # a view of the offsets the pack wrote, not a recomputation
        seg = getattr(mb, "_meshy_seg_src")[0].seg
        assert seg.data_ptr() <= got.data_ptr() < seg.data_ptr() + seg.numel() * seg.element_size()


def test_16_long_sequences_micros(dev):
    """Long-context planner edge cases materialised: exact-budget fits and a full 131072 micro."""
    from meshy_amd import workloads
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import PlannerConfig, build_plan

    rng = np.random.default_rng(3)
    for lengths in ([131072], [65536, 65536], [131071, 1], [100000, 31073]):
        prompt = np.full(len(lengths), 16)
        batch = workloads.RaggedBatch(prompt, np.array(lengths) - 16, rng)
        samples = batch.sample_dicts()
        cfg = PlannerConfig(layout="packed", mini_batch_size=len(lengths), seq_len=131072, align=2048,
                            max_tokens_per_micro=131072)
        plan = build_plan(lengths, lengths, 1, cfg)
        micros = [m for mini in plan.per_rank[0] for m in mini.micros]
        mbs = build_micro_batches(samples, micros, layout="packed", device=dev, sharder=_NoCp(),
                                  need_rollout_lp=False)
        for mb, m in zip(mbs, micros):
            assert m.seq_len <= 131072
            ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout="packed",
                                           need_rollout_lp=False)
            _assert_same(mb, ref, "packed")


def test_deterministic_and_repeatable(dev):
    from meshy_amd import workloads
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import PlannerConfig, build_plan

    batch, rewards, _ = workloads.grpo_256_samples(1)
    samples = batch.sample_dicts(rewards=rewards, advantages=rewards)
    cfg = PlannerConfig(layout="packed", mini_batch_size=256, seq_len=8192, align=2048,
                        max_tokens_per_micro=8192)
    plan = build_plan(batch.lengths.tolist(), batch.loss_tokens(8192).tolist(), 1, cfg)
    samples = plan.local_samples(samples, 0)
    micros = [m for mini in plan.per_rank[0] for m in mini.micros]
    a = build_micro_batches(samples, micros, layout="packed", device=dev, need_rollout_lp=True)
    b = build_micro_batches(samples, micros, layout="packed", device=dev, need_rollout_lp=True)
    for x, y in zip(a, b):
        assert torch.equal(x.input_ids, y.input_ids) and torch.equal(x.mask, y.mask)
        assert torch.equal(x.attention_masks.cu_seq_q, y.attention_masks.cu_seq_q)


def test_packed_micro_with_many_documents(dev):
    """1500 short documents in one packed micro: more than the in-LDS offset table holds."""
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import MicroPlan

    g = torch.Generator().manual_seed(11)
    lens = torch.randint(2, 5, (1500,), generator=g).tolist()
    samples = [_sample(L, prompt=1, seed=j) for j, L in enumerate(lens)]
    small = MicroPlan((0, 1), 16, (lens[0], lens[1]))
    big = MicroPlan(tuple(range(1500)), sum(lens) + 100, tuple(lens))
    mbs = build_micro_batches(samples, [small, big], layout="packed", device=dev, sharder=_NoCp(),
                              need_rollout_lp=True)
    for mb, m in zip(mbs, [small, big]):
        ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout="packed",
                                       need_rollout_lp=True)
        _assert_same(mb, ref, "packed")


def test_cpu_device_is_rejected():
    from meshy_amd.batch import build_micro_batch
    from meshy_amd.plan import MicroPlan

    with pytest.raises(ValueError):
        build_micro_batch([_sample(4)], MicroPlan((0,), 4, (4,)), layout="packed",
                          device=torch.device("cpu"), sharder=_NoCp(), need_rollout_lp=False)


# ---------------------------------------------------------------------- GRPO

def test_grpo_known_answer(dev):
    # test_rollout_advantage.py:13-18 (pins the unbiased std)
    from meshy_amd.advantage import grpo_advantages

    adv = grpo_advantages(torch.tensor([1.0, 2.0, 3.0], device=dev), torch.tensor([0, 3], device=dev))
    assert adv.cpu().tolist() == pytest.approx([-1.0, 0.0, 1.0], abs=1e-6)


def test_grpo_special_cases(dev):
    from meshy_amd.advantage import grpo_advantages

    r = torch.tensor([1.0, 1.0, 1.0, 0.0, 0.0, 0.5, 0.7], device=dev)
    off = torch.tensor([0, 3, 5, 6, 7], device=dev)
    adv = grpo_advantages(r, off).cpu()
    assert adv[:5].abs().max() == 0.0  # all-equal groups -> 0
    assert adv[5].item() == 0.5         # size-1 groups keep their reward
    assert adv[6].item() == pytest.approx(0.7)


def test_grpo_offsets_clamped_to_the_rewards(dev):
    """Offsets past the end of the rewards are clamped to them: the groups that
    fit are normalised as usual and nothing outside the arrays is touched."""
    from meshy_amd.advantage import grpo_advantages

    rewards = torch.tensor([1.0, 0.0, 1.0, 1.0, 0.0, 0.0], device=dev)
    off = torch.tensor([0, 3, 9], dtype=torch.int64, device=dev)  # the last group claims 6, holds 3
    adv = grpo_advantages(rewards, off).cpu()
    r = rewards.cpu().tolist()
    ref = torch.tensor(ogrpo.grpo_group(r[:3]) + ogrpo.grpo_group(r[3:]))
    assert torch.allclose(adv, ref, atol=1e-6)


def test_grpo_256_samples_matches_oracle(dev):
    from meshy_amd import workloads
    from meshy_amd.advantage import grpo_advantages

    _, rewards, group_offsets = workloads.grpo_256_samples(0)
    r = torch.from_numpy(rewards)
    off = torch.from_numpy(group_offsets)
    got = grpo_advantages(r.to(dev), off.to(dev)).cpu()
    ref = ogrpo.grpo_batched(r, off)
    assert (got - ref).abs().max().item() <= 1e-5
    # ragged groups with random float rewards
    g = torch.Generator().manual_seed(0)
    r = torch.rand(100, generator=g)
    off = torch.tensor([0, 1, 9, 10, 40, 41, 100])
    got = grpo_advantages(r.to(dev), off.to(dev)).cpu()
    assert (got - ogrpo.grpo_batched(r, off)).abs().max().item() <= 1e-4


def test_zero_variance_known_answers(dev):
    # test_rollout_advantage.py:90-93, each group of the known answers in one call
    from meshy_amd.advantage import zero_variance_groups

    groups = [[0.0, 0.0, 0.0], [1.0, 1.0], [0.0, 1.0], [], [1.0, 1.0 + 2e-8], [1.0, 1.0]]
    flat = torch.tensor([x for g in groups for x in g], dtype=torch.float64, device=dev)
    off = torch.tensor(np.cumsum([0] + [len(g) for g in groups]), device=dev)
    got = zero_variance_groups(flat, off).cpu().tolist()
    # all equal, all equal, mixed, empty, a spread of 2e-8 (float64, not float32), all equal
    assert got == [True, True, False, True, False, True]


def test_zero_variance_groups_match_oracle(dev):
    """Ragged groups (empty, size 1, up to 200 samples) with spreads at the
    tolerance, NaN first or later, +-inf, and offsets past the end (clamped):
    every flag equals the oracle's."""
    from meshy_amd.advantage import zero_variance_groups

    rng = np.random.default_rng(11)
    sizes = [0, 1, 2, 8, 8, 8, 200, 3, 0, 64, 65, 8]
    vals, offs = [], [0]
    for i, n in enumerate(sizes):
        base = float(rng.choice([0.0, 1.0, -2.0, 1e6]))
        g = [base] * n
        kind = i % 6
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
        vals += g
        offs.append(len(vals))
    offs.append(len(vals) + 5)  # a last group that claims five more samples than there are
    for tol in (1e-8, 0.0, 2.0):
        got = zero_variance_groups(torch.tensor(vals, dtype=torch.float64, device=dev),
                                   torch.tensor(offs, device=dev), tol).cpu().tolist()
        clamped = offs[:-1] + [len(vals)]
        want = ogrpo.zero_variance_batched(vals, clamped, tol)
        assert got == want, tol
    assert zero_variance_groups(torch.zeros(0, dtype=torch.float64, device=dev),
                                torch.zeros(3, dtype=torch.int64, device=dev)).cpu().tolist() == [True, True]
    # the host filter gives the device filter's flags; mixed placements are refused
    host = zero_variance_groups(torch.tensor(vals, dtype=torch.float64), torch.tensor(offs)).tolist()
    dev_flags = zero_variance_groups(torch.tensor(vals, dtype=torch.float64, device=dev),
                                     torch.tensor(offs, device=dev)).cpu().tolist()
    assert host == dev_flags
    with pytest.raises(ValueError, match="on the GPU or both on the host"):
        zero_variance_groups(torch.tensor(vals, dtype=torch.float64, device=dev), torch.tensor(offs))


# ------------------------------------------------------------ pack_step (256 GRPO samples)

def test_packed_batch_is_a_batch(dev):
    """The pack's batches are Batch objects whose fields are views made on
    first read: asdict and replace see the same tensors, a field set before
    its first read stays as set, and micros of one launch read independently."""
    import dataclasses

    from meshy_amd import workloads
    from meshy_amd.batch import Batch
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    cfg = PlannerConfig(layout="packed", mini_batch_size=256, seq_len=8192, align=2048, max_tokens_per_micro=8192)
    res = pack_step(ragged, cfg, dev)
    a, b = res.batches[0], res.batches[1]
    assert isinstance(a, Batch)
    d = dataclasses.asdict(b)
    assert set(d) == {f.name for f in dataclasses.fields(Batch)}
    assert torch.equal(d["input_ids"], b.input_ids) and torch.equal(d["doc_ids"], b.doc_ids)  # asdict copies
    r = dataclasses.replace(b, n_docs=b.n_docs)
    assert r.labels.data_ptr() == b.labels.data_ptr() and r.n_docs == b.n_docs
    c = res.batches[2]  # no field of micro 2 read yet
    c.mask = torch.ones(1, 5, device=dev)
    assert c.input_ids.shape[1] == c.labels.shape[1] != 5  # reads the rest of the group
    assert c.mask.shape == (1, 5)  # the field set before the first read stays as set
    c.advantages = torch.zeros(3, device=dev)
    assert c.lengths.numel() == c.n_docs and c.advantages.numel() == 3
    assert a.input_ids.shape == (1, a.labels.shape[1])


def test_pack_step_256_samples_matches_oracle(dev):
    """Plan + one H2D + GRPO + pack: micro map, cu_seqlens, positions bit-exact;
    advantages (per document and broadcast per token) within 1e-5."""
    from meshy_amd import workloads
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig
    from oracle import plan as oplan

    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    cfg = PlannerConfig(layout="packed", mini_batch_size=256, seq_len=8192, align=2048,
                        max_tokens_per_micro=8192)
    res = pack_step(ragged, cfg, dev)
    samples = batch.sample_dicts(rewards=rewards)
    lengths, loss = oplan.sample_lengths(samples, 8192)
    local, per_rank = oplan.build_plan(lengths, loss, 1, layout="packed", mini_batch_size=256, seq_len=8192,
                                       align=2048, max_tokens_per_micro=8192)
    ref_adv = ogrpo.grpo_batched(torch.from_numpy(rewards), torch.from_numpy(group_offsets))
    assert (res.advantages.cpu() - ref_adv).abs().max().item() <= 1e-5
    assert tuple(res.plan.local_indices[0]) == tuple(local[0])
    for s, a in zip(samples, ref_adv):
        s["advantage"] = a
    local_samples = [samples[i] for i in local[0]]
    micros = [m for mini in per_rank[0] for m in mini[0]]
    assert len(res.batches) == len(micros)
    for mb, (idx, seq_len, doc_lens) in zip(res.batches, micros):
        ref = obatch.build_micro_batch(local_samples, idx, seq_len, doc_lens, layout="packed",
                                       need_rollout_lp=True)
        for k in ("input_ids", "labels", "positions", "mask", "doc_ids"):
            assert torch.equal(getattr(mb, k).cpu(), ref[k]), k
        assert torch.equal(mb.rollout_logprobs.cpu(), ref["rollout_logprobs"])
        assert torch.equal(mb.attention_masks.cu_seq_q.cpu(), ref["cu_seqlens"])
        assert (mb.advantages.cpu() - ref["advantages"]).abs().max().item() <= 1e-5
        bcast = torch.cat([ref["advantages"], torch.zeros(1)])[ref["doc_ids"]]
        assert (mb.advantage_tokens.cpu() - bcast).abs().max().item() <= 1e-5


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_pack_step_without_plan_objects_builds_the_same_batches(dev, layout):
    """The Plan dataclasses are built when PackResult.plan is first read
    (with_plan_objects=True builds them inside the call): the batches are the
    same either way and so is the plan; two calls in a row over one staging
    buffer (the tables region is rewritten)."""
    from meshy_amd import workloads
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    cfg = PlannerConfig(layout=layout, mini_batch_size=64, seq_len=8192, align=2048, max_tokens_per_micro=8192)
    full = pack_step(ragged, cfg, dev, with_plan_objects=True)
    lite = pack_step(ragged, cfg, dev)
    assert lite._plan is None and full._plan is not None
    assert lite.plan == full.plan  # built from the tables on first read
    assert len(full.batches) == len(lite.batches) > 4
    for a, b in zip(full.batches, lite.batches):
        for k in ("input_ids", "labels", "positions", "mask", "doc_ids", "rollout_logprobs", "advantages",
                  "advantage_tokens", "lengths"):
            x, y = getattr(a, k), getattr(b, k)
            assert x.shape == y.shape and torch.equal(x, y), k
        assert a.n_docs == b.n_docs
    assert torch.equal(full.advantages, lite.advantages)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_empty_and_one_token_samples(dev, layout):
    """Samples of 0, 1 and 2 tokens among longer ones, planned and packed:
    every micro equals the oracle's (empty documents keep their cu_seqlens
    slot, one-token documents have no label)."""
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import PlannerConfig, build_plan

    lengths = [0, 1, 2, 0, 5, 300, 0, 1, 64, 3, 0, 2]
    samples = [_sample(L, prompt=min(L, 1), adv=0.25 * j, seed=30 + j) for j, L in enumerate(lengths)]
    cfg = PlannerConfig(layout=layout, mini_batch_size=len(lengths), seq_len=512, align=8,
                        max_tokens_per_micro=512)
    loss = [max(0, L - 1) for L in lengths]
    plan = build_plan(lengths, loss, 1, cfg)
    micros = [m for mini in plan.per_rank[0] for m in mini.micros]
    local = plan.local_samples(samples, 0)
    mbs = build_micro_batches(local, micros, layout=layout, device=dev, sharder=_NoCp(), need_rollout_lp=True)
    for mb, m in zip(mbs, micros):
        ref = obatch.build_micro_batch(local, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                       need_rollout_lp=True)
        _assert_same(mb, ref, layout)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_micros_of_only_empty_samples(dev, layout):
    """A batch whose samples are all empty: micros of no output elements that
    still carry their documents' advantages, lengths and cu_seqlens."""
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.plan import PlannerConfig, build_plan

    samples = [_sample(0, prompt=0, adv=1.0 + j, seed=50 + j) for j in range(3)]
    cfg = PlannerConfig(layout=layout, mini_batch_size=3, seq_len=64, align=8, max_tokens_per_micro=64)
    plan = build_plan([0, 0, 0], [0, 0, 0], 1, cfg)
    micros = [m for mini in plan.per_rank[0] for m in mini.micros]
    local = plan.local_samples(samples, 0)
    mbs = build_micro_batches(local, micros, layout=layout, device=dev, sharder=_NoCp(), need_rollout_lp=True)
    for mb, m in zip(mbs, micros):
        ref = obatch.build_micro_batch(local, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                       need_rollout_lp=True)
        _assert_same(mb, ref, layout)


@pytest.mark.parametrize("narrow", [False, True])
@pytest.mark.parametrize("layout", ["packed", "padded"])
@pytest.mark.parametrize("tok_dtype", [torch.int64, torch.int32])
def test_one_pass_staging_equals_the_general_staging(dev, layout, tok_dtype, narrow, monkeypatch):
    """The native one-pass staging stages the same bytes, and the pack makes the
    same batches, as the general staging on the same samples and micros; int64
    tokens of a staging at or above the narrowing's token count it stages as
    int32 (the general staging keeps them int64), the same values."""
    from meshy_amd import batch as B
    from meshy_amd.plan import MicroPlan

    monkeypatch.setattr(B, "_NARROW_MIN_TOKENS", 0 if narrow else 1 << 62)

    lengths = [11, 40, 3, 64, 25, 1, 70, 18]
    samples = []
    for i, L in enumerate(lengths):
        s = _sample(L, prompt=2, adv=0.5 * i - 1.0, seed=10 + i)
        s["tokens"] = s["tokens"].to(tok_dtype)
        s["reward"] = 0.3 * (i % 4)
        s["positive_lm_weight"] = 0.1 * (i + 1)
        samples.append(s)
    micros = [MicroPlan((0, 1, 2), 64, (11, 40, 3)), MicroPlan((3,), 64, (64,)), MicroPlan((), 64, ()),
              MicroPlan((4, 5, 6), 96, (25, 1, 70)), MicroPlan((7, 1), 64, (18, 40))]
    assert B._stage_common(samples, tuple(micros), layout, dev, True) is not None
    fast = B.stage_micro_batches(samples, micros, layout=layout, device=dev, need_rollout_lp=True)
    fast_mbs = B.launch_pack(fast, _NoCp())
    torch.cuda.synchronize()
    monkeypatch.setattr(B, "_stage_common", lambda *a: None)
    slow = B.stage_micro_batches(samples, micros, layout=layout, device=dev, need_rollout_lp=True)
    slow_mbs = B.launch_pack(slow, _NoCp())
    torch.cuda.synchronize()

    assert fast.lay.regions.keys() == slow.lay.regions.keys()
    assert fast.lay.regions["tokens"][2] == (torch.int32 if narrow else tok_dtype)
    assert slow.lay.regions["tokens"][2] == tok_dtype
    fbuf, sbuf = fast.dbuf.cpu(), slow.dbuf.cpu()
    for name, (lo, hi, dtype) in slow.lay.regions.items():
        flo, fhi, fdtype = fast.lay.regions[name]
        if name == "tokens":
            assert torch.equal(fbuf[flo:fhi].view(fdtype).long(), sbuf[lo:hi].view(dtype).long())
            continue
        assert fdtype == dtype and fhi - flo == hi - lo, name
        assert torch.equal(fbuf[flo:fhi], sbuf[lo:hi]), name
    for k in ("seq", "rows", "out_off", "doc_start"):
        a, b = getattr(fast, k), getattr(slow, k)
        assert a.dtype == b.dtype and np.array_equal(a, b), k
    assert (fast.n_samples, fast.max_elems, fast.max_docs) == (slow.n_samples, slow.max_elems, slow.max_docs)
    for mf, ms, m in zip(fast_mbs, slow_mbs, micros):
        ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                       need_rollout_lp=True)
        _assert_same(mf, ref, layout)
        _assert_same(ms, ref, layout)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_pack_step_byte_mask_equals_fp32_mask(dev, layout):
    """0/1 masks staged as bytes and the same masks staged as fp32 give the
    same batches, bit for bit; a fractional mask keeps fp32 staging and its
    values reach the batches' masks unchanged."""
    from meshy_amd import workloads
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    batch, rewards, group_offsets = workloads.grpo_256_samples(1)
    args = (batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards, group_offsets)
    as_bytes = RaggedSamples.from_arrays(*args)
    frac = batch.mask.copy()
    frac[int(batch.offsets[3]) + 1] = 0.5  # the fractional value makes from_arrays stage fp32
    as_fp32 = RaggedSamples.from_arrays(batch.tokens, frac, *args[2:])
    assert as_bytes.mask_u8 and not as_fp32.mask_u8
    budget = 8192 if layout == "packed" else 16384
    cfg = PlannerConfig(layout=layout, mini_batch_size=256, seq_len=8192, align=64 if layout == "packed" else 1,
                        max_tokens_per_micro=budget)
    frac_res = pack_step(as_fp32, cfg, dev)
    got = sum(int((mb.mask == 0.5).sum()) for mb in frac_res.batches)
    assert got == 1
    as_fp32.view("mask").copy_(torch.from_numpy(batch.mask))
    a = pack_step(as_bytes, cfg, dev)
    b = pack_step(as_fp32, cfg, dev)
    assert len(a.batches) == len(b.batches)
    for x, y in zip(a.batches, b.batches):
        for k in ("input_ids", "labels", "positions", "mask", "doc_ids", "rollout_logprobs", "advantages",
                  "lengths"):
            assert torch.equal(getattr(x, k), getattr(y, k)), k


def _random_micros(lengths, rng, layout):
    """Micros over the samples in a random order: packed ones hold up to
    seq_len tokens, padded ones up to 4 documents; documents longer than
    seq_len are cut; a filler micro last."""
    from meshy_amd.plan import MicroPlan

    seq = int(rng.choice([16, 64, 128, 512]))
    micros, cur, lens, used = [], [], [], 0
    for i in rng.permutation(len(lengths)).tolist():
        take = min(int(lengths[i]), seq)
        full = (used + take > seq) if layout == "packed" else len(cur) == 4
        if full and cur:
            micros.append(MicroPlan(tuple(cur), seq, tuple(lens)))
            cur, lens, used = [], [], 0
        cur.append(i)
        lens.append(take)
        used += take
    if cur:
        micros.append(MicroPlan(tuple(cur), seq, tuple(lens)))
    micros.append(MicroPlan((), seq, ()))
    return micros


@pytest.mark.parametrize("seed", range(12))
def test_random_batches_match_oracle(dev, seed, monkeypatch):
    """Random sample sets (empty and one-token samples among them) in random
    micros, both layouts, through the one-pass staging (int64 tokens narrowed
    to int32 or not, int32 tokens) or, with per-token advantages, the general
    staging: every micro equals the oracle's."""
    from meshy_amd import batch as B

    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    lengths = rng.integers(0, 300, n)
    lengths[rng.random(n) < 0.15] = 1
    lengths[rng.random(n) < 0.1] = 0
    samples = []
    for i, L in enumerate(lengths.tolist()):
        s = _sample(L, prompt=min(L, int(rng.integers(0, 5))), adv=float(rng.normal()), seed=100 * seed + i)
        s["reward"] = float(rng.random())
        s["positive_lm_weight"] = float(rng.random())
        if seed % 4 == 1:
            s["tokens"] = s["tokens"].to(torch.int32)
        if seed % 3 == 2:
            s[B.ADVANTAGE_TOKENS] = torch.randn(L)
        samples.append(s)
    monkeypatch.setattr(B, "_NARROW_MIN_TOKENS", 0 if seed % 2 else 1 << 62)
    for layout in ("packed", "padded"):
        micros = _random_micros(lengths, rng, layout)
        mbs = B.build_micro_batches(samples, micros, layout=layout, device=dev, sharder=_NoCp(),
                                    need_rollout_lp=bool(seed % 5))
        for mb, m in zip(mbs, micros):
            ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                           need_rollout_lp=bool(seed % 5))
            _assert_same(mb, ref, layout)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_per_token_advantages_are_decided_per_micro(dev, layout):
    """A micro takes per-token advantages when its first sample carries them
    (batch.py:110): here samples 0-3 do and 4-7 do not, and a micro led by
    sample 6 keeps per-document advantages although sample 2 in it has
    per-token ones; the filler micro's advantages are an empty per-document
    tensor."""
    from meshy_amd import batch as B
    from meshy_amd.plan import MicroPlan

    samples = []
    for i, L in enumerate([12, 30, 7, 20, 9, 25, 14, 3]):
        s = _sample(L, prompt=2, adv=0.25 * i - 1.0, seed=40 + i)
        if i < 4:
            s[B.ADVANTAGE_TOKENS] = torch.linspace(-1.0, 1.0, L) * (i + 1)
        samples.append(s)
    micros = [MicroPlan((0, 1), 64, (12, 30)), MicroPlan((4, 5), 64, (9, 25)), MicroPlan((6, 2, 3), 64, (14, 7, 20)),
              MicroPlan((7,), 64, (3,)), MicroPlan((), 64, ())]
    mbs = B.build_micro_batches(samples, micros, layout=layout, device=dev, sharder=_NoCp(), need_rollout_lp=True)
    for mb, m in zip(mbs, micros):
        ref = obatch.build_micro_batch(samples, m.sample_idx, m.seq_len, m.doc_lens, layout=layout,
                                       need_rollout_lp=True)
        _assert_same(mb, ref, layout)
    assert mbs[0].advantages.dim() == 2 and mbs[2].advantages.dim() == 1
    assert mbs[-1].advantages.shape == (0,)


@pytest.mark.parametrize("seed", range(10))
def test_random_pack_steps_match_oracle(dev, seed):
    """pack_step over random batches (groups of 4, lengths from 0 up, 0/1 or
    fractional masks, random planner settings in both layouts) against the
    oracle's plan, GRPO advantages and micro-batches."""
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig
    from oracle import plan as oplan

    rng = np.random.default_rng(1000 + seed)
    G = 4
    n = G * int(rng.integers(1, 12))
    lengths = rng.integers(0, 400, n)
    lengths[rng.random(n) < 0.1] = 1
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    total = int(offsets[-1])
    tokens = rng.integers(0, 150000, total)
    mask = (rng.random(total) < 0.7).astype(np.float32)
    if seed % 4 == 3:
        mask[rng.random(total) < 0.05] = 0.5  # not 0/1: staged as fp32
    logprobs = rng.normal(size=total).astype(np.float32)
    rewards = rng.integers(0, 2, n).astype(np.float32) if seed % 2 else rng.random(n).astype(np.float32)
    group_offsets = np.arange(0, n + 1, G, dtype=np.int64)
    layout = "packed" if seed % 2 == 0 else "padded"
    seq_len = int(rng.choice([256, 512, 1024]))
    align = int(rng.choice([1, 64, 256]))
    mini = int(rng.choice([d for d in range(1, n + 1) if n % d == 0]))
    kw = dict(layout=layout, mini_batch_size=mini, seq_len=seq_len, align=align,
              max_tokens_per_micro=seq_len if layout == "packed" or seed % 3 else None,
              micro_batch_size=None if layout == "packed" and seed % 3 else int(rng.integers(1, 5)))
    cfg = PlannerConfig(**kw)
    ragged = RaggedSamples.from_arrays(tokens, mask, logprobs, offsets, rewards, group_offsets)
    res = pack_step(ragged, cfg, dev)

    samples = [{"tokens": torch.from_numpy(tokens[a:b]), "mask_assistant": torch.from_numpy(mask[a:b]),
                "logprobs": torch.from_numpy(logprobs[a:b]), "reward": float(rewards[i])}
               for i, (a, b) in enumerate(zip(offsets[:-1], offsets[1:]))]
    lens, loss = oplan.sample_lengths(samples, seq_len)
    local, per_rank = oplan.build_plan(lens, loss, 1, **kw)
    ref_adv = ogrpo.grpo_batched(torch.from_numpy(rewards), torch.from_numpy(group_offsets))
    assert (res.advantages.cpu() - ref_adv).abs().max().item() <= 1e-5
    assert tuple(res.plan.local_indices[0]) == tuple(local[0])
    for s, a in zip(samples, ref_adv):
        s["advantage"] = a
    local_samples = [samples[i] for i in local[0]]
    micros = [m for mini_plan in per_rank[0] for m in mini_plan[0]]
    assert len(res.batches) == len(micros)
    for mb, (idx, s_len, doc_lens) in zip(res.batches, micros):
        ref = obatch.build_micro_batch(local_samples, idx, s_len, doc_lens, layout=layout, need_rollout_lp=True)
        for k in ("input_ids", "labels", "positions", "mask", "doc_ids"):
            assert torch.equal(getattr(mb, k).cpu(), ref[k]), k
        assert torch.equal(mb.rollout_logprobs.cpu(), ref["rollout_logprobs"])
        assert torch.equal(mb.lengths.cpu(), ref["lengths"])
        if layout == "packed":
            assert torch.equal(mb.attention_masks.cu_seq_q.cpu(), ref["cu_seqlens"])
        assert (mb.advantages.cpu() - ref["advantages"]).abs().max().item() <= 1e-5

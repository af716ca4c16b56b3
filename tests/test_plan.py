"""Planner parity (CPU): the native planner (libmeshy_amd, host C++) and the
oracle against golden plans recorded from the reference planner, the
reference's own known answers (tests/test_dynamic_batching.py,
tests/test_critic_batching.py) and brute-force invariants.
"""

from __future__ import annotations

import json
import os
import random

import pytest
from hypothesis import given, settings, strategies as st

from meshy_amd.plan import (
    MicroPlan,
    MiniPlan,
    Plan,
    PlannerConfig,
    build_plan,
    plan_stats,
    resolve_align,
    round_up,
)
from oracle import plan as oplan

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "plan_vectors.json")


def _golden():
    with open(GOLDEN) as f:
        return json.load(f)


def _plan_as_json(plan: Plan):
    return {
        "local_indices": [list(x) for x in plan.local_indices],
        "per_rank": [
            [
                {
                    "micros": [[list(m.sample_idx), m.seq_len, list(m.doc_lens)] for m in mini.micros],
                    "n_docs_global": mini.n_docs_global,
                    "n_tokens_global": mini.n_tokens_global,
                    "tokens_per_rank": list(mini.tokens_per_rank),
                }
                for mini in minis
            ]
            for minis in plan.per_rank
        ],
    }


def _oracle_as_json(res):
    local, per_rank = res
    return {
        "local_indices": [list(x) for x in local],
        "per_rank": [
            [
                {
                    "micros": [[list(s), L, list(d)] for s, L, d in micros],
                    "n_docs_global": nd,
                    "n_tokens_global": nt,
                    "tokens_per_rank": list(tpr),
                }
                for micros, nd, nt, tpr in minis
            ]
            for minis in per_rank
        ],
    }


@pytest.mark.parametrize("case", _golden(), ids=lambda c: c["name"])
def test_oracle_matches_reference_golden(case):
    res = oplan.build_plan(case["lengths"], case["loss_tokens"], case["dp_size"], **case["cfg"])
    assert _oracle_as_json(res) == case["plan"]


@pytest.mark.parametrize("case", _golden(), ids=lambda c: c["name"])
def test_native_matches_reference_golden(case):
    plan = build_plan(case["lengths"], case["loss_tokens"], case["dp_size"], PlannerConfig(**case["cfg"]))
    assert _plan_as_json(plan) == case["plan"]


def _cfg(**kw) -> PlannerConfig:
    base = dict(layout="padded", mini_batch_size=4, seq_len=4096, align=64,
                max_tokens_per_micro=None, micro_batch_size=1)
    base.update(kw)
    return PlannerConfig(**base)


def _check_invariants(plan, lengths, cfg, dp_size):
    # test_dynamic_batching.py:61-94
    n = len(lengths)
    assert plan.dp_size == dp_size
    assert sorted(i for idx in plan.local_indices for i in idx) == list(range(n))
    n_mini = len(plan.per_rank[0])
    for minis in plan.per_rank:
        assert len(minis) == n_mini
    for i in range(n_mini):
        assert len({len(plan.per_rank[r][i].micros) for r in range(dp_size)}) == 1
        assert len({(m.n_docs_global, m.n_tokens_global) for m in
                    (plan.per_rank[r][i] for r in range(dp_size))}) == 1
    for r, minis in enumerate(plan.per_rank):
        local = plan.local_indices[r]
        covered = []
        for mini in minis:
            assert len(mini.micros) > 0
            for m in mini.micros:
                assert m.seq_len % cfg.align == 0 and m.seq_len <= cfg.seq_len
                for p, L in zip(m.sample_idx, m.doc_lens):
                    assert L == min(lengths[local[p]], cfg.seq_len)
                    covered.append(p)
                if cfg.layout == "padded":
                    assert all(L <= m.seq_len for L in m.doc_lens)
                else:
                    assert m.n_tokens <= m.seq_len
                if cfg.max_tokens_per_micro is not None and len(m.sample_idx) > 1:
                    cost = m.n_rows * m.seq_len if cfg.layout == "padded" else m.seq_len
                    assert cost <= cfg.max_tokens_per_micro
                if cfg.max_tokens_per_micro is None and not m.is_filler:
                    assert len(m.sample_idx) <= cfg.micro_batch_size
        assert sorted(covered) == list(range(len(local)))


@pytest.mark.parametrize("layout", ["padded", "packed"])
@pytest.mark.parametrize("dp_size", [1, 2, 4])
def test_plan_invariants(layout, dp_size):
    # test_dynamic_batching.py:97-110
    rng = random.Random(7)
    lengths = [rng.randint(5, 5000) for _ in range(32)]
    loss_tokens = [max(0, L - 4) for L in lengths]
    cfg = _cfg(layout=layout, max_tokens_per_micro=3000, mini_batch_size=4)
    plan = build_plan(lengths, loss_tokens, dp_size, cfg)
    _check_invariants(plan, lengths, cfg, dp_size)
    assert sum(m.n_docs_global for m in plan.per_rank[0]) == 32
    assert sum(m.n_tokens_global for m in plan.per_rank[0]) == sum(loss_tokens)


def test_plan_is_deterministic():
    lengths = [random.Random(1).randint(1, 3000) for _ in range(16)]
    cfg = _cfg(layout="packed", max_tokens_per_micro=4096)
    assert build_plan(lengths, lengths, 2, cfg) == build_plan(lengths, lengths, 2, cfg)


def test_dp_partition_balances_tokens():
    # test_dynamic_batching.py:121-130
    lengths = [100 * (k + 1) for k in range(8) for _ in range(4)]
    plan = build_plan(lengths, lengths, 4, _cfg(mini_batch_size=8, micro_batch_size=8))
    per_rank = [sum(lengths[i] for i in idx) for idx in plan.local_indices]
    contiguous = [sum(lengths[r * 8:(r + 1) * 8]) for r in range(4)]
    assert max(per_rank) - min(per_rank) < max(contiguous) - min(contiguous)
    assert all(len(idx) == 8 for idx in plan.local_indices)


def test_padded_micro_uses_longest_sample_rounded_up():
    lengths = [1000, 130, 70]
    plan = build_plan(lengths, lengths, 1, _cfg(mini_batch_size=3, micro_batch_size=3, align=64))
    (mini,) = plan.per_rank[0]
    (micro,) = mini.micros
    assert micro.seq_len == round_up(1000, 64)
    assert sorted(micro.doc_lens) == sorted(lengths)


def test_token_budget_padded_groups_by_rows_times_row_len():
    lengths = [900, 800, 100, 90, 80]
    plan = build_plan(lengths, lengths, 1, _cfg(mini_batch_size=5, max_tokens_per_micro=2000, align=64))
    (mini,) = plan.per_rank[0]
    assert all(m.n_rows * m.seq_len <= 2000 for m in mini.micros)
    assert sorted(len(m.sample_idx) for m in mini.micros) == [2, 3]


@pytest.mark.parametrize("impl", ["native", "oracle"])
def test_token_budget_packed_first_fit_decreasing(impl):
    # test_dynamic_batching.py:155-167: [[1500,200],[1000,700],[600]]
    lengths = [1500, 1000, 700, 600, 200]
    kw = dict(layout="packed", mini_batch_size=5, seq_len=4096, align=64, max_tokens_per_micro=2048,
              micro_batch_size=1)
    if impl == "native":
        (mini,) = build_plan(lengths, lengths, 1, PlannerConfig(**kw)).per_rank[0]
        micros = [(m.sample_idx, m.seq_len, m.doc_lens) for m in mini.micros]
    else:
        _, per_rank = oplan.build_plan(lengths, lengths, 1, **kw)
        micros = per_rank[0][0][0]
    for _, seq_len, doc_lens in micros:
        assert seq_len <= 2048 and seq_len % 64 == 0 and sum(doc_lens) <= seq_len
    groups = sorted(sorted(d, reverse=True) for _, _, d in micros)
    assert groups == sorted([[1500, 200], [1000, 700], [600]])


@pytest.mark.parametrize("impl", ["native", "oracle"])
def test_single_sample_over_budget_gets_own_micro(impl):
    # test_dynamic_batching.py:170-177
    kw = dict(layout="packed", mini_batch_size=2, seq_len=4096, align=64, max_tokens_per_micro=1024,
              micro_batch_size=1)
    if impl == "native":
        (mini,) = build_plan([4000, 10], [4000, 10], 1, PlannerConfig(**kw)).per_rank[0]
        micros = [(m.sample_idx, m.seq_len, m.doc_lens) for m in mini.micros]
    else:
        micros = oplan.build_plan([4000, 10], [4000, 10], 1, **kw)[1][0][0][0]
    assert len(micros) == 2
    big = next(m for m in micros if 4000 in m[2])
    assert tuple(big[0]) == (0,) and big[1] == 4032


def test_filler_micros_equalise_counts_across_ranks():
    # test_dynamic_batching.py:180-189
    lengths = [3000, 100, 100, 100]
    cfg = _cfg(layout="packed", mini_batch_size=2, max_tokens_per_micro=1024, align=64)
    plan = build_plan(lengths, lengths, 2, cfg)
    counts = [len(plan.per_rank[r][0].micros) for r in range(2)]
    assert counts[0] == counts[1]
    fillers = [m for r in range(2) for m in plan.per_rank[r][0].micros if m.is_filler]
    assert fillers and all(m.seq_len == 64 and m.doc_lens == () for m in fillers)


def test_truncation_to_seq_len():
    plan = build_plan([10_000, 50], [10_000, 50], 1, _cfg(mini_batch_size=2, micro_batch_size=2))
    (mini,) = plan.per_rank[0]
    assert max(L for m in mini.micros for L in m.doc_lens) == 4096


def test_errors():
    with pytest.raises(ValueError, match="not divisible"):
        build_plan([1, 2, 3], [1, 2, 3], 2, _cfg())
    with pytest.raises(ValueError, match="empty"):
        build_plan([], [], 1, _cfg())
    with pytest.raises(ValueError):
        _cfg(layout="packed", max_tokens_per_micro=None)
    with pytest.raises(ValueError):
        _cfg(seq_len=100, align=64)
    with pytest.raises(ValueError):
        _cfg(max_tokens_per_micro=None, micro_batch_size=None)


def test_resolve_align():
    # test_dynamic_batching.py:205-210
    assert resolve_align(2048, 8, 131072) == 2048
    assert resolve_align(2048, 8, 512) == 512
    assert resolve_align(100, 8, 4000) == 200
    with pytest.raises(ValueError):
        resolve_align(3000, 8, 4096)


def test_plan_stats_padding_ratio():
    plan = build_plan([100, 100], [100, 100], 1, _cfg(mini_batch_size=2, micro_batch_size=2, align=128))
    stats = plan_stats(plan.per_rank[0], "padded")
    assert stats["n_micro"] == 1 and stats["tokens_per_micro"] == 200
    assert stats["padding_ratio"] == pytest.approx(1 - 200 / 256)


def _lognormal_lengths(n, seed=0):
    rng = random.Random(seed)
    return [min(4096, max(16, int(rng.lognormvariate(5.6, 1.1)))) for _ in range(n)]


@pytest.mark.parametrize("dp_size", [1, 2, 4])
def test_critic_window_shape(dp_size):
    # test_critic_batching.py:53-142 at the live run's length shape
    lengths = _lognormal_lengths(480)
    cfg = PlannerConfig(layout="padded", mini_batch_size=480 // dp_size, seq_len=4096, align=8,
                        max_tokens_per_micro=2048, micro_batch_size=None)
    plan = build_plan(lengths, lengths, dp_size, cfg)
    assert sorted(g for r in range(dp_size) for g in plan.local_indices[r]) == list(range(480))
    if dp_size == 2:
        per_rank = [sum(lengths[g] for g in plan.local_indices[r]) for r in range(2)]
        assert max(per_rank) / min(per_rank) < 1.02
    counts = {r: [len(m.micros) for m in plan.per_rank[r]] for r in range(dp_size)}
    assert len({tuple(c) for c in counts.values()}) == 1
    real = forward = 0
    for mini in plan.per_rank[0]:
        for micro in mini.micros:
            if micro.is_filler:
                continue
            assert len(micro.sample_idx) * micro.seq_len <= 2048 or len(micro.sample_idx) == 1
            real += micro.n_tokens
            forward += len(micro.sample_idx) * micro.seq_len
    assert 1.0 - real / forward < 0.15


@settings(max_examples=150, deadline=None)
@given(
    lengths=st.lists(st.integers(0, 3000), min_size=1, max_size=40),
    dp=st.sampled_from([1, 2, 4]),
    layout=st.sampled_from(["padded", "packed"]),
    align=st.sampled_from([1, 8, 64]),
    budget=st.sampled_from([None, 64, 700, 2048, 5000]),
    mbs=st.integers(1, 9),
    micro_bs=st.sampled_from([None, 1, 3]),
)
def test_native_equals_oracle_random(lengths, dp, layout, align, budget, mbs, micro_bs):
    lengths = lengths[: max(dp, len(lengths) // dp * dp)]
    if len(lengths) % dp:
        lengths = lengths + [1] * (dp - len(lengths) % dp)
    if layout == "packed" and budget is None:
        budget = 2048
    if budget is None and micro_bs is None:
        micro_bs = 2
    seq_len = align * (4096 // align)
    kw = dict(layout=layout, mini_batch_size=mbs, seq_len=seq_len, align=align,
              max_tokens_per_micro=budget, micro_batch_size=micro_bs)
    loss = [max(0, L - 1) for L in lengths]
    native = build_plan(lengths, loss, dp, PlannerConfig(**kw))
    assert _plan_as_json(native) == _oracle_as_json(oplan.build_plan(lengths, loss, dp, **kw))
    # With a budget above seq_len the reference itself packs micros longer than
    # seq_len, so its invariants (test_dynamic_batching.py:61-94) hold only below.
    if budget is None or budget <= seq_len:
        _check_invariants(native, lengths, PlannerConfig(**kw), dp)


@pytest.mark.parametrize("layout,budget,micro_bs", [("packed", 8192, None), ("padded", 16384, None),
                                                     ("padded", None, 5), ("packed", 3000, None)])
@pytest.mark.parametrize("dp", [1, 4])
def test_native_equals_oracle_large_batches(layout, budget, micro_bs, dp):
    """Batches of 1536 samples, where the native planner sorts by radix and
    finds each first fit through its capacity tree: the same plan as the
    oracle's sorts and linear scans.  Lengths repeat (ties broken by index),
    include 0 and lengths over seq_len (truncated), and span 2^11 and more."""
    rng = random.Random(f"{layout}-{budget}-{micro_bs}-{dp}")
    n = 1536
    lengths = [rng.choice([0, 1, 7, 2048, 8192, 9000]) if rng.random() < 0.1 else rng.randint(1, 6000)
               for _ in range(n)]
    loss = [max(0, L - rng.randint(1, 50)) for L in lengths]
    kw = dict(layout=layout, mini_batch_size=rng.choice([96, 384, 1536 // dp]), seq_len=8192, align=64,
              max_tokens_per_micro=budget, micro_batch_size=micro_bs)
    native = build_plan(lengths, loss, dp, PlannerConfig(**kw))
    assert _plan_as_json(native) == _oracle_as_json(oplan.build_plan(lengths, loss, dp, **kw))


def test_dataclass_contract():
    m = MicroPlan((), 64, ())
    assert m.is_filler and m.n_tokens == 0 and m.n_rows == 1
    mini = MiniPlan((MicroPlan((0, 1), 128, (10, 20)),), 2, 30, (30,))
    assert mini.n_docs_local == 2
    p = Plan(per_rank=((mini,),), local_indices=((5, 7),))
    assert p.dp_size == 1 and p.local_samples(list(range(10)), 0) == [5, 7]


def test_native_sample_lengths_match_oracle():
    from meshy_amd import workloads
    from meshy_amd.pipeline import RaggedSamples

    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    batch.mask[batch.offsets[3] + 1] = 0.0  # a hole inside a response
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    for seq_len in (8192, 700, 2):
        lengths, loss = ragged.sample_lengths(seq_len)
        ref_len, ref_loss = oplan.sample_lengths(batch.sample_dicts(), seq_len)
        assert lengths.tolist() == ref_len and loss.tolist() == ref_loss

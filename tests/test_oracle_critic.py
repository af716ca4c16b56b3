"""Pins the critic-reduction and rollout-metrics oracles (CPU only), and checks the
host-side wire format: the reference's known answers (test_rollout_metrics.py),
closed forms, and the samples <-> columns round trip of adapter.py."""

from __future__ import annotations

import math
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import critic as ocritic
from oracle import rollout_metrics as orm

# ------------------------------------------------------------------ rollout metrics


def _sample(length=40, prompt=10, *, reward=1.0, advantage=0.5, version=3, truncated=False, repetition=False,
            mixed=False, seed=0):
    # test_rollout_metrics.py:18-48, a plain dict in place of the TensorDict
    g = torch.Generator().manual_seed(seed)
    mask = torch.ones(length)
    mask[:prompt] = 0
    logprobs = -torch.rand(length, generator=g)
    logprobs[:prompt] = 0.0
    return {
        "tokens": torch.randint(1, 1000, (length,), generator=g),
        "logprobs": logprobs,
        "mask_assistant": mask,
        "advantage": torch.tensor(advantage),
        "weight_version": torch.tensor(version, dtype=torch.int64),
        "reward": torch.tensor(reward),
        "truncated": torch.tensor(int(truncated), dtype=torch.int64),
        "repetition": torch.tensor(int(repetition), dtype=torch.int64),
        "mixed_version": torch.tensor(int(mixed), dtype=torch.int64),
    }


def test_rollout_metrics_long_text_repetition_flag():
    # test_rollout_metrics.py:51-59
    m, _ = orm.rollout_metrics([_sample(length=30_000, prompt=5, repetition=False)], seq_len=131072)
    assert m["rollout/repetition_frac"] == 0.0


def test_rollout_metrics_use_stamps_and_rewards():
    # test_rollout_metrics.py:62-86
    samples = [
        _sample(reward=1.0, version=3, truncated=True, repetition=False, mixed=True, seed=1),
        _sample(reward=0.0, version=3, truncated=False, repetition=True, mixed=False, seed=2),
        _sample(reward=1.0, version=2, truncated=False, repetition=False, mixed=False, seed=3),
        _sample(reward=0.0, version=1, truncated=True, repetition=False, mixed=True, seed=4),
    ]
    m, hist = orm.rollout_metrics(samples, seq_len=131072, current_version=4)
    assert m["rollout/truncated_ratio"] == pytest.approx(0.5)
    assert m["rollout/repetition_frac"] == pytest.approx(0.25)
    assert m["rollout/weight_version/mixed_version_ratio"] == pytest.approx(0.5)
    assert m["rollout/weight_version/stale_ratio"] == pytest.approx(0.5)
    assert m["rollout/weight_version/staleness_mean"] == pytest.approx((1 + 1 + 2 + 3) / 4)
    assert m["rollout/weight_version/staleness_max"] == 3
    assert m["rollout/raw_reward_mean"] == pytest.approx(0.5)
    assert m["rollout/rewards"] == pytest.approx(0.5)
    assert m["rollout/pass_rate"] == pytest.approx(0.5)
    assert m["rollout/response_len/mean"] == 30
    assert m["rollout/seq_len_truncated_ratio"] == 0.0
    assert m["rollout/log_probs"] < 0.0
    assert len(hist["rollout/log_probs"]) == 4 * 30
    # closed form: the mean of the sampled tokens' log-probs
    kept = torch.cat([s["logprobs"][10:] for s in samples])
    assert m["rollout/log_probs"] == pytest.approx(float(kept.double().mean()), abs=1e-9)


def test_rollout_metrics_without_stamps_omit_the_tags():
    # test_rollout_metrics.py:89-106
    plain = [{"tokens": torch.arange(20), "logprobs": -torch.ones(20), "mask_assistant": torch.ones(20),
              "advantage": torch.tensor(0.0), "weight_version": torch.tensor(0)}]
    m, _ = orm.rollout_metrics(plain, seq_len=16)
    for tag in ("rollout/truncated_ratio", "rollout/repetition_frac",
                "rollout/weight_version/mixed_version_ratio", "rollout/raw_reward_mean"):
        assert tag not in m
    assert m["rollout/seq_len_truncated_ratio"] == 1.0


def test_rollout_metrics_percentiles_closed_form():
    samples = [_sample(length=10 + k, prompt=10, seed=k) for k in range(1, 6)]  # responses 1..5
    m, _ = orm.rollout_metrics(samples, seq_len=100)
    assert m["rollout/response_len/p25"] == 2.0 and m["rollout/response_len/p90"] == pytest.approx(4.6)
    assert m["rollout/response_len/median"] == 3.0


# ------------------------------------------------------------------ critic reductions


def test_per_sequence_mean_closed_form():
    adv = torch.tensor([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]])
    mask = torch.tensor([[0.0, 1.0, 1.0, 0.0], [0.0, 0.0, 0.0, 0.0]])
    doc = torch.tensor([[0, 0, 0, 0], [1, 1, 1, 1]])
    out = ocritic.advantages_to_per_sequence(adv, mask, doc, 2)
    assert out.tolist() == [2.5, 0.0]  # (2 + 3) / 2; an empty document -> 0 / max(0, 1)


def test_accumulator_closed_form():
    acc = ocritic.Accumulator()
    v = torch.tensor([[1.0, 2.0, 9.0]])
    r = torch.tensor([[0.0, 1.0, 5.0]])
    m = torch.tensor([[1.0, 1.0, 0.0]])
    acc.update(v, r, m, torch.tensor([1.0]), torch.tensor([7]))
    s = acc.state
    assert s["n_tokens"] == 2 and s["sum_r"] == 1.0 and s["sum_r2"] == 1.0
    assert s["sum_d"] == 2.0 and s["sum_d2"] == 2.0  # d = (1, 1)
    assert s["row_value"] == [1.5] and s["row_group"] == [7]


def test_clipped_value_error_closed_forms():
    v = torch.tensor([1.0, 3.0, 0.5])
    t = torch.tensor([0.0, 0.0, 0.0])
    o = torch.tensor([0.0, 0.0, 0.4])
    assert ocritic.clipped_value_error(v, t, None, None).tolist() == [1.0, 9.0, 0.25]
    # clip 0.2: clipped values (0.2, 0.2, 0.5): the larger squared error wins
    got = ocritic.clipped_value_error(v, t, o, 0.2)
    assert got.tolist() == pytest.approx([1.0, 9.0, 0.25])
    t2 = torch.tensor([2.0, 2.0, 2.0])
    got = ocritic.clipped_value_error(v, t2, o, 0.2)
    # v = 3 against target 2: the clipped value 0.2 is further away, 3.24 > 1
    assert got.tolist() == pytest.approx([(0.2 - 2) ** 2, (0.2 - 2) ** 2, 1.5 ** 2])


# ------------------------------------------------------------------ wire format (host side)


def test_wire_round_trip_and_validation():
    from meshy_amd import wire

    samples = [_sample(length=L, prompt=3, seed=L) for L in (5, 9, 4)]
    for s, k in zip(samples, (0, 1, 2)):
        s["teacher_topk_ids"] = torch.arange(len(s["tokens"]) * 3).reshape(-1, 3) + k
        s["note"] = f"obj{k}"
    fields = ["tokens", "logprobs", "mask_assistant", "reward", "weight_version", "teacher_topk_ids", "note"]
    cols = wire.samples_to_columns(samples, fields)
    assert cols["tokens"].is_nested and cols["reward"].shape == (3, 1)
    assert cols["weight_version"].dtype == torch.int64 and cols["note"] == ["obj0", "obj1", "obj2"]
    back = wire.columns_to_samples(cols)
    for s, b in zip(samples, back):
        assert torch.equal(b["tokens"], s["tokens"]) and torch.equal(b["teacher_topk_ids"], s["teacher_topk_ids"])
        assert b["reward"].dim() == 0 and float(b["reward"]) == float(s["reward"])
        assert int(b["weight_version"]) == int(s["weight_version"]) and b["note"] == s["note"]
    flat, off = wire.jagged_parts(cols["tokens"])
    assert off.tolist() == [0, 5, 14, 18] and torch.equal(flat, torch.cat([s["tokens"] for s in samples]))
    bad = [dict(samples[0]), dict(samples[1])]
    bad[1]["teacher_topk_ids"] = torch.zeros(9, 4, dtype=torch.long)
    with pytest.raises(ValueError, match="trailing dims"):
        wire.samples_to_columns(bad, ["teacher_topk_ids"])
    bad[1]["tokens"] = torch.zeros(3, 3, dtype=torch.long)
    with pytest.raises(ValueError, match="same rank"):
        wire.samples_to_columns(bad, ["tokens"])
    with pytest.raises(ValueError, match="empty"):
        wire.samples_to_columns([], ["tokens"])
    assert wire.field_kind("unknown") == "object"
    assert math.isclose(float(cols["reward"][0]), 1.0)


def _rollout_sample(seed, L, **kw):
    g = torch.Generator().manual_seed(seed)
    s = NS(tokens=torch.randint(0, 151936, (L,), generator=g).tolist(),
           logprobs=(-torch.rand(L, generator=g) * 3).tolist(),
           masks=[0] * min(3, L) + [1] * max(0, L - 3),
           reward=float(seed % 2), advantage=float(seed) / 7.0, raw_reward=None,
           truncated=seed % 3 == 0, repetition=seed % 4 == 0, mixed_version=seed % 5 == 0,
           positive_lm_weight=0.5 * (seed % 2))
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_sample_to_tensordict_known_answers():
    """test_rollout_stamps.py:34-46 and test_vapo_alignment.py:96-104."""
    from meshy_amd import wire

    s = NS(tokens=[1, 2, 3], logprobs=[0.0, -0.5, -0.5], masks=[0, 1, 1], reward=1.0, advantage=0.25,
           truncated=True, mixed_version=True, repetition=True)
    td = wire.sample_to_tensordict(s, weight_version=7)
    assert set(wire.GRPO_TRAINER_FIELDS) <= set(td)
    assert td["reward"].item() == 1.0 and td["truncated"].item() == 1
    assert td["mixed_version"].item() == 1 and td["repetition"].item() == 1
    assert td["weight_version"].item() == 7 and td["raw_reward"].item() == 1.0
    assert td["positive_lm_weight"].item() == 0.0  # absent: 0
    back = wire.columns_to_samples(wire.samples_to_columns([td, td], wire.GRPO_TRAINER_FIELDS),
                                   wire.GRPO_TRAINER_FIELDS)
    assert back[0]["truncated"].dtype == torch.int64 and back[1]["reward"].item() == 1.0
    group = [NS(tokens=[1, 2, 3], logprobs=[-1.0] * 3, masks=[0, 1, 1], reward=r, advantage=0.0,
                raw_reward=raw, positive_lm_weight=w)
             for r, raw, w in [(1.0, 1.0, 0.5), (0.4, 1.0, 0.5), (0.0, 0.0, 0.0), (0.0, 0.0, 0.0)]]
    fields = ("tokens", "logprobs", "mask_assistant", "reward", "positive_lm_weight")
    packed = wire.samples_to_columns([wire.sample_to_tensordict(x, 0) for x in reversed(group)], fields)
    assert packed["positive_lm_weight"].dtype == torch.float32
    assert packed["positive_lm_weight"].reshape(-1).tolist() == [0.0, 0.0, 0.5, 0.5]
    none_adv = wire.sample_to_tensordict(NS(tokens=[], logprobs=[], masks=[], reward=0.0, advantage=None), 1)
    assert none_adv["advantage"].item() == 0.0 and none_adv["tokens"].shape == (0,)


def test_rollout_group_columns_equal_the_per_sample_path():
    """The one-pass group conversion against samples_to_columns over
    sample_to_tensordict: sequences given as lists, tuples and numpy arrays,
    an empty sample, a missing advantage and raw reward, every column."""
    from meshy_amd import wire

    group = [_rollout_sample(k, L) for k, L in enumerate([5, 1, 0, 700, 33, 2048])]
    group[1].tokens = tuple(group[1].tokens)
    group[3].logprobs = np.asarray(group[3].logprobs, np.float64)
    group[4].advantage = None
    group[5].raw_reward = 0.75
    del group[0].positive_lm_weight
    fields = list(wire.GRPO_TRAINER_FIELDS) + ["positive_lm_weight", "raw_reward"]
    fast = wire.rollout_group_to_columns(group, 11, fields)
    ref = wire.samples_to_columns([wire.sample_to_tensordict(s, 11) for s in group], fields)
    for f in fields:
        if wire.field_kind(f) == "nested":
            (fv, fo), (rv, ro) = wire.jagged_parts(fast[f]), wire.jagged_parts(ref[f])
            assert fv.dtype == rv.dtype and torch.equal(fv, rv) and torch.equal(fo, ro), f
            assert all(torch.equal(a, b) for a, b in zip(fast[f].unbind(), ref[f].unbind())), f
        else:
            assert fast[f].dtype == ref[f].dtype and torch.equal(fast[f], ref[f]), f
    with pytest.raises(KeyError):
        wire.rollout_group_to_columns(group, 0, ["values"])
    with pytest.raises(ValueError, match="empty"):
        wire.rollout_group_to_columns([], 0)


def test_rollout_group_columns_feed_the_pack_buffers():
    """RaggedSamples.from_columns over the group columns stages the same bytes
    as from_samples over the per-sample tensors."""
    from meshy_amd import wire
    from meshy_amd.pipeline import RaggedSamples

    group = [_rollout_sample(k, L) for k, L in enumerate([9, 400, 17, 1024, 3, 250, 600, 64])]
    cols = wire.rollout_group_to_columns(group, 2)
    tds = [wire.sample_to_tensordict(s, 2) for s in group]
    a = RaggedSamples.from_columns(cols, [0, 4, 8])
    b = RaggedSamples.from_samples(tds, [0, 4, 8])
    assert a.view("tokens").dtype == torch.int32 and b.view("tokens").dtype == torch.int64
    assert torch.equal(a.view("tokens").long(), b.view("tokens"))
    for name in ("mask", "logprobs", "rewards", "group_off", "s_off"):
        assert torch.equal(a.view(name), b.view(name)), name


def test_weight_version_roundtrips_as_int64():
    """test_tq_grpo_pipeline.py:74-81: the version column stays int64 through
    the columns and back, for every sample of the batch."""
    from meshy_amd import wire

    samples = [wire.sample_to_tensordict(NS(tokens=[1, 2, 3][: i + 1], logprobs=[-0.5] * (i + 1),
                                            masks=[1] * (i + 1), reward=float(i % 2), advantage=0.5), 41)
               for i in range(3)]
    cols = wire.samples_to_columns(samples, wire.GRPO_TRAINER_FIELDS)
    assert cols["weight_version"].dtype == torch.int64
    back = wire.columns_to_samples(cols, wire.GRPO_TRAINER_FIELDS)
    assert len(back) == 3
    for s in back:
        assert s["weight_version"].dtype == torch.int64 and int(s["weight_version"]) == 41
    # the one-pass group conversion gives the same column
    grp = wire.rollout_group_to_columns([NS(tokens=[1, 2], logprobs=[-0.5, -0.5], masks=[1, 1], reward=1.0,
                                            advantage=0.5)] * 2, 41, wire.GRPO_TRAINER_FIELDS)
    assert grp["weight_version"].dtype == torch.int64 and grp["weight_version"].reshape(-1).tolist() == [41, 41]

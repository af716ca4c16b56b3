"""Pins the critic-reduction and rollout-metrics oracles (CPU only), and checks the
host-side wire format: the reference's known answers (test_rollout_metrics.py),
closed forms, and the samples <-> columns round trip of adapter.py."""

from __future__ import annotations

import math

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

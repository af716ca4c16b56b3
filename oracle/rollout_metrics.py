"""Oracle: TitanTrainer._rollout_metrics restated in plain Python (test infrastructure).

Follows meshy/backend/titan/metrics.py:72-131 (helpers) and 171-322 (the
metrics and histograms) over a list of dict-like samples.
"""

from __future__ import annotations

import math

import torch


def _field(sample, f, default=None):
    return sample.get(f, default) if hasattr(sample, "get") else getattr(sample, f, default)


def _as_list(value):
    if value is None:
        return []
    if torch.is_tensor(value):
        return value.detach().cpu().reshape(-1).tolist()
    try:
        return list(value)
    except TypeError:
        return [value]


def _values(samples, f):
    out = []
    for s in samples:
        v = _field(s, f, None)
        if v is None:
            continue
        for x in _as_list(v):
            try:
                out.append(float(x))
            except (TypeError, ValueError):
                pass
    return out


def _flags(samples, f):
    values = _values(samples, f)
    if len(values) != len(samples):
        return None
    return [1.0 if v > 0.5 else 0.0 for v in values]


def _percentile(values, q):
    if not values:
        return 0.0
    values = sorted(values)
    pos = (len(values) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    if lo == hi:
        return values[lo]
    return values[lo] + (values[hi] - values[lo]) * (pos - lo)


def _mean(values):
    return sum(values) / len(values) if values else 0.0


def rollout_metrics(samples, seq_len, current_version=None):
    """metrics.py:171-322."""
    rewards = _values(samples, "reward")
    raw_rewards = _values(samples, "raw_reward") or rewards
    shaped = bool(_values(samples, "raw_reward"))
    advantages = _values(samples, "advantage")
    weight_versions = _values(samples, "weight_version")
    lengths, response_lengths, logprobs = [], [], []
    for sample in samples:
        token_list = _as_list(_field(sample, "tokens", None))
        if token_list:
            lengths.append(float(len(token_list)))
        raw_mask = _field(sample, "mask_assistant", None)
        if raw_mask is None:
            raw_mask = _field(sample, "masks", None)
        mask_values = [float(v) > 0 for v in _as_list(raw_mask)]
        if raw_mask is not None:
            response_lengths.append(float(sum(mask_values)))
        lp = _as_list(_field(sample, "logprobs", None))
        if lp:
            if len(mask_values) == len(lp):
                logprobs.extend(float(v) for v, keep in zip(lp, mask_values) if keep)
            else:
                logprobs.extend(float(v) for v in lp)
    m = {}
    if response_lengths:
        m.update({
            "rollout/response_len/max": max(response_lengths),
            "rollout/response_len/mean": _mean(response_lengths),
            "rollout/response_len/median": _percentile(response_lengths, 0.5),
            "rollout/response_len/min": min(response_lengths),
            "rollout/response_len/p0": _percentile(response_lengths, 0.0),
            "rollout/response_len/p25": _percentile(response_lengths, 0.25),
            "rollout/response_len/p50": _percentile(response_lengths, 0.5),
            "rollout/response_len/p75": _percentile(response_lengths, 0.75),
            "rollout/response_len/p90": _percentile(response_lengths, 0.9),
            "rollout/response_len/p95": _percentile(response_lengths, 0.95),
            "rollout/response_len/p99": _percentile(response_lengths, 0.99),
            "rollout/response_lengths": _mean(response_lengths),
        })
    if lengths:
        m["rollout/total_lengths"] = _mean(lengths)
        m["rollout/seq_len_truncated_ratio"] = sum(v >= seq_len for v in lengths) / len(lengths)
    truncated = _flags(samples, "truncated")
    if truncated is not None:
        m["rollout/truncated_ratio"] = _mean(truncated)
        m["rollout/truncated"] = m["rollout/truncated_ratio"]
    repetition = _flags(samples, "repetition")
    if repetition is not None:
        m["rollout/repetition_frac"] = _mean(repetition)
    if advantages:
        nonzero = [v for v in advantages if abs(v) > 1e-8]
        m.update({
            "grpo_metrics/effective_count": float(len(nonzero)),
            "grpo_metrics/effective_ratio": len(nonzero) / len(advantages),
            "grpo_metrics/zero_advantage_ratio": 1.0 - len(nonzero) / len(advantages),
            "rollout/advantages": _mean(advantages),
            "rollout/advantages_abs_mean": _mean([abs(v) for v in advantages]),
        })
    if rewards:
        solved = [v > 0.5 for v in raw_rewards]
        m.update({
            "grpo_metrics/solve_all": float(all(solved)),
            "grpo_metrics/solve_none": float(not any(solved)),
            "rollout/raw_reward_mean": _mean(raw_rewards),
            "rollout/raw_reward": _mean(raw_rewards),
            "rollout/rewards": _mean(rewards),
            "rollout/reward_max": max(rewards),
            "rollout/reward_min": min(rewards),
            "rollout/pass_rate": _mean([1.0 if s else 0.0 for s in solved]),
        })
        if shaped:
            deltas = [r - raw for r, raw in zip(rewards, raw_rewards)]
            m.update({
                "rollout/shaped_reward_mean": _mean(rewards),
                "rollout/reward_shaping_delta_mean": _mean(deltas),
                "rollout/reward_penalised_ratio": _mean([1.0 if abs(d) > 1e-8 else 0.0 for d in deltas]),
            })
    if logprobs:
        m.update({"rollout/log_probs": _mean(logprobs), "rollout/rollout_log_probs": _mean(logprobs)})
    if weight_versions:
        newest = max(weight_versions)
        m.update({
            "rollout/weight_version/mean": _mean(weight_versions),
            "rollout/weight_version/min": min(weight_versions),
            "rollout/weight_version/max": newest,
            "rollout/weight_version/median": _percentile(weight_versions, 0.5),
            "rollout/weight_version/stale_ratio": _mean([1.0 if v < newest else 0.0 for v in weight_versions]),
            "rollout/weight_version/num_versions": float(len(set(weight_versions))),
        })
        if current_version is not None:
            staleness = [float(current_version) - v for v in weight_versions]
            m["rollout/weight_version/staleness_mean"] = _mean(staleness)
            m["rollout/weight_version/staleness_max"] = max(staleness)
    mixed = _flags(samples, "mixed_version")
    if mixed is not None:
        m["rollout/weight_version/mixed_version_ratio"] = _mean(mixed)
    hist = {"rollout/response_lengths": response_lengths, "rollout/total_lengths": lengths}
    if rewards:
        hist["rollout/rewards"] = rewards
    if shaped:
        hist["rollout/raw_rewards"] = raw_rewards
    if advantages:
        hist["rollout/advantages"] = advantages
    if logprobs:
        hist["rollout/log_probs"] = logprobs
    return m, hist

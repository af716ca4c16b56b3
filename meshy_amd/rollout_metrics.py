"""Batch-level rollout statistics with the call surface of
``TitanTrainer._rollout_metrics`` (meshy/backend/titan/metrics.py:171-322).

The per-token work -- response lengths, the sampled tokens' behaviour-policy
log-probs and their mean -- runs on the device over the jagged columns
(``meshy_ragged_token_stats``); the per-sample scalars (rewards, advantages,
weight versions, quality stamps, percentiles of the per-sample lengths) are
sample-level host arithmetic, as in the reference.  The histogram of sampled
log-probs is returned as a device tensor rather than a Python list.

``samples`` may be a list of mappings (the reference's input) or a batch of
wire columns (``meshy_amd.wire``): the jagged ``tokens`` / ``mask_assistant`` /
``logprobs`` columns are then read in place.
"""

from __future__ import annotations

import math
from typing import Any

import torch

from . import _lib
from .hostio import gather_into
from .wire import jagged_parts


def _percentile(values: list[float], q: float) -> float:
    """Linear-interpolated percentile of a sorted copy (metrics.py:123-131)."""
    if not values:
        return 0.0
    values = sorted(values)
    pos = (len(values) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    if lo == hi:
        return values[lo]
    return values[lo] + (values[hi] - values[lo]) * (pos - lo)


def _mean(values: list[float]) -> float:
    return sum(values) / len(values) if values else 0.0


def _get(sample: Any, f: str) -> Any:
    return sample.get(f, None) if hasattr(sample, "get") else getattr(sample, f, None)


# Every per-sample field the statistics read.
_FIELDS = ("reward", "raw_reward", "advantage", "weight_version", "truncated", "repetition", "mixed_version",
           "tokens", "mask_assistant", "masks", "logprobs")


def _per_sample(samples) -> dict[str, list]:
    """One list per field of the samples' values (None where a sample lacks the
    field): one comprehension per field over mappings, else one pass."""
    if all(isinstance(s, dict) for s in samples):
        return {f: [s.get(f) for s in samples] for f in _FIELDS}
    lists = tuple([] for _ in _FIELDS)
    pairs = tuple(zip(_FIELDS, lists))
    for s in samples:
        if isinstance(s, dict):
            for f, out in pairs:
                out.append(s.get(f))
        else:
            for f, out in pairs:
                out.append(_get(s, f))
    return dict(pairs)


def _scalars(per, columns, f: str) -> list[float]:
    """Per-sample values of a scalar column (the samples that carry one);
    ``per`` is ``_per_sample``'s lists when the input is a sample list."""
    if columns is not None:
        v = columns.get(f)
        if v is None:
            return []
        return [float(x) for x in (v.reshape(-1).tolist() if isinstance(v, torch.Tensor) else v)]
    present = [v for v in per[f] if v is not None]
    if present and all(isinstance(v, torch.Tensor) for v in present) and len({v.dtype for v in present}) == 1:
        if not present[0].is_cuda:
            # Host scalars: item() of each is cheaper than a stack and a copy.
            try:
                return [float(v.item()) for v in present]
            except RuntimeError:
                pass  # values of several elements: the stack below
        # One stack and one host copy instead of one per sample (one dtype, so
        # nothing is promoted or rounded; equal shapes flatten in sample order,
        # as the per-sample path below does).  Mixed devices or shapes raise.
        try:
            return [float(x) for x in torch.stack(present).detach().reshape(-1).cpu().tolist()]
        except RuntimeError:
            pass  # mixed devices or dtypes torch cannot stack: the general path below
    out = []
    for v in present:
        for x in (v.detach().cpu().reshape(-1).tolist() if torch.is_tensor(v) else
                  (list(v) if hasattr(v, "__iter__") else [v])):
            try:
                out.append(float(x))
            except (TypeError, ValueError):
                pass
    return out


def _flags(per, columns, n: int, f: str) -> list[float] | None:
    values = _scalars(per, columns, f)
    if len(values) != n:
        return None
    return [1.0 if v > 0.5 else 0.0 for v in values]


def _flat(col) -> tuple[torch.Tensor, torch.Tensor]:
    """(flat values, int64 offsets [B + 1]) of a jagged column, or of a list of
    per-sample values where None is an empty sample."""
    if isinstance(col, torch.Tensor):
        return jagged_parts(col)
    present = [v for v in col if v is not None]
    if (present and all(isinstance(v, torch.Tensor) and v.dim() == 1 for v in present)
            and len({v.dtype for v in present}) == 1):
        lengths = [0 if v is None else v.shape[0] for v in col]
        off = torch.zeros(len(col) + 1, dtype=torch.int64)
        torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0, out=off[1:])
        if all(not v.is_cuda for v in present) and torch.cuda.is_available():
            # Host tensors: one native multi-threaded gather into pinned
            # memory, so the copy to the device is one DMA.
            flat = torch.empty(int(off[-1]), dtype=present[0].dtype, pin_memory=True)
            return gather_into(present, flat), off
        # One concatenation in the samples' own dtype, converted once later.
        try:
            return torch.cat(present).detach(), off
        except RuntimeError:
            pass  # mixed devices: the per-sample path
    return jagged_parts([torch.zeros(0) if v is None else _as_float(v) for v in col])


def _token_stats(per, columns, device):
    """Per-sample total and response lengths and the kept log-probs (device),
    with the reference's presence rules (metrics.py:197-212): a length per sample
    with tokens, a response length per sample with a mask, log-probs kept where
    the mask is on when the sample's mask is as long as its log-probs."""
    if columns is not None:
        tok = columns.get("tokens")
        mask_col = columns.get("mask_assistant", columns.get("masks"))
        lp_col = columns.get("logprobs")
        lengths = [] if tok is None else [float(x) for x in torch.diff(jagged_parts(tok)[1]).tolist() if x > 0]
        has_mask = None if mask_col is None else [True] * (jagged_parts(mask_col)[1].numel() - 1)
    else:
        lengths = [float(n) for n in (t.shape[0] if isinstance(t, torch.Tensor) else len(t)
                                      for t in per["tokens"] if t is not None) if n > 0]
        masks = [ms if mk is None else mk for mk, ms in zip(per["mask_assistant"], per["masks"])]
        has_mask = [mk is not None for mk in masks]
        mask_col = masks if any(has_mask) else None
        lps = per["logprobs"]
        lp_col = None if all(v is None for v in lps) else lps
    if mask_col is None and lp_col is None:
        return lengths, [], None
    if mask_col is not None:
        mflat, moff = _flat(mask_col)
    else:
        mflat, moff = torch.zeros(0), torch.zeros(len(per["tokens"]) + 1, dtype=torch.int64)
    nsamp = moff.numel() - 1
    mflat = mflat.to(device=device, dtype=torch.float32, non_blocking=True).contiguous()
    moff_d = moff.to(device)
    lflat = loff_d = None
    if lp_col is not None:
        lflat, loff = _flat(lp_col)
        lflat = lflat.to(device=device, dtype=torch.float32, non_blocking=True).contiguous()
        loff_d = loff.to(device)
    resp = torch.empty(max(nsamp, 1), dtype=torch.int64, device=device)
    lp_sum = torch.empty(max(nsamp, 1), dtype=torch.float64, device=device)
    out_off = torch.empty(nsamp + 1, dtype=torch.int64, device=device)
    kept = torch.empty(max(lflat.numel() if lflat is not None else 0, 1), dtype=torch.float32, device=device)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.meshy_ragged_token_stats_workspace_size(nsamp)), 1), dtype=torch.uint8,
                     device=device)
    # Columns of no tokens have no storage; a one-element stand-in is never
    # read (every sample's range is empty) but keeps the column present.
    if mflat.numel() == 0:
        mflat = torch.zeros(1, dtype=torch.float32, device=device)
    if lflat is not None and lflat.numel() == 0:
        lflat = torch.zeros(1, dtype=torch.float32, device=device)
    rc = lib.meshy_ragged_token_stats(mflat.data_ptr(), _lib.ptr(lflat), moff_d.data_ptr(), _lib.ptr(loff_d),
                                      nsamp, resp.data_ptr(), lp_sum.data_ptr(), out_off.data_ptr(),
                                      _lib.ptr(kept if lflat is not None else None), ws.data_ptr(), ws.numel(),
                                      _lib.stream_of(device))
    _lib.check(rc, "meshy_ragged_token_stats")
    response_lengths = []
    if has_mask is not None:
        response_lengths = [float(x) for x, h in zip(resp[:nsamp].tolist(), has_mask) if h]
    logprobs = None
    if lflat is not None:
        n_kept = int(out_off[-1].item())
        logprobs = (kept[:n_kept], float(lp_sum[:nsamp].sum().item()))
    return lengths, response_lengths, logprobs


def _as_float(v: Any) -> torch.Tensor:
    t = v if torch.is_tensor(v) else torch.as_tensor(v)
    return t.reshape(-1).to(torch.float32)


def rollout_metrics(samples: Any, seq_len: int, current_version: int | None = None, *,
                    device=None) -> tuple[dict[str, float], dict[str, Any]]:
    """Drop-in for ``TitanTrainer._rollout_metrics`` (metrics.py:171-322)."""
    columns = samples if isinstance(samples, dict) else None
    if columns is not None:
        first = next(iter(columns.values()))
        n = first.size(0) if isinstance(first, torch.Tensor) else len(first)
    else:
        n = len(samples)
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    per = None if columns is not None else _per_sample(samples)
    rewards = _scalars(per, columns, "reward")
    raw = _scalars(per, columns, "raw_reward")
    raw_rewards = raw or rewards
    shaped = bool(raw)
    advantages = _scalars(per, columns, "advantage")
    weight_versions = _scalars(per, columns, "weight_version")
    lengths, response_lengths, lp = _token_stats(per, columns, torch.device(device))

    m: dict[str, float] = {}
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
    truncated = _flags(per, columns, n, "truncated")
    if truncated is not None:
        m["rollout/truncated_ratio"] = _mean(truncated)
        m["rollout/truncated"] = m["rollout/truncated_ratio"]
    repetition = _flags(per, columns, n, "repetition")
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
            deltas = [r - w for r, w in zip(rewards, raw_rewards)]
            m.update({
                "rollout/shaped_reward_mean": _mean(rewards),
                "rollout/reward_shaping_delta_mean": _mean(deltas),
                "rollout/reward_penalised_ratio": _mean([1.0 if abs(d) > 1e-8 else 0.0 for d in deltas]),
            })
    kept = None
    if lp is not None and lp[0].numel():
        kept, total = lp
        mean_lp = total / kept.numel()
        m.update({"rollout/log_probs": mean_lp, "rollout/rollout_log_probs": mean_lp})
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
    mixed = _flags(per, columns, n, "mixed_version")
    if mixed is not None:
        m["rollout/weight_version/mixed_version_ratio"] = _mean(mixed)

    hist: dict[str, Any] = {"rollout/response_lengths": response_lengths, "rollout/total_lengths": lengths}
    if rewards:
        hist["rollout/rewards"] = rewards
    if shaped:
        hist["rollout/raw_rewards"] = raw_rewards
    if advantages:
        hist["rollout/advantages"] = advantages
    if kept is not None:
        hist["rollout/log_probs"] = kept
    return m, hist


__all__ = ["rollout_metrics"]

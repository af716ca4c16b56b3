"""Oracle: GRPO group normalisation restated on CPU torch (test infrastructure).

Follows grpo_advantage (meshy/worker/rollout.py:88-97): a size-1 group keeps
its reward; otherwise (r - mean) / clamp(unbiased std, min=1e-8) in fp32.
zero_variance_group follows is_zero_variance_group (rollout.py:100-115).
"""

from __future__ import annotations

import torch


def grpo_group(rewards: list[float]) -> list[float]:
    if len(rewards) == 1:
        return [float(rewards[0])]
    r = torch.tensor(rewards, dtype=torch.float32)
    adv = (r - r.mean()) / r.std().clamp(min=1e-8)
    return [float(a) for a in adv]


def grpo_batched(rewards: torch.Tensor, group_offsets) -> torch.Tensor:
    out = torch.empty_like(rewards, dtype=torch.float32)
    offs = [int(x) for x in group_offsets]
    for g in range(len(offs) - 1):
        a, b = offs[g], offs[g + 1]
        out[a:b] = torch.tensor(grpo_group(rewards[a:b].tolist()))
    return out


def zero_variance_group(raw_rewards: list[float], tolerance: float = 1e-8) -> bool:
    """rollout.py:109-115: an empty group counts as zero variance; otherwise
    the spread max - min of the Python floats, taken with the builtins (their
    NaN behaviour included), is compared with the tolerance."""
    if not raw_rewards:
        return True
    rewards = [float(r) for r in raw_rewards]
    return max(rewards) - min(rewards) <= tolerance


def zero_variance_batched(raw_rewards, group_offsets, tolerance: float = 1e-8) -> list[bool]:
    offs = [int(x) for x in group_offsets]
    vals = [float(x) for x in raw_rewards]
    return [zero_variance_group(vals[offs[g]:offs[g + 1]], tolerance) for g in range(len(offs) - 1)]

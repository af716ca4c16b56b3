"""GRPO group-normalised advantages (meshy/worker/rollout.py:88-97) and the
zero-variance group filter (rollout.py:100-115).

``grpo_advantage(samples)`` keeps the advantage-plugin contract of the
rollout worker (called as ``fn(group, **kwargs)``, mutates
``sample.advantage``, rollout.py:580-587).  ``grpo_advantages`` normalises
every group of a batch in one launch on the device, which is what the packed
pipeline uses: a size-1 group keeps its reward, any other group gets
``(r - mean) / clamp(unbiased std, min=1e-8)``.

``zero_variance_groups`` flags every group of a batch whose raw rewards are
all equal within a tolerance, in one launch; ``is_zero_variance_group(samples)``
keeps the reference's per-group signature.  The per-group forms cost a
host-to-device copy, a launch and a synchronisation per group, more than the
reference's host arithmetic over a handful of scalars: callers that hold a
whole batch of groups use the batched forms.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib


def grpo_advantages(rewards: torch.Tensor, group_offsets: torch.Tensor) -> torch.Tensor:
    """Advantages of all groups at once; ``group_offsets`` is ``[n_groups + 1]``."""
    _lib.require_gpu(rewards, group_offsets)
    r = rewards.to(torch.float32).contiguous()
    off = group_offsets.to(torch.int64).contiguous()
    n_groups = off.numel() - 1
    if n_groups < 0:
        raise ValueError("group_offsets must hold at least one entry")
    adv = torch.empty_like(r)
    rc = _lib.load().meshy_grpo_advantage(r.data_ptr(), r.numel(), off.data_ptr(), n_groups, adv.data_ptr(),
                                          _lib.stream_of(r.device))
    _lib.check(rc, "meshy_grpo_advantage")
    return adv


def grpo_advantage(samples: list[Any], device: torch.device | str | None = None) -> None:
    """Plugin form: one group, ``sample.advantage`` set to a Python float."""
    if not samples:
        return
    if len(samples) == 1:
        # A size-1 group keeps its reward object as is (rollout.py:91-93).
        samples[0].advantage = samples[0].reward
        return
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    rewards = torch.tensor([float(s.reward) for s in samples], dtype=torch.float32).to(dev)
    off = torch.tensor([0, len(samples)], dtype=torch.int64).to(dev)
    adv = grpo_advantages(rewards, off).tolist()
    for s, a in zip(samples, adv):
        s.advantage = float(a)


def zero_variance_groups(raw_rewards: torch.Tensor, group_offsets: torch.Tensor,
                         tolerance: float = 1e-8) -> torch.Tensor:
    """Bool ``[n_groups]``: group g's raw rewards span at most ``tolerance``
    (rollout.py:100-115), compared in float64 as the reference's Python floats
    are.  An empty group is True; a group whose first reward is NaN is False;
    later NaNs are skipped, as Python's ``max``/``min`` skip them."""
    _lib.require_gpu(raw_rewards, group_offsets)
    r = raw_rewards.to(torch.float64).contiguous()
    off = group_offsets.to(torch.int64).contiguous()
    n_groups = off.numel() - 1
    if n_groups < 0:
        raise ValueError("group_offsets must hold at least one entry")
    flags = torch.empty(n_groups, dtype=torch.uint8, device=r.device)
    rc = _lib.load().meshy_zero_variance_groups(_lib.ptr(r) if r.numel() else None, r.numel(), off.data_ptr(),
                                                n_groups, float(tolerance), flags.data_ptr(),
                                                _lib.stream_of(r.device))
    _lib.check(rc, "meshy_zero_variance_groups")
    return flags.view(torch.bool)


def is_zero_variance_group(samples: list[Any], *, tolerance: float = 1e-8,
                           device: torch.device | str | None = None) -> bool:
    """Plugin form (rollout.py:100-115): whether all raw rewards of a completed
    group are equal.  The raw reward (``sample.raw_reward`` when set, else
    ``sample.reward``) is used, so length shaping does not hide a group whose
    outcomes were all the same."""
    if not samples:
        return True
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    raw = [float(s.reward if getattr(s, "raw_reward", None) is None else s.raw_reward) for s in samples]
    r = torch.tensor(raw, dtype=torch.float64).to(dev)
    off = torch.tensor([0, len(raw)], dtype=torch.int64).to(dev)
    return bool(zero_variance_groups(r, off, tolerance).item())


__all__ = ["grpo_advantage", "grpo_advantages", "is_zero_variance_group", "zero_variance_groups"]

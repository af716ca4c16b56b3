"""GRPO group-normalised advantages (meshy/worker/rollout.py:88-97).

``grpo_advantage(samples)`` keeps the advantage-plugin contract of the
rollout worker (called as ``fn(group, **kwargs)``, mutates
``sample.advantage``, rollout.py:580-587).  ``grpo_advantages`` normalises
every group of a batch in one launch on the device, which is what the packed
pipeline uses: a size-1 group keeps its reward, any other group gets
``(r - mean) / clamp(unbiased std, min=1e-8)``.
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


__all__ = ["grpo_advantage", "grpo_advantages"]

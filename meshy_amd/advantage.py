"""GRPO group-normalised advantages (meshy/worker/rollout.py:88-97) and the
zero-variance group filter (rollout.py:100-115), for every group of a step at
once.

``grpo_advantages(rewards, group_offsets)`` normalises all groups in one launch
on the device: a size-1 group keeps its reward, any other group gets
``(r - mean) / clamp(unbiased std, min=1e-8)``.  ``pack_step`` runs it on the
rewards it uploads with the samples.  ``zero_variance_groups`` flags every
group whose raw rewards are all equal within a tolerance, in one launch.

The reference calls its two functions once per completed group of the rollout
worker (rollout.py:572, 580-587), on rewards held on the host.  A device call
per group of a few scalars would cost a copy, a launch and a synchronisation,
several times the reference's host arithmetic, so host rewards are handled by
the library's host code: ``grpo_advantage`` is the per-group plugin form (one
native call per group), and both batched functions take host tensors as well
as device ones.  ``pack_step`` computes the advantages on the device from the
rewards it uploads with the samples.  The per-group filter keeps the
reference's Python function: eight comparisons are cheaper than any call into
a library; a batch of groups goes through ``zero_variance_groups``.
"""

from __future__ import annotations

import ctypes
from typing import Any

import torch

from . import _lib


def grpo_advantages(rewards: torch.Tensor, group_offsets: torch.Tensor) -> torch.Tensor:
    """Advantages of all groups at once; ``group_offsets`` is ``[n_groups + 1]``.
    Device tensors go through ``meshy_grpo_advantage``, host tensors through
    ``meshy_grpo_advantage_host``; the advantages come back where the rewards
    are."""
    if rewards.is_cuda != group_offsets.is_cuda:
        raise ValueError("rewards and group_offsets must both be on the GPU or both on the host")
    r = rewards.to(torch.float32).contiguous()
    off = group_offsets.to(torch.int64).contiguous()
    n_groups = off.numel() - 1
    if n_groups < 0:
        raise ValueError("group_offsets must hold at least one entry")
    adv = torch.empty_like(r)
    lib = _lib.load()
    if r.is_cuda:
        rc = lib.meshy_grpo_advantage(r.data_ptr(), r.numel(), off.data_ptr(), n_groups, adv.data_ptr(),
                                      _lib.stream_of(r.device))
    else:
        rc = lib.meshy_grpo_advantage_host(_lib.ptr(r) if r.numel() else None, r.numel(), off.data_ptr(), n_groups,
                                           _lib.ptr(adv) if adv.numel() else None)
    _lib.check(rc, "meshy_grpo_advantage")
    return adv


def grpo_advantage(samples: list[Any]) -> None:
    """Drop-in for ``grpo_advantage`` (rollout.py:88-97), the rollout worker's
    per-group advantage plugin (rollout.py:580-587): sets each sample's
    ``advantage`` from the group's rewards in one host call of the library
    (the rewards are host floats there, so no device round trip)."""
    n = len(samples)
    if n == 1:
        samples[0].advantage = samples[0].reward
        return
    if n == 0:
        return
    r = (ctypes.c_float * n)(*[float(s.reward) for s in samples])
    out = (ctypes.c_float * n)()
    off = (ctypes.c_int64 * 2)(0, n)
    _lib.check(_lib.load().meshy_grpo_advantage_host(r, n, off, 1, out), "meshy_grpo_advantage_host")
    for s, a in zip(samples, out):
        s.advantage = a


def zero_variance_groups(raw_rewards: torch.Tensor, group_offsets: torch.Tensor,
                         tolerance: float = 1e-8) -> torch.Tensor:
    """Bool ``[n_groups]``: group g's raw rewards span at most ``tolerance``
    (rollout.py:100-115), compared in float64 as the reference's Python floats
    are.  An empty group is True; a group whose first reward is NaN is False;
    later NaNs are skipped, as Python's ``max``/``min`` skip them.

    Device tensors are filtered by ``meshy_zero_variance_groups``; host
    tensors (the rewards as the rollout worker holds them) by
    ``meshy_zero_variance_groups_host``, without a device round trip.  The
    flags come back where the rewards are."""
    if raw_rewards.is_cuda != group_offsets.is_cuda:
        raise ValueError("raw_rewards and group_offsets must both be on the GPU or both on the host")
    r = raw_rewards.to(torch.float64).contiguous()
    off = group_offsets.to(torch.int64).contiguous()
    n_groups = off.numel() - 1
    if n_groups < 0:
        raise ValueError("group_offsets must hold at least one entry")
    flags = torch.empty(n_groups, dtype=torch.uint8, device=r.device)
    lib = _lib.load()
    rp = _lib.ptr(r) if r.numel() else None
    if r.is_cuda:
        rc = lib.meshy_zero_variance_groups(rp, r.numel(), off.data_ptr(), n_groups, float(tolerance),
                                            flags.data_ptr(), _lib.stream_of(r.device))
    else:
        rc = lib.meshy_zero_variance_groups_host(rp, r.numel(), off.data_ptr(), n_groups, float(tolerance),
                                                 flags.data_ptr())
    _lib.check(rc, "meshy_zero_variance_groups")
    return flags.view(torch.bool)


__all__ = ["grpo_advantage", "grpo_advantages", "zero_variance_groups"]

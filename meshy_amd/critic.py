"""Critic-side reductions with the call surfaces of the reference's critic path.

* ``advantages_to_per_sequence`` (meshy/backend/titan/critic/gae.py:296-312):
  ``meshy_per_sequence_mean``, one workgroup per document;
* ``Accumulator`` / ``AccumulatorState`` (meshy/backend/titan/critic/metrics.py:
  220-275): ``meshy_critic_accumulate`` folds each ``[rows, S]`` micro-batch on
  the device; the window sums stay there until ``state`` is read, so a window
  of micro-batches costs one host synchronisation instead of five per update;
* ``clipped_value_error`` (meshy/backend/titan/vapo.py:35-41): an autograd
  Function over ``meshy_clipped_value_error`` and its backward.

``compute_returns`` on the critic path (engine/critic.py:348-350) is
``meshy_amd.gae.compute_returns``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib
from .gae import compute_returns
from .loss import checked_segment_offsets


def advantages_to_per_sequence(adv: torch.Tensor, mask: torch.Tensor, doc_ids: torch.Tensor,
                               n_docs: int) -> torch.Tensor:
    """Masked token-mean of per-token ``adv``, one fp32 scalar per document
    (gae.py:296-312); the padding slot is ignored.  ``doc_ids`` must be
    non-decreasing over the flattened micro-batch, as both batch layouts make
    them (checked once per tensor: ValueError otherwise)."""
    _lib.require_gpu(adv, mask, doc_ids)
    n_docs = int(n_docs)
    out = torch.empty(n_docs, dtype=torch.float32, device=adv.device)
    if n_docs == 0:
        return out
    x = adv.reshape(-1).to(torch.float32).contiguous()
    m = mask.reshape(-1).to(torch.float32).contiguous()
    if m.numel() != x.numel() or doc_ids.numel() != x.numel():
        raise ValueError(f"adv has {x.numel()} tokens but mask and doc_ids have {m.numel()} and {doc_ids.numel()}")
    off = checked_segment_offsets(doc_ids, n_docs + 1)
    rc = _lib.load().meshy_per_sequence_mean(x.data_ptr(), m.data_ptr(), off.data_ptr(), n_docs, out.data_ptr(),
                                             _lib.stream_of(adv.device))
    _lib.check(rc, "meshy_per_sequence_mean")
    return out


@dataclass
class AccumulatorState:
    """Per-rank partial sums of one window (metrics.py:220-235)."""

    n_tokens: float = 0.0
    sum_r: float = 0.0
    sum_r2: float = 0.0
    sum_d: float = 0.0
    sum_d2: float = 0.0
    row_value: list[float] = field(default_factory=list)
    row_reward: list[float] = field(default_factory=list)
    row_group: list[int] = field(default_factory=list)


class Accumulator:
    """Fold ``[rows, S]`` micro-batches into an :class:`AccumulatorState`
    (metrics.py:238-275), on the device."""

    def __init__(self) -> None:
        self._sums: torch.Tensor | None = None  # fp64 [5] on the device
        self._row_value: list[torch.Tensor] = []
        self._row_reward: list[torch.Tensor] = []
        self._row_group: list[torch.Tensor] = []
        self._state: AccumulatorState | None = AccumulatorState()

    @torch.no_grad()
    def update(self, values: torch.Tensor, returns: torch.Tensor, mask: torch.Tensor, rewards: torch.Tensor,
               group_ids: torch.Tensor) -> None:
        if values.dim() != 2 or returns.shape != values.shape or mask.shape != values.shape:
            raise ValueError("values, returns and mask must be [rows, S] of one shape")
        _lib.require_gpu(values, returns, mask)
        dev = values.device
        rows, S = values.shape
        bf16 = values.dtype == torch.bfloat16
        v = values.contiguous() if bf16 else values.to(torch.float32).contiguous()
        r = returns.to(torch.float32).contiguous()
        m = mask.to(torch.float32).contiguous()
        sums = torch.empty(5, dtype=torch.float64, device=dev)
        row_value = torch.empty(rows, dtype=torch.float32, device=dev)
        lib = _lib.load()
        ws = torch.empty(max(int(lib.meshy_critic_accumulate_workspace_size(rows)), 1), dtype=torch.uint8,
                         device=dev)
        rc = lib.meshy_critic_accumulate(v.data_ptr(), int(bf16), r.data_ptr(), m.data_ptr(), rows, S,
                                         sums.data_ptr(), row_value.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream_of(dev))
        _lib.check(rc, "meshy_critic_accumulate")
        self._sums = sums if self._sums is None else self._sums + sums
        self._row_value.append(row_value)
        self._row_reward.append(rewards.detach().float().reshape(-1))
        self._row_group.append(group_ids.detach().reshape(-1))
        self._state = None

    @property
    def state(self) -> AccumulatorState:
        """The window's partials as host values (one synchronisation)."""
        if self._state is None:
            st = AccumulatorState()
            if self._sums is not None:
                # One device-to-host copy: the fp64 sums, the per-row values and
                # rewards as fp64, and the group ids bit-cast to fp64.
                vals = torch.cat(self._row_value).to(torch.float64)
                rews = torch.cat(self._row_reward).to(torch.float64)
                grps = torch.cat(self._row_group).to(torch.int64).view(torch.float64)
                host = torch.cat([self._sums, vals, rews, grps]).cpu()
                n = vals.numel()
                st.n_tokens, st.sum_r, st.sum_r2, st.sum_d, st.sum_d2 = host[:5].tolist()
                st.row_value = host[5:5 + n].tolist()
                st.row_reward = host[5 + n:5 + 2 * n].tolist()
                st.row_group = host[5 + 2 * n:].view(torch.int64).tolist()
            self._state = st
        return self._state


class _ClippedValueError(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v, t, o, clip):
        out = torch.empty_like(v)
        has = clip is not None
        rc = _lib.load().meshy_clipped_value_error(v.data_ptr(), t.data_ptr(), _lib.ptr(o), int(has),
                                                   float(clip) if has else 0.0, v.numel(), out.data_ptr(),
                                                   _lib.stream_of(v.device))
        _lib.check(rc, "meshy_clipped_value_error")
        ctx.save_for_backward(v, t, o if o is not None else v)
        ctx.clip = clip
        return out

    @staticmethod
    def backward(ctx, g):
        v, t, o = ctx.saved_tensors
        clip = ctx.clip
        has = clip is not None
        gv = torch.empty_like(v)
        gc = g.to(torch.float32)
        # The gradient of a sum or a mean is one value broadcast (stride 0):
        # the kernel reads it as such instead of a materialised copy.
        stride = 0 if gc.dim() == 1 and gc.stride(0) == 0 else 1
        if stride:
            gc = gc.contiguous()
        rc = _lib.load().meshy_clipped_value_error_bwd(v.data_ptr(), t.data_ptr(), o.data_ptr() if has else None,
                                                       int(has), float(clip) if has else 0.0, v.numel(),
                                                       gc.data_ptr(), stride, gv.data_ptr(),
                                                       _lib.stream_of(v.device))
        _lib.check(rc, "meshy_clipped_value_error_bwd")
        return gv, None, None, None


def clipped_value_error(values: torch.Tensor, targets: torch.Tensor, old_values: torch.Tensor | None,
                        clip: float | None) -> torch.Tensor:
    """Per-token ``(v - t)^2``, or with ``clip`` the PPO-style clipped maximum
    (vapo.py:35-41); differentiable in ``values``."""
    _lib.require_gpu(values, targets, old_values if clip is not None else None)
    shape = values.shape
    v = values.to(torch.float32).reshape(-1).contiguous()
    t = targets.detach().to(torch.float32).reshape(-1).contiguous()
    o = None
    if clip is not None:
        o = old_values.detach().to(torch.float32).reshape(-1).contiguous()
    for name, x in (("targets", t), ("old_values", o)):
        if x is not None and x.numel() != v.numel():
            raise ValueError(f"values has {v.numel()} elements but {name} has {x.numel()}")
    return _ClippedValueError.apply(v, t, o, clip).reshape(shape)


__all__ = ["Accumulator", "AccumulatorState", "advantages_to_per_sequence", "clipped_value_error",
           "compute_returns"]

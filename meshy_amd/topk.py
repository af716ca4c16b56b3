"""Student Top-K OPD kernels with the call surface of
meshy/backend/titan/topk_loss.py: Teacher Top-K extraction, the gather of
student log-probs at given ids, and the forward KL over the Teacher's Top-K.

The reference works on ``chunk``-row slices of the logits, upcasting each to
fp32 (topk_loss.py:26-31, 50-56) and recomputing the chunk in backward.  Here
each function streams every row of bf16 logits from HBM once:

* ``teacher_topk``     ``meshy_topk_logprobs`` (Top-K and log-sum-exp in one pass);
* ``gather_logprobs``  ``meshy_gather_logprobs_fwd`` / ``_bwd`` (the fused
                       log-softmax gather of the PPO path with K ids per row);
* ``forward_kl_topk``  ``meshy_forward_kl_topk`` / ``_bwd``.

``chunk`` is accepted for signature compatibility; no chunking is needed.
"""

from __future__ import annotations

import torch

from . import _lib
from .logprob import _prep, bwd_workspace


def _dense(logits: torch.Tensor) -> torch.Tensor:
    return logits.full_tensor() if hasattr(logits, "full_tensor") else logits


@torch.no_grad()
def teacher_topk(logits: torch.Tensor, k: int, *, chunk: int = 1024) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-K ids and their log-probs of ``logits`` ``[rows, S, V]`` -> ``[rows, S, K]``
    (topk_loss.py:20-32).  NaN ranks above +inf and ties (NaNs among themselves) by ascending
    vocabulary index, as a stable descending sort orders them."""
    logits, _ = _prep(_dense(logits), None)
    rows, S, V = logits.shape
    if not 1 <= int(k) <= V:
        raise ValueError(f"k must be in [1, {V}], got {k}")
    dev = logits.device
    ids = torch.empty(rows, S, int(k), dtype=torch.int64, device=dev)
    lps = torch.empty(rows, S, int(k), dtype=torch.float32, device=dev)
    rc = _lib.load().meshy_topk_logprobs(
        logits.data_ptr(), rows, S, V, logits.stride(0), logits.stride(1), int(k), ids.data_ptr(),
        lps.data_ptr(), None, _lib.stream_of(dev))
    _lib.check(rc, "meshy_topk_logprobs")
    return ids, lps


def _gather_fwd(logits, ids, want_lse: bool):
    rows, S, V = logits.shape
    K = ids.shape[-1]
    dev = logits.device
    out = torch.empty(rows, S, K, dtype=torch.float32, device=dev)
    lse = torch.empty(rows, S, dtype=torch.float32, device=dev) if want_lse else None
    rc = _lib.load().meshy_gather_logprobs_fwd(
        logits.data_ptr(), rows, S, V, logits.stride(0), logits.stride(1), ids.data_ptr(), K,
        out.data_ptr(), _lib.ptr(lse), _lib.stream_of(dev))
    _lib.check(rc, "meshy_gather_logprobs_fwd")
    return out, lse


class _GatherLogprobs(torch.autograd.Function):
    """out = log_softmax(logits.float()).gather(-1, ids) with a fused backward."""

    @staticmethod
    def forward(ctx, logits, ids):
        out, lse = _gather_fwd(logits, ids, want_lse=True)
        ctx.save_for_backward(logits, ids, lse)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        logits, ids, lse = ctx.saved_tensors
        rows, S, V = logits.shape
        K = ids.shape[-1]
        grad = torch.empty(rows, S, V, dtype=logits.dtype, device=logits.device)
        g = grad_out.float().contiguous()
        ws = bwd_workspace(rows * S, logits.device)
        rc = _lib.load().meshy_gather_logprobs_bwd(
            logits.data_ptr(), rows, S, V, logits.stride(0), logits.stride(1), ids.data_ptr(), K,
            lse.data_ptr(), g.data_ptr(), grad.data_ptr(), ws.data_ptr(), ws.numel(),
            _lib.stream_of(logits.device))
        _lib.check(rc, "meshy_gather_logprobs_bwd")
        return grad, None


def gather_logprobs(logits: torch.Tensor, ids: torch.Tensor, *, chunk: int = 1024) -> torch.Tensor:
    """``log_softmax(logits).gather(ids)`` without materialising ``[rows, S, V]`` fp32
    (topk_loss.py:40-57).  ``ids`` is ``[rows, S, K]``; the result has the same shape
    in fp32 and carries a gradient to ``logits`` when they require one."""
    logits, _ = _prep(_dense(logits), None)
    if ids.dim() != 3 or ids.shape[:2] != logits.shape[:2]:
        raise ValueError(f"ids {tuple(ids.shape)} do not match logits {tuple(logits.shape[:2])} + (K,)")
    _lib.require_gpu(ids)
    ids = ids.to(torch.int64).contiguous()
    if torch.is_grad_enabled() and logits.requires_grad:
        return _GatherLogprobs.apply(logits, ids)
    out, _ = _gather_fwd(logits, ids, want_lse=False)
    return out


def _kl_args(log_prob_min_clamp, loss_max_clamp):
    lp = log_prob_min_clamp is not None
    lm = loss_max_clamp is not None
    return (int(lp), float(log_prob_min_clamp) if lp else 0.0, int(lm), float(loss_max_clamp) if lm else 0.0)


class _ForwardKL(torch.autograd.Function):
    @staticmethod
    def forward(ctx, student, teacher, clamps):
        n, K = student.shape
        kl = torch.empty(n, dtype=torch.float32, device=student.device)
        rc = _lib.load().meshy_forward_kl_topk(student.data_ptr(), teacher.data_ptr(), n, K, *clamps,
                                               kl.data_ptr(), _lib.stream_of(student.device))
        _lib.check(rc, "meshy_forward_kl_topk")
        ctx.save_for_backward(student, teacher)
        ctx.clamps = clamps
        return kl

    @staticmethod
    def backward(ctx, grad_kl):
        student, teacher = ctx.saved_tensors
        n, K = student.shape
        g = grad_kl.float().contiguous()
        grad = torch.empty_like(student)
        rc = _lib.load().meshy_forward_kl_topk_bwd(student.data_ptr(), teacher.data_ptr(), n, K, *ctx.clamps,
                                                   g.data_ptr(), grad.data_ptr(), _lib.stream_of(student.device))
        _lib.check(rc, "meshy_forward_kl_topk_bwd")
        return grad, None, None


def forward_kl_topk(
    student_topk_logprobs: torch.Tensor,
    teacher_topk_logprobs: torch.Tensor,
    *,
    log_prob_min_clamp: float | None = None,
    loss_max_clamp: float | None = None,
) -> torch.Tensor:
    """Per-position ``sum_k p_T(k) (log p_T(k) - log p_S(k))`` over the Teacher's Top-K
    (topk_loss.py:60-80): both log-prob tensors clamped from below, the per-token KL
    from above and below.  Differentiable in the student log-probs."""
    if student_topk_logprobs.shape != teacher_topk_logprobs.shape:
        raise ValueError(f"student {tuple(student_topk_logprobs.shape)} and teacher "
                         f"{tuple(teacher_topk_logprobs.shape)} shapes differ")
    _lib.require_gpu(student_topk_logprobs, teacher_topk_logprobs)
    lead = student_topk_logprobs.shape[:-1]
    K = student_topk_logprobs.shape[-1]
    s = student_topk_logprobs.float().reshape(-1, K).contiguous()
    t = teacher_topk_logprobs.detach().float().reshape(-1, K).contiguous()
    clamps = _kl_args(log_prob_min_clamp, loss_max_clamp)
    return _ForwardKL.apply(s, t, clamps).reshape(lead)


__all__ = ["forward_kl_topk", "gather_logprobs", "teacher_topk"]

"""Fused packed logprob + entropy, the drop-in for the chunk loop of
TitanTrainer._forward_logprobs (meshy/backend/titan/trainer.py:451-527).

The reference upcasts every ``logprob_chunk_size`` slice of the bf16 logits
to fp32, runs ``-cross_entropy`` on it, then upcasts ``entropy_chunk_size``
slices again for ``logsumexp - sum(softmax * z)``.  Here one HIP kernel
(``meshy_logprob_entropy_fwd``) streams each row of bf16 logits from HBM
once and returns both values in fp32; under autograd the backward kernel
(``meshy_logprob_bwd``) rebuilds ``softmax`` from the saved per-row
log-sum-exp instead of a checkpointed recompute.
"""

from __future__ import annotations

import torch

from . import _lib

IGNORE_INDEX = -100


def _prep(logits: torch.Tensor, labels: torch.Tensor | None):
    if hasattr(logits, "full_tensor"):
        # A vocab-sharded DTensor: gathered like the reference's entropy path
        # (trainer.py:439-440).  A one-GPU run never takes this branch.
        logits = logits.full_tensor()
    if logits.dim() != 3:
        raise ValueError(f"logits must be [rows, T, V], got {tuple(logits.shape)}")
    if logits.dtype != torch.bfloat16:
        raise ValueError(f"logits must be bfloat16, got {logits.dtype}")
    _lib.require_gpu(logits, labels)
    if logits.stride(2) != 1:
        logits = logits.contiguous()
    if labels is not None:
        if labels.shape != logits.shape[:2]:
            raise ValueError(
                f"labels {tuple(labels.shape)} do not match logits {tuple(logits.shape[:2])}"
            )
        labels = labels.to(torch.int64).contiguous()
    return logits, labels


def _fwd(logits, labels, *, want_logp: bool, want_entropy: bool, want_lse: bool):
    rows, T, V = logits.shape
    dev = logits.device
    logp = torch.empty(rows, T, dtype=torch.float32, device=dev) if want_logp else None
    ent = torch.empty(rows, T, dtype=torch.float32, device=dev) if want_entropy else None
    lse = torch.empty(rows, T, dtype=torch.float32, device=dev) if want_lse else None
    lib = _lib.load()
    rc = lib.meshy_logprob_entropy_fwd(
        logits.data_ptr(), rows, T, V, logits.stride(0), logits.stride(1),
        _lib.ptr(labels), _lib.ptr(logp), _lib.ptr(ent), _lib.ptr(lse), _lib.stream_of(dev),
    )
    _lib.check(rc, "meshy_logprob_entropy_fwd")
    return logp, ent, lse


def bwd_workspace(n_rows: int, device) -> torch.Tensor:
    """Scratch of the logprob / gather backward: two floats per row."""
    nbytes = int(_lib.load().meshy_logprob_bwd_workspace_size(n_rows))
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


class _FusedLogprob(torch.autograd.Function):
    """logp = log_softmax(logits.float()).gather(labels) with a fused backward."""

    @staticmethod
    def forward(ctx, logits, labels, with_entropy):
        logp, ent, lse = _fwd(logits, labels, want_logp=True, want_entropy=with_entropy,
                              want_lse=True)
        ctx.save_for_backward(logits, labels, lse)
        if ent is not None:
            ctx.mark_non_differentiable(ent)
        # The backward reads only logp's gradient: no zero tensor for the entropy's.
        ctx.set_materialize_grads(False)
        return logp, ent

    @staticmethod
    def backward(ctx, grad_logp, grad_ent):
        if grad_logp is None:
            return None, None, None
        logits, labels, lse = ctx.saved_tensors
        rows, T, V = logits.shape
        grad = torch.empty(rows, T, V, dtype=logits.dtype, device=logits.device)
        g = grad_logp.float().contiguous()
        lib = _lib.load()
        ws = bwd_workspace(rows * T, logits.device)
        rc = lib.meshy_logprob_bwd(
            logits.data_ptr(), rows, T, V, logits.stride(0), logits.stride(1), labels.data_ptr(),
            lse.data_ptr(), g.data_ptr(), grad.data_ptr(), ws.data_ptr(), ws.numel(),
            _lib.stream_of(logits.device),
        )
        _lib.check(rc, "meshy_logprob_bwd")
        return grad, None, None


def logprobs_and_entropy(
    logits: torch.Tensor, labels: torch.Tensor, *, with_entropy: bool = False
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Per-position ``log p(label)`` (and the detached entropy) of ``[rows, T, V]`` logits.

    Drop-in for the chunk loop at trainer.py:505-527: returns what
    ``torch.cat(out_chunks, 1)`` (and ``torch.cat(ent_chunks, 1)``) return,
    fp32 ``[rows, T]``.  With grad enabled and ``logits.requires_grad`` the
    log-probs carry a gradient to the logits.
    """
    logits, labels = _prep(logits, labels)
    if torch.is_grad_enabled() and logits.requires_grad:
        logp, ent = _FusedLogprob.apply(logits, labels, with_entropy)
    else:
        logp, ent, _ = _fwd(logits, labels, want_logp=True, want_entropy=with_entropy,
                            want_lse=False)
    return (logp, ent) if with_entropy else logp


def chunk_logprobs(logits_chunk: torch.Tensor, labels_chunk: torch.Tensor) -> torch.Tensor:
    """Drop-in for ``TitanTrainer._chunk_logprobs`` (trainer.py:414-428)."""
    return logprobs_and_entropy(logits_chunk, labels_chunk)


@torch.no_grad()
def chunk_entropy(logits_chunk: torch.Tensor) -> torch.Tensor:
    """Drop-in for ``TitanTrainer._chunk_entropy`` (trainer.py:430-449), fp32 ``[rows, T]``."""
    logits, _ = _prep(logits_chunk, None)
    _, ent, _ = _fwd(logits, None, want_logp=False, want_entropy=True, want_lse=False)
    return ent


def logsumexp_rows(logits: torch.Tensor) -> torch.Tensor:
    """Per-row log-sum-exp of ``[rows, T, V]`` bf16 logits (what the backward consumes)."""
    logits, _ = _prep(logits, None)
    _, _, lse = _fwd(logits, None, want_logp=False, want_entropy=False, want_lse=True)
    return lse


__all__ = ["IGNORE_INDEX", "bwd_workspace", "chunk_entropy", "chunk_logprobs", "logprobs_and_entropy",
           "logsumexp_rows"]

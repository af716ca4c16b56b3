"""Oracle: the chunked logprob / entropy loop restated on CPU torch (test infrastructure).

Follows TitanTrainer._chunk_logprobs (trainer.py:414-428), _chunk_entropy
(trainer.py:430-449) and the chunk loop of _forward_logprobs
(trainer.py:508-522).  Math is the reference's: the bf16 logits are upcast to
fp32, logp = -cross_entropy(z, y), H = logsumexp(z) - sum(softmax(z) * z).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def chunk_logprobs(logits_chunk: torch.Tensor, labels_chunk: torch.Tensor,
                   dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """trainer.py:414-428.  ``dtype=torch.float64`` evaluates the same formula in
    double precision, for inputs where fp32's own rounding is the larger error."""
    B, T = labels_chunk.shape
    nll = F.cross_entropy(
        logits_chunk.to(dtype).reshape(B * T, -1), labels_chunk.reshape(B * T), reduction="none"
    ).view(B, T)
    return -nll


def chunk_entropy(logits_chunk: torch.Tensor, entropy_chunk_size: int = 512,
                  dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """trainer.py:430-449.  In fp32 the difference ``lse - sum(p * z)`` of two
    terms near a large common offset loses digits (about 1e-3 at an offset of
    120 over a 150k vocabulary); ``dtype=torch.float64`` gives the exact value."""
    out = []
    for s in range(0, logits_chunk.size(1), entropy_chunk_size):
        z = logits_chunk[:, s:s + entropy_chunk_size, :].to(dtype)
        lse = torch.logsumexp(z, dim=-1)
        out.append(lse - (torch.softmax(z, dim=-1) * z).sum(dim=-1))
    return torch.cat(out, dim=1)


def forward_logprobs(logits: torch.Tensor, labels: torch.Tensor, *, chunk: int = 1024,
                     with_entropy: bool = False, entropy_chunk_size: int = 512):
    """The chunk loop of trainer.py:505-527 (no-grad path), on given logits."""
    S = logits.size(1)
    chunk = chunk if S > chunk else S
    lps, ents = [], []
    for s in range(0, S, chunk):
        e = min(s + chunk, S)
        sl = logits[:, s:e, :]
        lps.append(chunk_logprobs(sl, labels[:, s:e]))
        if with_entropy:
            ents.append(chunk_entropy(sl, entropy_chunk_size))
    lp = torch.cat(lps, dim=1)
    if with_entropy:
        return lp, torch.cat(ents, dim=1)
    return lp


def logprob_entropy_f64(logits: torch.Tensor, labels: torch.Tensor):
    """Independent float64 evaluation used to pin the fp32 restatement."""
    z = logits.double()
    lse = torch.logsumexp(z, dim=-1)
    lp = z.gather(-1, labels.unsqueeze(-1).clamp(min=0)).squeeze(-1) - lse
    lp = torch.where(labels == -100, torch.zeros_like(lp), lp)
    p = torch.softmax(z, dim=-1)
    ent = -(p * torch.log_softmax(z, dim=-1)).sum(-1)
    return lp, ent, lse


def logprob_grad(logits: torch.Tensor, labels: torch.Tensor, grad_logp: torch.Tensor) -> torch.Tensor:
    """d/d logits of sum(grad_logp * logp) through the reference's fp32 path (autograd)."""
    z = logits.detach().float().requires_grad_(True)
    lp = chunk_logprobs(z, labels)
    (lp * grad_logp).sum().backward()
    return z.grad

"""Oracle: Student Top-K OPD kernels restated on CPU torch (test infrastructure).

Follows meshy/backend/titan/topk_loss.py: teacher_topk (20-32),
_chunk_gather_logprobs / gather_logprobs (35-57) and forward_kl_topk (60-80).
The logits are upcast to fp32 as in the reference.  teacher_topk breaks ties
between equal logits by ascending vocabulary index (a stable descending sort),
the order the HIP kernel guarantees; torch.topk leaves it unspecified.
"""

from __future__ import annotations

import torch


def teacher_topk(logits: torch.Tensor, k: int, *, chunk: int = 1024):
    """topk_loss.py:20-32: [rows, S, V] -> ids int64, log-probs fp32 [rows, S, k]."""
    ids, lps = [], []
    for s in range(0, logits.size(1), chunk):
        z = logits[:, s:s + chunk, :].float()
        vals, idx = torch.sort(z, dim=-1, descending=True, stable=True)
        ids.append(idx[..., :k])
        lps.append(vals[..., :k] - torch.logsumexp(z, dim=-1, keepdim=True))
    return torch.cat(ids, dim=1), torch.cat(lps, dim=1)


@torch.no_grad()
def teacher_topk_by_threshold(logits: torch.Tensor, k: int, *, chunk: int = 1024):
    """teacher_topk for rows without NaN, by one selection instead of a full
    sort, so that a 16384-row batch checks in seconds.  The k-th largest value
    tau of a row (torch.topk's values are exact whatever its tie order) admits
    every element >= tau; those candidates, taken in ascending index order,
    are sorted stably by value descending and the first k kept: the same ids
    as a stable descending sort of the whole row."""
    V = logits.size(-1)
    ids, lps = [], []
    for s in range(0, logits.size(1), chunk):
        z = logits[:, s:s + chunk, :].float()
        flat = z.reshape(-1, V)
        n = flat.size(0)
        tau = flat.topk(k, dim=-1).values[:, -1:]
        mask = flat >= tau
        cnt = mask.sum(-1)
        r, c = mask.nonzero(as_tuple=True)  # row-major: ascending index within a row
        pos = torch.arange(r.numel()) - (torch.cumsum(cnt, 0) - cnt)[r]
        width = int(cnt.max())
        vals = torch.full((n, width), float("-inf"))
        idx = torch.full((n, width), V, dtype=torch.int64)
        vals[r, pos] = flat[r, c]
        idx[r, pos] = c
        order = torch.sort(vals, dim=-1, descending=True, stable=True).indices[:, :k]
        top = idx.gather(-1, order).view(*z.shape[:-1], k)
        ids.append(top)
        lps.append(z.gather(-1, top) - torch.logsumexp(z, dim=-1, keepdim=True))
    return torch.cat(ids, dim=1), torch.cat(lps, dim=1)


@torch.no_grad()
def teacher_topk_reference_loop(logits: torch.Tensor, k: int, *, chunk: int = 1024):
    """The reference's own loop (topk_loss.py:24-32, torch.topk): the CPU baseline
    a benchmark times.  Its tie order is torch's, so parity checks use teacher_topk."""
    ids, lps = [], []
    for s in range(0, logits.size(1), chunk):
        z = logits[:, s:s + chunk, :].float()
        top = z.topk(k, dim=-1)
        ids.append(top.indices)
        lps.append(top.values - torch.logsumexp(z, dim=-1, keepdim=True))
    return torch.cat(ids, dim=1), torch.cat(lps, dim=1)


def gather_logprobs(logits: torch.Tensor, ids: torch.Tensor, *, chunk: int = 1024) -> torch.Tensor:
    """topk_loss.py:35-57 (no checkpointing: autograd through the plain ops)."""
    out = []
    for s in range(0, logits.size(1), chunk):
        z = logits[:, s:s + chunk, :].float()
        i = ids[:, s:s + chunk, :].long()
        out.append(z.gather(-1, i) - torch.logsumexp(z, dim=-1, keepdim=True))
    return torch.cat(out, dim=1)


def forward_kl_topk(student: torch.Tensor, teacher: torch.Tensor, *, log_prob_min_clamp=None,
                    loss_max_clamp=None) -> torch.Tensor:
    """topk_loss.py:60-80."""
    log_s = student.float()
    log_t = teacher.float()
    if log_prob_min_clamp is not None:
        log_s = log_s.clamp_min(log_prob_min_clamp)
        log_t = log_t.clamp_min(log_prob_min_clamp)
    kl = (log_t.exp() * (log_t - log_s)).sum(dim=-1)
    if loss_max_clamp is not None:
        kl = kl.clamp(min=-loss_max_clamp, max=loss_max_clamp)
    return kl

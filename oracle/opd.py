"""Oracle: Student Top-K distillation restated on CPU torch (test infrastructure).

Follows meshy/backend/titan/opd.py: layout_teacher_topk (58-89),
split_teacher_topk (92-110), the loss and sums of _distill_loss (153-197) and
_reduce_mini_metrics (234-251).
"""

from __future__ import annotations

import torch

from . import topk as otopk

TEACHER_FIELDS = ("teacher_topk_ids", "teacher_topk_logprobs")


def infer_top_k(samples, default: int = 1) -> int:
    """opd.py:39-44."""
    for td in samples:
        value = td.get(TEACHER_FIELDS[0], None)
        if value is not None:
            return int(value.shape[-1])
    return default


def _teacher_view(td, L: int):
    """opd.py:47-55."""
    ids, lps = td[TEACHER_FIELDS[0]], td[TEACHER_FIELDS[1]]
    if ids.shape[0] < L or lps.shape[0] < L:
        raise ValueError(
            f"teacher columns cover {int(ids.shape[0])} positions but the student "
            f"micro-batch needs {L}; the Teacher seq_len must be >= the Student's")
    return ids[:L].to(dtype=torch.long), lps[:L].to(dtype=torch.float32)


def layout_teacher_topk(samples, sample_idx, seq_len: int, doc_lens, *, layout: str):
    """opd.py:58-89 for the micro (sample_idx, seq_len, doc_lens)."""
    k = infer_top_k([samples[i] for i in sample_idx])
    if layout == "padded":
        rows = max(1, len(sample_idx))
        ids = torch.zeros(rows, seq_len, k, dtype=torch.long)
        lps = torch.zeros(rows, seq_len, k, dtype=torch.float32)
        for j, idx in enumerate(sample_idx):
            L = doc_lens[j]
            i, l = _teacher_view(samples[idx], L)
            ids[j, :L] = i
            lps[j, :L] = l
    elif layout == "packed":
        ids = torch.zeros(1, seq_len, k, dtype=torch.long)
        lps = torch.zeros(1, seq_len, k, dtype=torch.float32)
        off = 0
        for j, idx in enumerate(sample_idx):
            L = doc_lens[j]
            i, l = _teacher_view(samples[idx], L)
            ids[0, off:off + L] = i
            lps[0, off:off + L] = l
            off += L
    else:
        raise ValueError(f"unknown layout {layout!r}")
    return ids, lps


def split_teacher_topk(values, doc_lens, *, layout: str):
    """opd.py:92-110."""
    out = []
    if layout == "padded":
        for j, L in enumerate(doc_lens):
            out.append(values[j, :L])
    else:
        off = 0
        for L in doc_lens:
            out.append(values[0, off:off + L])
            off += L
    return out


def distill_loss(gathered, teacher_lps, mask, doc_ids, n_docs: int, *, rollout_lp=None, n_docs_global: int,
                 n_tokens_global: int, per_token_loss: bool, log_prob_min_clamp=-10.0, loss_max_clamp=10.0):
    """opd.py:161-197 from the [rows, S, K + 1] gather (K Teacher ids, then the label)."""
    k = teacher_lps.shape[-1]
    student_topk = gathered[..., :k]
    sampled_lp = gathered[..., k].detach()
    per_token = otopk.forward_kl_topk(student_topk, teacher_lps, log_prob_min_clamp=log_prob_min_clamp,
                                      loss_max_clamp=loss_max_clamp)
    per_token = per_token * mask
    n_slots = n_docs + 1
    flat_ids = doc_ids.reshape(-1)
    seg_sum = per_token.new_zeros(n_slots).index_add_(0, flat_ids, per_token.reshape(-1))
    seg_cnt = mask.new_zeros(n_slots).index_add_(0, flat_ids, mask.reshape(-1))
    if per_token_loss:
        loss = seg_sum[:n_docs].sum() / max(1, n_tokens_global)
    else:
        loss = (seg_sum[:n_docs] / seg_cnt[:n_docs].clamp(min=1)).sum() / max(1, n_docs_global)
    with torch.no_grad():
        sums = {
            "loss": loss.detach(),
            "token_count": mask.sum(),
            "student_mass_sum": (student_topk.detach().exp().sum(-1) * mask).sum(),
            "teacher_mass_sum": (teacher_lps.exp().sum(-1) * mask).sum(),
        }
        if rollout_lp is not None:
            lr = (rollout_lp - sampled_lp).clamp(-10.0, 10.0)
            k3 = lr.exp() - lr - 1.0
            sums["train_rollout_kl_sum"] = (torch.nan_to_num(k3) * mask).sum()
            sums["train_rollout_logdiff_abs_sum"] = (torch.nan_to_num((rollout_lp - sampled_lp).abs()) * mask).sum()
    return loss, sums


def reduce_distill_metrics(sums) -> dict:
    """opd.py:234-251 on one rank."""
    values = {k: float(v) for k, v in sums.items()}
    tokens = max(values["token_count"], 1.0)
    out = {
        "train/distill_loss": values["loss"],
        "train/student_topk_mass": values["student_mass_sum"] / tokens,
        "train/teacher_topk_mass": values["teacher_mass_sum"] / tokens,
    }
    if "train_rollout_kl_sum" in values:
        out["train_rollout_kl"] = values["train_rollout_kl_sum"] / tokens
        out["train_rollout_logdiff_abs"] = values["train_rollout_logdiff_abs_sum"] / tokens
    return out

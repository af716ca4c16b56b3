"""Oracle: the clipped PPO loss and its diagnostics restated on CPU torch
(test infrastructure).

Follows TitanTrainer._ppo_clip_loss (trainer.py:705-848) and
_reduce_mini_metrics (trainer.py:1020-1047) on one GPU (CP identity, no
loss-mesh all-reduce).  Inputs are plain tensors; gradients come from torch
autograd on ``new_lp``.
"""

from __future__ import annotations

import torch


def ppo_clip_loss(new_lp, old_lp, mask, doc_ids, advantages, n_docs, *, n_docs_global,
                  n_tokens_global, clip_low=0.2, clip_high=0.2, use_tis=False, use_icepop=False,
                  tis_min=0.5, tis_max=5.0, per_token_loss=False, positive_lm_coef=0.0,
                  positive_lm_weights=None, rollout_lp=None, train_lp_is_old=False,
                  entropy=None, cp_degree=1):
    n_slots = n_docs + 1
    log_ratio = new_lp - old_lp
    ratio = log_ratio.exp()
    adv = advantages
    adv_tok = torch.cat([adv, adv.new_zeros(1)])[doc_ids] if adv.dim() == 1 else adv
    pg_unclipped = ratio * adv_tok
    pg_clipped = torch.clamp(ratio, 1 - clip_low, 1 + clip_high) * adv_tok
    pg = -torch.min(pg_unclipped, pg_clipped)
    tis_ratio = ratio.detach()
    if use_icepop:
        tis_ratio = (old_lp - rollout_lp).detach().exp()
        tis_mask = (tis_ratio >= tis_min) & (tis_ratio <= tis_max)
        weight = torch.where(tis_mask, tis_ratio, 0)
        pg = torch.where(tis_mask, pg, 0) * weight
    elif use_tis:
        tis_mask = (ratio >= tis_min) & (ratio <= tis_max)
        pg = torch.where(tis_mask, pg, torch.zeros_like(pg))
    else:
        tis_mask = torch.ones_like(ratio, dtype=torch.bool)
    pg = pg * mask
    positive = torch.zeros_like(pg)
    if positive_lm_coef:
        weights = torch.cat([positive_lm_weights, new_lp.new_zeros(1)])[doc_ids]
        positive = -new_lp * weights * mask
    flat = doc_ids.reshape(-1)
    seg_sum = pg.new_zeros(n_slots).index_add_(0, flat, pg.reshape(-1))
    seg_cnt = mask.new_zeros(n_slots).index_add_(0, flat, mask.reshape(-1))
    n = n_docs
    if per_token_loss:
        loss = seg_sum[:n].sum() / max(1, n_tokens_global)
    else:
        loss = (seg_sum[:n] / seg_cnt[:n].clamp(min=1)).sum() / max(1, n_docs_global)
    pos_seg = positive.new_zeros(n_slots).index_add_(0, flat, positive.reshape(-1))
    if per_token_loss:
        pos_loss = pos_seg[:n].sum() / max(1, n_tokens_global)
    else:
        pos_loss = (pos_seg[:n] / seg_cnt[:n].clamp(min=1)).sum() / max(1, n_docs_global)
    pg_loss = loss
    loss = loss + positive_lm_coef * pos_loss
    with torch.no_grad():
        r = ratio.detach()
        lr = log_ratio.detach()
        sums = {
            "loss": pg_loss.detach(),
            "total_loss": loss.detach(),
            "positive_lm_loss": pos_loss.detach(),
            "tis_ratio_sum": (tis_ratio * mask).sum(),
            "ratio_sum": (r * mask).sum(),
            "clip_sum": (((r < 1 - clip_low) | (r > 1 + clip_high)).float() * mask).sum(),
            "tis_masked_sum": ((~tis_mask).float() * mask).sum(),
            "token_count": mask.sum(),
            "ppo_kl_sum": (-lr * mask).sum(),
            "log_ratio_abs_sum": (lr.abs() * mask).sum(),
        }
        seg_w = r.new_zeros(n_slots).index_add_(0, flat, (r * mask).reshape(-1))[:n]
        seg_w2 = r.new_zeros(n_slots).index_add_(0, flat, (r * r * mask).reshape(-1))[:n]
        cnt = seg_cnt[:n]
        ess = (seg_w * seg_w) / (cnt.clamp(min=1) * seg_w2.clamp(min=1e-8))
        sums["ess_sum"] = ess[cnt > 0].sum() / cp_degree
        sums["doc_count"] = (cnt > 0).float().sum() / cp_degree
        if rollout_lp is not None:
            train_lp = old_lp if train_lp_is_old else new_lp.detach()
            lr_rt = (rollout_lp - train_lp).clamp(-10.0, 10.0)
            k3 = lr_rt.exp() - lr_rt - 1.0
            sums["train_rollout_kl_sum"] = (torch.nan_to_num(k3) * mask).sum()
            sums["train_rollout_logdiff_abs_sum"] = (
                torch.nan_to_num((rollout_lp - train_lp).abs()) * mask
            ).sum()
        if entropy is not None:
            sums["entropy_sum"] = (entropy.float() * mask).sum()
    return loss, sums


def reduce_mini_metrics(sums):
    """trainer.py:1020-1047 without the loss-mesh all-reduce."""
    values = {k: float(v) for k, v in sums.items()}
    tokens = max(values["token_count"], 1.0)
    out = {
        "pg_loss": values["loss"],
        "ratio_mean": values["ratio_sum"] / tokens,
        "clip_frac": values["clip_sum"] / tokens,
        "tis_masked_frac": values["tis_masked_sum"] / tokens,
        "ppo_kl": values["ppo_kl_sum"] / tokens,
        "log_ratio_abs_mean": values["log_ratio_abs_sum"] / tokens,
        "ess_ratio": values["ess_sum"] / max(values.get("doc_count", 0.0), 1.0),
    }
    if "train_rollout_kl_sum" in values:
        out["train_rollout_kl"] = values["train_rollout_kl_sum"] / tokens
        out["train_rollout_logdiff_abs"] = values["train_rollout_logdiff_abs_sum"] / tokens
    if "entropy_sum" in values:
        out["entropy"] = values["entropy_sum"] / tokens
    if "tis_ratio_sum" in values:
        out["tis_ratio_mean"] = values["tis_ratio_sum"] / tokens
        out["positive_lm_loss"] = values["positive_lm_loss"]
        out["total_loss"] = values["total_loss"]
    return out

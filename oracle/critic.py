"""Oracle: critic-side reductions restated on CPU torch (test infrastructure).

Follows advantages_to_per_sequence (meshy/backend/titan/critic/gae.py:296-312),
Accumulator.update (meshy/backend/titan/critic/metrics.py:238-275),
clipped_value_error (meshy/backend/titan/vapo.py:35-41) and the window gauges
of metrics.py:58-217 and 278-328 (critic_diagnostics, diagnostics_from_states,
within_prompt_auc, prompt_pearson, variance_reduction, calibration_gap),
returned as plain dicts.
"""

from __future__ import annotations

import math

import torch


def advantages_to_per_sequence(adv, mask, doc_ids, n_docs: int):
    """gae.py:296-312."""
    flat_ids = doc_ids.reshape(-1)
    seg_sum = adv.new_zeros(n_docs + 1).index_add_(0, flat_ids, (adv * mask).reshape(-1))
    seg_cnt = mask.new_zeros(n_docs + 1).index_add_(0, flat_ids, mask.reshape(-1))
    return seg_sum[:n_docs] / seg_cnt[:n_docs].clamp(min=1)


class Accumulator:
    """metrics.py:238-275 (state as a plain dict)."""

    def __init__(self):
        self.state = dict(n_tokens=0.0, sum_r=0.0, sum_r2=0.0, sum_d=0.0, sum_d2=0.0, row_value=[], row_reward=[],
                          row_group=[])

    @torch.no_grad()
    def update(self, values, returns, mask, rewards, group_ids):
        s = self.state
        m = (mask > 0).float()
        v, r = values.float() * m, returns.float() * m
        d = v - r
        s["n_tokens"] += float(m.sum().item())
        s["sum_r"] += float(r.sum().item())
        s["sum_r2"] += float((r * r).sum().item())
        s["sum_d"] += float(d.sum().item())
        s["sum_d2"] += float((d * d).sum().item())
        row_value = v.sum(dim=1) / m.sum(dim=1).clamp(min=1.0)
        s["row_value"].extend(float(x) for x in row_value.tolist())
        s["row_reward"].extend(float(x) for x in rewards.float().tolist())
        s["row_group"].extend(int(x) for x in group_ids.tolist())


def clipped_value_error(values, targets, old_values, clip):
    """vapo.py:35-41."""
    error = (values.float() - targets.float()).square()
    if clip is None:
        return error
    old = old_values.detach().float()
    clipped = old + (values.float() - old).clamp(-clip, clip)
    return torch.maximum(error, (clipped - targets.float()).square())


def response_mean(values, mask):
    """metrics.py:58-62."""
    m = mask.float()
    return (values.float() * m).sum(dim=1) / m.sum(dim=1).clamp(min=1.0)


def prompt_pearson(row_value, row_reward, group_ids) -> float:
    """metrics.py:64-91: Pearson r of the groups' mean value and mean reward."""
    groups = torch.unique(group_ids)
    if groups.numel() < 2:
        return float("nan")
    v = torch.stack([row_value[group_ids == g].mean() for g in groups]).float()
    r = torch.stack([row_reward[group_ids == g].mean() for g in groups]).float()
    v_c, r_c = v - v.mean(), r - r.mean()
    denom = v_c.norm() * r_c.norm()
    if denom.item() == 0.0:
        return float("nan")
    return float((v_c @ r_c / denom).item())


def within_prompt_auc(row_value, row_correct, group_ids) -> float:
    """metrics.py:94-118: pooled (correct, incorrect) pairs within a group,
    ties 1/2; NaN without pairs."""
    wins = 0.0
    pairs = 0
    for g in torch.unique(group_ids):
        sel = group_ids == g
        v, c = row_value[sel].float(), row_correct[sel].bool()
        pos, neg = v[c], v[~c]
        if pos.numel() == 0 or neg.numel() == 0:
            continue
        diff = pos.unsqueeze(1) - neg.unsqueeze(0)
        wins += float((diff > 0).sum().item()) + 0.5 * float((diff == 0).sum().item())
        pairs += pos.numel() * neg.numel()
    return wins / pairs if pairs else float("nan")


def variance_reduction(values, returns, mask) -> float:
    """metrics.py:120-138: 1 - Var(r - v) / Var(r) over the selected tokens."""
    sel = mask.reshape(-1) > 0
    if int(sel.sum()) < 2:
        return float("nan")
    r = returns.reshape(-1)[sel].float()
    v = values.reshape(-1)[sel].float()
    var_r = r.var(unbiased=False)
    if var_r.item() == 0.0:
        return float("nan")
    return float((1.0 - (r - v).var(unbiased=False) / var_r).item())


def calibration_gap(values, returns, mask) -> float:
    """metrics.py:141-160."""
    m = mask.float()
    n = m.sum().clamp(min=1.0)
    return float((((values.float() - returns.float()) * m).sum() / n).item())


def critic_diagnostics(values, returns, mask, rewards, group_ids, correct_threshold=0.5) -> dict:
    """metrics.py:189-217."""
    m = mask.float()
    n_tok = m.sum().clamp(min=1.0)
    loss = float(((((values.float() - returns.float()) ** 2) * m).sum() / n_tok).item())
    row_value = response_mean(values, m)
    row_correct = rewards.float() >= correct_threshold
    return dict(
        value_loss=loss,
        critic_auc=within_prompt_auc(row_value, row_correct, group_ids),
        critic_var_ratio=variance_reduction(values, returns, m),
        critic_calibration_gap=calibration_gap(values, returns, m),
        prompt_pearson=prompt_pearson(row_value, rewards.float(), group_ids),
        n_rows=int(values.shape[0]),
        n_prompts=int(torch.unique(group_ids).numel()),
        n_tokens=int(m.sum().item()),
    )


def diagnostics_from_states(states, correct_threshold=0.5) -> dict:
    """metrics.py:278-328, states as the oracle Accumulator's dicts."""
    n = sum(s["n_tokens"] for s in states)
    if n <= 0:
        raise ValueError("cannot build diagnostics from states with no masked tokens")
    sum_r = sum(s["sum_r"] for s in states)
    sum_r2 = sum(s["sum_r2"] for s in states)
    sum_d = sum(s["sum_d"] for s in states)
    sum_d2 = sum(s["sum_d2"] for s in states)
    var_r = sum_r2 / n - (sum_r / n) ** 2
    var_d = sum_d2 / n - (sum_d / n) ** 2
    var_ratio = float("nan") if var_r == 0.0 or n < 2 else 1.0 - var_d / var_r
    row_value = torch.tensor([x for s in states for x in s["row_value"]], dtype=torch.float32)
    row_reward = torch.tensor([x for s in states for x in s["row_reward"]], dtype=torch.float32)
    group_ids = torch.tensor([x for s in states for x in s["row_group"]], dtype=torch.long)
    return dict(
        value_loss=sum_d2 / n,
        critic_auc=within_prompt_auc(row_value, row_reward >= correct_threshold, group_ids),
        critic_var_ratio=var_ratio,
        critic_calibration_gap=sum_d / n,
        prompt_pearson=prompt_pearson(row_value, row_reward, group_ids),
        n_rows=int(row_value.numel()),
        n_prompts=int(torch.unique(group_ids).numel()),
        n_tokens=int(n),
    )


def same_gauges(got: dict, want: dict, rel=1e-5, abs_=1e-6) -> bool:
    """Every gauge equal within the tolerance, NaN where the other is NaN."""
    for k, w in want.items():
        g = got[k]
        if isinstance(w, float) and math.isnan(w):
            if not (isinstance(g, float) and math.isnan(g)):
                return False
        elif abs(g - w) > abs_ + rel * abs(w):
            return False
    return True

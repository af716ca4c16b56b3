"""Oracle: critic-side reductions restated on CPU torch (test infrastructure).

Follows advantages_to_per_sequence (meshy/backend/titan/critic/gae.py:296-312),
Accumulator.update (meshy/backend/titan/critic/metrics.py:238-275) and
clipped_value_error (meshy/backend/titan/vapo.py:35-41).
"""

from __future__ import annotations

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

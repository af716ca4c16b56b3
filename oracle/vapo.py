"""Oracle: masked global whitening restated on CPU torch (test infrastructure).

Follows whiten_advantages (meshy/backend/titan/vapo.py:6-32) without the
distributed all-reduce (replication only divides the statistics).
"""

from __future__ import annotations

import torch

ADVANTAGE_TOKENS = "advantage_tokens"


def whiten_advantages(samples, seq_len, replication=1):
    stats = torch.zeros(3, dtype=torch.float64)
    entries = []
    for sample in samples:
        advantage = sample[ADVANTAGE_TOKENS]
        length = min(len(advantage), seq_len)
        mask = torch.zeros_like(advantage, dtype=torch.bool)
        if length > 1:
            mask[:length - 1] = sample["mask_assistant"][1:length].bool()
        selected = advantage[mask].double()
        stats += torch.stack((selected.sum(), selected.square().sum(),
                              selected.new_tensor(selected.numel())))
        entries.append((advantage, mask))
    stats /= replication
    total, squares, count = stats
    mean = total / count.clamp(min=1)
    variance = (squares / count.clamp(min=1) - mean.square()).clamp(min=0)
    if count >= 2:
        variance *= count / (count - 1)
    for advantage, mask in entries:
        advantage.copy_(torch.where(mask, (advantage - mean.to(advantage))
                                    * torch.rsqrt(variance.to(advantage) + 1e-8), 0))

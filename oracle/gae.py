"""Oracle: segment-aware GAE and returns restated on CPU torch (test infrastructure).

Follows meshy/backend/titan/critic/gae.py: _lambda_per_doc (70-74),
_continuation_mask (77-93), the sequential definition _reverse_scan_reference
(162-180), compute_returns (183-205) and compute_vapo_gae (208-293).  The
reference evaluates the same recursion through a float64 closed form where it
is representable (125-159); the oracle always runs the sequential definition,
which is what the closed form is checked against in the reference and what the
reference falls back to at gamma*lambda = 0.95.
"""

from __future__ import annotations

import torch


def lambda_per_doc(lengths, *, alpha, epsilon=1e-6):
    L = lengths.clamp(min=1).float()
    lam = 1.0 - 1.0 / (alpha * L)
    return lam.clamp(0.0, 1.0 - epsilon)


def continuation_mask(mask, doc_ids):
    rows, S = mask.shape
    valid = mask > 0
    same_doc = torch.zeros(rows, S, dtype=torch.bool)
    same_doc[:, :-1] = doc_ids[:, 1:] == doc_ids[:, :-1]
    next_valid = torch.zeros(rows, S, dtype=torch.bool)
    next_valid[:, :-1] = valid[:, 1:]
    return (valid & same_doc & next_valid).to(torch.float32)


def reverse_scan(x, decay, valid, cont):
    """The sequential recursion acc = x_t + decay_t * cont_t * acc (gae.py:162-180)."""
    rows, S = x.shape
    x = torch.where(valid, x, torch.zeros_like(x))
    out = torch.zeros_like(x)
    acc = torch.zeros(rows, dtype=x.dtype)
    for t in range(S - 1, -1, -1):
        acc = x[:, t] + decay[:, t] * cont[:, t] * acc
        out[:, t] = acc
    return torch.where(valid, out, torch.zeros_like(out))


def compute_returns(rewards, mask, doc_ids, *, gamma=1.0):
    rewards = rewards.float()
    cont = continuation_mask(mask, doc_ids)
    valid = mask > 0
    decay = torch.full_like(rewards, float(gamma))
    return reverse_scan(rewards, decay, valid, cont)


def compute_vapo_gae(rewards, values, mask, doc_ids, n_docs, *, lengths=None, gamma=1.0,
                     alpha=1.5, epsilon=1e-6):
    rows, S = rewards.shape
    values = values.float()
    rewards = rewards.float()
    flat = doc_ids.reshape(-1)
    if lengths is None:
        cnt = mask.new_zeros(n_docs + 1, dtype=torch.float32).index_add_(0, flat, mask.reshape(-1).float())
        lengths = cnt[:n_docs]
    lam_doc = torch.cat([lambda_per_doc(lengths, alpha=alpha, epsilon=epsilon), rewards.new_zeros(1)])
    lam = lam_doc[doc_ids]
    valid = mask > 0
    cont = continuation_mask(mask, doc_ids).to(values.dtype)
    shifted_v = torch.cat([values[:, 1:], values.new_zeros(rows, 1)], dim=1)
    delta = (rewards + gamma * shifted_v * cont - values) * valid.to(values.dtype)
    adv = reverse_scan(delta, gamma * lam, valid, cont)
    return adv, lam_doc[:n_docs]


def attach_gae_advantages(samples, *, seq_len, gamma=1.0, alpha=1.5, gae_lambda=None):
    """TitanTrainer._attach_gae_advantages (trainer.py:603-699): padded [rows, S]
    block on the next-token grid, one document per row.  Returns (per-sample
    advantages, metrics dict)."""
    if not samples:
        return [], {}
    rows = len(samples)
    widths = [min(int(len(td["tokens"])), seq_len) for td in samples]
    S = max(widths)
    mask = torch.zeros(rows, S)
    values = torch.zeros(rows, S)
    rewards = torch.zeros(rows, S)
    doc_ids = torch.arange(rows, dtype=torch.long).unsqueeze(1).expand(rows, S).contiguous()
    for j, td in enumerate(samples):
        L = widths[j]
        m = td["mask_assistant"][:L].to(torch.float32)
        v = td["values"][:L].to(torch.float32)
        if v.shape[0] != L:
            raise ValueError("critic and trainer disagree about the sequence")
        mask[j, :L - 1] = m[1:L]
        values[j, :L] = v
        response = (m > 0).nonzero()
        if response.numel() == 0:
            continue
        last = int(response[-1].item())
        if last == 0:
            continue
        rewards[j, last - 1] = float(td["reward"].reshape(-1)[0].item())
    if gae_lambda is None:
        lengths = None
    else:
        alpha = 1.0
        lengths = torch.full((rows,), 1.0 / max(1e-9, 1.0 - gae_lambda), dtype=torch.float32)
    adv, lam = compute_vapo_gae(rewards, values, mask, doc_ids, rows, gamma=gamma, alpha=alpha, lengths=lengths)
    per_sample = [adv[j, :widths[j]].clone() for j in range(rows)]
    counts = mask.sum(dim=1).clamp(min=1)
    per_seq = (adv * mask).sum(dim=1) / counts
    n_tokens = float(mask.sum())
    metrics = {
        "critic/value_mean": float((values * mask).sum() / max(1.0, n_tokens)),
        "critic/advantage_mean": float((adv * mask).sum() / max(1.0, n_tokens)),
        "critic/advantage_abs_mean": float((adv.abs() * mask).sum() / max(1.0, n_tokens)),
        "critic/advantage_seq_mean": float(per_seq.mean()),
        "critic/lambda_mean": float(lam.mean()),
    }
    return per_sample, metrics


def gae_brute_force(rewards, values, mask, doc_ids, lam_doc, gamma):
    """Independent O(S^2) evaluation of the GAE sum, for tiny inputs:
    A_t = sum_k (prod_{j<k} gamma*lam*cont_{t+j}) * delta_{t+k}, computed per
    position by walking forward along the run (no recursion)."""
    rows, S = rewards.shape
    out = torch.zeros(rows, S, dtype=torch.float64)
    for i in range(rows):
        for t in range(S):
            if not mask[i, t] > 0:
                continue
            total, w, k = 0.0, 1.0, t
            while True:
                d = int(doc_ids[i, k])
                c = (k + 1 < S and mask[i, k] > 0 and mask[i, k + 1] > 0
                     and int(doc_ids[i, k + 1]) == d)
                vn = float(values[i, k + 1]) if c else 0.0
                delta = float(rewards[i, k]) + gamma * vn - float(values[i, k])
                total += w * delta
                if not c:
                    break
                lam = float(lam_doc[d]) if d < len(lam_doc) else 0.0
                w *= gamma * lam
                k += 1
            out[i, t] = total
    return out

"""Oracle: micro-batch materialisation restated on CPU torch (test infrastructure).

Follows meshy/backend/titan/batch.py:84-243 for one micro.  Returns a plain
dict of CPU tensors (no device copy, no CP sharding: identity on one GPU).
"""

from __future__ import annotations

import torch

ADVANTAGE_TOKENS = "advantage_tokens"


def _shift(x: torch.Tensor) -> torch.Tensor:
    # batch.py:91-93: x[1:] ++ [0]
    return torch.cat([x[1:], x.new_zeros(1)])


def build_micro_batch(samples, sample_idx, seq_len, doc_lens, *, layout, need_rollout_lp):
    n_docs = len(sample_idx)
    lengths = torch.tensor(doc_lens, dtype=torch.int32)
    per_token_adv = n_docs > 0 and ADVANTAGE_TOKENS in samples[sample_idx[0]]
    advantages = None
    if not per_token_adv:
        advantages = torch.tensor(
            [float(samples[i].get("advantage", 0.0)) for i in sample_idx], dtype=torch.float32
        )
    cu = None
    max_len = None
    if layout == "padded":  # batch.py:118-141
        rows, S = max(1, n_docs), seq_len
        input_ids = torch.zeros(rows, S, dtype=torch.long)
        labels = torch.zeros(rows, S, dtype=torch.long)
        mask = torch.zeros(rows, S, dtype=torch.float32)
        doc_ids = torch.arange(rows, dtype=torch.long).unsqueeze(1).expand(rows, S).clone()
        rollout_lp = torch.zeros(rows, S) if need_rollout_lp else None
        adv_tok = torch.zeros(rows, S) if per_token_adv else None
        for j, idx in enumerate(sample_idx):
            L = doc_lens[j]
            td = samples[idx]
            tok = td["tokens"][:L].to(torch.long)
            input_ids[j, :L] = tok
            labels[j, :L] = _shift(tok)
            mask[j, :L] = _shift(td["mask_assistant"][:L].to(torch.float32))
            if rollout_lp is not None:
                rollout_lp[j, :L] = _shift(td["logprobs"][:L].to(torch.float32))
            if adv_tok is not None:
                adv_tok[j, :L] = td[ADVANTAGE_TOKENS][:L].to(torch.float32)
        if n_docs == 0:
            doc_ids.fill_(0)
        positions = torch.arange(S, dtype=torch.int32).unsqueeze(0).expand(rows, S).contiguous()
    else:  # batch.py:142-178
        T = seq_len
        used = sum(doc_lens)
        pad = T - used
        assert pad >= 0
        input_ids = torch.zeros(1, T, dtype=torch.long)
        labels = torch.zeros(1, T, dtype=torch.long)
        mask = torch.zeros(1, T, dtype=torch.float32)
        doc_ids = torch.full((1, T), n_docs, dtype=torch.long)
        positions = torch.zeros(1, T, dtype=torch.int32)
        rollout_lp = torch.zeros(1, T) if need_rollout_lp else None
        adv_tok = torch.zeros(1, T) if per_token_adv else None
        cu = [0]
        off = 0
        for j, idx in enumerate(sample_idx):
            L = doc_lens[j]
            td = samples[idx]
            tok = td["tokens"][:L].to(torch.long)
            input_ids[0, off:off + L] = tok
            labels[0, off:off + L] = _shift(tok)
            mask[0, off:off + L] = _shift(td["mask_assistant"][:L].to(torch.float32))
            doc_ids[0, off:off + L] = j
            positions[0, off:off + L] = torch.arange(L, dtype=torch.int32)
            if rollout_lp is not None:
                rollout_lp[0, off:off + L] = _shift(td["logprobs"][:L].to(torch.float32))
            if adv_tok is not None:
                adv_tok[0, off:off + L] = td[ADVANTAGE_TOKENS][:L].to(torch.float32)
            off += L
            cu.append(off)
        lens = list(doc_lens)
        if pad > 0:
            positions[0, off:] = torch.arange(pad, dtype=torch.int32)
            cu.append(T)
            lens.append(pad)
        cu = torch.tensor(cu, dtype=torch.int32)
        max_len = max(lens)
    positive = torch.tensor(
        [float(samples[i].get("positive_lm_weight", 0.0)) if float(samples[i].get("reward", 0.0)) > 0.5
         else 0.0 for i in sample_idx],
        dtype=torch.float32,
    )
    return {
        "input_ids": input_ids,
        "labels": labels,
        "positions": positions,
        "mask": mask,
        "doc_ids": doc_ids,
        "advantages": adv_tok if per_token_adv else advantages,
        "rollout_logprobs": rollout_lp,
        "lengths": lengths,
        "n_docs": n_docs,
        "cu_seqlens": cu,
        "max_seqlen": max_len,
        "positive_lm_weights": positive,
    }

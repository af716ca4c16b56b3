"""Oracle: the reference planner restated in plain Python (test infrastructure).

Follows meshy/backend/titan/plan.py:141-288.  Returns plain tuples instead of
the dataclasses so the oracle shares no code with the product:

    (local_indices, per_rank) where per_rank[r][i] =
        (micros, n_docs_global, n_tokens_global, tokens_per_rank) and
        micros = ((sample_idx, seq_len, doc_lens), ...)
"""

from __future__ import annotations


def round_up(x: int, align: int) -> int:
    # plan.py:141-142
    return ((x + align - 1) // align) * align


def snake(order, n_bins):
    # plan.py:145-155: boustrophedon deal, bins 0..n-1 then n-1..0, ...
    bins = [[] for _ in range(n_bins)]
    for k, idx in enumerate(order):
        rnd, pos = divmod(k, n_bins)
        bins[pos if rnd % 2 == 0 else n_bins - 1 - pos].append(idx)
    return bins


def pack_micros(local_pos, lengths, layout, align, budget, micro_batch_size):
    """First-fit-decreasing (plan.py:158-203)."""
    order = sorted(local_pos, key=lambda p: (-lengths[p], p))
    max_rows = micro_batch_size if budget is None else None
    micros = []  # [positions, doc_lens, row_len_or_total]
    for p in order:
        L = lengths[p]
        placed = False
        for m in micros:
            if max_rows is not None and len(m[0]) >= max_rows:
                continue
            if budget is not None:
                cost = (len(m[0]) + 1) * m[2] if layout == "padded" else round_up(m[2] + L, align)
                if cost > budget:
                    continue
            m[0].append(p)
            m[1].append(L)
            if layout == "packed":
                m[2] += L
            placed = True
            break
        if not placed:
            micros.append([[p], [L], round_up(L, align) if layout == "padded" else L])
    return [
        (tuple(pos), total if layout == "padded" else round_up(total, align), tuple(lens))
        for pos, lens, total in micros
    ]


def build_plan(lengths, loss_tokens, dp_size, *, layout, mini_batch_size, seq_len, align,
               max_tokens_per_micro=None, micro_batch_size=None):
    """plan.py:211-288."""
    n = len(lengths)
    if n == 0:
        raise ValueError("cannot plan an empty batch")
    if dp_size <= 0 or n % dp_size != 0:
        raise ValueError(f"batch size {n} is not divisible by DP size {dp_size}")
    trunc = [min(int(L), seq_len) for L in lengths]
    order = sorted(range(n), key=lambda i: (-trunc[i], i))
    rank_samples = snake(order, dp_size)
    n_local = n // dp_size
    n_mini = (n_local + mini_batch_size - 1) // mini_batch_size
    minis_of, members_of = [], []
    for r in range(dp_size):
        local = rank_samples[r]
        local_len = [trunc[g] for g in local]
        local_order = sorted(range(n_local), key=lambda p: (-local_len[p], p))
        members = snake(local_order, n_mini)
        members_of.append(members)
        minis_of.append([
            pack_micros(m, local_len, layout, align, max_tokens_per_micro, micro_batch_size)
            for m in members
        ])
    per_rank = []
    for r in range(dp_size):
        minis = []
        for i in range(n_mini):
            n_micro = max(len(minis_of[q][i]) for q in range(dp_size))
            micros = list(minis_of[r][i]) + [((), align, ())] * (n_micro - len(minis_of[r][i]))
            n_docs_global = sum(len(members_of[q][i]) for q in range(dp_size))
            n_tokens_global = 0
            tokens_per_rank = []
            for q in range(dp_size):
                globals_q = [rank_samples[q][p] for p in members_of[q][i]]
                n_tokens_global += sum(int(loss_tokens[g]) for g in globals_q)
                tokens_per_rank.append(sum(trunc[g] for g in globals_q))
            minis.append((tuple(micros), n_docs_global, n_tokens_global, tuple(tokens_per_rank)))
        per_rank.append(tuple(minis))
    return tuple(tuple(s) for s in rank_samples), tuple(per_rank)


def sample_lengths(samples, seq_len):
    """trainer.py:577-588: (token count, loss tokens after shift + truncation)."""
    lengths, loss_tokens = [], []
    for td in samples:
        n = int(len(td["tokens"]))
        L = min(n, seq_len)
        lengths.append(n)
        mask = td["mask_assistant"]
        loss_tokens.append(int((mask[1:L] > 0).sum().item()) if L > 1 else 0)
    return lengths, loss_tokens

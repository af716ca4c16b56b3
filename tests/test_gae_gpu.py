"""Segment-aware GAE, returns and whitening on the GPU against the oracle (the
reference's sequential recursion, critic/gae.py:162-180, and vapo.py:6-32).
Tolerance: 1e-3 absolute on fp32 advantages and returns."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gae as ogae
from oracle import vapo as ovapo

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _random_grid(rows, S, n_docs_per_row, seed, hole_p=0.05):
    g = torch.Generator().manual_seed(seed)
    doc_ids = torch.zeros(rows, S, dtype=torch.long)
    mask = torch.zeros(rows, S)
    next_id = 0
    for r in range(rows):
        cuts = sorted(torch.randint(1, S, (n_docs_per_row - 1,), generator=g).tolist())
        bounds = [0] + cuts + [S]
        for a, b in zip(bounds[:-1], bounds[1:]):
            doc_ids[r, a:b] = next_id
            p = int(torch.randint(0, max(1, (b - a) // 3 + 1), (1,), generator=g))
            mask[r, a + p:b] = 1.0
            next_id += 1
    holes = torch.rand(rows, S, generator=g) < hole_p
    mask[holes] = 0.0
    values = torch.randn(rows, S, generator=g)
    rewards = torch.zeros(rows, S)
    rewards[torch.rand(rows, S, generator=g) < 0.02] = 1.0
    return rewards, values, mask, doc_ids, next_id


@pytest.mark.parametrize("gamma,alpha,const_lam", [(1.0, 1.5, None), (0.99, 0.5, None), (1.0, 1.0, 0.95),
                                                   (0.9, 1.0, 0.0)])
def test_matches_sequential_oracle(dev, gamma, alpha, const_lam):
    from meshy_amd.gae import compute_returns, compute_vapo_gae, gae_and_returns

    rewards, values, mask, doc_ids, n_docs = _random_grid(5, 3000, 4, seed=int(gamma * 100))
    n_docs_total = n_docs
    lengths = None
    if const_lam is not None:
        lengths = torch.full((n_docs_total,), 1.0 / max(1e-9, 1.0 - const_lam))
    ref_adv, ref_lam = ogae.compute_vapo_gae(rewards, values, mask, doc_ids, n_docs_total, lengths=lengths,
                                             gamma=gamma, alpha=alpha)
    ref_ret = ogae.compute_returns(rewards, mask, doc_ids, gamma=gamma)
    d = [t.to(dev) for t in (rewards, values, mask, doc_ids)]
    adv, lam = compute_vapo_gae(*d, n_docs_total, lengths=None if lengths is None else lengths.to(dev),
                                gamma=gamma, alpha=alpha)
    ret = compute_returns(d[0], d[2], d[3], gamma=gamma)
    assert (adv.cpu() - ref_adv).abs().max().item() <= TOL
    assert (ret.cpu() - ref_ret).abs().max().item() <= TOL
    assert (lam.cpu() - ref_lam).abs().max().item() <= 1e-6
    a2, r2, l2 = gae_and_returns(*d, n_docs_total, lengths=None if lengths is None else lengths.to(dev),
                                 gamma=gamma, alpha=alpha)
    assert torch.equal(a2, adv) and torch.equal(r2, ret) and torch.equal(l2, lam)


def test_packed_with_padding_slot_and_bf16_values(dev):
    from meshy_amd.gae import compute_vapo_gae

    g = torch.Generator().manual_seed(2)
    lens = [5, 1, 300, 77, 4096 * 2 + 5]
    pad = 40
    T = sum(lens) + pad
    doc_ids = torch.cat([torch.full((L,), j) for j, L in enumerate(lens)] + [torch.full((pad,), len(lens))])
    mask = torch.ones(T)
    mask[doc_ids == len(lens)] = 0
    mask[torch.rand(T, generator=g) < 0.01] = 0
    values = torch.randn(T, generator=g).to(torch.bfloat16)
    rewards = torch.randn(T, generator=g)
    args = [x.reshape(1, -1) for x in (rewards, values, mask, doc_ids)]
    ref_adv, ref_lam = ogae.compute_vapo_gae(*args, len(lens), gamma=1.0, alpha=1.5)
    adv, lam = compute_vapo_gae(*[a.to(dev) for a in args], len(lens), gamma=1.0, alpha=1.5)
    assert (adv.cpu() - ref_adv).abs().max().item() <= TOL
    assert (lam.cpu() - ref_lam).abs().max().item() <= 1e-6


def test_closed_form_terminal_reward(dev):
    """V = 0, one terminal reward R, constant lambda, gamma = 1: A_t = lambda^(T-1-t) R,
    returns = R on the whole run (gae.py:196-199)."""
    from meshy_amd.gae import compute_returns, compute_vapo_gae

    S, R, lam = 5000, 0.75, 0.95
    mask = torch.ones(1, S)
    rewards = torch.zeros(1, S)
    rewards[0, -1] = R
    values = torch.zeros(1, S)
    doc_ids = torch.zeros(1, S, dtype=torch.long)
    lengths = torch.full((1,), 1.0 / (1.0 - lam))
    adv, _ = compute_vapo_gae(rewards.to(dev), values.to(dev), mask.to(dev), doc_ids.to(dev), 1,
                              lengths=lengths.to(dev), gamma=1.0, alpha=1.0)
    lam_f = float(1.0 - 1.0 / (1.0 * float(lengths[0])))
    expect = torch.tensor([lam_f ** (S - 1 - t) * R for t in range(S)], dtype=torch.float64)
    assert (adv[0].cpu().double() - expect).abs().max().item() <= 1e-5
    ret = compute_returns(rewards.to(dev), mask.to(dev), doc_ids.to(dev), gamma=1.0)
    assert torch.allclose(ret.cpu(), torch.full((1, S), R))


def test_gae_1024_docs_full_size(dev):
    """1024 docs (~5.9M tokens), values bf16, gamma 1, lambda 0.95 (lengths trick),
    packed [1, T] on the GPU against the sequential loop on padded [1024, S_max] rows."""
    from meshy_amd import workloads
    from meshy_amd.gae import gae_and_returns

    batch, values, terminal = workloads.gae_1024_docs(4)
    n = len(batch.lengths)
    L = batch.lengths
    S_max = int(L.max())
    doc_ids_flat = np.repeat(np.arange(n), L)
    pos = np.arange(batch.total) - np.repeat(batch.offsets[:-1], L)
    mask_flat = batch.mask
    rewards_flat = np.zeros(batch.total, np.float32)
    last = batch.offsets[1:] - 1
    rewards_flat[last] = terminal
    v_bf16 = torch.from_numpy(values).to(torch.bfloat16)
    lengths = torch.full((n,), 1.0 / (1.0 - 0.95))
    adv, ret, lam = gae_and_returns(
        torch.from_numpy(rewards_flat).reshape(1, -1).to(dev), v_bf16.reshape(1, -1).to(dev),
        torch.from_numpy(mask_flat).reshape(1, -1).to(dev),
        torch.from_numpy(doc_ids_flat).reshape(1, -1).to(dev), n, lengths=lengths.to(dev), gamma=1.0, alpha=1.0)
    # the same data as padded rows for the sequential oracle
    R = torch.zeros(n, S_max)
    Vp = torch.zeros(n, S_max)
    M = torch.zeros(n, S_max)
    R[doc_ids_flat, pos] = torch.from_numpy(rewards_flat)
    Vp[doc_ids_flat, pos] = v_bf16.float()
    M[doc_ids_flat, pos] = torch.from_numpy(mask_flat)
    ids = torch.arange(n).unsqueeze(1).expand(n, S_max).contiguous()
    ref_adv, _ = ogae.compute_vapo_gae(R, Vp, M, ids, n, lengths=lengths, gamma=1.0, alpha=1.0)
    ref_ret = ogae.compute_returns(R, M, ids, gamma=1.0)
    got_adv = torch.zeros(n, S_max)
    got_ret = torch.zeros(n, S_max)
    got_adv[doc_ids_flat, pos] = adv.reshape(-1).cpu()
    got_ret[doc_ids_flat, pos] = ret.reshape(-1).cpu()
    assert (got_adv - ref_adv).abs().max().item() <= TOL
    assert (got_ret - ref_ret).abs().max().item() <= TOL


def _run_suffix_sums(r, valid, doc):
    """Suffix sums of r over each maximal run of valid positions of one document."""
    n = len(r)
    cont = np.zeros(n, bool)
    cont[:-1] = valid[:-1] & valid[1:] & (doc[:-1] == doc[1:])
    rv = np.where(valid, r, 0).astype(np.int64)
    run_end = np.zeros(n, np.int64)  # index of the last position of t's run
    ends = np.flatnonzero(~cont)
    run_end[:] = ends[np.searchsorted(ends, np.arange(n))]
    suffix = np.concatenate([np.cumsum(rv[::-1])[::-1], [0]])
    return suffix[np.arange(n)] - suffix[run_end + 1]


@pytest.mark.parametrize("holes", [True, False])
@pytest.mark.parametrize("n", [4096 * 64, 4096 * 64 + 1, 4096 * 129 + 17, 4096 * 64 * 65 + 3])
def test_exact_carry_across_chunks(dev, n, holes):
    """gamma = lambda = 1 with integer rewards and values: G_t is the suffix sum of r
    over t's run of valid tokens and A_t = G_t - V_t (the deltas telescope), all
    exact in fp32, so every carry (between threads, workgroups and the chunks
    to the right up to the first cut) is checked bit for bit, on up to 17M
    tokens.  Without mask holes the documents (~300 k tokens, 128 chunks for
    the shortest n) run past 64 chunks of 2048 tokens, so the carry of most
    chunks folds more than one batch of 64 chunk maps."""
    from meshy_amd.gae import gae_and_returns

    rng = np.random.default_rng(n)
    n_docs = max(1, n // 300_000)
    cuts = np.sort(rng.choice(np.arange(1, n), n_docs - 1, replace=False)) if n_docs > 1 else np.array([], int)
    doc = np.zeros(n, np.int64)
    doc[cuts] = 1
    doc = np.cumsum(doc)
    valid = rng.random(n) > 1e-4 if holes else np.ones(n, bool)
    r = (rng.random(n) < 0.05).astype(np.float32)
    v = rng.integers(-8, 9, n).astype(np.float32)
    G = _run_suffix_sums(r, valid, doc).astype(np.float32)
    A = np.where(valid, G - v, 0).astype(np.float32)
    lengths = torch.full((n_docs,), 1e30, device=dev)
    adv, ret, lam = gae_and_returns(
        torch.from_numpy(r).reshape(1, -1).to(dev), torch.from_numpy(v).to(torch.bfloat16).reshape(1, -1).to(dev),
        torch.from_numpy(valid.astype(np.float32)).reshape(1, -1).to(dev),
        torch.from_numpy(doc).reshape(1, -1).to(dev), n_docs, lengths=lengths, gamma=1.0, alpha=1.0, epsilon=0.0)
    assert torch.equal(lam.cpu(), torch.ones(n_docs))
    assert np.array_equal(ret.reshape(-1).cpu().numpy(), G)
    assert np.array_equal(adv.reshape(-1).cpu().numpy(), A)


@pytest.mark.parametrize("holes", [True, False])
def test_waits_given_up_leave_the_call_to_the_exact_fix_pass(dev, holes):
    """With a poll limit of 0 the one-pass kernel gives up every wait for a
    neighbouring chunk's map that is not published at its first poll, and the
    fix-up pass redoes the call's outputs from the published maps: the same
    exact values on the integer case above (documents of ~300 k tokens, so
    carries fold several batches of maps), and the oracle's values within
    the tolerance on a random grid."""
    from meshy_amd import _lib
    from meshy_amd.gae import compute_vapo_gae, gae_and_returns

    n = 4096 * 129 + 17
    rng = np.random.default_rng(3)
    n_docs = 2
    doc = np.zeros(n, np.int64)
    doc[n // 3:] = 1
    valid = rng.random(n) > 1e-4 if holes else np.ones(n, bool)
    r = (rng.random(n) < 0.05).astype(np.float32)
    v = rng.integers(-8, 9, n).astype(np.float32)
    G = _run_suffix_sums(r, valid, doc).astype(np.float32)
    A = np.where(valid, G - v, 0).astype(np.float32)
    rewards, values, mask, doc_ids, n_grid = _random_grid(3, 60_000, 20, seed=9)
    ref_adv, _ = ogae.compute_vapo_gae(rewards, values, mask, doc_ids, n_grid, gamma=0.99, alpha=1.5)
    lib = _lib.load()
    before = lib.meshy_gae_set_poll_limit(0)
    try:
        adv, ret, _ = gae_and_returns(
            torch.from_numpy(r).reshape(1, -1).to(dev), torch.from_numpy(v).to(torch.bfloat16).reshape(1, -1).to(dev),
            torch.from_numpy(valid.astype(np.float32)).reshape(1, -1).to(dev),
            torch.from_numpy(doc).reshape(1, -1).to(dev), n_docs, lengths=torch.full((n_docs,), 1e30, device=dev),
            gamma=1.0, alpha=1.0, epsilon=0.0)
        got, _ = compute_vapo_gae(*[t.to(dev) for t in (rewards, values, mask, doc_ids)], n_grid, gamma=0.99,
                                  alpha=1.5)
        torch.cuda.synchronize()
    finally:
        assert lib.meshy_gae_set_poll_limit(-1) == 0
    assert before == 2000
    assert np.array_equal(ret.reshape(-1).cpu().numpy(), G)
    assert np.array_equal(adv.reshape(-1).cpu().numpy(), A)
    assert (got.cpu() - ref_adv).abs().max().item() <= TOL


def test_lambda_zero_is_not_a_cut_for_the_returns(dev):
    """lambda = 0 zeroes the advantage scan's slope at every position while the
    returns scan still carries (gamma = 1): a chunk with only the advantage
    slope at 0 must not stop the returns' carry.  One 600 k-token document
    without holes, integer rewards: G_t is the exact suffix sum and A_t the
    exact one-step delta r_t + V_{t+1} - V_t (0 after the last token)."""
    from meshy_amd.gae import gae_and_returns

    n = 600_000
    rng = np.random.default_rng(5)
    r = (rng.random(n) < 0.05).astype(np.float32)
    v = rng.integers(-8, 9, n).astype(np.float32)
    G = np.cumsum(r[::-1])[::-1].astype(np.float32)
    A = (r + np.append(v[1:], 0) - v).astype(np.float32)
    lengths = torch.ones(1, device=dev)  # lambda = clamp(1 - 1 / (1 * 1), 0, .) = 0
    adv, ret, lam = gae_and_returns(
        torch.from_numpy(r).reshape(1, -1).to(dev), torch.from_numpy(v).to(torch.bfloat16).reshape(1, -1).to(dev),
        torch.ones(1, n, device=dev), torch.zeros(1, n, dtype=torch.long, device=dev), 1, lengths=lengths,
        gamma=1.0, alpha=1.0, epsilon=0.0)
    assert lam.item() == 0.0
    assert np.array_equal(ret.reshape(-1).cpu().numpy(), G)
    assert np.array_equal(adv.reshape(-1).cpu().numpy(), A)


def test_scan_is_deterministic(dev):
    """Two calls on the same inputs give bitwise equal results: every fold has a
    fixed order, whichever workgroup finishes first."""
    from meshy_amd.gae import gae_and_returns

    g = torch.Generator().manual_seed(11)
    n = 4096 * 300 + 5
    doc = torch.cumsum((torch.rand(n, generator=g) < 1e-4).long(), 0)
    n_docs = int(doc[-1]) + 1
    args = [torch.randn(n, generator=g), torch.randn(n, generator=g),
            (torch.rand(n, generator=g) > 0.01).float(), doc]
    d = [a.reshape(1, -1).to(dev) for a in args]
    first = gae_and_returns(*d, n_docs, gamma=0.999, alpha=1.5)
    for _ in range(3):
        again = gae_and_returns(*d, n_docs, gamma=0.999, alpha=1.5)
        assert all(torch.equal(a, b) for a, b in zip(first, again))


def test_fractional_mask_without_lengths_is_deterministic(dev):
    """A fractional mask and no lengths: the masked document lengths (and so
    lambda and the advantages) come from fixed-order sums over each
    document's offsets range, the same bits on every call, and match the
    oracle's index_add lengths (gae.py:264-269)."""
    from meshy_amd.gae import gae_and_returns

    rewards, values, mask, doc_ids, n_docs = _random_grid(4, 9000, 5, seed=21)
    g = torch.Generator().manual_seed(22)
    mask = mask * (torch.rand(mask.shape, generator=g) * 0.9 + 0.1)
    d = [t.to(dev) for t in (rewards, values, mask, doc_ids)]
    first = gae_and_returns(*d, n_docs, gamma=0.99, alpha=1.5)
    for _ in range(4):
        again = gae_and_returns(*d, n_docs, gamma=0.99, alpha=1.5)
        assert all(torch.equal(a, b) for a, b in zip(first, again))
    ref_adv, ref_lam = ogae.compute_vapo_gae(rewards, values, mask, doc_ids, n_docs, gamma=0.99, alpha=1.5)
    assert (first[0].cpu() - ref_adv).abs().max().item() <= TOL
    assert (first[2].cpu() - ref_lam).abs().max().item() <= 1e-6


@pytest.mark.parametrize("docs_per_row", [3, 40, 700])
def test_offsets_and_atomic_counts_agree(dev, docs_per_row):
    """0/1 masks without lengths: the per-document counts from the segment
    offsets (fixed order) and from the atomic path are the same integers, so
    bitwise equal lambdas, advantages and returns; empty document slots
    included."""
    from meshy_amd import gae

    rewards, values, mask, doc_ids, n_docs = _random_grid(3, 12000, docs_per_row, seed=docs_per_row)
    doc_ids = doc_ids * 2  # every other slot empty
    n_docs = 2 * n_docs
    d = [t.to(dev) for t in (rewards, values, mask, doc_ids)]
    kw = dict(lengths=None, gamma=0.98, alpha=1.5, epsilon=1e-6, want_adv=True, want_returns=True, want_lam=True)
    a0, r0, l0 = gae._run(*d, n_docs, offsets=True, **kw)
    a1, r1, l1 = gae._run(*d, n_docs, offsets=False, **kw)
    assert torch.equal(a0, a1) and torch.equal(r0, r1) and torch.equal(l0, l1)
    ref_adv, ref_lam = ogae.compute_vapo_gae(rewards, values, mask, doc_ids, n_docs, gamma=0.98, alpha=1.5)
    assert (a0.cpu() - ref_adv).abs().max().item() <= TOL
    assert (l0.cpu() - ref_lam).abs().max().item() <= 1e-6


@pytest.mark.parametrize("docs_per_row,rows,S", [(2, 4, 9000), (12, 3, 12000), (20, 2, 12000), (3, 1, 70000)])
def test_scan_from_offsets_equals_scan_from_ids(dev, docs_per_row, rows, S):
    """With offsets the scan reads the ids only at chunk ends and takes the
    document starts between them from the offsets (chunks with up to four
    starts) or reads every id (more): the same ids either way, so advantages,
    returns and lambdas are bitwise equal to the per-token-id scan.  Doc sizes
    put chunks on both sides of the four-start limit; a padding slot ends the
    grid; bf16 and fp32 values; with and without lengths."""
    from meshy_amd import gae

    rewards, values, mask, doc_ids, n_docs = _random_grid(rows, S, docs_per_row, seed=S + docs_per_row)
    doc_ids[-1, -37:] = n_docs  # the padding slot
    mask[-1, -37:] = 0.0
    lengths = torch.rand(n_docs, generator=torch.Generator().manual_seed(1)) * 900 + 1
    for vals in (values, values.to(torch.bfloat16)):
        d = [t.to(dev) for t in (rewards, vals, mask, doc_ids)]
        for lens in (None, lengths.to(dev)):
            kw = dict(lengths=lens, gamma=0.97, alpha=1.5, epsilon=1e-6, want_adv=True, want_returns=True,
                      want_lam=True)
            a0, r0, l0 = gae._run(*d, n_docs, offsets=True, **kw)
            a1, r1, l1 = gae._run(*d, n_docs, offsets=False, **kw)
            assert torch.equal(a0, a1) and torch.equal(r0, r1) and torch.equal(l0, l1)
    ref_adv, _ = ogae.compute_vapo_gae(rewards, values, mask, doc_ids, n_docs, lengths=lengths, gamma=0.97,
                                       alpha=1.5)
    a, _, _ = gae._run(*[t.to(dev) for t in (rewards, values, mask, doc_ids)], n_docs, lengths=lengths.to(dev),
                       gamma=0.97, alpha=1.5, epsilon=1e-6, want_adv=True, want_returns=False, want_lam=False)
    assert (a.cpu() - ref_adv).abs().max().item() <= TOL


def test_scan_from_offsets_with_ids_outside_the_slots(dev, monkeypatch):
    """Sorted ids that start below 0 and end past the padding slot.  The
    public call raises ValueError, as the reference's indexing does.  Handed
    unchecked offsets through the C ABI, the kernels stay in bounds: chunks
    whose end ids leave [0, n_docs] read every id, so both scans agree bit for
    bit (ids outside the slots get lambda 0, as in the per-token scan)."""
    from meshy_amd import gae
    from meshy_amd.loss import segment_offsets

    rewards, values, mask, doc_ids, n_docs = _random_grid(1, 20000, 12, seed=77)
    doc_ids[0, :3000] = -1
    doc_ids[0, -2500:] = n_docs + 3
    d = [t.to(dev) for t in (rewards, values, mask, doc_ids)]
    with pytest.raises(ValueError, match="doc_ids must lie"):
        gae.compute_vapo_gae(d[0], d[1], d[2], d[3], n_docs)
    monkeypatch.setattr(gae, "_doc_offsets", lambda ids, n: segment_offsets(ids, n + 1))
    for lens in (None, torch.full((n_docs,), 20.0, device=dev)):
        kw = dict(lengths=lens, gamma=0.99, alpha=1.5, epsilon=1e-6, want_adv=True, want_returns=True, want_lam=True)
        a0, r0, l0 = gae._run(*d, n_docs, offsets=True, **kw)
        a1, r1, l1 = gae._run(*d, n_docs, offsets=False, **kw)
        assert torch.equal(a0, a1) and torch.equal(r0, r1) and torch.equal(l0, l1)


def test_scan_from_offsets_random_grids(dev):
    """40 seeded grids of random shape (1-4 rows of 1-9000 positions), document
    sizes from 1 token to whole rows, empty document slots, mask holes and a
    trailing padding slot: the offsets scan equals the per-token-id scan bit for
    bit, and the sequential oracle within 1e-3 on the smaller ones."""
    from meshy_amd import gae

    rng = np.random.default_rng(2024)
    for trial in range(40):
        rows = int(rng.integers(1, 5))
        S = int(rng.integers(1, 9001))
        n = rows * S
        # non-decreasing ids over the flattened grid with random run lengths
        runs = []
        while sum(runs) < n:
            runs.append(int(rng.choice([1, 2, 7, 50, 700, 3000, 20000])))
        ids = np.repeat(np.arange(len(runs)), runs)[:n]
        ids = ids * int(rng.choice([1, 2]))  # every other slot empty
        n_docs = int(ids.max()) + 1
        if rng.random() < 0.5:
            ids[-int(rng.integers(1, max(2, n // 10))):] = n_docs  # padding slot
        mask = (rng.random(n) > float(rng.choice([0.0, 0.05, 0.3]))).astype(np.float32)
        t = [torch.from_numpy(x.reshape(rows, S)) for x in
             (rng.standard_normal(n).astype(np.float32) * (rng.random(n) < 0.05),
              rng.standard_normal(n).astype(np.float32), mask, ids.astype(np.int64))]
        lengths = None if rng.random() < 0.5 else torch.from_numpy(rng.random(n_docs).astype(np.float32) * 50 + 1)
        d = [x.to(dev) for x in t]
        kw = dict(lengths=None if lengths is None else lengths.to(dev), gamma=float(rng.choice([1.0, 0.97])),
                  alpha=1.5, epsilon=1e-6, want_adv=True, want_returns=True, want_lam=True)
        a0, r0, l0 = gae._run(*d, n_docs, offsets=True, **kw)
        a1, r1, l1 = gae._run(*d, n_docs, offsets=False, **kw)
        assert torch.equal(a0, a1) and torch.equal(r0, r1) and torch.equal(l0, l1), trial
        if n <= 4000:
            ref_adv, _ = ogae.compute_vapo_gae(*t, n_docs, lengths=lengths, gamma=kw["gamma"], alpha=1.5)
            assert (a0.cpu() - ref_adv).abs().max().item() <= TOL, trial


def _critic_samples(n, seed, max_len=700, bf16=False):
    g = torch.Generator().manual_seed(seed)
    out = []
    for j in range(n):
        L = int(torch.randint(1, max_len, (1,), generator=g))
        prompt = int(torch.randint(0, max(1, L // 2), (1,), generator=g))
        mask = torch.zeros(L)
        mask[prompt:] = 1.0
        if j % 7 == 3:
            mask[:] = 0.0  # a sample without response tokens
        v = torch.randn(L, generator=g)
        out.append({"tokens": torch.arange(L), "mask_assistant": mask,
                    "values": v.to(torch.bfloat16) if bf16 else v,
                    "reward": torch.tensor(float(torch.rand(1, generator=g) < 0.5))})
    return out


@pytest.mark.parametrize("gae_lambda,alpha,gamma,seq_len,bf16", [
    (None, 1.5, 1.0, 10 ** 6, False),
    (0.95, 1.5, 1.0, 10 ** 6, True),
    (None, 0.3, 0.97, 300, False),
    (0.0, 1.0, 1.0, 500, False),
])
def test_attach_gae_advantages_matches_oracle(dev, gae_lambda, alpha, gamma, seq_len, bf16):
    from types import SimpleNamespace as NS

    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.gae import attach_gae_advantages

    samples = _critic_samples(40, seed=hash((gae_lambda, alpha)) % 1000, bf16=bf16)
    ref_adv, ref_m = ogae.attach_gae_advantages(
        [{k: (v.float() if k == "values" else v) for k, v in s.items()} for s in samples],
        seq_len=seq_len, gamma=gamma, alpha=alpha, gae_lambda=gae_lambda)
    trainer = NS(seq_len=seq_len, gae_gamma=gamma, gae_alpha=alpha, gae_lambda=gae_lambda, device=dev)
    metrics = attach_gae_advantages(trainer, samples)
    for s, r in zip(samples, ref_adv):
        got = s[ADVANTAGE_TOKENS]
        assert got.is_cuda and got.shape == r.shape
        assert (got.cpu() - r).abs().max().item() <= TOL
    assert set(metrics) == set(ref_m)
    for k in ref_m:
        assert abs(metrics[k] - ref_m[k]) <= TOL, k


def test_attach_stages_binary_masks_as_bytes_and_fractional_ones_as_fp32(dev):
    """Masks of only 0 and 1 travel as bytes and give the same advantages and
    metrics, bit for bit, as the same masks staged as fp32 (one sample's mask
    as bool sends the whole batch down the fp32 path); a fractional mask
    weight keeps fp32 and matches the oracle."""
    from types import SimpleNamespace as NS

    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.gae import attach_gae_advantages

    trainer = NS(seq_len=500, gae_gamma=1.0, gae_alpha=1.5, gae_lambda=None, device=dev)
    base = _critic_samples(30, seed=21)
    as_bytes = [dict(s) for s in base]
    as_fp32 = [dict(s) for s in base]
    as_fp32[4]["mask_assistant"] = as_fp32[4]["mask_assistant"].bool()
    m_bytes = attach_gae_advantages(trainer, as_bytes)
    m_fp32 = attach_gae_advantages(trainer, as_fp32)
    for a, b in zip(as_bytes, as_fp32):
        assert torch.equal(a[ADVANTAGE_TOKENS], b[ADVANTAGE_TOKENS])
    assert m_bytes == m_fp32
    frac = [dict(s) for s in base]
    g = torch.Generator().manual_seed(5)
    for s in frac[::3]:
        m = s["mask_assistant"].clone()
        m[torch.rand(m.numel(), generator=g) < 0.2] *= 0.5
        s["mask_assistant"] = m
    ref_adv, ref_m = ogae.attach_gae_advantages([dict(s) for s in frac], seq_len=500, gamma=1.0, alpha=1.5,
                                                gae_lambda=None)
    metrics = attach_gae_advantages(trainer, frac)
    for s, r in zip(frac, ref_adv):
        assert (s[ADVANTAGE_TOKENS].cpu() - r).abs().max().item() <= TOL
    for k in ref_m:
        assert abs(metrics[k] - ref_m[k]) <= TOL, k


def test_attach_reads_every_sample_form(dev):
    """Token lists, bool or int masks, rewards as Python floats or 1-element
    tensors, and values of mixed dtypes or non-contiguous take the converting
    path of the staging and give the same advantages and metrics as plain
    tensors; values shorter than the tokens are refused."""
    from types import SimpleNamespace as NS

    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.gae import attach_gae_advantages

    base = _critic_samples(24, seed=9)
    trainer = NS(seq_len=400, gae_gamma=1.0, gae_alpha=1.5, gae_lambda=None, device=dev)
    plain = [dict(s) for s in base]
    want_m = attach_gae_advantages(trainer, plain)
    odd = []
    for j, s in enumerate(base):
        t = dict(s)
        if j % 4 == 0:
            t["tokens"] = t["tokens"].tolist()
        if j % 4 == 1:
            t["mask_assistant"] = t["mask_assistant"].bool()
        if j % 4 == 2:
            t["reward"] = float(t["reward"])
        if j % 4 == 3:
            t["reward"] = t["reward"].reshape(1)
            t["values"] = torch.stack([t["values"], t["values"]], 1)[:, 0]  # non-contiguous
        if j % 5 == 0:
            t["mask_assistant"] = t["mask_assistant"].to(torch.int32)
        odd.append(t)
    got_m = attach_gae_advantages(trainer, odd)
    for a, b in zip(plain, odd):
        assert torch.equal(a[ADVANTAGE_TOKENS], b[ADVANTAGE_TOKENS])
    assert got_m == want_m
    short = [dict(s) for s in base[:3]]
    short[1]["values"] = short[1]["values"][:-1]
    with pytest.raises(ValueError, match="row 1: critic published"):
        attach_gae_advantages(NS(seq_len=10 ** 6, gae_gamma=1.0, gae_alpha=1.5, gae_lambda=None, device=dev), short)


def test_attach_then_whiten_and_pack(dev):
    """GAE advantages left on the device feed whitening (in place, one buffer)
    and the pack (per-token advantages gathered on the device)."""
    from types import SimpleNamespace as NS

    from meshy_amd.batch import ADVANTAGE_TOKENS, build_micro_batches
    from meshy_amd.gae import attach_gae_advantages
    from meshy_amd.plan import MicroPlan
    from meshy_amd.vapo import whiten_advantages
    from oracle import batch as obatch

    samples = _critic_samples(12, seed=5, max_len=300)
    trainer = NS(seq_len=256, gae_gamma=1.0, gae_alpha=1.5, gae_lambda=None, device=dev)
    attach_gae_advantages(trainer, samples)
    ref = [{**s, ADVANTAGE_TOKENS: s[ADVANTAGE_TOKENS].cpu().clone()} for s in samples]
    whiten_advantages(samples, 256, dev)
    ovapo.whiten_advantages(ref, 256)
    for s, r in zip(samples, ref):
        assert (s[ADVANTAGE_TOKENS].cpu() - r[ADVANTAGE_TOKENS]).abs().max().item() <= 1e-4
    for s, r in zip(samples, ref):
        s["logprobs"] = r["logprobs"] = torch.zeros(len(s["tokens"]))
    widths = [min(len(s["tokens"]), 256) for s in samples]
    micro = MicroPlan(tuple(range(4)), sum(widths[:4]) + 9, tuple(widths[:4]))
    mb = build_micro_batches(samples, [micro], layout="packed", device=dev, need_rollout_lp=True)[0]
    ref_mb = obatch.build_micro_batch(ref, micro.sample_idx, micro.seq_len, micro.doc_lens, layout="packed",
                                      need_rollout_lp=True)
    assert (mb.advantages.cpu() - ref_mb["advantages"]).abs().max().item() <= 1e-4
    assert torch.equal(mb.mask.cpu(), ref_mb["mask"])


def test_whitening_known_answers(dev):
    # test_vapo_alignment.py:39-46
    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.vapo import whiten_advantages

    def row(vals):
        return {ADVANTAGE_TOKENS: torch.tensor(vals, dtype=torch.float32),
                "mask_assistant": torch.tensor([0] + [1] * (len(vals) - 1))}

    s = row([2., 4., 1000.])
    whiten_advantages([s], 3, dev)
    torch.testing.assert_close(s[ADVANTAGE_TOKENS], torch.tensor([-2 ** -.5, 2 ** -.5, 0.]))
    s = row([2., 2., 1000.])
    whiten_advantages([s], 3, dev)
    assert s[ADVANTAGE_TOKENS].abs().sum() == 0
    whiten_advantages([], 3, dev)


def test_whitening_matches_oracle(dev):
    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.vapo import whiten_advantages

    g = torch.Generator().manual_seed(0)
    mk = []
    for j in range(20):
        n = int(torch.randint(1, 400, (1,), generator=g))
        mk.append({ADVANTAGE_TOKENS: torch.randn(n, generator=g) * 3 + 1,
                   "mask_assistant": (torch.rand(n, generator=g) > 0.3).float()})
    ref = [{k: v.clone() for k, v in s.items()} for s in mk]
    whiten_advantages(mk, 300, dev)
    ovapo.whiten_advantages(ref, 300)
    for a, b in zip(mk, ref):
        assert (a[ADVANTAGE_TOKENS] - b[ADVANTAGE_TOKENS]).abs().max().item() <= 1e-4


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 8191, 8192, 8193, 300_001])
def test_whiten_flat_sizes_and_alignment(dev, n, offset):
    """Flat buffers around the kernels' 8-element groups and 8192-element
    workgroup steps; offset 1 makes both pointers unaligned (the one-element path)."""
    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.vapo import whiten_flat

    g = torch.Generator().manual_seed(n + offset)
    a = torch.randn(n + offset, generator=g) * 2 + 0.5
    m = (torch.rand(n + offset, generator=g) > 0.25).float()
    ad, md = a.to(dev), m.to(dev)
    whiten_flat(ad[offset:], md[offset:])
    # The oracle's sample form: its loss mask is mask_assistant shifted by one,
    # and the appended last token is outside it.
    s = {ADVANTAGE_TOKENS: torch.cat([a[offset:], torch.zeros(1)]),
         "mask_assistant": torch.cat([torch.zeros(1), m[offset:]])}
    ovapo.whiten_advantages([s], n + 1)
    assert (ad[offset:].cpu() - s[ADVANTAGE_TOKENS][:n]).abs().max().item() <= 1e-4
    assert torch.equal(ad[:offset].cpu(), a[:offset])


def test_whiten_flat_more_elements_than_one_grid_pass(dev):
    """134 M elements: more than the largest grid covers in one step.  Checked by
    what whitening fixes: the masked values' mean is 0 and their unbiased
    variance var / (var + 1e-8); the rest are 0."""
    from meshy_amd.vapo import whiten_flat

    n = 16384 * 8192 + 13
    g = torch.Generator(device=dev).manual_seed(3)
    a = torch.randn(n, generator=g, device=dev) * 2 + 0.5
    m = (torch.rand(n, generator=g, device=dev) > 0.25).float()
    sel = a[m != 0].double()
    var = sel.var().item()
    whiten_flat(a, m)
    w = a[m != 0].double()
    assert abs(w.mean().item()) <= 1e-5
    assert abs(w.var().item() - var / (var + 1e-8)) <= 1e-4
    assert a[m == 0].abs().max().item() == 0.0


def _unaligned(x, dev):
    """The same values in a device view that starts one element past a 16-byte boundary."""
    buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=dev)
    buf[1:] = x.reshape(-1).to(dev)
    return buf[1:].view(x.shape)


@pytest.mark.parametrize("bf16", [False, True])
def test_vector_and_scalar_loads_and_renamed_ids_give_bitwise_equal_results(dev, bf16):
    """Aligned inputs (16-byte loads) and unaligned views (one element at a
    time) build the same maps, so bitwise equal advantages and returns.  The
    ids enter only through equality and the lambda lookup, so ids spread 40000
    apart with the lengths moved along give the same results too."""
    from meshy_amd.gae import gae_and_returns

    rewards, values, mask, doc_ids, n_docs = _random_grid(3, 20000, 7, seed=5)
    values = values.to(torch.bfloat16) if bf16 else values
    g = torch.Generator().manual_seed(6)
    lengths = torch.rand(n_docs, generator=g) * 500 + 1
    kw = dict(gamma=0.99, alpha=1.5)
    d = [t.to(dev) for t in (rewards, values, mask, doc_ids)]
    a0, r0, _ = gae_and_returns(*d, n_docs, lengths=lengths.to(dev), **kw)
    u = [_unaligned(t, dev) for t in (rewards, values, mask, doc_ids)]
    assert all(t.data_ptr() % 16 for t in u)
    a1, r1, _ = gae_and_returns(*u, n_docs, lengths=lengths.to(dev), **kw)
    spread = 40000
    far_lengths = torch.ones(n_docs * spread)
    far_lengths[torch.arange(n_docs) * spread] = lengths
    a2, r2, _ = gae_and_returns(d[0], d[1], d[2], d[3] * spread, n_docs * spread, lengths=far_lengths.to(dev), **kw)
    for a, r in ((a1, r1), (a2, r2)):
        assert torch.equal(a, a0) and torch.equal(r, r0)
    ref_adv, _ = ogae.compute_vapo_gae(rewards, values.float(), mask, doc_ids, n_docs, lengths=lengths, **kw)
    assert (a0.cpu() - ref_adv).abs().max().item() <= TOL
    # Negative ids (lambda 0 there), given to the kernels without the range
    # check of the public call: the vector and scalar loads agree.
    from meshy_amd import gae

    neg = d[3] - 3
    kw2 = dict(lengths=lengths.to(dev), alpha=1.5, epsilon=1e-6, want_adv=True, want_returns=True,
               want_lam=False, offsets=False, gamma=0.99)
    a3, r3, _ = gae._run(d[0], d[1], d[2], neg, n_docs, **kw2)
    a4, r4, _ = gae._run(*u[:3], _unaligned(neg, dev), n_docs, **kw2)
    assert torch.equal(a3, a4) and torch.equal(r3, r4)
    with pytest.raises(ValueError, match="doc_ids must lie"):
        gae_and_returns(d[0], d[1], d[2], neg, n_docs, lengths=lengths.to(dev), **kw)


def _assert_like_oracle(got, ref, what):
    got = got.cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(ref)), f"{what}: NaN pattern"
    inf = torch.isinf(ref)
    assert torch.equal(got[inf], ref[inf]), f"{what}: infinities"
    fin = torch.isfinite(ref)
    assert (got[fin] - ref[fin]).abs().max().item() <= TOL, what


@pytest.mark.parametrize("bf16", [False, True])
def test_nonfinite_inputs_follow_the_sequential_loop(dev, bf16):
    """NaN and infinite rewards or values, against the reference's sequential
    recursion (gae.py:162-180), where 0 * NaN is NaN: a non-finite term at a
    valid position reaches every valid position to its left in its row, across
    document ends, mask holes and chunk boundaries, and stops at the row's start
    (each row of the [rows, S] grid runs its own loop).  Rows of 5000 positions
    (row ends inside 2048-token chunks), then one row of 20000 with the NaN near
    its end (the carry folds across nine chunks), then a finite call again."""
    from meshy_amd.gae import gae_and_returns

    rewards, values, mask, doc_ids, n_docs = _random_grid(3, 5000, 4, seed=91)
    mask[:, 2000:2100] = 0.0
    mask[:, 3000:3100] = 1.0
    rewards[0, 2050] = float("nan")   # invalid position: nothing changes
    values[1, 3050] = float("nan")    # valid: row 1 up to 3050 (and 3049's delta) turns NaN
    rewards[2, 3060] = float("inf")   # valid: inf within its run, NaN across the cuts before it
    vals = values.to(torch.bfloat16) if bf16 else values
    lengths = torch.full((n_docs,), 20.0)
    ref_adv, _ = ogae.compute_vapo_gae(rewards, vals.float(), mask, doc_ids, n_docs, lengths=lengths, gamma=0.99,
                                       alpha=1.5)
    ref_ret = ogae.compute_returns(rewards, mask, doc_ids, gamma=0.99)
    d = [t.to(dev) for t in (rewards, vals, mask, doc_ids)]
    adv, ret, _ = gae_and_returns(*d, n_docs, lengths=lengths.to(dev), gamma=0.99, alpha=1.5)
    _assert_like_oracle(adv, ref_adv, "advantages")
    _assert_like_oracle(ret, ref_ret, "returns")
    assert torch.isfinite(ref_adv[0]).all() and torch.isnan(ref_adv[1, :3000]).any()
    assert torch.isfinite(ref_adv[1, 3100:]).all() and torch.isnan(ref_ret[2, :3000]).any()

    # One row: the NaN near the end reaches back over every document and chunk.
    r1, v1, m1, ids1, nd1 = _random_grid(1, 20000, 12, seed=92)
    m1[0, 19990] = 1.0
    r1[0, 19990] = float("nan")
    ref_adv, _ = ogae.compute_vapo_gae(r1, v1, m1, ids1, nd1, gamma=1.0, alpha=1.5)
    ref_ret = ogae.compute_returns(r1, m1, ids1, gamma=1.0)
    adv, ret, _ = gae_and_returns(*[t.to(dev) for t in (r1, v1, m1, ids1)], nd1, gamma=1.0, alpha=1.5)
    _assert_like_oracle(adv, ref_adv, "one row, advantages")
    _assert_like_oracle(ret, ref_ret, "one row, returns")
    assert torch.isnan(ref_ret[0, :19991][m1[0, :19991] > 0]).all()

    # Finite inputs after a call with non-finite ones: the same results as ever.
    r2, v2, m2, ids2, nd2 = _random_grid(2, 7000, 5, seed=93)
    ref_adv, _ = ogae.compute_vapo_gae(r2, v2, m2, ids2, nd2, gamma=1.0, alpha=1.5)
    adv, ret, _ = gae_and_returns(*[t.to(dev) for t in (r2, v2, m2, ids2)], nd2, gamma=1.0, alpha=1.5)
    assert (adv.cpu() - ref_adv).abs().max().item() <= TOL
    assert torch.isfinite(adv).all() and torch.isfinite(ret).all()


def test_negative_gamma_is_refused(dev):
    from meshy_amd.gae import compute_returns

    z = torch.zeros(1, 8, device=dev)
    with pytest.raises(ValueError, match="gamma"):
        compute_returns(z, z + 1, torch.zeros(1, 8, dtype=torch.long, device=dev), gamma=-0.5)


@pytest.mark.parametrize("seed", range(10))
def test_random_attach_matches_oracle(dev, seed):
    """Random critic batches (one-token samples, masks with holes, samples
    longer than seq_len, fp32 or bf16 values, float rewards) and random
    gamma, lambda and alpha: the attached advantages and the metrics equal
    the oracle's."""
    from types import SimpleNamespace as NS

    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.gae import attach_gae_advantages

    rng = np.random.default_rng(2000 + seed)
    bf16 = bool(seed % 2)
    samples = []
    for j in range(int(rng.integers(1, 60))):
        L = 1 if rng.random() < 0.1 else int(rng.integers(2, 900))
        mask = (rng.random(L) < 0.8).astype(np.float32)
        mask[: int(rng.integers(0, max(1, L // 3)))] = 0.0
        v = torch.from_numpy(rng.normal(size=L).astype(np.float32))
        samples.append({"tokens": torch.arange(L), "mask_assistant": torch.from_numpy(mask),
                        "values": v.to(torch.bfloat16) if bf16 else v,
                        "reward": torch.tensor(float(rng.normal()))})
    seq_len = int(rng.choice([64, 512, 10 ** 6]))
    gamma = float(rng.choice([1.0, 0.99, 0.9]))
    lam = None if seed % 3 == 0 else float(rng.choice([0.0, 0.9, 0.95, 1.0]))
    alpha = float(rng.uniform(0.2, 2.0))
    ref_adv, ref_m = ogae.attach_gae_advantages(
        [{k: (v.float() if k == "values" else v) for k, v in s.items()} for s in samples],
        seq_len=seq_len, gamma=gamma, alpha=alpha, gae_lambda=lam)
    trainer = NS(seq_len=seq_len, gae_gamma=gamma, gae_alpha=alpha, gae_lambda=lam, device=dev)
    metrics = attach_gae_advantages(trainer, samples)
    for s, r in zip(samples, ref_adv):
        got = s[ADVANTAGE_TOKENS]
        assert got.is_cuda and got.shape == r.shape
        assert (got.cpu() - r).abs().max().item() <= TOL
    assert set(metrics) == set(ref_m)
    for k in ref_m:
        assert abs(metrics[k] - ref_m[k]) <= TOL * max(1.0, abs(ref_m[k])), k

"""Pins the OPD part of the CPU oracle (CPU only): the reference's known answers
of test_opd_loss.py and test_opd_batch.py, a brute-force (value, index) sort for
the Top-K tie order, and closed forms of the distillation loss and its gradient."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import batch as obatch
from oracle import opd as oopd
from oracle import topk as otopk


def _logits(rows=2, S=7, V=50, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, S, V, generator=g) * 3


# ------------------------------------------------- topk_loss.py (test_opd_loss.py)


def test_teacher_topk_matches_dense_log_softmax():
    # test_opd_loss.py:13-20
    z = _logits()
    ids, lps = otopk.teacher_topk(z, 5, chunk=3)
    ref = torch.log_softmax(z, dim=-1).topk(5, dim=-1)
    assert torch.equal(ids, ref.indices)
    assert torch.allclose(lps, ref.values, atol=1e-6)
    assert ids.shape == (2, 7, 5) and lps.dtype == torch.float32


def test_teacher_topk_tie_order_brute_force():
    # Many equal logits: the oracle ranks by value, then by ascending index.
    g = torch.Generator().manual_seed(3)
    z = torch.randint(0, 4, (3, 5, 20), generator=g).float()
    ids, lps = otopk.teacher_topk(z, 7, chunk=2)
    for r in range(3):
        for t in range(5):
            row = z[r, t].tolist()
            want = sorted(range(20), key=lambda j: (-row[j], j))[:7]
            assert ids[r, t].tolist() == want
            lse = math.log(sum(math.exp(v) for v in row))
            assert lps[r, t].tolist() == pytest.approx([row[j] - lse for j in want], abs=1e-5)


@pytest.mark.parametrize("k", [1, 7, 64])
def test_teacher_topk_by_threshold_equals_the_stable_sort(k):
    """The one-selection form used on 16384-row batches gives the stable
    sort's ids and log-probs: ties at and above the k-th value (integer
    logits), -0 beside +0, a row of equal values, a row of -inf."""
    g = torch.Generator().manual_seed(k)
    z = torch.randint(-3, 4, (2, 9, 300), generator=g).float()
    z[0, 0, 5], z[0, 0, 6] = -0.0, 0.0
    z[1, 3, :] = 2.0
    z[1, 4, :] = float("-inf")
    z = z.to(torch.bfloat16)
    a_ids, a_lps = otopk.teacher_topk(z, k, chunk=4)
    b_ids, b_lps = otopk.teacher_topk_by_threshold(z, k, chunk=4)
    assert torch.equal(a_ids, b_ids)
    assert torch.equal(a_lps.nan_to_num(), b_lps.nan_to_num())
    w = (torch.randn(1, 40, 5000, generator=g) * 2.0).to(torch.bfloat16)
    assert torch.equal(otopk.teacher_topk(w, k)[0], otopk.teacher_topk_by_threshold(w, k)[0])


def test_gather_logprobs_matches_dense_and_propagates_grad():
    # test_opd_loss.py:23-33
    z = _logits().requires_grad_(True)
    ids = torch.randint(0, 50, (2, 7, 4), generator=torch.Generator().manual_seed(1))
    out = otopk.gather_logprobs(z, ids, chunk=2)
    ref = torch.log_softmax(z, dim=-1).gather(-1, ids)
    assert torch.allclose(out, ref, atol=1e-6)
    out.sum().backward()
    g1 = z.grad.clone()
    z.grad = None
    ref.sum().backward()
    assert torch.allclose(g1, z.grad, atol=1e-6)


def test_forward_kl_topk_formula_and_clamps():
    # test_opd_loss.py:36-49, plus the closed form of the first case
    log_t = torch.log(torch.tensor([[[0.5, 0.3, 0.2]]]))
    log_s = torch.log(torch.tensor([[[0.2, 0.3, 0.5]]]))
    kl = otopk.forward_kl_topk(log_s, log_t)
    assert float(kl) == pytest.approx(0.5 * math.log(2.5) + 0.2 * math.log(0.4), abs=1e-6)
    assert torch.allclose(otopk.forward_kl_topk(log_t, log_t), torch.zeros(1, 1))
    tiny = torch.log(torch.tensor([[[1e-30, 0.3, 0.5]]]))
    unclamped = otopk.forward_kl_topk(tiny, log_t)
    clamped = otopk.forward_kl_topk(tiny, log_t, log_prob_min_clamp=-10.0)
    assert unclamped.item() > clamped.item() > 0
    assert clamped.item() == pytest.approx(0.5 * (math.log(0.5) + 10.0) + 0.2 * math.log(0.4), abs=1e-5)
    assert otopk.forward_kl_topk(tiny, log_t, loss_max_clamp=1.0).item() == 1.0


# ------------------------------------------------- opd.py layout (test_opd_batch.py)

K = 3


def _sample(L: int, seed: int) -> dict:
    # test_opd_batch.py:22-39: candidate 0 of Teacher row t is tokens[t + 1]
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randint(0, 1000, (L,), generator=g)
    ids = torch.randint(0, 1000, (L, K), generator=g)
    ids[:-1, 0] = tokens[1:]
    return {
        "tokens": tokens,
        "logprobs": -torch.rand(L, generator=g),
        "mask_assistant": torch.ones(L),
        "advantage": torch.tensor(0.0),
        "teacher_topk_ids": ids,
        "teacher_topk_logprobs": -torch.rand(L, K, generator=g),
    }


@pytest.mark.parametrize("layout", ["padded", "packed"])
def test_teacher_rows_align_with_labels(layout):
    # test_opd_batch.py:42-57
    samples = [_sample(5, 0), _sample(8, 1), _sample(3, 2)]
    idx, seq_len, doc_lens = (1, 0, 2), (16 if layout == "packed" else 8), (8, 5, 3)
    mb = obatch.build_micro_batch(samples, idx, seq_len, doc_lens, layout=layout, need_rollout_lp=False)
    ids, lps = oopd.layout_teacher_topk(samples, idx, seq_len, doc_lens, layout=layout)
    assert ids.shape == mb["labels"].shape + (K,) and lps.shape == ids.shape
    on = mb["mask"] > 0
    assert torch.equal(ids[..., 0][on], mb["labels"][on])
    back = oopd.split_teacher_topk(ids, doc_lens, layout=layout)
    for j, i in enumerate(idx):
        assert torch.equal(back[j], samples[i]["teacher_topk_ids"][:doc_lens[j]])


def test_truncation_short_teacher_rows_filler_and_top_k():
    # test_opd_batch.py:60-75
    samples = [_sample(6, 0)]
    ids, _ = oopd.layout_teacher_topk(samples, (0,), 4, (4,), layout="padded")
    assert torch.equal(ids[0], samples[0]["teacher_topk_ids"][:4])
    short = _sample(6, 1)
    short["teacher_topk_ids"] = short["teacher_topk_ids"][:2]
    with pytest.raises(ValueError, match="Teacher seq_len"):
        oopd.layout_teacher_topk([short], (0,), 4, (4,), layout="padded")
    ids, lps = oopd.layout_teacher_topk([], (), 4, (), layout="padded")
    assert ids.shape == (1, 4, 1) and lps.shape == (1, 4, 1)
    assert oopd.infer_top_k([_sample(2, 0)]) == K


# ------------------------------------------------- opd.py:153-197 closed forms


def _halves(rows, S, mask, doc_ids):
    # Teacher (1/2, 1/2) on two candidates, student (1/4, 1/4): KL = ln 2 per token.
    teacher = torch.full((rows, S, 2), math.log(0.5))
    gathered = torch.full((rows, S, 3), math.log(0.25))
    gathered[..., 2] = -1.0  # the sampled label's log-prob
    return teacher, gathered.requires_grad_(True)


@pytest.mark.parametrize("per_token", [True, False])
def test_distill_loss_closed_form(per_token):
    S = 10
    mask = torch.ones(1, S)
    mask[0, 3] = 0.0
    doc_ids = torch.tensor([[0, 0, 0, 0, 1, 1, 1, 1, 1, 2]])  # two documents and a padding token
    mask[0, 9] = 0.0
    teacher, gathered = _halves(1, S, mask, doc_ids)
    rollout = torch.full((1, S), -1.0)
    n_tok = int(mask.sum())
    loss, sums = oopd.distill_loss(gathered, teacher, mask, doc_ids, 2, rollout_lp=rollout, n_docs_global=2,
                                   n_tokens_global=n_tok, per_token_loss=per_token)
    assert float(loss.detach()) == pytest.approx(math.log(2.0), abs=1e-6)
    assert float(sums["token_count"]) == n_tok
    assert float(sums["teacher_mass_sum"]) == pytest.approx(n_tok * 1.0, abs=1e-5)
    assert float(sums["student_mass_sum"]) == pytest.approx(n_tok * 0.5, abs=1e-5)
    assert float(sums["train_rollout_kl_sum"]) == 0.0 and float(sums["train_rollout_logdiff_abs_sum"]) == 0.0
    loss.backward()
    g = gathered.grad
    # d loss / d log_s_k = -p_T(k) * mask * D_doc; the sampled column gets nothing
    if per_token:
        want = torch.tensor([-0.5 / n_tok if m else 0.0 for m in mask[0].tolist()])
    else:
        cnt = {0: 3.0, 1: 5.0}
        want = torch.tensor([(-0.5 / cnt[d] / 2 if (m and d < 2) else 0.0)
                             for m, d in zip(mask[0].tolist(), doc_ids[0].tolist())])
    assert torch.allclose(g[0, :, 0], want, atol=1e-7) and torch.allclose(g[0, :, 1], want, atol=1e-7)
    assert (g[..., 2] == 0).all()
    m = oopd.reduce_distill_metrics(sums)
    assert m["train/teacher_topk_mass"] == pytest.approx(1.0) and m["train/student_topk_mass"] == pytest.approx(0.5)


def test_distill_loss_equal_distributions_is_zero():
    g = torch.Generator().manual_seed(5)
    t = torch.log_softmax(torch.randn(1, 12, 4, generator=g), -1)
    gathered = torch.cat([t, torch.zeros(1, 12, 1)], -1).requires_grad_(True)
    loss, _ = oopd.distill_loss(gathered, t, torch.ones(1, 12), torch.zeros(1, 12, dtype=torch.long), 1,
                                n_docs_global=1, n_tokens_global=12, per_token_loss=True)
    assert abs(float(loss.detach())) < 1e-6

"""Layout invariance of the whole path on the GPU: pack -> log-probs (with their
autograd backward) -> PPO loss, the properties the reference checks on a model
in tests/test_dynamic_batching_gpu.py:108-178:

* the packed and padded layouts of the same samples give the same per-token
  log-probs, the same loss and the same gradient;
* splitting the samples over one micro-batch each keeps the loss (a global
  mean over the mini-batch, not a mean per micro);
* a filler micro-batch contributes nothing;

and, for Student Top-K distillation (tests/test_opd_gpu.py:110-149), that the
Teacher's Top-K columns are a sorted sub-distribution, a student equal to its
Teacher has zero KL, and padded and packed students agree.

Synthetic bf16 logits stand in for the model: sample i owns one ``[L_i, V]``
leaf tensor, placed at that sample's positions in every layout, so both
layouts score the same numbers.  Per-token log-probs and gradients must agree
exactly (the kernels compute each row from that row alone); the loss to fp32
summation order (1e-5 relative)."""

from __future__ import annotations

from types import SimpleNamespace as NS

import pytest
import torch

pytestmark = pytest.mark.gpu

V = 512
SEQ = 256
LENGTHS = [37, 120, 64, 5, 200, 90, 150, 33, 256, 2]


class _NoCp:
    enabled = False

    def all_reduce_sum(self, value):
        return value


def _stub(per_token):
    return NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, use_icepop=False, tis_ratio_min=0.5,
              tis_ratio_max=5.0, calculate_per_token_loss=per_token, positive_lm_loss_coef=0.0,
              old_logprobs_source="rollout", sharder=_NoCp(), parallel_dims=NS(cp=1))


def _samples(seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i, L in enumerate(LENGTHS):
        mask = torch.zeros(L)
        mask[max(1, L // 3):] = 1.0
        out.append({"tokens": torch.randint(0, V, (L,), generator=g), "mask_assistant": mask,
                    "logprobs": -3.0 * torch.rand(L, generator=g),
                    "advantage": torch.tensor(float(torch.randn(1, generator=g))),
                    "reward": torch.tensor(float(i % 2))})
    return out


def _leaf_logits(seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return [(torch.randn(L, V, generator=g, device=dev) * 2.0).to(torch.bfloat16).requires_grad_(True)
            for L in LENGTHS]


def _plan(samples, layout, **cfg_kw):
    from meshy_amd.plan import PlannerConfig, build_plan

    cfg = PlannerConfig(layout=layout, mini_batch_size=len(samples), seq_len=SEQ, align=64, **cfg_kw)
    lengths = [len(s["tokens"]) for s in samples]
    loss_tokens = [int((s["mask_assistant"][1:min(L, SEQ)] > 0).sum()) if L > 1 else 0
                   for s, L in zip(samples, lengths)]
    return build_plan(lengths, loss_tokens, 1, cfg)


def _micro_logits(micro, layout, local, leaves, dev):
    """The micro's logits from the samples' leaves: packed [1, T, V] in document
    order with zero padding, padded [rows, S, V] one document per row."""
    parts = [leaves[local[i]][:L] for i, L in zip(micro.sample_idx, micro.doc_lens)]
    S = micro.seq_len
    zero = torch.zeros(0, V, dtype=torch.bfloat16, device=dev)
    if layout == "packed":
        used = sum(p.shape[0] for p in parts)
        pad = torch.zeros(S - used, V, dtype=torch.bfloat16, device=dev)
        return torch.cat(parts + [pad if S > used else zero]).unsqueeze(0)
    if not parts:
        return torch.zeros(1, S, V, dtype=torch.bfloat16, device=dev)
    rows = [torch.cat([p, torch.zeros(S - p.shape[0], V, dtype=torch.bfloat16, device=dev)]) for p in parts]
    return torch.stack(rows)


def _run(samples, plan, layout, leaves, per_token, dev, minis=None):
    """Sum of the micro losses of rank 0's mini-batches, the per-sample log-probs
    and the gradients of the leaves."""
    from meshy_amd import logprob
    from meshy_amd.batch import build_micro_batches
    from meshy_amd.loss import ppo_clip_loss

    for x in leaves:
        x.grad = None
    local = plan.local_indices[0]
    local_samples = plan.local_samples(samples, 0)
    stub = _stub(per_token)
    total = torch.zeros((), device=dev)
    per_sample = {}
    n_micro = 0
    for mini in (minis or plan.per_rank[0]):
        batches = build_micro_batches(local_samples, mini.micros, layout=layout, device=dev, need_rollout_lp=True)
        for micro, mb in zip(mini.micros, batches):
            n_micro += 1
            logits = _micro_logits(micro, layout, local, leaves, dev)
            lp = logprob.logprobs_and_entropy(logits, mb.labels)
            loss, _ = ppo_clip_loss(stub, lp, mb.rollout_logprobs, mb, mini)
            total = total + loss
            for j, (i, L) in enumerate(zip(micro.sample_idx, micro.doc_lens)):
                sel = (mb.doc_ids == j) & (mb.positions < L)
                per_sample[local[i]] = lp.detach()[sel]
    total.backward()
    grads = [x.grad.clone() if x.grad is not None else torch.zeros_like(x) for x in leaves]
    return total.item(), per_sample, grads, n_micro


@pytest.mark.parametrize("per_token", [False, True])
def test_layouts_give_same_logprobs_loss_and_grad(dev, per_token):
    samples = _samples(1)
    leaves = _leaf_logits(1, dev)
    res = {}
    for layout in ("padded", "packed"):
        plan = _plan(samples, layout, max_tokens_per_micro=512)
        res[layout] = _run(samples, plan, layout, leaves, per_token, dev)
    (la, pa, ga, na), (lb, pb, gb, nb) = res["padded"], res["packed"]
    assert na >= 2 and nb >= 2
    assert set(pa) == set(pb) == set(range(len(LENGTHS)))
    for i in pa:
        assert pa[i].shape == (LENGTHS[i],) and torch.equal(pa[i], pb[i]), i
    assert la == pytest.approx(lb, rel=1e-5, abs=1e-7)
    assert la != 0.0
    for i, (a, b) in enumerate(zip(ga, gb)):
        assert torch.equal(a, b), i
    assert any(g.abs().max().item() > 0 for g in ga)


def test_loss_is_a_global_mean_over_samples(dev):
    """One sample per micro-batch (the row cap) against as few micros as the budget allows."""
    samples = _samples(2)
    leaves = _leaf_logits(2, dev)
    one = _run(samples, _plan(samples, "padded", max_tokens_per_micro=4096), "padded", leaves, False, dev)
    many_plan = _plan(samples, "padded", max_tokens_per_micro=None, micro_batch_size=1)
    many = _run(samples, many_plan, "padded", leaves, False, dev)
    assert many[3] == len(LENGTHS) and one[3] < many[3]
    assert one[0] == pytest.approx(many[0], rel=1e-5)
    for a, b in zip(one[2], many[2]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("layout", ["padded", "packed"])
def test_filler_micro_contributes_nothing(dev, layout):
    from meshy_amd.plan import MicroPlan, MiniPlan

    samples = _samples(3)
    leaves = _leaf_logits(3, dev)
    plan = _plan(samples, layout, max_tokens_per_micro=512)
    mini = plan.per_rank[0][0]
    with_filler = MiniPlan(micros=mini.micros + (MicroPlan((), 64, ()),), n_docs_global=mini.n_docs_global,
                           n_tokens_global=mini.n_tokens_global, tokens_per_rank=mini.tokens_per_rank)
    ref = _run(samples, plan, layout, leaves, False, dev, minis=[mini])
    got = _run(samples, plan, layout, leaves, False, dev, minis=[with_filler])
    assert got[3] == ref[3] + 1
    assert got[0] == ref[0]
    for a, b in zip(ref[2], got[2]):
        assert torch.equal(a, b)


# ------------------------------------------------------------- Student Top-K OPD
# tests/test_opd_gpu.py:110-149: the Teacher's Top-K columns are a sorted
# sub-distribution, a student equal to its Teacher has zero KL, and padded and
# packed students agree on the loss and the gradient.

TOP_K = 8


def _scored(samples, teacher, dev):
    """Teacher columns from the Teacher's logits of each sample (score_samples)."""
    from meshy_amd import topk

    for s, z in zip(samples, teacher):
        ids, lps = topk.teacher_topk(z.detach().unsqueeze(0), k=TOP_K)
        s["teacher_topk_ids"] = ids[0].cpu()
        s["teacher_topk_logprobs"] = lps[0].cpu()
    return samples


class _Model:
    """Stands in for model_parts[0]: returns the logits set for the next micro."""

    logits = None

    def __call__(self, input_ids, positions=None, attention_masks=None):
        assert self.logits.shape[:2] == input_ids.shape
        return self.logits


def _run_opd(samples, plan, layout, leaves, per_token, dev):
    from meshy_amd import opd

    for x in leaves:
        x.grad = None
    local = plan.local_indices[0]
    model = _Model()
    stub = NS(calculate_per_token_loss=per_token, log_prob_min_clamp=-10.0, loss_max_clamp=10.0, sharder=None,
              parallel_dims=NS(cp=1), model_parts=[model], _LOGPROB_CHUNK=1024)
    total = torch.zeros((), device=dev)
    sums_all = []
    for mini in plan.per_rank[0]:
        batches = opd.build_topk_micro_batches(plan.local_samples(samples, 0), mini.micros, layout=layout,
                                               device=dev, need_rollout_lp=True)
        for micro, mb in zip(mini.micros, batches):
            model.logits = _micro_logits(micro, layout, local, leaves, dev)
            loss, sums = opd.distill_loss(stub, mb, mini)
            total = total + loss
            sums_all.append(sums)
    total.backward()
    metrics = opd.reduce_distill_metrics(stub, {k: sum(s[k] for s in sums_all) for k in sums_all[0]})
    return total.item(), metrics, [x.grad.clone() for x in leaves]


def test_teacher_topk_columns_are_a_sorted_subdistribution(dev):
    samples = _scored(_samples(4), _leaf_logits(40, dev), dev)
    for s, L in zip(samples, LENGTHS):
        lps, ids = s["teacher_topk_logprobs"], s["teacher_topk_ids"]
        assert lps.shape == ids.shape == (L, TOP_K)
        assert torch.all(lps <= 0) and torch.all(lps.exp().sum(-1) <= 1.0 + 1e-4)
        assert (lps[:, :-1] >= lps[:, 1:]).all() and ids.min() >= 0 and ids.max() < V


def test_student_equal_to_teacher_has_zero_kl(dev):
    teacher = _leaf_logits(41, dev)
    samples = _scored(_samples(5), teacher, dev)
    plan = _plan(samples, "padded", max_tokens_per_micro=512)
    loss, m, _ = _run_opd(samples, plan, "padded", teacher, True, dev)
    assert abs(loss) < 1e-5 and abs(m["train/distill_loss"]) < 1e-5
    assert m["train/student_topk_mass"] == pytest.approx(m["train/teacher_topk_mass"], abs=1e-5)
    assert 0.0 < m["train/teacher_topk_mass"] <= 1.0
    assert "train_rollout_kl" in m


@pytest.mark.parametrize("per_token", [False, True])
def test_padded_and_packed_students_agree(dev, per_token):
    samples = _scored(_samples(6), _leaf_logits(42, dev), dev)
    student = _leaf_logits(43, dev)
    res = {layout: _run_opd(samples, _plan(samples, layout, max_tokens_per_micro=512), layout, student, per_token,
                            dev)
           for layout in ("padded", "packed")}
    (la, ma, ga), (lb, mb, gb) = res["padded"], res["packed"]
    assert la > 0.0 and la == pytest.approx(lb, rel=1e-5)
    for k in ma:
        assert ma[k] == pytest.approx(mb[k], rel=1e-5, abs=1e-7), k
    for i, (a, b) in enumerate(zip(ga, gb)):
        assert torch.equal(a, b), i
    assert any(g.abs().max().item() > 0 for g in ga)

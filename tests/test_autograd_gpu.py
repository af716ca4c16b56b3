"""The C++ autograd nodes of the three loss drop-ins (PPO clip loss, Top-K
distillation loss, clipped value error) behave as autograd functions do:
gradients against the oracle (torch autograd through the reference's
restatement) under a scaled loss, torch.autograd.grad, retain_graph, no-grad
forwards, bf16 inputs and a side stream; a second backward after the graph was
freed and an in-place change of a tensor the backward reads raise.
Tolerance: 1e-3 absolute on losses and sums, 1e-6 on gradients."""

from __future__ import annotations

from types import SimpleNamespace as NS

import pytest
import torch

from oracle import critic as ocritic
from oracle import opd as oopd
from oracle import ppo as oppo

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _ppo_case(dev, per_token):
    from meshy_amd.batch import Batch
    from meshy_amd.plan import MiniPlan

    g = torch.Generator().manual_seed(11 if per_token else 12)
    lens = [700, 1300, 9, 2000]
    n, S = len(lens), sum(lens) + 24
    doc_ids = torch.cat([torch.repeat_interleave(torch.arange(n), torch.tensor(lens)),
                         torch.full((24,), n)]).reshape(1, S)
    mask = (torch.rand(1, S, generator=g) > 0.15).float()
    mask[0, -24:] = 0
    old = -torch.rand(1, S, generator=g) * 3
    new = old + torch.randn(1, S, generator=g) * 0.2
    adv = torch.randn(n, generator=g)
    z = torch.zeros(1, S, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask.to(dev), doc_ids.to(dev), adv.to(dev), None, torch.zeros(n, device=dev), n)
    mini = MiniPlan(micros=(), n_docs_global=n + 2, n_tokens_global=int(mask.sum()) + 50, tokens_per_rank=())
    stub = NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, calculate_per_token_loss=per_token,
              old_logprobs_source="rollout", sharder=None, parallel_dims=NS(cp=1))

    def oracle(scale=1.0):
        nr = new.clone().requires_grad_(True)
        loss, sums = oppo.ppo_clip_loss(nr, old, mask, doc_ids, adv, n, n_docs_global=mini.n_docs_global,
                                        n_tokens_global=mini.n_tokens_global, clip_low=0.2, clip_high=0.28,
                                        per_token_loss=per_token)
        (loss * scale).backward()
        return loss.detach(), sums, nr.grad

    return stub, mb, mini, old.to(dev), new, oracle


@pytest.mark.parametrize("per_token", [True, False])
def test_ppo_node_gradients_and_graph_rules(dev, per_token):
    from meshy_amd.loss import ppo_clip_loss

    stub, mb, mini, old_d, new, oracle = _ppo_case(dev, per_token)
    ref_loss, ref_sums, ref_grad = oracle(3.0)
    nd = new.to(dev).requires_grad_(True)
    loss, sums = ppo_clip_loss(stub, nd, old_d, mb, mini)
    assert loss.requires_grad and loss.grad_fn.name() == "MeshyPpoLossBackward"
    # new_lp's own node follows directly: no view node in between
    assert loss.grad_fn.next_functions[0][0].variable is nd
    assert abs(loss.item() - ref_loss.item()) <= TOL
    assert abs(sums["ppo_kl_sum"].item() - float(ref_sums["ppo_kl_sum"])) <= TOL
    (loss * 3.0).backward(retain_graph=True)
    assert (nd.grad.cpu() - ref_grad).abs().max().item() <= 1e-6
    # a retained graph runs again and accumulates
    loss.backward(retain_graph=True)
    assert (nd.grad.cpu() - ref_grad * (4.0 / 3.0)).abs().max().item() <= 1e-6
    # torch.autograd.grad through the same node
    (g,) = torch.autograd.grad(loss, nd, retain_graph=True)
    assert (g.cpu() - ref_grad / 3.0).abs().max().item() <= 1e-6
    loss.backward()  # frees the graph
    with pytest.raises(RuntimeError, match="second time"):
        loss.backward()
    # the forward alone: the same loss and sums, no graph
    with torch.no_grad():
        l0, s0 = ppo_clip_loss(stub, nd, old_d, mb, mini)
    assert not l0.requires_grad and l0.grad_fn is None
    assert abs(l0.item() - loss.item()) <= 1e-6 * max(1.0, abs(loss.item()))
    assert abs(s0["ppo_kl_sum"].item() - sums["ppo_kl_sum"].item()) <= 1e-6 * max(1.0, abs(sums["ppo_kl_sum"].item()))


def test_ppo_node_refuses_inplace_change_of_new_lp(dev):
    from meshy_amd.loss import ppo_clip_loss

    stub, mb, mini, old_d, new, _ = _ppo_case(dev, False)
    nd = new.to(dev).requires_grad_(True)
    loss, _ = ppo_clip_loss(stub, nd, old_d, mb, mini)
    with torch.no_grad():
        nd.mul_(1.0)  # bumps the version the backward checks
    with pytest.raises(RuntimeError, match="inplace"):
        loss.backward()


def test_ppo_node_bf16_new_lp_and_side_stream(dev):
    """new_lp in bf16 (the fp32 copy sits between it and the node) and the whole
    call on a side stream: the backward runs on the forward's stream."""
    from meshy_amd.loss import ppo_clip_loss

    stub, mb, mini, old_d, new, _ = _ppo_case(dev, True)
    new16 = new.to(torch.bfloat16)
    nr = new16.float().clone().requires_grad_(True)
    ref_loss, _ = oppo.ppo_clip_loss(nr, old_d.cpu(), mb.mask.cpu(), mb.doc_ids.cpu(), mb.advantages.cpu(),
                                     mb.n_docs, n_docs_global=mini.n_docs_global,
                                     n_tokens_global=mini.n_tokens_global, clip_low=0.2, clip_high=0.28,
                                     per_token_loss=True)
    ref_loss.backward()
    side = torch.cuda.Stream()
    nd = new16.to(dev).requires_grad_(True)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        loss, _ = ppo_clip_loss(stub, nd, old_d, mb, mini)
        loss.backward()
    side.synchronize()
    assert nd.grad.dtype == torch.bfloat16
    assert abs(loss.item() - ref_loss.item()) <= TOL
    assert (nd.grad.float().cpu() - nr.grad.to(torch.bfloat16).float()).abs().max().item() <= 1e-2 * max(
        nr.grad.abs().max().item(), 1e-6)


def test_distill_node_gradients_and_graph_rules(dev):
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan, MiniPlan

    K = 8
    g = torch.Generator().manual_seed(21)
    lens = [400, 33, 900]
    samples = []
    for i, L in enumerate(lens):
        m = torch.ones(L)
        m[: L // 5] = 0
        samples.append({"tokens": torch.randint(0, 1000, (L,), generator=g), "logprobs": -torch.rand(L, generator=g),
                        "mask_assistant": m, "advantage": torch.tensor(0.0),
                        "teacher_topk_ids": torch.randint(0, 1000, (L, K), generator=g),
                        "teacher_topk_logprobs": -torch.rand(L, K, generator=g) * 5})
    micro = MicroPlan((0, 1, 2), 1400, tuple(lens))
    mb = opd.build_topk_micro_batches(samples, [micro], layout="packed", device=dev, need_rollout_lp=True)[0]
    gathered = torch.log_softmax(torch.randn(1, 1400, K + 1, generator=g) * 3, -1)
    mini = MiniPlan((micro,), 4, int(mb.mask.sum().item()) + 7, (0,))
    stub = NS(calculate_per_token_loss=False, log_prob_min_clamp=-10.0, loss_max_clamp=10.0, sharder=None)
    gr = gathered.clone().requires_grad_(True)
    rl, rs = oopd.distill_loss(gr, mb.teacher_topk_logprobs.cpu(), mb.mask.cpu(), mb.doc_ids.cpu(), mb.n_docs,
                               rollout_lp=mb.rollout_logprobs.cpu(), n_docs_global=4,
                               n_tokens_global=mini.n_tokens_global, per_token_loss=False)
    (rl * 2.0).backward()
    gd = gathered.to(dev).requires_grad_(True)
    loss, sums = opd.distill_from_gathered(stub, gd, mb, mini)
    assert loss.grad_fn.name() == "MeshyDistillLossBackward"
    assert abs(loss.item() - rl.item()) <= TOL
    for key in rs:
        assert abs(float(sums[key]) - float(rs[key])) <= TOL + 1e-5 * abs(float(rs[key])), key
    (loss * 2.0).backward(retain_graph=True)
    assert (gd.grad.cpu() - gr.grad).abs().max().item() <= 1e-6
    loss.backward()
    assert (gd.grad.cpu() - gr.grad * 1.5).abs().max().item() <= 1e-6
    with pytest.raises(RuntimeError, match="second time"):
        loss.backward()
    loss2, _ = opd.distill_from_gathered(stub, gd, mb, mini)
    with torch.no_grad():
        gd.add_(0.0)
    with pytest.raises(RuntimeError, match="inplace"):
        loss2.backward()


@pytest.mark.parametrize("clip", [None, 0.2])
def test_clipped_value_error_node(dev, clip):
    """Broadcast gradients (a sum or a mean) and a materialised one (a weighted
    sum), fp32 and bf16 values; the in-place and second-backward rules."""
    from meshy_amd import critic

    g = torch.Generator().manual_seed(31)
    n = 70_001
    v = torch.randn(n, generator=g)
    t = torch.randn(n, generator=g)
    o = v + 0.3 * torch.randn(n, generator=g)
    w = torch.rand(n, generator=g)
    td, od, wd = t.to(dev), o.to(dev), w.to(dev)
    for dtype in (torch.float32, torch.bfloat16):
        vq = v.to(dtype)
        for reduce in ("sum", "mean", "weighted"):
            vr = vq.float().clone().requires_grad_(True)
            er = ocritic.clipped_value_error(vr, t, o, clip)
            (er.sum() if reduce == "sum" else er.mean() if reduce == "mean" else (er * w).sum()).backward()
            vd = vq.to(dev).requires_grad_(True)
            e = critic.clipped_value_error(vd, td, od, clip)
            assert (e.float().cpu() - er.detach()).abs().max().item() <= 1e-5 * max(1.0, er.abs().max().item())
            (e.sum() if reduce == "sum" else e.mean() if reduce == "mean" else (e * wd).sum()).backward()
            want = vr.grad.to(dtype).float()
            tol = 1e-6 if dtype == torch.float32 else 1e-2 * max(want.abs().max().item(), 1e-6)
            assert vd.grad.dtype == dtype
            assert (vd.grad.float().cpu() - want).abs().max().item() <= tol, (dtype, reduce)
    # a [rows, S] grid: the mean's gradient arrives broadcast over both dimensions
    v2, t2, o2 = (x[:70_000].reshape(70, 1000) for x in (v, t, o))
    vr = v2.clone().requires_grad_(True)
    ocritic.clipped_value_error(vr, t2, o2, clip).mean().backward()
    vd = v2.to(dev).requires_grad_(True)
    e = critic.clipped_value_error(vd, t2.to(dev), o2.to(dev), clip)
    assert e.shape == (70, 1000)
    e.mean().backward()
    assert vd.grad.shape == (70, 1000) and (vd.grad.cpu() - vr.grad).abs().max().item() <= 1e-6
    vd = v.to(dev).requires_grad_(True)
    s = critic.clipped_value_error(vd, td, od, clip).sum()
    s.backward()
    with pytest.raises(RuntimeError, match="second time"):
        s.backward()
    s = critic.clipped_value_error(vd, td, od, clip).sum()
    td.add_(1.0)  # targets are read by the backward
    with pytest.raises(RuntimeError, match="inplace"):
        s.backward()

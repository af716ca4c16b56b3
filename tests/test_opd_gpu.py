"""Student Top-K OPD kernels against the oracle (the reference's torch path on CPU).

Bars: Top-K ids bit-exact (ties by ascending index), teacher columns bit-exact,
1e-3 absolute on fp32 log-probs, KL, loss and sums (relative 1e-5 on token
sums), bf16 gradients within their rounding (4e-3 x |g|), fp32 gradients 1e-6.
"""

from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import logprob as olp
from oracle import opd as oopd
from oracle import topk as otopk

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _bf16_logits(rows, T, V, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(rows, T, V, generator=g) * scale).to(torch.bfloat16)


# ------------------------------------------------------------------ teacher_topk


@pytest.mark.parametrize("V,k", [(151936, 8), (50, 5), (8, 8), (1001, 7), (16387, 64), (4096, 1), (20000, 33)])
def test_topk_matches_oracle(dev, V, k):
    from meshy_amd import topk

    z = _bf16_logits(2, 19, V, seed=V + k)
    ids, lps = topk.teacher_topk(z.to(dev), k)
    rids, rlps = otopk.teacher_topk(z, k)
    assert ids.dtype == torch.int64 and lps.dtype == torch.float32 and ids.shape == (2, 19, k)
    assert torch.equal(ids.cpu(), rids)
    assert (lps.cpu() - rlps).abs().max().item() <= TOL


def test_topk_many_ties_and_strided_view(dev):
    from meshy_amd import topk

    g = torch.Generator().manual_seed(2)
    # Integer-valued logits: long runs of equal values around the K-th rank.
    z = torch.randint(-3, 4, (2, 40, 3000), generator=g).float().to(torch.bfloat16)
    zd = z.to(dev)
    ids, lps = topk.teacher_topk(zd[:, 5:33, :], 16)
    rids, rlps = otopk.teacher_topk(z[:, 5:33, :], 16)
    assert torch.equal(ids.cpu(), rids)
    assert (lps.cpu() - rlps).abs().max().item() <= TOL
    # values agree with torch.topk's (whose tie order is unspecified)
    tv = torch.log_softmax(z[:, 5:33].float(), -1).topk(16, dim=-1).values
    assert (lps.cpu() - tv).abs().max().item() <= TOL


def _special_rows(V, seed):
    """Rows of [12, V] fp32 logits holding NaN, +inf and -inf in the places a
    streaming selection treats differently: the first tile (which sets the
    floor), the middle, the row's last chunks and elements, more NaNs than any
    K, and rows made only of them."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(12, V, generator=g) * 2.0
    nan, inf = float("nan"), float("inf")
    pick = lambda n: torch.randperm(V, generator=g)[:n]
    z[0, pick(1)] = nan                                   # one NaN anywhere
    z[1, [3, V // 2, V - 1]] = nan                        # first tile, middle, last element
    z[2, pick(min(100, V // 2))] = nan                    # more NaNs than K: ties by index
    z[3, [5, V - 2]] = inf
    z[3, V // 3] = nan                                    # NaN ranks above +inf
    z[4, :] = -inf
    z[4, [1, V // 4, V - 3]] = torch.tensor([0.5, -1.0, 0.5])
    z[4, V // 2] = nan                                    # -inf row with NaN and ties
    z[5, :] = nan                                         # all NaN
    z[6, 0:8] = nan                                       # a whole 16-byte chunk of NaN
    z[6, V - 5] = inf
    z[7, [V - 1, V - 2]] = inf                            # +inf only, in the row's tail
    z[8, :] = -inf                                        # all -inf
    z[9, :] = -inf
    z[9, V - 1] = nan                                     # NaN as the very last element
    z[10, pick(7)] = -inf                                 # a few -inf, no NaN
    # row 11 stays an ordinary row
    return z


def _assert_topk_like_oracle(ids, lps, rids, rlps, what):
    assert torch.equal(ids, rids), f"{what}: ids differ"
    assert torch.equal(torch.isnan(lps), torch.isnan(rlps)), f"{what}: NaN pattern differs"
    inf = torch.isinf(rlps)
    assert torch.equal(lps[inf], rlps[inf]), f"{what}: infinities differ"
    fin = torch.isfinite(rlps)
    if fin.any():
        assert (lps[fin] - rlps[fin]).abs().max().item() <= TOL, what


@pytest.mark.parametrize("V", [500, 151936])
@pytest.mark.parametrize("k", [1, 8, 64])
def test_topk_nan_and_inf_rows_match_oracle(dev, V, k):
    """torch.topk's order on rows with NaN and infinities: NaN ranks above
    +inf, NaNs among themselves by index; the log-probs follow
    torch.logsumexp (NaN for a row holding NaN, +inf for a row whose max is
    +inf).  Aligned rows (vector path) and a misaligned view (generic path)."""
    from meshy_amd import topk

    z = _special_rows(V, seed=V + k).to(torch.bfloat16).view(1, 12, V)
    ids, lps = topk.teacher_topk(z.to(dev), k)
    rids, rlps = otopk.teacher_topk(z, k)
    _assert_topk_like_oracle(ids.cpu(), lps.cpu(), rids, rlps, f"vector V={V} k={k}")
    # Known answers of the rules themselves.
    if k == 8:
        assert rids[0, 2, :8].tolist() == sorted(torch.nonzero(torch.isnan(z[0, 2].float())).flatten().tolist())[:8]
        assert rids[0, 3, :3].tolist() == [V // 3, 5, V - 2]
        assert rids[0, 5].tolist() == list(range(8))
    # Misaligned rows: one element in, so the rows start 2 bytes off 16.
    zp = torch.cat([torch.zeros(1, 12, 1, dtype=torch.bfloat16), z], dim=-1)
    view = zp.to(dev)[:, :, 1:]
    ids2, lps2 = topk.teacher_topk(view, k)
    _assert_topk_like_oracle(ids2.cpu(), lps2.cpu(), rids, rlps, f"generic V={V} k={k}")


def test_topk_matches_torch_topk_on_nan(dev):
    """The reference's own call, z.topk(k), on the row of the known answer
    [1, nan, 3, 2, nan, inf]: indices [1, 4, 5, 2]."""
    from meshy_amd import topk

    z = torch.tensor([[[1.0, float("nan"), 3.0, 2.0, float("nan"), float("inf"), 0.0, -1.0]]])
    ids, lps = topk.teacher_topk(z.to(torch.bfloat16).to(dev), 4)
    assert ids.cpu().flatten().tolist() == [1, 4, 5, 2]
    assert torch.equal(ids.cpu(), z.topk(4, dim=-1).indices)
    assert torch.isnan(lps.cpu()).all()  # logsumexp of a row holding NaN is NaN


def test_topk_row_with_plus_inf_matches_logsumexp(dev):
    """A row whose max is +inf: torch.logsumexp is +inf, so the reference's
    candidates get NaN (the +inf logit) and -inf (finite ones)."""
    from meshy_amd import topk

    g = torch.Generator().manual_seed(4)
    z = torch.randn(1, 3, 300, generator=g)
    z[0, 0, 17] = float("inf")
    z[0, 2, 250] = float("inf")
    z[0, 2, 3] = float("inf")   # two: the smaller index ranks first
    zb = z.to(torch.bfloat16)
    ids, lps = topk.teacher_topk(zb.to(dev), k=4)
    rids, rlps = otopk.teacher_topk(zb, 4)
    assert torch.equal(ids.cpu(), rids)
    got = lps.cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(rlps))
    inf = torch.isinf(rlps)
    assert inf[0, 0, 1:].all() and inf[0, 2, 2:].all() and torch.equal(got[inf], rlps[inf])
    fin = torch.isfinite(rlps)
    assert (got[fin] - rlps[fin]).abs().max().item() <= TOL


def test_topk_full_size_every_row(dev):
    """[16384, 151936] bf16, K = 8: every row against the oracle (1024 rows at
    a time, by the one-selection form of the stable sort), plus
    size-independent properties."""
    from meshy_amd import topk

    T, V, K = 16384, 151936, 8
    gen = torch.Generator(device=dev).manual_seed(1)
    z = torch.randn(1, T, V, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0
    ids, lps = topk.teacher_topk(z, K)
    assert ((ids >= 0) & (ids < V)).all()
    assert (lps <= 1e-6).all() and torch.isfinite(lps).all()
    assert (lps[..., :-1] >= lps[..., 1:]).all()  # sorted by value
    srt = ids.sort(dim=-1).values
    assert (srt[..., 1:] != srt[..., :-1]).all()  # distinct
    ids, lps = ids.cpu(), lps.cpu()
    worst = 0.0
    for a in range(0, T, 1024):
        rids, rlps = otopk.teacher_topk_by_threshold(z[:, a:a + 1024].cpu(), K)
        assert torch.equal(ids[:, a:a + 1024], rids), a
        worst = max(worst, (lps[:, a:a + 1024] - rlps).abs().max().item())
    print(f"Top-K [16384, 151936] every row: ids equal, max|dlogp|={worst:.2e}")
    assert worst <= TOL


def test_topk_rejects_bad_k(dev):
    from meshy_amd import topk

    z = _bf16_logits(1, 2, 100, seed=0).to(dev)
    with pytest.raises(ValueError):
        topk.teacher_topk(z, 65)
    with pytest.raises(ValueError):
        topk.teacher_topk(z, 0)


# ------------------------------------------------------------------ gather_logprobs


@pytest.mark.parametrize("V", [151936, 1001, 64])
def test_gather_fwd_bwd_matches_oracle(dev, V):
    from meshy_amd import topk

    z = _bf16_logits(2, 11, V, seed=V)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, V, (2, 11, 9), generator=g)
    ids[0, 0, 3] = ids[0, 0, 1]  # duplicate ids add their gradients
    ids[1, 2, :] = ids[1, 2, 0]
    zd = z.to(dev).requires_grad_(True)
    out = topk.gather_logprobs(zd, ids.to(dev))
    ref = otopk.gather_logprobs(z, ids)
    assert out.shape == (2, 11, 9) and (out.detach().cpu() - ref).abs().max().item() <= TOL
    w = torch.randn(2, 11, 9, generator=g)
    (out * w.to(dev)).sum().backward()
    zr = z.float().requires_grad_(True)
    (otopk.gather_logprobs(zr, ids) * w).sum().backward()
    got = zd.grad.float().cpu()
    bound = 4e-3 * w.abs().sum(-1).max().item()
    assert (got - zr.grad).abs().max().item() <= bound


def test_gather_no_grad_and_strided(dev):
    from meshy_amd import topk

    z = _bf16_logits(1, 30, 2048, seed=8)
    ids = torch.randint(0, 2048, (1, 10, 5), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        out = topk.gather_logprobs(z.to(dev)[:, 10:20], ids.to(dev))
    assert (out.cpu() - otopk.gather_logprobs(z[:, 10:20], ids)).abs().max().item() <= TOL


# ------------------------------------------------------------------ backward paths of K1b


@pytest.mark.parametrize("case", ["flat", "rows", "any"])
def test_logprob_backward_paths(dev, case):
    """The flat grid-stride pass (contiguous), the per-row pass (strided view) and
    the generic pass (odd V) against autograd of the reference's fp32 path."""
    from meshy_amd import logprob

    V = 999 if case == "any" else 4096
    z = _bf16_logits(2, 24, V, seed=21)
    y = torch.randint(0, V, (2, 24), generator=torch.Generator().manual_seed(2))
    y[0, 5] = -100
    g = torch.randn(2, 24, generator=torch.Generator().manual_seed(3))
    if case == "rows":
        # every other row of an interleaved copy: a view equal to z with stride_t = 2 V
        base = torch.stack([z, z], dim=2).reshape(2, 48, V).to(dev).requires_grad_(True)
        zd = base[:, ::2]
        assert zd.stride(1) == 2 * V and torch.equal(zd.detach().cpu(), z)
    else:
        base = zd = z.to(dev).requires_grad_(True)
    lp = logprob.logprobs_and_entropy(zd, y.to(dev))
    (lp * g.to(dev)).sum().backward()
    ref = olp.logprob_grad(z, y, g)
    got = (base.grad[:, ::2] if case == "rows" else base.grad).float().cpu()
    assert (got - ref).abs().max().item() <= 4e-3 * g.abs().max().item()
    assert got[0, 5].abs().max().item() == 0.0


def test_logprob_backward_flat_equals_rows_bitwise(dev):
    from meshy_amd import _lib, logprob

    V = 4096
    z = _bf16_logits(1, 64, V, seed=31).to(dev)
    y = torch.randint(0, V, (1, 64), generator=torch.Generator().manual_seed(1)).to(dev)
    lse = logprob.logsumexp_rows(z)
    g = torch.randn(1, 64, generator=torch.Generator().manual_seed(2)).to(dev)
    lib = _lib.load()
    outs = []
    strided = torch.stack([z, z], dim=2).reshape(1, 128, V)[:, ::2]
    assert torch.equal(strided, z) and strided.stride(1) == 2 * V
    for zz in (z, strided):
        grad = torch.empty(1, 64, V, dtype=torch.bfloat16, device=dev)
        ws = logprob.bwd_workspace(64, dev)
        rc = lib.meshy_logprob_bwd(zz.data_ptr(), 1, 64, V, zz.stride(0), zz.stride(1), y.data_ptr(),
                                   lse.data_ptr(), g.data_ptr(), grad.data_ptr(), ws.data_ptr(), ws.numel(),
                                   _lib.stream_of(dev))
        _lib.check(rc, "meshy_logprob_bwd")
        outs.append(grad)
    assert torch.equal(outs[0], outs[1])


# ------------------------------------------------------------------ forward_kl_topk


@pytest.mark.parametrize("clamps", [(None, None), (-10.0, 10.0), (-3.0, 0.5)])
def test_forward_kl_matches_oracle(dev, clamps):
    from meshy_amd import topk

    g = torch.Generator().manual_seed(6)
    s = torch.log_softmax(torch.randn(3, 17, 8, generator=g) * 3, -1)
    t = torch.log_softmax(torch.randn(3, 17, 8, generator=g) * 3, -1)
    s[0, 0, 0] = -40.0  # below the clamp
    kw = dict(log_prob_min_clamp=clamps[0], loss_max_clamp=clamps[1])
    sd = s.to(dev).requires_grad_(True)
    kl = topk.forward_kl_topk(sd, t.to(dev), **kw)
    sr = s.clone().requires_grad_(True)
    rk = otopk.forward_kl_topk(sr, t, **kw)
    assert kl.shape == (3, 17) and (kl.detach().cpu() - rk).abs().max().item() <= TOL
    w = torch.randn(3, 17, generator=g)
    (kl * w.to(dev)).sum().backward()
    (rk * w).sum().backward()
    assert (sd.grad.cpu() - sr.grad).abs().max().item() <= 1e-5


# ------------------------------------------------------------------ Teacher columns in the pack


def _opd_sample(L, K, seed, V=1000):
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randint(0, V, (L,), generator=g)
    mask = torch.ones(L)
    mask[: max(1, L // 4)] = 0
    return {
        "tokens": tokens,
        "logprobs": -torch.rand(L, generator=g),
        "mask_assistant": mask,
        "advantage": torch.tensor(0.0),
        "teacher_topk_ids": torch.randint(0, V, (L, K), generator=g),
        "teacher_topk_logprobs": -torch.rand(L, K, generator=g) * 5,
    }


@pytest.mark.parametrize("ids", ["int64", "int32", "int64_wide", "int64_strided", "int64_general",
                                 "int64_wide_general"])
@pytest.mark.parametrize("layout", ["padded", "packed"])
def test_teacher_layout_matches_oracle(dev, layout, ids, monkeypatch):
    """Teacher ids as int64 (the Teacher's dtype, staged as int32), as int32, as
    int64 with one value int32 cannot hold (staged as int64 after the
    narrowing's check fails) and as strided int64 views; the "general" cases
    carry per-token advantages, which take the other columns through the
    Python staging instead of the one-pass native one."""
    from meshy_amd import batch as B
    from meshy_amd import opd
    from meshy_amd.batch import ADVANTAGE_TOKENS
    from meshy_amd.plan import MicroPlan

    monkeypatch.setattr(B, "_NARROW_MIN_TEACHER_IDS", 0)  # narrow these few ids too
    K = 8
    samples = [_opd_sample(L, K, i) for i, L in enumerate([37, 64, 5, 120, 90])]
    for i, s in enumerate(samples):
        if ids == "int32":
            s["teacher_topk_ids"] = s["teacher_topk_ids"].to(torch.int32)
        elif ids == "int64_strided":
            s["teacher_topk_ids"] = torch.cat([s["teacher_topk_ids"], -s["teacher_topk_ids"]], 1)[:, :K]
        if ids.endswith("_general"):
            s[ADVANTAGE_TOKENS] = torch.linspace(-1, 1, s["tokens"].numel()) + i
    if ids.startswith("int64_wide"):
        samples[4]["teacher_topk_ids"][7, 3] = 2**33 + 11  # within sample 4's first 60 positions
    micros = [MicroPlan((1, 0, 2), 128 if layout == "packed" else 64, (64, 37, 5)),
              MicroPlan((3, 4), 256 if layout == "packed" else 120, (120, 60)),  # sample 4 truncated
              MicroPlan((), 64, ())]  # filler
    mbs = opd.build_topk_micro_batches(samples, micros, layout=layout, device=dev, need_rollout_lp=True)
    for mb, m in zip(mbs, micros):
        rids, rlps = oopd.layout_teacher_topk(samples, m.sample_idx, m.seq_len, m.doc_lens, layout=layout)
        assert torch.equal(mb.teacher_topk_ids.cpu(), rids)
        assert torch.equal(mb.teacher_topk_logprobs.cpu(), rlps)
    ids, lps = opd.layout_teacher_topk(samples, micros[0], layout=layout, device=dev)
    back = opd.split_teacher_topk(ids, micros[0], layout=layout)
    for j, i in enumerate(micros[0].sample_idx):
        assert torch.equal(back[j].cpu(), samples[i]["teacher_topk_ids"][:micros[0].doc_lens[j]].long())


def test_teacher_layout_short_rows_raise(dev):
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan

    s = _opd_sample(6, 3, 1)
    s["teacher_topk_ids"] = s["teacher_topk_ids"][:2]
    with pytest.raises(ValueError, match="Teacher seq_len"):
        opd.layout_teacher_topk([s], MicroPlan((0,), 4, (4,)), layout="padded", device=dev)
    assert opd.infer_top_k([_opd_sample(2, 3, 0)]) == 3


# ------------------------------------------------------------------ the distillation loss


def _stub(per_token, lp_min=-10.0, loss_max=10.0, model=None):
    return NS(calculate_per_token_loss=per_token, log_prob_min_clamp=lp_min, loss_max_clamp=loss_max,
              sharder=None, parallel_dims=NS(cp=1), model_parts=[model], _LOGPROB_CHUNK=1024)


@pytest.mark.parametrize("per_token", [True, False])
@pytest.mark.parametrize("clamps", [(-10.0, 10.0), (None, None), (-2.0, 1.0)])
@pytest.mark.parametrize("rollout", [True, False])
def test_distill_from_gathered_matches_oracle(dev, per_token, clamps, rollout):
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan, MiniPlan

    K = 8
    samples = [_opd_sample(L, K, 10 + i) for i, L in enumerate([300, 41, 700, 2, 129])]
    micro = MicroPlan((0, 1, 2, 3, 4), 1280, (300, 41, 700, 2, 129))
    mb = opd.build_topk_micro_batches(samples, [micro], layout="packed", device=dev,
                                      need_rollout_lp=rollout)[0]
    g = torch.Generator().manual_seed(7)
    S = micro.seq_len
    gathered = torch.log_softmax(torch.randn(1, S, K + 1, generator=g) * 4, -1)
    gathered[0, 10, :3] = -30.0  # below the lp clamp
    mini = MiniPlan((micro,), 6, int(mb.mask.sum().item()) + 3, (0,))
    stub = _stub(per_token, *clamps)
    gd = gathered.to(dev).requires_grad_(True)
    loss, sums = opd.distill_from_gathered(stub, gd, mb, mini)
    gr = gathered.clone().requires_grad_(True)
    rl, rs = oopd.distill_loss(gr, mb.teacher_topk_logprobs.cpu(), mb.mask.cpu(), mb.doc_ids.cpu(), mb.n_docs,
                               rollout_lp=mb.rollout_logprobs.cpu() if rollout else None,
                               n_docs_global=mini.n_docs_global, n_tokens_global=mini.n_tokens_global,
                               per_token_loss=per_token, log_prob_min_clamp=clamps[0], loss_max_clamp=clamps[1])
    assert abs(float(loss.detach()) - float(rl.detach())) <= TOL
    assert set(sums) == set(rs)
    for key in rs:
        want = float(rs[key])
        assert abs(float(sums[key]) - want) <= TOL + 1e-5 * abs(want), key
    loss.backward()
    rl.backward()
    assert (gd.grad.cpu() - gr.grad).abs().max().item() <= 1e-6
    m = opd.reduce_distill_metrics(stub, sums)
    rm = oopd.reduce_distill_metrics(rs)
    for key in rm:
        assert m[key] == pytest.approx(rm[key], abs=TOL), key


@pytest.mark.parametrize("per_token", [True, False])
def test_distill_doc_ids_in_any_order(dev, per_token):
    """The tokens of a packed micro shuffled (so the document ids decrease):
    the loss, its sums and the gradient match the oracle's index_add_ over the
    shuffled order, as the reference accepts any order."""
    from types import SimpleNamespace as NS

    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan, MiniPlan

    K = 8
    samples = [_opd_sample(L, K, 40 + i) for i, L in enumerate([300, 41, 700, 129])]
    micro = MicroPlan((0, 1, 2, 3), 1280, (300, 41, 700, 129))
    mb = opd.build_topk_micro_batches(samples, [micro], layout="packed", device=dev, need_rollout_lp=True)[0]
    S = micro.seq_len
    g = torch.Generator().manual_seed(9)
    order = torch.randperm(S, generator=g).to(dev)
    sh = NS(teacher_topk_logprobs=mb.teacher_topk_logprobs[:, order].contiguous(),
            mask=mb.mask[:, order].contiguous(), rollout_logprobs=mb.rollout_logprobs[:, order].contiguous(),
            doc_ids=mb.doc_ids[:, order].contiguous(), n_docs=mb.n_docs)
    gathered = torch.log_softmax(torch.randn(1, S, K + 1, generator=g) * 4, -1)
    mini = MiniPlan((micro,), 5, int(mb.mask.sum().item()), (0,))
    stub = _stub(per_token)
    gd = gathered.to(dev).requires_grad_(True)
    loss, sums = opd.distill_from_gathered(stub, gd, sh, mini)
    gr = gathered.clone().requires_grad_(True)
    rl, rs = oopd.distill_loss(gr, sh.teacher_topk_logprobs.cpu(), sh.mask.cpu(), sh.doc_ids.cpu(), sh.n_docs,
                               rollout_lp=sh.rollout_logprobs.cpu(), n_docs_global=mini.n_docs_global,
                               n_tokens_global=mini.n_tokens_global, per_token_loss=per_token,
                               log_prob_min_clamp=-10.0, loss_max_clamp=10.0)
    assert abs(float(loss.detach()) - float(rl.detach())) <= TOL
    for key in rs:
        want = float(rs[key])
        assert abs(float(sums[key]) - want) <= TOL + 1e-5 * abs(want), key
    loss.backward()
    rl.backward()
    assert (gd.grad.cpu() - gr.grad).abs().max().item() <= 1e-6


def test_distill_inputs_cache_follows_edits(dev):
    """A second loss over one micro-batch reuses its flattened inputs; an
    in-place edit of the Teacher's log-probs or the mask, other clamps or a new
    mini-batch denominator rebuilds them, so every call matches the oracle."""
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan, MiniPlan

    K = 4
    samples = [_opd_sample(L, K, 40 + i) for i, L in enumerate([90, 300, 17])]
    micro = MicroPlan((0, 1, 2), 512, (90, 300, 17))
    mb = opd.build_topk_micro_batches(samples, [micro], layout="packed", device=dev, need_rollout_lp=True)[0]
    gathered = torch.log_softmax(torch.randn(1, 512, K + 1, generator=torch.Generator().manual_seed(5)) * 3, -1)

    def check(stub, n_tok):
        mini = MiniPlan((micro,), 3, n_tok, (0,))
        gd = gathered.to(dev).requires_grad_(True)
        loss, sums = opd.distill_from_gathered(stub, gd, mb, mini)
        loss.backward()
        gr = gathered.clone().requires_grad_(True)
        rl, rs = oopd.distill_loss(gr, mb.teacher_topk_logprobs.cpu(), mb.mask.cpu(), mb.doc_ids.cpu(), mb.n_docs,
                                   rollout_lp=mb.rollout_logprobs.cpu(), n_docs_global=3, n_tokens_global=n_tok,
                                   per_token_loss=stub.calculate_per_token_loss,
                                   log_prob_min_clamp=stub.log_prob_min_clamp, loss_max_clamp=stub.loss_max_clamp)
        rl.backward()
        assert abs(float(loss.detach()) - float(rl.detach())) <= TOL
        for key in rs:
            want = float(rs[key])
            assert abs(float(sums[key]) - want) <= TOL + 1e-5 * abs(want), key
        assert (gd.grad.cpu() - gr.grad).abs().max().item() <= 1e-6
        return mb.__dict__["_meshy_distill_inputs"][1]

    n_tok = int(mb.mask.sum().item())
    stub = _stub(True)
    first = check(stub, n_tok)
    assert check(stub, n_tok) is first  # reused
    mb.teacher_topk_logprobs.add_(-0.25)  # in place: a new version
    second = check(stub, n_tok)
    assert second is not first
    mb.mask[0, 5:40] = 0.0
    third = check(stub, int(mb.mask.sum().item()))
    assert third is not second
    assert check(_stub(True, -2.0, 1.0), int(mb.mask.sum().item())) is not third
    assert check(_stub(False), 7 * int(mb.mask.sum().item())) is not third


def test_distill_loss_drop_in_end_to_end(dev):
    """_distill_loss with a stub model: bf16 logits -> gather of K + 1 ids -> fused
    loss; loss, sums and d loss / d logits against the reference chain on CPU."""
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan, MiniPlan

    K, V = 8, 5000
    samples = [_opd_sample(L, K, 20 + i, V=V) for i, L in enumerate([200, 77, 33])]
    micro = MicroPlan((0, 1, 2), 320, (200, 77, 33))
    mb = opd.build_topk_micro_batches(samples, [micro], layout="packed", device=dev, need_rollout_lp=True)[0]
    z = _bf16_logits(1, 320, V, seed=3)
    zd = z.to(dev).requires_grad_(True)
    model = lambda ids, positions=None, attention_masks=None: zd  # noqa: E731
    mini = MiniPlan((micro,), 3, int(mb.mask.sum().item()), (0,))
    for per_token in (True, False):
        zd.grad = None
        stub = _stub(per_token, model=model)
        loss, sums = opd.distill_loss(stub, mb, mini)
        loss.backward()
        zr = z.float().requires_grad_(True)
        ids = torch.cat([mb.teacher_topk_ids.cpu(), mb.labels.cpu().unsqueeze(-1)], -1)
        gathered = otopk.gather_logprobs(zr, ids)
        rl, rs = oopd.distill_loss(gathered, mb.teacher_topk_logprobs.cpu(), mb.mask.cpu(), mb.doc_ids.cpu(),
                                   mb.n_docs, rollout_lp=mb.rollout_logprobs.cpu(), n_docs_global=3,
                                   n_tokens_global=mini.n_tokens_global, per_token_loss=per_token)
        rl.backward()
        assert abs(float(loss.detach()) - float(rl.detach())) <= TOL
        for key in rs:
            want = float(rs[key])
            assert abs(float(sums[key]) - want) <= TOL + 1e-5 * abs(want), key
        gmax = zr.grad.abs().max().item()
        assert (zd.grad.float().cpu() - zr.grad).abs().max().item() <= 4e-3 * max(gmax, 1e-6) + 1e-7


def test_distill_deterministic(dev):
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan, MiniPlan

    K = 4
    samples = [_opd_sample(L, K, 40 + i) for i, L in enumerate([1000, 1, 333, 4000])]
    micro = MicroPlan((0, 1, 2, 3), 5376, (1000, 1, 333, 4000))
    mb = opd.build_topk_micro_batches(samples, [micro], layout="packed", device=dev, need_rollout_lp=True)[0]
    gathered = torch.log_softmax(torch.randn(1, micro.seq_len, K + 1, generator=torch.Generator().manual_seed(1)),
                                 -1).to(dev)
    mini = MiniPlan((micro,), 4, 4000, (0,))
    a = opd.distill_from_gathered(_stub(False), gathered, mb, mini)
    b = opd.distill_from_gathered(_stub(False), gathered, mb, mini)
    assert torch.equal(a[0], b[0]) and all(torch.equal(a[1][k], b[1][k]) for k in a[1])


# ------------------------------------------------------------------ randomised sweeps


def _rand_case(seed):
    g = torch.Generator().manual_seed(1000 + seed)
    rows = int(torch.randint(1, 4, (1,), generator=g))
    T = int(torch.randint(1, 24, (1,), generator=g))
    V = int(torch.randint(1, 40000, (1,), generator=g))
    scale = [0.01, 1.0, 8.0, 100.0][seed % 4]
    z = torch.randn(rows, T, V, generator=g) * scale
    if seed % 3 == 0:
        z = torch.round(z * 2) / 2  # coarse values: many ties
    return g, z.to(torch.bfloat16), V


@pytest.mark.parametrize("seed", range(16))
def test_topk_random_sweep(dev, seed):
    from meshy_amd import topk

    g, z, V = _rand_case(seed)
    k = int(torch.randint(1, min(64, V) + 1, (1,), generator=g))
    ids, lps = topk.teacher_topk(z.to(dev), k)
    rids, rlps = otopk.teacher_topk(z, k)
    assert torch.equal(ids.cpu(), rids), (z.shape, k)
    assert (lps.cpu() - rlps).abs().max().item() <= TOL


# Vocabularies whose chunks of 8 left after the full tiles (2048 chunks per
# tile for K <= 16, 1024 above) make the row's last tile 4 to 8 loads per
# thread deep, with and without full tiles before it.
@pytest.mark.parametrize("V,k", [(24384, 8), (8800, 5), (43968, 16), (13600, 1), (32760, 8), (16192, 40)])
def test_topk_deep_row_tails(dev, V, k):
    from meshy_amd import topk

    g = torch.Generator().manual_seed(V)
    z = torch.randn(1, 4, V, generator=g) * 3
    z[0, 1] = torch.round(z[0, 1])  # many ties, broken by index
    z[0, 2, -7:] = z[0, 2].max() + 1  # the row's best values in its last chunk
    z = z.to(torch.bfloat16)
    ids, lps = topk.teacher_topk(z.to(dev), k)
    rids, rlps = otopk.teacher_topk(z, k)
    assert torch.equal(ids.cpu(), rids), (V, k)
    assert (lps.cpu() - rlps).abs().max().item() <= TOL


@pytest.mark.parametrize("seed", range(12))
def test_gather_random_sweep(dev, seed):
    from meshy_amd import topk

    g, z, V = _rand_case(seed + 50)
    rows, T, _ = z.shape
    n = int(torch.randint(1, 20, (1,), generator=g))
    ids = torch.randint(0, V, (rows, T, n), generator=g)
    ids[..., -1] = ids[..., 0]  # a duplicate in every row
    drop = torch.rand(rows, T, n, generator=g) < 0.1
    ids = torch.where(drop, torch.full_like(ids, -100), ids)
    out = topk.gather_logprobs(z.to(dev), ids.to(dev)).cpu()
    ref = otopk.gather_logprobs(z, ids.clamp(min=0))
    ref = torch.where(drop, torch.zeros_like(ref), ref)  # -100: 0, like cross_entropy's ignore_index
    assert (out - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("seed", range(8))
def test_random_teacher_layouts_match_oracle(dev, seed):
    """Random samples (empty and one-token ones among them) with Teacher columns
    of width 1, 3 or 8 in random micros, both layouts: the Teacher tensors
    equal the oracle's layout."""
    from meshy_amd import opd
    from meshy_amd.plan import MicroPlan

    rng = np.random.default_rng(500 + seed)
    K = int(rng.choice([1, 3, 8]))
    n = int(rng.integers(1, 24))
    lengths = rng.integers(0, 200, n)
    lengths[rng.random(n) < 0.15] = 1
    samples = [_opd_sample(int(L), K, 10 * seed + i, V=151936) for i, L in enumerate(lengths)]
    for layout in ("packed", "padded"):
        seq = int(rng.choice([32, 128, 256]))
        micros, cur, lens, used = [], [], [], 0
        for i in rng.permutation(n).tolist():
            take = min(int(lengths[i]), seq)
            if ((used + take > seq) if layout == "packed" else len(cur) == 3) and cur:
                micros.append(MicroPlan(tuple(cur), seq, tuple(lens)))
                cur, lens, used = [], [], 0
            cur.append(i)
            lens.append(take)
            used += take
        if cur:
            micros.append(MicroPlan(tuple(cur), seq, tuple(lens)))
        micros.append(MicroPlan((), seq, ()))
        mbs = opd.build_topk_micro_batches(samples, micros, layout=layout, device=dev, need_rollout_lp=True)
        for mb, m in zip(mbs, micros):
            rids, rlps = oopd.layout_teacher_topk(samples, m.sample_idx, m.seq_len, m.doc_lens, layout=layout)
            assert torch.equal(mb.teacher_topk_ids.cpu(), rids)
            assert torch.equal(mb.teacher_topk_logprobs.cpu(), rlps)

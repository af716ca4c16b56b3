"""Critic-side reductions, rollout statistics and the wire-format ingest against
the oracle.

Bars: per-sequence means, row values and the clipped value error within 1e-5
(fp32), window sums within 1e-6 relative, gradients 1e-6; rollout metrics within
1e-6 relative (sample-level values exact); packs built from wire columns equal
packs built from samples bit for bit.
"""

import math

import numpy as np
import pytest
import torch

from oracle import critic as ocritic
from oracle import rollout_metrics as orm

pytestmark = pytest.mark.gpu


def _critic_batch(rows, S, seed, lo=3):
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lo, S + 1, (rows,), generator=g)
    mask = torch.zeros(rows, S)
    for j, L in enumerate(lengths.tolist()):
        p = int(torch.randint(1, max(2, L // 2), (1,), generator=g))
        mask[j, p:L] = 1.0
    values = torch.randn(rows, S, generator=g)
    returns = torch.randn(rows, S, generator=g)
    doc = torch.arange(rows).unsqueeze(1).expand(rows, S).contiguous()
    return values, returns, mask, doc


@pytest.mark.parametrize("rows,S", [(7, 300), (64, 4096), (1, 1)])
def test_per_sequence_mean_padded(dev, rows, S):
    from meshy_amd import critic

    adv, _, mask, doc = _critic_batch(rows, S, seed=rows + S, lo=1)
    mask[0] = 0.0  # a document without masked tokens -> 0
    out = critic.advantages_to_per_sequence((adv * mask).to(dev), mask.to(dev), doc.to(dev), rows)
    ref = ocritic.advantages_to_per_sequence(adv * mask, mask, doc, rows)
    assert out.shape == (rows,) and (out.cpu() - ref).abs().max().item() <= 1e-5


def test_per_sequence_mean_packed_with_padding_slot(dev):
    from meshy_amd import critic

    g = torch.Generator().manual_seed(3)
    lens = [5, 1, 300, 77, 0, 2048]
    ids = torch.cat([torch.full((L,), d) for d, L in enumerate(lens)] + [torch.full((40,), len(lens))])
    n = ids.numel()
    adv = torch.randn(1, n, generator=g)
    mask = (torch.rand(1, n, generator=g) > 0.3).float()
    out = critic.advantages_to_per_sequence(adv.to(dev), mask.to(dev), ids.view(1, -1).to(dev), len(lens))
    ref = ocritic.advantages_to_per_sequence(adv, mask, ids.view(1, -1), len(lens))
    assert (out.cpu() - ref).abs().max().item() <= 1e-5


def test_per_sequence_mean_takes_doc_ids_in_any_order(dev):
    """Ids in any order (the reference sums with index_add_): the mean of each
    document's masked advantages, against the oracle."""
    from meshy_amd import critic

    ids = torch.tensor([[0, 0, 2, 1, 1]])
    adv = torch.tensor([[1.0, 2.0, 3.0, 4.0, 5.0]])
    mask = torch.tensor([[1.0, 1.0, 1.0, 0.0, 1.0]])
    out = critic.advantages_to_per_sequence(adv.to(dev), mask.to(dev), ids.to(dev), 3)
    assert torch.equal(out.cpu(), torch.tensor([1.5, 5.0, 3.0]))
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, 51, (3, 4000), generator=g)
    adv = torch.randn(3, 4000, generator=g)
    mask = (torch.rand(3, 4000, generator=g) > 0.3).float()
    out = critic.advantages_to_per_sequence(adv.to(dev), mask.to(dev), ids.to(dev), 50)
    ref = ocritic.advantages_to_per_sequence(adv, mask, ids, 50)
    assert (out.cpu() - ref).abs().max().item() <= 1e-5


@pytest.mark.parametrize("bf16", [False, True])
def test_accumulator_matches_oracle(dev, bf16):
    from meshy_amd import critic

    acc, ref = critic.Accumulator(), ocritic.Accumulator()
    # S = 500 and 5003 start odd rows off a multiple of 8 (head, body, tail); 4096
    # rows run the two-groups-in-flight loop.
    for k, (rows, S) in enumerate([(6, 500), (3, 4096), (1, 17), (4, 5003)]):
        v, r, m, _ = _critic_batch(rows, S, seed=10 + k)
        v = v.to(torch.bfloat16) if bf16 else v
        rewards = torch.rand(rows)
        groups = torch.arange(rows) // 2 + 100 * k
        if k % 2:
            # rewards as a strided device view, fp64; group ids as int32 on the host
            rw = torch.stack([rewards.double(), -rewards.double()], 1).to(dev)[:, 0]
            acc.update(v.to(dev), r.to(dev), m.to(dev), rw, groups.to(torch.int32))
        else:
            acc.update(v.to(dev), r.to(dev), m.to(dev), rewards.to(dev), groups.to(dev))
        ref.update(v, r, m, rewards, groups)
    st, rs = acc.state, ref.state
    for key in ("n_tokens", "sum_r", "sum_r2", "sum_d", "sum_d2"):
        want = rs[key]
        assert abs(getattr(st, key) - want) <= 1e-6 * max(1.0, abs(want)) + 1e-4, key
    assert np.allclose(st.row_value, rs["row_value"], atol=1e-5)
    assert st.row_reward == pytest.approx(rs["row_reward"]) and st.row_group == rs["row_group"]


def _gauge_window(rows=24, span=40, seed=0):
    """The window of the reference's gauge tests (test_critic_batching.py:145-154)."""
    g = torch.Generator().manual_seed(seed)
    mask = torch.zeros(rows, span)
    for j in range(rows):
        mask[j, 3 + j % 5:] = 1.0
    returns = torch.randn(rows, span, generator=g) * mask
    values = (returns + 0.3 * torch.randn(rows, span, generator=g)) * mask
    rewards = (torch.rand(rows, generator=g) > 0.5).float()
    groups = torch.arange(rows) // 4
    return values, returns, mask, rewards, groups


def _diag_dict(d):
    return d.as_dict()


def _odd_window(rows, S, seed, *, frac=False, bf16=False):
    """Rows in shuffled group order with arbitrary ids, all-correct and
    all-incorrect groups, tied row values, and (frac) a fractional mask."""
    g = torch.Generator().manual_seed(seed)
    mask = (torch.rand(rows, S, generator=g) > 0.3).float()
    mask[:, : S // 5] = 0.0
    if frac:
        mask = mask * torch.rand(rows, S, generator=g)
    mask[rows // 3] = 0.0  # a row with no token
    returns = torch.randn(rows, S, generator=g)
    values = returns + 0.5 * torch.randn(rows, S, generator=g)
    values[rows // 2] = 0.25  # ties across rows
    values[rows // 2 + 1] = 0.25
    groups = torch.randint(0, max(1, rows // 4), (rows,), generator=g) * 13 - 40
    rewards = (torch.rand(rows, generator=g) > 0.5).float()
    rewards[groups == groups[0]] = 1.0  # an all-correct group
    if bf16:
        values = values.to(torch.bfloat16)
    return values, returns, mask, rewards, groups


@pytest.mark.parametrize("rows,S,frac,bf16", [(24, 40, False, False), (37, 300, True, False), (64, 1000, False, True),
                                             (300, 129, True, True), (5, 5003, True, True), (3, 8200, False, False)])
def test_critic_diagnostics_matches_oracle(dev, rows, S, frac, bf16):
    from meshy_amd import critic

    v, r, m, rew, grp = _odd_window(rows, S, seed=rows + S, frac=frac, bf16=bf16)
    got = critic.critic_diagnostics(v.to(dev), r.to(dev), m.to(dev), rew.to(dev), grp.to(dev)).as_dict()
    want = ocritic.critic_diagnostics(v.float(), r, m, rew, grp)
    assert ocritic.same_gauges(got, want, rel=1e-4, abs_=1e-5), (got, want)
    assert got["n_rows"] == want["n_rows"] and got["n_prompts"] == want["n_prompts"]
    assert got["n_tokens"] == want["n_tokens"] or frac  # int() of a fractional sum may round apart


@pytest.mark.parametrize("bf16", [False, True])
def test_critic_window_sums_unaligned_storage(dev, bf16):
    """Arrays one element off a 16-byte boundary take the element-by-element
    path of the row pass: the same gauges as the aligned copies, and the
    oracle's.  S = 5003 runs the aligned copies through the head, the loop of
    two groups of 8 per thread in flight, the last single group and the tail."""
    from meshy_amd import critic

    rows, S = 4, 5003
    v, r, m, rew, grp = _odd_window(rows, S, seed=77, frac=True, bf16=bf16)

    def shifted(x):
        buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=dev)
        buf[1:] = x.reshape(-1).to(dev)
        out = buf[1:].view(rows, S)
        assert out.data_ptr() % 16 != 0
        return out

    aligned = critic.critic_diagnostics(v.to(dev), r.to(dev), m.to(dev), rew.to(dev), grp.to(dev)).as_dict()
    off = critic.critic_diagnostics(shifted(v), shifted(r), shifted(m), rew.to(dev), grp.to(dev)).as_dict()
    want = ocritic.critic_diagnostics(v.float(), r, m, rew, grp)
    assert ocritic.same_gauges(aligned, want, rel=1e-4, abs_=1e-5), (aligned, want)
    assert ocritic.same_gauges(off, aligned, rel=1e-6, abs_=1e-9), (off, aligned)


def test_critic_diagnostics_degenerate_windows(dev):
    """NaN where the reference gives NaN: one prompt (Pearson), no prompt with
    both classes (AUC), constant returns (variance ratio)."""
    from meshy_amd import critic

    v, r, m, rew, _ = _odd_window(12, 64, seed=5)
    one = torch.zeros(12, dtype=torch.long)
    d = critic.critic_diagnostics(v.to(dev), r.to(dev), m.to(dev), rew.to(dev), one.to(dev))
    assert math.isnan(d.prompt_pearson) and d.n_prompts == 1
    d = critic.critic_diagnostics(v.to(dev), r.to(dev), m.to(dev), torch.ones(12, device=dev), one.to(dev))
    assert math.isnan(d.critic_auc)
    d = critic.critic_diagnostics(v.to(dev), torch.full_like(r, 0.5).to(dev), m.to(dev), rew.to(dev), one.to(dev))
    assert math.isnan(d.critic_var_ratio)
    want = ocritic.critic_diagnostics(v, torch.full_like(r, 0.5), m, rew, one)
    assert math.isnan(want["critic_var_ratio"])
    assert "within_prompt_auc=" in str(d) and "[12 rows / 1 prompts /" in str(d)


def test_diagnostics_from_states_match_whole_window(dev):
    """test_critic_batching.py:158-213 through this library: device
    accumulators over 5-row micro-batches and an interleaved two-rank split give
    the gauges of critic_diagnostics on the whole window (0/1 mask), and the
    oracle's diagnostics_from_states on the same states."""
    from meshy_amd import critic

    for seed in (0, 1, 2):
        w = _gauge_window(seed=seed)
        want = critic.critic_diagnostics(*(x.to(dev) for x in w)).as_dict()
        assert ocritic.same_gauges(want, ocritic.critic_diagnostics(*w), rel=1e-5, abs_=1e-6)
        stream = critic.Accumulator()
        for lo in range(0, 24, 5):
            stream.update(*(x[lo:lo + 5].to(dev) for x in w))
        got = critic.diagnostics_from_states([stream.state]).as_dict()
        assert ocritic.same_gauges(got, want, rel=1e-5, abs_=1e-6), (got, want)
        states = []
        for rank in range(2):
            sel = torch.arange(rank, 24, 2)
            acc = critic.Accumulator()
            acc.update(*(x[sel].to(dev) for x in w))
            states.append(acc.state)
        got = critic.diagnostics_from_states(states).as_dict()
        assert ocritic.same_gauges(got, want, rel=1e-5, abs_=1e-6), (got, want)
        assert got["n_rows"] == 24 and got["n_tokens"] == want["n_tokens"]
    with pytest.raises(ValueError, match="no masked tokens"):
        critic.diagnostics_from_states([critic.AccumulatorState()])


@pytest.mark.parametrize("n", [1, 2, 65, 1000, 4097])
def test_group_gauges_match_oracle(dev, n):
    """AUC and Pearson over n rows with arbitrary, unsorted group ids, tied
    values and NaN values (they pair but never win)."""
    from meshy_amd import critic

    g = torch.Generator().manual_seed(n)
    vals = torch.round(torch.randn(n, generator=g) * 4) / 4
    if n > 10:
        vals[3] = float("nan")
    rew = torch.rand(n, generator=g)
    grp = torch.randint(-3, max(1, n // 6), (n,), generator=g) * 1000003
    want_auc = ocritic.within_prompt_auc(vals, rew >= 0.5, grp)
    want_r = ocritic.prompt_pearson(vals[~vals.isnan()], rew[~vals.isnan()], grp[~vals.isnan()])
    got_auc = critic.within_prompt_auc(vals.to(dev), (rew >= 0.5).to(dev), grp.to(dev))
    assert (math.isnan(want_auc) and math.isnan(got_auc)) or got_auc == pytest.approx(want_auc, abs=1e-12)
    if n <= 10:
        got_r = critic.prompt_pearson(vals.to(dev), rew.to(dev), grp.to(dev))
        assert (math.isnan(want_r) and math.isnan(got_r)) or got_r == pytest.approx(want_r, abs=1e-5)
    else:
        # a NaN value makes its group's mean NaN, and so the correlation
        assert math.isnan(critic.prompt_pearson(vals.to(dev), rew.to(dev), grp.to(dev)))
        ok = ~vals.isnan()
        got_r = critic.prompt_pearson(vals[ok].to(dev), rew[ok].to(dev), grp[ok].to(dev))
        assert (math.isnan(want_r) and math.isnan(got_r)) or got_r == pytest.approx(want_r, abs=1e-5)


def test_variance_reduction_and_calibration_gap(dev):
    from meshy_amd import critic

    v, r, m, _, _ = _odd_window(40, 200, seed=9, frac=True)
    assert critic.variance_reduction(v.to(dev), r.to(dev), m.to(dev)) == pytest.approx(
        ocritic.variance_reduction(v, r, m), rel=1e-5)
    assert critic.calibration_gap(v.to(dev), r.to(dev), m.to(dev)) == pytest.approx(
        ocritic.calibration_gap(v, r, m), rel=1e-5, abs=1e-7)
    assert math.isnan(critic.variance_reduction(v.to(dev), r.to(dev), torch.zeros_like(m).to(dev)))


def _sums(states):
    return {k: sum(getattr(s, k) for s in states) for k in ("n_tokens", "sum_r", "sum_r2", "sum_d", "sum_d2")}


def test_accumulator_streaming_split_and_filler_rows(dev):
    """test_critic_batching.py:158-212 on the states the gauges are built from:
    5-row micro-batches, an interleaved two-rank split and all-zero-mask filler
    rows give the window's sums (and its rows, in the split's order)."""
    from meshy_amd import critic

    w = [x.to(dev) for x in _gauge_window(seed=1)]
    whole = critic.Accumulator()
    whole.update(*w)
    want = _sums([whole.state])
    assert want["n_tokens"] == float(w[2].sum().item())

    def close(got):
        for k, v in want.items():
            assert got[k] == pytest.approx(v, rel=1e-5, abs=1e-6), k

    stream = critic.Accumulator()
    for lo in range(0, 24, 5):
        stream.update(*(x[lo:lo + 5] for x in w))
    close(_sums([stream.state]))
    assert stream.state.row_value == pytest.approx(whole.state.row_value, abs=1e-6)
    assert stream.state.row_group == whole.state.row_group

    ranks = []
    for rank in range(2):
        sel = torch.arange(rank, 24, 2, device=dev)
        acc = critic.Accumulator()
        acc.update(*(x[sel] for x in w))
        ranks.append(acc.state)
    close(_sums(ranks))
    assert sorted(x for s in ranks for x in s.row_group) == sorted(whole.state.row_group)
    assert sorted(x for s in ranks for x in s.row_value) == pytest.approx(sorted(whole.state.row_value), abs=1e-6)

    filled = critic.Accumulator()
    filled.update(*w)
    v, r, m, rw, gr = w
    filled.update(torch.randn_like(v[:3]), torch.randn_like(r[:3]), torch.zeros_like(m[:3]), rw[:3], gr[:3])
    close(_sums([filled.state]))
    assert filled.state.row_value[24:] == [0.0, 0.0, 0.0]


@pytest.mark.parametrize("clip", [None, 0.2])
def test_clipped_value_error_fwd_bwd(dev, clip):
    from meshy_amd import critic

    g = torch.Generator().manual_seed(5)
    v = torch.randn(4, 1000, generator=g)
    t = torch.randn(4, 1000, generator=g)
    o = v + torch.randn(4, 1000, generator=g) * 0.3
    o[0, :10] = v[0, :10]          # v == old: both branches equal -> ties
    o[1, :10] = v[1, :10] - 0.2     # |v - old| on the clamp boundary
    w = torch.randn(4, 1000, generator=g)
    vd = v.to(dev).requires_grad_(True)
    out = critic.clipped_value_error(vd, t.to(dev), o.to(dev), clip)
    vr = v.clone().requires_grad_(True)
    ref = ocritic.clipped_value_error(vr, t, o, clip)
    assert (out.detach().cpu() - ref).abs().max().item() <= 1e-5
    (out * w.to(dev)).sum().backward()
    (ref * w).sum().backward()
    assert (vd.grad.cpu() - vr.grad).abs().max().item() <= 1e-5


@pytest.mark.parametrize("clip", [None, 0.2])
@pytest.mark.parametrize("reduce", ["sum", "mean"])
@pytest.mark.parametrize("offset", [0, 1])
def test_clipped_value_error_broadcast_grad_and_tails(dev, clip, reduce, offset):
    """The gradient of a sum or a mean arrives as one broadcast value (read with
    stride 0); 3003 elements leave a tail of 3 after the 4-wide vectors, and a
    one-element offset makes every array misaligned (the scalar path)."""
    from meshy_amd import critic

    g = torch.Generator().manual_seed(9)
    n = 3003
    base = torch.randn(3, n + offset, generator=g)
    v, t = base[0, offset:], base[1, offset:]
    o = v + base[2, offset:] * 0.3
    vd_base = base[0].to(dev).clone().requires_grad_(True)
    vd = vd_base[offset:]
    td, od = base[1].to(dev)[offset:], (base[0] + base[2] * 0.3).to(dev)[offset:]
    out = critic.clipped_value_error(vd, td, od, clip)
    vr = v.clone().requires_grad_(True)
    ref = ocritic.clipped_value_error(vr, t, o, clip)
    assert (out.detach().cpu() - ref).abs().max().item() <= 1e-5
    getattr(out, reduce)().backward()
    getattr(ref, reduce)().backward()
    assert (vd_base.grad[offset:].cpu() - vr.grad).abs().max().item() <= 1e-6


def test_size_mismatches_raise(dev):
    from meshy_amd import critic, vapo

    v = torch.zeros(10, device=dev)
    with pytest.raises(ValueError, match="targets"):
        critic.clipped_value_error(v, torch.zeros(9, device=dev), None, None)
    with pytest.raises(ValueError, match="old_values"):
        critic.clipped_value_error(v, v, torch.zeros(11, device=dev), 0.2)
    with pytest.raises(ValueError, match="mask and doc_ids"):
        critic.advantages_to_per_sequence(v, torch.ones(9, device=dev), torch.zeros(10, dtype=torch.long,
                                                                                   device=dev), 1)
    with pytest.raises(ValueError, match="mask"):
        vapo.whiten_flat(v, torch.ones(12, device=dev))


def _rollout_samples(n, seed, *, stamps=True):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(n):
        L = int(torch.randint(2, 3000, (1,), generator=g))
        p = int(torch.randint(1, L, (1,), generator=g))
        mask = torch.zeros(L)
        mask[p:] = 1.0
        lp = -torch.rand(L, generator=g) * 3
        lp[:p] = 0.0
        s = {"tokens": torch.randint(0, 151936, (L,), generator=g), "logprobs": lp, "mask_assistant": mask,
             "advantage": torch.tensor(float(torch.randn(1, generator=g)) if i % 3 else 0.0),
             "reward": torch.tensor(float(i % 2)), "weight_version": torch.tensor(5 - i % 3)}
        if stamps:
            s.update(truncated=torch.tensor(i % 4 == 0, dtype=torch.int64),
                     repetition=torch.tensor(i % 5 == 0, dtype=torch.int64),
                     mixed_version=torch.tensor(i % 7 == 0, dtype=torch.int64),
                     raw_reward=torch.tensor(float(i % 2) + (0.25 if i % 3 == 0 else 0.0)))
        out.append(s)
    return out


def _compare(m, hist, rm, rh):
    assert set(m) == set(rm)
    for k, want in rm.items():
        assert m[k] == pytest.approx(want, rel=1e-6, abs=1e-9), k
    assert set(hist) == set(rh)
    for k, want in rh.items():
        got = hist[k]
        got = got.cpu().tolist() if torch.is_tensor(got) else got
        assert np.allclose(got, want, atol=1e-7), k


@pytest.mark.parametrize("stamps", [True, False])
def test_rollout_metrics_match_oracle(dev, stamps):
    from meshy_amd.rollout_metrics import rollout_metrics

    samples = _rollout_samples(40, seed=1, stamps=stamps)
    samples[3]["logprobs"] = samples[3]["logprobs"][:-5]  # shorter than its mask: every log-prob is kept
    del samples[4]["mask_assistant"]                        # no mask: no response length
    m, hist = rollout_metrics(samples, seq_len=2048, current_version=6)
    rm, rh = orm.rollout_metrics(samples, seq_len=2048, current_version=6)
    _compare(m, hist, rm, rh)


def test_rollout_metrics_step_boundaries(dev):
    """Samples around the token-stats kernels' 1024-token steps, several steps
    long, empty, and with log-prob columns longer or shorter than the mask."""
    from meshy_amd.rollout_metrics import rollout_metrics

    g = torch.Generator().manual_seed(5)
    samples = []
    for i, L in enumerate([1, 1023, 1024, 1025, 2048, 4097, 9001, 0, 3000]):
        mask = (torch.rand(L, generator=g) > 0.3).float()
        lp = -torch.rand(L + (7 if i == 5 else 0) - (3 if i == 6 and L else 0), generator=g) * 2
        samples.append({"tokens": torch.randint(0, 1000, (L,), generator=g), "logprobs": lp,
                        "mask_assistant": mask, "reward": torch.tensor(float(i % 2))})
    m, hist = rollout_metrics(samples, seq_len=4096)
    rm, rh = orm.rollout_metrics(samples, seq_len=4096)
    _compare(m, hist, rm, rh)


def test_rollout_metrics_from_wire_columns(dev):
    from meshy_amd import wire
    from meshy_amd.rollout_metrics import rollout_metrics

    samples = _rollout_samples(25, seed=2)
    fields = ["tokens", "logprobs", "mask_assistant", "advantage", "reward", "raw_reward", "weight_version",
              "truncated", "repetition", "mixed_version"]
    cols = wire.samples_to_columns(samples, fields)
    m, hist = rollout_metrics(cols, seq_len=1024, current_version=9)
    rm, rh = orm.rollout_metrics(samples, seq_len=1024, current_version=9)
    _compare(m, hist, rm, rh)


@pytest.mark.parametrize("layout", ["packed", "padded"])
def test_pack_from_wire_columns_equals_pack_from_samples(dev, layout):
    from meshy_amd import wire, workloads
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    samples = batch.sample_dicts(rewards=rewards)
    cols = wire.samples_to_columns(samples, ["tokens", "mask_assistant", "logprobs", "reward"])
    cfg = PlannerConfig(layout=layout, mini_batch_size=256, seq_len=8192, align=2048,
                        max_tokens_per_micro=8192 if layout == "packed" else None,
                        micro_batch_size=None if layout == "packed" else 4)
    a = pack_step(RaggedSamples.from_samples(samples, group_offsets), cfg, dev)
    b = pack_step(RaggedSamples.from_columns(cols, group_offsets), cfg, dev)
    assert a.plan == b.plan
    assert torch.equal(a.advantages, b.advantages)
    for x, y in zip(a.batches, b.batches):
        for f in ("input_ids", "labels", "positions", "mask", "doc_ids", "rollout_logprobs", "advantages"):
            assert torch.equal(getattr(x, f), getattr(y, f)), f


@pytest.mark.parametrize("seed", range(8))
def test_random_rollout_metrics_match_oracle(dev, seed):
    """Random rollout batches (1 to 80 samples, with or without the stamps,
    a sample whose log-probs are shorter than its mask, one without a mask,
    random seq_len and versions) against the oracle's metrics."""
    from meshy_amd.rollout_metrics import rollout_metrics

    rng = np.random.default_rng(3000 + seed)
    n = int(rng.integers(1, 80))
    samples = _rollout_samples(n, seed=seed + 17, stamps=bool(seed % 2))
    if n > 3 and seed % 3 == 0:
        samples[1]["logprobs"] = samples[1]["logprobs"][: max(1, samples[1]["logprobs"].numel() // 2)]
    if n > 4 and seed % 4 == 1:
        del samples[2]["mask_assistant"]
    seq_len = int(rng.choice([64, 1000, 2048, 100000]))
    version = int(rng.integers(3, 9))
    m, hist = rollout_metrics(samples, seq_len=seq_len, current_version=version)
    rm, rh = orm.rollout_metrics(samples, seq_len=seq_len, current_version=version)
    _compare(m, hist, rm, rh)

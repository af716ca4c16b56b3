"""meshy_step_plan (host): the fused loss-token count, planner and one rank's
pack tables equal the separate calls (meshy_sample_loss_tokens,
meshy_plan_build) and the tables derived from them as the pack reads them, on
random batches of both layouts over 1, 2 and 4 ranks, with truncated samples,
masks with holes and samples without loss tokens."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from meshy_amd import _lib
from meshy_amd.plan import PlannerConfig, PlanTables, plan_tables


def _stage(lengths, rng):
    offsets = np.zeros(len(lengths) + 1, np.int64)
    np.cumsum(lengths, out=offsets[1:])
    mask = (rng.random(int(offsets[-1])) < 0.7).astype(np.float32)
    mask[: int(offsets[1]) // 2] = 0.0
    return offsets, mask


def _derived(t, rank, packed):
    n_local, nm = t.n_local, t.n_micro_total
    seq = t.micro_seq_len[rank * n_local: rank * n_local + nm]
    start = t.micro_doc_start[rank * (n_local + 1): rank * (n_local + 1) + nm + 1]
    local = t.local_indices[rank * n_local:(rank + 1) * n_local]
    nd = int(start[-1])
    dsample = local[t.doc_sample[rank * n_local:(rank + 1) * n_local]][:nd]
    dlen = t.doc_len[rank * n_local:(rank + 1) * n_local][:nd]
    rows = np.ones(nm, np.int64) if packed else np.maximum(np.diff(start), 1)
    out_off = np.zeros(nm + 1, np.int64)
    np.cumsum(seq * rows, out=out_off[1:])
    return seq, out_off, start, dsample, dlen, int((seq * rows).max()) if nm else 0, \
        int(np.diff(start).max()) if nm else 0


@pytest.mark.parametrize("layout", ["packed", "padded"])
@pytest.mark.parametrize("dp", [1, 2, 4])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_step_plan_equals_the_separate_calls(layout, dp, seed):
    rng = np.random.default_rng(seed)
    n = 64 * dp
    lengths = rng.integers(1, 3000, n).astype(np.int64)
    lengths[::7] = 1  # no loss tokens
    offsets, mask = _stage(lengths, rng)
    cfg = PlannerConfig(layout=layout, mini_batch_size=32, seq_len=2048, align=64 if layout == "packed" else 1,
                        max_tokens_per_micro=4096)
    lib = _lib.load()
    ln = np.empty(n, np.int64)
    lt = np.empty(n, np.int64)
    assert lib.meshy_sample_loss_tokens(mask.ctypes.data, offsets.ctypes.data, n, cfg.seq_len, ln.ctypes.data,
                                        lt.ctypes.data) == 0
    want_t = plan_tables(ln, lt, dp, cfg)
    for rank in range(dp):
        t = PlanTables(n, dp, cfg.mini_batch_size)
        n_local = n // dp
        seq = np.zeros(n_local, np.int64)
        out_off = np.zeros(n_local + 1, np.int64)
        start = np.zeros(n_local + 1, np.int32)
        dsample = np.zeros(n_local, np.int32)
        dlen = np.zeros(n_local, np.int64)
        counts = np.zeros((2, n), np.int64)
        a = _lib.StepPlanArgs()
        a.mask, a.offsets, a.n, a.dp_size, a.rank = mask.ctypes.data, offsets.ctypes.data, n, dp, rank
        a.cfg.layout = _lib.MESHY_LAYOUT_PACKED if layout == "packed" else _lib.MESHY_LAYOUT_PADDED
        a.cfg.mini_batch_size, a.cfg.seq_len, a.cfg.align = cfg.mini_batch_size, cfg.seq_len, cfg.align
        a.cfg.max_tokens_per_micro = cfg.max_tokens_per_micro
        a.plan = t.c_struct()
        a.lengths, a.loss_tokens = counts[0].ctypes.data, counts[1].ctypes.data
        a.micro_seq_len, a.micro_out_off, a.micro_doc_start = seq.ctypes.data, out_off.ctypes.data, start.ctypes.data
        a.doc_sample, a.doc_len = dsample.ctypes.data, dlen.ctypes.data
        assert lib.meshy_step_plan(ctypes.byref(a)) == 0, lib.meshy_last_error()
        t.n_micro_total = a.plan.n_micro_total
        assert np.array_equal(counts[0], ln) and np.array_equal(counts[1], lt)
        for name, _, _ in PlanTables._FIELDS:
            assert np.array_equal(getattr(t, name), getattr(want_t, name)), name
        w_seq, w_off, w_start, w_ds, w_dl, w_max_e, w_max_d = _derived(want_t, rank, layout == "packed")
        nm, nd = a.n_micro, a.n_docs
        assert nm == want_t.n_micro_total and nd == int(w_start[-1])
        assert np.array_equal(seq[:nm], w_seq) and np.array_equal(out_off[:nm + 1], w_off)
        assert np.array_equal(start[:nm + 1], w_start)
        assert np.array_equal(dsample[:nd], w_ds) and np.array_equal(dlen[:nd], w_dl)
        assert (a.max_micro_elems, a.max_docs_per_micro) == (w_max_e, w_max_d)


def test_step_plan_refuses():
    lib = _lib.load()
    a = _lib.StepPlanArgs()
    assert lib.meshy_step_plan(None) == -2
    a.n = 0
    assert lib.meshy_step_plan(ctypes.byref(a)) == -6  # an empty batch
    a.n, a.dp_size, a.rank = 4, 2, 2
    assert lib.meshy_step_plan(ctypes.byref(a)) == -1
    assert b"rank" in lib.meshy_last_error()
    a.rank = 0
    assert lib.meshy_step_plan(ctypes.byref(a)) == -2  # no pack tables


@pytest.mark.parametrize("seed", [0, 1])
def test_byte_mask_counts_and_plan_equal_the_fp32_ones(seed):
    """meshy_sample_loss_tokens_u8 over the mask as bytes gives the fp32 call's
    counts, and meshy_step_plan gives the same plan and pack tables from
    either staging of the mask."""
    from meshy_amd.pipeline import RaggedSamples

    rng = np.random.default_rng(seed)
    n = 96
    lengths = rng.integers(1, 3000, n).astype(np.int64)
    offsets, mask = _stage(lengths, rng)
    lib = _lib.load()
    mb = mask.astype(np.uint8)
    out = [np.empty((2, n), np.int64) for _ in range(2)]
    assert lib.meshy_sample_loss_tokens(mask.ctypes.data, offsets.ctypes.data, n, 2048, out[0][0].ctypes.data,
                                        out[0][1].ctypes.data) == 0
    assert lib.meshy_sample_loss_tokens_u8(mb.ctypes.data, offsets.ctypes.data, n, 2048, out[1][0].ctypes.data,
                                           out[1][1].ctypes.data) == 0
    assert np.array_equal(out[0], out[1])
    tokens = rng.integers(0, 151936, int(offsets[-1])).astype(np.int32)
    lps = rng.standard_normal(int(offsets[-1])).astype(np.float32)
    rewards = rng.random(n).astype(np.float32)
    groups = np.arange(0, n + 1, 8, dtype=np.int64)
    as_bytes = RaggedSamples.from_arrays(tokens, mask, lps, offsets, rewards, groups)
    assert as_bytes.mask_u8
    assert np.array_equal(as_bytes.view("mask").numpy(), mb)
    frac = mask.copy()
    frac[5] = 0.5
    as_fp32 = RaggedSamples.from_arrays(tokens, frac, lps, offsets, rewards, groups)
    assert not as_fp32.mask_u8
    assert np.array_equal(as_fp32.view("mask").numpy(), frac)
    frac[5] = mask[5]
    as_fp32.view("mask").copy_(__import__("torch").from_numpy(frac))
    cfg = PlannerConfig(layout="packed", mini_batch_size=32, seq_len=2048, align=64, max_tokens_per_micro=4096)
    got = []
    for r in (as_bytes, as_fp32):
        assert np.array_equal(np.stack(r.sample_lengths(2048)), out[0])
        t = PlanTables(n, 1, cfg.mini_batch_size)
        a = r.step_plan_args(cfg, 1, 0, t)
        assert lib.meshy_step_plan(ctypes.byref(a)) == 0
        nm, nd = int(a.n_micro), int(a.n_docs)
        got.append((int(a.plan.n_micro_total), r.np_view("seq")[:nm].copy(), r.np_view("doc_start")[:nm + 1].copy(),
                    r.np_view("doc_sample")[:nd].copy(), r.np_view("doc_len")[:nd].copy(), t.local_indices.copy()))
    for x, y in zip(*got):
        assert np.array_equal(x, y)


def test_columns_and_samples_pick_the_byte_mask_for_binary_masks():
    import torch

    from meshy_amd.pipeline import RaggedSamples

    g = torch.Generator().manual_seed(3)
    samples = [{"tokens": torch.randint(0, 1000, (L,), generator=g), "mask_assistant": (torch.rand(L, generator=g) > 0.5).float(),
                "logprobs": torch.randn(L, generator=g), "reward": 1.0} for L in (5, 17, 300, 1)]
    r = RaggedSamples.from_samples(samples, [0, 2, 4])
    assert r.mask_u8
    assert torch.equal(r.view("mask"), torch.cat([s["mask_assistant"] for s in samples]).to(torch.uint8))
    samples[2]["mask_assistant"] = samples[2]["mask_assistant"].bool()  # not fp32: the fp32 staging
    r = RaggedSamples.from_samples(samples, [0, 2, 4])
    assert not r.mask_u8
    assert torch.equal(r.view("mask"), torch.cat([s["mask_assistant"].float() for s in samples]))

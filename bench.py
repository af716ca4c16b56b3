"""Benchmark of the ragged-batch hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]

A step is one pass of the fused packed logprob + entropy kernel over one
micro-batch of bf16 logits [T=16384, V=151936] (Qwen3-1.7B vocabulary),
already resident in HBM.  The device-side timing of the logits backward over
the same logits runs before the headline (without --quick), so the headline's
W warm-up steps start on a busy device.  Prints ONE JSON line with

* value / ms_per_step  packed tokens/s of that pass (the headline metric)
* roofline             algorithmic bytes per launch / average launch time
                       (HIP events over the timed region) against 8 TB/s
* cpu_baseline         the reference's chunk loop (fp32 upcast, 1024-row
                       -cross_entropy, 512-row entropy slices) restated on CPU
                       torch on a bounded row sample, on this host's cores
* pack_latency_us      256 GRPO samples (budget 8192) -> native plan -> one host-to-
                       device copy -> GRPO + pack kernels, wall clock
* kernels              per-kernel device time, algorithmic GB/s and the
                       restated CPU path for the 256-sample GRPO batch,
                       the 512-doc PPO batch, 16 long sequences and 1024 GAE docs
                       (legs of sub-millisecond calls average over at least
                       200 calls, whatever K is)
* end_to_end           pack + GRPO -> logprob+entropy -> PPO fwd+bwd -> logits
                       backward at T = 16384, GPU wall against the CPU
                       restatement, with the largest difference between the
                       two chains' losses, sums and gradients
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
T_TOK, VOCAB = 16384, 151936
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def _sync():
    import torch

    torch.cuda.synchronize()


# Host-bound calls (the drop-in wrappers, the pack, the autograd engine) run
# 2-3x slower for the first few hundred calls of a fresh process, until the
# host's clocks and caches settle: such legs keep warming for WARM_S seconds
# before the clock starts.  The headline leg does exactly its W warm-up steps.
WARM_S = 0.3


def _warm(fn, warmup: int, warm_s: float, before=None, gpu: bool = False) -> None:
    """At least `warmup` calls, and more until `warm_s` seconds have passed."""
    t_end = time.perf_counter() + warm_s
    i = 0
    while i < warmup or time.perf_counter() < t_end:
        if before is not None:
            before()
        fn()
        if gpu:
            _sync()
        i += 1


# Legs whose calls take well under a millisecond average over at least this
# many calls (a few milliseconds in all), whatever --steps is: with 20 calls the
# first launches' queueing shows in the average.
SMALL_STEPS = 200


def _small(steps: int) -> int:
    return max(steps, SMALL_STEPS)


def _gpu_ms(fn, steps: int, warmup: int, warm_s: float = WARM_S) -> float:
    """Average ms per call of `fn` (HIP events on the current stream)."""
    import torch

    _warm(fn, warmup, warm_s)
    _sync()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    _sync()
    return start.elapsed_time(stop) / steps


def _wall_ms(fn, runs: int, warmup: int = 1, gpu: bool = True, before=None, warm_s: float = WARM_S) -> float:
    """Median wall ms of `fn` (synchronized when `gpu`); `before` runs untimed
    ahead of each call (e.g. releasing the previous call's result)."""
    _warm(fn, warmup, warm_s, before=before, gpu=gpu)
    times = []
    for _ in range(runs):
        if before is not None:
            before()
        if gpu:
            _sync()
        t0 = time.perf_counter()
        fn()
        if gpu:
            _sync()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def _entry(us: float, nbytes: float, cpu_ms: float | None = None, **extra):
    gbs = nbytes / (us * 1e-6) / 1e9
    e = {"us": round(us, 2), "bytes": int(nbytes), "GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    if cpu_ms is not None:
        e["cpu_ms"] = round(cpu_ms, 3)
        e["speedup_vs_cpu"] = round(cpu_ms * 1e3 / us, 1)
    e.update(extra)
    return e


def _with_device(e: dict, device_us: float, nbytes: float) -> dict:
    """Adds the device time of the kernels alone (their C-ABI calls in a loop,
    without the Python wrapper or the autograd engine) to a drop-in call's entry."""
    gbs = nbytes / (device_us * 1e-6) / 1e9
    e["device_us"] = round(device_us, 2)
    e["device_GBps"] = round(gbs, 1)
    e["device_frac_hbm"] = round(gbs / HBM_PEAK_GBS, 4)
    return e


def _host_phases(call, runs: int = 200, warmup: int = 20) -> dict:
    """Median host µs of each phase of one drop-in call.  ``call(mark)`` makes
    the call, calling ``mark(name)`` at the end of each phase; the device is
    synchronized after each call, never inside one, so a phase's figure is the
    host time it takes to issue its work."""
    samples: dict[str, list[float]] = {}

    def run(record: bool) -> None:
        stamps = [time.perf_counter()]
        names = []

        def mark(name: str) -> None:
            stamps.append(time.perf_counter())
            names.append(name)

        call(mark)
        if record:
            for i, name in enumerate(names):
                samples.setdefault(name, []).append((stamps[i + 1] - stamps[i]) * 1e6)

    for _ in range(warmup):
        run(False)
        _sync()
    for _ in range(runs):
        run(True)
        _sync()
    out = {name: round(statistics.median(v), 1) for name, v in samples.items()}
    out["total"] = round(sum(out.values()), 1)
    return out


def _autograd_floor_us(dev) -> float:
    """Host µs of a custom autograd Function's forward and ``backward()`` that
    allocate one tensor each and launch nothing: what any drop-in loss pays to
    the autograd engine before its own work."""
    import torch

    class _Nothing(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            return torch.empty((), device=x.device)

        @staticmethod
        def backward(ctx, g):
            return torch.empty(1, device=g.device)

    x = torch.empty(1, device=dev, requires_grad=True)

    def call(mark):
        x.grad = None
        _Nothing.apply(x).backward()
        mark("forward_and_backward")

    return _host_phases(call)["forward_and_backward"]


def _checked(rc: int, what: str) -> None:
    from meshy_amd import _lib

    _lib.check(rc, what)


# ---------------------------------------------------------------- logits [16384, 151936]

def headline_inputs():
    """The headline workload: bf16 logits N(0, 2^2) [1, 16384, 151936] and uniform labels."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1)
    logits = torch.randn(1, T_TOK, VOCAB, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0
    labels = torch.randint(0, VOCAB, (1, T_TOK), generator=gen, device=dev)
    return logits, labels


def bench_logprob(logits, labels, steps, warmup):
    import torch

    from meshy_amd import logprob

    out = {}

    def step():
        out["r"] = logprob.logprobs_and_entropy(logits, labels, with_entropy=True)

    ms = _gpu_ms(step, steps, warmup, warm_s=0.0)  # exactly W untimed warm-up steps
    lp, ent = out["r"]
    assert torch.isfinite(lp).all() and torch.isfinite(ent).all()
    nbytes = T_TOK * VOCAB * 2 + T_TOK * 8 + T_TOK * 8
    return ms, nbytes


def bench_read_ceiling(logits, steps, warmup):
    """GB/s of a plain streaming read with K1's access pattern over the same logits."""
    import torch

    from meshy_amd import _lib

    lib = _lib.load()
    out = torch.zeros(1, dtype=torch.int32, device=logits.device)
    rows = logits.shape[0] * logits.shape[1]
    row_bytes = logits.shape[2] * 2

    def step():
        _lib.check(lib.meshy_stream_read(logits.data_ptr(), rows, row_bytes, out.data_ptr(),
                                         _lib.stream_of(logits.device)), "meshy_stream_read")

    ms = _gpu_ms(step, steps, warmup, warm_s=0.0)  # measured like the headline leg
    return rows * row_bytes / (ms * 1e-3) / 1e9


def bench_logprob_bwd(logits, labels, steps, warmup):
    """K1b: d logp / d logits written as bf16, one read of z and one write of dz."""
    import torch

    from meshy_amd import _lib, logprob

    lse = logprob.logsumexp_rows(logits)
    g = torch.ones_like(lse)
    grad = torch.empty_like(logits)
    rows, T, V = logits.shape
    lib = _lib.load()
    ws = logprob.bwd_workspace(rows * T, logits.device)

    def step():
        _lib.check(lib.meshy_logprob_bwd(logits.data_ptr(), rows, T, V, logits.stride(0), logits.stride(1),
                                         labels.data_ptr(), lse.data_ptr(), g.data_ptr(), grad.data_ptr(),
                                         ws.data_ptr(), ws.numel(), _lib.stream_of(logits.device)),
                   "meshy_logprob_bwd")

    ms = _gpu_ms(step, steps, warmup)
    del grad
    return ms, rows * T * V * 4 + rows * T * 16


def cpu_logprob_bwd_ms(logits_gpu, labels_gpu, rows: int) -> float:
    """The reference's backward of a logprob chunk on CPU torch: the checkpointed
    recompute of -cross_entropy(z.float(), y) plus autograd (trainer.py:504-517),
    on a row sample, scaled to every row."""
    import torch

    from oracle import logprob as olp

    z = logits_gpu[:, :rows].cpu()
    y = labels_gpu[:, :rows].cpu()
    g = torch.ones(z.shape[0], rows)

    def cpu():
        zr = z.detach().requires_grad_(True)
        (olp.chunk_logprobs(zr, y) * g).sum().backward()

    return _wall_ms(cpu, 3, gpu=False) * logits_gpu.shape[1] / rows


def cpu_logprob_tokens_per_s(logits_gpu, labels_gpu, rows: int, runs: int = 5):
    import torch

    from oracle import logprob as olp

    z = logits_gpu[:, :rows].cpu()
    y = labels_gpu[:, :rows].cpu()
    ms = _wall_ms(lambda: olp.forward_logprobs(z, y, chunk=1024, with_entropy=True, entropy_chunk_size=512),
                  runs, gpu=False)
    return rows / (ms * 1e-3), ms


# ---------------------------------------------------------------- OPD on the [16384, 151936] logits

def bench_opd(logits, labels, steps, warmup, no_cpu, cpu_rows=512):
    """Student Top-K OPD on the [16384, 151936] logits: Teacher Top-K (K = 8), the
    gather of K + 1 ids (Teacher's K plus the label) forward and backward, and the
    distillation loss forward + backward over the 16384 tokens."""
    from types import SimpleNamespace as NS

    import torch

    from meshy_amd import _lib, logprob, opd, topk
    from meshy_amd.batch import Batch
    from meshy_amd.plan import MiniPlan

    dev = logits.device
    rows, T, V = logits.shape
    K = 8
    out = {}
    res = {}
    ms = _gpu_ms(lambda: res.__setitem__("t", topk.teacher_topk(logits, K)), steps, warmup)
    t_ids, t_lps = res["t"]
    cpu_ms = None
    if not no_cpu:
        from oracle import topk as otopk

        zc = logits[:, :cpu_rows].cpu()
        cms = _wall_ms(lambda: otopk.teacher_topk_reference_loop(zc, K), 3, gpu=False)
        cpu_ms = cms * T / cpu_rows
    out["teacher_topk_K8_T16384_V151936"] = _entry(ms * 1e3, T * V * 2 + T * K * 12, cpu_ms,
                                                   cpu_sample=f"{cpu_rows} rows, scaled to T" if cpu_ms else None)
    ids = torch.cat([t_ids, labels.unsqueeze(-1)], -1).contiguous()
    ms = _gpu_ms(lambda: topk.gather_logprobs(logits, ids), steps, warmup)
    cpu_ms = cpu_bwd_ms = None
    if not no_cpu:
        from oracle import topk as otopk

        zc = logits[:, :cpu_rows].cpu()
        ic = ids[:, :cpu_rows].cpu()
        cpu_ms = _wall_ms(lambda: otopk.gather_logprobs(zc, ic), 3, gpu=False) * T / cpu_rows
        wc = torch.randn(rows, cpu_rows, K + 1)

        def cpu_bwd():
            zr = zc.detach().requires_grad_(True)  # bf16 leaf, as the model's logits
            (otopk.gather_logprobs(zr, ic) * wc).sum().backward()

        cpu_bwd_ms = _wall_ms(cpu_bwd, 3, gpu=False) * T / cpu_rows
    out["gather_logprobs_K9_fwd"] = _entry(ms * 1e3, T * V * 2 + T * (K + 1) * 12, cpu_ms,
                                           cpu_sample=f"{cpu_rows} rows, scaled to T" if cpu_ms else None)
    lse = logprob.logsumexp_rows(logits)
    g = torch.randn(rows, T, K + 1, device=dev)
    grad = torch.empty_like(logits)
    ws = logprob.bwd_workspace(rows * T, dev)
    lib = _lib.load()

    def bwd():
        _lib.check(lib.meshy_gather_logprobs_bwd(logits.data_ptr(), rows, T, V, logits.stride(0), logits.stride(1),
                                                 ids.data_ptr(), K + 1, lse.data_ptr(), g.data_ptr(),
                                                 grad.data_ptr(), ws.data_ptr(), ws.numel(),
                                                 _lib.stream_of(dev)), "meshy_gather_logprobs_bwd")

    ms = _gpu_ms(bwd, max(5, steps // 2), 2)
    out["gather_logprobs_K9_bwd"] = _entry(
        ms * 1e3, T * V * 4 + T * (K + 1) * 12, cpu_bwd_ms,
        cpu_sample=(f"{cpu_rows} rows, scaled to T; the reference's recompute of the chunk plus autograd"
                    if cpu_bwd_ms else None))
    del grad
    # distillation loss over the T tokens: 12 documents, gathered log-probs from the kernel above
    gathered = topk.gather_logprobs(logits, ids)
    n_docs = 12
    doc_ids = (torch.arange(T, device=dev) * n_docs // T).reshape(1, T)
    mask = torch.ones(1, T, device=dev)
    z = torch.zeros(1, 1, dtype=torch.long, device=dev)
    mb = opd.TopKBatch(z, labels, z.int(), mask, doc_ids, torch.zeros(n_docs, device=dev),
                       torch.full((1, T), -1.0, device=dev), torch.zeros(n_docs, device=dev), n_docs,
                       teacher_topk_ids=t_ids, teacher_topk_logprobs=t_lps)
    mini = MiniPlan((), n_docs, T, ())
    stub = NS(calculate_per_token_loss=False, log_prob_min_clamp=-10.0, loss_max_clamp=10.0, sharder=None)
    gd = gathered.detach().requires_grad_(True)

    def fresh_micro():
        # Each call sees a new micro-batch, as in the training loop (opd.py:207-214),
        # which builds every micro once and takes one loss of it.
        mb.__dict__.pop("_meshy_seg_offsets", None)
        mb.__dict__.pop("_meshy_distill_inputs", None)

    def loss_fb():
        fresh_micro()
        gd.grad = None
        loss, _ = opd.distill_from_gathered(stub, gd, mb, mini)
        loss.backward()

    def loss_phases(mark):
        # the steps of distill_from_gathered, one mark after each
        fresh_micro()
        gd.grad = None
        inputs = opd._cached_inputs(stub, mb, mini, K, gd, T)
        mark("inputs")
        loss, parts = _lib.autograd().distill_loss(gd, inputs.native)
        dict(zip(_lib.DISTILL_OUT_NAMES, parts))
        mark("forward")
        loss.backward()
        mark("backward")

    ms = _gpu_ms(loss_fb, _small(steps), warmup)
    cpu_ms = None
    if not no_cpu:
        from oracle import opd as oopd

        gc, tc, mc, dc, rc = (gathered.detach().cpu(), t_lps.cpu(), mask.cpu(), doc_ids.cpu(),
                              mb.rollout_logprobs.cpu())

        def cpu_loss():
            g2 = gc.clone().requires_grad_(True)
            loss, _ = oopd.distill_loss(g2, tc, mc, dc, n_docs, rollout_lp=rc, n_docs_global=n_docs,
                                        n_tokens_global=T, per_token_loss=False)
            loss.backward()

        cpu_ms = _wall_ms(cpu_loss, 5, gpu=False)
    # The kernels alone, through the C ABI: document offsets, loss, gradient.
    import ctypes

    from meshy_amd import _lib

    student = gd.detach().reshape(-1, K + 1)
    inputs = opd._Inputs(stub, mb, mini, K, T, dev)
    args = inputs.args(student)
    pa = ctypes.byref(args)
    lib, stream = _lib.load(), _lib.stream_of(dev)
    out_t = torch.empty(_lib.DISTILL_NOUT, device=dev)
    seg = torch.empty(n_docs + 1, device=dev)
    one = torch.ones(1, device=dev)
    grad = torch.empty_like(student)
    ids, off = mb.doc_ids.reshape(-1), inputs.seg_off

    def dev_fb():
        lib.meshy_segment_offsets(ids.data_ptr(), ids.numel(), n_docs + 1, off.data_ptr(), None, stream)
        lib.meshy_distill_loss_fwd(pa, out_t.data_ptr(), seg.data_ptr(), stream)
        lib.meshy_distill_loss_bwd(pa, seg.data_ptr(), one.data_ptr(), grad.data_ptr(), stream)

    _checked(lib.meshy_distill_loss_fwd(pa, out_t.data_ptr(), seg.data_ptr(), stream), "meshy_distill_loss_fwd")
    _checked(lib.meshy_distill_loss_bwd(pa, seg.data_ptr(), one.data_ptr(), grad.data_ptr(), stream),
             "meshy_distill_loss_bwd")
    dev_us = _gpu_ms(dev_fb, _small(steps), warmup) * 1e3
    # fwd reads student (K+1)*4 + teacher K*4 + mask 4 + rollout 4 + doc id 8 (+ 8 for the
    # offsets); bwd reads the same and writes (K+1)*4
    per_tok = (K + 1) * 4 + K * 4 + 16
    nbytes = T * (2 * per_tok + 8 + (K + 1) * 4)
    out["distill_loss_fwd_bwd_K8_T16384"] = _with_device(
        _entry(ms * 1e3, nbytes, cpu_ms, tokens=T, host_phases_us=_host_phases(loss_phases),
               note="a new micro-batch each call: its inputs are built every time"), dev_us, nbytes)
    return out


# ---------------------------------------------------------------- 256 GRPO samples

def bench_pack(runs, no_cpu):
    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    dev = torch.device("cuda:0")
    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    cfg = PlannerConfig(layout="packed", mini_batch_size=256, seq_len=8192, align=2048,
                        max_tokens_per_micro=8192)
    res = {}

    def full():
        res["r"] = pack_step(ragged, cfg, dev)

    # The previous call's micro-batches are released before the clock starts:
    # freeing a step's ~250 tensors is not part of packing the next one.
    drop = lambda: res.pop("r", None)  # noqa: E731
    wall = _wall_ms(full, runs, warmup=3, before=drop)
    eager = _wall_ms(lambda: res.__setitem__("r", pack_step(ragged, cfg, dev, with_plan_objects=True)), runs,
                     warmup=2, before=drop)

    fields = ("input_ids", "labels", "positions", "mask", "doc_ids", "advantages", "rollout_logprobs", "lengths",
              "attention_masks", "positive_lm_weights", "advantage_tokens")

    def full_views():
        r = pack_step(ragged, cfg, dev)
        for mb in r.batches:
            for name in fields:
                getattr(mb, name)
        res["r"] = r

    wall_views = _wall_ms(full_views, runs, warmup=2, before=drop)
    full()

    from meshy_amd import _lib
    from meshy_amd.plan import PlanTables, plan_tables, tables_to_plan

    lengths, loss = ragged.sample_lengths(8192)
    tables = plan_tables(lengths, loss, 1, cfg)
    count_ms = _wall_ms(lambda: ragged.sample_lengths(8192), runs, gpu=False)
    plan_ms = _wall_ms(lambda: plan_tables(lengths, loss, 1, cfg), runs, gpu=False)
    dc_ms = _wall_ms(lambda: tables_to_plan(tables), runs, gpu=False)

    def step_plan():
        # what pack_step runs on the host before its second copy: the loss-token
        # count, the planner and this rank's pack tables, in one native call
        t = PlanTables(ragged.n, 1, cfg.mini_batch_size)
        _lib.load().meshy_step_plan(_lib.ctypes.byref(ragged.step_plan_args(cfg, 1, 0, t)))

    step_ms = _wall_ms(step_plan, runs, gpu=False)
    r = res["r"]
    n_out = sum(mb.input_ids.numel() for mb in r.batches)
    real = int(sum(m.n_tokens for m in (mm for mini in r.plan.per_rank[0] for mm in mini.micros)))
    out = {
        # plan + staging + the two host-to-device copies + GRPO + pack kernels,
        # device-synchronized; each micro's Batch tensors are views made when
        # the trainer first reads them (as it builds each micro when reaching it)
        "pack_latency_us": round(wall * 1e3, 1),
        # the same with the Plan dataclasses built inside the call (they are
        # otherwise built when PackResult.plan is first read)
        "pack_latency_with_plan_dataclasses_us": round(eager * 1e3, 1),
        # the same with every field of every micro's Batch read once (all views made)
        "pack_latency_all_views_us": round(wall_views * 1e3, 1),
        # the host plan inside the call (one native call), and its parts run
        # as separate calls; the Plan dataclasses are built only when read
        "host_phases_us": {"step_plan": round(step_ms * 1e3, 1), "loss_token_count": round(count_ms * 1e3, 1),
                           "planner": round(plan_ms * 1e3, 1), "plan_dataclasses": round(dc_ms * 1e3, 1)},
        "host_plan_us": round(step_ms * 1e3, 1),
        "n_micro": len(r.batches),
        "tokens": real,
        "out_tokens": n_out,
        # reads: token 4 + mask 4 + logprob 4 per real token; writes: ids, labels,
        # doc_ids 8 each, positions 4, mask 4, rollout lp 4, adv_tok 4 per output token
        "bytes": real * 12 + n_out * 40,
    }
    # The trainer's drop-in (batch.py:96 build_micro_batch, all micros of the
    # mini-batch in one call): per-sample tensors staged by the host gather,
    # given the plan and the advantages.
    from meshy_amd.batch import build_micro_batches

    samples_t = [dict(s, advantage=torch.tensor(0.5)) for s in batch.sample_dicts(rewards=rewards)]
    local_t = r.plan.local_samples(samples_t, 0)
    micros = [m for mini in r.plan.per_rank[0] for m in mini.micros]
    held = {}
    out["build_micro_batches_from_samples_us"] = round(1e3 * _wall_ms(
        lambda: held.__setitem__("b", build_micro_batches(local_t, micros, layout="packed", device=dev,
                                                          need_rollout_lp=True)),
        runs, warmup=2, before=lambda: held.pop("b", None)), 1)
    # The trainer's own call pattern: one build_micro_batch per micro as it
    # reaches it (trainer.py:557-571), timed as the reference times it,
    # "train/pack_batch" with a device sync (trainer.py:972).
    from meshy_amd.batch import build_micro_batch

    per_micro = []
    for rep in range(max(3, runs // 20) + 2):
        for m in micros:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            mb = build_micro_batch(local_t, m, layout="packed", device=dev, need_rollout_lp=True)
            torch.cuda.synchronize()
            if rep >= 2:  # the first two passes warm up
                per_micro.append(time.perf_counter() - t0)
            del mb
    out["build_micro_batch_per_micro_us"] = {"median": round(float(np.median(per_micro)) * 1e6, 1),
                                             "mean": round(float(np.mean(per_micro)) * 1e6, 1),
                                             "micros": len(micros), "calls": len(per_micro)}
    # The OPD student's drop-in (opd.py:141-148): the same micros with the
    # Teacher's K = 8 int64 ids and fp32 log-probs per position.
    from meshy_amd.opd import build_topk_micro_batches

    gen = torch.Generator().manual_seed(8)
    for s in samples_t:
        L = s["tokens"].shape[0]
        s["teacher_topk_ids"] = torch.randint(0, 151936, (L, 8), generator=gen)
        s["teacher_topk_logprobs"] = -torch.rand(L, 8, generator=gen)
    out["build_topk_micro_batches_from_samples_us"] = round(1e3 * _wall_ms(
        lambda: held.__setitem__("b", build_topk_micro_batches(local_t, micros, layout="packed", device=dev,
                                                               need_rollout_lp=True)),
        runs, warmup=2, before=lambda: held.pop("b", None)), 1)
    held.clear()
    # The OPD student builds each micro as it reaches it too (opd.py:141-148).
    per_micro = []
    for rep in range(max(3, runs // 20) + 2):
        for m in micros:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            mb = build_topk_micro_batches(local_t, [m], layout="packed", device=dev, need_rollout_lp=True)
            torch.cuda.synchronize()
            if rep >= 2:  # the first two passes warm up
                per_micro.append(time.perf_counter() - t0)
            del mb
    out["build_topk_micro_batch_per_micro_us"] = {"median": round(float(np.median(per_micro)) * 1e6, 1),
                                                  "mean": round(float(np.mean(per_micro)) * 1e6, 1),
                                                  "micros": len(micros), "calls": len(per_micro)}
    if not no_cpu:
        from oracle import batch as obatch
        from oracle import grpo as ogrpo
        from oracle import plan as oplan

        samples = batch.sample_dicts(rewards=rewards)

        def cpu():
            lengths, loss = oplan.sample_lengths(samples, 8192)
            local, per_rank = oplan.build_plan(lengths, loss, 1, layout="packed", mini_batch_size=256,
                                               seq_len=8192, align=2048, max_tokens_per_micro=8192)
            adv = [0.0] * len(samples)
            for g in range(len(group_offsets) - 1):
                a, b = int(group_offsets[g]), int(group_offsets[g + 1])
                adv[a:b] = ogrpo.grpo_group([float(s["reward"]) for s in samples[a:b]])
            loc = [dict(samples[i], advantage=adv[i]) for i in local[0]]
            for micros, *_ in per_rank[0]:
                for idx, seq_len, doc_lens in micros:
                    obatch.build_micro_batch(loc, idx, seq_len, doc_lens, layout="packed", need_rollout_lp=True)

        out["cpu_ms"] = round(_wall_ms(cpu, 5, gpu=False), 2)
        out["speedup_vs_cpu"] = round(out["cpu_ms"] / wall, 1)
        # the reference's per-micro call restated on the CPU (batch.py:96-230,
        # device = cpu, so no host-to-device copy), per micro
        loc = [dict(s, advantage=0.5) for s in samples]
        loc = [loc[i] for i in r.plan.local_indices[0]]
        cpu_micro = []
        for rep in range(3):
            for m in micros:
                t0 = time.perf_counter()
                obatch.build_micro_batch(loc, m.sample_idx, m.seq_len, m.doc_lens, layout="packed",
                                         need_rollout_lp=True)
                if rep:
                    cpu_micro.append(time.perf_counter() - t0)
        out["cpu_build_micro_batch_per_micro_us"] = round(float(np.median(cpu_micro)) * 1e6, 1)
    return out, ragged, cfg


# ---------------------------------------------------------------- PPO over 512 docs

def bench_ppo(steps, warmup, no_cpu):
    from types import SimpleNamespace as NS

    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.advantage import grpo_advantages
    from meshy_amd.batch import Batch
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.plan import MiniPlan

    dev = torch.device("cuda:0")
    batch, old, new, rewards, group_offsets = workloads.ppo_512_docs(2)
    n = len(batch.lengths)
    T = batch.total
    adv = grpo_advantages(torch.from_numpy(rewards).to(dev), torch.from_numpy(group_offsets).to(dev))
    doc_ids = torch.from_numpy(np.repeat(np.arange(n), batch.lengths)).reshape(1, -1).to(dev)
    mask = torch.from_numpy(batch.mask).reshape(1, -1).to(dev)
    z = torch.zeros(1, 1, dtype=torch.long, device=dev)
    mb = Batch(z, z, z.int(), mask, doc_ids, adv, None, torch.zeros(n, device=dev), n)
    mini = MiniPlan((), n, int(mask.sum().item()), ())
    stub = NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, use_icepop=False,
              calculate_per_token_loss=True, old_logprobs_source="rollout", sharder=None, parallel_dims=NS(cp=1))
    old_d = torch.from_numpy(old).reshape(1, -1).to(dev)
    new_d = torch.from_numpy(new).reshape(1, -1).to(dev).requires_grad_(True)

    # The batch carries its document offsets, as one the pack kernels built
    # does (the pack writes them with cu_seqlens); a batch built elsewhere pays
    # one segment_offsets pass the first time (segment_offsets_us below).
    def fwd():
        with torch.no_grad():
            ppo_clip_loss(stub, new_d, old_d, mb, mini)

    def fwd_bwd():
        new_d.grad = None
        loss, _ = ppo_clip_loss(stub, new_d, old_d, mb, mini)
        loss.backward()

    fwd_ms = _gpu_ms(fwd, _small(steps), warmup)
    fb_ms = _gpu_ms(fwd_bwd, _small(steps), warmup)
    cpu_ms = None
    if not no_cpu:
        from oracle import ppo as oppo

        old_c = torch.from_numpy(old).reshape(1, -1)
        adv_c = adv.cpu()
        ids_c = doc_ids.cpu()
        mask_c = mask.cpu()

        def cpu():
            nr = torch.from_numpy(new).reshape(1, -1).requires_grad_(True)
            loss, sums = oppo.ppo_clip_loss(nr, old_c, mask_c, ids_c, adv_c, n, n_docs_global=n,
                                            n_tokens_global=mini.n_tokens_global, clip_low=0.2, clip_high=0.28,
                                            per_token_loss=True)
            loss.backward()
            oppo.reduce_mini_metrics(sums)

        cpu_ms = _wall_ms(cpu, 5, gpu=False)
    # The kernels alone, through the C ABI: the loss forward (which, for the
    # token mean, also writes each token's unit gradient), then the backward
    # (a scale by the loss's gradient); and the document offsets of a batch
    # that does not carry them.
    import ctypes

    from meshy_amd import _lib
    from meshy_amd import loss as loss_mod

    inputs = loss_mod._Inputs(stub, new_d, old_d, mb, mini, None)
    new_flat = new_d.detach().reshape(-1)
    unit = torch.empty_like(new_flat)
    args = inputs.args(new_flat, unit)
    args_nograd = inputs.args(new_flat)
    pa, pa0 = ctypes.byref(args), ctypes.byref(args_nograd)
    lib, stream = _lib.load(), _lib.stream_of(dev)
    out_t = torch.empty(_lib.PPO_NOUT, device=dev)
    one = torch.ones(1, device=dev)
    grad = torch.empty_like(new_flat)
    ids, off = mb.doc_ids.reshape(-1), inputs.seg_off

    def dev_fwd_nograd():
        lib.meshy_ppo_loss_fwd(pa0, out_t.data_ptr(), None, stream)

    def dev_fwd():
        lib.meshy_ppo_loss_fwd(pa, out_t.data_ptr(), None, stream)

    def dev_bwd():
        lib.meshy_ppo_loss_bwd(pa, None, one.data_ptr(), grad.data_ptr(), stream)

    def dev_offsets():
        lib.meshy_segment_offsets(ids.data_ptr(), ids.numel(), n + 1, off.data_ptr(), None, stream)

    _checked(lib.meshy_ppo_loss_fwd(pa, out_t.data_ptr(), None, stream), "meshy_ppo_loss_fwd")
    _checked(lib.meshy_ppo_loss_bwd(pa, None, one.data_ptr(), grad.data_ptr(), stream), "meshy_ppo_loss_bwd")
    fwd0_dev = _gpu_ms(dev_fwd_nograd, _small(steps), warmup) * 1e3
    fwd_dev = _gpu_ms(dev_fwd, _small(steps), warmup) * 1e3
    bwd_dev = _gpu_ms(dev_bwd, _small(steps), warmup) * 1e3
    off_dev = _gpu_ms(dev_offsets, _small(steps), warmup) * 1e3
    # fwd: new, old, mask read 12 B/token (+ the unit gradient written, 4 B,
    # when a backward follows); bwd: unit gradient read + gradient written 8 B/token
    fwd_bytes = T * 12
    fb_bytes = T * (16 + 8)

    def fb_phases(mark):
        # the steps of ppo_clip_loss, one mark after each
        new_d.grad = None
        inputs = loss_mod._cached_inputs(stub, new_d, old_d, mb, mini, None)
        mark("inputs")
        loss, parts = _lib.autograd().ppo_loss(new_d, inputs.native)
        dict(zip(_lib.PPO_OUT_NAMES[:12], parts[:12]))
        mark("forward")
        loss.backward()
        mark("backward")

    def inputs_uncached(mark):
        loss_mod._Inputs(stub, new_d, old_d, mb, mini, None)
        mark("inputs_uncached")

    phases = _host_phases(fb_phases)
    phases["inputs_uncached"] = _host_phases(inputs_uncached)["inputs_uncached"]
    return {
        "ppo_loss_fwd": _with_device(_entry(fwd_ms * 1e3, fwd_bytes, tokens=T), fwd0_dev, fwd_bytes),
        "ppo_loss_fwd_bwd": _with_device(_entry(fb_ms * 1e3, fb_bytes, cpu_ms, tokens=T, host_phases_us=phases,
                                                autograd_floor_us=_autograd_floor_us(dev)),
                                         fwd_dev + bwd_dev, fb_bytes),
        "segment_offsets_us": round(off_dev, 2),
    }


# ---------------------------------------------------------------- 16 long sequences

def bench_long_context(steps, warmup, no_cpu):
    import torch

    from meshy_amd import logprob, workloads
    from meshy_amd.plan import PlannerConfig, build_plan

    dev = torch.device("cuda:0")
    lengths = workloads.long_context_16_lengths(3).tolist()
    cfg = PlannerConfig(layout="packed", mini_batch_size=16, seq_len=131072, align=2048,
                        max_tokens_per_micro=131072)
    plan = build_plan(lengths, lengths, 1, cfg)
    T = max(m.seq_len for mini in plan.per_rank[0] for m in mini.micros)
    V = 131072
    # logits N(0, 2^2) from the counter-based Box-Muller generator, so the
    # CPU leg regenerates its rows on the host instead of copying them
    logits = workloads.synth_logits(T, V, seed=3, scale=2.0, device=dev).unsqueeze(0)
    labels = torch.randint(0, V, (1, T), generator=torch.Generator(device=dev).manual_seed(3), device=dev)
    ms = _gpu_ms(lambda: logprob.logprobs_and_entropy(logits, labels, with_entropy=True), steps, warmup)
    cpu_ms = None
    rows = 8192
    if not no_cpu:
        from oracle import logprob as olp

        z = workloads.synth_logit_rows(range(rows), V, seed=3, scale=2.0).unsqueeze(0)
        y = labels[:, :rows].cpu()
        cms = _wall_ms(lambda: olp.forward_logprobs(z, y, chunk=1024, with_entropy=True, entropy_chunk_size=512),
                       3, gpu=False)
        cpu_ms = cms * T / rows  # scaled to the full micro
    del logits
    torch.cuda.empty_cache()
    nbytes = T * V * 2 + 16 * T
    return _entry(ms * 1e3, nbytes, cpu_ms, T=T, V=V, tokens_per_s=round(T / (ms * 1e-3)),
                  cpu_sample=f"{rows} rows regenerated on the host, scaled to T",
                  data="logits N(0, 2^2) bf16 from a counter-based Box-Muller generator (meshy_synth_bf16, seed 3)")


# ---------------------------------------------------------------- GAE over 1024 docs

def bench_gae(steps, warmup, no_cpu):
    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.gae import gae_and_returns

    dev = torch.device("cuda:0")
    batch, values, terminal = workloads.gae_1024_docs(4)
    n = len(batch.lengths)
    T = batch.total
    rewards = np.zeros(T, np.float32)
    rewards[batch.offsets[1:] - 1] = terminal
    doc_ids = torch.from_numpy(np.repeat(np.arange(n), batch.lengths)).reshape(1, -1).to(dev)
    r = torch.from_numpy(rewards).reshape(1, -1).to(dev)
    v = torch.from_numpy(values).to(torch.bfloat16).reshape(1, -1).to(dev)
    m = torch.from_numpy(batch.mask).reshape(1, -1).to(dev)
    lengths = torch.full((n,), 1.0 / (1.0 - 0.95), device=dev)
    ms = _gpu_ms(lambda: gae_and_returns(r, v, m, doc_ids, n, lengths=lengths, gamma=1.0, alpha=1.0), _small(steps), warmup)
    cpu_ms = None
    if not no_cpu:
        from oracle import gae as ogae

        L = batch.lengths
        S = int(L.max())
        pos = np.arange(T) - np.repeat(batch.offsets[:-1], L)
        ids = np.repeat(np.arange(n), L)
        R = torch.zeros(n, S)
        Vp = torch.zeros(n, S)
        M = torch.zeros(n, S)
        R[ids, pos] = torch.from_numpy(rewards)
        Vp[ids, pos] = v.reshape(-1).float().cpu()
        M[ids, pos] = torch.from_numpy(batch.mask)
        rid = torch.arange(n).unsqueeze(1).expand(n, S).contiguous()
        lc = lengths.cpu()

        def cpu():
            ogae.compute_vapo_gae(R, Vp, M, rid, n, lengths=lc, gamma=1.0, alpha=1.0)
            ogae.compute_returns(R, M, rid, gamma=1.0)

        cpu_ms = _wall_ms(cpu, 3, gpu=False)
    # The kernels alone: the same call through the C ABI in a loop (outputs,
    # workspace and the cached offsets made once), without the wrapper's
    # allocations and argument building.
    import ctypes

    from meshy_amd import _lib
    from meshy_amd.loss import checked_segment_offsets

    lib, stream = _lib.load(), _lib.stream_of(dev)
    adv_o, ret_o, lam_o = torch.empty(T, device=dev), torch.empty(T, device=dev), torch.empty(n, device=dev)
    ws = torch.empty(max(int(lib.meshy_gae_workspace_size(1, T, n)), 1), dtype=torch.uint8, device=dev)
    off = checked_segment_offsets(doc_ids, n + 1)
    ga = _lib.GaeArgs()
    ga.rewards, ga.values, ga.mask, ga.doc_ids = r.data_ptr(), v.data_ptr(), m.data_ptr(), doc_ids.data_ptr()
    ga.lengths = lengths.data_ptr()
    ga.rows, ga.S, ga.n_docs = 1, T, n
    ga.gamma, ga.alpha, ga.epsilon = 1.0, 1.0, 1e-6
    ga.values_bf16 = 1
    ga.adv, ga.returns, ga.lam_doc = adv_o.data_ptr(), ret_o.data_ptr(), lam_o.data_ptr()
    ga.workspace, ga.workspace_bytes = ws.data_ptr(), ws.numel()
    ga.seg_offsets = off.data_ptr()
    pg = ctypes.byref(ga)
    _checked(lib.meshy_gae(pg, stream), "meshy_gae")
    dev_us = _gpu_ms(lambda: lib.meshy_gae(pg, stream), _small(steps), warmup) * 1e3
    # reads rewards 4 + values 2 + mask 4, writes adv 4 + returns 4; document
    # starts come from the segment offsets of doc_ids (computed and
    # order-checked on the first call for the tensor, then reused), the ids
    # themselves are read at chunk ends
    return _with_device(_entry(ms * 1e3, T * 18, cpu_ms, tokens=T, docs=n,
                               cpu_sample="sequential loop on padded [1024, S_max]",
                               note="doc_ids offsets cached after the first call"), dev_us, T * 18)


def bench_gae_cache(steps):
    """Where GAE reads from: meshy_gae over the 1024 documents back to back
    (the 114 MB of inputs and outputs can stay in the 256 MB Infinity Cache
    between calls), then each call after a 1 GiB read that evicts the L2s and
    the Infinity Cache (the scan then reads HBM), then a 268,435,456 B device
    copy three times (counter calibration).  Device us per call from HIP
    events around the call alone."""
    import numpy as np
    import torch

    from meshy_amd import _lib, workloads
    from meshy_amd.loss import checked_segment_offsets

    dev = torch.device("cuda:0")
    batch, values, terminal = workloads.gae_1024_docs(4)
    n, T = len(batch.lengths), int(batch.total)
    rewards = np.zeros(T, np.float32)
    rewards[batch.offsets[1:] - 1] = terminal
    doc_ids = torch.from_numpy(np.repeat(np.arange(n), batch.lengths)).reshape(1, -1).to(dev)
    r = torch.from_numpy(rewards).to(dev)
    v = torch.from_numpy(values).to(torch.bfloat16).to(dev)
    m = torch.from_numpy(batch.mask).to(dev)
    lengths = torch.full((n,), 1.0 / (1.0 - 0.95), device=dev)
    lib, stream = _lib.load(), _lib.stream_of(dev)
    adv_o, ret_o, lam_o = torch.empty(T, device=dev), torch.empty(T, device=dev), torch.empty(n, device=dev)
    ws = torch.empty(max(int(lib.meshy_gae_workspace_size(1, T, n)), 1), dtype=torch.uint8, device=dev)
    off = checked_segment_offsets(doc_ids, n + 1)
    ga = _lib.GaeArgs()
    ga.rewards, ga.values, ga.mask, ga.doc_ids = r.data_ptr(), v.data_ptr(), m.data_ptr(), doc_ids.data_ptr()
    ga.lengths, ga.seg_offsets = lengths.data_ptr(), off.data_ptr()
    ga.rows, ga.S, ga.n_docs = 1, T, n
    ga.gamma, ga.alpha, ga.epsilon, ga.values_bf16 = 1.0, 1.0, 1e-6, 1
    ga.adv, ga.returns, ga.lam_doc = adv_o.data_ptr(), ret_o.data_ptr(), lam_o.data_ptr()
    ga.workspace, ga.workspace_bytes = ws.data_ptr(), ws.numel()
    pg = ctypes.byref(ga)
    _checked(lib.meshy_gae(pg, stream), "meshy_gae")
    big = torch.ones(256 * 1024 * 1024, device=dev)  # 1 GiB
    sink = torch.empty((), device=dev)

    def per_call(flush: bool) -> float:
        times = []
        for i in range(steps + 3):
            if flush:
                torch.sum(big, dim=0, out=sink)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            lib.meshy_gae(pg, stream)
            b.record()
            b.synchronize()
            if i >= 3:
                times.append(a.elapsed_time(b) * 1e3)
        return round(statistics.median(times), 2)

    out = {"back_to_back_us": per_call(False), "after_1GiB_read_us": per_call(True), "tokens": T, "docs": n,
           "inputs_MB": round(T * 10 / 1e6, 1), "outputs_MB": round(T * 8 / 1e6, 1)}
    src = torch.ones(64 * 1024 * 1024, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return out


# ---------------------------------------------------------------- GAE attach over 1024 docs, pack of 16 long sequences

def bench_attach_gae(runs, no_cpu):
    """_attach_gae_advantages over 1024 samples (values bf16, terminal
    rewards, constant lambda 0.95): GPU wall per call, samples staged from the host."""
    from types import SimpleNamespace as NS

    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.gae import attach_gae_advantages

    dev = torch.device("cuda:0")
    batch, values, terminal = workloads.gae_1024_docs(4)
    samples = []
    for i in range(len(batch.lengths)):
        a, b = int(batch.offsets[i]), int(batch.offsets[i + 1])
        samples.append({"tokens": torch.zeros(b - a, dtype=torch.int64),
                        "mask_assistant": torch.from_numpy(batch.mask[a:b].copy()),
                        "values": torch.from_numpy(values[a:b].copy()).to(torch.bfloat16),
                        "reward": torch.tensor(float(terminal[i]))})
    trainer = NS(seq_len=32768 + 256, gae_gamma=1.0, gae_alpha=1.5, gae_lambda=0.95, device=dev)
    ms = _wall_ms(lambda: attach_gae_advantages(trainer, samples), runs, warmup=2)
    out = {"gpu_ms": round(ms, 3), "samples": len(samples), "tokens": int(batch.total)}
    if not no_cpu:
        from oracle import gae as ogae

        fs = [{k: (v.float() if k == "values" else v) for k, v in smp.items()} for smp in samples]
        cms = _wall_ms(lambda: ogae.attach_gae_advantages(fs, seq_len=trainer.seq_len, gamma=1.0, alpha=1.5,
                                                          gae_lambda=0.95), 2, warmup=0, gpu=False)
        out["cpu_ms"] = round(cms, 1)
        out["speedup_vs_cpu"] = round(cms / ms, 1)
        out["cpu_sample"] = "the reference's padded [1024, S_max] block and sequential scan"
    return out


def bench_pack_long_context(runs, no_cpu):
    """16 samples U{8192..131072} under a 131072-token budget, align 2048."""
    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(3)
    lengths = workloads.long_context_16_lengths(3)
    offsets = np.zeros(len(lengths) + 1, np.int64)
    np.cumsum(lengths, out=offsets[1:])
    total = int(offsets[-1])
    tokens = rng.integers(0, 131072, total, dtype=np.int32)
    pos = np.arange(total) - np.repeat(offsets[:-1], lengths)
    prompt = np.repeat(rng.integers(64, 257, len(lengths)), lengths)
    mask = (pos >= prompt).astype(np.float32)
    lps = (-rng.uniform(0.0, 2.0, total)).astype(np.float32)
    rewards = (rng.random(len(lengths)) < 0.4).astype(np.float32)
    group_offsets = np.array([0, 8, 16], np.int64)
    ragged = RaggedSamples.from_arrays(tokens, mask, lps, offsets, rewards, group_offsets)
    cfg = PlannerConfig(layout="packed", mini_batch_size=16, seq_len=131072, align=2048,
                        max_tokens_per_micro=131072)
    res = {}
    ms = _wall_ms(lambda: res.__setitem__("r", pack_step(ragged, cfg, dev)), runs, warmup=2,
                  before=lambda: res.pop("r", None))
    res["r"] = pack_step(ragged, cfg, dev)
    r = res["r"]
    n_out = sum(mb.input_ids.numel() for mb in r.batches)
    out = {"pack_latency_us": round(ms * 1e3, 1), "n_micro": len(r.batches), "tokens": total, "out_tokens": n_out,
           "bytes": total * 12 + n_out * 40}
    out["GBps"] = round(out["bytes"] / (ms * 1e-3) / 1e9, 1)
    if not no_cpu:
        from oracle import batch as obatch
        from oracle import grpo as ogrpo
        from oracle import plan as oplan

        samples = []
        for i in range(len(lengths)):
            a, b = int(offsets[i]), int(offsets[i + 1])
            samples.append({"tokens": torch.from_numpy(tokens[a:b].astype(np.int64)),
                            "mask_assistant": torch.from_numpy(mask[a:b].copy()),
                            "logprobs": torch.from_numpy(lps[a:b].copy()), "reward": float(rewards[i])})

        def cpu():
            ln, loss = oplan.sample_lengths(samples, 131072)
            local, per_rank = oplan.build_plan(ln, loss, 1, layout="packed", mini_batch_size=16, seq_len=131072,
                                               align=2048, max_tokens_per_micro=131072)
            adv = ogrpo.grpo_group([float(x) for x in rewards[:8]]) + ogrpo.grpo_group([float(x) for x in rewards[8:]])
            loc = [dict(samples[i], advantage=adv[i]) for i in local[0]]
            for micros, *_ in per_rank[0]:
                for idx, seq_len, doc_lens in micros:
                    obatch.build_micro_batch(loc, idx, seq_len, doc_lens, layout="packed", need_rollout_lp=True)

        out["cpu_ms"] = round(_wall_ms(cpu, 3, gpu=False), 2)
        out["speedup_vs_cpu"] = round(out["cpu_ms"] / ms, 1)
    return out


# ---------------------------------------------------------------- critic reductions and rollout metrics

def bench_critic(steps, warmup, no_cpu):
    """1024 docs (lognormal(6000, 0.8) responses): per-sequence mean and clipped value error over the 6.35 M
    packed tokens, the Accumulator over the padded [1024, S_max] critic grid."""
    import numpy as np
    import torch

    from meshy_amd import critic, workloads

    dev = torch.device("cuda:0")
    batch, values, _ = workloads.gae_1024_docs(4)
    n = len(batch.lengths)
    T = batch.total
    g = torch.Generator(device=dev).manual_seed(4)
    doc_ids = torch.from_numpy(np.repeat(np.arange(n), batch.lengths)).reshape(1, -1).to(dev)
    mask = torch.from_numpy(batch.mask).reshape(1, -1).to(dev)
    adv = torch.randn(1, T, generator=g, device=dev)
    out = {}
    ms = _gpu_ms(lambda: critic.advantages_to_per_sequence(adv, mask, doc_ids, n), _small(steps), warmup)
    cpu_ms = None
    if not no_cpu:
        from oracle import critic as ocritic

        a_c, m_c, d_c = adv.cpu(), mask.cpu(), doc_ids.cpu()
        cpu_ms = _wall_ms(lambda: ocritic.advantages_to_per_sequence(a_c * m_c, m_c, d_c, n), 5, gpu=False)
    # reads adv 4 + mask 4 per token; the segment offsets of doc_ids (8 B per
    # token, one pass) are computed and order-checked on the first call for
    # the tensor and reused after
    out["per_sequence_mean_1024_docs"] = _entry(ms * 1e3, T * 8, cpu_ms, tokens=T, docs=n,
                                                note="doc_ids offsets cached after the first call")
    v = torch.randn(T, generator=g, device=dev).requires_grad_(True)
    t = torch.randn(T, generator=g, device=dev)
    o = (v.detach() + 0.1 * torch.randn(T, generator=g, device=dev))

    def cve():
        v.grad = None
        critic.clipped_value_error(v, t, o, 0.2).sum().backward()

    ms = _gpu_ms(cve, _small(steps), warmup)
    cpu_ms = None
    if not no_cpu:
        from oracle import critic as ocritic

        vc, tc, oc = v.detach().cpu().requires_grad_(True), t.cpu(), o.cpu()

        def cpu():
            vc.grad = None
            ocritic.clipped_value_error(vc, tc, oc, 0.2).sum().backward()

        cpu_ms = _wall_ms(cpu, 5, gpu=False)
    # The two kernels alone, through the C ABI (the gradient broadcast, stride 0).
    from meshy_amd import _lib

    lib, stream = _lib.load(), _lib.stream_of(dev)
    vf, tf, of = v.detach().reshape(-1), t.reshape(-1), o.reshape(-1)
    err = torch.empty_like(vf)
    gv = torch.empty_like(vf)
    one = torch.ones(1, device=dev)

    def dev_fb():
        lib.meshy_clipped_value_error(vf.data_ptr(), tf.data_ptr(), of.data_ptr(), 1, 0.2, T, err.data_ptr(), stream)
        lib.meshy_clipped_value_error_bwd(vf.data_ptr(), tf.data_ptr(), of.data_ptr(), 1, 0.2, T, one.data_ptr(), 0,
                                          gv.data_ptr(), stream)

    _checked(lib.meshy_clipped_value_error(vf.data_ptr(), tf.data_ptr(), of.data_ptr(), 1, 0.2, T, err.data_ptr(),
                                           stream), "meshy_clipped_value_error")
    dev_us = _gpu_ms(dev_fb, _small(steps), warmup) * 1e3
    # fwd: v, t, o read + out written; bwd (the sum's gradient is one broadcast
    # value): v, t, o read + grad written
    def cve_phases(mark):
        v.grad = None
        e = critic.clipped_value_error(v, t, o, 0.2)
        mark("forward")
        total = e.sum()
        mark("reduce")
        total.backward()
        mark("backward")

    out["clipped_value_error_fwd_bwd_1024_docs"] = _with_device(
        _entry(ms * 1e3, T * 32, cpu_ms, tokens=T, host_phases_us=_host_phases(cve_phases),
               note="us includes the .sum() whose gradient the backward reads"), dev_us, T * 32)
    S = int(batch.lengths.max())
    rows = n
    pos = np.arange(T) - np.repeat(batch.offsets[:-1], batch.lengths)
    ids = np.repeat(np.arange(n), batch.lengths)
    flat = torch.from_numpy(ids * S + pos).to(dev)
    vals = torch.zeros(rows * S, device=dev, dtype=torch.bfloat16)
    vals[flat] = torch.from_numpy(values).to(dev).to(torch.bfloat16)
    rets = torch.zeros(rows * S, device=dev)
    rets[flat] = torch.randn(T, generator=g, device=dev)
    msk = torch.zeros(rows * S, device=dev)
    msk[flat] = mask.reshape(-1)
    vals, rets, msk = vals.view(rows, S), rets.view(rows, S), msk.view(rows, S)
    rew = torch.rand(rows, device=dev)
    grp = torch.arange(rows, device=dev) // 8

    def acc():
        a = critic.Accumulator()
        a.update(vals, rets, msk, rew, grp)
        return a.state

    ms = _wall_ms(acc, steps // 5 + 3, warmup=2)
    cpu_ms = None
    if not no_cpu:
        from oracle import critic as ocritic

        vc, rc, mc, rwc, gc = vals.cpu(), rets.cpu(), msk.cpu(), rew.cpu(), grp.cpu()

        def cpu_acc():
            a = ocritic.Accumulator()
            a.update(vc, rc, mc, rwc, gc)

        cpu_ms = _wall_ms(cpu_acc, 3, gpu=False)
    # reads values 2 + returns 4 + mask 4 per grid element
    out["accumulator_update_1024_docs_padded"] = _entry(ms * 1e3, rows * S * 10, cpu_ms, rows=rows, S=S,
                                                      note="wall time including the state's host read")
    # critic_diagnostics over the same window (groups of 8 rows): the token
    # sums, the per-prompt AUC and Pearson, one host read
    dms = _wall_ms(lambda: critic.critic_diagnostics(vals, rets, msk, rew, grp), steps // 5 + 3, warmup=2)
    dcpu = None
    if not no_cpu:
        dcpu = _wall_ms(lambda: ocritic.critic_diagnostics(vc, rc, mc, rwc, gc), 3, gpu=False)
    out["critic_diagnostics_1024_docs_padded"] = _entry(dms * 1e3, rows * S * 10, dcpu, rows=rows, S=S,
                                                      note="wall time including the host read of the gauges")
    out["whiten_1024_docs"] = bench_whiten(batch, dev, steps, warmup, no_cpu)
    return out


def bench_whiten(batch, dev, steps, warmup, no_cpu):
    """Masked whitening (vapo.py:6-32) of the 6.35 M per-token advantages of the
    1024 documents, held in one flat device buffer as GAE leaves them."""
    import torch

    from meshy_amd import _lib, vapo

    T = batch.total
    g = torch.Generator(device=dev).manual_seed(21)
    adv = torch.randn(T, generator=g, device=dev) * 3.0 + 1.0
    mask = torch.from_numpy(batch.mask).to(dev)
    ms = _gpu_ms(lambda: vapo.whiten_flat(adv, mask), _small(steps), warmup)
    lib, stream = _lib.load(), _lib.stream_of(dev)
    stats = torch.empty(3, dtype=torch.float64, device=dev)
    ws = torch.empty(int(lib.meshy_whiten_workspace_size(T)), dtype=torch.uint8, device=dev)

    def dev_call():
        lib.meshy_whiten_stats(adv.data_ptr(), mask.data_ptr(), T, 1.0, stats.data_ptr(), ws.data_ptr(), ws.numel(),
                               stream)
        lib.meshy_whiten_apply(adv.data_ptr(), mask.data_ptr(), T, stats.data_ptr(), stream)

    _checked(lib.meshy_whiten_stats(adv.data_ptr(), mask.data_ptr(), T, 1.0, stats.data_ptr(), ws.data_ptr(),
                                    ws.numel(), stream), "meshy_whiten_stats")
    dev_us = _gpu_ms(dev_call, _small(steps), warmup) * 1e3
    cpu_ms = None
    if not no_cpu:
        from oracle import vapo as ovapo

        a_c, m_c = adv.cpu(), torch.from_numpy(batch.mask)
        samples = []
        for i in range(len(batch.lengths)):
            lo, hi = int(batch.offsets[i]), int(batch.offsets[i + 1])
            # the sample's loss mask is mask_assistant shifted by one
            ma = torch.zeros(hi - lo)
            ma[1:] = m_c[lo:hi - 1]
            samples.append({ovapo.ADVANTAGE_TOKENS: a_c[lo:hi].clone(), "mask_assistant": ma})
        cpu_ms = _wall_ms(lambda: ovapo.whiten_advantages(samples, 1 << 20), 3, gpu=False)
    # stats: adv + mask read (8 B per token); apply: both read, adv written (12 B)
    return _with_device(_entry(ms * 1e3, T * 20, cpu_ms, tokens=T), dev_us, T * 20)


def bench_rollout_metrics(runs, no_cpu):
    """The 256 GRPO samples: _rollout_metrics from the sample list and from the
    wire columns, wall time including every host read of the result."""
    import torch

    from meshy_amd import wire, workloads
    from meshy_amd.rollout_metrics import rollout_metrics

    batch, rewards, _ = workloads.grpo_256_samples(0)
    samples = batch.sample_dicts(rewards=rewards)
    for i, s in enumerate(samples):
        s.update(weight_version=torch.tensor(3 - i % 2), truncated=torch.tensor(i % 9 == 0),
                 repetition=torch.tensor(0), mixed_version=torch.tensor(0), advantage=torch.tensor(0.5))
    fields = list(samples[0])
    cols = wire.samples_to_columns(samples, fields)
    out = {"samples": len(samples), "tokens": int(batch.total)}
    # The rollout side of the same wire (rollout.py:611-615): Python-list
    # samples to columns, one pass per column against a tensor per sample.
    from types import SimpleNamespace as NS

    rollout = [NS(tokens=batch.tokens[a:b].astype(int).tolist(), logprobs=batch.logprobs[a:b].tolist(),
                  masks=batch.mask[a:b].astype(int).tolist(), reward=float(rewards[i]), advantage=0.5,
                  truncated=i % 9 == 0, repetition=False, mixed_version=False)
               for i, (a, b) in enumerate(zip(batch.offsets[:-1], batch.offsets[1:]))]
    out["wire_group_to_columns_ms"] = round(
        _wall_ms(lambda: wire.rollout_group_to_columns(rollout, 3), runs, warmup=1, gpu=False), 3)
    out["wire_per_sample_ms"] = round(_wall_ms(lambda: wire.samples_to_columns(
        [wire.sample_to_tensordict(s, 3) for s in rollout], wire.GRPO_TRAINER_FIELDS), runs, warmup=1, gpu=False), 3)
    out["gpu_from_samples_ms"] = round(_wall_ms(lambda: rollout_metrics(samples, 8192, 4), runs, warmup=2), 3)
    out["gpu_from_columns_ms"] = round(_wall_ms(lambda: rollout_metrics(cols, 8192, 4), runs, warmup=2), 3)
    if not no_cpu:
        from oracle import rollout_metrics as orm

        out["cpu_ms"] = round(_wall_ms(lambda: orm.rollout_metrics(samples, 8192, 4), 3, gpu=False), 3)
        out["speedup_vs_cpu"] = round(out["cpu_ms"] / out["gpu_from_columns_ms"], 1)
    return out


# ---------------------------------------------------------------- end to end

def bench_group_advantages(runs, no_cpu):
    """GRPO advantages and the zero-variance filter of a whole step (the 32
    groups of 8 of the 256-sample GRPO batch): the advantages in one device
    call (the rewards' host-to-device copy, one launch, the copy back) and
    through the per-group plugin form (a host call per group), the filter in
    one host call over the host rewards (and, for the record, in one device
    call), next to the reference's per-group host functions (rollout.py:
    88-115) called once per group as its rollout worker does, summed over the
    32 groups."""
    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.advantage import grpo_advantages, zero_variance_groups

    dev = torch.device("cuda:0")
    _, rewards, group_offsets = workloads.grpo_256_samples(0)
    n_groups = len(group_offsets) - 1
    reps = max(runs, 10)

    def batched(fn, dtype):
        def run():
            r = torch.from_numpy(rewards.astype(dtype)).to(dev)
            fn(r, torch.from_numpy(group_offsets).to(dev)).tolist()
        return _wall_ms(run, reps, gpu=False) * 1e3

    def host_filter():
        # the rewards where the rollout worker holds them: on the host
        zero_variance_groups(torch.from_numpy(rewards.astype(np.float64)), torch.from_numpy(group_offsets)).tolist()

    # the per-group advantage plugin, called once per group on sample objects
    # as the rollout worker calls its advantage_fn (rollout.py:580-587)
    from types import SimpleNamespace as NS

    from meshy_amd.advantage import grpo_advantage

    group_samples = [[NS(reward=float(x), advantage=None) for x in rewards[group_offsets[g]:group_offsets[g + 1]]]
                     for g in range(n_groups)]

    def plugin_all():
        for grp in group_samples:
            grpo_advantage(grp)

    out = {
        "group_size": 8, "n_groups": n_groups,
        "grpo_advantages_us_all_groups": round(batched(grpo_advantages, np.float32), 1),
        "zero_variance_groups_us_all_groups": round(_wall_ms(host_filter, reps, gpu=False) * 1e3, 1),
        "zero_variance_groups_device_us_all_groups": round(batched(zero_variance_groups, np.float64), 1),
        "grpo_advantage_plugin_us_all_groups": round(_wall_ms(plugin_all, reps, gpu=False) * 1e3, 1),
    }
    if not no_cpu:
        from oracle import grpo as ogrpo

        groups = [[float(r) for r in rewards[group_offsets[g]:group_offsets[g + 1]]] for g in range(n_groups)]

        def per_group_total(fn):
            def run():
                for g in groups:
                    fn(g)
            return _wall_ms(run, reps, gpu=False) * 1e3

        # The reference's arithmetic on the host: CPU torch for the advantages,
        # Python builtins for the filter.
        out["reference_grpo_advantage_us_all_groups"] = round(per_group_total(ogrpo.grpo_group), 1)
        out["reference_is_zero_variance_group_us_all_groups"] = round(per_group_total(ogrpo.zero_variance_group), 1)
    return out


def bench_end_to_end(runs, no_cpu):
    """The composed path at T = 16384: the 256 GRPO samples planned and packed
    (one host-to-device copy, GRPO, every micro), then over the first two
    micros (8192 tokens each, rows [0, 16384) of one [16384, 151936] bf16
    logits tensor): fused logprob + entropy, PPO loss forward and backward, and
    the backward into the logits.  The CPU leg restates the same chain on the
    oracle; the entry reports both walls and the largest differences between
    the two chains' outputs."""
    from types import SimpleNamespace as NS

    import torch

    from meshy_amd import logprob, workloads
    from meshy_amd.loss import ppo_clip_loss
    from meshy_amd.pipeline import RaggedSamples, pack_step
    from meshy_amd.plan import PlannerConfig

    dev = torch.device("cuda:0")
    micro = 8192
    batch, rewards, group_offsets = workloads.grpo_256_samples(0)
    n = len(batch.lengths)
    ragged = RaggedSamples.from_arrays(batch.tokens, batch.mask, batch.logprobs, batch.offsets, rewards,
                                       group_offsets)
    cfg = PlannerConfig(layout="packed", mini_batch_size=n, seq_len=micro, align=2048, max_tokens_per_micro=micro)
    gen = torch.Generator(device=dev).manual_seed(5)
    logits = torch.randn(1, T_TOK, VOCAB, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0
    stub = NS(ppo_clip_eps_low=0.2, ppo_clip_eps_high=0.28, use_tis=False, use_icepop=False,
              calculate_per_token_loss=True, old_logprobs_source="rollout", sharder=None, parallel_dims=NS(cp=1))
    info = {}

    def gpu_step():
        res = pack_step(ragged, cfg, dev)
        mini = res.plan.per_rank[0][0]
        outs = []
        for j, mb in enumerate(res.batches[:T_TOK // micro]):
            if mb.input_ids.shape[1] != micro:
                raise RuntimeError("the first micros of the 256 GRPO samples are expected to be full")
            z = logits[:, j * micro:(j + 1) * micro].detach().requires_grad_(True)
            lp, ent = logprob.logprobs_and_entropy(z, mb.labels, with_entropy=True)
            lp.retain_grad()
            loss, sums = ppo_clip_loss(stub, lp, mb.rollout_logprobs, mb, mini, entropy=ent)
            loss.backward()
            outs.append((loss, sums, lp.grad, z.grad))
        info["outs"] = outs
        info["micros"] = len(res.batches)

    gpu_ms = _wall_ms(gpu_step, runs, warmup=2)
    out = {"gpu_ms": round(gpu_ms, 3), "tokens": T_TOK, "V": VOCAB, "packed_micros": info["micros"],
           "work": "pack 256 samples (all micros) + GRPO, then logprob+entropy, PPO fwd+bwd and the logits "
                   "backward over the first two 8192-token micros"}
    if not no_cpu:
        from oracle import batch as obatch
        from oracle import grpo as ogrpo
        from oracle import logprob as olp
        from oracle import plan as oplan
        from oracle import ppo as oppo

        samples = batch.sample_dicts(rewards=rewards)
        zc_all = logits.cpu()
        cinfo = {}

        def cpu_step():
            lengths, loss_t = oplan.sample_lengths(samples, micro)
            local, per_rank = oplan.build_plan(lengths, loss_t, 1, layout="packed", mini_batch_size=n,
                                               seq_len=micro, align=2048, max_tokens_per_micro=micro)
            adv = []
            for g in range(len(group_offsets) - 1):
                adv += ogrpo.grpo_group([float(r) for r in rewards[group_offsets[g]:group_offsets[g + 1]]])
            loc = [dict(samples[i], advantage=adv[i]) for i in local[0]]
            micros, n_docs_g, n_tok_g, _ = per_rank[0][0]
            mbcs = [obatch.build_micro_batch(loc, idx, seq_len, doc_lens, layout="packed", need_rollout_lp=True)
                    for idx, seq_len, doc_lens in micros]
            outs = []
            for j in range(T_TOK // micro):
                mbc = mbcs[j]
                z = zc_all[:, j * micro:(j + 1) * micro].float().requires_grad_(True)
                lp = olp.forward_logprobs(z, mbc["labels"])
                with torch.no_grad():
                    ent = olp.chunk_entropy(z.detach())
                lp.retain_grad()
                loss, sums = oppo.ppo_clip_loss(lp, mbc["rollout_logprobs"], mbc["mask"], mbc["doc_ids"],
                                                mbc["advantages"], mbc["n_docs"], n_docs_global=n_docs_g,
                                                n_tokens_global=n_tok_g, clip_low=0.2, clip_high=0.28,
                                                per_token_loss=True, entropy=ent,
                                                rollout_lp=mbc["rollout_logprobs"])
                loss.backward()
                outs.append((loss, sums, lp.grad, z.grad))
            cinfo["outs"] = outs

        cpu_ms = _wall_ms(cpu_step, 2, warmup=0, gpu=False)
        out["cpu_ms"] = round(cpu_ms, 1)
        out["cpu_threads"] = torch.get_num_threads()
        out["speedup_vs_cpu"] = round(cpu_ms / gpu_ms, 1)
        d_loss = d_sum = d_new = d_z = 0.0
        for (gl, gs, gn, gz), (cl, cs, cn, cz) in zip(info["outs"], cinfo["outs"]):
            d_loss = max(d_loss, abs(gl.item() - cl.item()))
            for k, v in cs.items():
                d_sum = max(d_sum, abs(float(gs[k]) - float(v)) / max(1.0, abs(float(v))))
            cn = cn.reshape(-1)
            d_new = max(d_new, (gn.reshape(-1).cpu() - cn).abs().max().item() / max(cn.abs().max().item(), 1e-30))
            for a in range(0, micro, 1024):
                diff = (gz[0, a:a + 1024].float().cpu() - cz[0, a:a + 1024]).abs()
                d_z = max(d_z, (diff / (cn[a:a + 1024, None].abs() + 1e-30)).max().item())
        out["max_abs_diff_loss"] = d_loss
        out["max_diff_sums_abs_or_rel"] = d_sum
        out["max_rel_diff_dloss_dnew_lp"] = d_new
        out["max_diff_dloss_dlogits_over_row_grad"] = d_z
    del logits
    info.clear()
    torch.cuda.empty_cache()
    return out


# One workload leg each, for `--leg NAME` (the full run calls them in main).
LEGS = {
    "pack": lambda a: bench_pack(20, a.no_cpu)[0],
    "opd": lambda a: bench_opd(*headline_inputs(), a.steps, a.warmup, a.no_cpu),
    "ppo": lambda a: bench_ppo(a.steps, a.warmup, a.no_cpu),
    "gae": lambda a: bench_gae(a.steps, a.warmup, a.no_cpu),
    "gae_cache": lambda a: bench_gae_cache(a.steps),
    "critic": lambda a: bench_critic(a.steps, a.warmup, a.no_cpu),
    "attach_gae": lambda a: bench_attach_gae(5, a.no_cpu),
    "long_context": lambda a: bench_long_context(max(3, a.steps // 10), 2, a.no_cpu),
    "pack_long_context": lambda a: bench_pack_long_context(10, a.no_cpu),
    "rollout_metrics": lambda a: bench_rollout_metrics(10, a.no_cpu),
    "group_advantages": lambda a: bench_group_advantages(10, a.no_cpu),
    "end_to_end": lambda a: bench_end_to_end(5, a.no_cpu),
}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true", help="skip every CPU reference timing")
    ap.add_argument("--quick", action="store_true", help="headline kernel only")
    ap.add_argument("--pmc-kernels", action="store_true",
                    help="for counter runs: logprob + entropy, the plain read, Top-K (K = 8) and the logprob "
                         "backward x 3 each and a device copy x 3 over the [16384, 151936] logits, no JSON line")
    ap.add_argument("--pmc-workloads", action="store_true",
                    help="for counter runs: the pack, PPO, GAE, critic and whitening legs with a few steps each, "
                         "then a 256 MiB device copy x 3 to calibrate, no JSON line")
    ap.add_argument("--leg", choices=sorted(LEGS), help="run one workload leg and print its entry only")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the hot path's kernels run per GPU and no multi-GPU figure "
              "is produced (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    torch.set_num_threads(os.cpu_count() or 1)
    if args.pmc_kernels:
        return pmc_kernels()
    if args.pmc_workloads:
        return pmc_workloads()
    if args.leg:
        print(json.dumps({args.leg: LEGS[args.leg](args)}), flush=True)
        return 0

    logits, labels = headline_inputs()
    bwd = None
    if not args.quick:
        # The logits backward leg (its own entry below) runs first, on the device
        # only: the headline is then timed on a device that has been busy, as it
        # is right after a model forward in training.  Straight after process
        # start its first launches run ~2 % slower while the clocks rise.
        bwd = bench_logprob_bwd(logits, labels, max(5, args.steps // 2), 2)
    ms, nbytes = bench_logprob(logits, labels, args.steps, args.warmup)
    achieved = nbytes / (ms * 1e-3) / 1e9
    read_ceiling = bench_read_ceiling(logits, args.steps, args.warmup)
    traffic = traffic_src = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            stored = json.load(f).get("k_lpe_fwd_vec", {})
        traffic = stored.get("hbm_bytes_per_launch")
        traffic_src = ("stored, not measured in this run: FETCH_SIZE x 2 + WRITE_SIZE per launch from separate "
                       f"rocprofv3 --pmc runs, {stored.get('source')}")
    result = {
        "metric": "packed tokens/sec for logprob+entropy (V=151936) + % of HBM peak; pack latency",
        "value": T_TOK / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: logits N(0, 2^2) bf16 from a seeded generator, labels uniform in [0, V)",
        "config": {"workload": "fused packed logprob+entropy over one micro-batch of logits", "T": T_TOK,
                   "V": VOCAB, "global_batch": T_TOK, "seq_len": T_TOK, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "read_ceiling": round(read_ceiling, 1),
                     "frac_of_read_ceiling": round(achieved / read_ceiling, 4)},
    }
    if not args.no_cpu:
        tps, cms = cpu_logprob_tokens_per_s(logits, labels, args.cpu_rows)
        result["cpu_baseline"] = {
            "value": round(tps, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"first {args.cpu_rows} rows of the same [16384, 151936] bf16 logits, median of 5 "
                      f"after 1 warm-up ({cms:.1f} ms per pass)"}
    kernels = {"logprob_entropy_fwd_T16384_V151936": _entry(ms * 1e3, nbytes,
                                                             result.get("cpu_baseline") and
                                                             T_TOK / result["cpu_baseline"]["value"] * 1e3),
               "stream_read_ceiling_T16384_V151936": {"GBps": round(read_ceiling, 1),
                                                      "frac_hbm": round(read_ceiling / HBM_PEAK_GBS, 4)}}
    if not args.quick:
        bms, bbytes = bwd
        bcpu = None if args.no_cpu else cpu_logprob_bwd_ms(logits, labels, 512)
        kernels["logprob_bwd_T16384_V151936"] = _entry(bms * 1e3, bbytes, bcpu,
                                                       cpu_sample="512 rows, scaled to T" if bcpu else None)
        kernels["opd"] = bench_opd(logits, labels, args.steps, args.warmup, args.no_cpu)
    del logits, labels
    torch.cuda.empty_cache()
    if not args.quick:
        pack, _, _ = bench_pack(20, args.no_cpu)
        result["pack_latency_us"] = pack["pack_latency_us"]
        # the trainer's per-micro drop-in, the call the reference times as
        # train/pack_batch (median over the 23 micros)
        result["pack_latency_per_micro_us"] = pack["build_micro_batch_per_micro_us"]["median"]
        kernels["pack_grpo_256_samples"] = pack
        kernels.update(bench_ppo(args.steps, args.warmup, args.no_cpu))
        kernels["gae_returns_1024_docs"] = bench_gae(args.steps, args.warmup, args.no_cpu)
        kernels["logprob_entropy_16_long_sequences"] = bench_long_context(max(3, args.steps // 10), 2, args.no_cpu)
        kernels["critic"] = bench_critic(args.steps, args.warmup, args.no_cpu)
        kernels["attach_gae_1024_docs"] = bench_attach_gae(5, args.no_cpu)
        kernels["pack_16_long_sequences"] = bench_pack_long_context(10, args.no_cpu)
        kernels["rollout_metrics_256_samples"] = bench_rollout_metrics(10, args.no_cpu)
        kernels["group_advantages_32_groups_of_8"] = bench_group_advantages(10, args.no_cpu)
        result["kernels"] = kernels
        result["end_to_end"] = bench_end_to_end(5, args.no_cpu)
        if result.get("cpu_baseline"):
            result["cpu_baseline"]["host"] = _host_info()
    print(json.dumps(result), flush=True)
    return 0


def pmc_kernels() -> int:
    """The dispatches the counter runs read: each big kernel three times (the
    fused log-prob + entropy, the plain streaming read over the same logits,
    Top-K, the log-prob backward), then a device copy of known size
    (4,978,638,848 B) to calibrate."""
    import torch

    from meshy_amd import _lib, logprob, topk

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1)
    z = torch.randn(1, T_TOK, VOCAB, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0
    y = torch.randint(0, VOCAB, (1, T_TOK), generator=gen, device=dev)
    for _ in range(3):
        logprob.logprobs_and_entropy(z, y, with_entropy=True)
    lib = _lib.load()
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(3):
        _lib.check(lib.meshy_stream_read(z.data_ptr(), T_TOK, VOCAB * 2, sink.data_ptr(), _lib.stream_of(dev)),
                   "meshy_stream_read")
    for _ in range(3):
        topk.teacher_topk(z, 8)
    lse = logprob.logsumexp_rows(z)
    gl = torch.ones(1, T_TOK, device=dev)
    grad = torch.empty_like(z)
    ws = logprob.bwd_workspace(T_TOK, dev)
    for _ in range(3):
        _lib.check(lib.meshy_logprob_bwd(z.data_ptr(), 1, T_TOK, VOCAB, z.stride(0), z.stride(1), y.data_ptr(),
                                         lse.data_ptr(), gl.data_ptr(), grad.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream_of(dev)), "meshy_logprob_bwd")
    for _ in range(3):
        grad.copy_(z)
    torch.cuda.synchronize()
    print("pmc kernels done", flush=True)
    return 0


def pmc_workloads() -> int:
    """The dispatches of the per-workload traffic counter runs: the 256 GRPO
    samples' pack, the 512-document PPO loss, GAE over 1024 documents (with and
    without lengths), the critic reductions and whitening, a few times each;
    then a device copy of exactly 268,435,456 B read and written, three times,
    to calibrate the counters."""
    import numpy as np
    import torch

    from meshy_amd import workloads
    from meshy_amd.gae import gae_and_returns

    bench_pack(3, True)
    bench_ppo(3, 1, True)
    bench_gae(3, 1, True)
    dev = torch.device("cuda:0")
    batch, values, terminal = workloads.gae_1024_docs(4)
    n = len(batch.lengths)
    doc_ids = torch.from_numpy(np.repeat(np.arange(n), batch.lengths)).reshape(1, -1).to(dev)
    r = torch.zeros(1, batch.total, device=dev)
    v = torch.from_numpy(values).to(torch.bfloat16).reshape(1, -1).to(dev)
    m = torch.from_numpy(batch.mask).reshape(1, -1).to(dev)
    for _ in range(3):
        gae_and_returns(r, v, m, doc_ids, n, gamma=1.0, alpha=1.5)  # masked lengths counted (k_gae_doc_count)
    bench_critic(3, 1, True)
    src = torch.ones(64 * 1024 * 1024, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc workloads done", flush=True)
    return 0


def _host_info():
    import platform

    model = platform.processor()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count()}


if __name__ == "__main__":
    sys.exit(main())

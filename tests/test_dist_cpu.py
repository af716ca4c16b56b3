"""The cross-rank reductions of the loss metrics over a real process group (CPU,
gloo, world size 2): each rank's sums are all-reduced on the ``loss`` mesh
(trainer.py:1020-1047, opd.py:234-251) and must give the metrics of one process
holding both ranks' sums."""

from __future__ import annotations

import os
import socket
from types import SimpleNamespace as NS

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

PPO_KEYS = ("loss", "total_loss", "positive_lm_loss", "tis_ratio_sum", "ratio_sum", "clip_sum", "tis_masked_sum",
            "token_count", "ppo_kl_sum", "log_ratio_abs_sum", "ess_sum", "doc_count", "train_rollout_kl_sum",
            "train_rollout_logdiff_abs_sum", "entropy_sum")
OPD_KEYS = ("loss", "token_count", "student_mass_sum", "teacher_mass_sum", "train_rollout_kl_sum",
            "train_rollout_logdiff_abs_sum")


def _sums(keys, rank):
    g = torch.Generator().manual_seed(100 + rank)
    vals = torch.rand(len(keys), generator=g) * 10 + 1
    return {k: vals[i].clone() for i, k in enumerate(keys)}


class _Mesh:
    def get_group(self):
        return dist.group.WORLD


def _stub():
    return NS(parallel_dims=NS(get_optional_mesh=lambda name: _Mesh() if name == "loss" else None))


def _worker(rank, world, port, q):
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        from meshy_amd import loss, opd

        ppo = loss.reduce_mini_metrics(_stub(), _sums(PPO_KEYS, rank))
        dis = opd.reduce_distill_metrics(_stub(), _sums(OPD_KEYS, rank))
        q.put((rank, ppo, dis))
    finally:
        dist.destroy_process_group()


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def test_metric_all_reduce_over_two_ranks():
    from meshy_amd import loss, opd

    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_worker, args=(r, 2, port, q)) for r in range(2)]
    for p in procs:
        p.start()
    results = [q.get(timeout=120) for _ in procs]
    for p in procs:
        p.join(timeout=60)
        assert p.exitcode == 0
    total_ppo = {k: _sums(PPO_KEYS, 0)[k] + _sums(PPO_KEYS, 1)[k] for k in PPO_KEYS}
    total_opd = {k: _sums(OPD_KEYS, 0)[k] + _sums(OPD_KEYS, 1)[k] for k in OPD_KEYS}
    want_ppo = loss.reduce_mini_metrics(NS(), total_ppo)
    want_opd = opd.reduce_distill_metrics(NS(), total_opd)
    for _, ppo, dis in results:
        assert ppo.keys() == want_ppo.keys() and dis.keys() == want_opd.keys()
        for k in want_ppo:
            assert ppo[k] == pytest.approx(want_ppo[k], rel=1e-6), k
        for k in want_opd:
            assert dis[k] == pytest.approx(want_opd[k], rel=1e-6), k

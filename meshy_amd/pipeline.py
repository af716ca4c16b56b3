"""The packed step between rollout and trainer, end to end, with one host-to-device copy.

``RaggedSamples`` holds one step's samples as flat pinned host arrays (tokens,
assistant mask, rollout logprobs, per-sample rewards and group offsets) plus
room for the plan tables: the jagged layout the rollout's columns already use.
``pack_step`` then

1. counts tokens and loss tokens per sample on the host (``meshy_sample_loss_tokens``,
   trainer.py:577-588) and plans the batch (``meshy_plan_build``, plan.py:211-288);
2. writes the rank's micro tables into the same pinned buffer and copies it to
   the device in ONE transfer;
3. normalises rewards per group (``meshy_grpo_advantage``, rollout.py:88-97) and
   materialises every micro of the rank (``meshy_pack_micro_batches``,
   batch.py:96-230).  Documents index the samples' global positions, so no gather
   is needed between the two kernels.
"""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np
import torch

from . import _lib
from .batch import Batch, PackJob, _Layout, launch_pack
from .hostio import gather_into
from .plan import Plan, PlannerConfig, plan_tables, tables_to_plan
from .wire import jagged_parts


_NP_DTYPES = {torch.int32: np.int32, torch.int64: np.int64, torch.float32: np.float32}


class RaggedSamples:
    """One step's samples as flat pinned host arrays, in global sample order."""

    def __init__(self, lengths: np.ndarray, n_groups: int, need_rollout_lp: bool,
                 token_dtype: torch.dtype = torch.int32) -> None:
        n = len(lengths)
        self.n = n
        self.lengths = np.asarray(lengths, np.int64)
        self.offsets = np.zeros(n + 1, np.int64)
        np.cumsum(self.lengths, out=self.offsets[1:])
        self.total = int(self.offsets[-1])
        self.need_rollout_lp = need_rollout_lp
        lay = _Layout()
        if token_dtype not in (torch.int32, torch.int64):
            raise ValueError("token ids are staged as int32 or int64")
        lay.add("tokens", self.total, token_dtype)
        lay.add("mask", self.total, torch.float32)
        if need_rollout_lp:
            lay.add("logprobs", self.total, torch.float32)
        lay.add("s_off", n + 1, torch.int64)
        lay.add("rewards", max(n, 1), torch.float32)
        lay.add("group_off", n_groups + 1, torch.int64)
        lay.add("pos_w", max(n, 1), torch.float32)
        # Everything above is the samples' and goes to the device as soon as a
        # pack starts; the plan tables below follow once they are computed.
        self.tables_at = lay.size
        # plan tables of one rank: at most n micros and n documents
        lay.add("seq", max(n, 1), torch.int64)
        lay.add("out_off", n + 1, torch.int64)
        lay.add("doc_len", max(n, 1), torch.int64)
        lay.add("doc_start", n + 1, torch.int32)
        lay.add("doc_sample", max(n, 1), torch.int32)
        lay.add("adv_samples", max(n, 1), torch.float32)  # written on the device
        self.lay = lay
        self.n_groups = n_groups
        # Pinned when a device is present, so the one copy to it is a DMA.
        self.buf = torch.empty(lay.size, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        self._np_buf = self.buf.numpy()
        self._np: dict[str, np.ndarray] = {}
        self.copied = None  # event of the last copy of the plan tables out of buf
        self.view("s_off").copy_(torch.from_numpy(self.offsets))
        self.view("pos_w").zero_()

    def view(self, name: str) -> torch.Tensor:
        return self.lay.view(self.buf, name)

    def np_view(self, name: str) -> np.ndarray:
        """The region as a numpy array over the same pinned memory (cached)."""
        v = self._np.get(name)
        if v is None:
            lo, hi, dtype = self.lay.regions[name]
            v = self._np_buf[lo:hi].view(_NP_DTYPES[dtype])
            self._np[name] = v
        return v

    @classmethod
    def from_arrays(cls, tokens, mask, logprobs, offsets, rewards, group_offsets) -> "RaggedSamples":
        """From flat numpy arrays (sample i = [offsets[i], offsets[i+1]))."""
        offsets = np.asarray(offsets, np.int64)
        r = cls(np.diff(offsets), len(group_offsets) - 1, logprobs is not None)
        r.view("tokens").copy_(torch.from_numpy(np.ascontiguousarray(tokens, np.int32)))
        r.view("mask").copy_(torch.from_numpy(np.ascontiguousarray(mask, np.float32)))
        if logprobs is not None:
            r.view("logprobs").copy_(torch.from_numpy(np.ascontiguousarray(logprobs, np.float32)))
        r.view("rewards")[:r.n] = torch.from_numpy(np.ascontiguousarray(rewards, np.float32))
        r.view("group_off").copy_(torch.from_numpy(np.asarray(group_offsets, np.int64)))
        return r

    @classmethod
    def from_samples(cls, samples: Sequence[Any], group_offsets, need_rollout_lp: bool = True) -> "RaggedSamples":
        """From TensorDict-like samples (``tokens``, ``mask_assistant``, ``logprobs``, ``reward``)."""
        toks = [s["tokens"] for s in samples]
        lengths = np.array([t.shape[0] if isinstance(t, torch.Tensor) else len(t) for t in toks], np.int64)
        # int64 ids (the reference's dtype) are staged as they are, others as int32.
        tok64 = all(isinstance(t, torch.Tensor) and t.dtype == torch.int64 for t in toks)
        r = cls(lengths, len(group_offsets) - 1, need_rollout_lp, torch.int64 if tok64 else torch.int32)
        gather_into(toks, r.view("tokens"))
        gather_into([s["mask_assistant"] for s in samples], r.view("mask"))
        if need_rollout_lp:
            gather_into([s["logprobs"] for s in samples], r.view("logprobs"))
        r.view("rewards")[:r.n] = torch.tensor([float(s["reward"]) for s in samples], dtype=torch.float32)
        r.view("group_off").copy_(torch.as_tensor(np.asarray(group_offsets, np.int64)))
        return r

    @classmethod
    def from_columns(cls, columns, group_offsets, need_rollout_lp: bool = True) -> "RaggedSamples":
        """From a batch of wire columns (``meshy_amd.wire``, adapter.py:39-132): the
        jagged ``tokens`` / ``mask_assistant`` / ``logprobs`` columns are copied from
        their flat ``values()`` in one pass each, ``reward`` from its ``[B, 1]`` column."""
        tok, off = jagged_parts(columns["tokens"])
        r = cls(torch.diff(off).numpy(), len(group_offsets) - 1, need_rollout_lp)
        r.view("tokens").copy_(tok.reshape(-1).to(torch.int32))
        names = ["mask_assistant"] + (["logprobs"] if need_rollout_lp else [])
        for name, region in zip(names, ["mask", "logprobs"]):
            flat, o = jagged_parts(columns[name])
            if not torch.equal(o.cpu(), off.cpu()):
                raise ValueError(f"column {name!r} is not as long as 'tokens' in every sample")
            r.view(region).copy_(flat.reshape(-1).to(torch.float32))
        r.view("rewards")[:r.n] = torch.as_tensor(columns["reward"]).reshape(-1).to(torch.float32)
        r.view("group_off").copy_(torch.as_tensor(np.asarray(group_offsets, np.int64)))
        return r

    def sample_lengths(self, seq_len: int) -> tuple[np.ndarray, np.ndarray]:
        """(token count, loss tokens) per sample, natively (trainer.py:577-588)."""
        lengths = np.empty(self.n, np.int64)
        loss = np.empty(self.n, np.int64)
        rc = _lib.load().meshy_sample_loss_tokens(
            self.view("mask").data_ptr(), self.offsets.ctypes.data, self.n, seq_len,
            lengths.ctypes.data, loss.ctypes.data)
        _lib.check(rc, "meshy_sample_loss_tokens")
        return lengths, loss


class PackResult:
    """A packed step: the plan (the reference's dataclasses, built from the
    flat tables the first time ``plan`` is read), the tables, one ``Batch`` per
    micro of the rank and the per-sample advantages on the device."""

    def __init__(self, plan: Plan | None, tables, batches: list[Batch], advantages: torch.Tensor) -> None:
        self._plan = plan
        self.tables = tables
        self.batches = batches
        self.advantages = advantages

    @property
    def plan(self) -> Plan:
        if self._plan is None:
            self._plan = tables_to_plan(self.tables)
        return self._plan


def pack_step(ragged: RaggedSamples, cfg: PlannerConfig, device, *, dp_size: int = 1, rank: int = 0,
              with_plan_objects: bool = False, broadcast_advantages: bool = True) -> PackResult:
    """Plan, copy, normalise rewards and build every micro of ``rank``.

    The samples' part of the staging buffer is copied to the device first, so
    the transfer runs while the host plans; the plan tables follow in a second,
    small copy.  The Plan dataclasses are built when ``PackResult.plan`` is
    first read (``with_plan_objects`` builds them here)."""
    device = torch.device(device)
    stream = torch.cuda.current_stream(device)
    lay = ragged.lay
    dbuf = torch.empty(lay.size, dtype=torch.uint8, device=device)
    cut = ragged.tables_at
    dbuf[:cut].copy_(ragged.buf[:cut], non_blocking=True)
    lengths, loss = ragged.sample_lengths(cfg.seq_len)
    t = plan_tables(lengths, loss, dp_size, cfg)
    if ragged.copied is not None:
        ragged.copied.synchronize()  # the tables below reuse the pinned buffer
    n_local = t.n_local
    nm = t.n_micro_total
    seq = t.micro_seq_len[rank * n_local: rank * n_local + nm]
    start = t.micro_doc_start[rank * (n_local + 1): rank * (n_local + 1) + nm + 1]
    local = t.local_indices[rank * n_local:(rank + 1) * n_local]
    dsample = local[t.doc_sample[rank * n_local:(rank + 1) * n_local]]  # global sample index
    dlen = t.doc_len[rank * n_local:(rank + 1) * n_local]
    n_docs = np.diff(start)
    packed = cfg.layout == "packed"
    rows = np.ones(nm, np.int64) if packed else np.maximum(n_docs, 1)
    elems = seq * rows
    out_off = np.zeros(nm + 1, np.int64)
    np.cumsum(elems, out=out_off[1:])
    ragged.np_view("seq")[:nm] = seq
    ragged.np_view("out_off")[:nm + 1] = out_off
    ragged.np_view("doc_start")[:nm + 1] = start
    nd_total = int(start[-1])
    ragged.np_view("doc_sample")[:nd_total] = dsample[:nd_total]
    ragged.np_view("doc_len")[:nd_total] = dlen[:nd_total]

    dbuf[cut:].copy_(ragged.buf[cut:], non_blocking=True)
    ragged.copied = torch.cuda.Event()
    ragged.copied.record(stream)

    adv = lay.view(dbuf, "adv_samples")[:ragged.n]
    rc = _lib.load().meshy_grpo_advantage(lay.view(dbuf, "rewards").data_ptr(), ragged.n,
                                          lay.view(dbuf, "group_off").data_ptr(), ragged.n_groups, adv.data_ptr(),
                                          stream.cuda_stream)
    _lib.check(rc, "meshy_grpo_advantage")

    sq, st, dl = seq.tolist(), start.tolist(), dlen[:nd_total].tolist()
    micros = tuple(_LiteMicro(sq[k], st[k + 1] - st[k], sum(dl[st[k]:st[k + 1]]), tuple(dl[st[k]:st[k + 1]]))
                   for k in range(nm))
    job = PackJob(
        micros=micros, layout=cfg.layout, device=device, dbuf=dbuf, lay=lay,
        need_rollout_lp=ragged.need_rollout_lp, per_token_adv=False, n_samples=ragged.n, seq=seq,
        rows=rows, out_off=out_off, doc_start=start, max_elems=int(elems.max()) if nm else 0,
        max_docs=int(n_docs.max()) if nm else 0, adv_samples=adv, broadcast_advantages=broadcast_advantages,
    )
    batches = launch_pack(job)
    return PackResult(tables_to_plan(t) if with_plan_objects else None, t, batches, adv)


class _LiteMicro:
    """What ``launch_pack`` reads of a MicroPlan, without building the dataclasses."""

    __slots__ = ("seq_len", "n_docs", "n_tokens", "doc_lens")
    is_filler = property(lambda self: self.n_docs == 0)

    def __init__(self, seq_len: int, n_docs: int, n_tokens: int, doc_lens: tuple) -> None:
        self.seq_len = seq_len
        self.n_docs = n_docs
        self.n_tokens = n_tokens
        self.doc_lens = doc_lens

    @property
    def n_rows(self) -> int:
        return max(1, self.n_docs)


__all__ = ["PackResult", "RaggedSamples", "pack_step"]

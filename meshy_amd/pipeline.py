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
from .plan import Plan, PlannerConfig, PlanTables, tables_to_plan
from .wire import jagged_parts


_NP_DTYPES = {torch.int32: np.int32, torch.int64: np.int64, torch.float32: np.float32, torch.uint8: np.uint8}


class RaggedSamples:
    """One step's samples as flat pinned host arrays, in global sample order."""

    def __init__(self, lengths: np.ndarray, n_groups: int, need_rollout_lp: bool,
                 token_dtype: torch.dtype = torch.int32, mask_u8: bool = False) -> None:
        """``mask_u8`` stages the mask as one byte per token (for masks of only
        0 and 1: a quarter of the mask's copy to the device, the same values
        in the batches); the constructors below choose it when they can."""
        n = len(lengths)
        self.mask_u8 = bool(mask_u8)
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
        lay.add("mask", self.total, torch.uint8 if self.mask_u8 else torch.float32)
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
        self.adv_at = lay.size  # the second copy ends here
        lay.add("adv_samples", max(n, 1), torch.float32)  # written on the device, last
        self.lay = lay
        self.n_groups = n_groups
        # Pinned when a device is present, so the one copy to it is a DMA.
        self.buf = torch.empty(lay.size, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        self._np_buf = self.buf.numpy()
        self._np: dict[str, np.ndarray] = {}
        self.copied = None  # event of the last copy of the plan tables out of buf
        self._step_args = None  # meshy_step_plan's struct over this buffer
        self._cfg_key = None  # the settings last written into it
        self._stream = None  # (raw handle, torch Stream) of the last copy's stream
        self.view("s_off").copy_(torch.from_numpy(self.offsets))
        self.view("pos_w").zero_()

    def view(self, name: str) -> torch.Tensor:
        return self.lay.view(self.buf, name)

    def step_plan_args(self, cfg: PlannerConfig, dp_size: int, rank: int, tables: PlanTables) -> "_lib.StepPlanArgs":
        """The argument struct of ``meshy_step_plan`` for this step: the staged
        mask and offsets, scratch for the counts, ``tables`` for the plan and
        this buffer's pack-table regions (the pointers made once)."""
        a = self._step_args
        if a is None:
            a = self._step_args = _lib.StepPlanArgs()
            base = self.buf.data_ptr()
            self._counts = np.empty((2, self.n), np.int64)
            a.mask = self.lay.addr(base, "mask")
            a.mask_u8 = int(self.mask_u8)
            a.offsets = self.lay.addr(base, "s_off")
            a.n = self.n
            a.lengths = self._counts[0].ctypes.data
            a.loss_tokens = self._counts[1].ctypes.data
            for field, region in (("micro_seq_len", "seq"), ("micro_out_off", "out_off"),
                                  ("micro_doc_start", "doc_start"), ("doc_sample", "doc_sample"),
                                  ("doc_len", "doc_len")):
                setattr(a, field, self.lay.addr(base, region))
        # The planner settings are written when they change (a step's config
        # repeats from step to step).
        key = (dp_size, rank, cfg.layout, cfg.mini_batch_size, cfg.seq_len, cfg.align, cfg.max_tokens_per_micro,
               cfg.micro_batch_size)
        if key != self._cfg_key:
            self._cfg_key = key
            a.dp_size, a.rank = dp_size, rank
            c = a.cfg
            c.layout = _lib.MESHY_LAYOUT_PACKED if cfg.layout == "packed" else _lib.MESHY_LAYOUT_PADDED
            c.mini_batch_size = cfg.mini_batch_size
            c.seq_len = cfg.seq_len
            c.align = cfg.align
            c.max_tokens_per_micro = cfg.max_tokens_per_micro or 0
            c.micro_batch_size = cfg.micro_batch_size or 0
        a.plan = tables.c_struct()
        return a

    def record_copy(self, device: torch.device) -> None:
        """Marks the end of the copy just queued out of this buffer (on the
        current stream of ``device``), which the next step waits for before it
        rewrites the plan tables."""
        ev = self.copied
        if ev is None:
            ev = self.copied = torch.cuda.Event()
        # The stream object is kept while the device's current stream stays the
        # same (building one per call costs more than the rest of the record).
        handle = _lib.stream_of(device)
        if self._stream is None or self._stream[0] != handle:
            self._stream = (handle, torch.cuda.current_stream(device))
        ev.record(self._stream[1])

    def np_view(self, name: str) -> np.ndarray:
        """The region as a numpy array over the same pinned memory (cached)."""
        v = self._np.get(name)
        if v is None:
            lo, hi, dtype = self.lay.regions[name]
            v = self._np_buf[lo:hi].view(_NP_DTYPES[dtype])
            self._np[name] = v
        return v

    @classmethod
    def _with_mask(cls, make, parts) -> "RaggedSamples":
        """``make(mask_u8)`` with its mask region filled from ``parts`` (the
        samples' masks in order): as bytes when every part is a CPU contiguous
        fp32 tensor holding only 0 and 1 (one native pass converts and
        checks), else as fp32."""
        if parts and all(isinstance(p, torch.Tensor) and p.device.type == "cpu" and p.dtype == torch.float32
                         and p.is_contiguous() for p in parts):
            r = make(True)
            ptrs = np.array([p.data_ptr() for p in parts], np.uint64)
            counts = np.array([p.numel() for p in parts], np.int64)
            binary = _lib.ctypes.c_int32(0)
            _lib.check(_lib.load().meshy_host_gather_mask_u8(ptrs.ctypes.data, counts.ctypes.data, len(parts),
                                                             r.view("mask").data_ptr(), 0, _lib.ctypes.byref(binary)),
                       "meshy_host_gather_mask_u8")
            if binary.value:
                return r
        r = make(False)
        gather_into(parts, r.view("mask"))
        return r

    @classmethod
    def from_arrays(cls, tokens, mask, logprobs, offsets, rewards, group_offsets) -> "RaggedSamples":
        """From flat numpy arrays (sample i = [offsets[i], offsets[i+1]))."""
        offsets = np.asarray(offsets, np.int64)
        m = torch.from_numpy(np.ascontiguousarray(mask, np.float32))
        r = cls._with_mask(lambda u8: cls(np.diff(offsets), len(group_offsets) - 1, logprobs is not None,
                                          mask_u8=u8), [m])
        r.view("tokens").copy_(torch.from_numpy(np.ascontiguousarray(tokens, np.int32)))
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
        tdt = torch.int64 if tok64 else torch.int32
        r = cls._with_mask(lambda u8: cls(lengths, len(group_offsets) - 1, need_rollout_lp, tdt, mask_u8=u8),
                           [s["mask_assistant"] for s in samples])
        gather_into(toks, r.view("tokens"))
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
        flats = {}
        for name in ["mask_assistant"] + (["logprobs"] if need_rollout_lp else []):
            flat, o = jagged_parts(columns[name])
            if not torch.equal(o.cpu(), off.cpu()):
                raise ValueError(f"column {name!r} is not as long as 'tokens' in every sample")
            flats[name] = flat.reshape(-1).to(device="cpu", dtype=torch.float32).contiguous()
        lengths = torch.diff(off).numpy()
        r = cls._with_mask(lambda u8: cls(lengths, len(group_offsets) - 1, need_rollout_lp, mask_u8=u8),
                           [flats["mask_assistant"]])
        r.view("tokens").copy_(tok.reshape(-1).to(torch.int32))
        if need_rollout_lp:
            r.view("logprobs").copy_(flats["logprobs"])
        r.view("rewards")[:r.n] = torch.as_tensor(columns["reward"]).reshape(-1).to(torch.float32)
        r.view("group_off").copy_(torch.as_tensor(np.asarray(group_offsets, np.int64)))
        return r

    def sample_lengths(self, seq_len: int) -> tuple[np.ndarray, np.ndarray]:
        """(token count, loss tokens) per sample, natively (trainer.py:577-588)."""
        lengths = np.empty(self.n, np.int64)
        loss = np.empty(self.n, np.int64)
        lib = _lib.load()
        fn = lib.meshy_sample_loss_tokens_u8 if self.mask_u8 else lib.meshy_sample_loss_tokens
        rc = fn(self.view("mask").data_ptr(), self.offsets.ctypes.data, self.n, seq_len,
                lengths.ctypes.data, loss.ctypes.data)
        _lib.check(rc, "meshy_sample_loss_tokens")
        return lengths, loss


class PackResult:
    """A packed step: the plan (the reference's dataclasses, built from the
    flat tables the first time ``plan`` is read), the tables, one ``Batch`` per
    micro of the rank and the per-sample advantages on the device."""

    def __init__(self, plan: Plan | None, tables, batches: list[Batch], advantages) -> None:
        self._plan = plan
        self.tables = tables
        self.batches = batches
        # A device tensor, or (buffer, layout, n): its view, made when first read.
        self._adv = advantages

    @property
    def advantages(self) -> torch.Tensor:
        adv = self._adv
        if isinstance(adv, tuple):
            buf, lay, n = adv
            adv = self._adv = lay.view(buf, "adv_samples")[:n]
        return adv

    @property
    def plan(self) -> Plan:
        if self._plan is None:
            self._plan = tables_to_plan(self.tables)
        return self._plan


def pack_step(ragged: RaggedSamples, cfg: PlannerConfig, device, *, dp_size: int = 1, rank: int = 0,
              with_plan_objects: bool = False, broadcast_advantages: bool = True) -> PackResult:
    """Plan, copy, normalise rewards and build every micro of ``rank``.

    The samples' part of the staging buffer is copied to the device first and
    the GRPO kernel queued behind it, so both run while the host plans.  One
    native call
    (``meshy_step_plan``) counts the loss tokens, plans and writes this rank's
    pack tables into the staging buffer; they follow in a second, small copy.
    The Plan dataclasses are built when ``PackResult.plan`` is first read
    (``with_plan_objects`` builds them here)."""
    device = torch.device(device)
    handle = _lib.stream_of(device)
    lay = ragged.lay
    lib = _lib.load()
    dbuf = torch.empty(lay.size, dtype=torch.uint8, device=device)
    base = dbuf.data_ptr()
    hbase = ragged.buf.data_ptr()
    cut = ragged.tables_at
    # Raw asynchronous copies from the pinned buffer, on the device's current
    # stream; the buffer outlives them (ragged.copied marks the second).
    if dp_size <= 0 or ragged.n % dp_size != 0:
        raise ValueError(
            f"batch size {ragged.n} is not divisible by DP size {dp_size}; adjust "
            "rollout.batch_size * group_size to a multiple of dp_replicate * dp_shard"
        )
    _lib.check(lib.meshy_copy_to_device(base, hbase, cut, handle), "meshy_copy_to_device")
    # GRPO reads only the rewards and group offsets of the first copy: it runs
    # while the host plans.  Its output region lies past the plan tables, so
    # the second copy stops short of it.
    adv = lay.addr(base, "adv_samples")
    rc = lib.meshy_grpo_advantage(lay.addr(base, "rewards"), ragged.n, lay.addr(base, "group_off"), ragged.n_groups,
                                  adv, handle)
    _lib.check(rc, "meshy_grpo_advantage")
    if ragged.copied is not None:
        ragged.copied.synchronize()  # the tables below reuse the pinned buffer the last copy read
    t = PlanTables(ragged.n, dp_size, cfg.mini_batch_size)
    a = ragged.step_plan_args(cfg, dp_size, rank, t)
    _lib.check(lib.meshy_step_plan(_lib.ctypes.byref(a)), "meshy_step_plan")
    t.n_micro_total = int(a.plan.n_micro_total)
    nm, nd_total = int(a.n_micro), int(a.n_docs)

    _lib.check(lib.meshy_copy_to_device(base + cut, hbase + cut, ragged.adv_at - cut, handle), "meshy_copy_to_device")
    ragged.record_copy(device)

    seq = ragged.np_view("seq")[:nm]
    start = ragged.np_view("doc_start")[:nm + 1]
    out_off = ragged.np_view("out_off")[:nm + 1]
    packed = cfg.layout == "packed"
    job = PackJob.fast(
        micros=_LiteMicros(seq, start, ragged.np_view("doc_len")[:nd_total]),
        layout=cfg.layout, device=device, dbuf=dbuf, lay=lay,
        need_rollout_lp=ragged.need_rollout_lp, per_token_adv=False, n_samples=ragged.n, seq=seq,
        rows=np.ones(nm, np.int64) if packed else np.maximum(np.diff(start), 1), out_off=out_off, doc_start=start,
        max_elems=int(a.max_micro_elems), max_docs=int(a.max_docs_per_micro), adv_samples=adv,
        broadcast_advantages=broadcast_advantages, stream=handle, mask_u8=ragged.mask_u8,
    )
    batches = launch_pack(job)
    return PackResult(tables_to_plan(t) if with_plan_objects else None, t, batches, (dbuf, lay, ragged.n))


class _LiteMicros:
    """The micros of a step as ``launch_pack`` reads them, each made on first
    use from the plan's tables (numpy views, read as lists the first time a
    micro is needed; no dataclass per micro)."""

    __slots__ = ("_arrays", "_lists", "_n", "_made")

    def __init__(self, seq, start, dlen) -> None:
        self._arrays = (seq, start, dlen)
        self._lists = None
        self._n = len(seq)
        self._made: dict = {}

    def __len__(self) -> int:
        return self._n

    def __getitem__(self, k: int) -> "_LiteMicro":
        m = self._made.get(k)
        if m is None:
            if not -self._n <= k < self._n:
                raise IndexError(k)
            k %= self._n
            if self._lists is None:
                self._lists = tuple(x.tolist() for x in self._arrays)
            seq, start, dlen = self._lists
            a, b = start[k], start[k + 1]
            dl = tuple(dlen[a:b])
            m = self._made[k] = _LiteMicro(seq[k], b - a, sum(dl), dl)
        return m

    def __iter__(self):
        return (self[k] for k in range(self._n))


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

"""Micro-batch materialisation with the call surface of meshy/backend/titan/batch.py.

``build_micro_batch`` (batch.py:96-230) builds one micro; ``build_micro_batches``
builds any number of micros of one rank in one go.  Either way the samples'
tokens, masks, rollout logprobs and per-token advantages are gathered into one
pinned staging buffer next to the plan tables, copied to the device in ONE
host-to-device transfer, and laid out by the ``meshy_pack_micro_batches``
kernel: per-document shift-by-one, doc ids with the padding slot, per-document
positions and ``cu_seqlens`` (a device prefix scan).  ``Batch`` keeps the
reference's fields (batch.py:52-74) so the forward and the loss read it as is.
"""

from __future__ import annotations

from dataclasses import MISSING, dataclass, fields
from typing import Any, NamedTuple, Sequence

import numpy as np
import torch

from . import _lib
from .hostio import gather_into
from .plan import Layout, MicroPlan

#: Per-token advantage column (batch.py:81): already on the next-token grid,
#: laid out like rollout logprobs but not shifted again.
ADVANTAGE_TOKENS = "advantage_tokens"

#: OPD Teacher columns of a sample (meshy/config.py:506), ``[L, K]`` each.
TEACHER_FIELDS = ("teacher_topk_ids", "teacher_topk_logprobs")


class VarlenMetadata(NamedTuple):
    """Document boundaries for variable-length attention.

    Same fields as torchtitan's ``VarlenMetadata`` (cu_seq_q, cu_seq_k, max_q,
    max_k), which batch.py:233-243 constructs.
    """

    cu_seq_q: torch.Tensor
    cu_seq_k: torch.Tensor
    max_q: int
    max_k: int


@dataclass
class Batch:
    """One micro-batch, next-token aligned (batch.py:52-74)."""

    input_ids: torch.Tensor
    labels: torch.Tensor
    positions: torch.Tensor
    mask: torch.Tensor
    doc_ids: torch.Tensor
    advantages: torch.Tensor
    rollout_logprobs: torch.Tensor | None
    lengths: torch.Tensor
    n_docs: int
    attention_masks: Any = None
    positive_lm_weights: torch.Tensor | None = None
    #: Per-document advantages broadcast over the micro's tokens (padding slot
    #: 0), i.e. the ``adv_tok`` the loss derives (trainer.py:753-756); only
    #: filled when the pack is asked for it.
    advantage_tokens: torch.Tensor | None = None

    @property
    def n_slots(self) -> int:
        """Segment-buffer size: one slot per sample plus one for padding."""
        return self.n_docs + 1


def make_varlen_metadata(cu_seqlens, max_len: int, device) -> VarlenMetadata:
    """VarlenMetadata from explicit document boundaries (batch.py:233-243)."""
    cu = cu_seqlens if isinstance(cu_seqlens, torch.Tensor) else torch.tensor(
        list(cu_seqlens), dtype=torch.int32)
    cu = cu.to(device=device, dtype=torch.int32)
    return VarlenMetadata(cu_seq_q=cu, cu_seq_k=cu, max_q=int(max_len), max_k=int(max_len))


class _Staging:
    """A grow-only pinned host buffer, reused once its last copy has landed."""

    def __init__(self) -> None:
        self.buf: torch.Tensor | None = None
        self.np: np.ndarray | None = None  # the same pinned memory, as numpy
        self.event = None
        self._stream = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.event is not None:
            self.event.synchronize()
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, pin_memory=True)
            self.np = self.buf.numpy()
        return self.buf

    def mark(self, device: torch.device, handle: int) -> None:
        """Records the end of the copy just queued out of the buffer, on the
        stream whose raw handle is ``handle`` (the stream object is kept while
        the device's current stream stays the same)."""
        if self.event is None:
            self.event = torch.cuda.Event()
        if self._stream is None or self._stream[0] != handle:
            self._stream = (handle, torch.cuda.current_stream(device))
        self.event.record(self._stream[1])


_STAGING: dict[int, _Staging] = {}


class _Layout:
    """Byte layout of the staging buffer: 256-byte aligned regions."""

    def __init__(self) -> None:
        self.size = 0
        self.regions: dict[str, tuple[int, int, torch.dtype]] = {}

    def add(self, name: str, n: int, dtype: torch.dtype) -> None:
        nbytes = n * (_ITEMSIZE.get(dtype) or dtype.itemsize)
        self.regions[name] = (self.size, self.size + nbytes, dtype)
        self.size += (nbytes + 255) // 256 * 256

    def view(self, buf: torch.Tensor, name: str) -> torch.Tensor:
        lo, hi, dtype = self.regions[name]
        return buf[lo:hi].view(dtype)

    def addr(self, base: int, name: str) -> int:
        """Address of a region inside a buffer that starts at ``base``."""
        return base + self.regions[name][0]

    def np_view(self, buf: np.ndarray, name: str) -> np.ndarray:
        """The region of a uint8 numpy buffer as a numpy array of its dtype."""
        lo, hi, dtype = self.regions[name]
        return buf[lo:hi].view(_NP_DTYPE[dtype])


_NP_DTYPE = {torch.int32: np.int32, torch.int64: np.int64, torch.float32: np.float32, torch.uint8: np.uint8}
# dtype.itemsize is a property call; a dict lookup is a tenth of it.
_ITEMSIZE = {d: d.itemsize for d in (torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64, torch.float16,
                                      torch.bfloat16, torch.float32, torch.float64, torch.bool)}


# Records of meshy_amd._stage.columns: one per used sample.
_REC = np.dtype([("ptr", "<u8"), ("dim0", "<i8"), ("row", "<i8"), ("dtype", "<i4"), ("flags", "<i4")])
# c10::ScalarType codes of the dtypes the staging writes.
_SCALAR_TYPE = {torch.uint8: 0, torch.int8: 1, torch.int16: 2, torch.int32: 3, torch.int64: 4, torch.float16: 5,
                torch.float32: 6, torch.float64: 7, torch.bool: 11, torch.bfloat16: 15}
_CPU_CONTIGUOUS_TENSOR = 7  # record flags: a tensor, on the CPU, contiguous


def _column(samples: Sequence[Any], used_b: bytes, key: str) -> np.ndarray:
    return np.frombuffer(_lib.stage().columns(samples, used_b, key), _REC)


_GATHER_FN: int | None = None


def _gather_fn() -> int:
    """Address of the library's meshy_host_gather, for meshy_amd._stage.gather."""
    global _GATHER_FN
    if _GATHER_FN is None:
        _GATHER_FN = _lib.ctypes.cast(_lib.load().meshy_host_gather, _lib.ctypes.c_void_p).value
    return _GATHER_FN


_GATHER_I32_FN: int | None = None


# Staging int64 tokens as int32 halves their copy but narrows on the host:
# for the 23 micros of the 256 GRPO samples at once (181 k tokens) it saved
# 10 us of 225, for one micro of ~8 k tokens it cost 1.2 us of 39.
_NARROW_MIN_TOKENS = 65536


def _gather_i32_fn() -> int:
    """Address of the library's meshy_host_gather_i32, with which
    meshy_amd._stage.stage_micros stages int64 tokens as int32."""
    global _GATHER_I32_FN
    if _GATHER_I32_FN is None:
        _GATHER_I32_FN = _lib.ctypes.cast(_lib.load().meshy_host_gather_i32, _lib.ctypes.c_void_p).value
    return _GATHER_I32_FN


def _gather_column(samples: Sequence[Any], used: np.ndarray, used_b: bytes, need: np.ndarray, key: str,
                   out: torch.Tensor, row: int = 1, recs: np.ndarray | None = None) -> None:
    """The first ``need[j]`` rows (``row`` elements each) of ``samples[used[j]][key]``
    for every j, concatenated into the host tensor ``out``: columns that are CPU
    contiguous tensors of ``out``'s dtype are read in place (one native call
    when all are), any other is converted first."""
    n = len(used)
    if n == 0:
        return
    nbytes = int(need.sum()) * row * out.element_size()
    if nbytes != out.numel() * out.element_size():
        raise ValueError(f"column {key!r}: the samples hold {nbytes} bytes, the staging wants "
                         f"{out.numel() * out.element_size()}")
    if _lib.stage().gather(samples, used_b, need.tobytes(), key, out.data_ptr() if nbytes else 0,
                           _SCALAR_TYPE[out.dtype], out.element_size(), row, _gather_fn()):
        return
    if recs is None:
        recs = _column(samples, used_b, key)
    short = np.flatnonzero((recs["flags"] & 1).astype(bool) & (recs["dim0"] < need))
    if short.size:
        j = int(short[0])
        raise ValueError(f"column {key!r} of sample {int(used[j])} holds {int(recs['dim0'][j])} rows, "
                         f"{int(need[j])} are needed")
    ptrs = recs["ptr"].copy()
    odd = np.flatnonzero((recs["flags"] != _CPU_CONTIGUOUS_TENSOR) | (recs["dtype"] != _SCALAR_TYPE[out.dtype])
                         | (recs["row"] != row))
    keep = []  # converted copies stay alive until the gather is done
    for j in odd.tolist():
        L = int(need[j])
        c = torch.as_tensor(samples[int(used[j])][key])
        if c.shape[0] < L:
            raise ValueError(f"column {key!r} of sample {int(used[j])} holds {c.shape[0]} rows, {L} are needed")
        c = c[:L].to(device="cpu", dtype=out.dtype).contiguous()
        if c.numel() != L * row:
            raise ValueError(f"column {key!r} of sample {int(used[j])} has rows of {c.numel() // max(L, 1)} "
                             f"elements, {row} expected")
        keep.append(c)
        ptrs[j] = c.data_ptr() if L else 0
    sizes = need * (row * out.element_size())
    nbytes = int(sizes.sum())
    if nbytes != out.numel() * out.element_size():
        raise ValueError(f"column {key!r}: the samples hold {nbytes} bytes, the staging wants "
                         f"{out.numel() * out.element_size()}")
    if nbytes == 0:  # only empty samples (an empty view has no address)
        return
    rc = _lib.load().meshy_host_gather(ptrs.ctypes.data, sizes.ctypes.data, n, out.data_ptr(), 0)
    _lib.check(rc, "meshy_host_gather")


@dataclass
class PackJob:
    """Device-resident inputs of one pack launch (see ``stage_micro_batches``)."""

    micros: tuple
    layout: str
    device: torch.device
    dbuf: torch.Tensor
    lay: Any
    need_rollout_lp: bool
    per_token_adv: bool
    n_samples: int
    seq: np.ndarray
    rows: np.ndarray
    out_off: np.ndarray
    doc_start: np.ndarray
    max_elems: int
    max_docs: int
    #: Device per-sample advantages indexed like ``doc_sample`` (overrides the
    #: staged ``sample["advantage"]`` values): a tensor or a device address.
    adv_samples: torch.Tensor | int | None = None
    #: Also write ``Batch.advantage_tokens`` (per-document advantage per token).
    broadcast_advantages: bool = False
    #: Per-token advantages gathered on the device (indexed like the staged tokens).
    adv_tokens_dev: torch.Tensor | None = None
    #: Teacher Top-K width staged with the samples (0: no Teacher columns).
    teacher_k: int = 0
    #: The staged mask holds one byte per token (0 or 1) instead of fp32.
    mask_u8: bool = False
    #: Per micro, whether its advantages are per token (None: every micro
    #: with documents, when per_token_adv).
    per_token_micros: tuple | None = None

    @classmethod
    def fast(cls, **fields) -> "PackJob":
        """A job built without the dataclass constructor (the per-step pack
        builds one per call): the defaults, then ``fields``."""
        job = object.__new__(cls)
        d = job.__dict__
        d.update(_PACK_JOB_DEFAULTS)
        d.update(fields)
        return job
    #: The HIP stream handle to launch on (None: the device's current stream).
    stream: int | None = None
    #: Per micro (ids, logprobs) Teacher columns in the micro's layout, filled by
    #: ``launch_pack`` when ``teacher_k`` > 0.
    teacher_views: list | None = None


_PACK_JOB_DEFAULTS = {f.name: f.default for f in fields(PackJob) if f.default is not MISSING}


def stage_micro_batches(
    samples: Sequence[Any],
    micros: Sequence[MicroPlan],
    *,
    layout: Layout,
    device,
    need_rollout_lp: bool,
    teacher: bool = False,
) -> PackJob:
    """Gather what ``micros`` read from ``samples`` into one pinned buffer and copy it
    to the device in one transfer (asynchronous on the current stream).

    With ``teacher`` the samples' OPD Teacher columns (``teacher_topk_ids``,
    ``teacher_topk_logprobs``, ``[L, K]`` each) travel too and the pack lays them
    out like ``layout_teacher_topk`` (opd.py:58-89)."""
    if layout not in ("padded", "packed"):
        raise ValueError(f"unknown layout {layout!r}")
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("meshy_amd builds micro-batches on a HIP device; pass a cuda device")

    micros = tuple(micros)
    job = _stage_common(samples, micros, layout, device, need_rollout_lp, teacher)
    if job is not None:
        return job

    # Samples used by these micros, remapped to a compact list in order of
    # first use, with the longest prefix any micro reads of each, and the
    # per-document tables: one native pass over the micros.
    used_b, need_b, ds_b, dl_b, seq_b, nd_b, nt_b = _lib.stage().plan_tables(micros, len(samples))
    used = np.frombuffer(used_b, np.int64)
    need_len = np.frombuffer(need_b, np.int64)
    seq = np.frombuffer(seq_b, np.int64)
    n_docs = np.frombuffer(nd_b, np.int64)
    if layout == "packed":
        over = np.flatnonzero(np.frombuffer(nt_b, np.int64) > seq)
        if over.size:
            m = micros[int(over[0])]
            raise AssertionError(f"micro seq_len {m.seq_len} smaller than its tokens {m.n_tokens}")
    n_s = len(used)
    # Token ids travel in the samples' own int64 (the reference's dtype) or as
    # int32 (any vocabulary fits), and come out int64 either way.
    tok_recs = _column(samples, used_b, "tokens")
    tok_tensor = (tok_recs["flags"] & 1).astype(bool)
    n_tk = np.where(tok_tensor, tok_recs["dim0"], 0)
    for j in np.flatnonzero(~tok_tensor).tolist():  # lists and arrays: their length
        n_tk[j] = len(samples[int(used[j])]["tokens"])
    short = np.flatnonzero(n_tk < need_len)
    if short.size:
        j = int(short[0])
        raise ValueError(f"sample {int(used[j])} has {int(n_tk[j])} tokens, micro wants {int(need_len[j])}")
    tok64 = bool(tok_tensor.all() and (tok_recs["dtype"] == _SCALAR_TYPE[torch.int64]).all())
    # Per-token advantages are a micro's when its first sample carries them
    # (batch.py:110): a micro without documents, or whose first sample has
    # none, keeps per-document advantages.
    per_token_micros = tuple(bool(m.sample_idx) and ADVANTAGE_TOKENS in samples[m.sample_idx[0]] for m in micros)
    per_token_adv = any(per_token_micros)
    adv_cols = _advantage_tokens(samples, micros, per_token_micros, used) if per_token_adv else None
    s_off = np.zeros(n_s + 1, np.int64)
    np.cumsum(need_len, out=s_off[1:])
    total = int(s_off[-1])

    # Plan tables.
    n_micro = len(micros)
    rows = (np.ones(n_micro, np.int64) if layout == "packed"
            else np.array([m.n_rows for m in micros], np.int64))
    elems = seq * rows
    out_off = np.zeros(n_micro + 1, np.int64)
    np.cumsum(elems, out=out_off[1:])
    doc_start = np.zeros(n_micro + 1, np.int32)
    np.cumsum(n_docs, out=doc_start[1:])
    n_docs_total = int(doc_start[-1])
    doc_sample = np.frombuffer(ds_b, np.int32)
    doc_len = np.frombuffer(dl_b, np.int64)
    st = _lib.stage()
    adv_samples = np.frombuffer(st.scalars(samples, used_b, "advantage", 0.0), np.float64).astype(np.float32)
    # Positive-LM weights only for rewards above 0.5 (batch.py:225-229).
    pos_used = np.where(np.frombuffer(st.scalars(samples, used_b, "reward", 0.0), np.float64) > 0.5,
                        np.frombuffer(st.scalars(samples, used_b, "positive_lm_weight", 0.0), np.float64),
                        0.0).astype(np.float32)
    pos_w = pos_used[doc_sample] if n_docs_total else np.zeros(0, np.float32)
    tok_dtype = torch.int64 if tok64 else torch.int32

    # Per-token advantages already on the device (attach_gae_advantages leaves
    # them there) are gathered on the device; host ones travel with the rest.
    adv_dev = None
    if per_token_adv and n_s and all(c is None or c.is_cuda for c in adv_cols):
        adv_dev = torch.cat(_advantage_parts(adv_cols, need_len, device))

    lay = _Layout()
    lay.add("tokens", total, tok_dtype)
    lay.add("mask", total, torch.float32)
    if need_rollout_lp:
        lay.add("logprobs", total, torch.float32)
    if per_token_adv and adv_dev is None:
        lay.add("adv_tokens", total, torch.float32)
    lay.add("adv_samples", max(n_s, 1), torch.float32)
    lay.add("s_off", n_s + 1, torch.int64)
    lay.add("seq", n_micro, torch.int64)
    lay.add("out_off", n_micro + 1, torch.int64)
    lay.add("doc_len", max(n_docs_total, 1), torch.int64)
    lay.add("doc_start", n_micro + 1, torch.int32)
    lay.add("doc_sample", max(n_docs_total, 1), torch.int32)
    lay.add("pos_w", max(n_docs_total, 1), torch.float32)
    base_size = lay.size
    tea = _TeacherStaging(samples, used, used_b, need_len, lay) if teacher and n_s else None

    stage = _STAGING.setdefault(device.index or 0, _Staging())
    host = stage.get(tea.reserve if tea else lay.size)
    if n_s:
        # the first need_len[i] positions of each sample's columns
        _gather_column(samples, used, used_b, need_len, "tokens", lay.view(host, "tokens"), recs=tok_recs)
        _gather_column(samples, used, used_b, need_len, "mask_assistant", lay.view(host, "mask"))
        if need_rollout_lp:
            _gather_column(samples, used, used_b, need_len, "logprobs", lay.view(host, "logprobs"))
        if per_token_adv and adv_dev is None:
            parts = _advantage_parts(adv_cols, need_len, torch.device("cpu"))
            gather_into(parts, lay.view(host, "adv_tokens"))
    hnp = stage.np
    lay.np_view(hnp, "adv_samples")[:n_s] = adv_samples
    lay.np_view(hnp, "s_off")[:] = s_off
    lay.np_view(hnp, "seq")[:] = seq
    lay.np_view(hnp, "out_off")[:] = out_off
    lay.np_view(hnp, "doc_start")[:] = doc_start
    if n_docs_total:
        lay.np_view(hnp, "doc_len")[:n_docs_total] = doc_len
        lay.np_view(hnp, "doc_sample")[:n_docs_total] = doc_sample
        lay.np_view(hnp, "pos_w")[:n_docs_total] = pos_w

    handle = _lib.stream_of(device)
    dbuf = torch.empty(tea.reserve if tea else lay.size, dtype=torch.uint8, device=device)
    _copy_to_device(dbuf, host, 0, base_size, handle)
    if tea:
        tea.stage(lay, host, dbuf, handle)
    stage.mark(device, handle)
    return PackJob(
        micros=tuple(micros), layout=layout, device=device, dbuf=dbuf, lay=lay,
        need_rollout_lp=need_rollout_lp, per_token_adv=per_token_adv, per_token_micros=per_token_micros,
        n_samples=n_s, seq=seq, rows=rows,
        out_off=out_off, doc_start=doc_start, max_elems=int(elems.max()) if n_micro else 0,
        max_docs=int(n_docs.max()) if n_micro else 0, adv_tokens_dev=adv_dev, teacher_k=tea.k if tea else 0,
        stream=handle,
    )


def _advantage_tokens(samples, micros, per_token_micros, used: np.ndarray) -> list:
    """The per-token advantage column of each used sample: required of the
    samples of micros with per-token advantages (a missing one raises, as
    batch.py:110-116 does), None for other samples that have none."""
    need = {i for m, f in zip(micros, per_token_micros) if f for i in m.sample_idx}
    cols = []
    for i in used.tolist():
        s = samples[i]
        if i in need or ADVANTAGE_TOKENS in s:
            cols.append(s[ADVANTAGE_TOKENS])
        else:
            cols.append(None)
    return cols


def _advantage_parts(cols: list, need_len: np.ndarray, device: torch.device) -> list:
    """The first need_len[j] advantages of each column as fp32 on ``device``,
    zero-padded (zeros for a sample without the column)."""
    parts = []
    for c, L in zip(cols, need_len.tolist()):
        if c is None:
            parts.append(torch.zeros(L, dtype=torch.float32, device=device))
            continue
        a = c[:L].to(device=device, dtype=torch.float32)
        if a.numel() < L:
            a = torch.cat([a, a.new_zeros(L - a.numel())])
        parts.append(a)
    return parts


# Staging regions in the order stage_micro_batches lays them out without
# per-token advantages or Teacher columns (the tokens' dtype is chosen per call).
_COMMON_REGIONS = (("tokens", None), ("mask", torch.float32), ("logprobs", torch.float32),
                   ("adv_samples", torch.float32), ("s_off", torch.int64), ("seq", torch.int64),
                   ("out_off", torch.int64), ("doc_len", torch.int64), ("doc_start", torch.int32),
                   ("doc_sample", torch.int32), ("pos_w", torch.float32))


def _stage_common(samples, micros: tuple, layout: str, device: torch.device, need_rollout_lp: bool,
                  teacher: bool = False) -> PackJob | None:
    """``stage_micro_batches`` in one native pass when every used sample's
    tokens (all int64 or all int32), mask and log-probs are CPU contiguous
    tensors and none has per-token advantages; None otherwise (nothing
    staged), and the general path runs.  int64 tokens of a large staging
    are staged as int32 (each checked; one outside int32 leaves the call to
    the general path, which keeps the int64s).  Teacher columns follow
    (_TeacherStaging)."""
    stage = _STAGING.setdefault(device.index or 0, _Staging())
    host = stage.get(0)  # waits for the buffer's previous copy
    st = _lib.stage()
    packed = layout == "packed"
    res = st.stage_micros(samples, micros, packed, need_rollout_lp, host.data_ptr(), host.numel(), _gather_fn(),
                          _gather_i32_fn(), _NARROW_MIN_TOKENS)
    if isinstance(res, int):  # the buffer is too small: grow it and stage again
        host = stage.get(res)
        res = st.stage_micros(samples, micros, packed, need_rollout_lp, host.data_ptr(), host.numel(), _gather_fn(),
                              _gather_i32_fn(), _NARROW_MIN_TOKENS)
    if res is None:
        return None
    (size, bounds_b, n_s, _total, tok64, _nd, max_elems, max_docs, seq_b, rows_b, out_off_b, doc_start_b,
     used_b, need_b) = res
    bounds = np.frombuffer(bounds_b, np.int64).tolist()
    lay = _Layout()
    lay.size = size
    tok_dtype = torch.int64 if tok64 else torch.int32
    lay.regions = {name: (bounds[2 * i], bounds[2 * i + 1], dtype or tok_dtype)
                   for i, (name, dtype) in enumerate(_COMMON_REGIONS) if bounds[2 * i] >= 0}
    tea = None
    if teacher and n_s:
        tea = _TeacherStaging(samples, np.frombuffer(used_b, np.int64), used_b, np.frombuffer(need_b, np.int64), lay)
        if host.numel() < tea.reserve:  # room for the Teacher columns: grow the buffer and stage again
            host = stage.get(tea.reserve)
            res = st.stage_micros(samples, micros, packed, need_rollout_lp, host.data_ptr(), host.numel(),
                                  _gather_fn(), _gather_i32_fn(), _NARROW_MIN_TOKENS)
            if res is None or isinstance(res, int) or res[0] != size:
                raise RuntimeError("stage_micros: the staging changed between two calls on the same samples")
    handle = _lib.stream_of(device)
    dbuf = torch.empty(tea.reserve if tea else size, dtype=torch.uint8, device=device)
    # Raw asynchronous copies: the pinned buffer is reused only after the
    # event stage.mark records has passed.
    _copy_to_device(dbuf, host, 0, size, handle)
    if tea:
        tea.stage(lay, host, dbuf, handle)
    stage.mark(device, handle)
    return PackJob.fast(
        micros=micros, layout=layout, device=device, dbuf=dbuf, lay=lay, need_rollout_lp=need_rollout_lp,
        per_token_adv=False, n_samples=n_s, seq=np.frombuffer(seq_b, np.int64),
        rows=np.frombuffer(rows_b, np.int64), out_off=np.frombuffer(out_off_b, np.int64),
        doc_start=np.frombuffer(doc_start_b, np.int32), max_elems=max_elems, max_docs=max_docs,
        teacher_k=tea.k if tea else 0, stream=handle,
    )


def _copy_to_device(dbuf: torch.Tensor, host: torch.Tensor, lo: int, hi: int, handle: int) -> None:
    """Bytes [lo, hi) of the pinned buffer to the same offsets of ``dbuf``,
    asynchronously on the stream whose raw handle is ``handle``."""
    if hi > lo:
        _lib.check(_lib.load().meshy_copy_to_device(dbuf.data_ptr() + lo, host.data_ptr() + lo, hi - lo, handle),
                   "meshy_copy_to_device")


# Narrowing Teacher ids pays from about this many: at 262144 int64s it took
# as long on the host as copying them and saved a 1 MB copy to the device; at
# 65536 (one micro of ~8 k tokens, K = 8) it took 35 us against a 20 us copy.
_NARROW_MIN_TEACHER_IDS = 262144


class _TeacherStaging:
    """The OPD Teacher columns (``teacher_topk_logprobs``, then
    ``teacher_topk_ids``, ``[L, K]`` each) as the last two staging regions.

    They are most of the bytes a distillation step stages.  Each is copied as
    soon as it is gathered, so the copy of the regions before it runs while it
    is gathered (a queued host-to-device copy holds the host's next one until
    it has run, so a few large copies overlap the gathers better than many
    small ones).  int64 ids in CPU tensors (the Teacher's dtype), when there
    are enough of them, are narrowed to int32 as they are gathered, which
    checks that each fits and halves their bytes; the ids' region has room
    for int64s and holds them when one does not fit."""

    def __init__(self, samples, used: np.ndarray, used_b: bytes, need_len: np.ndarray, lay: _Layout) -> None:
        self.samples, self.used, self.used_b, self.need = samples, used, used_b, need_len
        self.k, ids64, self.recs = _teacher_width(samples, used, used_b, need_len)
        self.total = total = int(need_len.sum())
        self.narrow = bool(self.k and ids64 and total * self.k >= _NARROW_MIN_TEACHER_IDS
                           and self.recs[0] is not None and (self.recs[0]["flags"] == _CPU_CONTIGUOUS_TENSOR).all())
        self.reserve = lay.size
        if not self.k:
            return
        lay.add("teacher_lps", total * self.k, torch.float32)
        lay.add("teacher_ids", total * self.k, torch.int64 if ids64 and not self.narrow else torch.int32)
        self.reserve = lay.size + (total * self.k * 4 + 256 if self.narrow else 0)

    def stage(self, lay: _Layout, host: torch.Tensor, dbuf: torch.Tensor, handle: int) -> None:
        """Gather into ``host`` and copy to ``dbuf`` on the stream ``handle``."""
        if not self.k:
            return
        k = self.k
        _gather_column(self.samples, self.used, self.used_b, self.need, TEACHER_FIELDS[1],
                       lay.view(host, "teacher_lps"), row=k, recs=self.recs[1])
        ids_lo = lay.regions["teacher_ids"][0]
        _copy_to_device(dbuf, host, lay.regions["teacher_lps"][0], ids_lo, handle)
        if not (self.narrow and _gather_ids_i32(self.recs[0], self.need * k, lay.view(host, "teacher_ids"))):
            if self.narrow:  # an id outside int32: the region holds the int64s
                lay.size = lay.regions.pop("teacher_ids")[0]
                lay.add("teacher_ids", self.total * k, torch.int64)
            _gather_column(self.samples, self.used, self.used_b, self.need, TEACHER_FIELDS[0],
                           lay.view(host, "teacher_ids"), row=k, recs=self.recs[0])
        _copy_to_device(dbuf, host, ids_lo, lay.size, handle)


def _gather_ids_i32(recs: np.ndarray, counts: np.ndarray, out: torch.Tensor) -> bool:
    """The first ``counts[j]`` int64s of each column ``recs`` describes, as
    int32 into ``out``; False (``out`` then undefined) when a value does not
    fit."""
    fits = _lib.ctypes.c_int32(0)
    ptrs = np.ascontiguousarray(recs["ptr"])
    counts = np.ascontiguousarray(counts, np.int64)
    _lib.check(_lib.load().meshy_host_gather_i32(ptrs.ctypes.data, counts.ctypes.data, len(recs), out.data_ptr(), 0,
                                                 _lib.ctypes.byref(fits)), "meshy_host_gather_i32")
    return bool(fits.value)


def _teacher_width(samples, used, used_b, need_len) -> tuple[int, bool, tuple]:
    """Top-K width of the used samples' Teacher columns, whether all their ids
    are int64, and the columns' records; checks they cover the micros
    (opd.py:39-55)."""
    recs = (_column(samples, used_b, TEACHER_FIELDS[0]), _column(samples, used_b, TEACHER_FIELDS[1]))
    if not all((r["flags"] & 1).all() for r in recs):  # columns that are not tensors: one by one
        k, ids64 = 0, True
        for i, L in zip(used.tolist(), need_len.tolist()):
            ids, lps = samples[i][TEACHER_FIELDS[0]], samples[i][TEACHER_FIELDS[1]]
            if ids.shape[0] < L or lps.shape[0] < L:
                raise ValueError(
                    f"teacher columns cover {int(min(ids.shape[0], lps.shape[0]))} positions but the student "
                    f"micro-batch needs {L}; the Teacher seq_len must be >= the Student's"
                )
            width = int(ids.shape[-1])
            if k and width != k:
                raise ValueError(f"Teacher Top-K widths differ across samples ({k} vs {width})")
            k = width
            ids64 = ids64 and isinstance(ids, torch.Tensor) and ids.dtype == torch.int64
        return k, ids64, (None, None)
    ids, lps = recs
    cover = np.minimum(ids["dim0"], lps["dim0"])
    short = np.flatnonzero(cover < need_len)
    if short.size:
        j = int(short[0])
        raise ValueError(f"teacher columns cover {int(cover[j])} positions but the student micro-batch needs "
                         f"{int(need_len[j])}; the Teacher seq_len must be >= the Student's")
    widths = ids["row"]
    if widths.size and (widths != widths[0]).any():
        j = int(np.flatnonzero(widths != widths[0])[0])
        raise ValueError(f"Teacher Top-K widths differ across samples ({int(widths[0])} vs {int(widths[j])})")
    k = int(widths[0]) if widths.size else 0
    return k, bool((ids["dtype"] == _SCALAR_TYPE[torch.int64]).all()), recs


_OUT_LAYOUTS: dict[tuple, _Layout] = {}


def _out_layout(n_out: int, n_docs_total: int, n_micro: int, rollout_lp: bool, adv_tok: bool,
                teacher_k: int) -> _Layout:
    """The pack's output regions for these sizes (read-only, cached: the same
    sizes recur from step to step)."""
    key = (n_out, n_docs_total, n_micro, rollout_lp, adv_tok, teacher_k)
    out_lay = _OUT_LAYOUTS.get(key)
    if out_lay is not None:
        return out_lay
    out_lay = _Layout()
    for name, dtype in (("input_ids", torch.int64), ("labels", torch.int64), ("positions", torch.int32),
                        ("mask", torch.float32), ("doc_ids", torch.int64)):
        out_lay.add(name, n_out, dtype)
    if rollout_lp:
        out_lay.add("rollout_lp", n_out, torch.float32)
    if adv_tok:
        out_lay.add("adv_tok", n_out, torch.float32)
    out_lay.add("adv_doc", max(n_docs_total, 1), torch.float32)
    out_lay.add("lengths", max(n_docs_total, 1), torch.int32)
    out_lay.add("cu", n_docs_total + 2 * n_micro, torch.int32)
    out_lay.add("seg", n_docs_total + 2 * n_micro, torch.int64)
    if teacher_k:
        out_lay.add("teacher_ids", n_out * teacher_k, torch.int64)
        out_lay.add("teacher_lps", n_out * teacher_k, torch.float32)
    if len(_OUT_LAYOUTS) >= 4096:
        _OUT_LAYOUTS.clear()
    _OUT_LAYOUTS[key] = out_lay
    return out_lay


def launch_pack(job: PackJob, sharder=None) -> list[Batch]:
    """Run the pack kernels over a staged job and return one ``Batch`` per micro."""
    lib = _lib.load()
    device, lay, dbuf, layout = job.device, job.lay, job.dbuf, job.layout
    n_micro = len(job.micros)
    n_docs_total = int(job.doc_start[-1])
    n_out = int(job.out_off[-1])
    # Every output lives in one device allocation; the kernel gets addresses
    # inside it, and the typed tensors are views made when a micro first needs
    # them (_PackViews).
    adv_tok = bool(job.per_token_adv or job.broadcast_advantages)
    out_lay = _out_layout(n_out, n_docs_total, n_micro, bool(job.need_rollout_lp), adv_tok, job.teacher_k)
    obuf = torch.empty(max(out_lay.size, 1), dtype=torch.uint8, device=device)
    obase = obuf.data_ptr()
    o = out_lay.regions

    a = _lib.PackArgs()
    base = dbuf.data_ptr()
    r = lay.regions
    tok = r["tokens"]
    a.tokens = base + tok[0]
    a.tokens_elem_bytes = _ITEMSIZE[tok[2]]
    a.layout = _lib.MESHY_LAYOUT_PACKED if layout == "packed" else _lib.MESHY_LAYOUT_PADDED
    a.mask = base + r["mask"][0]
    a.mask_u8 = int(job.mask_u8)
    if job.need_rollout_lp:
        a.logprobs = base + r["logprobs"][0]
    if job.adv_tokens_dev is not None:
        a.adv_tokens = job.adv_tokens_dev.data_ptr()
    elif job.per_token_adv:
        a.adv_tokens = base + r["adv_tokens"][0]
    src = job.adv_samples
    a.adv_samples = (base + r["adv_samples"][0] if src is None
                     else src if isinstance(src, int) else src.data_ptr())
    a.sample_offsets = base + r["s_off"][0]
    a.n_samples = job.n_samples
    a.n_micro = n_micro
    a.micro_seq_len = base + r["seq"][0]
    a.micro_out_off = base + r["out_off"][0]
    a.micro_doc_start = base + r["doc_start"][0]
    a.doc_sample = base + r["doc_sample"][0]
    a.doc_len = base + r["doc_len"][0]
    a.max_micro_elems = job.max_elems
    a.max_docs_per_micro = job.max_docs
    a.input_ids = obase + o["input_ids"][0]
    a.labels = obase + o["labels"][0]
    a.positions = obase + o["positions"][0]
    a.mask_out = obase + o["mask"][0]
    a.doc_ids = obase + o["doc_ids"][0]
    if job.need_rollout_lp:
        a.rollout_lp = obase + o["rollout_lp"][0]
    if adv_tok:
        a.adv_tok = obase + o["adv_tok"][0]
    a.adv_doc = obase + o["adv_doc"][0]
    a.doc_len_out = obase + o["lengths"][0]
    a.cu_seqlens = obase + o["cu"][0]
    a.seg_offsets = obase + o["seg"][0]
    if job.teacher_k:
        a.teacher_k = job.teacher_k
        a.teacher_ids = base + r["teacher_ids"][0]
        a.teacher_ids_elem_bytes = _ITEMSIZE[r["teacher_ids"][2]]
        a.teacher_lps = base + r["teacher_lps"][0]
        a.teacher_ids_out = obase + o["teacher_ids"][0]
        a.teacher_lps_out = obase + o["teacher_lps"][0]
    rc = lib.meshy_pack_micro_batches(_lib.ctypes.byref(a),
                                      job.stream if job.stream is not None else _lib.stream_of(device))
    _lib.check(rc, "meshy_pack_micro_batches")
    views = _PackViews(job, sharder, obuf, out_lay, lay, dbuf)

    if job.teacher_k:
        K = job.teacher_k
        t_ids, t_lps = out_lay.view(obuf, "teacher_ids"), out_lay.view(obuf, "teacher_lps")
        sizes_k = [n * K for n in views.sizes]
        tv = []
        for part_i, part_l, R, S, m in zip(torch.split(t_ids, sizes_k), torch.split(t_lps, sizes_k), views.rows,
                                           views.seq, job.micros):
            if m.is_filler:
                # infer_top_k of no samples is 1 (opd.py:39-44)
                tv.append((torch.zeros(R, S, 1, dtype=torch.int64, device=device),
                           torch.zeros(R, S, 1, dtype=torch.float32, device=device)))
            else:
                tv.append((part_i.view(R, S, K), part_l.view(R, S, K)))
        if layout == "padded" and sharder is not None:
            tv = [tuple(sharder.shard_seq(i, l)) for i, l in tv]
        job.teacher_views = tv

    out: list[Batch] = []
    new = object.__new__
    nd = views.nd
    for k in range(n_micro):
        mb = new(PackedBatch)
        mb.__dict__ = {"n_docs": nd[k], "_src": views, "_k": k}
        out.append(mb)
    return out


class _PackViews:
    """The flat outputs of one pack launch and where each micro lies in them.
    A micro's tensors are views of these, made when its batch first needs them."""

    _TOK = ("input_ids", "labels", "positions", "mask", "doc_ids", "rollout_lp", "adv_tok")

    def __init__(self, job: PackJob, sharder, obuf: torch.Tensor, out_lay: _Layout, lay: _Layout,
                 dbuf: torch.Tensor) -> None:
        self.packed = job.layout == "packed"
        self.sharder = sharder
        self.per_token_adv = job.per_token_adv
        # Which micros take per-token advantages (batch.py:110): those with
        # documents whose first sample carries them.
        self.tok_adv = None
        if job.per_token_adv:
            self.tok_adv = (job.per_token_micros if job.per_token_micros is not None
                            else tuple(bool(m.sample_idx) for m in job.micros))
        self.broadcast_only = job.broadcast_advantages and not job.per_token_adv
        # The launch's one output buffer and its layout; the positive-LM
        # weights stay in the staging buffer, where the host wrote them.
        self.obuf, self.out_lay = obuf, out_lay
        # Every view shares obuf's version counter: its value now, against
        # which a later in-place change of any output is seen.
        self.version0 = obuf._version
        self.pos_w_src = (lay, dbuf)
        self._job = job
        self.doc_start = job.doc_start.tolist()
        self.nd = [b - a for a, b in zip(self.doc_start, self.doc_start[1:])]
        self.micros = job.micros
        self._tok = self._doc = self._cu = self._seg = None

    # The per-micro sizes the views read, as lists, made when a view first needs them.
    @property
    def out_off(self) -> list:
        v = self.__dict__.get("_out_off")
        if v is None:
            v = self._out_off = self._job.out_off.tolist()
        return v

    @property
    def sizes(self) -> list:
        v = self.__dict__.get("_sizes")
        if v is None:
            o = self.out_off
            v = self._sizes = [b - a for a, b in zip(o, o[1:])]
        return v

    @property
    def rows(self) -> list:
        v = self.__dict__.get("_rows")
        if v is None:
            v = self._rows = self._job.rows.tolist()
        return v

    @property
    def seq(self) -> list:
        v = self.__dict__.get("_seq")
        if v is None:
            v = self._seq = self._job.seq.tolist()
        return v

    def _flat(self, name: str) -> torch.Tensor | None:
        """The whole-launch tensor of one output (None when not produced)."""
        if name not in self.out_lay.regions:
            return None
        return self.out_lay.view(self.obuf, name)

    @property
    def seg(self) -> torch.Tensor:
        if self._seg is None:
            self._seg = self._flat("seg")
        return self._seg

    def seg_offsets(self, k: int, ids: torch.Tensor, n_docs: int) -> torch.Tensor | None:
        """The segment offsets the pack wrote for micro k (n_docs + 2 of
        them) when ``ids`` is still that micro's unchanged doc_ids view."""
        nd = self.nd[k]
        if n_docs != nd or ids._version != self.version0:
            return None
        d0 = self.doc_start[k] + 2 * k
        return self.seg[d0:d0 + nd + 2]

    # Each group's views are made for every micro at once, the first time any
    # micro needs them: one torch.split per tensor (a third of a microsecond
    # per view) instead of a slice and a view per micro and field.

    def _token_views(self) -> list:
        if self._tok is None:
            sizes = self.sizes
            tok = [self._flat(name) for name in self._TOK]
            if self.packed:
                cols = [None if t is None else torch.split(t.view(1, -1), sizes, dim=1) for t in tok]
            else:
                cols = [None if t is None else [p.view(R, S) for p, R, S in zip(torch.split(t, sizes), self.rows,
                                                                                 self.seq)]
                        for t in tok]
            self._tok = [tuple(None if c is None else c[k] for c in cols) for k in range(len(sizes))]
        return self._tok

    def tokens(self, mb: "PackedBatch", f: dict) -> None:
        """input_ids, labels, positions, mask, doc_ids, rollout_logprobs and the
        advantage tokens of micro mb._k (one CP shard call in the padded layout,
        batch.py:195-207; the identity on one GPU)."""
        k = mb._k
        ii, lb, ps, mk, di, rl, at = self._token_views()[k]
        if not self.packed and self.sharder is not None:
            optional = [t for t in (rl, at) if t is not None]
            sharded = self.sharder.shard_seq(ii, lb, ps, mk, di, *optional)
            ii, lb, ps, mk, sdi = sharded[:5]
            rest = list(sharded[5:])
            rl = rest.pop(0) if rl is not None else None
            at = rest.pop(0) if at is not None else None
        else:
            sdi = di
        setd = f.setdefault  # a field the caller set before its first read stays
        setd("input_ids", ii)
        setd("labels", lb)
        setd("positions", ps)
        setd("mask", mk)
        setd("doc_ids", sdi)
        setd("rollout_logprobs", rl)
        setd("advantage_tokens", at if self.broadcast_only else None)
        if self.tok_adv is not None and self.tok_adv[k]:
            setd("advantages", at)
        if sdi is di:  # not replaced by a context-parallel shard
            # The offsets the pack wrote for this micro (seg_offsets below),
            # valid while this doc_ids tensor is the batch's and unchanged.
            f["_meshy_seg_src"] = (self, k, di)

    def doc_fields(self, mb: "PackedBatch", f: dict) -> None:
        """Per-document advantages, lengths and positive-LM weights of micro mb._k."""
        if self._doc is None:
            n = self.doc_start[-1]
            lay, dbuf = self.pos_w_src
            docs = (self._flat("adv_doc"), self._flat("lengths"), lay.view(dbuf, "pos_w"))
            self._doc = [torch.split(t[:n], self.nd) for t in docs]
        k = mb._k
        adv, lengths, pos_w = self._doc
        setd = f.setdefault  # a field the caller set before its first read stays
        setd("lengths", lengths[k])
        setd("positive_lm_weights", pos_w[k])
        if self.tok_adv is None or not self.tok_adv[k]:
            setd("advantages", adv[k])

    def attention(self, mb: "PackedBatch", f: dict) -> None:
        """cu_seqlens (n_docs + 1 slots, + 1 with a padding document) and the
        longest document of micro mb._k, as make_varlen_metadata builds them."""
        if not self.packed:
            f.setdefault("attention_masks", None)
            return
        if self._cu is None:
            sizes, pads = [], []
            for k, m in enumerate(self.micros):
                pad = self.seq[k] - m.n_tokens
                pads.append(pad)
                n_cu = self.nd[k] + 1 + (1 if pad > 0 else 0)
                sizes += [n_cu, self.nd[k] + 2 - n_cu]
            self._cu = (torch.split(self._flat("cu"), sizes)[0::2], pads)
        cus, pads = self._cu
        k = mb._k
        m, pad, cu = self.micros[k], pads[k], cus[k]
        max_len = max(max(m.doc_lens, default=0), pad if pad > 0 else 0)
        f.setdefault("attention_masks",
                     VarlenMetadata(cu_seq_q=cu, cu_seq_k=cu, max_q=int(max_len), max_k=int(max_len)))


class _Lazy:
    """A field of PackedBatch that is not yet in the instance: made (with its
    whole group) on first read.  A non-data descriptor, so once the instance
    holds the value, reads and writes are plain attribute accesses."""

    __slots__ = ("name", "group")

    def __init__(self, name: str, group: str) -> None:
        self.name, self.group = name, group

    def __get__(self, obj, cls=None):
        if obj is None:
            return self
        d = obj.__dict__
        src = d.get("_src")
        if src is not None:
            getattr(src, self.group)(obj, d)
            if self.name not in d:  # `advantages` is per token: the other group has it
                getattr(src, "doc_fields" if self.group == "tokens" else "tokens")(obj, d)
        try:
            return d[self.name]
        except KeyError:
            raise AttributeError(self.name) from None


class PackedBatch(Batch):
    """A ``Batch`` over one micro of a pack launch.  All micros of the launch
    live in flat device buffers; a micro's tensors are views of them, made on
    first access (per group, for every micro of the launch at once: the
    per-token tensors, the per-document tensors, the attention metadata), as
    the reference's trainer builds each micro when it reaches it
    (trainer.py:557-571).  Once made, fields are plain attributes."""


# Each lazy field and the view group that makes it.
_LAZY_FIELDS = (("input_ids", "tokens"), ("labels", "tokens"), ("positions", "tokens"), ("mask", "tokens"),
                ("doc_ids", "tokens"), ("rollout_logprobs", "tokens"), ("advantage_tokens", "tokens"),
                ("advantages", "doc_fields"), ("lengths", "doc_fields"),
                ("positive_lm_weights", "doc_fields"), ("attention_masks", "attention"))


def make_lazy(cls: type) -> type:
    """Gives ``cls`` (a Batch subclass) the lazy pack-view fields of PackedBatch."""
    for name, group in _LAZY_FIELDS:
        setattr(cls, name, _Lazy(name, group))
    return cls


make_lazy(PackedBatch)


def build_micro_batches(
    samples: Sequence[Any],
    micros: Sequence[MicroPlan],
    *,
    layout: Layout,
    device,
    sharder=None,
    need_rollout_lp: bool,
) -> list[Batch]:
    """Materialise ``micros`` from the rank-local ``samples`` in one transfer and one launch."""
    job = stage_micro_batches(samples, micros, layout=layout, device=device, need_rollout_lp=need_rollout_lp)
    return launch_pack(job, sharder)


def build_micro_batch(
    samples: Sequence[Any],
    micro: MicroPlan,
    *,
    layout: Layout,
    device,
    sharder=None,
    need_rollout_lp: bool,
) -> Batch:
    """Materialise one ``micro`` from the rank-local ``samples`` (batch.py:96-230)."""
    return build_micro_batches(samples, [micro], layout=layout, device=device, sharder=sharder,
                               need_rollout_lp=need_rollout_lp)[0]


__all__ = ["ADVANTAGE_TOKENS", "TEACHER_FIELDS", "Batch", "PackJob", "PackedBatch", "VarlenMetadata", "build_micro_batch",
           "build_micro_batches", "launch_pack", "make_varlen_metadata", "stage_micro_batches"]

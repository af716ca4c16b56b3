"""Token-budget planner with the call surface of meshy/backend/titan/plan.py.

``build_plan`` runs the C++ planner of libmeshy_amd (``meshy_plan_build``)
and returns the same frozen dataclasses as the reference (plan.py:51-138), so
plans compare with ``==`` and every consumer keeps working.  The dataclasses
and the small helpers keep the reference's field names and semantics because
they are the interface the trainer, the critic and the tests read.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal, Sequence

import numpy as np

from . import _lib

Layout = Literal["padded", "packed"]


@dataclass(frozen=True)
class PlannerConfig:
    """Planner knobs (plan.py:51-81), validated on construction."""

    layout: Layout
    mini_batch_size: int
    seq_len: int
    align: int
    max_tokens_per_micro: int | None = None
    micro_batch_size: int | None = None

    def __post_init__(self) -> None:
        if self.layout not in ("padded", "packed"):
            raise ValueError(f"unknown layout {self.layout!r}")
        if self.mini_batch_size <= 0:
            raise ValueError("mini_batch_size must be positive")
        if self.align <= 0 or self.seq_len <= 0:
            raise ValueError("align and seq_len must be positive")
        if self.seq_len % self.align != 0:
            raise ValueError(
                f"seq_len ({self.seq_len}) must be a multiple of align ({self.align})"
            )
        if self.max_tokens_per_micro is not None and self.max_tokens_per_micro <= 0:
            raise ValueError("max_tokens_per_micro must be positive")
        if self.micro_batch_size is not None and self.micro_batch_size <= 0:
            raise ValueError("micro_batch_size must be positive")
        if self.max_tokens_per_micro is None and self.micro_batch_size is None:
            raise ValueError("either max_tokens_per_micro or micro_batch_size must be set")
        if self.layout == "packed" and self.max_tokens_per_micro is None:
            raise ValueError("packed layout requires max_tokens_per_micro")


@dataclass(frozen=True)
class MicroPlan:
    """One forward/backward pass (plan.py:83-109).

    ``sample_idx`` indexes the rank-local sample list, ``doc_lens`` are the
    truncated lengths, ``seq_len`` the padded row length (``padded``) or the
    packed total with tail rounding (``packed``).  Empty ``sample_idx`` marks
    a filler.
    """

    sample_idx: tuple[int, ...]
    seq_len: int
    doc_lens: tuple[int, ...]

    @property
    def is_filler(self) -> bool:
        return not self.sample_idx

    @property
    def n_tokens(self) -> int:
        return sum(self.doc_lens)

    @property
    def n_rows(self) -> int:
        return max(1, len(self.sample_idx))


@dataclass(frozen=True)
class MiniPlan:
    """One optimizer step and its global loss denominators (plan.py:111-123)."""

    micros: tuple[MicroPlan, ...]
    n_docs_global: int
    n_tokens_global: int
    tokens_per_rank: tuple[int, ...]

    @property
    def n_docs_local(self) -> int:
        return sum(len(m.sample_idx) for m in self.micros)


@dataclass(frozen=True)
class Plan:
    """Per-rank mini-batch plans and the global indices each rank owns (plan.py:125-138)."""

    per_rank: tuple[tuple[MiniPlan, ...], ...]
    local_indices: tuple[tuple[int, ...], ...]

    @property
    def dp_size(self) -> int:
        return len(self.per_rank)

    def local_samples(self, batch: Sequence, rank: int) -> list:
        """The rank-local sample list that ``MicroPlan.sample_idx`` indexes."""
        return [batch[i] for i in self.local_indices[rank]]


def round_up(x: int, align: int) -> int:
    """Smallest multiple of ``align`` that is >= ``x`` (plan.py:141-142)."""
    return -(-x // align) * align


def filler_micro(cfg: PlannerConfig) -> MicroPlan:
    """A zero-weight micro used to equalise micro counts (plan.py:206-208)."""
    return MicroPlan((), cfg.align, ())


def _np_ptr(a: np.ndarray) -> int:
    return a.__array_interface__["data"][0]


def _frozen(cls, **fields):
    """An instance of the frozen dataclass ``cls`` with ``fields`` set directly:
    the values come from the native planner, which already enforces what
    ``__init__`` would (there is no validation hook on these types)."""
    obj = object.__new__(cls)
    obj.__dict__.update(fields)
    return obj


class PlanTables:
    """The flat CSR tables ``meshy_plan_build`` fills (see include/meshy_amd.h),
    as numpy views of one zeroed host buffer."""

    def __init__(self, n: int, dp: int, mini_batch_size: int) -> None:
        n_local = n // dp
        n_mini = -(-n_local // mini_batch_size)
        self.n, self.dp, self.n_local, self.n_mini = n, dp, n_local, n_mini
        shape = (n, dp, mini_batch_size)
        layout = self._LAYOUTS.get(shape)
        if layout is None:
            counts = (dp * n_local, n_mini, n_mini, n_mini, n_mini * dp, dp * n_local, dp * (n_local + 1),
                      dp * n_local, dp * n_local)
            offs, total = [], 0
            for (_, _, size), c in zip(self._FIELDS, counts):
                offs.append(total)
                total += -(-c * size // 8) * 8
            layout = self._LAYOUTS[shape] = (offs, counts, max(total, 8))
            if len(self._LAYOUTS) > 64:
                self._LAYOUTS.pop(next(iter(self._LAYOUTS)))
        self._offs, self._counts, total = layout
        self._buf = np.zeros(total, np.uint8)
        self._base = self._buf.__array_interface__["data"][0]
        self.n_micro_total = 0

    _FIELDS = (("local_indices", np.int32, 4), ("mini_n_micro", np.int32, 4), ("mini_n_docs_global", np.int64, 8),
               ("mini_n_tokens_global", np.int64, 8), ("mini_tokens_per_rank", np.int64, 8),
               ("micro_seq_len", np.int64, 8), ("micro_doc_start", np.int32, 4), ("doc_sample", np.int32, 4),
               ("doc_len", np.int64, 8))
    _INDEX = {f[0]: i for i, f in enumerate(_FIELDS)}
    # Field offsets per (n, dp, mini_batch_size): one step's shape repeats.
    _LAYOUTS: dict = {}

    def __getattr__(self, name: str):
        # Each table is a numpy view of the buffer, made when first read.
        i = PlanTables._INDEX.get(name)
        if i is None:
            raise AttributeError(name)
        _, dtype, size = self._FIELDS[i]
        o, c = self._offs[i], self._counts[i]
        v = self.__dict__[name] = self._buf[o:o + c * size].view(dtype)
        return v

    def c_struct(self) -> _lib.PlanOut:
        b = self._base
        return _lib.PlanOut(*[b + o for o in self._offs], 0, 0)


def _as_int64(x: Sequence[int]) -> np.ndarray:
    """A contiguous int64 copy of ``x`` (no Python loop when it is already an array)."""
    if isinstance(x, np.ndarray) and x.dtype.kind in "iu":
        return np.ascontiguousarray(x, dtype=np.int64)
    return np.ascontiguousarray(np.asarray([int(v) for v in x], dtype=np.int64))


def plan_tables(
    lengths: Sequence[int], loss_tokens: Sequence[int], dp_size: int, cfg: PlannerConfig
) -> PlanTables:
    """Run the native planner and return its flat tables (no dataclasses)."""
    n = len(lengths)
    if n == 0:
        raise ValueError("cannot plan an empty batch")
    if len(loss_tokens) != n:
        raise ValueError("lengths and loss_tokens must have the same size")
    if dp_size <= 0 or n % dp_size != 0:
        raise ValueError(
            f"batch size {n} is not divisible by DP size {dp_size}; adjust "
            "rollout.batch_size * group_size to a multiple of dp_replicate * dp_shard"
        )
    lib = _lib.load()
    lens = _as_int64(lengths)
    loss = _as_int64(loss_tokens)
    c = _lib.PlannerCfg()
    c.layout = _lib.MESHY_LAYOUT_PACKED if cfg.layout == "packed" else _lib.MESHY_LAYOUT_PADDED
    c.mini_batch_size = cfg.mini_batch_size
    c.seq_len = cfg.seq_len
    c.align = cfg.align
    c.max_tokens_per_micro = cfg.max_tokens_per_micro or 0
    c.micro_batch_size = cfg.micro_batch_size or 0
    t = PlanTables(n, dp_size, cfg.mini_batch_size)
    out = t.c_struct()
    rc = lib.meshy_plan_build(_np_ptr(lens), _np_ptr(loss), n, dp_size, _lib.ctypes.byref(c),
                              _lib.ctypes.byref(out))
    _lib.check(rc, "meshy_plan_build")
    t.n_micro_total = int(out.n_micro_total)
    return t


def tables_to_plan(t: PlanTables) -> Plan:
    """Materialise the reference's dataclasses from the flat tables."""
    dp, n_local = t.dp, t.n_local
    local = t.local_indices.reshape(dp, n_local).tolist()
    n_micro = t.mini_n_micro.tolist()
    docs_g = t.mini_n_docs_global.tolist()
    toks_g = t.mini_n_tokens_global.tolist()
    tpr = t.mini_tokens_per_rank.reshape(t.n_mini, dp).tolist()
    per_rank = []
    for r in range(dp):
        seq = t.micro_seq_len[r * n_local:(r + 1) * n_local].tolist()
        start = t.micro_doc_start[r * (n_local + 1):(r + 1) * (n_local + 1)].tolist()
        dsample = t.doc_sample[r * n_local:(r + 1) * n_local].tolist()
        dlen = t.doc_len[r * n_local:(r + 1) * n_local].tolist()
        minis = []
        k = 0
        for i in range(t.n_mini):
            micros = []
            for _ in range(n_micro[i]):
                a, b = start[k], start[k + 1]
                micros.append(_frozen(MicroPlan, sample_idx=tuple(dsample[a:b]), seq_len=seq[k],
                                      doc_lens=tuple(dlen[a:b])))
                k += 1
            minis.append(_frozen(MiniPlan, micros=tuple(micros), n_docs_global=docs_g[i],
                                 n_tokens_global=toks_g[i], tokens_per_rank=tuple(tpr[i])))
        per_rank.append(tuple(minis))
    return _frozen(Plan, per_rank=tuple(per_rank), local_indices=tuple(tuple(x) for x in local))


def build_plan(
    lengths: Sequence[int],
    loss_tokens: Sequence[int],
    dp_size: int,
    cfg: PlannerConfig,
) -> Plan:
    """Plan one ``train_step`` over the global batch (plan.py:211-288).

    Args:
        lengths: per-sample token count before truncation to ``seq_len``.
        loss_tokens: per-sample loss-token count after shift and truncation.
        dp_size: number of data-parallel ranks.
        cfg: planner configuration.
    """
    return tables_to_plan(plan_tables(lengths, loss_tokens, dp_size, cfg))


def plan_stats(minis: Sequence[MiniPlan], layout: Layout) -> dict[str, float]:
    """Padding ratio, micro count and DP imbalance of one rank's plan (plan.py:291-310)."""
    n_micro = 0
    real_tokens = 0
    forward_tokens = 0
    for mini in minis:
        for m in mini.micros:
            n_micro += 1
            real_tokens += m.n_tokens
            forward_tokens += (m.n_rows if layout == "padded" else 1) * m.seq_len
    tokens_per_rank = [t for mini in minis for t in mini.tokens_per_rank]
    mean_tpr = sum(tokens_per_rank) / max(1, len(tokens_per_rank))
    imbalance = (max(tokens_per_rank) / mean_tpr) if mean_tpr > 0 else 1.0
    return {
        "n_micro": float(n_micro),
        "tokens_per_micro": real_tokens / max(1, n_micro),
        "padding_ratio": 1.0 - real_tokens / max(1, forward_tokens),
        "dp_token_imbalance": float(imbalance),
    }


def resolve_align(seq_bucket: int, divisor: int, seq_len: int) -> int:
    """Rounding granularity lcm(seq_bucket, divisor), capped at seq_len (plan.py:313-324)."""
    align = math.lcm(max(1, seq_bucket), max(1, divisor))
    if align >= seq_len:
        align = seq_len
    if seq_len % align != 0:
        raise ValueError(
            f"seq_len ({seq_len}) must be a multiple of the sequence alignment "
            f"({align} = lcm(seq_bucket={seq_bucket}, divisor={divisor}))"
        )
    return align


__all__ = [
    "Layout",
    "MicroPlan",
    "MiniPlan",
    "Plan",
    "PlannerConfig",
    "build_plan",
    "filler_micro",
    "plan_stats",
    "plan_tables",
    "resolve_align",
    "round_up",
    "tables_to_plan",
]

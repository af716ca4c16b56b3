"""The rollout -> trainer wire format with the semantics of
meshy/transferqueue/adapter.py: per-sample columns batched as jagged nested
tensors (variable-length ``[L]`` / ``[L, K]`` columns), dense ``[B, 1]`` scalars
and object lists.

``tensordict`` is not a dependency here, so a batch is a plain ``dict`` of
columns rather than a ``TensorDict``; the column forms are the ones
``samples_to_td`` puts and ``td_to_samples`` accepts (adapter.py:96-182).

``RaggedSamples.from_columns`` (pipeline.py) ingests such a batch straight from
the jagged columns' ``values()`` and ``offsets()``: no per-sample tensor is
touched on the way into the pack.
"""

from __future__ import annotations

import itertools
from typing import Any, Iterable

import numpy as np
import torch

from . import _lib

# How each known column is materialised in a batch (adapter.py:39-71).
FIELD_KINDS: dict[str, str] = {
    "tokens": "nested",
    "logprobs": "nested",
    "mask_assistant": "nested",
    "advantage": "scalar",
    "reward": "scalar",
    "raw_reward": "scalar",
    "positive_lm_weight": "scalar",
    "values": "nested",
    "truncated": "scalar",
    "repetition": "scalar",
    "mixed_version": "scalar",
    "weight_version": "scalar",
    "teacher_topk_ids": "nested",
    "teacher_topk_logprobs": "nested",
}

_SCALAR_DTYPE: dict[str, torch.dtype] = {
    "reward": torch.float32,
    "raw_reward": torch.float32,
    "positive_lm_weight": torch.float32,
    "advantage": torch.float32,
    "weight_version": torch.int64,
    "truncated": torch.int64,
    "repetition": torch.int64,
    "mixed_version": torch.int64,
}


# The columns a GRPO rollout writes (meshy/config.py:248-261) and the shaped
# reward's companion column (rollout.py:35).
GRPO_TRAINER_FIELDS: tuple[str, ...] = ("tokens", "logprobs", "mask_assistant", "advantage", "weight_version",
                                        "reward", "truncated", "repetition", "mixed_version")
RAW_REWARD_FIELD = "raw_reward"

# Per-token columns of a rollout sample: the sample attribute and dtype they
# come from (rollout.py:124-126).
_SEQ_SOURCE: dict[str, tuple[str, torch.dtype]] = {
    "tokens": ("tokens", torch.int64),
    "logprobs": ("logprobs", torch.float32),
    "mask_assistant": ("masks", torch.float32),
}


def field_kind(field: str) -> str:
    """The storage kind of ``field``; unknown columns are ``"object"`` (adapter.py:86-88)."""
    return FIELD_KINDS.get(field, "object")


def _as_tensor(value: Any) -> torch.Tensor:
    return value if isinstance(value, torch.Tensor) else torch.as_tensor(value)


def samples_to_columns(samples: list[Any], fields: Iterable[str]) -> dict[str, Any]:
    """Batch per-sample mappings into columns (adapter.py:96-132): ``nested`` ->
    jagged nested tensor, ``scalar`` -> ``[B, 1]`` tensor, ``object`` -> list."""
    fields = list(fields)
    batch = len(samples)
    if batch == 0:
        raise ValueError("samples_to_td received an empty sample list")
    out: dict[str, Any] = {}
    for f in fields:
        kind = field_kind(f)
        values = [s[f] for s in samples]
        if kind == "nested":
            tensors = [_as_tensor(v) for v in values]
            ndims = {t.dim() for t in tensors}
            if len(ndims) != 1:
                raise ValueError(f"column {f!r}: all samples must have the same rank, got {sorted(ndims)}")
            if tensors[0].dim() >= 2:
                trailing = {tuple(t.shape[1:]) for t in tensors}
                if len(trailing) != 1:
                    raise ValueError(
                        f"column {f!r}: trailing dims must match across samples, got {sorted(trailing)}")
            out[f] = torch.nested.nested_tensor(tensors, layout=torch.jagged)
        elif kind == "scalar":
            dtype = _SCALAR_DTYPE.get(f, torch.float32)
            out[f] = torch.stack([_as_tensor(v).reshape(-1)[0].to(dtype) for v in values]).reshape(batch, 1)
        else:
            out[f] = list(values)
    return out


def _stamp_raw_reward(sample: Any, weight_version: int) -> float:
    raw = getattr(sample, "raw_reward", None)
    return float(sample.reward if raw is None else raw)


# A rollout sample's scalar columns (rollout.py:127-152): a missing advantage is
# 0, a missing raw reward is the reward, the quality stamps are 0/1.
_STAMPS: dict[str, Any] = {
    "advantage": lambda s, v: 0.0 if s.advantage is None else float(s.advantage),
    "weight_version": lambda s, v: int(v),
    "reward": lambda s, v: float(s.reward),
    "positive_lm_weight": lambda s, v: float(getattr(s, "positive_lm_weight", 0.0)),
    RAW_REWARD_FIELD: _stamp_raw_reward,
    "truncated": lambda s, v: int(bool(getattr(s, "truncated", False))),
    "repetition": lambda s, v: int(bool(getattr(s, "repetition", False))),
    "mixed_version": lambda s, v: int(bool(getattr(s, "mixed_version", False))),
}


def _stamp(sample: Any, f: str, weight_version: int) -> float | int:
    """One scalar column's value for one rollout sample."""
    return _STAMPS[f](sample, weight_version)


_ROLLOUT_SCALARS = ("advantage", "weight_version", "reward", "positive_lm_weight", RAW_REWARD_FIELD, "truncated",
                    "repetition", "mixed_version")


def sample_to_tensordict(sample: Any, weight_version: int) -> dict[str, torch.Tensor]:
    """One rollout sample as its columns (rollout.py:118-153), a ``dict`` in place
    of the ``TensorDict``: the token, log-prob and mask sequences as ``[L]``
    tensors (int64, fp32, fp32) and every scalar stamp as a 0-dim tensor."""
    out: dict[str, torch.Tensor] = {}
    for f, (attr, dt) in _SEQ_SOURCE.items():
        out[f] = torch.tensor(list(getattr(sample, attr)), dtype=dt)
    for f in _ROLLOUT_SCALARS:
        out[f] = torch.tensor(_stamp(sample, f, weight_version), dtype=_SCALAR_DTYPE[f])
    return out


def rollout_group_to_columns(group: list[Any], weight_version: int,
                             fields: Iterable[str] = GRPO_TRAINER_FIELDS) -> dict[str, Any]:
    """``samples_to_columns([sample_to_tensordict(s, v) for s in group], fields)``
    (the write of rollout.py:611-615) without a tensor per sample: each
    per-token column is converted from the samples' sequences in one pass into
    flat values plus offsets and wrapped as a jagged nested tensor over them;
    each scalar column is one ``[B, 1]`` tensor."""
    fields = list(fields)
    batch = len(group)
    if batch == 0:
        raise ValueError("samples_to_td received an empty sample list")
    out: dict[str, Any] = {}
    for f in fields:
        if f in _SEQ_SOURCE:
            attr, dt = _SEQ_SOURCE[f]
            flat, off = flatten_sequences([getattr(s, attr) for s in group], dt)
            out[f] = torch.nested.nested_tensor_from_jagged(torch.from_numpy(flat), torch.from_numpy(off))
        elif f in _ROLLOUT_SCALARS:
            stamp = _STAMPS[f]
            out[f] = torch.tensor([stamp(s, weight_version) for s in group],
                                  dtype=_SCALAR_DTYPE[f]).reshape(batch, 1)
        else:
            raise KeyError(f"a rollout sample has no column {f!r}")
    return out


def flatten_sequences(seqs: list[Any], dtype: torch.dtype) -> tuple[np.ndarray, np.ndarray]:
    """(flat values, int64 offsets [len(seqs) + 1]) of a list of number
    sequences, as int64 (``torch.int64``) or float32 (any other dtype).

    Lists and tuples of Python ints, floats and bools go through
    ``meshy_amd._pyio`` in one native pass; anything else (numpy arrays,
    tensors, numpy scalars, ints beyond int64) through ``np.fromiter``, whose
    conversions the native pass reproduces bit for bit."""
    npdt = np.int64 if dtype == torch.int64 else np.float32
    pyio = _lib.pyio()
    off = np.empty(len(seqs) + 1, np.int64)
    total = pyio.seq_offsets(seqs, off)
    if total is not None:
        flat = np.empty(total, npdt)
        if pyio.flatten_into(seqs, flat, "q" if npdt is np.int64 else "f"):
            return flat, off
    else:
        off[0] = 0
        np.cumsum(np.fromiter((len(x) for x in seqs), np.int64, len(seqs)), out=off[1:])
    return np.fromiter(itertools.chain.from_iterable(seqs), npdt, int(off[-1])), off


def _explode(value: Any, f: str, batch: int) -> list[Any]:
    """One batched column -> ``batch`` independent values (adapter.py:135-159)."""
    if isinstance(value, list):
        return list(value)
    if isinstance(value, torch.Tensor):
        parts = value.unbind() if value.is_nested else [value[i] for i in range(batch)]
        if field_kind(f) == "scalar":
            return [p.reshape(-1)[0].clone() for p in parts]
        return [p.clone() for p in parts]
    return [value[i] for i in range(batch)]


def columns_to_samples(columns: dict[str, Any], fields: Iterable[str] | None = None) -> list[dict]:
    """Inverse of :func:`samples_to_columns` (adapter.py:162-182): scalars come back
    0-dim, nested columns in their ``[L]`` / ``[L, K]`` shape, each value on its own
    storage."""
    fields = list(columns) if fields is None else list(fields)
    if not fields:
        return []
    first = columns[fields[0]]
    batch = first.size(0) if isinstance(first, torch.Tensor) else len(first)
    cols = {f: _explode(columns[f], f, batch) for f in fields}
    return [{f: cols[f][i] for f in fields} for i in range(batch)]


def jagged_parts(column: Any) -> tuple[torch.Tensor, torch.Tensor]:
    """(flat values, int64 offsets [B + 1]) of a nested column: a jagged nested
    tensor, or a list of per-sample tensors (concatenated once)."""
    if isinstance(column, torch.Tensor) and column.is_nested:
        return column.values(), column.offsets().to(torch.int64)
    tensors = [_as_tensor(v) for v in column]
    lengths = torch.tensor([t.shape[0] for t in tensors], dtype=torch.int64)
    off = torch.zeros(len(tensors) + 1, dtype=torch.int64)
    torch.cumsum(lengths, 0, out=off[1:])
    flat = torch.cat([t.reshape(t.shape[0], *t.shape[1:]) for t in tensors]) if tensors else torch.empty(0)
    return flat, off


__all__ = ["FIELD_KINDS", "GRPO_TRAINER_FIELDS", "RAW_REWARD_FIELD", "columns_to_samples", "field_kind",
           "flatten_sequences", "jagged_parts", "rollout_group_to_columns", "sample_to_tensordict", "samples_to_columns"]

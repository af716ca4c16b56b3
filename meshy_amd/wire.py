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

from typing import Any, Iterable

import torch

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


__all__ = ["FIELD_KINDS", "columns_to_samples", "field_kind", "jagged_parts", "samples_to_columns"]

"""Host staging of jagged per-sample columns.

``gather_into(parts, out)`` is ``torch.cat(parts, out=out)`` for host tensors:
the pieces are copied into ``out`` (usually a view of a pinned staging buffer
that then goes to the device in one copy) by ``meshy_host_gather`` on a pool of
host threads, instead of torch.cat's single thread.  It stands in for the
per-sample concatenations of the critic path (trainer.py:644-667) and of
``build_micro_batch`` (batch.py:126-178).
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib


def gather_into(parts: Sequence, out: torch.Tensor) -> torch.Tensor:
    """Concatenate ``parts`` (flattened, converted to ``out``'s dtype where they
    differ) into the contiguous host tensor ``out``; returns ``out``."""
    if out.is_cuda or not out.is_contiguous():
        raise ValueError("gather_into writes a contiguous host tensor")
    dt = out.dtype
    n = len(parts)
    keep = []  # converted copies stay alive until the copy is done
    ptrs = [0] * n
    sizes = [0] * n
    total = 0
    for i, p in enumerate(parts):
        if not isinstance(p, torch.Tensor):
            p = torch.as_tensor(p)
        if p.dtype is not dt or p.is_cuda or not p.is_contiguous():
            p = p.to(device="cpu", dtype=dt).contiguous()
            keep.append(p)
        k = p.numel()
        ptrs[i] = p.data_ptr() if k else 0
        sizes[i] = k
        total += k
    if total != out.numel():
        raise ValueError(f"the parts hold {total} elements but out has {out.numel()}")
    if n == 0 or total == 0:
        return out
    es = out.element_size()
    c_ptrs = (ctypes.c_void_p * n)(*ptrs)
    c_sizes = (ctypes.c_int64 * n)(*[s * es for s in sizes])
    rc = _lib.load().meshy_host_gather(c_ptrs, c_sizes, n, out.data_ptr(), 0)
    _lib.check(rc, "meshy_host_gather")
    return out


__all__ = ["gather_into"]

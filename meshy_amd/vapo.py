"""Masked global whitening of per-token advantages (meshy/backend/titan/vapo.py:6-32).

``whiten_advantages(samples, seq_len, device, mesh=None, replication=1)`` keeps
the reference's in-place contract on ``sample[ADVANTAGE_TOKENS]``.  The samples'
advantages and loss masks are gathered into one flat device buffer; the fp64
statistics (sum, sum of squares, count) come from ``meshy_whiten_stats``, are
all-reduced over ``mesh`` when one is given, and ``meshy_whiten_apply`` writes
``(x - mean) * rsqrt(var + 1e-8)`` on the mask and 0 elsewhere.
"""

from __future__ import annotations

import torch
import torch.distributed as dist

from . import _lib
from .batch import ADVANTAGE_TOKENS


def whiten_flat(adv: torch.Tensor, mask: torch.Tensor, mesh=None, replication: int = 1) -> torch.Tensor:
    """Whiten a flat device buffer in place over ``mask != 0``; returns ``adv``."""
    _lib.require_gpu(adv, mask)
    if adv.dtype != torch.float32 or not adv.is_contiguous():
        raise ValueError("adv must be a contiguous float32 tensor")
    m = mask.to(torch.float32).contiguous()
    n = adv.numel()
    if m.numel() != n:
        raise ValueError(f"adv has {n} elements but mask has {m.numel()}")
    dev = adv.device
    lib = _lib.load()
    stats = torch.empty(3, dtype=torch.float64, device=dev)
    ws = torch.empty(int(lib.meshy_whiten_workspace_size(n)), dtype=torch.uint8, device=dev)
    rep = float(replication) if mesh is not None else 1.0
    stream = _lib.stream_of(dev)
    rc = lib.meshy_whiten_stats(adv.data_ptr(), m.data_ptr(), n, rep, stats.data_ptr(), ws.data_ptr(),
                                ws.numel(), stream)
    _lib.check(rc, "meshy_whiten_stats")
    if mesh is not None:
        dist.all_reduce(stats, group=mesh.get_group())
    rc = lib.meshy_whiten_apply(adv.data_ptr(), m.data_ptr(), n, stats.data_ptr(), stream)
    _lib.check(rc, "meshy_whiten_apply")
    return adv


def whiten_advantages(samples, seq_len, device, mesh=None, replication=1) -> None:
    """In-place whitening of every sample's per-token advantages (vapo.py:6-32)."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("meshy_amd whitens on a HIP device; pass a cuda device")
    advs, masks = [], []
    for sample in samples:
        a = sample[ADVANTAGE_TOKENS]
        length = min(len(a), seq_len)
        m = torch.zeros(len(a), dtype=torch.float32)
        if length > 1:
            m[:length - 1] = (sample["mask_assistant"][1:length] != 0).to(torch.float32)
        advs.append(a)
        masks.append(m)
    if not advs:
        stats_only = torch.zeros(0, dtype=torch.float32, device=device)
        whiten_flat(stats_only, stats_only, mesh, replication)
        return
    flat_mask = torch.cat(masks).to(device, non_blocking=True)
    base = _tiled_view(advs)
    if base is not None:
        whiten_flat(base, flat_mask, mesh, replication)
        return
    flat = torch.cat([a.to(device=device, dtype=torch.float32) for a in advs])
    whiten_flat(flat, flat_mask, mesh, replication)
    o = 0
    for a in advs:
        n = len(a)
        a.copy_(flat[o:o + n])
        o += n


def _tiled_view(tensors) -> torch.Tensor | None:
    """The flat device view the tensors tile, in order, if they do (else None)."""
    t0 = tensors[0]
    if not all(t.is_cuda and t.dtype == torch.float32 and t.dim() == 1 and t.is_contiguous() for t in tensors):
        return None
    ptr = t0.untyped_storage().data_ptr()
    off = t0.storage_offset()
    for t in tensors:
        if t.untyped_storage().data_ptr() != ptr or t.storage_offset() != off:
            return None
        off += t.numel()
    return t0.as_strided((off - t0.storage_offset(),), (1,), t0.storage_offset())


__all__ = ["whiten_advantages", "whiten_flat"]

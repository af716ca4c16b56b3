"""Segment-aware GAE and returns with the call surface of
meshy/backend/titan/critic/gae.py.

``compute_vapo_gae`` (gae.py:208-293) and ``compute_returns`` (gae.py:183-205)
run the ``meshy_gae`` kernels: the recursion ``A_t = x_t + decay_t * cont_t *
A_{t+1}`` as a reverse scan of affine maps over the flattened ``[rows, S]``
grid, in fp32, with no closed form and therefore no underflow fallback
(gae.py:149-150).  ``gae_and_returns`` produces both in one pass.  When the
flattened doc_ids are non-decreasing (both batch layouts) and no lengths are
given, the kernels take their segment offsets: the masked document lengths
are then fixed-order sums, bitwise reproducible for fractional masks too.
"""

from __future__ import annotations

import math
from typing import Any, Sequence

import numpy as np
import torch

from . import _lib
from .loss import DocIdRangeError, checked_segment_offsets


def _doc_offsets(doc_ids: torch.Tensor, n_docs: int) -> torch.Tensor | None:
    """The segment offsets of ``doc_ids`` over its ``n_docs + 1`` slots when its
    flattened values are non-decreasing (checked once per tensor version, one
    device sync), else None: the kernels then count lengths with atomics.  An
    id outside [0, n_docs] raises, as the reference's indexing does
    (gae.py:266-276)."""
    try:
        return checked_segment_offsets(doc_ids, n_docs + 1)
    except DocIdRangeError:
        raise
    except ValueError:
        return None


def _run(rewards, values, mask, doc_ids, n_docs, *, lengths, gamma, alpha, epsilon, want_adv,
         want_returns, want_lam, offsets=True):
    if rewards.dim() != 2:
        raise ValueError(f"expected [rows, S] tensors, got {tuple(rewards.shape)}")
    rows, S = rewards.shape
    for name, t in (("values", values), ("mask", mask), ("doc_ids", doc_ids)):
        if t is not None and tuple(t.shape) != (rows, S):
            raise ValueError(f"{name} {tuple(t.shape)} does not match rewards {(rows, S)}")
    _lib.require_gpu(rewards, values, mask, doc_ids, lengths)
    dev = rewards.device
    r = rewards.to(torch.float32).contiguous()
    m = mask.to(torch.float32).contiguous()
    ids = doc_ids.to(torch.int64).contiguous()
    v = None
    bf16 = 0
    if values is not None:
        if values.dtype == torch.bfloat16:
            v, bf16 = values.contiguous(), 1
        else:
            v = values.to(torch.float32).contiguous()
    lens = None if lengths is None else lengths.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    if lens is not None and lens.numel() < n_docs:
        raise ValueError(f"lengths has {lens.numel()} entries for {n_docs} documents")
    adv = torch.empty(rows, S, dtype=torch.float32, device=dev) if want_adv else None
    ret = torch.empty(rows, S, dtype=torch.float32, device=dev) if want_returns else None
    lam = torch.empty(max(n_docs, 1), dtype=torch.float32, device=dev) if want_lam else None
    lib = _lib.load()
    ws = torch.empty(max(int(lib.meshy_gae_workspace_size(rows, S, n_docs)), 1), dtype=torch.uint8,
                     device=dev)
    g = _lib.GaeArgs()
    g.rewards = r.data_ptr()
    g.values = _lib.ptr(v)
    g.mask = m.data_ptr()
    g.doc_ids = ids.data_ptr()
    g.lengths = _lib.ptr(lens)
    g.rows, g.S, g.n_docs = rows, S, int(n_docs)
    g.gamma, g.alpha, g.epsilon = float(gamma), float(alpha), float(epsilon)
    g.values_bf16 = bf16
    g.adv = _lib.ptr(adv)
    g.returns = _lib.ptr(ret)
    g.lam_doc = _lib.ptr(lam)
    g.workspace = ws.data_ptr()
    g.workspace_bytes = ws.numel()
    # The offsets give the scan its document starts (the ids are then read at
    # chunk ends only) and, without `lengths`, fixed-order masked lengths.
    need = n_docs > 0 and rows * S > 0 and (want_adv or want_returns or want_lam)
    off = _doc_offsets(doc_ids, n_docs) if offsets and need else None
    g.seg_offsets = _lib.ptr(off)
    rc = lib.meshy_gae(_lib.ctypes.byref(g), _lib.stream_of(dev))
    _lib.check(rc, "meshy_gae")
    return adv, ret, (lam[:n_docs] if lam is not None else None)


def compute_vapo_gae(
    rewards: torch.Tensor,
    values: torch.Tensor,
    mask: torch.Tensor,
    doc_ids: torch.Tensor,
    n_docs: int,
    *,
    lengths: torch.Tensor | None = None,
    gamma: float = 1.0,
    alpha: float = 1.5,
    epsilon: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """VAPO GAE with per-document lambda = 1 - 1/(alpha * L) (gae.py:208-293)."""
    adv, _, lam = _run(rewards, values, mask, doc_ids, n_docs, lengths=lengths, gamma=gamma,
                       alpha=alpha, epsilon=epsilon, want_adv=True, want_returns=False, want_lam=True)
    return adv, lam


def compute_returns(
    rewards: torch.Tensor,
    mask: torch.Tensor,
    doc_ids: torch.Tensor,
    *,
    gamma: float = 1.0,
) -> torch.Tensor:
    """Discounted return-to-go G_t = r_t + gamma * cont_t * G_{t+1} (gae.py:183-205)."""
    _, ret, _ = _run(rewards, None, mask, doc_ids, 0, lengths=None, gamma=gamma, alpha=1.0,
                     epsilon=1e-6, want_adv=False, want_returns=True, want_lam=False, offsets=False)
    return ret


def gae_and_returns(
    rewards: torch.Tensor,
    values: torch.Tensor,
    mask: torch.Tensor,
    doc_ids: torch.Tensor,
    n_docs: int,
    *,
    lengths: torch.Tensor | None = None,
    gamma: float = 1.0,
    alpha: float = 1.5,
    epsilon: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Advantages, returns and lambda per document from one pass over the inputs."""
    return _run(rewards, values, mask, doc_ids, n_docs, lengths=lengths, gamma=gamma, alpha=alpha,
                epsilon=epsilon, want_adv=True, want_returns=True, want_lam=True)


CRITIC_METRICS = (
    "critic/value_mean",
    "critic/advantage_mean",
    "critic/advantage_abs_mean",
    "critic/advantage_seq_mean",
    "critic/lambda_mean",
)


def _attach_layout(total: int, n: int, vdt: torch.dtype, mask_u8: bool, dev: torch.device):
    """The attach's staging layout (masks as bytes or fp32, values, rewards,
    offsets), a pinned host buffer and a device buffer of its size."""
    from .batch import _Layout

    lay = _Layout()
    lay.add("mask", total, torch.uint8 if mask_u8 else torch.float32)
    lay.add("values", total, vdt)
    lay.add("reward", n, torch.float32)
    lay.add("offsets", n + 1, torch.int64)
    host = torch.empty(lay.size, dtype=torch.uint8, pin_memory=True)
    dbuf = torch.empty(lay.size, dtype=torch.uint8, device=dev)
    return lay, host, dbuf


def attach_gae_advantages(self: Any, samples: Sequence[Any]) -> dict[str, float]:
    """Drop-in for ``TitanTrainer._attach_gae_advantages`` (trainer.py:603-699).

    Reads ``self.seq_len``, ``self.gae_gamma``, ``self.gae_alpha``,
    ``self.gae_lambda`` and ``self.device``.  The samples' masks, values and
    rewards travel to the device in two copies (the masks' while the values
    are gathered on the host; masks of only 0 and 1 as one byte per token);
    ``meshy_gae_attach`` shifts them
    onto the next-token grid, places each reward, runs the reverse scan over the
    samples laid end to end (one document per sample, so no padding rows) and
    reduces the critic metrics.  Each sample gets ``ADVANTAGE_TOKENS``, a device
    view of its advantages, of length ``min(len(tokens), seq_len)``.
    """
    from .batch import _CPU_CONTIGUOUS_TENSOR, _SCALAR_TYPE, ADVANTAGE_TOKENS, _column, _gather_column

    if not samples:
        return {}
    seq_len = int(self.seq_len)
    dev = torch.device(getattr(self, "device", None) or "cuda")
    if dev.type != "cuda":
        raise ValueError("meshy_amd runs GAE on a HIP device; self.device must be a cuda device")
    n = len(samples)
    # The samples' columns are read by the native staging module: pointer,
    # length and dtype records of every sample's tokens and values, then one
    # threaded gather per column into the pinned staging buffer.
    used = np.arange(n, dtype=np.int64)
    used_b = used.tobytes()
    trec = _column(samples, used_b, "tokens")
    lens = trec["dim0"].copy()
    for j in np.flatnonzero((trec["flags"] & 1) == 0).tolist():  # token lists
        lens[j] = len(samples[j]["tokens"])
    widths = np.minimum(lens, seq_len)
    vrec = _column(samples, used_b, "values")
    short = np.flatnonzero(((vrec["flags"] & 1) == 0) | (vrec["dim0"] < widths))
    if short.size:
        j = int(short[0])
        raise ValueError(
            f"row {j}: critic published {tuple(samples[j]['values'].shape)} values "
            f"for {int(widths[j])} tokens; the critic and the trainer disagree about "
            f"the sequence"
        )
    offsets = np.zeros(n + 1, np.int64)
    np.cumsum(widths, out=offsets[1:])
    total = int(offsets[-1])
    bf16 = bool((vrec["dtype"] == _SCALAR_TYPE[torch.bfloat16]).all())
    vdt = torch.bfloat16 if bf16 else torch.float32
    # Masks that hold only 0 and 1 travel as bytes (a quarter of the copy, the
    # same values); fractional ones, and columns that are not CPU fp32
    # tensors, as fp32.
    mrec = _column(samples, used_b, "mask_assistant")
    lay, host, dbuf = _attach_layout(total, n, vdt, True, dev)
    mask_u8 = bool(((mrec["flags"] == _CPU_CONTIGUOUS_TENSOR) & (mrec["dtype"] == _SCALAR_TYPE[torch.float32])
                    & (mrec["row"] == 1) & (mrec["dim0"] >= widths)).all())
    if mask_u8:
        ptrs = np.ascontiguousarray(mrec["ptr"])
        counts = np.ascontiguousarray(widths, dtype=np.int64)
        binary = _lib.ctypes.c_int32(0)
        _lib.check(_lib.load().meshy_host_gather_mask_u8(ptrs.ctypes.data, counts.ctypes.data, n,
                                                         lay.addr(host.data_ptr(), "mask"), 0,
                                                         _lib.ctypes.byref(binary)), "meshy_host_gather_mask_u8")
        mask_u8 = bool(binary.value)
    if not mask_u8:
        lay, host, dbuf = _attach_layout(total, n, vdt, False, dev)
        _gather_column(samples, used, used_b, widths, "mask_assistant", lay.view(host, "mask"), recs=mrec)
    # The masks travel to the device while the values are gathered (finer runs
    # of samples, each copied once staged, measured no faster).
    cut = lay.regions["values"][0]
    dbuf[:cut].copy_(host[:cut], non_blocking=True)
    _gather_column(samples, used, used_b, widths, "values", lay.view(host, "values"), recs=vrec)
    r64 = np.frombuffer(_lib.stage().scalars(samples, used_b, "reward", math.nan), np.float64)
    if np.isnan(r64).any():
        # absent, None, empty or NaN somewhere: each sample's reward read as it is
        rewards = [td["reward"] for td in samples]
        reward = torch.tensor([float(r.reshape(-1)[0]) if isinstance(r, torch.Tensor) else float(r)
                               for r in rewards], dtype=torch.float32)
    else:
        reward = torch.from_numpy(r64.astype(np.float32))
    lay.view(host, "reward").copy_(reward)
    lay.view(host, "offsets").copy_(torch.from_numpy(offsets))
    dbuf[cut:].copy_(host[cut:], non_blocking=True)
    widths = widths.tolist()

    lib = _lib.load()
    adv = torch.empty(max(total, 1), dtype=torch.float32, device=dev)
    lam = torch.empty(n, dtype=torch.float32, device=dev)
    metrics = torch.empty(len(CRITIC_METRICS), dtype=torch.float32, device=dev)
    ws = torch.empty(int(lib.meshy_gae_attach_workspace_size(n, total)), dtype=torch.uint8, device=dev)
    g = _lib.GaeAttachArgs()
    g.mask_assistant = lay.view(dbuf, "mask").data_ptr()
    g.values = lay.view(dbuf, "values").data_ptr()
    g.reward = lay.view(dbuf, "reward").data_ptr()
    g.offsets = lay.view(dbuf, "offsets").data_ptr()
    g.n, g.total = n, total
    g.gamma = float(self.gae_gamma)
    g.alpha = float(self.gae_alpha)
    lam_const = getattr(self, "gae_lambda", None)
    g.lambda_ = -1.0 if lam_const is None else float(lam_const)
    g.epsilon = 1e-6
    g.values_bf16 = int(bf16)
    g.mask_u8 = int(mask_u8)
    g.adv = adv.data_ptr()
    g.grid_mask = None
    g.lam_doc = lam.data_ptr()
    g.metrics = metrics.data_ptr()
    g.workspace = ws.data_ptr()
    g.workspace_bytes = ws.numel()
    rc = lib.meshy_gae_attach(_lib.ctypes.byref(g), _lib.stream_of(dev))
    _lib.check(rc, "meshy_gae_attach")
    for td, view in zip(samples, torch.split(adv[:total], widths)):
        td[ADVANTAGE_TOKENS] = view
    return dict(zip(CRITIC_METRICS, metrics.tolist()))


__all__ = ["CRITIC_METRICS", "attach_gae_advantages", "compute_returns", "compute_vapo_gae", "gae_and_returns"]

"""Student Top-K on-policy distillation with the call surface of
meshy/backend/titan/opd.py: the Teacher columns in the micro-batch layout and
the distillation loss with its metrics.

* ``layout_teacher_topk`` / ``build_topk_micro_batches``  the Teacher's
  ``[L, K]`` columns laid out like the micro (opd.py:58-89), written by the
  pack kernel in the same launch as the rest of the micro-batch;
* ``split_teacher_topk``, ``infer_top_k``, ``TopKBatch``  as in opd.py;
* ``distill_loss``  drop-in for ``StudentTopKTrainer._distill_loss``
  (opd.py:153-197): the model forward, one fused gather of the K Teacher ids
  plus the sampled label (``meshy_gather_logprobs_fwd``), then
  ``meshy_distill_loss_fwd`` for the loss and every sum; ``loss.backward()``
  runs ``meshy_distill_loss_bwd`` and ``meshy_gather_logprobs_bwd``;
* ``reduce_distill_metrics``  ``StudentTopKTrainer._reduce_mini_metrics``
  (opd.py:234-251).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Sequence

import torch
import torch.distributed as dist

from . import _lib
from .batch import TEACHER_FIELDS, Batch, launch_pack, make_lazy, stage_micro_batches
from .loss import UnsortedDocIdsError, batch_cached, batch_segment_offsets, doc_ordered, tensor_key
from .plan import Layout, MicroPlan
from .topk import gather_logprobs


OPD_TEACHER_FIELDS = list(TEACHER_FIELDS)


def infer_top_k(samples: Sequence[Any], default: int = 1) -> int:
    """Top-K width of the first sample carrying Teacher columns (opd.py:39-44)."""
    for td in samples:
        value = td.get(OPD_TEACHER_FIELDS[0], None)
        if value is not None:
            return int(value.shape[-1])
    return default


@dataclass
class TopKBatch(Batch):
    """A :class:`Batch` plus the Teacher's Top-K columns in the same layout (opd.py:115-120)."""

    teacher_topk_ids: torch.Tensor | None = None       # [rows, S_local, K] long
    teacher_topk_logprobs: torch.Tensor | None = None  # [rows, S_local, K] float


class PackedTopKBatch(TopKBatch):
    """A :class:`TopKBatch` over one micro of a pack launch: the Teacher
    columns are set, and the :class:`Batch` fields are views of the launch's
    outputs made on first read, as :class:`~meshy_amd.batch.PackedBatch`'s."""


make_lazy(PackedTopKBatch)


def build_topk_micro_batches(
    samples: Sequence[Any],
    micros: Sequence[MicroPlan],
    *,
    layout: Layout,
    device,
    sharder=None,
    need_rollout_lp: bool,
) -> list[TopKBatch]:
    """``build_micro_batch`` plus ``layout_teacher_topk`` for every micro, in one
    transfer and one pack launch (what ``StudentTopKTrainer._build_micro`` does per
    micro, opd.py:141-148)."""
    job = stage_micro_batches(samples, micros, layout=layout, device=device, need_rollout_lp=need_rollout_lp,
                              teacher=any(m.sample_idx for m in micros))
    batches = launch_pack(job, sharder)
    out = []
    new = object.__new__
    for k, mb in enumerate(batches):
        if job.teacher_views is not None:
            ids, lps = job.teacher_views[k]
        else:  # only fillers: infer_top_k of no samples is 1
            m = job.micros[k]
            shape = (m.n_rows, m.seq_len, 1) if layout == "padded" else (1, m.seq_len, 1)
            ids = torch.zeros(shape, dtype=torch.int64, device=job.device)
            lps = torch.zeros(shape, dtype=torch.float32, device=job.device)
        # The same lazy views as the pack's batch (its micro of the launch's
        # outputs), plus the Teacher columns.
        tb = new(PackedTopKBatch)
        tb.__dict__ = {**mb.__dict__, "teacher_topk_ids": ids, "teacher_topk_logprobs": lps}
        out.append(tb)
    return out


def layout_teacher_topk(
    samples: Sequence[Any],
    micro: MicroPlan,
    *,
    layout: Layout,
    device,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``[rows, S, K]`` Teacher ids / log-probs in the micro-batch's layout (opd.py:58-89)."""
    if layout not in ("padded", "packed"):
        raise ValueError(f"unknown layout {layout!r}")
    mb = build_topk_micro_batches(samples, [micro], layout=layout, device=device, need_rollout_lp=False)[0]
    return mb.teacher_topk_ids, mb.teacher_topk_logprobs


def split_teacher_topk(values: torch.Tensor, micro: MicroPlan, *, layout: Layout) -> list[torch.Tensor]:
    """Inverse of :func:`layout_teacher_topk` for one ``[rows, S, K]`` tensor
    (opd.py:92-110): one ``[L_j, K]`` view per ``micro.sample_idx[j]``."""
    out: list[torch.Tensor] = []
    if layout == "padded":
        for j, L in enumerate(micro.doc_lens):
            out.append(values[j, :L])
    elif layout == "packed":
        off = 0
        for L in micro.doc_lens:
            out.append(values[0, off:off + L])
            off += L
    else:
        raise ValueError(f"unknown layout {layout!r}")
    return out


class _Inputs:
    """Everything the distillation kernels read besides the student log-probs,
    read once per micro-batch (``native``: the argument struct over the
    batch's tensors, which each call's backward holds)."""

    def __init__(self, stub, mb, mini, k: int, n_tokens: int, device) -> None:
        self.k = k
        self.n_tokens = n_tokens
        self.has_rollout = mb.rollout_logprobs is not None
        _lib.require_gpu(mb.doc_ids)
        self.seg_off = batch_segment_offsets(mb)
        # The native reader checks that every tensor is on the GPU and has the
        # student's tokens, and flattens them.
        lp_min = getattr(stub, "log_prob_min_clamp", None)
        loss_max = getattr(stub, "loss_max_clamp", None)
        self.native = _lib.autograd().distill_inputs(
            mb.teacher_topk_logprobs, mb.mask, mb.rollout_logprobs, mb.doc_ids, self.seg_off, k, n_tokens,
            int(mb.n_docs), int(mini.n_docs_global), int(mini.n_tokens_global),
            None if lp_min is None else float(lp_min), None if loss_max is None else float(loss_max),
            bool(stub.calculate_per_token_loss))

    def args(self, student: torch.Tensor | None) -> _lib.DistillArgs:
        """The argument struct with the student set, for callers that drive the
        C ABI themselves."""
        a = _lib.DistillArgs.from_buffer_copy(_lib.autograd().args_bytes(self.native))
        a.student = _lib.ptr(student)
        return a


def _cached_inputs(stub, mb, mini, k: int, student: torch.Tensor, n_tokens: int) -> _Inputs:
    """The _Inputs of this call, reused from the micro-batch's previous call
    while nothing it was built from has changed."""
    key = (k, n_tokens, student.device, tensor_key(mb.teacher_topk_logprobs), tensor_key(mb.mask),
           tensor_key(mb.rollout_logprobs), tensor_key(mb.doc_ids), int(mb.n_docs),
           getattr(stub, "log_prob_min_clamp", None), getattr(stub, "loss_max_clamp", None),
           bool(stub.calculate_per_token_loss), int(mini.n_docs_global), int(mini.n_tokens_global))
    return batch_cached(mb, "_meshy_distill_inputs", key,
                        (mb.teacher_topk_logprobs, mb.mask, mb.rollout_logprobs, mb.doc_ids),
                        lambda: _Inputs(stub, mb, mini, k, n_tokens, student.device))


def distill_from_gathered(self: Any, gathered: torch.Tensor, mb: Any, mini: Any):
    """The loss and sums of ``_distill_loss`` from the ``[rows, S, K + 1]`` gather
    (K Teacher ids then the sampled label), opd.py:161-197."""
    sharder = getattr(self, "sharder", None)
    if sharder is not None and getattr(sharder, "enabled", False):
        raise NotImplementedError(
            "context-parallel distillation needs the per-document count all-reduce between the two "
            "kernel phases; this library drives one GPU")
    k = gathered.shape[-1] - 1
    # The kernels read the gather as one [tokens, K + 1] fp32 array; a
    # contiguous fp32 gather is passed as it is, so that no view node sits
    # between the loss's node and the gather's.
    student = gathered
    if student.dtype != torch.float32:
        student = student.float()
    if not student.is_contiguous():
        student = student.contiguous()
    try:
        inputs = _cached_inputs(self, mb, mini, k, student, student.numel() // (k + 1))
    except UnsortedDocIdsError:
        # Ids that decrease: the same loss over the tokens in document order
        # (the gather's copy carries the gradient back to its positions).
        od = doc_ordered(mb, ("mask", "rollout_logprobs", "teacher_topk_logprobs"))
        return distill_from_gathered(self, od.gather(gathered), od, mini)
    # One native call: the forward kernels, the loss (carrying a C++ backward
    # node when the student requires grad) and every sum as a 0-dim view.
    loss, parts = _lib.autograd().distill_loss(student, inputs.native)
    names = _lib.DISTILL_OUT_NAMES
    sums = dict(zip(names[:4], parts[:4]))
    if inputs.has_rollout:
        sums["train_rollout_kl_sum"] = parts[4]
        sums["train_rollout_logdiff_abs_sum"] = parts[5]
    return loss, sums


def distill_loss(self: Any, mb: TopKBatch, mini: Any) -> tuple[torch.Tensor, dict[str, torch.Tensor]]:
    """Drop-in for ``StudentTopKTrainer._distill_loss`` (opd.py:153-197).

    Reads what the reference reads: ``model_parts``, ``_LOGPROB_CHUNK``,
    ``log_prob_min_clamp``, ``loss_max_clamp``, ``calculate_per_token_loss`` and
    ``sharder``."""
    logits = self.model_parts[0](mb.input_ids, positions=mb.positions, attention_masks=mb.attention_masks)
    # One gather for the Teacher's K candidates plus the sampled token (opd.py:156-159).
    ids = torch.cat([mb.teacher_topk_ids, mb.labels.unsqueeze(-1)], dim=-1)
    gathered = gather_logprobs(logits, ids, chunk=getattr(self, "_LOGPROB_CHUNK", 1024))
    del logits
    return distill_from_gathered(self, gathered, mb, mini)


def reduce_distill_metrics(self: Any, sums: dict[str, torch.Tensor]) -> dict[str, float]:
    """Per-rank sums -> distillation metrics (opd.py:234-251)."""
    keys = list(sums)
    stacked = torch.stack([sums[k].float().reshape(()) for k in keys])
    pd = getattr(self, "parallel_dims", None)
    loss_mesh = pd.get_optional_mesh("loss") if pd is not None and hasattr(pd, "get_optional_mesh") else None
    if loss_mesh is not None:
        dist.all_reduce(stacked, op=dist.ReduceOp.SUM, group=loss_mesh.get_group())
    values = dict(zip(keys, stacked.tolist()))
    tokens = max(values["token_count"], 1.0)
    out = {
        "train/distill_loss": values["loss"],
        "train/student_topk_mass": values["student_mass_sum"] / tokens,
        "train/teacher_topk_mass": values["teacher_mass_sum"] / tokens,
    }
    if "train_rollout_kl_sum" in values:
        out["train_rollout_kl"] = values["train_rollout_kl_sum"] / tokens
        out["train_rollout_logdiff_abs"] = values["train_rollout_logdiff_abs_sum"] / tokens
    return out


__all__ = [
    "OPD_TEACHER_FIELDS",
    "PackedTopKBatch",
    "TopKBatch",
    "build_topk_micro_batches",
    "distill_from_gathered",
    "distill_loss",
    "infer_top_k",
    "layout_teacher_topk",
    "reduce_distill_metrics",
    "split_teacher_topk",
]

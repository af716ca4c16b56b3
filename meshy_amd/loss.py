"""Clipped PPO loss with the call surface of TitanTrainer._ppo_clip_loss.

``ppo_clip_loss(self, new_lp, old_lp, mb, mini, entropy=None)`` reads only the
attributes the reference reads (trainer.py:705-848): ``ppo_clip_eps_low/high``,
``use_tis``, ``use_icepop``, ``tis_ratio_min/max``, ``calculate_per_token_loss``,
``positive_lm_loss_coef``, ``old_logprobs_source``, ``sharder`` and
``parallel_dims.cp``; it can be called unbound on a ``SimpleNamespace`` like the
reference's tests do.  The forward is ``meshy_ppo_loss_fwd`` (one tiled pass over
the tokens plus one combine; with the token-mean reduction the pass also
writes each token's unit gradient), the gradient with respect to
``new_lp`` is ``meshy_ppo_loss_bwd``, run by a C++ autograd node that the one
native forward call hangs on the loss, so ``loss.backward()`` works as before.  ``reduce_mini_metrics`` is
_reduce_mini_metrics (trainer.py:1020-1047).
"""

from __future__ import annotations

import weakref
from typing import Any

import torch
import torch.distributed as dist

from . import _lib


def batch_segment_offsets(mb: Any) -> torch.Tensor:
    """``segment_offsets`` of a micro-batch's ``doc_ids`` over its ``n_docs + 1``
    slots, cached on the batch object: the PPO and distillation losses of one
    micro (forward, backward, later epochs) share it.  A batch from the pack
    kernels carries the offsets the pack wrote; for any other batch the order
    of ``doc_ids`` is checked once (ValueError when it decreases).  The keys
    include the tensor's version counter, so an in-place change of ``doc_ids``
    recomputes."""
    ids = mb.doc_ids
    key = (id(ids), ids._version, ids.data_ptr(), int(mb.n_docs))
    # Both caches name their doc_ids tensor by a weak reference as well as by
    # its id: a replaced tensor may reuse the id and the address of a freed one.
    hit = getattr(mb, "_meshy_seg_offsets", None)
    if hit is not None and hit[0] == key and hit[2]() is ids:
        return hit[1]
    src = getattr(mb, "_meshy_seg_src", None)
    # Written by the pack kernel next to doc_ids: no pass over the ids.
    off = src[0].seg_offsets(src[1], ids, key[3]) if src is not None and src[2] is ids else None
    if off is None:
        off = checked_segment_offsets(ids, int(mb.n_docs) + 1)
    try:
        object.__setattr__(mb, "_meshy_seg_offsets", (key, off, weakref.ref(ids)))
    except (AttributeError, TypeError):
        pass  # a batch type without an attribute dict: no cache
    return off


class DocIdRangeError(ValueError):
    """A doc id outside the document slots and the padding slot (the
    reference's ``index_add_`` raises there)."""


class UnsortedDocIdsError(ValueError):
    """doc_ids that decrease somewhere over the flattened micro-batch.  The
    losses and the per-sequence mean then run on the tokens in document order
    (``doc_order``); the offsets-based kernels alone refuse them."""


# Segment offsets of recently seen doc_ids tensors whose order was checked,
# or the ValueError a rejected tensor raised.  Entries hold a weak reference to
# their tensor: a hit needs the same live object (its id and data pointer
# may be reused once it is freed), and the cache never keeps a batch alive.
_CHECKED: dict[tuple, tuple[weakref.ref, torch.Tensor | ValueError]] = {}
_CHECKED_MAX = 16


def checked_segment_offsets(doc_ids: torch.Tensor, n_slots: int) -> torch.Tensor:
    """``segment_offsets`` of ``doc_ids`` after checking, once per tensor and
    version (one device sync), that its flattened values are non-decreasing
    and lie in ``[0, n_slots - 1]``; raises ValueError otherwise (the
    reference's ``index_add_`` raises on an id out of range).  The kernels that
    take these offsets rely on that order, which both batch layouts have
    (batch.py:123, 150-162), and visit only tokens inside the slots' ranges."""
    key = (id(doc_ids), doc_ids._version, doc_ids.data_ptr(), int(n_slots))
    hit = _CHECKED.get(key)
    if hit is not None and hit[0]() is doc_ids:
        off = hit[1]
    else:
        try:
            off = segment_offsets(doc_ids, n_slots, check_sorted=True)
        except ValueError as e:
            off = e
        _CHECKED.pop(key, None)
        if len(_CHECKED) >= _CHECKED_MAX:
            _CHECKED.pop(next(iter(_CHECKED)))
        _CHECKED[key] = (weakref.ref(doc_ids), off)
    if isinstance(off, ValueError):
        raise type(off)(*off.args)
    return off


def segment_offsets(doc_ids: torch.Tensor, n_slots: int, check_sorted: bool = False) -> torch.Tensor:
    """Token offsets of each document slot of a non-decreasing ``doc_ids`` tensor."""
    ids = doc_ids.reshape(-1).to(torch.int64).contiguous()
    off = torch.empty(n_slots + 1, dtype=torch.int64, device=ids.device)
    flag = torch.zeros(1, dtype=torch.int32, device=ids.device) if check_sorted else None
    rc = _lib.load().meshy_segment_offsets(ids.data_ptr(), ids.numel(), n_slots, off.data_ptr(),
                                           _lib.ptr(flag), _lib.stream_of(ids.device))
    _lib.check(rc, "meshy_segment_offsets")
    if check_sorted:
        bad = int(flag.item())
        if bad & 2:
            raise DocIdRangeError(f"doc_ids must lie in [0, {n_slots - 1}] (the document slots and the padding slot)")
        if bad & 1:
            raise UnsortedDocIdsError("doc_ids must be non-decreasing over the flattened micro-batch")
    return off


def doc_order(doc_ids: torch.Tensor, n_slots: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(perm, sorted_ids)``: the stable order of the flattened ``doc_ids``'
    tokens by document (``perm[k]`` is the k-th token's position, equal ids
    keep their order) and the ids in that order, from ``meshy_doc_order``.
    The ids must lie in ``[0, n_slots)``."""
    ids = doc_ids.reshape(-1).to(torch.int64).contiguous()
    n = ids.numel()
    perm = torch.empty(n, dtype=torch.int64, device=ids.device)
    sorted_ids = torch.empty_like(perm)
    if n == 0:
        return perm, sorted_ids
    lib = _lib.load()
    with torch.cuda.device(ids.device):
        ws_bytes = int(lib.meshy_doc_order_workspace_size(n, n_slots))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=ids.device)
        rc = lib.meshy_doc_order(ids.data_ptr(), n, n_slots, sorted_ids.data_ptr(), perm.data_ptr(), ws.data_ptr(),
                                 ws_bytes, _lib.stream_of(ids.device))
    _lib.check(rc, "meshy_doc_order")
    return perm, sorted_ids


class DocOrdered:
    """A micro-batch's tokens in document order: the per-token tensors named
    in ``token_fields`` gathered through ``perm`` into ``[1, T, ...]`` tensors,
    ``doc_ids`` sorted, every other attribute the batch's own.  The losses run
    on it as on a batch whose ids never decrease; per-token inputs passed
    beside the batch go through ``gather``, which keeps the autograd graph, so
    gradients land back on the original positions."""

    def __init__(self, mb: Any, token_fields: tuple[str, ...]) -> None:
        n_slots = int(mb.n_docs) + 1
        self.perm, sorted_ids = doc_order(mb.doc_ids, n_slots)
        self._mb = mb
        self._cache: dict[tuple, torch.Tensor] = {}
        self.doc_ids = sorted_ids.reshape(1, -1)
        for name in token_fields:
            t = getattr(mb, name, None)
            object.__setattr__(self, name, None if t is None else self.gather(t))

    def gather(self, t: torch.Tensor) -> torch.Tensor:
        """``t``'s tokens in document order: ``[1, T]`` for one value per token,
        ``[1, T, K]`` for K (the leading dimensions of ``t`` hold the T tokens)."""
        T = self.perm.numel()
        if t.numel() == T:
            return t.reshape(T).index_select(0, self.perm).reshape(1, T)
        if T == 0 or t.numel() % T:
            raise ValueError(f"a per-token tensor of {t.numel()} elements for {T} tokens")
        return t.reshape(T, -1).index_select(0, self.perm).reshape(1, T, -1)

    def gather_cached(self, t: torch.Tensor | None) -> torch.Tensor | None:
        """``gather`` of a tensor that needs no gradient, kept while it is unchanged."""
        if t is None:
            return None
        key = tensor_key(t)
        hit = self._cache.get(key)
        if hit is None:
            hit = self.gather(t.detach())
            self._cache.clear()
            self._cache[key] = hit
        return hit

    def __getattr__(self, name: str) -> Any:
        # The library's own caches (offsets, inputs) belong to each object.
        if name.startswith("_meshy"):
            raise AttributeError(name)
        return getattr(self._mb, name)


def doc_ordered(mb: Any, token_fields: tuple[str, ...]) -> DocOrdered:
    """The batch's ``DocOrdered`` copy, kept on the batch while its ids and
    the gathered fields are unchanged (later epochs over one micro)."""
    refs = (mb.doc_ids, *[getattr(mb, f, None) for f in token_fields])
    key = (tuple(tensor_key(t) for t in refs), int(mb.n_docs), token_fields)
    return batch_cached(mb, "_meshy_doc_ordered", key, refs, lambda: DocOrdered(mb, token_fields))


class _Inputs:
    """Everything the two kernels read besides new_lp, read once per micro-batch
    (``native``: the argument struct over the batch's tensors, which each
    call's backward holds)."""

    def __init__(self, stub, new_lp, old_lp, mb, mini, entropy) -> None:
        self.n_tokens = new_lp.numel()
        self.has_rollout = mb.rollout_logprobs is not None
        self.has_entropy = entropy is not None
        use_icepop = bool(getattr(stub, "use_icepop", False))
        coef = float(getattr(stub, "positive_lm_loss_coef", 0.0) or 0.0)
        if use_icepop and not self.has_rollout:
            raise ValueError("IcePop requires rollout log-probabilities")
        if coef and mb.positive_lm_weights is None:
            raise ValueError("Positive LM loss requires group weights")
        _lib.require_gpu(new_lp, mb.doc_ids)
        self.seg_off = batch_segment_offsets(mb)
        # The native reader checks that every tensor is on the GPU and has the
        # tokens (or documents) the kernels read, and flattens them.
        self.native = _lib.autograd().ppo_inputs(
            old_lp, mb.mask, mb.rollout_logprobs, entropy, mb.advantages,
            mb.positive_lm_weights if coef else None, mb.doc_ids, self.seg_off, self.n_tokens, int(mb.n_docs),
            int(mini.n_docs_global), int(mini.n_tokens_global), float(stub.ppo_clip_eps_low),
            float(stub.ppo_clip_eps_high), float(getattr(stub, "tis_ratio_min", 0.5)),
            float(getattr(stub, "tis_ratio_max", 5.0)), coef, bool(stub.use_tis) and not use_icepop, use_icepop,
            bool(stub.calculate_per_token_loss), getattr(stub, "old_logprobs_source", "rollout") == "train",
            max(1, int(getattr(getattr(stub, "parallel_dims", None), "cp", 1) or 1)))

    def args(self, new_flat: torch.Tensor | None, grad_unit: torch.Tensor | None = None) -> _lib.PpoArgs:
        """The argument struct with new_lp and grad_unit set, for callers that
        drive the C ABI themselves."""
        a = _lib.PpoArgs.from_buffer_copy(_lib.autograd().args_bytes(self.native))
        a.new_lp = _lib.ptr(new_flat)
        a.grad_unit = _lib.ptr(grad_unit)
        return a


def tensor_key(t: torch.Tensor | None) -> tuple:
    return (None,) if t is None else (id(t), t._version, t.data_ptr())


def _inputs_key(stub, new_lp, old_lp, mb, mini, entropy) -> tuple:
    """Everything an _Inputs is built from: each tensor's identity, version and
    address, the batch's document count, the loss settings and the global
    denominators."""
    pd = getattr(stub, "parallel_dims", None)
    return (new_lp.numel(), new_lp.device, tensor_key(old_lp), tensor_key(mb.mask),
            tensor_key(mb.rollout_logprobs), tensor_key(entropy), tensor_key(mb.advantages),
            tensor_key(mb.positive_lm_weights), tensor_key(mb.doc_ids), int(mb.n_docs),
            stub.ppo_clip_eps_low, stub.ppo_clip_eps_high, stub.use_tis, getattr(stub, "use_icepop", False),
            getattr(stub, "tis_ratio_min", 0.5), getattr(stub, "tis_ratio_max", 5.0),
            getattr(stub, "positive_lm_loss_coef", 0.0), stub.calculate_per_token_loss,
            getattr(stub, "old_logprobs_source", "rollout"), getattr(pd, "cp", 1),
            int(mini.n_docs_global), int(mini.n_tokens_global))


def batch_cached(mb: Any, attr: str, key: tuple, refs: tuple, build):
    """``build()``'s value, kept on the batch object under ``attr`` and reused
    while ``key`` and the tensors ``refs`` name are unchanged (later PPO epochs
    over one micro).  The tensors are named by weak references as well as by
    id, since a freed tensor's id and address may be reused; an in-place
    change bumps a version, which ``key`` carries."""
    hit = getattr(mb, attr, None)
    if hit is not None and hit[0] == key and all((r is None and t is None) or (r is not None and r() is t)
                                                 for r, t in zip(hit[2], refs)):
        return hit[1]
    value = build()
    try:
        object.__setattr__(mb, attr, (key, value, tuple(None if t is None else weakref.ref(t) for t in refs)))
    except (AttributeError, TypeError):
        pass  # a batch type without an attribute dict: no cache
    return value


def _cached_inputs(stub, new_lp, old_lp, mb, mini, entropy) -> _Inputs:
    """The _Inputs of this call, reused from the batch's previous call when
    nothing it was built from has changed."""
    return batch_cached(mb, "_meshy_ppo_inputs", _inputs_key(stub, new_lp, old_lp, mb, mini, entropy),
                        (old_lp, mb.mask, mb.rollout_logprobs, entropy, mb.advantages, mb.positive_lm_weights,
                         mb.doc_ids),
                        lambda: _Inputs(stub, new_lp, old_lp, mb, mini, entropy))


def ppo_clip_loss(
    self: Any,
    new_lp: torch.Tensor,
    old_lp: torch.Tensor,
    mb: Any,
    mini: Any,
    entropy: torch.Tensor | None = None,
) -> tuple[torch.Tensor, dict[str, torch.Tensor]]:
    """Drop-in for ``TitanTrainer._ppo_clip_loss`` (trainer.py:705-848)."""
    sharder = getattr(self, "sharder", None)
    if sharder is not None and getattr(sharder, "enabled", False):
        raise NotImplementedError(
            "context-parallel PPO loss needs the per-document all-reduce between the two "
            "kernel phases; this library drives one GPU")
    try:
        inputs = _cached_inputs(self, new_lp, old_lp, mb, mini, entropy)
    except UnsortedDocIdsError:
        # Ids that decrease: the same loss over the tokens in document order
        # (new_lp's gather carries the gradient back to its positions).
        per_token_adv = mb.advantages is not None and mb.advantages.dim() != 1
        od = doc_ordered(mb, ("mask", "rollout_logprobs") + (("advantages",) if per_token_adv else ()))
        return ppo_clip_loss(self, od.gather(new_lp), od.gather_cached(old_lp), od, mini,
                             None if entropy is None else od.gather(entropy))
    # The kernels read new_lp as one flat fp32 array; a contiguous fp32 tensor
    # of any shape is passed as it is, so that no view node sits between the
    # loss's node and new_lp's (each autograd node costs host time).
    new_flat = new_lp
    if new_flat.dtype != torch.float32:
        new_flat = new_flat.float()
    if not new_flat.is_contiguous():
        new_flat = new_flat.contiguous()
    # One native call: the forward kernels, the loss (carrying a C++ backward
    # node when new_lp requires grad) and every sum as a 0-dim view.
    loss, parts = _lib.autograd().ppo_loss(new_flat, inputs.native)
    names = _lib.PPO_OUT_NAMES
    sums = dict(zip(names[:12], parts[:12]))
    if inputs.has_rollout:
        sums["train_rollout_kl_sum"] = parts[12]
        sums["train_rollout_logdiff_abs_sum"] = parts[13]
    if inputs.has_entropy:
        sums["entropy_sum"] = parts[14]
    return loss, sums


def reduce_mini_metrics(self: Any, sums: dict[str, torch.Tensor]) -> dict[str, float]:
    """Per-rank sums -> mini-batch metrics (trainer.py:1020-1047)."""
    keys = list(sums)
    stacked = torch.stack([sums[k].float().reshape(()) for k in keys])
    pd = getattr(self, "parallel_dims", None)
    loss_mesh = pd.get_optional_mesh("loss") if pd is not None and hasattr(pd, "get_optional_mesh") else None
    if loss_mesh is not None:
        dist.all_reduce(stacked, op=dist.ReduceOp.SUM, group=loss_mesh.get_group())
    values = dict(zip(keys, stacked.tolist()))
    tokens = max(values["token_count"], 1.0)
    out = {
        "pg_loss": values["loss"],
        "ratio_mean": values["ratio_sum"] / tokens,
        "clip_frac": values["clip_sum"] / tokens,
        "tis_masked_frac": values["tis_masked_sum"] / tokens,
        "ppo_kl": values["ppo_kl_sum"] / tokens,
        "log_ratio_abs_mean": values["log_ratio_abs_sum"] / tokens,
        "ess_ratio": values["ess_sum"] / max(values.get("doc_count", 0.0), 1.0),
    }
    if "train_rollout_kl_sum" in values:
        out["train_rollout_kl"] = values["train_rollout_kl_sum"] / tokens
        out["train_rollout_logdiff_abs"] = values["train_rollout_logdiff_abs_sum"] / tokens
    if "entropy_sum" in values:
        out["entropy"] = values["entropy_sum"] / tokens
    if "tis_ratio_sum" in values:
        out["tis_ratio_mean"] = values["tis_ratio_sum"] / tokens
        out["positive_lm_loss"] = values["positive_lm_loss"]
        out["total_loss"] = values["total_loss"]
    return out


__all__ = ["DocIdRangeError", "DocOrdered", "UnsortedDocIdsError", "batch_segment_offsets", "checked_segment_offsets",
           "doc_order", "doc_ordered", "ppo_clip_loss", "reduce_mini_metrics",
           "segment_offsets"]

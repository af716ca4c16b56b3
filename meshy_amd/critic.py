"""Critic-side reductions with the call surfaces of the reference's critic path.

* ``advantages_to_per_sequence`` (meshy/backend/titan/critic/gae.py:296-312):
  ``meshy_per_sequence_mean``, one workgroup per document;
* ``Accumulator`` / ``AccumulatorState`` (meshy/backend/titan/critic/metrics.py:
  220-275): ``meshy_critic_accumulate`` folds each ``[rows, S]`` micro-batch on
  the device; the window sums stay there until ``state`` is read, so a window
  of micro-batches costs one host synchronisation instead of five per update;
* ``clipped_value_error`` (meshy/backend/titan/vapo.py:35-41):
  ``meshy_clipped_value_error`` with its backward as a C++ autograd node.

* ``critic_diagnostics`` / ``diagnostics_from_states`` / ``CriticDiagnostics``
  and the gauges ``within_prompt_auc``, ``prompt_pearson``,
  ``variance_reduction``, ``calibration_gap`` (metrics.py:58-217, 278-328):
  ``meshy_critic_window_sums`` reduces the window's tokens and
  ``meshy_group_gauges`` its rows; one host read per call.

``compute_returns`` on the critic path (engine/critic.py:348-350) is
``meshy_amd.gae.compute_returns``.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field

import numpy as np
import torch

from . import _lib
from .gae import compute_returns
from .loss import UnsortedDocIdsError, checked_segment_offsets, doc_order


def _as_f32(t: torch.Tensor) -> torch.Tensor:
    """``t`` as a contiguous fp32 tensor of its shape, ``t`` itself when it
    already is one (differentiable: ``values`` keeps its graph)."""
    if t.dtype == torch.float32 and t.is_contiguous():
        return t
    return t.to(torch.float32).contiguous()


def advantages_to_per_sequence(adv: torch.Tensor, mask: torch.Tensor, doc_ids: torch.Tensor,
                               n_docs: int) -> torch.Tensor:
    """Masked token-mean of per-token ``adv``, one fp32 scalar per document
    (gae.py:296-312); the padding slot is ignored.  ``doc_ids`` in any order
    (non-decreasing, as both batch layouts make them, reads them as they
    are; otherwise the tokens are taken in document order first)."""
    _lib.require_gpu(adv, mask, doc_ids)
    n_docs = int(n_docs)
    out = torch.empty(n_docs, dtype=torch.float32, device=adv.device)
    if n_docs == 0:
        return out
    x = adv.reshape(-1).to(torch.float32).contiguous()
    m = mask.reshape(-1).to(torch.float32).contiguous()
    if m.numel() != x.numel() or doc_ids.numel() != x.numel():
        raise ValueError(f"adv has {x.numel()} tokens but mask and doc_ids have {m.numel()} and {doc_ids.numel()}")
    try:
        off = checked_segment_offsets(doc_ids, n_docs + 1)
    except UnsortedDocIdsError:
        perm, sorted_ids = doc_order(doc_ids, n_docs + 1)
        x, m = x.index_select(0, perm), m.index_select(0, perm)
        off = checked_segment_offsets(sorted_ids, n_docs + 1)
    rc = _lib.load().meshy_per_sequence_mean(x.data_ptr(), m.data_ptr(), off.data_ptr(), n_docs, out.data_ptr(),
                                             _lib.stream_of(adv.device))
    _lib.check(rc, "meshy_per_sequence_mean")
    return out


@dataclass
class AccumulatorState:
    """Per-rank partial sums of one window (metrics.py:220-235)."""

    n_tokens: float = 0.0
    sum_r: float = 0.0
    sum_r2: float = 0.0
    sum_d: float = 0.0
    sum_d2: float = 0.0
    row_value: list[float] = field(default_factory=list)
    row_reward: list[float] = field(default_factory=list)
    row_group: list[int] = field(default_factory=list)


class Accumulator:
    """Fold ``[rows, S]`` micro-batches into an :class:`AccumulatorState`
    (metrics.py:238-275), on the device."""

    def __init__(self) -> None:
        self._sums: torch.Tensor | None = None  # fp64 [5] on the device
        self._row_value: list[torch.Tensor] = []
        self._row_reward: list[torch.Tensor] = []
        self._row_group: list[torch.Tensor] = []
        self._state: AccumulatorState | None = AccumulatorState()

    @torch.no_grad()
    def update(self, values: torch.Tensor, returns: torch.Tensor, mask: torch.Tensor, rewards: torch.Tensor,
               group_ids: torch.Tensor) -> None:
        if values.dim() != 2 or returns.shape != values.shape or mask.shape != values.shape:
            raise ValueError("values, returns and mask must be [rows, S] of one shape")
        _lib.require_gpu(values, returns, mask)
        dev = values.device
        rows, S = values.shape
        bf16 = values.dtype == torch.bfloat16
        v = values.contiguous() if bf16 else values.to(torch.float32).contiguous()
        r = returns.to(torch.float32).contiguous()
        m = mask.to(torch.float32).contiguous()
        sums = torch.empty(5, dtype=torch.float64, device=dev)
        row_value = torch.empty(rows, dtype=torch.float32, device=dev)
        lib = _lib.load()
        ws = torch.empty(max(int(lib.meshy_critic_accumulate_workspace_size(rows)), 1), dtype=torch.uint8,
                         device=dev)
        rc = lib.meshy_critic_accumulate(v.data_ptr(), int(bf16), r.data_ptr(), m.data_ptr(), rows, S,
                                         sums.data_ptr(), row_value.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream_of(dev))
        _lib.check(rc, "meshy_critic_accumulate")
        self._sums = sums if self._sums is None else self._sums + sums
        self._row_value.append(row_value)
        self._row_reward.append(rewards.detach().reshape(-1).to(device=dev, dtype=torch.float32).contiguous())
        self._row_group.append(group_ids.detach().reshape(-1).to(device=dev, dtype=torch.int64).contiguous())
        self._state = None

    @property
    def state(self) -> AccumulatorState:
        """The window's partials as host values (one synchronisation)."""
        if self._state is None:
            st = AccumulatorState()
            if self._sums is not None:
                # One concatenation of the bytes and one device-to-host copy:
                # the fp64 sums, the fp32 row values and rewards, the int64
                # group ids, each read back on the host with its own type.
                parts = [self._sums, *self._row_value, *self._row_reward, *self._row_group]
                host = torch.cat([t.view(torch.uint8) for t in parts]).cpu().numpy()
                nv = sum(t.numel() for t in self._row_value)
                nr = sum(t.numel() for t in self._row_reward)
                ng = sum(t.numel() for t in self._row_group)
                o_v = 5 * 8
                o_r = o_v + 4 * nv
                o_g = o_r + 4 * nr
                st.n_tokens, st.sum_r, st.sum_r2, st.sum_d, st.sum_d2 = np.frombuffer(host, np.float64, 5).tolist()
                st.row_value = np.frombuffer(host, np.float32, nv, o_v).tolist()
                st.row_reward = np.frombuffer(host, np.float32, nr, o_r).tolist()
                st.row_group = np.frombuffer(host, np.int64, ng, o_g).tolist()
            self._state = st
        return self._state


@dataclass(frozen=True)
class CriticDiagnostics:
    """The window's critic gauges (metrics.py:162-186): the same fields, dict
    form and one-line text."""

    value_loss: float
    critic_auc: float
    critic_var_ratio: float
    critic_calibration_gap: float
    prompt_pearson: float
    n_rows: int
    n_prompts: int
    n_tokens: int

    def as_dict(self) -> dict[str, float]:
        return asdict(self)

    def __str__(self) -> str:
        return (
            f"value_loss={self.value_loss:.4f}  "
            f"within_prompt_auc={self.critic_auc:.4f}  "
            f"var_reduction={self.critic_var_ratio:+.4f}  "
            f"calib_gap={self.critic_calibration_gap:+.4f}  "
            f"prompt_pearson={self.prompt_pearson:+.4f}  "
            f"[{self.n_rows} rows / {self.n_prompts} prompts / {self.n_tokens} tokens]"
        )


def _window_sums(values: torch.Tensor, returns: torch.Tensor, mask: torch.Tensor):
    """The token sums of ``meshy_critic_window_sums`` (fp64 [10], device) and
    each row's masked mean value."""
    if values.dim() != 2 or returns.shape != values.shape or mask.shape != values.shape:
        raise ValueError("values, returns and mask must be [rows, S] of one shape")
    _lib.require_gpu(values, returns, mask)
    dev = values.device
    rows, S = values.shape
    bf16 = values.dtype == torch.bfloat16
    v = values.contiguous() if bf16 else values.to(torch.float32).contiguous()
    r = returns.to(torch.float32).contiguous()
    m = mask.to(torch.float32).contiguous()
    sums = torch.empty(_lib.CW_VALS, dtype=torch.float64, device=dev)
    row_value = torch.empty(rows, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.meshy_critic_window_workspace_size(rows)), 1), dtype=torch.uint8, device=dev)
    rc = lib.meshy_critic_window_sums(v.data_ptr(), int(bf16), r.data_ptr(), m.data_ptr(), rows, S, sums.data_ptr(),
                                      row_value.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(dev))
    _lib.check(rc, "meshy_critic_window_sums")
    return sums, row_value


def _group_gauges(row_value: torch.Tensor, row_reward: torch.Tensor, group_ids: torch.Tensor,
                  correct_threshold: float, device: torch.device) -> torch.Tensor:
    """``meshy_group_gauges`` on the device: fp64 [wins, pairs, groups, Pearson r]."""
    v = row_value.detach().reshape(-1).to(device=device, dtype=torch.float32).contiguous()
    r = row_reward.detach().reshape(-1).to(device=device, dtype=torch.float32).contiguous()
    g = group_ids.detach().reshape(-1).to(device=device, dtype=torch.int64).contiguous()
    n = v.numel()
    if r.numel() != n or g.numel() != n:
        raise ValueError(f"{n} row values but {r.numel()} rewards and {g.numel()} group ids")
    out = torch.empty(4, dtype=torch.float64, device=device)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.meshy_group_gauges_workspace_size(n)), 1), dtype=torch.uint8, device=device)
    rc = lib.meshy_group_gauges(v.data_ptr(), r.data_ptr(), g.data_ptr(), n, float(correct_threshold),
                                out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(device))
    _lib.check(rc, "meshy_group_gauges")
    return out


def _gauge_device(*tensors: torch.Tensor) -> torch.device:
    for t in tensors:
        if t.is_cuda:
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("the critic gauges run on a HIP device and none is available")
    return torch.device("cuda", torch.cuda.current_device())


def _auc(gauges: list[float]) -> float:
    return gauges[0] / gauges[1] if gauges[1] > 0 else float("nan")


def within_prompt_auc(row_value: torch.Tensor, row_correct: torch.Tensor, group_ids: torch.Tensor) -> float:
    """Pooled-pairs AUC of V ranking a prompt's correct rows above its
    incorrect ones, ties 1/2; NaN when no prompt holds both (metrics.py:94-118)."""
    dev = _gauge_device(row_value, row_correct, group_ids)
    return _auc(_group_gauges(row_value, row_correct.float(), group_ids, 0.5, dev).tolist())


def prompt_pearson(row_value: torch.Tensor, row_reward: torch.Tensor, group_ids: torch.Tensor) -> float:
    """Pearson r between each prompt's mean V and its mean reward; NaN for
    fewer than two prompts or a constant side (metrics.py:64-91)."""
    dev = _gauge_device(row_value, row_reward, group_ids)
    return float(_group_gauges(row_value, row_reward, group_ids, 0.5, dev)[3].item())


def _var_ratio(c: list[float]) -> float:
    n = c[_lib.CW_SEL]
    if n < 2 or c[_lib.CW_RMIN] == c[_lib.CW_RMAX]:
        return float("nan")  # too few tokens, or constant returns (zero variance)
    var_r = c[_lib.CW_R2] / n - (c[_lib.CW_R] / n) ** 2
    var_d = c[_lib.CW_D2] / n - (c[_lib.CW_D] / n) ** 2
    return 1.0 - var_d / var_r


def variance_reduction(values: torch.Tensor, returns: torch.Tensor, mask: torch.Tensor) -> float:
    """``1 - Var(return - V) / Var(return)`` over the tokens with mask > 0
    (metrics.py:120-138)."""
    sums, _ = _window_sums(values, returns, mask)
    return _var_ratio(sums.tolist())


def calibration_gap(values: torch.Tensor, returns: torch.Tensor, mask: torch.Tensor) -> float:
    """Mean signed error ``sum (V - return) m / max(sum m, 1)`` (metrics.py:141-160)."""
    c = _window_sums(values, returns, mask)[0].tolist()
    return c[_lib.CW_EM] / max(c[_lib.CW_M], 1.0)


def critic_diagnostics(values: torch.Tensor, returns: torch.Tensor, mask: torch.Tensor, rewards: torch.Tensor,
                       group_ids: torch.Tensor, *, correct_threshold: float = 0.5) -> CriticDiagnostics:
    """The four gauges plus the masked value loss of a whole [rows, S] window
    (metrics.py:189-217), from one pass over its tokens and one over its rows."""
    sums, row_value = _window_sums(values, returns, mask)
    if rewards.numel() != values.shape[0] or group_ids.numel() != values.shape[0]:
        raise ValueError(f"{values.shape[0]} rows but {rewards.numel()} rewards and {group_ids.numel()} group ids")
    gauges = _group_gauges(row_value, rewards.float(), group_ids, correct_threshold, values.device)
    c = torch.cat([sums, gauges]).tolist()  # one host read
    g = c[_lib.CW_VALS:]
    n_tok = max(c[_lib.CW_M], 1.0)
    return CriticDiagnostics(
        value_loss=c[_lib.CW_E2M] / n_tok,
        critic_auc=_auc(g),
        critic_var_ratio=_var_ratio(c),
        critic_calibration_gap=c[_lib.CW_EM] / n_tok,
        prompt_pearson=g[3],
        n_rows=int(values.shape[0]),
        n_prompts=int(g[2]),
        n_tokens=int(c[_lib.CW_M]),
    )


def diagnostics_from_states(states: list[AccumulatorState], *, correct_threshold: float = 0.5,
                            device: torch.device | str | None = None) -> CriticDiagnostics:
    """Merge per-rank partials into the gauges ``critic_diagnostics`` gives
    (metrics.py:278-328): the token gauges from the five sums, the per-prompt
    gauges from the rows (any order, any rank) on the device."""
    n = sum(s.n_tokens for s in states)
    if n <= 0:
        raise ValueError("cannot build diagnostics from states with no masked tokens")
    sum_r = sum(s.sum_r for s in states)
    sum_r2 = sum(s.sum_r2 for s in states)
    sum_d = sum(s.sum_d for s in states)
    sum_d2 = sum(s.sum_d2 for s in states)
    # Var(x) = E[x^2] - E[x]^2, the population form
    var_r = sum_r2 / n - (sum_r / n) ** 2
    var_d = sum_d2 / n - (sum_d / n) ** 2
    var_ratio = float("nan") if var_r == 0.0 or n < 2 else 1.0 - var_d / var_r
    dev = torch.device(device) if device is not None else _gauge_device()
    row_value = torch.tensor([x for s in states for x in s.row_value], dtype=torch.float32)
    row_reward = torch.tensor([x for s in states for x in s.row_reward], dtype=torch.float32)
    group_ids = torch.tensor([x for s in states for x in s.row_group], dtype=torch.int64)
    g = _group_gauges(row_value, row_reward, group_ids, correct_threshold, dev).tolist()
    return CriticDiagnostics(
        value_loss=sum_d2 / n,
        critic_auc=_auc(g),
        critic_var_ratio=var_ratio,
        critic_calibration_gap=sum_d / n,
        prompt_pearson=g[3],
        n_rows=int(row_value.numel()),
        n_prompts=int(g[2]),
        n_tokens=int(n),
    )


def clipped_value_error(values: torch.Tensor, targets: torch.Tensor, old_values: torch.Tensor | None,
                        clip: float | None) -> torch.Tensor:
    """Per-token ``(v - t)^2``, or with ``clip`` the PPO-style clipped maximum
    (vapo.py:35-41); differentiable in ``values``."""
    _lib.require_gpu(values, targets, old_values if clip is not None else None)
    v = _as_f32(values)
    t = _as_f32(targets.detach())
    o = None
    if clip is not None:
        o = _as_f32(old_values.detach())
    # One native call (which checks the sizes); the output has values' shape
    # and carries a C++ backward node when values requires grad.  Contiguous
    # fp32 inputs are passed as they are: no view node sits between the
    # output's node and values' (each autograd node costs host time).
    return _lib.autograd().clipped_value_error(v, t, o, None if clip is None else float(clip))


__all__ = ["Accumulator", "AccumulatorState", "CriticDiagnostics", "advantages_to_per_sequence",
           "calibration_gap", "clipped_value_error", "compute_returns", "critic_diagnostics",
           "diagnostics_from_states", "prompt_pearson", "variance_reduction", "within_prompt_auc"]

"""ctypes binding of libmeshy_amd.so (declared in include/meshy_amd.h).

The library is the only compute path of this package: every public function
routes through it, and loading fails loudly when the shared object has not
been built (``python -c "import __graft_entry__ as g; g.build()"``).
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p

LIB_NAME = "libmeshy_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

MESHY_LAYOUT_PADDED = 0
MESHY_LAYOUT_PACKED = 1

# enum meshy_ppo_out
PPO_OUT_NAMES = (
    "loss",
    "total_loss",
    "positive_lm_loss",
    "tis_ratio_sum",
    "ratio_sum",
    "clip_sum",
    "tis_masked_sum",
    "token_count",
    "ppo_kl_sum",
    "log_ratio_abs_sum",
    "ess_sum",
    "doc_count",
    "train_rollout_kl_sum",
    "train_rollout_logdiff_abs_sum",
    "entropy_sum",
)
PPO_NOUT = len(PPO_OUT_NAMES)

# meshy_critic_window_sums' value order (MESHY_CW_* in include/meshy_amd.h)
CW_SEL, CW_R, CW_R2, CW_D, CW_D2, CW_M, CW_E2M, CW_EM, CW_RMIN, CW_RMAX = range(10)
CW_VALS = 10


class PlannerCfg(ctypes.Structure):
    _fields_ = [
        ("layout", c_int32),
        ("reserved", c_int32),
        ("mini_batch_size", c_int64),
        ("seq_len", c_int64),
        ("align", c_int64),
        ("max_tokens_per_micro", c_int64),
        ("micro_batch_size", c_int64),
    ]


class PlanOut(ctypes.Structure):
    # int32_t* / int64_t* tables, set from numpy addresses
    _fields_ = [
        ("local_indices", c_void_p),
        ("mini_n_micro", c_void_p),
        ("mini_n_docs_global", c_void_p),
        ("mini_n_tokens_global", c_void_p),
        ("mini_tokens_per_rank", c_void_p),
        ("micro_seq_len", c_void_p),
        ("micro_doc_start", c_void_p),
        ("doc_sample", c_void_p),
        ("doc_len", c_void_p),
        ("n_micro_total", c_int32),
        ("reserved", c_int32),
    ]


class StepPlanArgs(ctypes.Structure):
    _fields_ = [
        ("mask", c_void_p),
        ("offsets", c_void_p),
        ("n", c_int64),
        ("dp_size", c_int64),
        ("rank", c_int64),
        ("cfg", PlannerCfg),
        ("plan", PlanOut),
        ("lengths", c_void_p),
        ("loss_tokens", c_void_p),
        ("micro_seq_len", c_void_p),
        ("micro_out_off", c_void_p),
        ("micro_doc_start", c_void_p),
        ("doc_sample", c_void_p),
        ("doc_len", c_void_p),
        ("n_micro", c_int64),
        ("n_docs", c_int64),
        ("max_micro_elems", c_int64),
        ("max_docs_per_micro", c_int64),
        ("mask_u8", c_int32),
        ("reserved", c_int32),
    ]


class PackArgs(ctypes.Structure):
    _fields_ = [
        ("tokens", c_void_p),
        ("tokens_elem_bytes", c_int32),
        ("layout", c_int32),
        ("mask", c_void_p),
        ("logprobs", c_void_p),
        ("adv_tokens", c_void_p),
        ("adv_samples", c_void_p),
        ("sample_offsets", c_void_p),
        ("n_samples", c_int64),
        ("n_micro", c_int64),
        ("micro_seq_len", c_void_p),
        ("micro_out_off", c_void_p),
        ("micro_doc_start", c_void_p),
        ("doc_sample", c_void_p),
        ("doc_len", c_void_p),
        ("max_micro_elems", c_int64),
        ("max_docs_per_micro", c_int64),
        ("input_ids", c_void_p),
        ("labels", c_void_p),
        ("positions", c_void_p),
        ("mask_out", c_void_p),
        ("doc_ids", c_void_p),
        ("rollout_lp", c_void_p),
        ("adv_tok", c_void_p),
        ("adv_doc", c_void_p),
        ("doc_len_out", c_void_p),
        ("cu_seqlens", c_void_p),
        ("teacher_k", c_int64),
        ("teacher_ids", c_void_p),
        ("teacher_lps", c_void_p),
        ("teacher_ids_out", c_void_p),
        ("teacher_lps_out", c_void_p),
        ("teacher_ids_elem_bytes", c_int32),
        ("mask_u8", c_int32),
        ("seg_offsets", c_void_p),
    ]


# enum meshy_distill_out
DISTILL_OUT_NAMES = (
    "loss",
    "token_count",
    "student_mass_sum",
    "teacher_mass_sum",
    "train_rollout_kl_sum",
    "train_rollout_logdiff_abs_sum",
)
DISTILL_NOUT = len(DISTILL_OUT_NAMES)


class DistillArgs(ctypes.Structure):
    _fields_ = [
        ("student", c_void_p),
        ("teacher", c_void_p),
        ("mask", c_void_p),
        ("rollout_lp", c_void_p),
        ("seg_offsets", c_void_p),
        ("doc_ids", c_void_p),
        ("n_tokens", c_int64),
        ("n_docs", c_int64),
        ("k", c_int64),
        ("n_docs_global", c_int64),
        ("n_tokens_global", c_int64),
        ("lp_min_clamp", c_float),
        ("loss_max_clamp", c_float),
        ("has_lp_clamp", c_int32),
        ("has_loss_clamp", c_int32),
        ("per_token_loss", c_int32),
        ("reserved", c_int32),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
    ]


class PpoArgs(ctypes.Structure):
    _fields_ = [
        ("new_lp", c_void_p),
        ("old_lp", c_void_p),
        ("mask", c_void_p),
        ("rollout_lp", c_void_p),
        ("entropy", c_void_p),
        ("adv", c_void_p),
        ("positive_lm_weights", c_void_p),
        ("seg_offsets", c_void_p),
        ("doc_ids", c_void_p),
        ("grad_unit", c_void_p),
        ("n_tokens", c_int64),
        ("n_docs", c_int64),
        ("n_docs_global", c_int64),
        ("n_tokens_global", c_int64),
        ("clip_low", c_float),
        ("clip_high", c_float),
        ("tis_min", c_float),
        ("tis_max", c_float),
        ("positive_lm_coef", c_float),
        ("adv_per_token", c_int32),
        ("use_tis", c_int32),
        ("use_icepop", c_int32),
        ("per_token_loss", c_int32),
        ("train_lp_is_old", c_int32),
        ("cp_degree", c_int32),
        ("reserved", c_int32),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
    ]


class GaeArgs(ctypes.Structure):
    _fields_ = [
        ("rewards", c_void_p),
        ("values", c_void_p),
        ("mask", c_void_p),
        ("doc_ids", c_void_p),
        ("lengths", c_void_p),
        ("rows", c_int64),
        ("S", c_int64),
        ("n_docs", c_int64),
        ("gamma", c_float),
        ("alpha", c_float),
        ("epsilon", c_float),
        ("values_bf16", c_int32),
        ("adv", c_void_p),
        ("returns", c_void_p),
        ("lam_doc", c_void_p),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
        ("seg_offsets", c_void_p),
    ]


class GaeAttachArgs(ctypes.Structure):
    _fields_ = [
        ("mask_assistant", c_void_p),
        ("values", c_void_p),
        ("reward", c_void_p),
        ("offsets", c_void_p),
        ("n", c_int64),
        ("total", c_int64),
        ("gamma", c_float),
        ("alpha", c_float),
        ("lambda_", c_float),
        ("epsilon", c_float),
        ("values_bf16", c_int32),
        ("mask_u8", c_int32),
        ("adv", c_void_p),
        ("grid_mask", c_void_p),
        ("lam_doc", c_void_p),
        ("metrics", c_void_p),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
    ]


# name -> (restype, argtypes); every symbol include/meshy_amd.h declares.
SIGNATURES = {
    "meshy_last_error": (ctypes.c_char_p, []),
    "meshy_abi_version": (c_int, []),
    "meshy_copy_to_device": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "meshy_plan_build": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, POINTER(PlannerCfg), POINTER(PlanOut)],
    ),
    "meshy_sample_loss_tokens": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "meshy_sample_loss_tokens_u8": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "meshy_step_plan": (c_int, [POINTER(StepPlanArgs)]),
    "meshy_host_gather": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int]),
    "meshy_host_gather_mask_u8": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int, POINTER(c_int32)]),
    "meshy_host_gather_i32": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int, POINTER(c_int32)]),
    "meshy_pack_micro_batches": (c_int, [POINTER(PackArgs), c_void_p]),
    "meshy_grpo_advantage": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "meshy_zero_variance_groups": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_double, c_void_p, c_void_p]),
    "meshy_zero_variance_groups_host": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_double, c_void_p]),
    "meshy_grpo_advantage_host": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "meshy_logprob_entropy_fwd": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p],
    ),
    "meshy_logprob_bwd_workspace_size": (c_size_t, [c_int64]),
    "meshy_logprob_bwd": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "meshy_logprob_bwd_noalloc": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p],
    ),
    "meshy_gather_logprobs_fwd": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p,
         c_void_p, c_void_p],
    ),
    "meshy_gather_logprobs_bwd": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p,
         c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "meshy_topk_logprobs": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p,
         c_void_p, c_void_p],
    ),
    "meshy_forward_kl_topk": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int32, c_float, c_int32, c_float, c_void_p,
         c_void_p],
    ),
    "meshy_forward_kl_topk_bwd": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int32, c_float, c_int32, c_float, c_void_p,
         c_void_p, c_void_p],
    ),
    "meshy_distill_workspace_size": (c_size_t, [c_int64, c_int64]),
    "meshy_distill_loss_fwd": (c_int, [POINTER(DistillArgs), c_void_p, c_void_p, c_void_p]),
    "meshy_distill_loss_bwd": (c_int, [POINTER(DistillArgs), c_void_p, c_void_p, c_void_p, c_void_p]),
    "meshy_segment_offsets": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "meshy_ppo_workspace_size": (c_size_t, [c_int64, c_int64]),
    "meshy_ppo_loss_fwd": (c_int, [POINTER(PpoArgs), c_void_p, c_void_p, c_void_p]),
    "meshy_ppo_loss_bwd": (c_int, [POINTER(PpoArgs), c_void_p, c_void_p, c_void_p, c_void_p]),
    "meshy_gae_workspace_size": (c_size_t, [c_int64, c_int64, c_int64]),
    "meshy_gae": (c_int, [POINTER(GaeArgs), c_void_p]),
    "meshy_gae_set_poll_limit": (c_int, [c_int]),
    "meshy_doc_order_workspace_size": (c_size_t, [c_int64, c_int64]),
    "meshy_doc_order": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "meshy_gae_attach_workspace_size": (c_size_t, [c_int64, c_int64]),
    "meshy_gae_attach": (c_int, [POINTER(GaeAttachArgs), c_void_p]),
    "meshy_whiten_workspace_size": (c_size_t, [c_int64]),
    "meshy_whiten_stats": (
        c_int, [c_void_p, c_void_p, c_int64, c_double, c_void_p, c_void_p, c_size_t, c_void_p]
    ),
    "meshy_whiten_apply": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "meshy_stream_read": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "meshy_per_sequence_mean": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "meshy_critic_accumulate_workspace_size": (c_size_t, [c_int64]),
    "meshy_synth_bf16": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_uint64, c_float, c_void_p]),
    "meshy_synth_bf16_rows_host": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_uint64, c_float]),
    "meshy_critic_window_workspace_size": (c_size_t, [c_int64]),
    "meshy_critic_window_sums": (
        c_int, [c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                c_size_t, c_void_p]
    ),
    "meshy_group_gauges_workspace_size": (c_size_t, [c_int64]),
    "meshy_group_gauges": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_float, c_void_p, c_void_p, c_size_t, c_void_p]
    ),
    "meshy_critic_accumulate": (
        c_int, [c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                c_size_t, c_void_p]
    ),
    "meshy_clipped_value_error": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_float, c_int64, c_void_p, c_void_p]
    ),
    "meshy_clipped_value_error_bwd": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_float, c_int64, c_void_p, c_int64, c_void_p, c_void_p]
    ),
    "meshy_ragged_token_stats_workspace_size": (c_size_t, [c_int64]),
    "meshy_ragged_token_stats": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                c_void_p, c_size_t, c_void_p]
    ),
}

ABI_VERSION = 14

_LIB: ctypes.CDLL | None = None


class MeshyError(RuntimeError):
    """A HIP error raised by a launch inside libmeshy_amd."""


def load() -> ctypes.CDLL:
    """Load libmeshy_amd.so once; raise if it is missing or stale."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.meshy_abi_version() != ABI_VERSION:
        raise ImportError(f"{LIB_PATH} has ABI {lib.meshy_abi_version()}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


_PYIO = None


def pyio():
    """The CPython helper module meshy_amd._pyio (built beside the library)."""
    global _PYIO
    if _PYIO is None:
        try:
            from . import _pyio as mod
        except ImportError as e:
            raise ImportError("meshy_amd._pyio is not built; run __graft_entry__.build()") from e
        _PYIO = mod
    return _PYIO


_STAGE = None


def stage():
    """The CPython helper module meshy_amd._stage (built beside the library)."""
    global _STAGE
    if _STAGE is None:
        try:
            from . import _stage as mod
        except ImportError as e:
            raise ImportError("meshy_amd._stage is not built; run __graft_entry__.build()") from e
        _STAGE = mod
    return _STAGE


_AUTOGRAD = None


def autograd():
    """The CPython extension meshy_amd._autograd (the loss drop-ins' autograd
    nodes, built beside the library)."""
    global _AUTOGRAD
    if _AUTOGRAD is None:
        load()  # the module links libmeshy_amd.so; load it (and its checks) first
        try:
            from . import _autograd as mod
        except ImportError as e:
            raise ImportError("meshy_amd._autograd is not built; run __graft_entry__.build()") from e
        mod.set_error_type(MeshyError)
        _AUTOGRAD = mod
    return _AUTOGRAD


def check(rc: int, what: str) -> None:
    """Raise the Python error matching a C-ABI return code."""
    if rc == 0:
        return
    msg = load().meshy_last_error().decode(errors="replace") or what
    if rc < 0:
        raise ValueError(msg)
    raise MeshyError(f"{what}: {msg} (hip error {rc})")


def ptr(t) -> int | None:
    """Device (or host) address of a tensor, or None."""
    if t is None:
        return None
    return t.data_ptr()


def stream_of(device) -> int:
    """The current HIP stream of `device` as an integer handle (the raw getter:
    no Stream object is built on the hot path)."""
    import torch

    if isinstance(device, int):
        idx = device
    else:
        idx = device.index if isinstance(device, torch.device) else torch.device(device).index
        if idx is None:
            idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def require_gpu(*tensors) -> None:
    """Every kernel entry point runs on a HIP device; CPU tensors are an error."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(
                "meshy_amd kernels run on the GPU; got a CPU tensor (move inputs to a HIP device)"
            )

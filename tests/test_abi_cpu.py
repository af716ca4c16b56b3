"""Argument validation of the C ABI (CPU only): every device entry point rejects
bad shapes, NULL pointers and short workspaces with a negative MESHY_E* code
and a message, before anything reaches a device.  No call here passes its
checks, so no kernel is launched."""

from __future__ import annotations

import ctypes

import pytest

from meshy_amd import _lib

EINVAL, ENULL, EALIGN, ESPACE = -1, -2, -3, -4
FAKE = 0x1000  # a non-NULL address never dereferenced: each call fails its checks first


def _call(name, *args):
    lib = _lib.load()
    rc = getattr(lib, name)(*args)
    msg = lib.meshy_last_error().decode()
    return rc, msg


@pytest.mark.parametrize("name,args,code,text", [
    # logits, rows, T, V, stride_b, stride_t, labels, logp, entropy, lse, stream
    ("meshy_logprob_entropy_fwd", (None, 1, 4, 8, 32, 8, FAKE, FAKE, None, None, None), ENULL, "logits is NULL"),
    ("meshy_logprob_entropy_fwd", (FAKE, 1, 4, 0, 32, 8, FAKE, FAKE, None, None, None), EINVAL, "bad shape"),
    ("meshy_logprob_entropy_fwd", (FAKE, 1, 4, 8, -1, 8, FAKE, FAKE, None, None, None), EINVAL, "negative stride"),
    ("meshy_logprob_entropy_fwd", (FAKE, 1, 4, 8, 32, 8, None, FAKE, None, None, None), ENULL, "logp needs labels"),
    ("meshy_logprob_entropy_fwd", (FAKE, 1 << 16, 1 << 16, 8, 8, 8, FAKE, FAKE, None, None, None), EINVAL,
     "too many rows"),
    ("meshy_gather_logprobs_fwd", (FAKE, 1, 4, 8, 32, 8, FAKE, 0, FAKE, None, None), EINVAL, "n_ids"),
    ("meshy_gather_logprobs_fwd", (FAKE, 1, 4, 8, 32, 8, FAKE, 257, FAKE, None, None), EINVAL, "n_ids"),
    ("meshy_gather_logprobs_fwd", (FAKE, 1, 4, 8, 32, 8, None, 3, FAKE, None, None), ENULL, "ids and out"),
    # logits, rows, T, V, sb, st, labels, lse, grad_logp, grad, ws, ws_bytes, stream
    ("meshy_logprob_bwd", (FAKE, 1, 4, 8, 32, 8, FAKE, FAKE, FAKE, None, FAKE, 4096, None), ENULL, "required"),
    ("meshy_logprob_bwd", (FAKE, 1, 4, 8, 32, 8, FAKE, FAKE, FAKE, FAKE, FAKE, 8, None), ESPACE, "workspace"),
    # logits, rows, T, V, sb, st, labels, lse, grad_logp, grad, stream: one row past the static scratch's
    # 262144 (refused before any HIP call)
    ("meshy_logprob_bwd_noalloc", (FAKE, 1, 262145, 8, 262145 * 8, 8, FAKE, FAKE, FAKE, FAKE, None), ESPACE,
     "static scratch"),
    ("meshy_logprob_bwd_noalloc", (FAKE, 1, 4, 8, 32, 8, FAKE, FAKE, FAKE, None, None), ENULL, "required"),
    ("meshy_gather_logprobs_bwd", (FAKE, 1, 4, 8, 32, 8, FAKE, 300, FAKE, FAKE, FAKE, FAKE, 4096, None), EINVAL,
     "n_ids"),
    # logits, rows, T, V, sb, st, k, ids, logprobs, lse, stream
    ("meshy_topk_logprobs", (FAKE, 1, 4, 100, 400, 100, 65, FAKE, FAKE, None, None), EINVAL, "k must be"),
    ("meshy_topk_logprobs", (FAKE, 1, 4, 5, 20, 5, 8, FAKE, FAKE, None, None), EINVAL, "k must be"),
    ("meshy_topk_logprobs", (FAKE, 1, 4, 100, 400, 100, 0, FAKE, FAKE, None, None), EINVAL, "k must be"),
    ("meshy_topk_logprobs", (FAKE, 1, 4, 100, 400, 100, 8, None, FAKE, None, None), ENULL, "required"),
    ("meshy_forward_kl_topk", (FAKE, FAKE, 4, 0, 0, 0.0, 0, 0.0, FAKE, None), EINVAL, "bad sizes"),
    ("meshy_forward_kl_topk", (None, FAKE, 4, 3, 0, 0.0, 0, 0.0, FAKE, None), ENULL, "NULL"),
    ("meshy_per_sequence_mean", (None, FAKE, FAKE, 3, FAKE, None), ENULL, "NULL"),
    ("meshy_per_sequence_mean", (FAKE, FAKE, FAKE, -1, FAKE, None), EINVAL, "n_docs"),
    ("meshy_clipped_value_error", (FAKE, FAKE, None, 1, 0.2, 10, FAKE, None), ENULL, "NULL"),
    ("meshy_clipped_value_error", (FAKE, FAKE, None, 0, 0.2, -1, FAKE, None), EINVAL, "negative"),
    # values, targets, old, has_clip, clip, n, grad_out, grad_stride, grad_values, stream
    ("meshy_clipped_value_error_bwd", (FAKE, FAKE, None, 0, 0.2, 10, FAKE, 2, FAKE, None), EINVAL, "grad_stride"),
    ("meshy_clipped_value_error_bwd", (FAKE, FAKE, None, 1, 0.2, 10, FAKE, 0, FAKE, None), ENULL, "NULL"),
    ("meshy_critic_accumulate", (FAKE, 0, FAKE, FAKE, 4, 16, FAKE, FAKE, FAKE, 8, None), ESPACE, "workspace"),
    ("meshy_critic_accumulate", (FAKE, 0, FAKE, FAKE, -4, 16, FAKE, FAKE, FAKE, 4096, None), EINVAL, "bad shape"),
    ("meshy_ragged_token_stats", (FAKE, None, FAKE, None, 4, FAKE, FAKE, None, None, FAKE, 4096, None), ENULL,
     "out_off"),
    ("meshy_ragged_token_stats", (FAKE, FAKE, FAKE, None, 4, FAKE, FAKE, FAKE, None, FAKE, 4096, None), ENULL,
     "lp_offsets"),
    ("meshy_ragged_token_stats", (FAKE, None, FAKE, None, 4, FAKE, FAKE, FAKE, None, FAKE, 8, None), ESPACE,
     "workspace"),
    # rewards, n_rewards, group_offsets, n_groups, adv, stream
    ("meshy_grpo_advantage", (FAKE, 8, FAKE, -1, FAKE, None), EINVAL, "negative"),
    ("meshy_grpo_advantage", (FAKE, -8, FAKE, 1, FAKE, None), EINVAL, "negative"),
    ("meshy_grpo_advantage", (None, 8, FAKE, 3, FAKE, None), ENULL, "NULL"),
    # values, bf16, returns, mask, rows, S, sums, row_value, workspace, bytes, stream
    ("meshy_critic_window_sums", (FAKE, 0, FAKE, FAKE, -1, 8, FAKE, FAKE, FAKE, 4096, None), EINVAL, "bad shape"),
    ("meshy_critic_window_sums", (FAKE, 0, None, FAKE, 2, 8, FAKE, FAKE, FAKE, 4096, None), ENULL, "NULL"),
    ("meshy_critic_window_sums", (FAKE, 0, FAKE, FAKE, 64, 8, FAKE, FAKE, FAKE, 8, None), ESPACE, "workspace"),
    # row_value, row_reward, group_ids, n, threshold, out, workspace, bytes, stream
    ("meshy_group_gauges", (FAKE, FAKE, FAKE, -3, 0.5, FAKE, FAKE, 4096, None), EINVAL, "bad size"),
    ("meshy_group_gauges", (FAKE, None, FAKE, 3, 0.5, FAKE, FAKE, 4096, None), ENULL, "NULL"),
    ("meshy_group_gauges", (FAKE, FAKE, FAKE, 300, 0.5, FAKE, FAKE, 8, None), ESPACE, "workspace"),
    # out, rows, cols, row_stride, seed, scale, stream
    ("meshy_synth_bf16", (FAKE, 4, 8, 7, 1, 2.0, None), EINVAL, "bad shape"),
    ("meshy_synth_bf16", (FAKE, 4, 8, 8, 1, -1.0, None), EINVAL, "bad scale"),
    ("meshy_synth_bf16", (None, 4, 8, 8, 1, 2.0, None), ENULL, "NULL"),
    # out, row_ids, n_rows, cols, seed, scale (host)
    ("meshy_synth_bf16_rows_host", (FAKE, None, 2, 8, 1, 2.0), ENULL, "NULL"),
    ("meshy_synth_bf16_rows_host", (FAKE, FAKE, -2, 8, 1, 2.0), EINVAL, "bad shape"),
    # raw_rewards, n_rewards, group_offsets, n_groups, tolerance, flags, stream
    ("meshy_zero_variance_groups", (FAKE, 8, FAKE, -1, 1e-8, FAKE, None), EINVAL, "negative"),
    ("meshy_zero_variance_groups", (None, 8, FAKE, 2, 1e-8, FAKE, None), ENULL, "NULL"),
    ("meshy_zero_variance_groups", (FAKE, 8, FAKE, 2, 1e-8, None, None), ENULL, "NULL"),
    ("meshy_zero_variance_groups_host", (FAKE, -1, FAKE, 2, 1e-8, FAKE), EINVAL, "negative"),
    ("meshy_grpo_advantage_host", (FAKE, 8, FAKE, -1, FAKE), EINVAL, "negative"),
    ("meshy_grpo_advantage_host", (FAKE, 8, None, 2, FAKE), ENULL, "NULL"),
    ("meshy_zero_variance_groups_host", (FAKE, 8, None, 2, 1e-8, FAKE), ENULL, "NULL"),
    ("meshy_segment_offsets", (FAKE, 10, 0, FAKE, None, None), EINVAL, "bad sizes"),
    ("meshy_doc_order", (FAKE, -1, 4, FAKE, FAKE, FAKE, 1 << 20, None), EINVAL, "bad sizes"),
    ("meshy_doc_order", (FAKE, 10, 0, FAKE, FAKE, FAKE, 1 << 20, None), EINVAL, "bad sizes"),
    ("meshy_doc_order", (FAKE, 1 << 31, 4, FAKE, FAKE, FAKE, 1 << 20, None), EINVAL, "too many tokens"),
    ("meshy_doc_order", (None, 10, 4, FAKE, FAKE, FAKE, 1 << 20, None), ENULL, "required"),
    ("meshy_doc_order", (FAKE, 10, 4, FAKE, None, FAKE, 1 << 20, None), ENULL, "required"),
    ("meshy_stream_read", (FAKE, 4, 17, FAKE, None), EINVAL, "bad shape"),
    ("meshy_stream_read", (FAKE + 4, 4, 32, FAKE, None), EALIGN, "misaligned"),
])
def test_entry_point_rejects(name, args, code, text):
    rc, msg = _call(name, *args)
    assert rc == code, (rc, msg)
    assert text in msg, msg


@pytest.mark.parametrize("name,args", [
    # logits, rows, T, V, stride_b, stride_t, labels, logp, entropy, lse, stream
    ("meshy_logprob_entropy_fwd", (None, 1, 0, 8, 0, 8, None, None, None, None, None)),
    ("meshy_logprob_entropy_fwd", (None, 0, 5, 8, 40, 8, None, None, None, None, None)),
    ("meshy_gather_logprobs_fwd", (None, 1, 0, 8, 0, 8, None, 3, None, None, None)),
    ("meshy_logprob_bwd", (None, 1, 0, 8, 0, 8, None, None, None, None, None, 0, None)),
    ("meshy_logprob_bwd_noalloc", (None, 1, 0, 8, 0, 8, None, None, None, None, None)),
    ("meshy_gather_logprobs_bwd", (None, 1, 0, 8, 0, 8, None, 9, None, None, None, None, 0, None)),
    ("meshy_topk_logprobs", (None, 1, 0, 100, 0, 100, 8, None, None, None, None)),
    ("meshy_clipped_value_error", (None, None, None, 1, 0.2, 0, None, None)),
    ("meshy_whiten_apply", (None, None, 0, None, None)),
])
def test_empty_calls_accept_null_arrays(name, args):
    """An empty tensor has no storage: with nothing to read or write, every
    entry point returns success for NULL arrays (before any device call)."""
    rc, msg = _call(name, *args)
    assert rc == 0, (rc, msg)


def test_struct_entry_points_reject():
    lib = _lib.load()
    a = _lib.DistillArgs()
    a.k = 0
    assert lib.meshy_distill_loss_fwd(ctypes.byref(a), FAKE, None, None) == EINVAL
    a.k = 8
    a.n_tokens = 16
    assert lib.meshy_distill_loss_fwd(ctypes.byref(a), FAKE, None, None) == ENULL  # student missing
    a.student = a.teacher = a.mask = a.seg_offsets = a.doc_ids = FAKE
    a.workspace, a.workspace_bytes = FAKE, 1
    assert lib.meshy_distill_loss_fwd(ctypes.byref(a), FAKE, None, None) == ESPACE
    assert b"workspace" in lib.meshy_last_error()
    assert lib.meshy_distill_loss_bwd(ctypes.byref(a), None, FAKE, FAKE, None) == ENULL
    p = _lib.PackArgs()
    p.n_micro, p.layout, p.tokens_elem_bytes = 1, 7, 4
    assert lib.meshy_pack_micro_batches(ctypes.byref(p), None) == EINVAL
    p.layout, p.teacher_k = _lib.MESHY_LAYOUT_PACKED, -1
    p.micro_seq_len = p.micro_out_off = p.micro_doc_start = FAKE
    p.input_ids = p.labels = p.positions = p.mask_out = p.doc_ids = p.cu_seqlens = FAKE
    p.max_micro_elems = 16
    assert lib.meshy_pack_micro_batches(ctypes.byref(p), None) == EINVAL
    assert b"teacher_k" in lib.meshy_last_error()
    p.teacher_k, p.teacher_ids_elem_bytes = 0, 2
    assert lib.meshy_pack_micro_batches(ctypes.byref(p), None) == EINVAL
    assert b"int32 or int64" in lib.meshy_last_error()
    p.teacher_ids_elem_bytes = 0
    g = _lib.PpoArgs()
    g.n_tokens = -1
    assert lib.meshy_ppo_loss_fwd(ctypes.byref(g), FAKE, None, None) == EINVAL
    g.n_tokens, g.n_docs = 16, 1 << 31
    g.new_lp = g.old_lp = g.mask = g.adv = g.seg_offsets = g.doc_ids = FAKE
    assert lib.meshy_ppo_loss_fwd(ctypes.byref(g), FAKE, None, None) == EINVAL
    assert b"too many documents" in lib.meshy_last_error()
    e = _lib.GaeArgs()
    e.rewards = e.mask = e.doc_ids = e.values = e.adv = FAKE
    e.rows, e.S, e.n_docs, e.gamma, e.alpha = 1, 100, 1, 1.0, 0.0
    assert lib.meshy_gae(ctypes.byref(e), None) == EINVAL
    assert b"alpha" in lib.meshy_last_error()
    e.alpha = 1.0
    e.workspace, e.workspace_bytes = FAKE, lib.meshy_gae_workspace_size(1, 100, 1) - 1
    assert lib.meshy_gae(ctypes.byref(e), None) == ESPACE
    e.adv, e.values = FAKE, None
    assert lib.meshy_gae(ctypes.byref(e), None) == ENULL


def test_workspace_sizes_are_consistent():
    lib = _lib.load()
    assert lib.meshy_logprob_bwd_workspace_size(1000) >= 8 * 1000
    assert lib.meshy_logprob_bwd_workspace_size(-1) == 0
    assert lib.meshy_distill_workspace_size(10_000, 12) >= 4 * 2 * (40 + 13)
    assert lib.meshy_critic_accumulate_workspace_size(7) >= 7 * 5 * 8
    assert lib.meshy_ragged_token_stats_workspace_size(9) >= 9 * 8


def test_autograd_module_checks_its_arguments():
    """The native autograd module loads beside the library and refuses, before
    any device work, host tensors and a capsule of the other loss."""
    import torch

    ag = _lib.autograd()
    z = torch.zeros(3)
    with pytest.raises(ValueError, match="run on the GPU"):
        ag.ppo_inputs(z, z, None, None, z, None, z.long(), z.long(), 3, 1, 1, 3, 0.2, 0.28, 0.5, 5.0, 0.0,
                      False, False, True, False, 1)
    with pytest.raises(ValueError, match="run on the GPU"):
        ag.distill_inputs(z, z, None, z.long(), z.long(), 1, 3, 1, 1, 3, None, None, True)
    with pytest.raises(TypeError, match="must be a tensor"):
        ag.distill_inputs([0.0], z, None, z.long(), z.long(), 1, 3, 1, 1, 3, None, None, True)
    with pytest.raises(TypeError, match="ppo_inputs capsule"):
        ag.ppo_loss(z, object())
    with pytest.raises(TypeError, match="distill_inputs capsule"):
        ag.args_bytes(object())
    with pytest.raises(ValueError, match="device tensor"):
        ag.clipped_value_error(z, z, None, None)

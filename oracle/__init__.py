"""CPU oracle for the ragged-batch path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithms that the HIP
kernels of ``meshy_amd`` replace.  It exists to check the product, never to
be the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the expected side of a comparison or
as the timed CPU baseline.  Nothing in ``meshy_amd`` imports it.

Modules and what pins each one (the checks live in ``tests/test_oracle_*.py``):

    plan     build_plan & co. (plan.py:141-324)      reference known answers
                                                      (test_dynamic_batching.py,
                                                      test_critic_batching.py),
                                                      golden plans written by
                                                      tests/golden/make_plan_vectors.py,
                                                      brute-force invariants
    batch    build_micro_batch (batch.py:84-243)      reference known answers
                                                      (test_dynamic_batching.py:240-316)
    logprob  _chunk_logprobs / _chunk_entropy         torch log_softmax/gather in
             (trainer.py:414-449)                     fp64, closed forms (uniform
                                                      logits -> ln V, one-hot -> 0)
    grpo     grpo_advantage (rollout.py:88-97)        test_rollout_advantage.py:13-18,
                                                      closed forms (G=1, all-equal)
    ppo      _ppo_clip_loss, _reduce_mini_metrics     test_ppo_diagnostics.py:58-95,
             (trainer.py:705-848, 1020-1047)          test_vapo_alignment.py:116-149,
                                                      torch autograd for the gradient
    gae      compute_vapo_gae, compute_returns        closed forms (V=0 terminal
             (critic/gae.py:70-93, 162-205, 208-293)  reward -> lambda^k R; lambda=0 ->
                                                      delta; returns -> R broadcast),
                                                      brute force on tiny inputs
    vapo     whiten_advantages (vapo.py:6-32)         test_vapo_alignment.py:24-46
    topk     teacher_topk, gather_logprobs,           test_opd_loss.py:13-49, brute-force
             forward_kl_topk (topk_loss.py:20-80)     (value, index) sort, closed-form KL
    opd      layout_teacher_topk, split_teacher_topk, test_opd_batch.py:42-75, closed
             _distill_loss, _reduce_mini_metrics      forms (equal distributions -> 0,
             (opd.py:39-251)                          ln 2 per token), torch autograd
    critic   advantages_to_per_sequence,              closed forms, torch autograd for
             Accumulator.update, clipped_value_error  the clipped value error
             (critic/gae.py:296-312, critic/metrics.py:238-275, vapo.py:35-41)
    rollout_metrics  _rollout_metrics                 test_rollout_metrics.py:51-106
             (metrics.py:72-322)
"""

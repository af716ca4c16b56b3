"""meshy_amd: MI355X-native ragged-batch path of OpenBMB/Meshy.

Drop-in replacements, with the reference's call surface, for

* the token-budget planner      ``meshy_amd.plan``      (plan.py)
* micro-batch materialisation   ``meshy_amd.batch``     (batch.py)
* fused logprob + entropy       ``meshy_amd.logprob``   (trainer.py:414-527)
* GRPO advantages               ``meshy_amd.advantage`` (rollout.py:88-97)
* clipped PPO loss              ``meshy_amd.loss``      (trainer.py:705-1047)
* segment-aware GAE / returns   ``meshy_amd.gae``       (critic/gae.py)
* advantage whitening           ``meshy_amd.vapo``      (vapo.py:6-32)
* Student Top-K OPD kernels     ``meshy_amd.topk``      (topk_loss.py)
* OPD layout and loss           ``meshy_amd.opd``       (opd.py)
* critic-side reductions        ``meshy_amd.critic``    (critic/gae.py:296-312,
                                                         critic/metrics.py:220-275,
                                                         vapo.py:35-41)
* rollout statistics            ``meshy_amd.rollout_metrics`` (metrics.py:171-322)
* rollout -> trainer columns    ``meshy_amd.wire``      (transferqueue/adapter.py)
* the packed step end to end    ``meshy_amd.pipeline``  (one host-to-device copy)

All compute runs in libmeshy_amd.so (HIP for gfx950, C ABI in
include/meshy_amd.h); this package is the thin Python layer around it.
"""

from . import _lib

__all__ = ["_lib"]

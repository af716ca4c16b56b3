"""Write golden planner vectors from the reference planner.

The reference's own tests pin groupings on hand-made cases but not the exact
assignment (snake direction, first-fit order, filler placement) at the
benchmark sizes, so this script loads the reference's stdlib-only
meshy/backend/titan/plan.py by file path, in the build container only, and
records its output for the seeded 256-sample GRPO and 16-sequence long-context lengths, the long-context
edge lists and a sweep of layouts, DP sizes and budgets.  The vectors are data
(inputs and the expected plan); no reference code is kept.

    python tests/golden/make_plan_vectors.py /root/reference
"""

from __future__ import annotations

import importlib.util
import json
import os
import random
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from meshy_amd import workloads  # noqa: E402


def load_reference_planner(ref_root: str):
    path = os.path.join(ref_root, "meshy", "backend", "titan", "plan.py")
    spec = importlib.util.spec_from_file_location("reference_plan", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["reference_plan"] = mod
    spec.loader.exec_module(mod)
    return mod


def plan_to_json(plan):
    return {
        "local_indices": [list(x) for x in plan.local_indices],
        "per_rank": [
            [
                {
                    "micros": [[list(m.sample_idx), m.seq_len, list(m.doc_lens)] for m in mini.micros],
                    "n_docs_global": mini.n_docs_global,
                    "n_tokens_global": mini.n_tokens_global,
                    "tokens_per_rank": list(mini.tokens_per_rank),
                }
                for mini in minis
            ]
            for minis in plan.per_rank
        ],
    }


def cases():
    b0, _, _ = workloads.grpo_256_samples(0)
    lt0 = b0.loss_tokens(8192)
    base0 = dict(layout="packed", mini_batch_size=256, seq_len=8192, align=2048,
                 max_tokens_per_micro=8192, micro_batch_size=None)
    yield "grpo256", b0.lengths.tolist(), lt0.tolist(), 1, base0
    for align in (1, 64):
        yield f"grpo256_align{align}", b0.lengths.tolist(), lt0.tolist(), 1, dict(base0, align=align)
    yield "grpo256_mini64", b0.lengths.tolist(), lt0.tolist(), 1, dict(base0, mini_batch_size=64)
    yield "grpo256_dp4", b0.lengths.tolist(), lt0.tolist(), 4, dict(base0, mini_batch_size=32)
    yield "grpo256_padded", b0.lengths.tolist(), lt0.tolist(), 2, dict(
        base0, layout="padded", mini_batch_size=64)
    l3 = workloads.long_context_16_lengths(3).tolist()
    base3 = dict(layout="packed", mini_batch_size=16, seq_len=131072, align=2048,
                 max_tokens_per_micro=131072, micro_batch_size=None)
    yield "long16", l3, l3, 1, base3
    for k, edge in enumerate(workloads.LONG_CONTEXT_EDGE_LISTS):
        yield f"long_edge{k}", list(edge), list(edge), 1, dict(base3, mini_batch_size=len(edge))
    rng = random.Random(1234)
    for k in range(24):
        layout = rng.choice(["padded", "packed"])
        dp = rng.choice([1, 2, 4])
        n = dp * rng.randint(1, 12)
        align = rng.choice([1, 8, 64, 128])
        seq_len = align * rng.randint(4, 64)
        lengths = [rng.randint(0 if k % 5 == 0 else 1, seq_len + 300) for _ in range(n)]
        loss = [max(0, L - rng.randint(0, 5)) for L in lengths]
        budget = rng.choice([None, seq_len, 2 * seq_len, align * 3]) if layout == "padded" else rng.choice(
            [seq_len, 2 * seq_len, align * 3])
        mbs = rng.choice([1, 2, 3]) if budget is None else rng.choice([None, 2])
        cfg = dict(layout=layout, mini_batch_size=rng.randint(1, max(1, n // dp)), seq_len=seq_len,
                   align=align, max_tokens_per_micro=budget, micro_batch_size=mbs)
        yield f"random{k}", lengths, loss, dp, cfg


def main(ref_root: str) -> None:
    ref = load_reference_planner(ref_root)
    out = []
    for name, lengths, loss, dp, cfg in cases():
        plan = ref.build_plan(lengths, loss, dp, ref.PlannerConfig(**cfg))
        out.append({"name": name, "lengths": lengths, "loss_tokens": loss, "dp_size": dp,
                    "cfg": cfg, "plan": plan_to_json(plan)})
    path = os.path.join(HERE, "plan_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {len(out)} cases to {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

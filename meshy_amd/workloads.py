"""Seeded synthetic workloads of the benchmarks and full-size tests (numpy, host side).

Lognormal lengths with "mean m, sigma s" use mu = ln m - s^2 / 2, so the mean
of the distribution is m; values are rounded to integers and clipped.  Every
generator takes a seed and is reproducible on any host.

    grpo_256_samples         pack + GRPO: 256 samples in 32 groups of 8, prompt U{64..256},
                             response lognormal(600, 0.8) clipped [1, 2048], budget 8192
    ppo_512_docs             PPO loss: 512 docs, response lognormal(4000, 0.8) clipped [16, 8192]
    long_context_16_lengths  long context: 16 sequences U{8192..131072}, budget 131072
    gae_1024_docs            GAE: 1024 docs, response lognormal(6000, 0.8) clipped [32, 32768]
    synth_logits             bf16 logits N(0, scale^2) from the counter-based Box-Muller
                             generator (meshy_synth_bf16), filled on the device;
                             synth_logit_rows regenerates any of their rows on the host, bit
                             for bit
"""

from __future__ import annotations

import math

import numpy as np

VOCAB = 151936


def lognormal_lengths(rng: np.random.Generator, n: int, mean: float, sigma: float, lo: int,
                      hi: int) -> np.ndarray:
    mu = math.log(mean) - sigma * sigma / 2.0
    x = rng.lognormal(mu, sigma, n)
    return np.clip(np.rint(x), lo, hi).astype(np.int64)


class RaggedBatch:
    """Samples as flat host arrays: sample i is [offsets[i], offsets[i+1])."""

    def __init__(self, prompt: np.ndarray, response: np.ndarray, rng: np.random.Generator,
                 vocab: int = VOCAB, with_tokens: bool = True) -> None:
        self.prompt = prompt.astype(np.int64)
        self.response = response.astype(np.int64)
        self.lengths = self.prompt + self.response
        self.offsets = np.zeros(len(self.lengths) + 1, np.int64)
        np.cumsum(self.lengths, out=self.offsets[1:])
        total = int(self.offsets[-1])
        self.total = total
        pos = np.arange(total, dtype=np.int64) - np.repeat(self.offsets[:-1], self.lengths)
        self.mask = (pos >= np.repeat(self.prompt, self.lengths)).astype(np.float32)
        if with_tokens:
            self.tokens = rng.integers(0, vocab, total, dtype=np.int32)
            self.logprobs = (-rng.uniform(0.0, 2.0, total)).astype(np.float32)
        else:
            self.tokens = None
            self.logprobs = None

    def loss_tokens(self, seq_len: int) -> np.ndarray:
        """#(mask[1:L] > 0) with L = min(length, seq_len) (trainer.py:577-588)."""
        L = np.minimum(self.lengths, seq_len)
        out = np.zeros(len(L), np.int64)
        for i, (o, n) in enumerate(zip(self.offsets[:-1], L)):
            if n > 1:
                out[i] = int(np.count_nonzero(self.mask[o + 1:o + n] > 0))
        return out

    def sample_dicts(self, rewards=None, advantages=None):
        """The samples as dicts of CPU torch tensors, as the trainer receives them."""
        import torch

        out = []
        for i in range(len(self.lengths)):
            a, b = int(self.offsets[i]), int(self.offsets[i + 1])
            d = {
                "tokens": torch.from_numpy(self.tokens[a:b].astype(np.int64)),
                "mask_assistant": torch.from_numpy(self.mask[a:b].copy()),
                "logprobs": torch.from_numpy(self.logprobs[a:b].copy()),
            }
            if rewards is not None:
                d["reward"] = torch.tensor(float(rewards[i]))
            if advantages is not None:
                d["advantage"] = torch.tensor(float(advantages[i]))
            out.append(d)
        return out


def grpo_256_samples(seed: int = 0):
    rng = np.random.default_rng(seed)
    n_groups, group = 32, 8
    n = n_groups * group
    prompt = rng.integers(64, 257, n)
    response = lognormal_lengths(rng, n, 600.0, 0.8, 1, 2048)
    batch = RaggedBatch(prompt, response, rng)
    rewards = (rng.random(n) < 0.4).astype(np.float32)
    group_offsets = np.arange(0, n + 1, group, dtype=np.int64)
    return batch, rewards, group_offsets


def ppo_512_docs(seed: int = 2):
    rng = np.random.default_rng(seed)
    n_docs, group = 512, 8
    prompt = rng.integers(64, 257, n_docs)
    response = lognormal_lengths(rng, n_docs, 4000.0, 0.8, 16, 8192)
    batch = RaggedBatch(prompt, response, rng, with_tokens=False)
    total = batch.total
    old = rng.uniform(-8.0, 0.0, total).astype(np.float32)
    new = (old + rng.normal(0.0, 0.05, total)).astype(np.float32)
    rewards = (rng.random(n_docs) < 0.4).astype(np.float32)
    group_offsets = np.arange(0, n_docs + 1, group, dtype=np.int64)
    return batch, old, new, rewards, group_offsets


def long_context_16_lengths(seed: int = 3) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(8192, 131072 + 1, 16).astype(np.int64)


LONG_CONTEXT_EDGE_LISTS = (
    [131072],
    [65536, 65536],
    [131071, 1],
    [100000, 31073],
    [131072, 1],
)


def gae_1024_docs(seed: int = 4):
    rng = np.random.default_rng(seed)
    n_docs = 1024
    prompt = rng.integers(64, 257, n_docs)
    response = lognormal_lengths(rng, n_docs, 6000.0, 0.8, 32, 32768)
    batch = RaggedBatch(prompt, response, rng, with_tokens=False)
    values = rng.standard_normal(batch.total).astype(np.float32)
    terminal = (rng.random(n_docs) < 0.5).astype(np.float32)
    return batch, values, terminal


def synth_logits(rows: int, cols: int, seed: int, scale: float = 2.0, device=None):
    """A [rows, cols] bf16 tensor of counter-based synthetic logits drawn from
    N(0, scale^2) (a Box-Muller pair per hash), filled on the HIP device."""
    import torch

    from . import _lib

    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(rows, cols, dtype=torch.bfloat16, device=dev)
    _lib.require_gpu(out)
    rc = _lib.load().meshy_synth_bf16(out.data_ptr(), rows, cols, cols, int(seed) & (2**64 - 1), float(scale),
                                      _lib.stream_of(dev))
    _lib.check(rc, "meshy_synth_bf16")
    return out


def synth_logit_rows(row_ids, cols: int, seed: int, scale: float = 2.0):
    """Rows ``row_ids`` of ``synth_logits(*, cols, seed, scale)``, regenerated
    on the host (CPU bf16 tensor [len(row_ids), cols])."""
    import torch

    from . import _lib

    ids = torch.as_tensor(row_ids, dtype=torch.int64).reshape(-1).contiguous()
    out = torch.empty(ids.numel(), cols, dtype=torch.bfloat16)
    rc = _lib.load().meshy_synth_bf16_rows_host(out.data_ptr(), ids.data_ptr(), ids.numel(), cols,
                                                int(seed) & (2**64 - 1), float(scale))
    _lib.check(rc, "meshy_synth_bf16_rows_host")
    return out

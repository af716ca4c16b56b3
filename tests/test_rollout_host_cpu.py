"""Host side of ``rollout_metrics`` over a sample list: the one-pass field
lists, the stacked scalars and the concatenated jagged columns give what the
per-sample path gives (metrics.py:171-322 reads each sample's fields), for
uniform inputs (one stack / one concatenation) and for the inputs that take the
per-sample path (None entries, mixed dtypes and shapes, 2-D entries, Python
numbers)."""

from __future__ import annotations

from types import SimpleNamespace as NS

import torch

from meshy_amd import rollout_metrics as R
from meshy_amd.wire import jagged_parts


def _per_sample_scalars(values):
    out = []
    for v in values:
        if v is None:
            continue
        out += [float(x) for x in (v.reshape(-1).tolist() if torch.is_tensor(v) else [v])]
    return out


def _per_sample_flat(values):
    return jagged_parts([torch.zeros(0) if v is None else R._as_float(v) for v in values])


def test_field_lists_from_dicts_and_objects():
    samples = [{"reward": torch.tensor(1.0), "tokens": torch.arange(3)},
               NS(reward=torch.tensor(0.0), tokens=torch.arange(2), masks=torch.ones(2)),
               {"advantage": 0.5}]
    per = R._per_sample(samples)
    assert set(per) == set(R._FIELDS)
    assert [None if v is None else float(v) for v in per["reward"]] == [1.0, 0.0, None]
    assert per["advantage"] == [None, None, 0.5]
    assert per["masks"][1] is samples[1].masks and per["masks"][0] is None


def test_scalars_stack_and_fallback_agree():
    g = torch.Generator().manual_seed(0)
    cases = [
        [torch.rand((), generator=g) for _ in range(37)],                    # one stack
        [torch.tensor(i % 3 == 0) for i in range(10)],                       # bool
        [torch.tensor(i, dtype=torch.int64) for i in range(10)],             # int64
        [torch.rand(2, generator=g) for _ in range(5)],                      # equal shapes: flattened in order
        [torch.tensor(1.0), None, torch.tensor(2.0, dtype=torch.float64)],   # mixed dtypes
        [torch.tensor(1.0), torch.tensor([2.0, 3.0]), None, 4.0],            # mixed shapes, a number
        [None, None],
    ]
    for values in cases:
        assert R._scalars({"reward": values}, None, "reward") == _per_sample_scalars(values)


def test_flat_columns_concatenation_and_fallback_agree():
    g = torch.Generator().manual_seed(1)
    cases = [
        [torch.rand(int(n), generator=g) for n in torch.randint(0, 50, (64,), generator=g)],  # one cat
        [torch.ones(3, dtype=torch.bool), None, torch.zeros(2, dtype=torch.bool)],            # bool, None
        [torch.ones(3), None, torch.zeros(2, dtype=torch.float64), torch.ones(1, 2)],         # mixed
        [torch.arange(4), torch.arange(0)],                                                   # int64, empty
        [[1.0, 0.0], torch.ones(2)],                                                          # a list
    ]
    for values in cases:
        a, ao = R._flat(values)
        b, bo = _per_sample_flat(values)
        assert torch.equal(ao, bo)
        assert torch.equal(a.to(torch.float32), b)

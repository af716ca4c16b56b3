"""The native flatten of the rollout wire's per-token columns (meshy_amd._pyio)
against numpy's own conversion of the same Python objects.

``wire.flatten_sequences`` feeds ``rollout_group_to_columns``, the one-pass form
of ``sample_to_tensordict`` + ``samples_to_td`` (rollout.py:118-153,
adapter.py:96-132).  numpy's ``fromiter`` over the chained sequences is the
pin: every value the native pass accepts must come out with numpy's bits, and
every value it declines must give numpy's result or numpy's error.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

from meshy_amd import _lib, wire


def _numpy_flat(seqs, npdt):
    n = sum(len(s) for s in seqs)
    return np.fromiter(itertools.chain.from_iterable(seqs), npdt, n)


def _check(seqs, dtype):
    npdt = np.int64 if dtype == torch.int64 else np.float32
    flat, off = wire.flatten_sequences(seqs, dtype)
    assert flat.dtype == npdt and off.dtype == np.int64
    assert off.tolist() == [0] + list(itertools.accumulate(len(s) for s in seqs))
    ref = _numpy_flat(seqs, npdt)
    assert flat.tobytes() == ref.tobytes()
    return flat


def test_int64_columns_match_numpy():
    rng = np.random.default_rng(0)
    seqs = [rng.integers(-2**62, 2**62, size=int(L)).tolist() for L in rng.integers(0, 300, size=40)]
    seqs += [[], [2**63 - 1, -2**63, 0, -1, 1], [True, False, 7], (3, 4, 5), []]
    _check(seqs, torch.int64)


@pytest.mark.filterwarnings("ignore:overflow encountered in cast:RuntimeWarning")
def test_float32_columns_match_numpy():
    rng = np.random.default_rng(1)
    seqs = [rng.normal(0, 3, size=int(L)).tolist() for L in rng.integers(0, 300, size=40)]
    specials = [0.0, -0.0, math.inf, -math.inf, 1e-45, 1.4e-45, 7e-46, 3.4028235e38, 3.4028236e38,
                1e39, -1e39, 1.0000000596046448, 1.0000001788139343, 2.0 ** -149, 2.0 ** -150]
    ints = [0, 1, -1, 2**24 + 1, 2**24 + 3, 2**53 + 1, -(2**53) - 3, 2**62 + 2**38 + 1, 2**63 - 1, -2**63]
    seqs += [specials, ints, [True, False, 0.5, 3], tuple(specials[:4]), []]
    _check(seqs, torch.float32)
    # NaN compares by bits only when it is the same NaN: numpy and C both keep
    # the double's quiet NaN payload in the float.
    flat, _ = wire.flatten_sequences([[math.nan, 1.0]], torch.float32)
    assert math.isnan(flat[0]) and flat[1] == 1.0


def test_declined_values_fall_back_to_numpy():
    # numpy arrays, tensors and numpy scalars are not lists of Python numbers.
    arr = [np.arange(5), np.arange(3, dtype=np.int32)]
    _check(arr, torch.int64)
    _check([[np.float64(0.25), np.float32(1.5)], [1.0]], torch.float32)
    _check([torch.arange(4).tolist(), torch.arange(2)], torch.int64)
    # Ints beyond int64: numpy's float conversion, numpy's overflow error.
    _check([[2**70, -(2**80)], [1]], torch.float32)
    with pytest.raises(OverflowError):
        wire.flatten_sequences([[1, 2**64]], torch.int64)
    with pytest.raises((ValueError, TypeError)):
        wire.flatten_sequences([[1, "x"]], torch.float32)


def test_empty_inputs():
    flat, off = wire.flatten_sequences([], torch.int64)
    assert flat.size == 0 and off.tolist() == [0]
    flat, off = wire.flatten_sequences([[], ()], torch.float32)
    assert flat.size == 0 and off.tolist() == [0, 0, 0]


def test_native_argument_checks():
    pyio = _lib.pyio()
    with pytest.raises(ValueError, match="len\\(seqs\\) \\+ 1"):
        pyio.seq_offsets([[1], [2]], np.empty(2, np.int64))
    assert pyio.seq_offsets([[1], np.arange(2)], np.empty(3, np.int64)) is None
    assert pyio.seq_offsets(([1], [2, 3]), np.empty(3, np.int64)) == 3
    with pytest.raises(ValueError, match="kind"):
        pyio.flatten_into([[1]], np.empty(1, np.int64), "d")
    with pytest.raises(ValueError, match="whole number"):
        pyio.flatten_into([[1]], np.empty(3, np.uint8), "f")
    # A buffer of the wrong length is declined, not overrun.
    assert pyio.flatten_into([[1, 2, 3]], np.empty(2, np.int64), "q") is False
    assert pyio.flatten_into([[1, 2]], np.empty(3, np.int64), "q") is False
    with pytest.raises(TypeError):
        pyio.flatten_into([[1]], b"\0" * 8, "q")  # read-only buffer


def test_group_columns_use_the_native_pass():
    """rollout_group_to_columns over list samples equals the per-sample path."""
    from types import SimpleNamespace as NS

    rng = np.random.default_rng(2)
    group = []
    for k, L in enumerate([5, 0, 130, 1, 64]):
        group.append(NS(tokens=rng.integers(0, 151936, L).tolist(), logprobs=rng.normal(-1, 1, L).tolist(),
                        masks=rng.integers(0, 2, L).tolist(), reward=float(k % 2), advantage=None if k == 1 else 0.25,
                        truncated=k == 2, repetition=False, mixed_version=k == 4))
    fields = list(wire.GRPO_TRAINER_FIELDS) + ["raw_reward", "positive_lm_weight"]
    fast = wire.rollout_group_to_columns(group, 5, fields)
    ref = wire.samples_to_columns([wire.sample_to_tensordict(s, 5) for s in group], fields)
    for f in fields:
        if wire.field_kind(f) == "nested":
            (fv, fo), (rv, ro) = wire.jagged_parts(fast[f]), wire.jagged_parts(ref[f])
            assert fv.dtype == rv.dtype and torch.equal(fv, rv) and torch.equal(fo, ro), f
        else:
            assert fast[f].dtype == ref[f].dtype and torch.equal(fast[f], ref[f]), f


@settings(max_examples=120, deadline=None)
@given(
    lengths=st.lists(st.integers(0, 40), min_size=0, max_size=30),
    kind=st.sampled_from(["int", "float", "mixed"]),
    dtype=st.sampled_from([torch.int64, torch.float32]),
    seed=st.integers(0, 2**31 - 1),
    use_tuples=st.booleans(),
)
def test_random_columns_match_numpy(lengths, kind, dtype, seed, use_tuples):
    """Random jagged columns of ints, floats, bools and mixes: the native pass
    (or its numpy fallback, for floats in an int64 column) equals numpy."""
    rng = np.random.default_rng(seed)

    def value():
        pick = kind if kind != "mixed" else rng.choice(["int", "float", "bool"])
        if pick == "int":
            return int(rng.integers(-2**40, 2**40))
        if pick == "float":
            return float(rng.normal(0, 1e3))
        return bool(rng.integers(0, 2))

    seqs = [[value() for _ in range(L)] for L in lengths]
    if use_tuples:
        seqs = [tuple(s) for s in seqs]
    npdt = np.int64 if dtype == torch.int64 else np.float32
    try:
        ref = _numpy_flat(seqs, npdt)
    except (TypeError, ValueError, OverflowError) as e:
        with pytest.raises(type(e)):
            wire.flatten_sequences(seqs, dtype)
        return
    flat, off = wire.flatten_sequences(seqs, dtype)
    assert flat.tobytes() == ref.tobytes()
    assert off.tolist() == [0] + list(itertools.accumulate(lengths))


def test_long_columns_split_over_threads_match_numpy():
    """Columns of more than 64 k values are converted by several threads, cut
    at sample boundaries by element count: lengths from 0 to 50 k, so that cuts
    fall on long and empty samples alike."""
    rng = np.random.default_rng(9)
    lengths = [0, 50_000, 1, 0, 30_000, 7, 45_000, 0, 0, 12_345, 3, 60_000, 0, 20_000]
    ints = [rng.integers(-2**62, 2**62, L).tolist() for L in lengths]
    floats = [rng.normal(0, 5, L).tolist() for L in lengths]
    _check(ints, torch.int64)
    _check(floats, torch.float32)
    # a declined value deep in a late run still sends the column to numpy
    bad = [list(x) for x in ints]
    bad[11][59_999] = np.int64(5)
    _check(bad, torch.int64)

"""The one-pass native staging of build_micro_batches (meshy_amd._stage.stage_micros)
on host memory: the regions it writes against the samples' columns and the
plan's tables, and the inputs it leaves to the general staging."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from meshy_amd import _lib
from meshy_amd.batch import _COMMON_REGIONS, _gather_fn
from meshy_amd.plan import MicroPlan


def _samples(lengths, seed, tok_dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i, L in enumerate(lengths):
        out.append({
            "tokens": torch.randint(0, 150000, (L,), generator=g).to(tok_dtype),
            "mask_assistant": (torch.rand(L, generator=g) > 0.3).float(),
            "logprobs": torch.randn(L, generator=g),
            "advantage": torch.tensor(float(i) - 2.5),
            "reward": float(i % 3) * 0.4,
            "positive_lm_weight": 0.25 * (i + 1),
        })
    return out


def _micros(lengths, seq_len=64):
    """Greedy packing of the samples into micros of ``seq_len`` tokens, the
    last document of a micro cut to fit, plus one filler micro."""
    micros, cur, lens, used = [], [], [], 0
    for i, L in enumerate(lengths):
        take = min(L, seq_len)
        if used + take > seq_len and cur:
            micros.append(MicroPlan(tuple(cur), seq_len, tuple(lens)))
            cur, lens, used = [], [], 0
        cur.append(i)
        lens.append(take)
        used += take
    if cur:
        micros.append(MicroPlan(tuple(cur), seq_len, tuple(lens)))
    micros.append(MicroPlan((), seq_len, ()))
    return micros


def _stage(samples, micros, packed=True, need_lp=True, capacity=1 << 20):
    buf = np.zeros(capacity, np.uint8)
    res = _lib.stage().stage_micros(samples, micros, packed, need_lp, buf.ctypes.data, capacity, _gather_fn())
    return res, buf


@pytest.mark.parametrize("tok_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("packed,need_lp", [(True, True), (False, False), (True, False)])
def test_regions_hold_the_columns_and_tables(tok_dtype, packed, need_lp):
    lengths = [5, 17, 40, 1, 64, 70, 9, 3]
    samples = _samples(lengths, 3, tok_dtype)
    micros = _micros(lengths)
    res, buf = _stage(samples, micros, packed, need_lp)
    assert res is not None and not isinstance(res, int)
    (size, bounds_b, n_s, total, tok64, nd, max_elems, max_docs, seq_b, rows_b, out_off_b, doc_start_b,
     used_r, need_r) = res
    bounds = np.frombuffer(bounds_b, np.int64).reshape(-1, 2)
    assert len(bounds) == len(_COMMON_REGIONS)
    assert tok64 == (tok_dtype == torch.int64)

    used_b, need_b, ds_b, dl_b, seq_t, nd_b, _ = _lib.stage().plan_tables(micros, len(samples))
    assert (used_r, need_r) == (used_b, need_b)
    used = np.frombuffer(used_b, np.int64)
    need = np.frombuffer(need_b, np.int64)
    assert n_s == len(used) and total == int(need.sum())
    doc_sample = np.frombuffer(ds_b, np.int32)
    n_docs = np.frombuffer(nd_b, np.int64)
    assert nd == len(doc_sample) == int(n_docs.sum())

    def region(name, dtype):
        i = [r[0] for r in _COMMON_REGIONS].index(name)
        lo, hi = bounds[i]
        assert lo % 256 == 0
        return buf[lo:hi].view(dtype)

    def cat(key, dtype):
        return np.concatenate([samples[int(u)][key][:int(L)].numpy().astype(dtype) for u, L in zip(used, need)])

    tok_np = np.int64 if tok64 else np.int32
    np.testing.assert_array_equal(region("tokens", tok_np), cat("tokens", tok_np))
    np.testing.assert_array_equal(region("mask", np.float32), cat("mask_assistant", np.float32))
    if need_lp:
        np.testing.assert_array_equal(region("logprobs", np.float32), cat("logprobs", np.float32))
    else:
        assert tuple(bounds[2]) == (-1, -1)
    adv = np.array([float(samples[int(u)]["advantage"]) for u in used], np.float32)
    np.testing.assert_array_equal(region("adv_samples", np.float32), adv)
    np.testing.assert_array_equal(region("s_off", np.int64), np.concatenate([[0], np.cumsum(need)]))
    seq = np.frombuffer(seq_t, np.int64)
    np.testing.assert_array_equal(region("seq", np.int64), seq)
    np.testing.assert_array_equal(np.frombuffer(seq_b, np.int64), seq)
    rows = np.ones(len(micros), np.int64) if packed else np.array([m.n_rows for m in micros], np.int64)
    np.testing.assert_array_equal(np.frombuffer(rows_b, np.int64), rows)
    out_off = np.concatenate([[0], np.cumsum(seq * rows)])
    np.testing.assert_array_equal(region("out_off", np.int64), out_off)
    np.testing.assert_array_equal(np.frombuffer(out_off_b, np.int64), out_off)
    doc_start = np.concatenate([[0], np.cumsum(n_docs)]).astype(np.int32)
    np.testing.assert_array_equal(region("doc_start", np.int32), doc_start)
    np.testing.assert_array_equal(np.frombuffer(doc_start_b, np.int32), doc_start)
    np.testing.assert_array_equal(region("doc_len", np.int64), np.frombuffer(dl_b, np.int64))
    np.testing.assert_array_equal(region("doc_sample", np.int32), doc_sample)
    # positive-LM weights of documents whose sample's reward is above 0.5
    pos = []
    for d in doc_sample:
        s = samples[int(used[d])]
        pos.append(s["positive_lm_weight"] if s["reward"] > 0.5 else 0.0)
    np.testing.assert_array_equal(region("pos_w", np.float32), np.array(pos, np.float32))
    assert max_elems == int((seq * rows).max()) and max_docs == int(n_docs.max())
    assert size == int(bounds[-1][0]) + (int(bounds[-1][1] - bounds[-1][0]) + 255) // 256 * 256


def test_small_capacity_returns_the_size_and_writes_nothing():
    lengths = [30, 40, 50]
    samples = _samples(lengths, 1)
    micros = _micros(lengths)
    full, _ = _stage(samples, micros)
    res, buf = _stage(samples, micros, capacity=512)
    assert res == full[0] > 512
    assert not buf.any()


def test_scalars_follow_the_staging_rules():
    """Missing or None scalars read 0; tensors read their first element."""
    samples = _samples([4, 4, 4], 2)
    del samples[0]["advantage"]
    samples[1]["advantage"] = None
    samples[2]["advantage"] = torch.tensor([1.5, 9.0])
    samples[2]["reward"] = torch.tensor(0.75)
    del samples[1]["positive_lm_weight"]
    micros = [MicroPlan((0, 1, 2), 16, (4, 4, 4))]
    res, buf = _stage(samples, micros)
    bounds = np.frombuffer(res[1], np.int64).reshape(-1, 2)
    lo, hi = bounds[3]
    np.testing.assert_array_equal(buf[lo:hi].view(np.float32), np.array([0.0, 0.0, 1.5], np.float32))
    lo, hi = bounds[10]
    np.testing.assert_array_equal(buf[lo:hi].view(np.float32), np.array([0.0, 0.0, 0.75], np.float32))


class _Mapping:
    """A sample that is a mapping but not a dict."""

    def __init__(self, d):
        self._d = d

    def __getitem__(self, k):
        return self._d[k]

    def __contains__(self, k):
        return k in self._d

    def get(self, k, default=None):
        return self._d.get(k, default)


def test_mapping_samples_stage_like_dicts():
    lengths = [7, 20, 33]
    samples = _samples(lengths, 4)
    micros = _micros(lengths)
    a, abuf = _stage(samples, micros)
    b, bbuf = _stage([_Mapping(s) for s in samples], micros)
    assert a[0] == b[0] and a[1] == b[1]
    for lo, hi in np.frombuffer(a[1], np.int64).reshape(-1, 2):
        if lo >= 0:
            np.testing.assert_array_equal(abuf[lo:hi], bbuf[lo:hi])


def _variant(kind):
    samples = _samples([6, 9, 12], 5)
    if kind == "per_token_adv":
        samples[1]["advantage_tokens"] = torch.ones(9)
    elif kind == "mixed_tokens":
        samples[2]["tokens"] = samples[2]["tokens"].int()
    elif kind == "list_tokens":
        samples[0]["tokens"] = samples[0]["tokens"].tolist()
    elif kind == "f64_mask":
        samples[1]["mask_assistant"] = samples[1]["mask_assistant"].double()
    elif kind == "strided_lp":
        samples[2]["logprobs"] = torch.randn(24)[::2]
    elif kind == "short_tokens":
        samples[1]["tokens"] = samples[1]["tokens"][:5]
    elif kind == "missing_mask":
        del samples[0]["mask_assistant"]
    elif kind == "bad_scalar":
        samples[0]["advantage"] = "x"
    elif kind == "uint8_tokens":
        samples[0]["tokens"] = samples[0]["tokens"].to(torch.uint8)
    return samples


@pytest.mark.parametrize("kind", ["per_token_adv", "mixed_tokens", "list_tokens", "f64_mask", "strided_lp",
                                  "short_tokens", "missing_mask", "bad_scalar", "uint8_tokens"])
def test_other_inputs_are_left_to_the_general_staging(kind):
    samples = _variant(kind)
    micros = [MicroPlan((0, 1, 2), 32, (6, 9, 12))]
    res, buf = _stage(samples, micros)
    assert res is None
    assert not buf.any()


def test_packed_overflow_is_left_to_the_general_staging():
    samples = _samples([20, 20], 6)
    micros = [MicroPlan((0, 1), 32, (20, 20))]
    assert _stage(samples, micros, packed=True)[0] is None
    assert _stage(samples, micros, packed=False)[0] is not None


def test_no_samples_stage_empty_int64_tokens():
    res, _ = _stage([], [MicroPlan((), 16, ())])
    assert res is not None
    size, bounds_b, n_s, total, tok64 = res[:5]
    assert (n_s, total, tok64) == (0, 0, 1)
    bounds = np.frombuffer(bounds_b, np.int64).reshape(-1, 2)
    assert tuple(bounds[0]) == (0, 0)


@pytest.mark.parametrize("packed", [True, False])
def test_int64_tokens_narrowed_to_int32(packed):
    """With the narrowing gather, int64 tokens land as int32 (the same values)
    and every other region is byte-equal to the staging without it."""
    from meshy_amd.batch import _gather_i32_fn

    lengths = [5, 17, 40, 1, 64, 70, 9, 3]
    samples = _samples(lengths, 4)
    samples[2]["tokens"][3] = 2**31 - 1  # the largest id that fits
    samples[5]["tokens"][0] = -(2**31)
    micros = _micros(lengths)
    wide, wbuf = _stage(samples, micros, packed, True)
    buf = np.zeros(1 << 20, np.uint8)
    res = _lib.stage().stage_micros(samples, micros, packed, True, buf.ctypes.data, buf.size, _gather_fn(),
                                    _gather_i32_fn())
    assert res is not None and not isinstance(res, int)
    assert res[4] == 0 and wide[4] == 1  # tokens staged as int32 / int64
    nb = np.frombuffer(res[1], np.int64).reshape(-1, 2)
    wb = np.frombuffer(wide[1], np.int64).reshape(-1, 2)
    lo, hi = nb[0]
    wlo, whi = wb[0]
    np.testing.assert_array_equal(buf[lo:hi].view(np.int32), wbuf[wlo:whi].view(np.int64).astype(np.int32))
    assert (hi - lo) * 2 == whi - wlo
    for r in range(1, len(_COMMON_REGIONS)):
        (a, b), (c, d) = nb[r], wb[r]
        assert (a < 0) == (c < 0)
        if a >= 0:
            np.testing.assert_array_equal(buf[a:b], wbuf[c:d])
    assert res[2:4] == wide[2:4] and res[5:] == wide[5:]


@pytest.mark.parametrize("bad", [2**31, -(2**31) - 1, 2**32 + 7])
def test_token_outside_int32_is_left_to_the_general_staging(bad):
    from meshy_amd.batch import _gather_i32_fn

    lengths = [5, 17, 40]
    samples = _samples(lengths, 5)
    samples[1]["tokens"][16] = bad
    buf = np.zeros(1 << 20, np.uint8)
    res = _lib.stage().stage_micros(samples, _micros(lengths), True, True, buf.ctypes.data, buf.size, _gather_fn(),
                                    _gather_i32_fn())
    assert res is None

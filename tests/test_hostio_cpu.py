"""The host gather (meshy_host_gather / meshy_amd.hostio.gather_into) against
torch.cat on the CPU: dtype conversion, empty, strided and 0-d parts, gathers
large enough for every pool thread, concurrent callers and a forked child."""

from __future__ import annotations

import ctypes
import multiprocessing as mp
import threading

import pytest
import torch

from meshy_amd import _lib
from meshy_amd.hostio import gather_into


def _parts(seed, n, hi, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    sizes = torch.randint(0, hi, (n,), generator=g).tolist()
    return [torch.randn(s, generator=g).to(dtype) for s in sizes]


@pytest.mark.parametrize("n,hi", [(1, 10), (7, 3), (300, 5000), (1024, 12000), (20000, 40)])
def test_matches_cat(n, hi):
    parts = _parts(n, n, hi)
    out = torch.empty(sum(p.numel() for p in parts))
    gather_into(parts, out)
    assert torch.equal(out, torch.cat(parts))


def test_converts_dtype_and_layout():
    g = torch.Generator().manual_seed(3)
    ints = torch.randint(0, 151936, (50, 7), generator=g)
    parts = [ints[:, 2],                                   # strided
             torch.tensor(5),                              # 0-d
             torch.arange(10, dtype=torch.int64),          # another dtype
             torch.zeros(0, dtype=torch.int32),            # empty
             torch.arange(6, dtype=torch.int32).reshape(2, 3),
             [1, 2, 3]]                                    # not a tensor
    out = torch.empty(50 + 1 + 10 + 0 + 6 + 3, dtype=torch.int32)
    gather_into(parts, out)
    ref = torch.cat([ints[:, 2].to(torch.int32), torch.tensor([5], dtype=torch.int32),
                     torch.arange(10, dtype=torch.int32), torch.arange(6, dtype=torch.int32),
                     torch.tensor([1, 2, 3], dtype=torch.int32)])
    assert torch.equal(out, ref)
    bf = [torch.randn(100, generator=g) for _ in range(3)]
    out = torch.empty(300, dtype=torch.bfloat16)
    gather_into(bf, out)
    assert torch.equal(out, torch.cat(bf).to(torch.bfloat16))


def test_large_gather_every_thread_count():
    parts = _parts(11, 64, 300_000)
    ref = torch.cat(parts)
    lib = _lib.load()
    ptrs = (ctypes.c_void_p * len(parts))(*[p.data_ptr() for p in parts])
    sizes = (ctypes.c_int64 * len(parts))(*[p.numel() * 4 for p in parts])
    for threads in (1, 2, 3, 16, 0):
        out = torch.full_like(ref, float("nan"))
        assert lib.meshy_host_gather(ptrs, sizes, len(parts), out.data_ptr(), threads) == 0
        assert torch.equal(out, ref), threads


def test_concurrent_callers():
    jobs = [_parts(100 + k, 40, 200_000) for k in range(6)]
    outs = [torch.empty(sum(p.numel() for p in ps)) for ps in jobs]
    errors = []

    def work(k):
        try:
            for _ in range(5):
                gather_into(jobs[k], outs[k])
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(k,)) for k in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    for ps, out in zip(jobs, outs):
        assert torch.equal(out, torch.cat(ps))


def _child(q):
    # torch's OpenMP pool does not survive fork(): the child's own torch ops
    # stay on one thread (the gather's pool is what is under test).
    torch.set_num_threads(1)
    parts = _parts(7, 32, 200_000)
    out = torch.empty(sum(p.numel() for p in parts))
    gather_into(parts, out)
    q.put(bool(torch.equal(out, torch.cat(parts))))


def test_forked_child_has_its_own_pool():
    gather_into(_parts(1, 32, 200_000), torch.empty(sum(p.numel() for p in _parts(1, 32, 200_000))))
    ctx = mp.get_context("fork")
    q = ctx.Queue()
    p = ctx.Process(target=_child, args=(q,), daemon=True)
    p.start()
    try:
        ok = q.get(timeout=60)
    finally:
        p.join(timeout=10)
        if p.is_alive():
            p.kill()
    assert ok and p.exitcode == 0


def test_errors():
    with pytest.raises(ValueError, match="elements"):
        gather_into([torch.ones(3)], torch.empty(4))
    lib = _lib.load()
    sizes = (ctypes.c_int64 * 2)(4, -1)
    ptrs = (ctypes.c_void_p * 2)(0x1000, 0x1000)
    assert lib.meshy_host_gather(ptrs, sizes, 2, 0x1000, 0) == -1
    assert "negative size" in lib.meshy_last_error().decode()
    sizes = (ctypes.c_int64 * 2)(4, 4)
    ptrs = (ctypes.c_void_p * 2)(0x1000, None)
    assert lib.meshy_host_gather(ptrs, sizes, 2, 0x1000, 0) == -2
    assert lib.meshy_host_gather(None, sizes, 2, 0x1000, 0) == -2
    assert lib.meshy_host_gather(ptrs, sizes, -1, 0x1000, 0) == -1
    assert lib.meshy_host_gather(None, None, 0, None, 0) == 0


def _mask_u8(parts, threads=0):
    lib = _lib.load()
    ptrs = (ctypes.c_void_p * max(1, len(parts)))(*[p.data_ptr() for p in parts])
    counts = (ctypes.c_int64 * max(1, len(parts)))(*[p.numel() for p in parts])
    out = torch.full((sum(p.numel() for p in parts),), 7, dtype=torch.uint8)
    binary = ctypes.c_int32(-1)
    rc = lib.meshy_host_gather_mask_u8(ptrs, counts, len(parts), out.data_ptr(), threads, ctypes.byref(binary))
    return rc, binary.value, out


@pytest.mark.parametrize("n,hi", [(1, 10), (9, 3), (300, 5000), (64, 300_000)])
def test_mask_u8_gather_of_binary_masks(n, hi):
    """0/1 fp32 masks come out as the same values in bytes, on every thread count."""
    g = torch.Generator().manual_seed(n)
    parts = [(torch.rand(int(s), generator=g) > 0.4).float() for s in torch.randint(0, hi, (n,), generator=g)]
    ref = torch.cat(parts).to(torch.uint8)
    for threads in (1, 3, 0):
        rc, binary, out = _mask_u8(parts, threads)
        assert (rc, binary) == (0, 1)
        assert torch.equal(out, ref)


@pytest.mark.parametrize("bad", [0.5, -0.0, 2.0, float("nan"), float("inf"), -1.0, 1e-45])
def test_mask_u8_gather_reports_other_values(bad):
    """Any float other than +0.0 and 1.0 (a fractional weight, -0.0, a
    denormal, NaN) clears `binary`, wherever it lies."""
    big = torch.ones(400_000)
    for where in (0, 123_457, 399_999):
        m = big.clone()
        m[where] = bad
        rc, binary, _ = _mask_u8([torch.zeros(5), m, torch.ones(3)])
        assert (rc, binary) == (0, 0)


def test_mask_u8_gather_errors():
    lib = _lib.load()
    binary = ctypes.c_int32(-1)
    counts = (ctypes.c_int64 * 1)(-1)
    ptrs = (ctypes.c_void_p * 1)(0x1000)
    assert lib.meshy_host_gather_mask_u8(ptrs, counts, 1, 0x1000, 0, ctypes.byref(binary)) == -1
    assert binary.value == 0
    assert lib.meshy_host_gather_mask_u8(ptrs, counts, 1, 0x1000, 0, None) == -2
    binary.value = -1
    assert lib.meshy_host_gather_mask_u8(None, None, 0, None, 0, ctypes.byref(binary)) == 0
    assert binary.value == 1


def _ids_i32(parts, threads=0):
    lib = _lib.load()
    ptrs = (ctypes.c_void_p * max(1, len(parts)))(*[p.data_ptr() for p in parts])
    counts = (ctypes.c_int64 * max(1, len(parts)))(*[p.numel() for p in parts])
    out = torch.full((sum(p.numel() for p in parts),), 7, dtype=torch.int32)
    fits = ctypes.c_int32(-1)
    rc = lib.meshy_host_gather_i32(ptrs, counts, len(parts), out.data_ptr(), threads, ctypes.byref(fits))
    return rc, fits.value, out


@pytest.mark.parametrize("n,hi", [(1, 10), (9, 3), (300, 5000), (64, 300_000)])
def test_i32_gather_of_ids_that_fit(n, hi):
    """int64 ids within int32 (both ends included) come out as the same values,
    on every thread count."""
    g = torch.Generator().manual_seed(n)
    parts = [torch.randint(-(2**31), 2**31, (int(s),), generator=g) for s in torch.randint(0, hi, (n,), generator=g)]
    parts[0][:2] = torch.tensor([2**31 - 1, -(2**31)])[: parts[0].numel()]
    ref = torch.cat(parts).to(torch.int32)
    for threads in (1, 3, 0):
        rc, fits, out = _ids_i32(parts, threads)
        assert (rc, fits) == (0, 1)
        assert torch.equal(out, ref)


@pytest.mark.parametrize("bad", [2**31, -(2**31) - 1, 2**32, 2**32 + 5, -(2**63), 2**63 - 1])
def test_i32_gather_reports_values_outside_int32(bad):
    """A value that int32 cannot hold clears `fits` wherever it lies, also one
    whose low 32 bits are a valid id (2**32 + 5)."""
    big = torch.arange(400_000, dtype=torch.int64)
    for where in (0, 123_457, 399_999):
        m = big.clone()
        m[where] = bad
        rc, fits, _ = _ids_i32([torch.zeros(5, dtype=torch.int64), m, torch.ones(3, dtype=torch.int64)])
        assert (rc, fits) == (0, 0)


def test_i32_gather_errors():
    lib = _lib.load()
    fits = ctypes.c_int32(-1)
    counts = (ctypes.c_int64 * 1)(-1)
    ptrs = (ctypes.c_void_p * 1)(0x1000)
    assert lib.meshy_host_gather_i32(ptrs, counts, 1, 0x1000, 0, ctypes.byref(fits)) == -1
    assert fits.value == 0
    assert lib.meshy_host_gather_i32(ptrs, counts, 1, 0x1000, 0, None) == -2
    fits.value = -1
    assert lib.meshy_host_gather_i32(None, None, 0, None, 0, ctypes.byref(fits)) == 0
    assert fits.value == 1

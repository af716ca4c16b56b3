"""meshy_logprob_bwd_noalloc (the allocation-free backward) against
meshy_logprob_bwd, both called through the C ABI.

Both run the same kernels, the first with its per-row scratch in a static
device array, the second in a caller workspace, so the bf16 gradients must be
bitwise equal.  Two calls in a row, the second smaller, check that the array
keeps nothing a later call depends on.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(rows, T, V, seed, dev):
    from meshy_amd import logprob

    g = torch.Generator().manual_seed(seed)
    z = (torch.randn(rows, T, V, generator=g) * 2.0).to(torch.bfloat16).to(dev)
    y = torch.randint(0, V, (rows, T), generator=g)
    y[0, 0] = -100  # ignored label: a zero row
    y = y.to(dev)
    gl = torch.randn(rows, T, generator=g).to(dev)
    lse = logprob.logsumexp_rows(z)
    return z, y, gl, lse


def _with_workspace(z, y, gl, lse):
    from meshy_amd import _lib, logprob

    rows, T, V = z.shape
    lib = _lib.load()
    grad = torch.full((rows, T, V), 7.0, dtype=torch.bfloat16, device=z.device)
    ws = logprob.bwd_workspace(rows * T, z.device)
    _lib.check(lib.meshy_logprob_bwd(z.data_ptr(), rows, T, V, z.stride(0), z.stride(1), y.data_ptr(),
                                     lse.data_ptr(), gl.data_ptr(), grad.data_ptr(), ws.data_ptr(), ws.numel(),
                                     _lib.stream_of(z.device)), "meshy_logprob_bwd")
    return grad


def _no_alloc(z, y, gl, lse):
    from meshy_amd import _lib

    rows, T, V = z.shape
    lib = _lib.load()
    grad = torch.full((rows, T, V), -3.0, dtype=torch.bfloat16, device=z.device)
    _lib.check(lib.meshy_logprob_bwd_noalloc(z.data_ptr(), rows, T, V, z.stride(0), z.stride(1), y.data_ptr(),
                                             lse.data_ptr(), gl.data_ptr(), grad.data_ptr(),
                                             _lib.stream_of(z.device)), "meshy_logprob_bwd_noalloc")
    return grad


def test_no_alloc_matches_workspace_entry_point_on_two_calls(dev):
    # First call: 2 x 300 rows of the Qwen3 vocabulary; second: 1 x 77 rows.
    for rows, T, V, seed in ((2, 300, 151936, 11), (1, 77, 151936, 12)):
        print(f"no-alloc bwd rows={rows} T={T} V={V} seed={seed}", flush=True)
        z, y, gl, lse = _inputs(rows, T, V, seed, dev)
        a = _no_alloc(z, y, gl, lse)
        b = _with_workspace(z, y, gl, lse)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        assert torch.isfinite(a.float()).all()
        assert (a[0, 0].float() == 0).all()  # the ignored label's row

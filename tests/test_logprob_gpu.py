"""Fused logprob + entropy kernel against the oracle (the reference's fp32 torch path).

Tolerance: 1e-3 absolute on fp32 logp and entropy (the bar for this path).
"""

import math

import pytest
import torch

from oracle import logprob as olp

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _logits(rows, T, V, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    z = (torch.randn(rows, T, V, generator=g) * scale).to(torch.bfloat16)
    y = torch.randint(0, V, (rows, T), generator=g)
    return z, y


def _check(z, y, dev, with_entropy=True, ref_dtype=torch.float32):
    from meshy_amd import logprob

    lp, ent = logprob.logprobs_and_entropy(z.to(dev), y.to(dev), with_entropy=True)
    ref_lp = olp.chunk_logprobs(z, y, dtype=ref_dtype).float()
    ref_ent = olp.chunk_entropy(z, dtype=ref_dtype).float()
    assert lp.dtype == torch.float32 and lp.shape == y.shape
    assert (lp.cpu() - ref_lp).abs().max().item() <= TOL
    assert (ent.cpu() - ref_ent).abs().max().item() <= TOL


@pytest.mark.parametrize("V", [151936, 131072, 50, 8, 7, 2, 1, 1001, 4096 * 4 + 3])
def test_matches_oracle_across_vocab_sizes(dev, V):
    z, y = _logits(2, 33, V, seed=V)
    _check(z, y, dev)


# Vocabularies whose chunks of 8 left after the full 2048-chunk tiles make
# the row's last tile 4 to 8 loads per thread deep (with and without full
# tiles before it); the last row holds its largest logits in the tail.
@pytest.mark.parametrize("V", [24384, 8800, 43968, 13600, 32760])
def test_matches_oracle_with_deep_row_tails(dev, V):
    z, y = _logits(2, 5, V, seed=V)
    z[1, 4, -9:] = 40.0  # far above the row's running max: the tail raises it
    _check(z, y, dev)


def test_strided_chunk_view(dev):
    # logits[:, s:e, :] views as the reference's chunk loop makes them.
    z, y = _logits(2, 40, 1024, seed=3)
    zd = z.to(dev)
    from meshy_amd import logprob

    lp = logprob.chunk_logprobs(zd[:, 8:30, :], y[:, 8:30].to(dev))
    assert (lp.cpu() - olp.chunk_logprobs(z[:, 8:30, :], y[:, 8:30])).abs().max() <= TOL


def test_unaligned_rows_take_generic_path(dev):
    # V odd: row starts are not 16-byte aligned.
    z, y = _logits(1, 17, 999, seed=5)
    _check(z, y, dev)


def test_ignore_index_and_out_of_range_labels(dev):
    from meshy_amd import logprob

    z, y = _logits(1, 6, 300, seed=7)
    y[0, 1] = -100
    y[0, 2] = 300  # out of range -> NaN (torch would raise)
    lp = logprob.chunk_logprobs(z.to(dev), y.to(dev)).cpu()
    assert lp[0, 1].item() == 0.0
    assert math.isnan(lp[0, 2].item())
    ok = torch.tensor([0, 3, 4, 5])
    ref = olp.chunk_logprobs(z[:, ok], y[:, ok])
    assert (lp[:, ok] - ref).abs().max() <= TOL


def test_closed_forms(dev):
    from meshy_amd import logprob

    V = 151936
    # Uniform logits: logp = -ln V, H = ln V.
    z = torch.full((1, 4, V), 3.0).to(torch.bfloat16)
    y = torch.tensor([[0, 5, V - 1, 77]])
    lp, ent = logprob.logprobs_and_entropy(z.to(dev), y.to(dev), with_entropy=True)
    assert torch.allclose(lp.cpu(), torch.full((1, 4), -math.log(V)), atol=1e-4)
    assert torch.allclose(ent.cpu(), torch.full((1, 4), math.log(V)), atol=1e-4)
    # One dominant logit: p -> 1 on it, H -> 0.
    z = torch.zeros(1, 1, V)
    z[0, 0, 123] = 200.0
    lp, ent = logprob.logprobs_and_entropy(z.to(torch.bfloat16).to(dev), torch.tensor([[123]]).to(dev),
                                           with_entropy=True)
    assert abs(lp.item()) < 1e-4 and abs(ent.item()) < 1e-4


def test_large_dynamic_range(dev):
    # Logits far from zero exercise the online max rescaling.
    z, y = _logits(2, 9, 5000, seed=11, scale=40.0)
    z = (z.float() + 500.0).to(torch.bfloat16)
    _check(z, y, dev)


@pytest.mark.parametrize("pattern", ["ramp", "late_rise", "late_spikes"])
def test_running_max_raised_in_later_tiles(dev, pattern):
    """Rows whose later register tiles exceed the running max a thread holds
    by more than 44 (a tile sum above 2^64): each such tile takes the exact
    update with its own max.  The ramp does it on nearly every tile of every
    thread; the spikes on one tile of one thread."""
    V = 151936
    g = torch.Generator().manual_seed(17)
    z = torch.randn(3, 5, V, generator=g) * 2.0
    y = torch.randint(0, V, (3, 5), generator=g)
    if pattern == "ramp":
        z += torch.linspace(-600.0, 600.0, V)
        y[:, 0] = V - 1
    elif pattern == "late_rise":
        z[..., V // 2:] += 120.0
    else:
        z[..., V - 100] = 250.0
        z[..., V - 7001] = 180.0
        y[:, 1] = V - 100
        y[:, 2] = V - 7001
    # Broad rows at an offset of 120: the fp32 formula is itself ~1.3e-3 off
    # in entropy there, so the expected values are the formula in fp64.
    _check(z.to(torch.bfloat16), y, dev, ref_dtype=torch.float64)


def test_non_finite_logits_propagate_like_torch(dev):
    """cross_entropy's log_softmax and the entropy formula on rows with +inf
    (label elsewhere and at the +inf), NaN, all -inf, and a -inf label:
    NaN wherever torch gives NaN, the same infinities, the rest within TOL."""
    from meshy_amd import logprob

    g = torch.Generator().manual_seed(9)
    z = torch.randn(1, 6, 1000, generator=g)
    z[0, 0, 3] = float("inf")
    z[0, 1, 3] = float("inf")
    z[0, 2, 500] = float("nan")
    z[0, 3, :] = float("-inf")
    z[0, 4, 7] = float("-inf")
    y = torch.tensor([[0, 3, 0, 0, 7, 1]])
    zb = z.to(torch.bfloat16)
    lp, ent = logprob.logprobs_and_entropy(zb.to(dev), y.to(dev), with_entropy=True)
    for got, want in ((lp.cpu(), olp.chunk_logprobs(zb, y)), (ent.cpu(), olp.chunk_entropy(zb))):
        assert torch.equal(torch.isnan(got), torch.isnan(want)), (got, want)
        inf = torch.isinf(want)
        assert torch.equal(got[inf], want[inf])
        fin = torch.isfinite(want)
        assert (got[fin] - want[fin]).abs().max().item() <= TOL


def test_deterministic(dev):
    from meshy_amd import logprob

    z, y = _logits(3, 16, 151936, seed=13)
    zd, yd = z.to(dev), y.to(dev)
    a = logprob.logprobs_and_entropy(zd, yd, with_entropy=True)
    b = logprob.logprobs_and_entropy(zd, yd, with_entropy=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_backward_matches_autograd(dev):
    from meshy_amd import logprob

    z, y = _logits(2, 12, 3000, seed=17)
    y[1, 3] = -100
    g = torch.randn(2, 12, generator=torch.Generator().manual_seed(1))
    zd = z.to(dev).requires_grad_(True)
    lp = logprob.logprobs_and_entropy(zd, y.to(dev))
    (lp * g.to(dev)).sum().backward()
    ref = olp.logprob_grad(z, y, g)
    got = zd.grad.float().cpu()
    # bf16 gradient: relative rounding 2^-8 on |grad| <= |g|.
    assert (got - ref).abs().max().item() <= 4e-3 * g.abs().max().item()
    assert got[1, 3].abs().max().item() == 0.0


def test_full_size_every_row(dev):
    """T=16384, V=151936 (the headline shape): every row against the oracle,
    1024 rows at a time, plus size-independent properties."""
    from meshy_amd import logprob

    T, V = 16384, 151936
    gen = torch.Generator(device=dev).manual_seed(1)
    z = (torch.randn(1, T, V, generator=gen, device=dev, dtype=torch.bfloat16) * 2.0)
    y = torch.randint(0, V, (1, T), generator=gen, device=dev)
    lp, ent = logprob.logprobs_and_entropy(z, y, with_entropy=True)
    # properties: logp <= 0, 0 <= H <= ln V, finite
    assert torch.isfinite(lp).all() and torch.isfinite(ent).all()
    assert (lp <= 1e-6).all()
    assert (ent >= -1e-6).all() and (ent <= math.log(V) + 1e-4).all()
    lp, ent, yc = lp.cpu(), ent.cpu(), y.cpu()
    worst_lp = worst_ent = 0.0
    for a in range(0, T, 1024):
        zs = z[:, a:a + 1024].cpu()
        worst_lp = max(worst_lp, (lp[:, a:a + 1024] - olp.chunk_logprobs(zs, yc[:, a:a + 1024])).abs().max().item())
        worst_ent = max(worst_ent, (ent[:, a:a + 1024] - olp.chunk_entropy(zs)).abs().max().item())
    print(f"[16384, 151936] every row: max|dlogp|={worst_lp:.2e} max|dH|={worst_ent:.2e}")
    assert worst_lp <= TOL and worst_ent <= TOL

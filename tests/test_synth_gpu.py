"""The counter-based synthetic logits: the device fill (meshy_synth_bf16)
equals the host regeneration bit for bit, for whole blocks, row strides,
unaligned widths and rows far into a large block."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from meshy_amd import _lib, workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,seed,scale", [(3, 8, 0, 2.0), (5, 131, 1, 2.0), (64, 151936, 7, 2.0),
                                                  (2, 1, 9, 0.5)])
def test_device_fill_equals_host_rows(dev, rows, cols, seed, scale):
    z = workloads.synth_logits(rows, cols, seed, scale, device=dev)
    host = workloads.synth_logit_rows(range(rows), cols, seed, scale)
    assert torch.equal(z.cpu().view(torch.int16), host.view(torch.int16))


def test_row_stride_and_far_rows(dev):
    rows, cols, stride = 4, 1000, 1024
    buf = torch.full((rows, stride), -1, dtype=torch.int16, device=dev)
    rc = _lib.load().meshy_synth_bf16(buf.data_ptr(), rows, cols, stride, 5, 2.0, _lib.stream_of(dev))
    _lib.check(rc, "meshy_synth_bf16")
    got = buf.cpu()
    assert (got[:, cols:] == -1).all()  # nothing written past a row's columns
    assert torch.equal(got[:, :cols], workloads.synth_logit_rows(range(rows), cols, 5).view(torch.int16))
    # rows deep in a [129024, 131072] block: fill a 2-row slice at the right element offset
    V = 131072
    far = [100000, 129023]
    z = workloads.synth_logits(1, V, 11, device=dev)
    assert torch.equal(z.cpu(), workloads.synth_logit_rows([0], V, 11))
    rng = np.random.default_rng(0)
    ids = np.sort(rng.choice(129024, 4, replace=False))
    a = workloads.synth_logit_rows(list(ids) + far, V, 11)
    b = torch.cat([workloads.synth_logit_rows([int(i)], V, 11) for i in list(ids) + far])
    assert torch.equal(a, b)

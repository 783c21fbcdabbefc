"""The achievable-peak probes (lkv_probe_read / lkv_probe_mfma) do the work they are timed for:
the read probe's per-thread XOR equals the host's XOR over that thread's grid-stride chunks, and
the MFMA probe gives finite, seed-determined results."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("chunks,wgs", [(1000, 1), (40000, 3), (123457, 16)])
def test_probe_read_touches_every_chunk(chunks, wgs):
    g = torch.Generator(device=DEV).manual_seed(chunks)
    x = torch.randint(-2 ** 31, 2 ** 31 - 1, (chunks, 4), generator=g, device=DEV, dtype=torch.int64).to(torch.int32)
    sink = ops.probe_read(x, workgroups=wgs)
    per_chunk = np.bitwise_xor.reduce(x.cpu().numpy().view(np.uint32), axis=1)
    threads = wgs * ops.PROBE_THREADS
    want = np.zeros(threads, np.uint32)
    for t in range(min(threads, chunks)):
        want[t] = np.bitwise_xor.reduce(per_chunk[t::threads])
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)


def test_probe_mfma_is_finite_and_seed_determined():
    a, flops = ops.probe_mfma(DEV, 8, 64, seed=5)
    b, _ = ops.probe_mfma(DEV, 8, 64, seed=5)
    c, _ = ops.probe_mfma(DEV, 8, 64, seed=6)
    av = a.cpu().numpy().view(np.float32)
    assert flops == 8 * 4 * 64 * 8 * 16384
    assert np.all(np.isfinite(av)) and np.any(av != 0)
    assert torch.equal(a, b) and not torch.equal(a, c)

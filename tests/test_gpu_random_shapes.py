"""Seeded random shapes for the attention entry points against the oracle (GPU).

Each case draws a batch, GQA geometry, query count, older-segment length, ring size and start
(wrapping or not), causal or bidirectional masking; prefill runs through the automatic kernel
choice (decode kernel for <= 64 query rows per kv head, MFMA tiles above) and through the tile
kernel forced with tile_waves = 4, decode through one and several key splits."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16

from test_gpu_decode import _bf, _close, _t, _two_segments

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 4))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 3, 4, 5, 8]))
    L = int(rng.choice([1, 2, 3, 5, 8, 13, 33, 70]))
    T0 = int(rng.integers(1, 400))
    ring_blocks = int(rng.integers(-(-L // 32) + 1, 12))
    n1 = int(rng.integers(L, ring_blocks * 32 + 1))
    start = int(rng.integers(0, ring_blocks * 32))
    causal = bool(rng.integers(0, 2))
    return rng, B, Hkv, G, L, T0, ring_blocks, n1, start, causal


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill_shapes_match_oracle(seed):
    rng, B, Hkv, G, L, T0, ring_blocks, n1, start, causal = _case(seed)
    Hq = G * Hkv
    seg, k, v = _two_segments(rng, B, Hkv, T0=T0, n1=n1, start=start, ring_blocks=ring_blocks)
    q = _bf(rng, (B, L, Hq, 128))
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
    want_out = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    label = f"seed {seed}: B={B} Hkv={Hkv} G={G} L={L} T0={T0} ring={ring_blocks} n1={n1} start={start} causal={causal}"
    print(label, flush=True)
    for tw in (0, 4):
        lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
        out = ops.prefill_attention(_t(q), causal=causal, lse=lse, tile_waves=tw, **seg)
        _close(out, want_out, f"{label} tile_waves={tw}")
        np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("seed", range(12))
def test_random_decode_shapes_match_oracle(seed):
    rng, B, Hkv, G, _, T0, ring_blocks, n1, start, _ = _case(seed + 100)
    Hq = G * Hkv
    n1 = max(1, n1)
    seg, k, v = _two_segments(rng, B, Hkv, T0=T0, n1=n1, start=start, ring_blocks=ring_blocks)
    q = _bf(rng, (B, Hq, 1, 128))
    want, want_lse = A.attention(q, k, v)
    label = f"seed {seed}: B={B} Hkv={Hkv} G={G} T0={T0} ring={ring_blocks} n1={n1} start={start}"
    print(label, flush=True)
    for splits in (1, 5):
        lse = torch.empty((B, Hq), dtype=torch.float32, device=DEV)
        out = ops.decode_attention(_t(q), num_splits=splits, lse=lse, **seg)
        _close(out, bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"{label} splits={splits}")
        np.testing.assert_allclose(lse.cpu().numpy(), want_lse[:, :, 0], rtol=1e-4, atol=1e-4)

"""Seeded random shapes for the attention entry points against the oracle (GPU).

Each case draws a batch, GQA geometry, query count, older-segment length, ring size and start
(wrapping or not), causal or bidirectional masking.  Every prefill case runs three ways: the
automatic kernel choice (decode kernel for <= 64 query rows per kv head, MFMA tiles above) and
the tile kernel forced with tile_waves = 4 and 8 (at <= 64 rows per kv head that is the 2-wave
tile instance, whose probabilities are split into fp16 hi + lo).  The bar is the north star's:
max-abs 2e-2 and rel-L2 1e-3 of the bf16 outputs against the fp64 oracle rounded to bf16.  The
sweep covers 300 shapes in six tests of 50 (``pytest -x`` stops at the first failing shape);
seeds 5039, 5049, 5114, 5139 and 5227 are the shapes on which the 2-wave tile instance exceeded
rel-L2 1e-3 (1.02-1.08e-3) before it split P, kept as named regression cases.  A second sweep
draws wide calls (65-600 query rows per kv head, up to 3K keys) on the default tile path and
reports its worst margin.  Decode runs through one and several key splits.  A long sweep runs 2,000
more shapes (20 tests of 100) and 100 wide calls through every tile choice (4 tests of 25)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16

from test_gpu_decode import MAX_ABS, REL_L2, _bf, _t, _two_segments

pytestmark = pytest.mark.gpu
DEV = "cuda"

SWEEP_SEED0 = 5000
SWEEP_SHAPES = 300
SWEEP_PART = 50
REGRESSION_SEEDS = [5039, 5049, 5114, 5139, 5227]

_worst: dict[str, float] = {}


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


def _check(out, want, label, key):
    a = out.float().cpu().numpy()
    ma, rl = A.max_abs(a, want), A.rel_l2(a, want)
    _worst[key] = max(_worst.get(key, 0.0), rl)
    assert ma <= MAX_ABS and rl <= REL_L2, f"{label}: max_abs={ma} rel_l2={rl}"
    return rl


def _prefill_case(seed, waves=(0, 4, 8)):
    rng, B, Hkv, G, L, T0, ring_blocks, n1, start, causal = _case(seed)
    Hq = G * Hkv
    seg, k, v = _two_segments(rng, B, Hkv, T0=T0, n1=n1, start=start, ring_blocks=ring_blocks)
    q = _bf(rng, (B, L, Hq, 128))
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
    want_out = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    label = f"seed {seed}: B={B} Hkv={Hkv} G={G} L={L} T0={T0} ring={ring_blocks} n1={n1} start={start} causal={causal}"
    small = L * G <= 64
    rels = []
    for tw in waves:
        lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
        out = ops.prefill_attention(_t(q), causal=causal, lse=lse, tile_waves=tw, **seg)
        kernel = ("decode" if tw == 0 else "tile2") if small else f"tile{tw or 'auto'}"
        rels.append(_check(out, want_out, f"{label} tile_waves={tw}", kernel))
        np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    return label, rels


@pytest.mark.parametrize("part", range(SWEEP_SHAPES // SWEEP_PART))
def test_random_prefill_sweep(part):
    """Shapes SWEEP_SEED0 + [50 part, 50 part + 50): automatic choice and tile_waves 4 and 8."""

    seeds = range(SWEEP_SEED0 + part * SWEEP_PART, SWEEP_SEED0 + (part + 1) * SWEEP_PART)
    for seed in seeds:
        label, rels = _prefill_case(seed)
        if seed % 10 == 0:
            print(f"{label}: rel_l2 auto/4/8 = {rels[0]:.2e}/{rels[1]:.2e}/{rels[2]:.2e}", flush=True)
    print("worst rel_l2 so far by kernel: " + ", ".join(f"{k} {v:.3e}" for k, v in sorted(_worst.items())), flush=True)


@pytest.mark.parametrize("seed", REGRESSION_SEEDS)
def test_prefill_tile_small_call_regressions(seed):
    """The forced 2-wave tile calls that exceeded rel-L2 1e-3 with single fp16 probabilities."""

    label, rels = _prefill_case(seed, waves=(4, 8))
    print(f"{label}: rel_l2 tile 4/8 = {rels[0]:.2e}/{rels[1]:.2e}", flush=True)


def _wide_case(seed):
    rng = np.random.default_rng(9000 + seed)
    B = int(rng.integers(1, 3))
    Hkv = int(rng.choice([1, 2]))
    G = int(rng.choice([1, 2, 4, 8]))
    L = int(rng.integers(-(-65 // G), -(-600 // G) + 1))
    T0 = int(rng.integers(0, 2500))
    ring_blocks = int(rng.integers(-(-L // 32) + 1, -(-L // 32) + 40))
    n1 = int(rng.integers(L, ring_blocks * 32 + 1))
    start = int(rng.integers(0, ring_blocks * 32))
    causal = bool(rng.integers(0, 2))
    return rng, B, Hkv, G, L, T0, ring_blocks, n1, start, causal


@pytest.mark.parametrize("seed", range(12))
def test_random_wide_prefill_tile_margin(seed):
    """Calls above 64 query rows per kv head on the default tile path (automatic 4- or 8-wave tiles)."""

    rng, B, Hkv, G, L, T0, ring_blocks, n1, start, causal = _wide_case(seed)
    Hq = G * Hkv
    older_args = dict(T0=max(T0, 1), n1=n1, start=start, ring_blocks=ring_blocks)
    seg, k, v = _two_segments(rng, B, Hkv, **older_args)
    q = _bf(rng, (B, L, Hq, 128))
    want, _ = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
    want_out = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    label = f"wide seed {seed}: B={B} Hkv={Hkv} G={G} L={L} T0={max(T0, 1)} ring={ring_blocks} n1={n1} causal={causal}"
    out = ops.prefill_attention(_t(q), causal=causal, **seg)
    rl = _check(out, want_out, label, "tile-wide")
    print(f"{label}: rel_l2={rl:.3e}; worst wide so far {_worst['tile-wide']:.3e}", flush=True)


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
        _check(out, bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"{label} splits={splits}", f"decode-s{splits}")
        np.testing.assert_allclose(lse.cpu().numpy(), want_lse[:, :, 0], rtol=1e-4, atol=1e-4)


LONG_SWEEP_SEED0 = 20000
LONG_SWEEP_SHAPES = 2000
LONG_SWEEP_PART = 100
LONG_WIDE_SEED0 = 3000
LONG_WIDE_SHAPES = 100
LONG_WIDE_PART = 25


@pytest.mark.parametrize("part", range(LONG_SWEEP_SHAPES // LONG_SWEEP_PART))
def test_long_random_prefill_sweep(part):
    """2,000 more shapes of the same generator (automatic choice and tile_waves 4 and 8) in parts of
    100: every call within the bar; prints the worst rel-L2 per kernel path so far."""

    seed0 = LONG_SWEEP_SEED0 + part * LONG_SWEEP_PART
    for seed in range(seed0, seed0 + LONG_SWEEP_PART):
        _prefill_case(seed)
    print("worst rel_l2 so far by kernel: " + ", ".join(f"{k} {v:.3e}" for k, v in sorted(_worst.items())), flush=True)


@pytest.mark.parametrize("part", range(LONG_WIDE_SHAPES // LONG_WIDE_PART))
def test_long_random_wide_sweep(part):
    """100 wide calls (65-600 query rows per kv head) through all three tile choices, in parts of 25;
    the last part prints the worst rel-L2 per kernel path (the figures quoted for the tiles' margin)."""

    seed0 = LONG_WIDE_SEED0 + part * LONG_WIDE_PART
    for seed in range(seed0, seed0 + LONG_WIDE_PART):
        rng, B, Hkv, G, L, T0, ring_blocks, n1, start, causal = _wide_case(seed)
        seg, k, v = _two_segments(rng, B, Hkv, T0=max(T0, 1), n1=n1, start=start, ring_blocks=ring_blocks)
        q = _bf(rng, (B, L, G * Hkv, 128))
        want, _ = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
        want_out = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
        for tw in (0, 4, 8):
            out = ops.prefill_attention(_t(q), causal=causal, tile_waves=tw, **seg)
            _check(out, want_out, f"wide seed {seed} tile_waves={tw}", f"wide-tw{tw}")
    print("worst rel_l2 by kernel: " + ", ".join(f"{k} {v:.3e}" for k, v in sorted(_worst.items())), flush=True)

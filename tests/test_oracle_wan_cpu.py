"""Pins oracle/wan.py (the Wan shared-history restatement) on the CPU.

- shared-store and per-layer-store rollouts compose bit-identical histories (the property the
  reference's own test checks, test_videogen_inference.py:63-78);
- the reference test's known answer for the retained prefix (test_videogen_inference.py:84-98);
- a per-position brute force of the composed history (written position by position from the
  reference's rules, a different code shape than the oracle's slicing);
- limits: alpha = 1 gives the shared values, alpha = 0 the layer's own, keep beyond the history
  keeps everything local; the block attention with no history is plain bidirectional attention.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as A
from oracle import bf16
from oracle import wan as W


def _kvs(rng, layers, B, S, H, D):
    return [(bf16.round_bf16(rng.standard_normal((B, S, H, D)).astype(np.float32)),
             bf16.round_bf16(rng.standard_normal((B, S, H, D)).astype(np.float32))) for _ in range(layers)]


@pytest.mark.parametrize("keep", [3, 12, 17, 40])
def test_shared_and_native_rollouts_compose_identical_histories(keep):
    rng = np.random.default_rng(keep)
    L, B, S, H, D, blocks = 3, 2, 12, 2, 8, 4
    alphas = [W.alpha_bf16(rng.standard_normal(H)) for _ in range(L)]
    shared = W.WanCache(L, B, H, S * (blocks - 1), S, keep, shared=True, dim=D)
    native = W.WanCache(L, B, H, S * (blocks - 1), S, keep, shared=False, dim=D)
    for n in range(blocks - 1):
        for l in range(L):
            hs, hn = shared.history(l, n * S, S, alphas[l]), native.history(l, n * S, S, alphas[l])
            assert (hs is None) == (hn is None) == (n == 0)
            if hs is not None:
                assert np.array_equal(hs[0], hn[0]) and np.array_equal(hs[1], hn[1])
        kvs = _kvs(rng, L, B, S, H, D)
        shared.commit(kvs, n * S)
        native.commit(kvs, n * S)


def test_retained_prefix_known_answer():
    """test_videogen_inference.py:84-98: layer l appends K = 99 with K[:, :3] = l + 1 and V = -K
    at position 0 of a 24-token cache (block 12, keep 3); history_kv(12) then reads l + 1 in the
    first 3 positions and 99 after, V = -K."""

    L, H, D = 3, 2, 8
    cache = W.WanCache(L, 1, H, 24, 12, 3, shared=True, dim=D)
    kvs = []
    for l in range(L):
        k = np.full((1, 12, H, D), 99.0, np.float32)
        k[:, :3] = l + 1
        kvs.append((k, -k))
    cache.commit(kvs, 0)
    for l in range(L):
        k, v = cache.deep(l, 12)
        assert np.all(k[:, :3] == l + 1) and np.all(k[:, 3:] == 99) and np.array_equal(v, -k)


def _brute_history(kv_blocks, layer, h, S, keep, alpha):
    """Position-by-position composition: p < prev_start -> own if p < keep else final layer;
    p in the previous block -> own if p < keep else bf16(bf16(a*src) + bf16(bf16(1-a)*own))."""

    B, _, H, D = kv_blocks[0][0][0].shape
    prev_start = h - min(S, h)
    k = np.zeros((B, h, H, D), np.float32)
    v = np.zeros((B, h, H, D), np.float32)
    for p in range(h):
        n, i = divmod(p, S)
        own_k, own_v = kv_blocks[n][layer][0][:, i], kv_blocks[n][layer][1][:, i]
        src_k, src_v = kv_blocks[n][-1][0][:, i], kv_blocks[n][-1][1][:, i]
        if p < keep:
            k[:, p], v[:, p] = own_k, own_v
        elif p < prev_start:
            k[:, p], v[:, p] = src_k, src_v
        else:
            for h_ in range(H):
                a = np.float32(alpha[h_])
                om = bf16.round_bf16(np.float32(1.0) - a)
                k[:, p, h_] = bf16.round_bf16(bf16.round_bf16(a * src_k[:, h_]) + bf16.round_bf16(om * own_k[:, h_]))
                v[:, p, h_] = bf16.round_bf16(bf16.round_bf16(a * src_v[:, h_]) + bf16.round_bf16(om * own_v[:, h_]))
    return k, v


@pytest.mark.parametrize("keep", [5, 12, 30])
def test_history_matches_position_brute_force(keep):
    rng = np.random.default_rng(40 + keep)
    L, B, S, H, D = 2, 1, 10, 3, 4
    alphas = [W.alpha_bf16(rng.standard_normal(H)) for _ in range(L)]
    cache = W.WanCache(L, B, H, 50, S, keep, shared=True, dim=D)
    blocks = []
    for n in range(5):
        kvs = _kvs(rng, L, B, S, H, D)
        blocks.append(kvs)
        cache.commit(kvs, n * S)
        for l in range(L):
            h = (n + 1) * S
            got = cache.history(l, h, S, alphas[l])
            want = _brute_history(blocks, l, h, S, keep, alphas[l])
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), (n, l)


def test_alpha_and_keep_limits():
    rng = np.random.default_rng(2)
    L, B, S, H, D = 2, 1, 8, 2, 4
    cache = W.WanCache(L, B, H, 32, S, 3, shared=True, dim=D)
    blocks = [_kvs(rng, L, B, S, H, D) for _ in range(3)]
    for n, kvs in enumerate(blocks):
        cache.commit(kvs, n * S)
    for l in range(L):
        k1, _ = cache.history(l, 24, S, np.ones(H, np.float32))  # alpha = 1: shared values
        assert np.array_equal(k1[:, 19:], blocks[2][-1][0][:, 3:])
        k0, _ = cache.history(l, 24, S, np.zeros(H, np.float32))  # alpha = 0: the layer's own
        assert np.array_equal(k0[:, 16:], blocks[2][l][0])
    wide = W.WanCache(L, B, H, 32, S, 100, shared=True, dim=D)  # keep beyond the history: all own
    for n, kvs in enumerate(blocks):
        wide.commit(kvs, n * S)
    for l in range(L):
        k, v = wide.history(l, 24, S, np.full(H, 0.5, np.float32))
        assert np.array_equal(k, np.concatenate([b[l][0] for b in blocks], 1))
        assert np.array_equal(v, np.concatenate([b[l][1] for b in blocks], 1))


def test_block_attention_without_history_is_plain_bidirectional():
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((1, 6, 2, 8)) for _ in range(3))
    got = W.block_attention(q, k, v, None)
    s = np.einsum("bqhd,bkhd->bhqk", q, k) / np.sqrt(8)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = np.einsum("bhqk,bkhd->bqhd", p, v)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert A.max_abs(got, want) < 1e-12

"""GPU parity of the Wan history path (lastkv_amd.videogen) and of the paged append it writes with.

- ``lkv_append_paged``: rows written at unaligned positions, with and without a ring wrap, read
  back through ``lkv_cache_unpack`` (pinned against oracle/layout.py) equal the input bit for bit,
  and no other position changes.
- ``WanKVCache`` rollouts against oracle/wan.py (the reference's cache.py + model.py:153-272
  restated): after every commit each layer's history equals the oracle's bit for bit (the blend is
  bf16 op for op); every block attention, in denoising passes and in the clean update pass, is
  within max-abs 2e-2 / rel-L2 1e-3 of fp64 bidirectional attention over the oracle's history,
  rounded to bf16.  Block sizes straddle pages, ``keep`` is unaligned, and the ring wraps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from lastkv_amd.videogen import WanKVCache
from oracle import attention as A
from oracle import bf16
from oracle import wan as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(actual: torch.Tensor, expected, label: str):
    a = actual.float().cpu().numpy()
    e = bf16.round_bf16(np.asarray(expected, np.float32))
    ma, rl = A.max_abs(a, e), A.rel_l2(a, e)
    print(f"{label}: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= 2e-2 and rl <= 1e-3, f"{label}: max_abs={ma} rel_l2={rl}"


def _read(pool: ops.PagedKV, table: torch.Tensor, tokens: int):
    """Cache positions [0, tokens) through ``table`` [B, W] as [B, tokens, H, 128] (K, V)."""

    B, Wd = table.shape
    idx = table.reshape(-1).long()
    tk = pool.kp[idx].reshape(B, Wd, pool.heads, 4096).permute(0, 2, 1, 3).contiguous()
    tv = pool.vp[idx].reshape(B, Wd, pool.heads, 4096).permute(0, 2, 1, 3).contiguous()
    k = ops.cache_unpack(tk, ops.KIND_K, 0, tokens)
    v = ops.cache_unpack(tv, ops.KIND_V, 0, tokens)
    return k.transpose(1, 2), v.transpose(1, 2)


@pytest.mark.parametrize("token0,T,wrap", [(0, 64, 0), (13, 50, 0), (37, 3, 0), (150, 90, 192), (181, 11, 192)])
def test_append_paged_round_trip(token0, T, wrap):
    g = torch.Generator(device=DEV).manual_seed(token0 + T)
    B, H, Wd = 2, 3, 8
    pool = ops.PagedKV.zeros(3 * B * Wd, H, DEV)
    pool.k.copy_(torch.randn(pool.k.shape, generator=g, device=DEV).bfloat16())
    pool.v.copy_(torch.randn(pool.v.shape, generator=g, device=DEV).bfloat16())
    perm = torch.randperm(3 * B * Wd, generator=torch.Generator().manual_seed(1))[: B * Wd]
    table = perm.view(B, Wd).to(DEV, torch.int32)
    before_k, before_v = _read(pool, table, Wd * 32)
    base = torch.randn((B, T, H + 1, 128), generator=g, device=DEV).bfloat16()
    k, v = base[:, :, :H], base[:, :, 1:]  # strided views, as from a fused projection
    ops.append_paged(k, v, pool, table, token0=token0, wrap_tokens=wrap)
    after_k, after_v = _read(pool, table, Wd * 32)
    pos = torch.arange(token0, token0 + T) % (wrap or 10**9)
    mask = torch.zeros(Wd * 32, dtype=torch.bool)
    mask[pos] = True
    assert torch.equal(after_k[:, pos.to(DEV)], k) and torch.equal(after_v[:, pos.to(DEV)], v)
    keep = (~mask).to(DEV)
    assert torch.equal(after_k[:, keep], before_k[:, keep]) and torch.equal(after_v[:, keep], before_v[:, keep])


def test_set_alphas_matches_oracle():
    logits = torch.randn(4, 6, generator=torch.Generator().manual_seed(3)) * 3
    cache = WanKVCache(num_layers=4, num_heads=6, block_tokens=64, total_tokens=128, keep_tokens=10, device=DEV)
    cache.set_alphas(logits)
    want = W.alpha_bf16(logits.double().numpy())
    assert np.array_equal(cache.alpha.view(4, 6).cpu().numpy(), want)
    assert np.array_equal(cache.one_minus_alpha.view(4, 6).cpu().numpy(), bf16.rsub(want, 1.0))


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, torch.bfloat16)


def _random_rollout(seed):
    rng = np.random.default_rng(740 + seed)
    S = int(rng.integers(5, 260))
    keep = [None, int(rng.integers(1, 2 * S)), 10 ** 6][int(rng.integers(0, 3))]
    return int(rng.integers(1, 3)), S, keep, int(rng.integers(1, 7)), int(rng.integers(3, 7))


@pytest.mark.parametrize("B,S,keep,H,blocks", [(1, 200, 70, 4, 5), (2, 96, 32, 2, 5), (1, 136, None, 3, 5),
                                               (1, 64, 1000, 2, 5)] + [_random_rollout(i) for i in range(6)])
def test_wan_rollout_matches_oracle(B, S, keep, H, blocks):
    """Block-causal rollouts through WanKVCache against the oracle: every layer's attention of every
    pass (denoising and the clean update pass) and the history after each commit; the four fixed
    cases and six seeded random ones (block sizes 5-259 tokens, kept prefixes short, long or the
    whole history, 1-6 heads, 3-6 blocks)."""

    rng = np.random.default_rng(S + (keep or 0))
    L = 3
    total = S * (blocks - 1)
    cache = WanKVCache(num_layers=L, num_heads=H, block_tokens=S, total_tokens=total, keep_tokens=keep, batch=B,
                       device=DEV)
    cache.set_alphas(torch.from_numpy(rng.standard_normal((L, H))).float())
    alphas = cache.alpha.view(L, H).cpu().numpy()
    oracle = W.WanCache(L, B, H, total, S, S if keep is None else keep, shared=True)

    def rnd():
        return bf16.round_bf16(rng.standard_normal((B, S, H, 128)).astype(np.float32))

    for n in range(blocks):
        s = n * S
        passes = [[(rnd(), rnd(), rnd()) for _ in range(L)]]  # one denoising pass
        clean = [(rnd(), rnd(), rnd()) for _ in range(L)]
        if n < blocks - 1:
            passes.append(clean)  # the update pass attends with the clean block, then commits
        for p, layer_qkv in enumerate(passes):
            for l, (q, k, v) in enumerate(layer_qkv):
                out = cache.attention(l, _t(q), _t(k), _t(v), s)
                want = W.block_attention(q, k, v, oracle.history(l, s, S, alphas[l]))
                _close(out, want, f"block {n} pass {p} layer {l}")
        if n < blocks - 1:
            cache.commit(s, [(_t(k), _t(v)) for _, k, v in clean])
            oracle.commit([(k, v) for _, k, v in clean], s)
            for l in range(L):
                hk, hv = cache.history(l)
                wk, wv = oracle.history(l, s + S, S, alphas[l])
                assert np.array_equal(hk.float().cpu().numpy(), wk), f"history K block {n} layer {l}"
                assert np.array_equal(hv.float().cpu().numpy(), wv), f"history V block {n} layer {l}"

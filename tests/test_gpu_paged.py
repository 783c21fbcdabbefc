"""Paged segments: the same K/V scattered into a shuffled page pool and addressed through block
tables gives bit-identical decode and prefill outputs to the contiguous per-slot caches (same
arithmetic in the same order), for the shared older segment, the ring, and both together."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _rand_cache(g, slots, heads, tokens):
    shape = (slots, heads, tokens // 32, 4096)
    return ops.TiledKV(torch.randn(shape, generator=g, device=DEV).bfloat16(),
                       torch.randn(shape, generator=g, device=DEV).bfloat16())


def _scatter(cache: ops.TiledKV, pool: ops.PagedKV, pages: torch.Tensor) -> torch.Tensor:
    """Copy every (slot, block) of ``cache`` into pool page ``pages[slot, block]``; returns the table."""

    S, H, nb, _ = cache.k.shape
    flat = pages.reshape(-1).long()
    pool.kp[flat] = cache.k.permute(0, 2, 1, 3).reshape(S * nb, H, 4096)
    pool.vp[flat] = cache.v.permute(0, 2, 1, 3).reshape(S * nb, H, 4096)
    return pages.to(torch.int32).contiguous()


def _paged_copies(g, older, ring, extra_pages=17):
    B, H = older.slots, older.heads
    no, nr = older.blocks, ring.blocks
    total = B * (no + nr) + extra_pages
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(7)).to(DEV)
    pool = ops.PagedKV.zeros(total, H, DEV)
    pool.k.copy_(torch.randn(pool.k.shape, generator=g, device=DEV).bfloat16())  # junk in unused pages
    pool.v.copy_(torch.randn(pool.v.shape, generator=g, device=DEV).bfloat16())
    otab = _scatter(older, pool, perm[: B * no].view(B, no))
    rtab = _scatter(ring, pool, perm[B * no : B * (no + nr)].view(B, nr))
    # widen the tables with junk columns past the used width (never read)
    otab = torch.cat([otab, torch.full((B, 3), 10**6, dtype=torch.int32, device=DEV)], 1)
    return pool, otab, rtab


@pytest.mark.parametrize("older_len,local_len,start", [(900, 70, 100), (1024, 0, 0), (0, 150, 250), (37, 5, 31)])
def test_decode_paged_equals_contiguous(older_len, local_len, start):
    g = torch.Generator(device=DEV).manual_seed(older_len + local_len)
    B, Hq, Hkv = 3, 16, 4
    older = _rand_cache(g, B, Hkv, 1024)
    ring = _rand_cache(g, B, Hkv, 288)
    pool, otab, rtab = _paged_copies(g, older, ring)
    q = torch.randn((B, Hq, 128), generator=g, device=DEV).bfloat16()
    vs = torch.rand(Hkv, generator=g, device=DEV) + 0.5
    seg_c, seg_p = {}, {}
    if older_len:
        seg_c.update(older=older, older_len=older_len, vscale=vs)
        seg_p.update(older=pool, older_table=otab, older_len=older_len, vscale=vs)
    if local_len:
        seg_c.update(local=ring, local_len=local_len, local_start=start)
        seg_p.update(local=pool, local_table=rtab, local_len=local_len, local_start=start)
    for splits in (1, 3):
        a = ops.decode_attention(q, num_splits=splits, **seg_c)
        b = ops.decode_attention(q, num_splits=splits, **seg_p)
        assert torch.equal(a, b), f"splits={splits}"


@pytest.mark.parametrize("L,older_len,local_len,start,causal", [
    (64, 640, 96, 200, True), (17, 96, 17, 0, True), (300, 0, 300, 13, False), (100, 1000, 100, 283, True),
    (3, 500, 40, 290, True)])
def test_prefill_paged_equals_contiguous(L, older_len, local_len, start, causal):
    g = torch.Generator(device=DEV).manual_seed(L * 7 + older_len)
    B, Hq, Hkv = 2, 8, 2
    older = _rand_cache(g, B, Hkv, 1024)
    ring = _rand_cache(g, B, Hkv, 320)
    pool, otab, rtab = _paged_copies(g, older, ring)
    q = torch.randn((B, L, Hq, 128), generator=g, device=DEV).bfloat16()
    vs = torch.rand(Hkv, generator=g, device=DEV) + 0.5
    lse_c = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
    lse_p = torch.empty_like(lse_c)
    seg_c = dict(local=ring, local_len=local_len, local_start=start, causal=causal)
    seg_p = dict(local=pool, local_table=rtab, local_len=local_len, local_start=start, causal=causal)
    if older_len:
        seg_c.update(older=older, older_len=older_len, vscale=vs)
        seg_p.update(older=pool, older_table=otab, older_len=older_len, vscale=vs)
    for tw in (0, 4, 8):  # (L = 3: the decode kernel at 0, the tile kernel otherwise)
        a = ops.prefill_attention(q, lse=lse_c, tile_waves=tw, **seg_c)
        b = ops.prefill_attention(q, lse=lse_p, tile_waves=tw, **seg_p)
        assert torch.equal(a, b), f"tile_waves={tw}"
        assert torch.equal(lse_c, lse_p), f"tile_waves={tw}"


def test_corrupt_page_ids_stay_inside_the_pool():
    """Page ids outside [0, pages) are clamped: the call completes and reads only pool memory."""

    g = torch.Generator(device=DEV).manual_seed(3)
    B, Hq, Hkv = 2, 8, 2
    pool = ops.PagedKV.zeros(6, Hkv, DEV)
    table = torch.tensor([[0, 1, -5, 99], [5, 2**30, 3, -1]], dtype=torch.int32, device=DEV)
    q = torch.randn((B, Hq, 128), generator=g, device=DEV).bfloat16()
    out = ops.decode_attention(q, older=pool, older_table=table, older_len=128)
    ql = torch.randn((B, 40, Hq, 128), generator=g, device=DEV).bfloat16()
    out2 = ops.prefill_attention(ql, older=pool, older_table=table, older_len=128)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(out2.float()).all()


def _gather(pool: ops.PagedKV, table: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Pool pages listed in ``table`` [S, nb] back into contiguous [S, H, nb, 4096] caches."""

    S, nb = table.shape
    idx = table.reshape(-1).long()
    k = pool.kp[idx].reshape(S, nb, pool.heads, 4096).permute(0, 2, 1, 3).contiguous()
    v = pool.vp[idx].reshape(S, nb, pool.heads, 4096).permute(0, 2, 1, 3).contiguous()
    return k, v


def test_epilogue_paged_equals_contiguous():
    g = torch.Generator(device=DEV).manual_seed(9)
    B, L, Hq, Hkv, p0 = 3, 20, 8, 2, 50
    ring = _rand_cache(g, B, Hkv, 128)
    deep = _rand_cache(g, B, Hkv, 256)
    perm = torch.randperm(B * 12 + 5, generator=torch.Generator().manual_seed(1)).to(DEV)
    pool = ops.PagedKV.zeros(B * 12 + 5, Hkv, DEV)
    rtab = _scatter(ring, pool, perm[: B * 4].view(B, 4))
    dtab = _scatter(deep, pool, perm[B * 4 : B * 12].view(B, 8))
    q = torch.randn((B, L, Hq * 128), generator=g, device=DEV).bfloat16()
    k = torch.randn((B, L, Hkv * 128), generator=g, device=DEV).bfloat16()
    v = torch.randn((B, L, Hkv * 128), generator=g, device=DEV).bfloat16()
    cos = torch.rand((1, L, 128), generator=g, device=DEV).bfloat16()
    sin = torch.rand((1, L, 128), generator=g, device=DEV).bfloat16()
    w = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
    pos = torch.tensor([p0, p0 + 37, p0 + 90], dtype=torch.int32, device=DEV)
    kw = dict(num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=w, k_norm_weight=w, eps=1e-5, positions=pos)
    qa = ops.qkv_epilogue(q, k, v, cos, sin, ring=ring, deep=deep, **kw)
    qb = ops.qkv_epilogue(q, k, v, cos, sin, ring=pool, ring_table=rtab, deep=pool, deep_table=dtab, **kw)
    assert torch.equal(qa, qb)
    rk, rv = _gather(pool, rtab)
    dk, dv = _gather(pool, dtab)
    assert torch.equal(rk, ring.k) and torch.equal(rv, ring.v)
    assert torch.equal(dk, deep.k) and torch.equal(dv, deep.v)


def test_blend_paged_equals_contiguous():
    g = torch.Generator(device=DEV).manual_seed(4)
    layers, B, H, C = 3, 2, 2, 64
    R = ops.ring_tokens_for_chunk(C)
    deep = _rand_cache(g, B, H, 256)
    ring_k = torch.randn((layers, B, H, R // 32, 4096), generator=g, device=DEV).bfloat16()
    ring_v = torch.randn_like(ring_k)
    pages = layers * B * (R // 32) + B * 8 + 3
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(2)).to(DEV)
    pool = ops.PagedKV.zeros(pages, H, DEV)
    rtab = torch.stack([_scatter(ops.TiledKV(ring_k[l].contiguous(), ring_v[l].contiguous()), pool,
                                 perm[l * B * (R // 32) : (l + 1) * B * (R // 32)].view(B, R // 32)) for l in range(layers)])
    dtab = _scatter(deep, pool, perm[layers * B * (R // 32) : layers * B * (R // 32) + B * 8].view(B, 8))
    alpha = torch.rand(layers * H, generator=g, device=DEV).bfloat16().float()
    om = (1 - alpha).bfloat16().float()
    vs = (torch.rand(layers * H, generator=g, device=DEV) + 0.5).bfloat16().float()
    kw = dict(batch=B, chunk_start=2 * C, chunk_len=C, alpha=alpha, one_minus_alpha=om, vscale=vs)
    ops.blend_chunk(ring_k, ring_v, deep, **kw)
    ops.blend_chunk(pool.k, pool.v, pool, ring_table=rtab.contiguous(), deep_table=dtab, **kw)
    for l in range(layers):
        k, v = _gather(pool, rtab[l])
        assert torch.equal(k, ring_k[l]) and torch.equal(v, ring_v[l])

"""GPU parity of the split-K shared-KV decode kernel (lkv_decode_attn) and the layout kernels.

Tolerance (north star): attention outputs within max-abs 2e-2 and rel-L2 1e-3 in bf16 of the
reference path evaluated on the same bf16 inputs.  "Reference path" here is the fp64 numpy
oracle (small shapes) or the reference's torch composition + SDPA computed in fp32 on the GPU
(full shapes); both outputs are rounded to bf16 before comparison, as the reference's output is.
torch's own bf16 SDPA is also compared, within its measured deviation from the fp32 path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16, layout
from oracle import reference_path as R

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-3
DEV = "cuda"


def _bf(rng, shape, scale=1.0):
    return bf16.round_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, torch.bfloat16)


def _close(actual: torch.Tensor, expected, label: str):
    a = actual.float().cpu().numpy()
    e = np.asarray(expected, np.float64)
    ma, rl = A.max_abs(a, e), A.rel_l2(a, e)
    print(f"{label}: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= MAX_ABS and rl <= REL_L2, f"{label}: max_abs={ma} rel_l2={rl}"
    return ma, rl


def test_pack_unpack_bit_exact_against_layout_oracle():
    rng = np.random.default_rng(0)
    x = _bf(rng, (2, 3, 77, 128))
    for kind in (ops.KIND_K, ops.KIND_V):
        cache = torch.zeros((2, 3, 4, 4096), dtype=torch.bfloat16, device=DEV)
        ops.cache_pack(_t(x), cache, kind)
        want = layout.pack(x, kind, 128)
        assert np.array_equal(cache.float().cpu().numpy().view(np.uint32), want.view(np.uint32))
        back = ops.cache_unpack(cache, kind, 0, 77)
        assert np.array_equal(back.float().cpu().numpy(), x)
        # offset write into a partially filled cache
        ops.cache_pack(_t(x[:, :, :10]), cache, kind, token0=100)
        assert np.array_equal(ops.cache_unpack(cache, kind, 100, 10).float().cpu().numpy(), x[:, :, :10])


@pytest.mark.parametrize("tokens", [1, 31, 32, 33, 100, 161, 193, 1000, 8193])
@pytest.mark.parametrize("splits", [1, 3])
def test_shared_only_decode_matches_oracle(tokens, splits):
    """Block counts 1-257 per sequence: 161 and 193 tokens (6 and 7 blocks) leave two and three of
    a workgroup's four waves one block more than the last wave (the extra block is fetched with
    the wave's first one and computed after its loop), 8193 tokens one wave (257 blocks, a 1-token
    last block)."""

    rng = np.random.default_rng(tokens * 7 + splits)
    B, Hq, Hkv = 3, 8, 2
    q = _bf(rng, (B, Hq, 1, 128))
    k = _bf(rng, (B, Hkv, tokens, 128))
    v = _bf(rng, (B, Hkv, tokens, 128))
    cap = -(-tokens // 32) * 32
    cache = ops.TiledKV.zeros(B, Hkv, cap, DEV)
    ops.pack_kv(_t(k), _t(v), cache)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=DEV)
    out = ops.decode_attention(_t(q), older=cache, older_len=tokens, num_splits=splits, lse=lse)
    want, want_lse = A.attention(q, k, v)
    _close(out, bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"shared T={tokens} S={splits}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse[:, :, 0], rtol=1e-5, atol=1e-5)


def _ring_case(rng, B, Hq, Hkv, chunk, position):
    """Random final-layer history, this layer's previous/current chunks and parameters."""

    r = A.plan_regions(position, chunk)
    rec, cur = r.recent[0], r.current[0]
    deep_k, deep_v = _bf(rng, (B, Hkv, cur, 128)), _bf(rng, (B, Hkv, cur, 128))
    prev = (_bf(rng, (B, Hkv, chunk, 128)), _bf(rng, (B, Hkv, chunk, 128))) if cur else None
    n_cur = position + 1 - cur
    cur_kv = (_bf(rng, (B, Hkv, n_cur, 128)), _bf(rng, (B, Hkv, n_cur, 128)))
    logits = bf16.round_bf16(rng.standard_normal(Hkv).astype(np.float32))
    scale = bf16.round_bf16(rng.uniform(0.3, 1.3, Hkv).astype(np.float32))
    q = _bf(rng, (B, Hq, 1, 128))
    return r, deep_k, deep_v, prev, cur_kv, logits, scale, q


def _ring_inputs(r, deep_k, deep_v, prev, cur_kv, logits, scale, chunk, B, Hkv):
    """Build the kernel's caches: shared older history + the layer ring [recent blend | current]."""

    rec, cur = r.recent[0], r.current[0]
    older = ops.TiledKV.zeros(B, Hkv, max(32, -(-cur // 32) * 32), DEV)
    if cur:
        ops.pack_kv(_t(deep_k), _t(deep_v), older)
    ring = ops.TiledKV.zeros(B, Hkv, 2 * chunk, DEV)
    if cur:
        # the boundary commit materialises the recent blend once (bf16, reference op order)
        rk = A.blend_chunk_bf16(deep_k[:, :, rec:cur], prev[0], logits)
        rv = A.blend_chunk_bf16(deep_v[:, :, rec:cur], prev[1], logits, scale)
        ops.pack_kv(_t(rk), _t(rv), ring, token0=rec % (2 * chunk))
    ops.pack_kv(_t(cur_kv[0]), _t(cur_kv[1]), ring, token0=cur % (2 * chunk))
    start = torch.full((B,), rec % (2 * chunk), dtype=torch.int32, device=DEV)
    return older, ring, start


@pytest.mark.parametrize("position", [5, 63, 64, 100, 200, 300, 511])
def test_lastkv_region_decode_matches_oracle(position):
    rng = np.random.default_rng(position)
    B, Hq, Hkv, C = 2, 8, 2, 64
    r, deep_k, deep_v, prev, cur_kv, logits, scale, q = _ring_case(rng, B, Hq, Hkv, C, position)
    older, ring, start = _ring_inputs(r, deep_k, deep_v, prev, cur_kv, logits, scale, C, B, Hkv)
    rec = r.recent[0]
    out = ops.decode_attention(
        _t(q), older=older, older_len=rec, vscale=torch.from_numpy(scale).to(DEV),
        local=ring, local_len=position + 1 - rec, local_start=start, num_splits=2,
    )
    full_k, full_v = A.compose_history_bf16(deep_k, deep_v, prev and prev[0], prev and prev[1], cur_kv[0], cur_kv[1],
                                            logits, scale, C)
    want, _ = A.attention(q, full_k, full_v)
    _close(out, bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"regions p={position}")
    # the reference's torch path on the GPU, composed from the same pieces
    tdeep = (_t(deep_k), _t(deep_v)) if r.current[0] else None
    tprev = (_t(prev[0]), _t(prev[1])) if prev is not None else None
    ref32 = R.lastkv_attention(_t(q), tdeep, tprev, (_t(cur_kv[0]), _t(cur_kv[1])), torch.from_numpy(logits).to(DEV),
                               torch.from_numpy(scale).to(DEV), C, compute_dtype=torch.float32)
    _close(out, ref32[:, :, 0].float().cpu().numpy(), f"regions p={position} vs torch fp32 path")


def test_ragged_batch_with_device_lengths_and_slots():
    rng = np.random.default_rng(11)
    B, Hq, Hkv, cap = 5, 16, 4, 256
    lens = np.array([1, 255, 64, 0, 130], np.int32)
    slots = np.array([4, 0, 2, 1, 3], np.int32)
    kv = [(_bf(rng, (1, Hkv, cap, 128)), _bf(rng, (1, Hkv, cap, 128))) for _ in range(5)]
    cache = ops.TiledKV.zeros(5, Hkv, cap, DEV)
    for s in range(5):
        ops.cache_pack(_t(kv[s][0]), cache.k[s:s + 1], ops.KIND_K)
        ops.cache_pack(_t(kv[s][1]), cache.v[s:s + 1], ops.KIND_V)
    q = _bf(rng, (B, Hq, 1, 128))
    out = ops.decode_attention(_t(q), older=cache, older_len=torch.from_numpy(lens).to(DEV),
                               older_slot=torch.from_numpy(slots).to(DEV), num_splits=3)
    for b in range(B):
        s, n = slots[b], lens[b]
        if n == 0:
            assert torch.count_nonzero(out[b]) == 0
            continue
        want, _ = A.attention(q[b:b + 1], kv[s][0][:, :, :n], kv[s][1][:, :, :n])
        _close(out[b:b + 1], bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"ragged b={b} n={n}")
    # an out-of-range slot reads nothing and yields zeros instead of faulting
    bad = torch.tensor([7, 0, 2, 1, 3], dtype=torch.int32, device=DEV)
    out = ops.decode_attention(_t(q), older=cache, older_len=torch.from_numpy(lens).to(DEV), older_slot=bad)
    assert torch.count_nonzero(out[0]) == 0


@pytest.fixture(scope="module")
def config2():
    """q [32, 32, 1, 128], one shared K/V [32, 8, 8192, 128], N(0, 1) bf16."""

    g = torch.Generator(device=DEV).manual_seed(2)
    k = torch.randn((32, 8, 8192, 128), generator=g, device=DEV).bfloat16()
    v = torch.randn((32, 8, 8192, 128), generator=g, device=DEV).bfloat16()
    q = torch.randn((32, 32, 1, 128), generator=g, device=DEV).bfloat16()
    cache = ops.TiledKV.zeros(32, 8, 8192, DEV)
    ops.pack_kv(k, v, cache)
    return q, k, v, cache


def test_config2_full_size_matches_reference_sdpa(config2):
    q, k, v, cache = config2
    out = ops.decode_attention(q, older=cache, older_len=8192)
    ref32 = R.sdpa_bottom_right(q, k, v, compute_dtype=torch.float32)[:, :, 0]
    _close(out, ref32.float().cpu().numpy(), "config2 vs fp32 SDPA")
    ref16 = R.sdpa_bottom_right(q, k, v)[:, :, 0]
    sdpa_dev = A.rel_l2(ref16.float().cpu().numpy(), ref32.float().cpu().numpy())
    ours = A.rel_l2(out.float().cpu().numpy(), ref16.float().cpu().numpy())
    print(f"config2: torch bf16 SDPA vs fp32 rel_l2={sdpa_dev:.3e}; ours vs torch bf16 rel_l2={ours:.3e}", flush=True)
    assert ours <= max(REL_L2, 1.5 * sdpa_dev)
    assert A.max_abs(out.float().cpu().numpy(), ref16.float().cpu().numpy()) <= MAX_ABS


def test_config2_two_token_call_on_decode_kernel_matches_tile_kernel(config2):
    """Full size: two query tokens per sequence over the 1 GiB shared cache (no causal part: the
    cache is all older history) on the decode kernel's (token, head) columns with non-temporal
    loads, against the same call on the MFMA tile kernel."""

    q1, _, _, cache = config2
    q = torch.stack([q1[:, :, 0], q1[:, :, 0].flip(1).contiguous()], 1)  # [32, 2, 32, 128]
    got = ops.prefill_attention(q, older=cache, older_len=8192, causal=False)
    tile = ops.prefill_attention(q, older=cache, older_len=8192, causal=False, tile_waves=4)
    _close(got, tile.float().cpu().numpy(), "config2 two-token call: decode kernel vs tile kernel")
    one = ops.decode_attention(q1, older=cache, older_len=8192, num_splits=1)
    assert torch.equal(got[:, 0], one), "token 0 equals the one-token decode call"


def test_config2_split_invariance_and_power_of_two_vscale_linearity(config2):
    q, _, _, cache = config2
    base = ops.decode_attention(q, older=cache, older_len=8192, num_splits=1)
    for splits in (2, 8, 64):
        other = ops.decode_attention(q, older=cache, older_len=8192, num_splits=splits)
        _close(other, base.float().cpu().numpy(), f"config2 splits={splits} vs 1")
    # s = 2 is exact in bf16 and commutes with every fp32 rounding: out(2V) == 2 out(V) bitwise
    two = torch.full((8,), 2.0, dtype=torch.float32, device=DEV)
    scaled = ops.decode_attention(q, older=cache, older_len=8192, vscale=two, num_splits=1)
    assert torch.equal(scaled, base * 2)
    # the 1 GiB cache takes non-temporal K/V loads by default; the default cache policy gives the same bits
    for hint in (1, 2):
        assert torch.equal(ops.decode_attention(q, older=cache, older_len=8192, num_splits=1, kv_cache_hint=hint), base)


@pytest.mark.parametrize("tokens", [1, 4, 40])
@pytest.mark.parametrize("bf16_scale", [True, False])
def test_older_vscale_equals_prescaled_cache_bitwise(tokens, bf16_scale):
    """The older segment's V scale gives the same bits as a cache whose V holds bf16(V * s)
    (torch: fp32 product, one round to bf16), for bf16-valued and other fp32 scales; 1 and 4
    tokens run the decode kernel, 40 tokens the tile kernel's V pre-pass.  The local segment
    stays unscaled."""

    rng = np.random.default_rng(11 + tokens)
    B, Hq, Hkv, T0, n1 = 3, 16, 4, 1000, 77
    ok, ov = _bf(rng, (B, Hkv, T0, 128)), _bf(rng, (B, Hkv, T0, 128), 3.0)
    lk, lv = _bf(rng, (B, Hkv, n1, 128)), _bf(rng, (B, Hkv, n1, 128))
    s = rng.uniform(0.3, 1.7, Hkv).astype(np.float32)
    s[0] = 1.0
    if bf16_scale:
        s = bf16.round_bf16(s)
    else:
        s[1:] = np.where(bf16.round_bf16(s[1:]) == s[1:], s[1:] * (1 + 2.0 ** -12), s[1:])
        assert not np.any(bf16.round_bf16(s[1:]) == s[1:])
    older = ops.TiledKV.zeros(B, Hkv, 1024, DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    vs = torch.from_numpy(s).to(DEV)
    pre = ops.TiledKV(older.k.clone(), (older.v.float() * vs.view(1, Hkv, 1, 1)).bfloat16())
    ring = ops.TiledKV.zeros(B, Hkv, 128, DEV)
    ops.pack_kv(_t(lk), _t(lv), ring)
    seg = dict(older_len=T0, local=ring, local_len=n1)
    if tokens == 1:
        q = _t(_bf(rng, (B, Hq, 128)))
        got = ops.decode_attention(q, older=older, vscale=vs, num_splits=2, **seg)
        want = ops.decode_attention(q, older=pre, num_splits=2, **seg)
    else:
        q = _t(_bf(rng, (B, tokens, Hq, 128)))
        got = ops.prefill_attention(q, older=older, vscale=vs, causal=True, **seg)
        want = ops.prefill_attention(q, older=pre, causal=True, **seg)
    assert torch.equal(got, want)


def _two_segments(rng, B, Hkv, T0, n1, start, ring_blocks):
    """Older segment of T0 tokens and a ring of ring_blocks blocks holding n1 tokens from ring token
    `start` (wrapping), with a bf16 older V scale; returns the caches and the composed fp32 K/V the
    kernel must attend to (older V as bf16(V * s))."""

    ok, ov = _bf(rng, (B, Hkv, T0, 128)), _bf(rng, (B, Hkv, T0, 128))
    lk, lv = _bf(rng, (B, Hkv, n1, 128)), _bf(rng, (B, Hkv, n1, 128))
    s = bf16.round_bf16(rng.uniform(0.4, 1.4, Hkv).astype(np.float32))
    older = ops.TiledKV.zeros(B, Hkv, max(32, -(-T0 // 32) * 32), DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    ring = ops.TiledKV.zeros(B, Hkv, ring_blocks * 32, DEV)
    R = ring_blocks * 32
    first = min(n1, R - start)
    ops.pack_kv(_t(lk[:, :, :first]), _t(lv[:, :, :first]), ring, token0=start)
    if first < n1:
        ops.pack_kv(_t(lk[:, :, first:]), _t(lv[:, :, first:]), ring, token0=0)
    k = np.concatenate([ok, lk], 2)
    v = np.concatenate([bf16.mul(ov, s.reshape(1, -1, 1, 1)), lv], 2)
    seg = dict(older=older, older_len=T0, vscale=torch.from_numpy(s).to(DEV), local=ring, local_len=n1,
               local_start=start)
    return seg, k, v


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (6, 2), (7, 1), (16, 2), (32, 2), (48, 3), (24, 1), (64, 2), (64, 1)])
@pytest.mark.parametrize("splits", [1, 4])
def test_decode_gqa_group_sizes(Hq, Hkv, splits):
    """GQA groups 1 (MHA) to 64 (above 16 the multi-column instances: 24, 32, 64), odd and not
    powers of two, over an older segment with V scale and a wrapping ring segment; query head h
    reads kv head h // G."""

    rng = np.random.default_rng(Hq * 31 + Hkv * 7 + splits)
    B = 2
    seg, k, v = _two_segments(rng, B, Hkv, T0=203, n1=150, start=90, ring_blocks=7)
    q = _bf(rng, (B, Hq, 1, 128))
    lse = torch.empty((B, Hq), dtype=torch.float32, device=DEV)
    out = ops.decode_attention(_t(q), num_splits=splits, lse=lse, **seg)
    want, want_lse = A.attention(q, k, v)
    _close(out, bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"decode G={Hq // Hkv} Hkv={Hkv} S={splits}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse[:, :, 0], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("L,Hq,Hkv", [(40, 16, 1), (17, 6, 2), (9, 3, 1), (70, 20, 4)])
def test_prefill_gqa_group_sizes_causal(L, Hq, Hkv):
    """Prefill rows are (token, head) pairs of one GQA group: groups 16, 3, 5, with the causal
    limit of each query token over the local segment (its last L tokens are the queries' own)."""

    rng = np.random.default_rng(L * 13 + Hq + Hkv)
    B = 2
    seg, k, v = _two_segments(rng, B, Hkv, T0=96, n1=L + 45, start=20, ring_blocks=5)
    q = _bf(rng, (B, L, Hq, 128))
    lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
    out = ops.prefill_attention(_t(q), causal=True, lse=lse, **seg)
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=True)
    _close(out, bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32)), f"prefill G={Hq // Hkv} L={L}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("splits", [1, 3])
def test_decode_kv_cache_hint_does_not_change_results(splits):
    """Default and non-temporal K/V loads (and the automatic choice) give the same bits, and
    both match the oracle; an unknown hint is rejected."""

    rng = np.random.default_rng(40 + splits)
    B, Hq, Hkv = 3, 16, 4
    seg, k, v = _two_segments(rng, B, Hkv, T0=517, n1=77, start=150, ring_blocks=6)
    q = _bf(rng, (B, Hq, 1, 128))
    outs, lses = [], []
    for hint in (0, 1, 2):
        lse = torch.empty((B, Hq), dtype=torch.float32, device=DEV)
        outs.append(ops.decode_attention(_t(q), num_splits=splits, lse=lse, kv_cache_hint=hint, **seg))
        lses.append(lse)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    assert torch.equal(lses[0], lses[1]) and torch.equal(lses[1], lses[2])
    want, want_lse = A.attention(q, k, v)
    _close(outs[2], bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"decode nt S={splits}")
    np.testing.assert_allclose(lses[2].cpu().numpy(), want_lse[:, :, 0], rtol=1e-4, atol=1e-4)
    with pytest.raises(RuntimeError, match="kv_cache_hint"):
        ops.decode_attention(_t(q), num_splits=splits, kv_cache_hint=3, **seg)


@pytest.mark.parametrize("L,Hq,Hkv,causal,B", [(2, 32, 8, True, 2), (4, 8, 2, True, 3), (3, 15, 3, False, 1),
                                              (16, 16, 16, True, 2), (1, 64, 4, True, 2), (5, 6, 2, True, 1),
                                              (8, 32, 8, True, 1), (11, 6, 2, False, 2), (32, 8, 8, True, 1),
                                              (16, 32, 8, True, 1), (13, 12, 3, False, 2), (40, 8, 8, True, 1),
                                              (2, 64, 2, True, 1), (1, 64, 1, True, 2)])
def test_short_prefill_on_decode_kernel(L, Hq, Hkv, causal, B):
    """Prefill calls of at most 64 query rows per kv head run on the decode kernel, one score column
    per (token, head) with its own causal limit, in one or two 16-column groups per wave (two wave
    pairs splitting the columns above 32): against the oracle
    (older V scale, a wrapping ring, split partials combined per (token, head) when the batch is
    small) and against the tile kernel."""

    rng = np.random.default_rng(L * 100 + Hq + B)
    seg, k, v = _two_segments(rng, B, Hkv, T0=203, n1=L + 150, start=150, ring_blocks=8)
    q = _bf(rng, (B, L, Hq, 128))
    lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
    out = ops.prefill_attention(_t(q), causal=causal, lse=lse, **seg)
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
    want_out = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    _close(out, want_out, f"short prefill L={L} G={Hq // Hkv} B={B}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    tile = ops.prefill_attention(_t(q), causal=causal, tile_waves=4, **seg)
    _close(tile, out.float().cpu().numpy(), f"short prefill tile vs decode kernel L={L}")


# block-maximum jumps (exp2 units) along each wave's blocks: the decode kernel raises its softmax
# reference only when a block maximum exceeds it by more than 8; jumps just below, at and above that,
# a far one and a second raise after a first
LAZY_PATTERNS = {
    "below 7.5": [0.0, 7.5, 7.0, 7.5],
    "at 8.0": [0.0, 8.0, 3.0, 8.0],
    "above 8.0625": [0.0, 8.0625, 1.0, 8.0625],
    "8.5": [0.0, 8.5, 4.0, -2.0],
    "far 20": [0.0, 20.0, 5.0, 19.5],
    "second raise": [0.0, 8.5, 17.25, 17.0],
}


def _lazy_case(pattern, blocks, Hq, Hkv, seed):
    """K whose dim 0 carries the scores (q = e_0, sm_scale = ln 2: scores in exp2 units equal the K
    values): the block with index j peaks at pattern[(j // 4) % 4] (each of the 4 waves of a
    decode workgroup walks blocks w, w + 4, ..., so every wave meets the jumps in order), its other
    tokens below it; bf16 values, so every product is exact."""

    rng = np.random.default_rng(seed)
    T = blocks * 32
    k = np.zeros((1, Hkv, T, 128), np.float32)
    for h in range(Hkv):
        for j in range(blocks):
            top = pattern[(j // 4) % len(pattern)] + 0.25 * h
            vals = top - rng.uniform(0.5, 12.0, 32)
            vals[rng.integers(0, 32)] = top
            k[0, h, j * 32:(j + 1) * 32, 0] = vals
    k = bf16.round_bf16(k)
    v = _bf(rng, (1, Hkv, T, 128))
    q = np.zeros((1, Hq, 1, 128), np.float32)
    q[..., 0] = 1.0
    return q, k, v


@pytest.mark.parametrize("name", list(LAZY_PATTERNS))
def test_decode_lazy_rescale_threshold_regimes(name):
    """The decode kernel's lazy softmax reference with constructed block-maximum jumps of 7.5, 8,
    8.0625, 8.5 and 20 exp2 units and a second raise after a first, through one and five key
    splits and a short prefill call on the decode kernel, against the fp64 oracle."""

    Hq, Hkv, blocks = 8, 2, 80
    q, k, v = _lazy_case(LAZY_PATTERNS[name], blocks, Hq, Hkv, seed=len(name))
    sm = float(np.log(2.0))  # scale * log2(e) = 1: exp2 units = raw scores
    cache = ops.TiledKV.zeros(1, Hkv, blocks * 32, DEV)
    ops.pack_kv(_t(k), _t(v), cache)
    want, want_lse = A.attention(q, k, v, scale=sm)
    for splits in (1, 5):
        lse = torch.empty((1, Hq), dtype=torch.float32, device=DEV)
        out = ops.decode_attention(_t(q), older=cache, older_len=blocks * 32, num_splits=splits, sm_scale=sm, lse=lse)
        _close(out, bf16.round_bf16(want[:, :, 0].astype(np.float32)), f"lazy {name} splits={splits}")
        np.testing.assert_allclose(lse.cpu().numpy(), want_lse[:, :, 0], rtol=1e-5, atol=1e-4)
    # two query tokens (8 score columns) on the decode kernel: the older segment is fully visible
    q2 = np.concatenate([q, q * 0.5], 2).transpose(0, 2, 1, 3)  # [1, 2, Hq, 128]
    out = ops.prefill_attention(_t(q2), older=cache, older_len=blocks * 32, causal=True, sm_scale=sm)
    want2, _ = A.attention(q2.transpose(0, 2, 1, 3), k, v, scale=sm)
    _close(out, bf16.round_bf16(want2.transpose(0, 2, 1, 3).astype(np.float32)), f"lazy {name} short prefill")

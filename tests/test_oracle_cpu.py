"""Pins the CPU oracle against library routines, closed forms and brute force (no GPU)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import attention as A
from oracle import bf16, layout
from oracle import reference_path as R


# ------------------------------------------------------------------ bf16 emulation
def test_round_bf16_matches_torch_on_random_ties_overflow_and_nan():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
        # exact ties between two bf16 values, both parities
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([3.4e38, -3.4e38, 1e-45, -0.0, 0.0, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    actual = bf16.round_bf16(x)
    assert np.array_equal(actual.view(np.uint32), expected.view(np.uint32))
    nan = bf16.round_bf16(np.array([np.nan], np.float32))
    assert np.isnan(nan).all()


def test_bf16_ops_match_torch_elementwise():
    rng = np.random.default_rng(1)
    a = bf16.round_bf16(rng.standard_normal(5000).astype(np.float32))
    b = bf16.round_bf16(rng.standard_normal(5000).astype(np.float32) * 1e-3)
    ta, tb = torch.from_numpy(a).bfloat16(), torch.from_numpy(b).bfloat16()
    assert np.array_equal(bf16.mul(a, b), (ta * tb).float().numpy())
    assert np.array_equal(bf16.add(a, b), (ta + tb).float().numpy())
    assert np.array_equal(bf16.rsub(a), (1 - ta).float().numpy())


# ------------------------------------------------------------------ region planning
@pytest.mark.parametrize("chunk", [1, 3, 4, 32])
def test_plan_regions_enumeration(chunk):
    for p in range(5 * chunk + 3):
        r = A.plan_regions(p, chunk)
        seen = p + 1
        assert r.older[0] == 0 and r.older[1] == r.recent[0] and r.recent[1] == r.current[0]
        assert r.current[1] == seen
        # cache invariants of the reference test (test_llm_inference.py:118-121), measured
        # after the token at p was processed: deep holds the completed chunks
        deep_after = seen // chunk * chunk
        cur_len_after = seen % chunk
        assert deep_after in (r.current[0], r.current[1])
        assert cur_len_after == (r.current[1] - r.current[0]) % chunk
        # the local window (recent + current) never exceeds two chunks
        assert r.current[1] - r.recent[0] <= 2 * chunk
        # brute force: token j's region by chunk index difference
        for j in range(seen):
            diff = p // chunk - j // chunk
            region = "current" if diff == 0 else "recent" if diff == 1 else "older"
            lo, hi = getattr(r, region)
            assert lo <= j < hi


# ------------------------------------------------------------------ attention
def _brute_attention(q, k, v, scale, causal):
    B, Hq, Lq, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    out = np.zeros((B, Hq, Lq, D))
    lse = np.full((B, Hq, Lq), -np.inf)
    for b in range(B):
        for h in range(Hq):
            g = h // (Hq // Hkv)
            for i in range(Lq):
                scores = []
                for j in range(S):
                    if causal and j > i + S - Lq:
                        continue
                    scores.append((j, sum(q[b, h, i, d] * k[b, g, j, d] for d in range(D)) * scale))
                if not scores:
                    continue
                m = max(s for _, s in scores)
                w = [(j, math.exp(s - m)) for j, s in scores]
                total = sum(x for _, x in w)
                for d in range(D):
                    out[b, h, i, d] = sum(x * v[b, g, j, d] for j, x in w) / total
                lse[b, h, i] = m + math.log(total)
    return out, lse


def test_attention_matches_brute_force_and_torch_float64():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 4, 3, 5))
    k = rng.standard_normal((2, 2, 7, 5))
    v = rng.standard_normal((2, 2, 7, 5))
    for causal in (False, True):
        out, lse = A.attention(q, k, v, scale=0.37, causal_bottom_right=causal)
        bo, bl = _brute_attention(q, k, v, 0.37, causal)
        np.testing.assert_allclose(out, bo, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse, bl, rtol=1e-12, atol=1e-12)
    # library routine: torch SDPA in float64 (no mask), GQA expanded
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk.repeat_interleave(2, 1), tv.repeat_interleave(2, 1), scale=0.37)
    out, _ = A.attention(q, k, v, scale=0.37)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_attention_rows_without_keys_are_zero_with_minus_inf_lse():
    q = np.ones((1, 1, 3, 2))
    k = np.ones((1, 1, 1, 2))
    v = np.ones((1, 1, 1, 2))
    # bottom-right mask with Lq > S: first two queries see nothing
    out, lse = A.attention(q, k, v, causal_bottom_right=True)
    assert np.all(out[0, 0, :2] == 0) and np.all(np.isneginf(lse[0, 0, :2]))
    assert np.allclose(out[0, 0, 2], 1.0)


def test_merge_states_equals_attention_over_union():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 2, 4, 8))
    k = rng.standard_normal((1, 2, 11, 8))
    v = rng.standard_normal((1, 2, 11, 8))
    full, full_lse = A.attention(q, k, v)
    a, la = A.attention(q, k[:, :, :6], v[:, :, :6])
    b, lb = A.attention(q, k[:, :, 6:], v[:, :, 6:])
    m, lm = A.merge_states(a, la, b, lb)
    np.testing.assert_allclose(m, full, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(lm, full_lse, rtol=1e-12)
    # an empty source (LSE -inf) leaves the local state unchanged (fastpath.py:717-718)
    m2, lm2 = A.merge_states(np.zeros_like(b), np.full_like(lb, -np.inf), b, lb)
    np.testing.assert_allclose(m2, b, rtol=0, atol=0)
    np.testing.assert_allclose(lm2, lb, rtol=0, atol=0)


def test_vscale_linearity_and_lse_invariance():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 4, 1, 16))
    k = rng.standard_normal((1, 1, 40, 16))
    v = rng.standard_normal((1, 1, 40, 16))
    o1, l1 = A.attention(q, k, v)
    o2, l2 = A.attention(q, k, 0.37 * v)
    np.testing.assert_allclose(o2, 0.37 * o1, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(l2, l1, rtol=0, atol=0)


# ------------------------------------------------------------------ history composition
def _bf(rng, shape, scale=1.0):
    return bf16.round_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def _torch_compose(deep, prev, cur, logits, scale, chunk):
    t = lambda x: torch.from_numpy(x).bfloat16()
    full_k, full_v = R.compose((t(deep[0]), t(deep[1])) if deep[0].shape[2] else None,
                               (t(prev[0]), t(prev[1])) if prev is not None else None,
                               (t(cur[0]), t(cur[1])), torch.from_numpy(logits).bfloat16(),
                               torch.from_numpy(scale).bfloat16(), chunk)
    return full_k.float().numpy(), full_v.float().numpy()


@pytest.mark.parametrize("chunks_done", [0, 1, 3])
def test_compose_history_bf16_matches_torch_op_for_op(chunks_done):
    rng = np.random.default_rng(10 + chunks_done)
    C, B, H, D = 8, 2, 3, 16
    deep = (_bf(rng, (B, H, chunks_done * C, D)), _bf(rng, (B, H, chunks_done * C, D)))
    prev = (_bf(rng, (B, H, C, D)), _bf(rng, (B, H, C, D))) if chunks_done else None
    cur = (_bf(rng, (B, H, 5, D)), _bf(rng, (B, H, 5, D)))
    logits = bf16.round_bf16(rng.standard_normal(H).astype(np.float32))
    scale = bf16.round_bf16(rng.uniform(0.3, 1.3, H).astype(np.float32))
    k, v = A.compose_history_bf16(deep[0], deep[1], prev and prev[0], prev and prev[1], cur[0], cur[1], logits, scale, C)
    tk, tv = _torch_compose(deep, prev, cur, logits, scale, C)
    assert np.array_equal(k.view(np.uint32), tk.view(np.uint32))
    assert np.array_equal(v.view(np.uint32), tv.view(np.uint32))


def test_compose_history_limits():
    rng = np.random.default_rng(5)
    C, B, H, D = 4, 1, 2, 8
    deep = (_bf(rng, (B, H, 2 * C, D)), _bf(rng, (B, H, 2 * C, D)))
    prev = (_bf(rng, (B, H, C, D)), _bf(rng, (B, H, C, D)))
    cur = (_bf(rng, (B, H, 2, D)), _bf(rng, (B, H, 2, D)))
    ones = np.ones(H, np.float32)
    # alpha -> 1: the recent chunk is the shared one (V scaled)
    k, v = A.compose_history_bf16(*deep, *prev, *cur, np.full(H, 60.0, np.float32), ones, C)
    assert np.array_equal(k[:, :, C:2 * C], deep[0][:, :, C:])
    assert np.array_equal(v[:, :, C:2 * C], deep[1][:, :, C:])
    # alpha -> 0: the recent chunk is the layer's own
    k, v = A.compose_history_bf16(*deep, *prev, *cur, np.full(H, -60.0, np.float32), ones, C)
    assert np.array_equal(k[:, :, C:2 * C], prev[0]) and np.array_equal(v[:, :, C:2 * C], prev[1])
    # s = 1 leaves older V untouched; older K is always the shared K
    assert np.array_equal(v[:, :, :C], deep[1][:, :, :C]) and np.array_equal(k[:, :, :C], deep[0][:, :, :C])
    # blend_chunk_bf16 is the recent slice of the composition
    logits = np.array([0.3, -1.1], np.float32)
    s = np.array([0.5, 1.25], np.float32)
    k, v = A.compose_history_bf16(*deep, *prev, *cur, logits, s, C)
    assert np.array_equal(A.blend_chunk_bf16(deep[0][:, :, C:], prev[0], logits), k[:, :, C:2 * C])
    assert np.array_equal(A.blend_chunk_bf16(deep[1][:, :, C:], prev[1], logits, s), v[:, :, C:2 * C])


def test_reference_path_matches_numpy_oracle_and_degenerates_to_gqa():
    rng = np.random.default_rng(6)
    C, B, Hq, H, D = 4, 2, 4, 2, 8
    deep = (rng.standard_normal((B, H, 2 * C, D)).astype(np.float32), rng.standard_normal((B, H, 2 * C, D)).astype(np.float32))
    prev = (rng.standard_normal((B, H, C, D)).astype(np.float32), rng.standard_normal((B, H, C, D)).astype(np.float32))
    cur = (rng.standard_normal((B, H, 3, D)).astype(np.float32), rng.standard_normal((B, H, 3, D)).astype(np.float32))
    logits = rng.standard_normal(H).astype(np.float32)
    s = rng.uniform(0.5, 1.5, H).astype(np.float32)
    q = rng.standard_normal((B, Hq, 2, D)).astype(np.float32)
    t = lambda x: torch.from_numpy(x).double()
    got = R.lastkv_attention(t(q), (t(deep[0]), t(deep[1])), (t(prev[0]), t(prev[1])), (t(cur[0]), t(cur[1])),
                             t(logits), t(s), C).numpy()
    # fp64 oracle with exact (unrounded) composition
    a = A.sigmoid(logits).reshape(1, -1, 1, 1)
    sc = s.reshape(1, -1, 1, 1).astype(np.float64)
    full_k = np.concatenate([deep[0][:, :, :C], a * deep[0][:, :, C:] + (1 - a) * prev[0], cur[0]], axis=2)
    full_v = np.concatenate([sc * deep[1][:, :, :C], a * sc * deep[1][:, :, C:] + (1 - a) * prev[1], cur[1]], axis=2)
    want, _ = A.attention(q, full_k, full_v, causal_bottom_right=True)
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)
    # no completed chunk: plain causal GQA attention
    got = R.lastkv_attention(t(q), None, None, (t(cur[0]), t(cur[1])), t(logits), t(s), C).numpy()
    ref = F.scaled_dot_product_attention(t(q), t(cur[0]).repeat_interleave(2, 1), t(cur[1]).repeat_interleave(2, 1),
                                         attn_mask=torch.tensor([[True, True, False], [True, True, True]]))
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ tiled layout
def test_layout_maps_are_bijections_and_operand_loads_are_contiguous():
    w, d = np.meshgrid(np.arange(32), np.arange(128), indexing="ij")
    for fn in (layout.k_offset, layout.v_offset):
        assert np.array_equal(np.sort(fn(w, d).ravel()), np.arange(4096))
    # decode kernel K loads: lane (r = l % 16, g = l // 16) reads dims 32*kb + 8g .. +8 of token
    # tau(u, r) = 8*(r//4) + 4u + r%4; the 64 lanes of one (u, kb) load cover one 1 KiB run
    for u in range(2):
        for kb in range(4):
            starts = []
            for lane in range(64):
                r, g = lane % 16, lane // 16
                tok = 8 * (r // 4) + 4 * u + r % 4
                offs = layout.k_offset(tok, 32 * kb + 8 * g + np.arange(8))
                assert np.array_equal(offs, offs[0] + np.arange(8))
                starts.append(int(offs[0]))
            assert sorted(starts) == list(range(min(starts), min(starts) + 512, 8))
    # V loads: lane (n, g) reads tokens 8g..8g+7 of dim 16*nb + n
    for nb in range(8):
        starts = []
        for lane in range(64):
            n, g = lane % 16, lane // 16
            offs = layout.v_offset(8 * g + np.arange(8), 16 * nb + n)
            assert np.array_equal(offs, offs[0] + np.arange(8))
            starts.append(int(offs[0]))
        assert sorted(starts) == list(range(min(starts), min(starts) + 512, 8))


def test_layout_pack_unpack_round_trip():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 3, 77, 128)).astype(np.float32)
    for kind in (0, 1):
        c = layout.pack(x, kind, 96)
        assert np.array_equal(layout.unpack(c, kind, 0, 77), x)
        assert np.array_equal(layout.unpack(c, kind, 40, 30), x[:, :, 40:70])

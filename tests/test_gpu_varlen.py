"""Ragged (varlen) calls: one attention and one epilogue launch for a step whose sequences carry
different numbers of query tokens (cu_seqlens), the reference's single FA3 varlen call per layer
(vllm/src/lastkv/vllm/backends/rmarin_flashinfer/fastpath.py:643-648).

1. ``prefill_attention(cu_seqlens_q=...)`` over sequences of 0-300 query tokens (every column class
   of the decode kernel and the tile kernel in one call) equals the per-sequence uniform calls bit
   for bit when both fix the decode kernel's split count, and is within the north-star bar of the
   fp64 oracle with the automatic split count (contiguous and paged caches, causal and
   bidirectional, V scale and output scale).
2. ``qkv_epilogue(cu_seqlens=...)`` equals per-sequence calls bit for bit (normalised queries,
   ring and shared-store contents) in both rounding contracts, per-token and block forms.
3. The serving path's mixed step (31 decode rows + one 1024-token prefill row + one 7-token row)
   through ``LastKVServingModel`` against the oracle model run per sequence.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from lastkv_amd.serving import LastKVServingModel
from oracle import attention as A
from oracle import bf16

from test_gpu_decode import MAX_ABS, REL_L2, _bf, _t
from test_gpu_llm import _no_worse_than_reference_bf16, _o16, _o32, _tiny

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ragged_case(rng, lengths, Hkv, G, paged, causal):
    """Per sequence b: an older segment of T0_b tokens (slot b of a tiled store, or pages of a pool)
    and a ring holding n1_b >= L_b tokens from a random start; returns the kernel segments, the
    composed K / V per sequence (older V as bf16(V * s)) and the lengths."""

    B = len(lengths)
    ring_blocks = max(-(-max(lengths) // 32) + 2, 6)
    R = ring_blocks * 32
    T0 = [int(rng.integers(0, 700)) for _ in range(B)]
    n1 = [int(rng.integers(max(L, 1), R + 1)) for L in lengths]
    start = [int(rng.integers(0, R)) for _ in range(B)]
    cap = max(32, -(-max(T0) // 32) * 32)
    s = bf16.round_bf16(rng.uniform(0.4, 1.4, Hkv).astype(np.float32))
    older = ops.TiledKV.zeros(B, Hkv, cap, DEV)
    ring = ops.TiledKV.zeros(B, Hkv, R, DEV)
    ks, vs = [], []
    for b in range(B):
        ok, ov = _bf(rng, (1, Hkv, T0[b], 128)), _bf(rng, (1, Hkv, T0[b], 128))
        lk, lv = _bf(rng, (1, Hkv, n1[b], 128)), _bf(rng, (1, Hkv, n1[b], 128))
        if T0[b]:
            ops.pack_kv(_t(ok), _t(ov), ops.TiledKV(older.k[b:b + 1], older.v[b:b + 1]))
        one = ops.TiledKV(ring.k[b:b + 1], ring.v[b:b + 1])
        first = min(n1[b], R - start[b])
        ops.pack_kv(_t(lk[:, :, :first]), _t(lv[:, :, :first]), one, token0=start[b])
        if first < n1[b]:
            ops.pack_kv(_t(lk[:, :, first:]), _t(lv[:, :, first:]), one, token0=0)
        ks.append(np.concatenate([ok, lk], 2))
        vs.append(np.concatenate([bf16.mul(ov, s.reshape(1, -1, 1, 1)), lv], 2))
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    seg = dict(older_len=i32(T0), vscale=torch.from_numpy(s).to(DEV), local_len=i32(n1), local_start=i32(start))
    if paged:
        # the same blocks as pages of one head-major pool: older pages first, then the rings
        ob, rb = cap // 32, ring_blocks
        pool = ops.PagedKV.zeros(B * (ob + rb) + 1, Hkv, DEV)
        perm = torch.randperm(B * (ob + rb), generator=torch.Generator().manual_seed(3)).to(DEV, torch.int32)
        otab = perm[:B * ob].view(B, ob).contiguous()
        rtab = perm[B * ob:].view(B, rb).contiguous()
        for b in range(B):
            for j in range(ob):
                pool.k[:, otab[b, j]] = older.k[b, :, j]
                pool.v[:, otab[b, j]] = older.v[b, :, j]
            for j in range(rb):
                pool.k[:, rtab[b, j]] = ring.k[b, :, j]
                pool.v[:, rtab[b, j]] = ring.v[b, :, j]
        seg.update(older=pool, older_table=otab, local=pool, local_table=rtab, local_ring_blocks=rb)
    else:
        seg.update(older=older, local=ring)
    return seg, ks, vs, (T0, n1, start)


def _one(seg, b, meta):
    """Segment arguments of sequence b alone (host-constant lengths)."""

    T0, n1, start = meta
    one = dict(vscale=seg["vscale"], older_len=T0[b], local_len=n1[b], local_start=start[b])
    if "older_table" in seg:
        one.update(older=seg["older"], older_table=seg["older_table"][b:b + 1], local=seg["local"],
                   local_table=seg["local_table"][b:b + 1], local_ring_blocks=seg["local_ring_blocks"])
    else:
        sl = lambda c: ops.TiledKV(c.k[b:b + 1], c.v[b:b + 1])
        one.update(older=sl(seg["older"]), local=sl(seg["local"]))
    return one


LENGTHS = [1, 0, 5, 16, 17, 1, 33, 70, 200, 3, 300, 1]


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("causal", [True, False])
def test_ragged_prefill_equals_per_sequence_calls_and_oracle(paged, causal):
    rng = np.random.default_rng(41 + 2 * paged + causal)
    Hkv, G = 2, 4
    Hq = Hkv * G
    seg, ks, vs, meta = _ragged_case(rng, LENGTHS, Hkv, G, paged, causal)
    cu = np.concatenate([[0], np.cumsum(LENGTHS)]).astype(np.int32)
    T = int(cu[-1])
    q = _bf(rng, (T, Hq, 128))
    cu_t = torch.from_numpy(cu).to(DEV)
    out_scale = torch.from_numpy(bf16.round_bf16(rng.uniform(0.5, 1.5, Hkv).astype(np.float32))).to(DEV)
    label = f"paged={paged} causal={causal}"
    for splits in (1, 0):
        lse = torch.empty((T, Hq), dtype=torch.float32, device=DEV)
        out = ops.prefill_attention(_t(q), causal=causal, cu_seqlens_q=cu_t, max_seqlen_q=max(LENGTHS), lse=lse,
                                    num_splits=splits, **seg)
        scaled = ops.prefill_attention(_t(q), causal=causal, cu_seqlens_q=cu_t, max_seqlen_q=max(LENGTHS),
                                       num_splits=splits, out_scale=out_scale, **seg)
        worst = 0.0
        for b, L in enumerate(LENGTHS):
            if L == 0:
                continue
            rows = slice(int(cu[b]), int(cu[b + 1]))
            want, want_lse = A.attention(q[rows].transpose(1, 0, 2)[None], ks[b], vs[b], causal_bottom_right=causal)
            want = bf16.round_bf16(want[0].transpose(1, 0, 2).astype(np.float32))
            got = out[rows].float().cpu().numpy()
            ma, rl = A.max_abs(got, want), A.rel_l2(got, want)
            worst = max(worst, rl)
            assert ma <= MAX_ABS and rl <= REL_L2, f"{label} splits={splits} sequence {b} (L={L}): {ma} {rl}"
            np.testing.assert_allclose(lse[rows].cpu().numpy(), want_lse[0].T, rtol=1e-4, atol=1e-4)
            # the output scale is bf16(bf16(o) * s) of the unscaled rows
            s_q = out_scale.repeat_interleave(G)[None, :, None]
            assert torch.equal(scaled[rows], (out[rows].float() * s_q).bfloat16()), f"{label} out_scale sequence {b}"
            if splits == 1:  # the per-sequence uniform call, same arithmetic
                alone = ops.prefill_attention(_t(q[rows][None]), causal=causal, num_splits=1, **_one(seg, b, meta))
                assert torch.equal(out[rows], alone[0]), f"{label}: sequence {b} (L={L}) differs from its own call"
        print(f"{label} splits={splits}: worst rel_l2 {worst:.2e} over {len(LENGTHS)} sequences", flush=True)


def test_ragged_prefill_forced_tiles_and_short_only_calls():
    """tile_waves 4 / 8: a ragged call whose sequences all have at most 64 rows per kv head runs on
    the 2-wave tiles (fp16 hi + lo probabilities), one with a longer sequence runs that one on tiles
    of that many waves and its short sequences on the decode kernel; with tile_waves 0 a call of
    short sequences runs on the decode kernel alone."""

    rng = np.random.default_rng(77)
    Hkv, G = 2, 4
    for lengths in ([1, 16, 9, 2, 1], [3, 80, 1, 40]):
        seg, ks, vs, _ = _ragged_case(rng, lengths, Hkv, G, False, True)
        cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        q = _bf(rng, (int(cu[-1]), Hkv * G, 128))
        for tw in (0, 4, 8):
            out = ops.prefill_attention(_t(q), causal=True, cu_seqlens_q=torch.from_numpy(cu).to(DEV),
                                        max_seqlen_q=max(lengths), tile_waves=tw, **seg)
            for b in range(len(lengths)):
                rows = slice(int(cu[b]), int(cu[b + 1]))
                want, _ = A.attention(q[rows].transpose(1, 0, 2)[None], ks[b], vs[b], causal_bottom_right=True)
                want = bf16.round_bf16(want[0].transpose(1, 0, 2).astype(np.float32))
                got = out[rows].float().cpu().numpy()
                assert A.max_abs(got, want) <= MAX_ABS and A.rel_l2(got, want) <= REL_L2, (lengths, tw, b)


@pytest.mark.parametrize("paged", [False, True])
def test_ragged_prefill_more_than_64_sequences(paged):
    """150 sequences of 0-100 query tokens: the workgroups find their sequence by scanning
    cu_seqlens 64 sequences per step (the tile grid's compaction and the decode classes' ranks and
    split counts), so every sequence past the first 64 must land on its own rows too."""

    rng = np.random.default_rng(90 + paged)
    Hkv, G = 2, 4
    lengths = [int(x) for x in rng.choice([0, 1, 1, 1, 2, 7, 12, 16, 17, 40, 100], size=150)]
    lengths[140] = 100  # a tile-path sequence in the third step of 64
    seg, ks, vs, meta = _ragged_case(rng, lengths, Hkv, G, paged, True)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    q = _bf(rng, (int(cu[-1]), Hkv * G, 128))
    cu_t = torch.from_numpy(cu).to(DEV)
    one_split = ops.prefill_attention(_t(q), causal=True, cu_seqlens_q=cu_t, max_seqlen_q=max(lengths), num_splits=1,
                                      **seg)
    auto = ops.prefill_attention(_t(q), causal=True, cu_seqlens_q=cu_t, max_seqlen_q=max(lengths), **seg)
    worst = 0.0
    for b, L in enumerate(lengths):
        if L == 0:
            continue
        rows = slice(int(cu[b]), int(cu[b + 1]))
        alone = ops.prefill_attention(_t(q[rows][None]), causal=True, num_splits=1, **_one(seg, b, meta))
        assert torch.equal(one_split[rows], alone[0]), f"paged={paged}: sequence {b} (L={L}) differs from its own call"
        want, _ = A.attention(q[rows].transpose(1, 0, 2)[None], ks[b], vs[b], causal_bottom_right=True)
        want = bf16.round_bf16(want[0].transpose(1, 0, 2).astype(np.float32))
        got = auto[rows].float().cpu().numpy()
        worst = max(worst, A.rel_l2(got, want))
        assert A.max_abs(got, want) <= MAX_ABS and A.rel_l2(got, want) <= REL_L2, f"paged={paged} sequence {b} (L={L})"
    print(f"paged={paged}: 150 sequences, {sum(lengths)} rows, worst rel_l2 {worst:.2e} (automatic splits)", flush=True)


@pytest.mark.parametrize("case", range(6))
def test_ragged_host_offsets_plan_the_same_results(case):
    """cu_seqlens_q_host (the offsets on the host) only plans the launches: decode column classes that
    hold no sequence are not launched, a class of one split gets no merge, and a call without a
    sequence above 64 rows per kv head runs no tile kernel (also when max_seqlen_q overstates its
    longest sequence); outputs and LSE equal the call without it, bit for bit."""

    rng = np.random.default_rng(600 + case)
    lengths = [[1] * 9, [1, 3, 2, 1], [5, 0, 7, 1], [1] * 5 + [100], [40, 100, 33], [0, 1, 16, 17, 70, 1, 2]][case]
    max_seqlen = max(lengths) + (150 if case in (0, 2) else 0)
    Hkv, G = 2, 4
    Hq = Hkv * G
    seg, ks, vs, _ = _ragged_case(rng, lengths, Hkv, G, case % 2 == 1, True)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    T = int(cu[-1])
    q = _bf(rng, (T, Hq, 128))
    cu_t = torch.from_numpy(cu).to(DEV)
    outs, lses = [], []
    for host in (None, cu):
        lse = torch.full((T, Hq), 7.0, dtype=torch.float32, device=DEV)
        out = ops.prefill_attention(_t(q), causal=True, cu_seqlens_q=cu_t, max_seqlen_q=max_seqlen, lse=lse,
                                    cu_seqlens_q_host=host, **seg)
        outs.append(out)
        lses.append(lse)
    assert torch.equal(outs[0], outs[1]) and torch.equal(lses[0], lses[1]), f"lengths {lengths}"
    for b, L in enumerate(lengths):
        if L == 0:
            continue
        rows = slice(int(cu[b]), int(cu[b + 1]))
        want, _ = A.attention(q[rows].transpose(1, 0, 2)[None], ks[b], vs[b], causal_bottom_right=True)
        want = bf16.round_bf16(want[0].transpose(1, 0, 2).astype(np.float32))
        got = outs[1][rows].float().cpu().numpy()
        assert A.max_abs(got, want) <= MAX_ABS and A.rel_l2(got, want) <= REL_L2, (lengths, b)
    with pytest.raises(ValueError, match="cu_seqlens_q_host"):
        ops.prefill_attention(_t(q), causal=True, cu_seqlens_q=cu_t, max_seqlen_q=max_seqlen,
                              cu_seqlens_q_host=cu[:-1], **seg)


RAGGED_SWEEP_SEED0 = 7000
RAGGED_SWEEP_CASES = 60
RAGGED_SWEEP_PART = 10


def _ragged_sweep_case(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 25))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    pool_of_lengths = [0, 1, 1, 1, 1, 2, 3, 5, 8, 9, 16, 17, 31, 33, 64, 65, 100, 129, 250]
    lengths = [int(x) for x in rng.choice(pool_of_lengths, size=B)]
    if sum(lengths) == 0:
        lengths[0] = 1
    paged = bool(rng.integers(0, 2))
    causal = bool(rng.integers(0, 2))
    splits = int(rng.choice([0, 0, 1, 3]))
    waves = int(rng.choice([0, 0, 0, 4, 8]))
    return rng, lengths, Hkv, G, paged, causal, splits, waves


@pytest.mark.parametrize("part", range(RAGGED_SWEEP_CASES // RAGGED_SWEEP_PART))
def test_random_ragged_sweep(part):
    """Seeded random ragged calls: 1-24 sequences of 0-250 query tokens (decode rows, every column
    class of the decode kernel and tile-path rows mixed), GQA groups 1-8 over 1-4 kv heads, tiled or
    paged caches, causal or bidirectional, automatic / 1 / 3 key splits and automatic or forced tile
    waves, each sequence against the fp64 oracle at the north-star bar; with one split and the
    automatic tiles every sequence also equals its own uniform call bit for bit."""

    worst = 0.0
    for seed in range(RAGGED_SWEEP_SEED0 + part * RAGGED_SWEEP_PART, RAGGED_SWEEP_SEED0 + (part + 1) * RAGGED_SWEEP_PART):
        rng, lengths, Hkv, G, paged, causal, splits, waves = _ragged_sweep_case(seed)
        Hq = Hkv * G
        seg, ks, vs, meta = _ragged_case(rng, lengths, Hkv, G, paged, causal)
        cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        T = int(cu[-1])
        q = _bf(rng, (T, Hq, 128))
        lse = torch.empty((T, Hq), dtype=torch.float32, device=DEV)
        label = (f"seed {seed}: lengths={lengths} Hkv={Hkv} G={G} paged={paged} causal={causal} "
                 f"splits={splits} tile_waves={waves}")
        out = ops.prefill_attention(_t(q), causal=causal, cu_seqlens_q=torch.from_numpy(cu).to(DEV),
                                    max_seqlen_q=max(lengths), lse=lse, num_splits=splits, tile_waves=waves, **seg)
        for b, L in enumerate(lengths):
            if L == 0:
                continue
            rows = slice(int(cu[b]), int(cu[b + 1]))
            want, want_lse = A.attention(q[rows].transpose(1, 0, 2)[None], ks[b], vs[b], causal_bottom_right=causal)
            want = bf16.round_bf16(want[0].transpose(1, 0, 2).astype(np.float32))
            got = out[rows].float().cpu().numpy()
            ma, rl = A.max_abs(got, want), A.rel_l2(got, want)
            worst = max(worst, rl)
            assert ma <= MAX_ABS and rl <= REL_L2, f"{label}: sequence {b} (L={L}) max_abs={ma} rel_l2={rl}"
            np.testing.assert_allclose(lse[rows].cpu().numpy(), want_lse[0].T, rtol=1e-4, atol=1e-4,
                                       err_msg=f"{label}: lse of sequence {b}")
            if splits == 1 and waves == 0:
                alone = ops.prefill_attention(_t(q[rows][None]), causal=causal, num_splits=1, **_one(seg, b, meta))
                assert torch.equal(out[rows], alone[0]), f"{label}: sequence {b} (L={L}) differs from its own call"
        print(f"{label}: ok", flush=True)
    print(f"part {part}: worst rel_l2 {worst:.2e}", flush=True)


def _rotary(positions):
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, device=positions.device).float() / 128))
    f = positions[..., None].float() * inv
    emb = torch.cat((f, f), -1)
    return emb.cos().bfloat16(), emb.sin().bfloat16()


@pytest.mark.parametrize("rounding", ["torch", "vllm"])
@pytest.mark.parametrize("lengths", [[1, 3, 0, 2], [1, 40, 7, 100, 1, 33]])
def test_ragged_epilogue_equals_per_sequence_calls(rounding, lengths):
    g = torch.Generator(device=DEV).manual_seed(len(lengths) + (rounding == "vllm"))
    Hq, Hkv, R, cap = 8, 2, 256, 512
    B = len(lengths)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=DEV)
    T = int(cu[-1])
    pos = torch.tensor([int(x) for x in np.random.default_rng(B).integers(0, 300, B)], dtype=torch.int32, device=DEV)
    fused = torch.randn((T, (Hq + 2 * Hkv) * 128), generator=g, device=DEV).bfloat16()
    q, k, v = fused.split([Hq * 128, Hkv * 128, Hkv * 128], dim=-1)
    flat = torch.cat([torch.arange(int(pos[b]), int(pos[b]) + L, device=DEV) for b, L in enumerate(lengths)])
    cos, sin = _rotary(flat[None])
    qw = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
    kw = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
    vmul = (torch.rand(Hkv, generator=g, device=DEV) + 0.5) if rounding == "vllm" else None
    kwargs = dict(num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=qw, k_norm_weight=kw, eps=1e-5, rounding=rounding,
                  ring_v_mul=vmul)
    ring_a, deep_a = ops.TiledKV.zeros(B, Hkv, R, DEV), ops.TiledKV.zeros(B, Hkv, cap, DEV)
    ring_b, deep_b = ops.TiledKV.zeros(B, Hkv, R, DEV), ops.TiledKV.zeros(B, Hkv, cap, DEV)
    qa = ops.qkv_epilogue(q, k, v, cos, sin, positions=pos, ring=ring_a, deep=deep_a, cu_seqlens=cu,
                          max_seqlen=max(lengths), **kwargs)
    for b, L in enumerate(lengths):
        if L == 0:
            continue
        rows = slice(int(cu[b]), int(cu[b + 1]))
        sl = lambda c: ops.TiledKV(c.k[b:b + 1], c.v[b:b + 1])
        qb = ops.qkv_epilogue(q[rows][None], k[rows][None], v[rows][None], cos[:, rows], sin[:, rows],
                              positions=int(pos[b]), ring=sl(ring_b), deep=sl(deep_b), **kwargs)
        assert torch.equal(qa[rows], qb[0]), f"sequence {b}: normalised queries differ"
    assert torch.equal(ring_a.k, ring_b.k) and torch.equal(ring_a.v, ring_b.v), "ring contents differ"
    assert torch.equal(deep_a.k, deep_b.k) and torch.equal(deep_a.v, deep_b.v), "shared-store contents differ"


@pytest.mark.parametrize("part", range(4))
def test_random_ragged_epilogue_sweep(part):
    """Seeded random ragged epilogue calls (10 per part): 1-30 sequences of 0-129 tokens at positions
    0-400, GQA 1-4 over 1-8 kv heads, tiled or paged rings and shared stores, both rounding contracts
    (the vLLM one with a ring V multiplier), with and without the shared store; the normalised
    queries and every ring and shared-store byte equal the per-sequence calls'."""

    for case in range(10):
        seed = 8000 + 10 * part + case
        rng = np.random.default_rng(seed)
        g = torch.Generator(device=DEV).manual_seed(seed)
        B = int(rng.integers(1, 31))
        Hkv = int(rng.choice([1, 2, 3, 4, 5, 8]))  # (odd counts: the block form's last K/V workgroup holds one head)
        Hq = Hkv * int(rng.choice([1, 2, 4]))
        lengths = [int(x) for x in rng.choice([0, 1, 1, 1, 2, 3, 7, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 129], size=B)]
        if sum(lengths) == 0:
            lengths[-1] = 1
        rounding = str(rng.choice(["torch", "vllm"]))
        paged, with_deep = bool(rng.integers(0, 2)), bool(rng.integers(0, 3))
        R, cap = 256, 576
        pos_h = [int(x) for x in rng.integers(0, 401, B)]
        cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=DEV)
        T = int(cu[-1])
        pos = torch.tensor(pos_h, dtype=torch.int32, device=DEV)
        fused = torch.randn((T, (Hq + 2 * Hkv) * 128), generator=g, device=DEV).bfloat16()
        q, k, v = fused.split([Hq * 128, Hkv * 128, Hkv * 128], dim=-1)
        flat = torch.cat([torch.arange(pos_h[b], pos_h[b] + L, device=DEV) for b, L in enumerate(lengths)])
        cos, sin = _rotary(flat[None])
        qw = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
        kw = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
        vmul = (torch.rand(Hkv, generator=g, device=DEV) + 0.5) if rounding == "vllm" else None
        kwargs = dict(num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=qw, k_norm_weight=kw, eps=1e-5,
                      rounding=rounding, ring_v_mul=vmul)
        label = f"seed {seed}: lengths={lengths} Hq={Hq} Hkv={Hkv} {rounding} paged={paged} deep={with_deep}"
        if paged:
            rb, db = R // 32, cap // 32
            perm = torch.from_numpy(rng.permutation(B * (rb + db))).to(DEV, torch.int32)
            rtab, dtab = perm[:B * rb].view(B, rb).contiguous(), perm[B * rb:].view(B, db).contiguous()
            stores = [ops.PagedKV.zeros(B * (rb + db), Hkv, DEV) for _ in range(2)]

            def where(st, sl):
                return dict(ring=st, ring_table=rtab[sl], ring_tokens=R, deep=st if with_deep else None,
                            deep_table=dtab[sl] if with_deep else None)
        else:
            stores = [(ops.TiledKV.zeros(B, Hkv, R, DEV), ops.TiledKV.zeros(B, Hkv, cap, DEV)) for _ in range(2)]

            def where(st, sl):
                one = lambda c: ops.TiledKV(c.k[sl], c.v[sl])
                return dict(ring=one(st[0]), deep=one(st[1]) if with_deep else None)
        qa = ops.qkv_epilogue(q, k, v, cos, sin, positions=pos, cu_seqlens=cu, max_seqlen=max(lengths),
                              **where(stores[0], slice(0, B)), **kwargs)
        for b, L in enumerate(lengths):
            if L == 0:
                continue
            rows = slice(int(cu[b]), int(cu[b + 1]))
            qb = ops.qkv_epilogue(q[rows][None], k[rows][None], v[rows][None], cos[:, rows], sin[:, rows],
                                  positions=pos_h[b], **where(stores[1], slice(b, b + 1)), **kwargs)
            assert torch.equal(qa[rows], qb[0]), f"{label}: normalised queries of sequence {b} differ"
        a_t = [stores[0]] if paged else list(stores[0])
        b_t = [stores[1]] if paged else list(stores[1])
        for x, y in zip(a_t, b_t):
            assert torch.equal(x.k, y.k) and torch.equal(x.v, y.v), f"{label}: cache contents differ"
        print(f"{label}: ok", flush=True)


def test_serving_mixed_step_31_decode_1024_and_7_rows_match_oracle():
    """A step of 31 decode rows, one 1024-token prefill row (positions 2048-3071: 1024 older keys
    and a causal local segment of 2048) and one 7-token row, one epilogue and one attention launch
    per layer, against the oracle model run per sequence."""

    oracle, ours = _tiny(chunk=1024, layers=2)
    runner = LastKVServingModel(ours, max_batch=33, max_tokens_per_slot=3104)
    gen = torch.Generator().manual_seed(12)
    prompts = [torch.randint(3, 97, (int(n),), generator=gen).to(DEV) for n in torch.randint(20, 90, (31,), generator=gen)]
    long_seq = torch.randint(3, 97, (3072,), generator=gen).to(DEV)
    short_seq = torch.randint(3, 97, (40,), generator=gen).to(DEV)
    slots = [runner.add_sequence() for _ in range(33)]
    with torch.inference_mode():
        first = runner.step([(s, p) for s, p in zip(slots[:31], prompts)])  # a ragged prefill step
        runner.step([(slots[31], long_seq[:1024]), (slots[32], short_seq[:33])])
        runner.step([(slots[31], long_seq[1024:2048])])
        nxt = first.argmax(-1)
        seqs = [torch.cat([p, nxt[i:i + 1]]) for i, p in enumerate(prompts)]
        rows = [(s, seqs[i][-1:]) for i, s in enumerate(slots[:31])]
        rows += [(slots[31], long_seq[2048:]), (slots[32], short_seq[33:])]
        assert sorted({int(ids.numel()) for _, ids in rows}) == [1, 7, 1024]
        logits = runner.step(rows)
        fulls = seqs + [long_seq, short_seq]
        got = logits.float()
        want = torch.stack([_o32(oracle)(s[None])[0][0, -1] for s in fulls]).float()
        ref16 = torch.stack([_o16(oracle)(s[None])[0][0, -1] for s in fulls]).float()
    _no_worse_than_reference_bf16(got[None], want[None], ref16[None], "mixed step (31 decode + 1024 + 7 rows)")

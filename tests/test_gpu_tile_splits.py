"""Key splits of the prefill tile kernel (GPU).

A call whose tile grid would leave CUs idle (few sequences, few query tiles) splits each tile's keys
over up to 4 workgroups when it leaves the split counts to the library (num_splits 0) and its
workspace holds the splits' states (lkv_prefill_workspace_bytes); each split begins with an older
block, writes its rows' normalised fp32 O and base-2 LSE, and a merge kernel combines them.  The
bar is the north-star one against the fp64 oracle (outputs and LSE), on contiguous and paged
caches, causal and bidirectional, with an older segment long enough for 4 equal splits; one of 3
blocks, where no equal split would start inside it, runs unsplit (the num_splits = 1 bits), as
does the call with the minimum workspace; a ragged step (one long row among decode rows and a
short row) takes the split too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16

from test_gpu_decode import MAX_ABS, REL_L2, _bf, _t
from test_gpu_varlen import _ragged_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(rng, B, Hkv, T0, L, paged):
    """B sequences with an older segment of T0 tokens and a ring of L + 300 tokens from a random
    start; returns the kernel segments and the composed K / V (older V as bf16(V * s))."""

    R = (-(-(L + 300) // 32) + 2) * 32
    n1, start = L + 300, int(rng.integers(0, R))
    ok, ov = _bf(rng, (B, Hkv, T0, 128)), _bf(rng, (B, Hkv, T0, 128))
    lk, lv = _bf(rng, (B, Hkv, n1, 128)), _bf(rng, (B, Hkv, n1, 128))
    s = bf16.round_bf16(rng.uniform(0.4, 1.4, Hkv).astype(np.float32))
    older = ops.TiledKV.zeros(B, Hkv, -(-T0 // 32) * 32, DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    ring = ops.TiledKV.zeros(B, Hkv, R, DEV)
    first = min(n1, R - start)
    ops.pack_kv(_t(lk[:, :, :first]), _t(lv[:, :, :first]), ring, token0=start)
    if first < n1:
        ops.pack_kv(_t(lk[:, :, first:]), _t(lv[:, :, first:]), ring, token0=0)
    seg = dict(older_len=T0, vscale=torch.from_numpy(s).to(DEV), local_len=n1, local_start=start)
    if paged:
        ob, rb = older.k.shape[2], ring.k.shape[2]
        pool = ops.PagedKV.zeros(B * (ob + rb) + 1, Hkv, DEV)
        perm = torch.randperm(B * (ob + rb), generator=torch.Generator().manual_seed(5)).to(DEV, torch.int32)
        otab, rtab = perm[:B * ob].view(B, ob).contiguous(), perm[B * ob:].view(B, rb).contiguous()
        for b in range(B):
            for j in range(ob):
                pool.k[:, otab[b, j]], pool.v[:, otab[b, j]] = older.k[b, :, j], older.v[b, :, j]
            for j in range(rb):
                pool.k[:, rtab[b, j]], pool.v[:, rtab[b, j]] = ring.k[b, :, j], ring.v[b, :, j]
        seg.update(older=pool, older_table=otab, local=pool, local_table=rtab, local_ring_blocks=rb)
    else:
        seg.update(older=older, local=ring)
    k = np.concatenate([ok, lk], 2)
    v = np.concatenate([bf16.mul(ov, s.reshape(1, -1, 1, 1)), lv], 2)
    return seg, k, v


@pytest.mark.parametrize("T0", [3000, 70])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("causal", [True, False])
def test_key_splits_match_oracle_and_minimum_workspace_runs_unsplit(T0, paged, causal):
    rng = np.random.default_rng(11 + 2 * paged + causal + T0)
    B, Hkv, G, L = 1, 2, 4, 512
    seg, k, v = _case(rng, B, Hkv, T0, L, paged)
    q = _bf(rng, (B, L, Hkv * G, 128))
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
    want = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    lse = torch.empty((B, L, Hkv * G), dtype=torch.float32, device=DEV)
    split = ops.prefill_attention(_t(q), causal=causal, lse=lse, **seg)  # automatic: 4 splits for T0 = 3000, none for 70
    got = split.float().cpu().numpy()
    ma, rl = A.max_abs(got, want), A.rel_l2(got, want)
    print(f"T0={T0} paged={paged} causal={causal}: key splits max_abs {ma:.2e} rel_l2 {rl:.2e}", flush=True)
    assert ma <= MAX_ABS and rl <= REL_L2
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    unsplit = ops.prefill_attention(_t(q), causal=causal, num_splits=1, **seg)
    if T0 == 70:  # 3 older blocks: no equal split starts inside them
        assert torch.equal(split, unsplit)
    else:
        assert not torch.equal(split, unsplit)  # (the split merge rounds differently somewhere)
    # the minimum workspace (no room for the states): the same arithmetic as num_splits = 1
    need = ops.prefill_workspace_bytes(B, Hkv, T0, seg["local_len"], seg["local_start"] % 32)
    small = ops.prefill_attention(_t(q), causal=causal, workspace=torch.empty(need, dtype=torch.uint8, device=DEV),
                                  **seg)
    assert torch.equal(small, unsplit)


def test_ragged_step_long_row_takes_key_splits():
    """One 300-token row among eleven one-token rows and a 7-token row: the long row's tiles split
    their keys (its older segment is not empty); every row within the bar of the oracle."""

    rng = np.random.default_rng(23)
    Hkv, G = 2, 4
    lengths = [1] * 5 + [300] + [1] * 6 + [7]
    seg, ks, vs, _ = _ragged_case(rng, lengths, Hkv, G, True, True)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    q = _bf(rng, (int(cu[-1]), Hkv * G, 128))
    out = ops.prefill_attention(_t(q), causal=True, cu_seqlens_q=torch.from_numpy(cu).to(DEV),
                                max_seqlen_q=max(lengths), **seg)
    worst = 0.0
    for b in range(len(lengths)):
        rows = slice(int(cu[b]), int(cu[b + 1]))
        want, _ = A.attention(q[rows].transpose(1, 0, 2)[None], ks[b], vs[b], causal_bottom_right=True)
        want = bf16.round_bf16(want[0].transpose(1, 0, 2).astype(np.float32))
        got = out[rows].float().cpu().numpy()
        worst = max(worst, A.rel_l2(got, want))
        assert A.max_abs(got, want) <= MAX_ABS and A.rel_l2(got, want) <= REL_L2, f"sequence {b}"
    print(f"ragged step with a long row: worst rel_l2 {worst:.2e}", flush=True)

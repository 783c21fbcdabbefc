"""V values beyond fp16's range in the prefill tile kernel (GPU).

The tile kernel runs P V in fp16, which holds every bf16 value up to 65280 exactly but none of
magnitude 65536 or more.  Its V pre-pass flags each key block holding such a value (older blocks
after the V scale, bf16(V * s)), the fp16 instance skips the query tiles that read a flagged
block, and a second instance runs them with bf16 V and the probabilities split into bf16 hi + lo.
These calls must match the fp64 oracle whatever the magnitudes: a few V values of 1e5 - 3e6 in the
older segment, in the ring, or reaching that range only through the older segment's scale, in one
(sequence, kv head) pair of three sequences (the others stay on the fp16 instance), on the
automatic tile choice and on 4- and 8-wave tiles; a V of 65280, the largest bf16 that fp16 holds,
stays on the fp16 instance and is exact there (see ``_check_edge`` for that case's bar).  The bar
is rel-L2 1e-3 and every element within max(2e-2, one bf16 ulp of the exact value): outputs near
1e5 have a bf16 spacing of 512.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16

from test_gpu_decode import REL_L2, _bf, _t

pytestmark = pytest.mark.gpu
DEV = "cuda"

B, HKV, G, L, T0, RING = 3, 2, 4, 96, 900, 12


def _case(where, seed):
    """Older segment of T0 tokens and a ring of RING blocks holding L + 200 tokens from ring token 57,
    with large V values planted in sequence 1, kv head 0; returns the kernel segments and the
    composed K / V (older V as bf16(V * s))."""

    rng = np.random.default_rng(seed)
    n1, start = L + 200, 57
    ok, ov = _bf(rng, (B, HKV, T0, 128)), _bf(rng, (B, HKV, T0, 128))
    lk, lv = _bf(rng, (B, HKV, n1, 128)), _bf(rng, (B, HKV, n1, 128))
    s = bf16.round_bf16(np.array([1.5, 0.75], np.float32))
    if where == "older":  # raw older values far beyond fp16
        for t, d, x in ((5, 3, 2.0e5), (400, 77, -3.0e6), (899, 127, 7.0e4)):
            ov[1, 0, t, d] = x
    elif where == "local":  # ring values, used as stored
        for t, d, x in ((0, 9, 1.0e5), (150, 64, -2.5e5), (n1 - 1, 0, 9.0e4)):
            lv[1, 0, t, d] = x
    elif where == "scaled":  # under 65536 raw, above it once scaled by s = 1.5
        for t, d, x in ((17, 40, 50000.0), (600, 2, -60000.0)):
            ov[1, 0, t, d] = x
    elif where == "edge":  # 65280 once scaled: the largest value fp16 holds exactly
        ov[1, 0, 33, 5] = 43520.0  # 43520 * 1.5 = 65280
        lv[1, 0, 10, 6] = -65280.0
    ov, lv = bf16.round_bf16(ov), bf16.round_bf16(lv)
    older = ops.TiledKV.zeros(B, HKV, -(-T0 // 32) * 32, DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    ring = ops.TiledKV.zeros(B, HKV, RING * 32, DEV)
    R = RING * 32
    first = min(n1, R - start)
    ops.pack_kv(_t(lk[:, :, :first]), _t(lv[:, :, :first]), ring, token0=start)
    if first < n1:
        ops.pack_kv(_t(lk[:, :, first:]), _t(lv[:, :, first:]), ring, token0=0)
    k = np.concatenate([ok, lk], 2)
    v = np.concatenate([bf16.mul(ov, s.reshape(1, -1, 1, 1)), lv], 2)
    seg = dict(older=older, older_len=T0, vscale=torch.from_numpy(s).to(DEV), local=ring, local_len=n1,
               local_start=start)
    return seg, k, v, rng


def _check(out, want, label):
    got = out.float().cpu().numpy().astype(np.float64)
    rl = A.rel_l2(got, bf16.round_bf16(want.astype(np.float32)))
    err = np.abs(got - want)
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(want), 2.0 ** -100))[1] - 8)
    ratio = float(np.max(err / np.maximum(ulp, 2e-2)))
    print(f"{label}: rel_l2 {rl:.2e}, worst error / max(2e-2, 1 ulp) {ratio:.2f}, max |out| {np.abs(got).max():.3g}",
          flush=True)
    assert rl <= REL_L2 and ratio <= 1.0, label


def _check_edge(out, q, k, v, want, tile_waves):
    """65280 is exact in fp16, so these tiles stay on the fp16 instance: every element must be within
    one bf16 ulp of the exact value, and the pairs without planted values within rel-L2 1e-3.  The
    affected pair's outputs are dominated by one key's weight times 65280, so the last bf16 bit of
    each is decided by that weight's fp16 rounding (11 bits): their rel-L2 is bounded by the
    reference's own bf16 SDPA path on the same inputs (evaluated on the CPU), which rounds the
    weights to 8 bits."""

    from oracle.reference_path import sdpa_bottom_right

    got = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - want)
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(want), 2.0 ** -100))[1] - 8)
    ratio = float(np.max(err / np.maximum(ulp, 2e-2)))
    assert ratio <= 1.0, f"edge tile_waves={tile_waves}: an element is more than one bf16 ulp off ({ratio:.2f})"
    rel = lambda a, w: A.rel_l2(a, bf16.round_bf16(w.astype(np.float32)))
    aff = (slice(1, 2), slice(None), slice(0, G))
    rest = [rel(got[0], want[0]), rel(got[2], want[2]), rel(got[1, :, G:], want[1, :, G:])]
    tq = lambda x: torch.from_numpy(np.ascontiguousarray(x)).bfloat16()
    ref = sdpa_bottom_right(tq(q.transpose(0, 2, 1, 3)), tq(k), tq(v)).transpose(1, 2).float().numpy()
    ours_aff, ref_aff = rel(got[aff], want[aff]), rel(ref[aff], want[aff])
    print(f"edge tile_waves={tile_waves}: worst element {ratio:.2f} of max(2e-2, 1 ulp); rel_l2 unaffected pairs "
          f"{max(rest):.2e}; affected pair {ours_aff:.2e} (reference bf16 SDPA {ref_aff:.2e})", flush=True)
    assert max(rest) <= REL_L2 and ours_aff <= ref_aff


@pytest.mark.parametrize("where", ["older", "local", "scaled", "edge"])
@pytest.mark.parametrize("tile_waves", [0, 4, 8])
def test_prefill_v_beyond_fp16_range_matches_oracle(where, tile_waves):
    seg, k, v, rng = _case(where, seed=7)
    q = _bf(rng, (B, L, G * HKV, 128))
    want, _ = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=True)
    want = want.transpose(0, 2, 1, 3)
    out = ops.prefill_attention(_t(q), causal=True, tile_waves=tile_waves, **seg)
    if where == "edge":
        _check_edge(out, q, k, v, want, tile_waves)
    else:
        _check(out, want, f"{where} tile_waves={tile_waves}")
    # the planted values carry weight in the affected pair's outputs (unit-scale data elsewhere)
    assert float(out[1, :, :G].float().abs().max()) > 10.0
    assert float(out[0].float().abs().max()) < 10.0

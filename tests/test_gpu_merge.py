"""GPU parity of lkv_merge_states, the exact LSE merge of two attention states.

Checked against the oracle's merge (pinned on the CPU by merge(attn(K1), attn(K2)) == attn(K1 u K2))
and, end to end, against single-pass attention over the union of two key segments.  Tolerances:
outputs within max-abs 2e-2 and rel-L2 1e-3 of the fp64 result rounded to bf16; LSEs within 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(x, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, dtype)


def _close(actual: torch.Tensor, expected, label: str):
    a = actual.float().cpu().numpy()
    e = np.asarray(expected, np.float64)
    ma, rl = A.max_abs(a, e), A.rel_l2(a, e)
    print(f"{label}: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= 2e-2 and rl <= 1e-3, f"{label}: max_abs={ma} rel_l2={rl}"


def _states(rng, T, H, D):
    a = bf16.round_bf16(rng.standard_normal((T, H, D)).astype(np.float32))
    b = bf16.round_bf16(rng.standard_normal((T, H, D)).astype(np.float32))
    la = (rng.standard_normal((T, H)) * 4).astype(np.float32)
    lb = (rng.standard_normal((T, H)) * 4).astype(np.float32)
    la[::5, :] = -np.inf  # rows without older history (the serving path's nosrc rows)
    la[3, 2] = lb[3, 2] = -np.inf  # no keys on either side
    lb[7, 1] = -np.inf
    return a, la, b, lb


@pytest.mark.parametrize("layout", ["th", "ht"])
@pytest.mark.parametrize("scaled", [False, True])
def test_merge_matches_oracle(layout, scaled):
    rng = np.random.default_rng(11 + scaled)
    T, H, D = 37, 12, 128
    a, la, b, lb = _states(rng, T, H, D)
    s = bf16.round_bf16(rng.uniform(0.3, 1.3, H).astype(np.float32)) if scaled else None

    def lse_tensor(x):
        # [T, H] values viewed through the requested memory layout
        return _t(x, torch.float32) if layout == "th" else _t(x.T, torch.float32).t()

    out_lse = torch.empty((T, H), dtype=torch.float32, device=DEV) if layout == "th" else \
        torch.empty((H, T), dtype=torch.float32, device=DEV).t()
    out, _ = ops.merge_states(_t(a), lse_tensor(la), _t(b), lse_tensor(lb),
                              prefix_scale=None if s is None else _t(s, torch.float32), out_lse=out_lse)
    a_in = bf16.mul(a, s[None, :, None]) if scaled else a
    want, want_lse = A.merge_states(a_in, la, b, lb)
    _close(out, bf16.round_bf16(want.astype(np.float32)), f"merge layout={layout} scaled={scaled}")
    got_lse = out_lse.cpu().numpy()
    assert np.array_equal(np.isinf(got_lse), np.isinf(want_lse))
    fin = np.isfinite(want_lse)
    np.testing.assert_allclose(got_lse[fin], want_lse[fin], rtol=1e-5, atol=1e-5)
    assert np.all(out[3, 2].float().cpu().numpy() == 0)  # both sides empty -> zero output


def test_merge_vllm_and_flashinfer_orders():
    rng = np.random.default_rng(5)
    T, H, D = 9, 4, 64
    a, la, b, lb = _states(rng, T, H, D)
    want, want_lse = A.merge_states(a, la, b, lb)
    out = torch.empty((T, H, D), dtype=torch.bfloat16, device=DEV)
    out_lse_ht = torch.empty((H, T), dtype=torch.float32, device=DEV)
    ops.merge_attn_states(out, _t(a), _t(la.T, torch.float32), _t(b), _t(lb.T, torch.float32), out_lse_ht)
    _close(out, bf16.round_bf16(want.astype(np.float32)), "vLLM order, LSE [H, T]")
    fin = np.isfinite(want_lse)
    np.testing.assert_allclose(out_lse_ht.t().cpu().numpy()[fin], want_lse[fin], rtol=1e-5, atol=1e-5)
    v, s = ops.merge_state(_t(a), _t(la, torch.float32), _t(b), _t(lb, torch.float32))
    _close(v, bf16.round_bf16(want.astype(np.float32)), "FlashInfer order, LSE [T, H]")
    np.testing.assert_allclose(s.cpu().numpy()[fin], want_lse[fin], rtol=1e-5, atol=1e-5)


def test_merged_passes_equal_single_pass_over_union():
    """Older segment and local segment attended separately (each with its LSE) and merged, as the
    reference's two-pass serving path does.  Each partial output is checked against the oracle's
    partial (standard bar), and the merge against the oracle merge of the same two bf16 partials
    the kernel merged (standard bar; comparing with the merge of the oracle's partials instead
    would count each partial's bf16 rounding flips twice).  Against one pass over [older | local]
    the two intermediate bf16 roundings add up to about one bf16 ulp, so that comparison allows
    rel-L2 4e-3 (the same holds for the reference's own two-pass FA3 path)."""

    rng = np.random.default_rng(23)
    B, L, Hq, Hkv, T0, n_local = 2, 48, 8, 2, 300, 96
    q = bf16.round_bf16(rng.standard_normal((B, L, Hq, 128)).astype(np.float32))
    ok = bf16.round_bf16(rng.standard_normal((B, Hkv, T0, 128)).astype(np.float32))
    ov = bf16.round_bf16(rng.standard_normal((B, Hkv, T0, 128)).astype(np.float32))
    lk = bf16.round_bf16(rng.standard_normal((B, Hkv, n_local, 128)).astype(np.float32))
    lv = bf16.round_bf16(rng.standard_normal((B, Hkv, n_local, 128)).astype(np.float32))
    s = bf16.round_bf16(rng.uniform(0.4, 1.2, Hkv).astype(np.float32))
    older = ops.TiledKV.zeros(B, Hkv, 320, DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    ring = ops.TiledKV.zeros(B, Hkv, 128, DEV)
    ops.pack_kv(_t(lk), _t(lv), ring, token0=5)
    vs = _t(s, torch.float32)
    lse_o = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
    lse_l = torch.empty_like(lse_o)
    out_o = ops.prefill_attention(_t(q), older=older, older_len=T0, vscale=vs, lse=lse_o)
    out_l = ops.prefill_attention(_t(q), local=ring, local_len=n_local, local_start=5, causal=True, lse=lse_l)
    single = ops.prefill_attention(_t(q), older=older, older_len=T0, vscale=vs, local=ring, local_len=n_local,
                                   local_start=5, causal=True)
    merged, _ = ops.merge_states(out_o.view(B * L, Hq, 128), lse_o.view(B * L, Hq),
                                 out_l.view(B * L, Hq, 128), lse_l.view(B * L, Hq))
    merged = merged.view(B, L, Hq, 128)
    qt = q.transpose(0, 2, 1, 3)
    sv = bf16.mul(ov, s[None, :, None, None])
    # oracle partial states (bottom-right causal over the local segment alone: query i sees
    # local tokens [0, n_local - L + i])
    po, plo = A.attention(qt, ok, sv)
    pl, pll = A.attention(qt, lk, lv, causal_bottom_right=True)
    np.testing.assert_allclose(lse_o.cpu().numpy(), plo.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(lse_l.cpu().numpy(), pll.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    _close(out_o, bf16.round_bf16(po.transpose(0, 2, 1, 3).astype(np.float32)), "older partial vs oracle")
    _close(out_l, bf16.round_bf16(pl.transpose(0, 2, 1, 3).astype(np.float32)), "local partial vs oracle")
    go = out_o.float().cpu().numpy().transpose(0, 2, 1, 3)
    gl = out_l.float().cpu().numpy().transpose(0, 2, 1, 3)
    want_m, _ = A.merge_states(go, lse_o.cpu().numpy().transpose(0, 2, 1), gl, lse_l.cpu().numpy().transpose(0, 2, 1))
    _close(merged, bf16.round_bf16(want_m.transpose(0, 2, 1, 3).astype(np.float32)), "merged vs oracle merge of the same partials")
    want, _ = A.attention(qt, np.concatenate([ok, lk], 2), np.concatenate([sv, lv], 2), causal_bottom_right=True)
    want = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    _close(single, want, "single pass vs oracle")
    got = merged.float().cpu().numpy()
    ma, rl = A.max_abs(got, want), A.rel_l2(got, want)
    print(f"merged vs union: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert ma <= 2e-2 and rl <= 4e-3

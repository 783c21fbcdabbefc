"""GPU parity of the chunked-prefill kernel, the fused QKV epilogue and the boundary blend.

Tolerances: attention outputs within max-abs 2e-2 and rel-L2 1e-3 of the reference path
(oracle fp64 over the reference's bf16-composed history, output rounded to bf16); the blend is
bit-exact (elementwise bf16 ops in the reference's order); the epilogue is bit-exact except where
the fp32 sum of squares inside RMSNorm rounds differently from torch's reduction order, bounded
at 0.1% of elements and one bf16 ulp.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
from oracle import attention as A
from oracle import bf16
from oracle import model as M

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


def _history(rng, B, Hkv, chunk, p0, L):
    """Final-layer history, the layer's previous chunk and the current chunk up to p0 + L."""

    r = A.plan_regions(p0 + L - 1, chunk)
    rec, cur = r.recent[0], r.current[0]
    assert p0 >= cur, "a prefill piece never crosses a chunk boundary"
    deep = (_bf(rng, (B, Hkv, cur, 128)), _bf(rng, (B, Hkv, cur, 128)))
    prev = (_bf(rng, (B, Hkv, chunk, 128)), _bf(rng, (B, Hkv, chunk, 128))) if cur else None
    n_cur = p0 + L - cur
    cur_kv = (_bf(rng, (B, Hkv, n_cur, 128)), _bf(rng, (B, Hkv, n_cur, 128)))
    logits = bf16.round_bf16(rng.standard_normal(Hkv).astype(np.float32))
    scale = bf16.round_bf16(rng.uniform(0.3, 1.3, Hkv).astype(np.float32))
    return r, deep, prev, cur_kv, logits, scale


def _caches(r, deep, prev, cur_kv, logits, scale, chunk, B, Hkv):
    rec, cur = r.recent[0], r.current[0]
    R = ops.ring_tokens_for_chunk(chunk)
    older = ops.TiledKV.zeros(B, Hkv, max(32, -(-cur // 32) * 32), DEV)
    if cur:
        ops.pack_kv(_t(deep[0]), _t(deep[1]), older)
    ring = ops.TiledKV.zeros(B, Hkv, R, DEV)

    def put(k, v, pos):
        # write token by token range, splitting where the ring wraps
        n = k.shape[2]
        first = min(n, R - pos % R)
        ops.pack_kv(_t(k[:, :, :first]), _t(v[:, :, :first]), ring, token0=pos % R)
        if first < n:
            ops.pack_kv(_t(k[:, :, first:]), _t(v[:, :, first:]), ring, token0=0)

    if cur:
        put(A.blend_chunk_bf16(deep[0][:, :, rec:cur], prev[0], logits),
            A.blend_chunk_bf16(deep[1][:, :, rec:cur], prev[1], logits, scale), rec)
    put(cur_kv[0], cur_kv[1], cur)
    return older, ring, rec % R


@pytest.mark.parametrize("chunk,p0,L", [
    (64, 0, 1), (64, 0, 37), (64, 128, 64), (64, 200, 20), (64, 70, 50), (64, 320, 1),
    (4, 8, 4), (4, 13, 3), (12, 40, 8), (48, 150, 42), (1024, 2048, 300),
])
def test_prefill_regions_match_oracle(chunk, p0, L):
    rng = np.random.default_rng(chunk * 1000 + p0 + L)
    B, Hq, Hkv = 2, 8, 2
    r, deep, prev, cur_kv, logits, scale = _history(rng, B, Hkv, chunk, p0, L)
    older, ring, start = _caches(r, deep, prev, cur_kv, logits, scale, chunk, B, Hkv)
    rec = r.recent[0]
    q = _bf(rng, (B, L, Hq, 128))
    lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
    out = ops.prefill_attention(_t(q), older=older, older_len=rec, vscale=torch.from_numpy(scale).to(DEV),
                                local=ring, local_len=p0 + L - rec, local_start=start, causal=True, lse=lse)
    full_k, full_v = A.compose_history_bf16(deep[0], deep[1], prev and prev[0], prev and prev[1], cur_kv[0], cur_kv[1],
                                            logits, scale, chunk)
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), full_k, full_v, causal_bottom_right=True)
    _close(out, bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32)), f"prefill C={chunk} p0={p0} L={L}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("L,Hq,Hkv,T0,n_local", [(5, 8, 2, 100, 0), (300, 12, 12, 500, 300), (64, 32, 8, 40, 64)])
def test_prefill_bidirectional_local_segment(L, Hq, Hkv, T0, n_local):
    """causal = 0: every query sees every local token (Wan's current block)."""

    rng = np.random.default_rng(L + T0)
    B = 1
    q = _bf(rng, (B, L, Hq, 128))
    ok, ov = _bf(rng, (B, Hkv, T0, 128)), _bf(rng, (B, Hkv, T0, 128))
    older = ops.TiledKV.zeros(B, Hkv, -(-T0 // 32) * 32, DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    kwargs = dict(older=older, older_len=T0, causal=False)
    ks, vs = [ok], [ov]
    if n_local:
        lk, lv = _bf(rng, (B, Hkv, n_local, 128)), _bf(rng, (B, Hkv, n_local, 128))
        ring = ops.TiledKV.zeros(B, Hkv, -(-n_local // 32) * 32 + 32, DEV)
        ops.pack_kv(_t(lk), _t(lv), ring, token0=7)
        kwargs.update(local=ring, local_len=n_local, local_start=7)
        ks.append(lk)
        vs.append(lv)
    out = ops.prefill_attention(_t(q), **kwargs)
    want, _ = A.attention(q.transpose(0, 2, 1, 3), np.concatenate(ks, 2), np.concatenate(vs, 2))
    _close(out, bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32)), f"bidirectional L={L} Hq={Hq}")


@pytest.mark.parametrize("L,Hq,Hkv,causal", [(300, 8, 2, True), (129, 12, 12, False), (520, 32, 8, True)])
def test_prefill_tile_waves_agree_and_match_oracle(L, Hq, Hkv, causal):
    """The 4-wave and 8-wave tiles give the same bits (blocks past a row's causal limit add exact
    zeros) with their keys unsplit (num_splits = 1), and match the oracle, as does the automatic
    call (whose small grid splits the tiles' keys); 4 x 32 and 8 x 32 row tiles end at different
    rows, so tile edges fall inside GQA groups and causal steps."""

    rng = np.random.default_rng(L + Hq)
    B, T0, n_local = 2, 233, L + 61
    q = _bf(rng, (B, L, Hq, 128))
    ok, ov = _bf(rng, (B, Hkv, T0, 128)), _bf(rng, (B, Hkv, T0, 128))
    lk, lv = _bf(rng, (B, Hkv, n_local, 128)), _bf(rng, (B, Hkv, n_local, 128))
    older = ops.TiledKV.zeros(B, Hkv, -(-T0 // 32) * 32, DEV)
    ops.pack_kv(_t(ok), _t(ov), older)
    ring_tokens = -(-n_local // 32) * 32 + 32
    ring = ops.TiledKV.zeros(B, Hkv, ring_tokens, DEV)
    start = ring_tokens - 40  # the segment wraps
    ops.pack_kv(_t(lk[:, :, :40]), _t(lv[:, :, :40]), ring, token0=start)
    ops.pack_kv(_t(lk[:, :, 40:]), _t(lv[:, :, 40:]), ring, token0=0)
    kw = dict(older=older, older_len=T0, local=ring, local_len=n_local, local_start=start, causal=causal)
    outs, lses = [], []
    for tw in (4, 8, 0):
        lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
        outs.append(ops.prefill_attention(_t(q), tile_waves=tw, lse=lse, num_splits=1, **kw))
        lses.append(lse)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert torch.equal(lses[0], lses[1]) and torch.equal(lses[0], lses[2])
    want, want_lse = A.attention(q.transpose(0, 2, 1, 3), np.concatenate([ok, lk], 2), np.concatenate([ov, lv], 2),
                                 causal_bottom_right=causal)
    want = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    _close(outs[0], want, f"tile waves L={L} Hq={Hq}")
    np.testing.assert_allclose(lses[0].cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    lse = torch.empty((B, L, Hq), dtype=torch.float32, device=DEV)
    _close(ops.prefill_attention(_t(q), lse=lse, **kw), want, f"automatic (key splits) L={L} Hq={Hq}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse.transpose(0, 2, 1), rtol=1e-4, atol=1e-4)
    with pytest.raises(RuntimeError, match="tile_waves"):
        ops.prefill_attention(_t(q), tile_waves=5, **kw)


def test_prefill_agrees_with_decode_for_single_token():
    rng = np.random.default_rng(5)
    B, Hq, Hkv, C, p = 3, 16, 4, 64, 250
    r, deep, prev, cur_kv, logits, scale = _history(rng, B, Hkv, C, p, 1)
    older, ring, start = _caches(r, deep, prev, cur_kv, logits, scale, C, B, Hkv)
    rec = r.recent[0]
    q = _bf(rng, (B, 1, Hq, 128))
    vs = torch.from_numpy(scale).to(DEV)
    a = ops.prefill_attention(_t(q), older=older, older_len=rec, vscale=vs, local=ring, local_len=p + 1 - rec, local_start=start)
    d = ops.decode_attention(_t(q)[:, 0], older=older, older_len=rec, vscale=vs, local=ring, local_len=p + 1 - rec,
                             local_start=start)
    _close(a[:, 0], d.float().cpu().numpy(), "prefill L=1 vs decode")


def _torch_fp32_attention(q, k, v, n_local_visible_last):
    """fp32 GQA attention on the GPU with a bottom-right causal mask over the last keys.
    q [Hq, L, D], k/v [Hkv, T, D] float32 tensors; query i sees keys [0, T - L + i]."""

    Hq, L, _ = q.shape
    Hkv, T, _ = k.shape
    g = Hq // Hkv
    kk = k.repeat_interleave(g, 0).contiguous()
    vv = v.repeat_interleave(g, 0).contiguous()
    scores = torch.matmul(q, kk.transpose(1, 2).contiguous()) * (128 ** -0.5)
    i = torch.arange(L, device=q.device)[:, None]
    j = torch.arange(T, device=q.device)[None, :]
    scores = scores.masked_fill(j > T - L + i, float("-inf"))
    return torch.matmul(torch.softmax(scores, -1), vv)


def test_prefill_config3_piece_matches_torch_fp32():
    """The longest config-3 prefill piece at full per-sequence size (C = 1024, chunk 7 of an
    8192-token prompt: 6144 older + 1024 blended recent + 1024 causal current keys, Hq 32, Hkv 8)
    against fp32 attention over the same composed keys; B = 2 of the benchmark's 32 sequences."""

    rng = np.random.default_rng(77)
    B, Hq, Hkv, C, p0, L = 2, 32, 8, 1024, 7 * 1024, 1024
    r, deep, prev, cur_kv, logits, scale = _history(rng, B, Hkv, C, p0, L)
    older, ring, start = _caches(r, deep, prev, cur_kv, logits, scale, C, B, Hkv)
    rec = r.recent[0]
    q = _bf(rng, (B, L, Hq, 128))
    ws = torch.empty(ops.prefill_workspace_bytes(B, Hkv, rec, p0 + L - rec, start % 32), dtype=torch.uint8, device=DEV)
    out = ops.prefill_attention(_t(q), older=older, older_len=rec, vscale=torch.from_numpy(scale).to(DEV), local=ring,
                                local_len=p0 + L - rec, local_start=start, causal=True, workspace=ws)
    full_k, full_v = A.compose_history_bf16(deep[0], deep[1], prev[0], prev[1], cur_kv[0], cur_kv[1], logits, scale, C)
    for b in range(B):
        want = _torch_fp32_attention(torch.from_numpy(q[b].transpose(1, 0, 2).copy()).to(DEV),
                                     torch.from_numpy(np.ascontiguousarray(full_k[b], np.float32)).to(DEV),
                                     torch.from_numpy(np.ascontiguousarray(full_v[b], np.float32)).to(DEV), L)
        want = want.transpose(0, 1).bfloat16().float().cpu().numpy()
        _close(out[b], want, f"config-3 piece 7, sequence {b}")


def test_prefill_workspace_contract():
    """The workspace query is exact for host-constant lengths and a short workspace is rejected."""

    B, Hq, Hkv = 2, 8, 2
    older = ops.TiledKV.zeros(B, Hkv, 256, DEV)
    ring = ops.TiledKV.zeros(B, Hkv, 128, DEV)
    q = torch.zeros((B, 40, Hq, 128), dtype=torch.bfloat16, device=DEV)
    kw = dict(older=older, older_len=100, local=ring, local_len=40, local_start=70)
    need = ops.prefill_workspace_bytes(B, Hkv, 100, 40, 70 % 32)
    # fp16 V of 6 blocks, a 16-byte row of block flags per (sequence, kv head), one 16-byte word
    assert need == B * Hkv * ((4 + 2) * 8192 + 16) + 16
    ops.prefill_attention(q, workspace=torch.empty(need, dtype=torch.uint8, device=DEV), **kw)
    with pytest.raises(ValueError, match="workspace"):
        ops.prefill_attention(q, workspace=torch.empty(need - 8192, dtype=torch.uint8, device=DEV), **kw)


# ------------------------------------------------------------------ epilogue
def _ulp_stats(actual: np.ndarray, expected: np.ndarray):
    diff = actual.view(np.uint32).astype(np.int64) - expected.view(np.uint32).astype(np.int64)
    mism = np.count_nonzero(diff)
    return mism / diff.size, int(np.max(np.abs(diff >> 16))) if mism else 0


@pytest.mark.parametrize("B,L,p0,last,C", [(2, 1, 37, False, 32), (3, 17, 100, True, 32), (1, 64, 0, True, 32),
                                          (2, 300, 1000, True, 1024), (2, 200, 1950, True, 1024), (1, 1024, 3072, False, 1024)])
def test_qkv_epilogue_matches_reference_ops(B, L, p0, last, C):
    """Decode-sized calls take one wave per (token, head); calls of 16 tokens or more the block form
    (16-byte accesses, V tiles through LDS), here with partial blocks at both ends of the call and a
    ring that wraps inside it (positions 1950-2149 in a 2048-token ring)."""

    rng = np.random.default_rng(B * 100 + L)
    Hq, Hkv = 8, 2
    q = _bf(rng, (B, L, Hq * 128))
    k = _bf(rng, (B, L, Hkv * 128))
    v = _bf(rng, (B, L, Hkv * 128))
    cfg = M.config_8b(num_hidden_layers=2)
    inv, sc = M.rope_inv_freq(cfg)
    pos = torch.arange(p0, p0 + L)[None].expand(B, L)
    cos, sin = M.rotary_cos_sin(inv, sc, pos, torch.bfloat16)
    qw = torch.linspace(0.7, 1.3, 128).bfloat16()
    kw = torch.linspace(1.2, 0.8, 128).bfloat16()
    ring = ops.TiledKV.zeros(B, Hkv, ops.ring_tokens_for_chunk(C), DEV)
    deep = ops.TiledKV.zeros(B, Hkv, -(-(p0 + L) // 32) * 32, DEV) if last else None
    q_out = ops.qkv_epilogue(_t(q), _t(k), _t(v), cos.to(DEV), sin.to(DEV), num_q_heads=Hq, num_kv_heads=Hkv,
                             q_norm_weight=qw.to(DEV), k_norm_weight=kw.to(DEV), eps=1e-5, positions=p0, ring=ring, deep=deep)
    # the reference's ops in bf16 on the CPU (modeling.py:100-106)
    tq = torch.from_numpy(q).bfloat16().view(B, L, Hq, 128).transpose(1, 2)
    tk = torch.from_numpy(k).bfloat16().view(B, L, Hkv, 128).transpose(1, 2)
    rq, rk = M.apply_rope(tq, tk, cos, sin)
    qn, kn = M.RMSNorm(128, 1e-5).bfloat16(), M.RMSNorm(128, 1e-5).bfloat16()
    with torch.no_grad():
        qn.weight.copy_(qw)
        kn.weight.copy_(kw)
        rq, rk = qn(rq), kn(rk)
    frac, ulp = _ulp_stats(q_out.float().cpu().numpy(), rq.transpose(1, 2).float().numpy())
    print(f"epilogue q: mismatch fraction {frac:.2e}, max ulp {ulp}", flush=True)
    assert frac <= 1e-3 and ulp <= 1
    R = ring.capacity_tokens
    got_k = [ops.unpack_kv(ring, (p0 + i) % R, 1)[0] for i in range(L)]
    got_v = [ops.unpack_kv(ring, (p0 + i) % R, 1)[1] for i in range(L)]
    got_k = torch.cat(got_k, 2).float().cpu().numpy()
    got_v = torch.cat(got_v, 2).float().cpu().numpy()
    frac, ulp = _ulp_stats(got_k, rk.float().numpy())
    assert frac <= 1e-3 and ulp <= 1
    assert np.array_equal(got_v, torch.from_numpy(v).view(B, L, Hkv, 128).transpose(1, 2).numpy())
    if last:
        dk, dv = ops.unpack_kv(deep, p0, L)
        assert np.array_equal(dk.float().cpu().numpy(), got_k) and np.array_equal(dv.float().cpu().numpy(), got_v)


@pytest.mark.parametrize("L", [8, 40])
def test_qkv_epilogue_signed_zeros_and_tiny_values(L):
    """Rows of zeros (both signs), zeros mixed into ordinary rows and rows of tiny values (whose
    rotary products are fp32 denormals) through both epilogue forms (8 tokens: one wave per (token,
    head); 40: the block form), against the reference's bf16 torch ops on the CPU: every bit equal,
    the sign of each zero included, up to the RMSNorm summation-order flips the other epilogue tests
    allow (at most 0.1 % of values, one ulp)."""

    rng = np.random.default_rng(400 + L)
    B, Hq, Hkv, p0 = 2, 8, 2, 5

    def rows(heads):
        x = _bf(rng, (B, L, heads, 128))
        x[0, 0] = 0.0                                          # a token of +0 rows
        x[0, 1] = -0.0                                         # and of -0 rows
        x[1, 2, :, ::3] = np.where(rng.random((heads, 43)) < 0.5, 0.0, -0.0)  # zeros among values
        x[1, 3] = bf16.round_bf16((rng.standard_normal((heads, 128)) * 1e-36).astype(np.float32))
        return x.reshape(B, L, heads * 128)

    q, k, v = rows(Hq), rows(Hkv), _bf(rng, (B, L, Hkv * 128))
    cfg = M.config_8b(num_hidden_layers=2)
    inv, sc = M.rope_inv_freq(cfg)
    cos, sin = M.rotary_cos_sin(inv, sc, torch.arange(p0, p0 + L)[None].expand(B, L), torch.bfloat16)
    qw = torch.linspace(0.7, 1.3, 128).bfloat16()
    kw = torch.linspace(1.2, 0.8, 128).bfloat16()
    ring = ops.TiledKV.zeros(B, Hkv, ops.ring_tokens_for_chunk(32), DEV)
    q_out = ops.qkv_epilogue(_t(q), _t(k), _t(v), cos.to(DEV), sin.to(DEV), num_q_heads=Hq, num_kv_heads=Hkv,
                             q_norm_weight=qw.to(DEV), k_norm_weight=kw.to(DEV), eps=1e-5, positions=p0, ring=ring)
    tq = torch.from_numpy(q).bfloat16().view(B, L, Hq, 128).transpose(1, 2)
    tk = torch.from_numpy(k).bfloat16().view(B, L, Hkv, 128).transpose(1, 2)
    rq, rk = M.apply_rope(tq, tk, cos, sin)
    qn, kn = M.RMSNorm(128, 1e-5).bfloat16(), M.RMSNorm(128, 1e-5).bfloat16()
    with torch.no_grad():
        qn.weight.copy_(qw)
        kn.weight.copy_(kw)
        rq, rk = qn(rq), kn(rk)
    want_q = rq.transpose(1, 2).float().numpy()
    got_q = q_out.float().cpu().numpy()
    assert np.count_nonzero(want_q == 0) > 1000 and np.count_nonzero(np.signbit(want_q) & (want_q == 0)) > 100
    frac, ulp = _ulp_stats(got_q, want_q)
    assert frac <= 1e-3 and ulp <= 1, (frac, ulp)
    got_k = torch.cat([ops.unpack_kv(ring, p0 + i, 1)[0] for i in range(L)], 2).float().cpu().numpy()
    frac, ulp = _ulp_stats(got_k, rk.float().numpy())
    assert frac <= 1e-3 and ulp <= 1, (frac, ulp)


@pytest.mark.parametrize("rounding", ["torch", "vllm"])
def test_epilogue_forms_agree_bit_for_bit(rounding):
    """The per-token kernel (calls of fewer than 16 tokens) and the block form (16 or more) sum the
    RMSNorm squares in the same fixed order, so the same rows give the same bits either way: 72
    tokens of 2 sequences as one call against nine calls of 8 tokens (normalised queries, ring and
    shared-store bytes), with norm gains and a ring V multiplier on the vLLM contract."""

    rng = np.random.default_rng(61 + (rounding == "vllm"))
    B, L, Hq, Hkv, p0 = 2, 72, 16, 4, 37
    q, k, v = _bf(rng, (B, L, Hq * 128)), _bf(rng, (B, L, Hkv * 128)), _bf(rng, (B, L, Hkv * 128))
    cfg = M.config_8b(num_hidden_layers=2)
    inv, sc = M.rope_inv_freq(cfg)
    cos, sin = M.rotary_cos_sin(inv, sc, torch.arange(p0, p0 + L)[None].expand(B, L), torch.bfloat16)
    cos, sin = cos.to(DEV), sin.to(DEV)
    qw = torch.from_numpy(bf16.round_bf16(rng.uniform(0.5, 1.6, 128).astype(np.float32))).bfloat16().to(DEV)
    kw = torch.from_numpy(bf16.round_bf16(rng.uniform(0.5, 1.6, 128).astype(np.float32))).bfloat16().to(DEV)
    vmul = torch.from_numpy(rng.uniform(0.5, 2.0, Hkv).astype(np.float32)).to(DEV) if rounding == "vllm" else None
    kwargs = dict(num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=qw, k_norm_weight=kw, eps=1e-5, rounding=rounding,
                  ring_v_mul=vmul)
    stores = [(ops.TiledKV.zeros(B, Hkv, 256, DEV), ops.TiledKV.zeros(B, Hkv, 128, DEV)) for _ in range(2)]
    whole = ops.qkv_epilogue(_t(q), _t(k), _t(v), cos, sin, positions=p0, ring=stores[0][0], deep=stores[0][1], **kwargs)
    parts = []
    for i in range(0, L, 8):
        sl = slice(i, i + 8)
        parts.append(ops.qkv_epilogue(_t(q)[:, sl], _t(k)[:, sl], _t(v)[:, sl], cos[:, sl], sin[:, sl], positions=p0 + i,
                                      ring=stores[1][0], deep=stores[1][1], **kwargs))
    assert torch.equal(whole, torch.cat(parts, 1)), "normalised queries differ between the two forms"
    for a, b in zip(stores[0], stores[1]):
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v), "cache bytes differ between the two forms"


# ------------------------------------------------------------------ blend
@pytest.mark.parametrize("chunk,cidx", [(64, 1), (64, 4), (1024, 2), (4, 3), (12, 5)])
def test_blend_chunk_bit_exact(chunk, cidx):
    rng = np.random.default_rng(chunk + cidx)
    layers, B, H = 3, 2, 4
    R = ops.ring_tokens_for_chunk(chunk)
    start = cidx * chunk
    deep_k, deep_v = _bf(rng, (B, H, start + chunk, 128)), _bf(rng, (B, H, start + chunk, 128))
    deep = ops.TiledKV.zeros(B, H, -(-(start + chunk) // 32) * 32, DEV)
    ops.pack_kv(_t(deep_k), _t(deep_v), deep)
    ring_k = torch.zeros((layers, B, H, R // 32, 4096), dtype=torch.bfloat16, device=DEV)
    ring_v = torch.zeros_like(ring_k)
    own = []
    for l in range(layers):
        ok, ov = _bf(rng, (B, H, R, 128)), _bf(rng, (B, H, R, 128))
        ops.cache_pack(_t(ok), ring_k[l], ops.KIND_K)
        ops.cache_pack(_t(ov), ring_v[l], ops.KIND_V)
        own.append((ok, ov))
    logits = bf16.round_bf16(rng.standard_normal((layers, H)).astype(np.float32))
    s = bf16.round_bf16(rng.uniform(0.1, 1.3, (layers, H)).astype(np.float32))
    alpha = bf16.round_bf16(A.sigmoid(logits).astype(np.float32))
    om = bf16.rsub(alpha, 1.0)
    ops.blend_chunk(ring_k, ring_v, deep, batch=B, chunk_start=start, chunk_len=chunk,
                    alpha=torch.from_numpy(alpha.ravel()).to(DEV), one_minus_alpha=torch.from_numpy(om.ravel()).to(DEV),
                    vscale=torch.from_numpy(s.ravel()).to(DEV))
    pos = np.arange(start, start + chunk) % R
    for l in range(layers):
        gk = ops.cache_unpack(ring_k[l], ops.KIND_K, 0, R).float().cpu().numpy()
        gv = ops.cache_unpack(ring_v[l], ops.KIND_V, 0, R).float().cpu().numpy()
        wk = A.blend_chunk_bf16(deep_k[:, :, start:], own[l][0][:, :, pos], logits[l])
        wv = A.blend_chunk_bf16(deep_v[:, :, start:], own[l][1][:, :, pos], logits[l], s[l])
        assert np.array_equal(gk[:, :, pos], wk) and np.array_equal(gv[:, :, pos], wv)
        # every other ring token is untouched
        rest = np.setdiff1d(np.arange(R), pos)
        assert np.array_equal(gk[:, :, rest], own[l][0][:, :, rest]) and np.array_equal(gv[:, :, rest], own[l][1][:, :, rest])


def _torch_rmsnorm(x, w, eps):
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w * h.to(torch.bfloat16)


@pytest.mark.parametrize("rows,hidden,add", [(1, 4096, False), (32, 4096, True), (7, 1536, True), (33, 8, False),
                                             (3, 16384, True)])
def test_rmsnorm_matches_llama_rmsnorm(rows, hidden, add):
    """lkv_rmsnorm against transformers' LlamaRMSNorm expression in torch (with the residual add
    before it, a bf16 add): the residual is bit-exact; the normalised values differ only where the
    fp32 sum of squares is rounded in another order (at most one bf16 ulp, on few elements)."""

    g = torch.Generator(device=DEV).manual_seed(rows * 7 + hidden)
    x = (torch.randn((rows, hidden), generator=g, device=DEV) * 3).bfloat16()
    res = torch.randn((rows, hidden), generator=g, device=DEV).bfloat16()
    w = (1 + 0.1 * torch.randn(hidden, generator=g, device=DEV)).bfloat16()
    eps = 1e-5
    want_res = res + x if add else None
    want = _torch_rmsnorm(want_res if add else x, w, eps)
    r = res.clone()
    got = ops.rmsnorm(x, w, eps, residual=r if add else None)
    torch.cuda.synchronize()
    if add:
        assert torch.equal(r, want_res)
    else:
        assert torch.equal(r, res)
    diff = (got.float() - want.float()).abs()
    ulp = want.float().abs().clamp_min(1e-30) * 2.0 ** -7
    assert bool((diff <= ulp).all()), float((diff / ulp).max())
    assert float((diff > 0).float().mean()) < 0.01


def test_silu_mul_bit_exact():
    g = torch.Generator(device=DEV).manual_seed(11)
    gate = (torch.randn((37, 14336), generator=g, device=DEV) * 4).bfloat16()
    up = torch.randn((37, 14336), generator=g, device=DEV).bfloat16()
    got = ops.silu_mul(gate, up)
    want = torch.nn.functional.silu(gate) * up
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_lazy_rescale_threshold_regimes(causal):
    """The tile kernel keeps block 0's exact row maximum and rescales only when a later
    probability reaches 2^9.  Rows here see near-zero scores in block 0 and one later key (older
    block 2) whose exp2 argument jumps by d: d from 0.5 to 80 across the rows, so some rows keep the
    old reference with probabilities up to 2^8.99 in fp16, some sit just past the threshold and
    rescale once, some jump far beyond it.  A second key (local block 1) jumps further still on
    half the rows (a second rescale).  Tile kernel (automatic / 4 / 8 waves) against the fp64
    oracle; causal runs put the second key inside every row's visible range."""

    rng = np.random.default_rng(91)
    B, Hkv, G, L, T0, n_local = 1, 2, 4, 64, 96, 128
    Hq = G * Hkv
    c = 128 ** -0.5 * 1.4426950408889634  # exp2 argument per unit of raw score
    jumps = np.array([0.5, 2.0, 5.0, 8.5, 8.95, 9.05, 9.5, 12.0, 20.0, 40.0, 80.0, 1.0, 8.8, 9.2, 30.0, 0.0])
    a = (jumps / (128 * c)).astype(np.float32)  # q = a * ones: the special key (k = ones) scores 128 a
    rows = (np.arange(L)[:, None] * Hq + np.arange(Hq)[None, :]) % len(jumps)
    q = a[rows][None, :, :, None] * np.ones((1, 1, 1, 128), np.float32)
    q = bf16.round_bf16((q + 0.002 * rng.standard_normal((B, L, Hq, 128))).astype(np.float32))
    keys = T0 + n_local
    k = bf16.round_bf16((0.05 * rng.standard_normal((B, Hkv, keys, 128))).astype(np.float32))
    k[:, :, 70] = 1.0  # older block 2
    k[:, :, T0 + 40, :] = bf16.round_bf16(np.where(np.arange(128) < 64, 1.5, 1.0).astype(np.float32))  # local block 1
    v = _bf(rng, (B, Hkv, keys, 128))
    older = ops.TiledKV.zeros(B, Hkv, 128, DEV)
    ops.pack_kv(_t(k[:, :, :T0]), _t(v[:, :, :T0]), older)
    ring = ops.TiledKV.zeros(B, Hkv, n_local, DEV)
    ops.pack_kv(_t(k[:, :, T0:]), _t(v[:, :, T0:]), ring)
    kw = dict(older=older, older_len=T0, local=ring, local_len=n_local, causal=causal)
    want, _ = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=causal)
    want = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    for tw in (0, 4, 8):
        out = ops.prefill_attention(_t(q), tile_waves=tw, **kw)
        _close(out, want, f"rescale regimes causal={causal} tile_waves={tw}")


@pytest.mark.parametrize("L,G", [(160, 4), (12, 4)])
def test_prefill_extreme_score_ranges(L, G):
    """Regression: rows whose first visible scores are all far below zero (scaled scores near -180,
    as q/k RMSNorm gains of ~8 produce) once made the tile kernel rescale its empty state by
    2^(0 - m c) = inf and return NaN rows.  Keys of the first blocks point against the queries,
    later keys along them (the running maximum then jumps by ~360), causal, over an older segment
    and the local ring; the tile kernel (4 / 8 / automatic waves) and, for the short call, the
    decode kernel, against the fp64 oracle."""

    rng = np.random.default_rng(L)
    B, Hkv, T0 = 2, 2, 40
    Hq = G * Hkv
    n_local = L + 70
    u = bf16.round_bf16(np.full(128, 1.0, np.float32))
    q = bf16.round_bf16((16 * u + rng.standard_normal((B, L, Hq, 128))).astype(np.float32))
    keys = T0 + n_local
    sign = np.where(np.arange(keys) < 48, -1.0, 1.0)[None, None, :, None]
    k = bf16.round_bf16((sign * u + 0.3 * rng.standard_normal((B, Hkv, keys, 128))).astype(np.float32))
    v = _bf(rng, (B, Hkv, keys, 128))
    older = ops.TiledKV.zeros(B, Hkv, 64, DEV)
    ops.pack_kv(_t(k[:, :, :T0]), _t(v[:, :, :T0]), older)
    ring = ops.TiledKV.zeros(B, Hkv, -(-n_local // 32) * 32, DEV)
    ops.pack_kv(_t(k[:, :, T0:]), _t(v[:, :, T0:]), ring)
    kw = dict(older=older, older_len=T0, local=ring, local_len=n_local, causal=True)
    want, _ = A.attention(q.transpose(0, 2, 1, 3), k, v, causal_bottom_right=True)
    want = bf16.round_bf16(want.transpose(0, 2, 1, 3).astype(np.float32))
    for tw in (0, 4, 8):
        out = ops.prefill_attention(_t(q), tile_waves=tw, **kw)
        assert not torch.isnan(out.float()).any(), f"tile_waves={tw}: NaN rows"
        _close(out, want, f"extreme scores L={L} G={G} tile_waves={tw}")

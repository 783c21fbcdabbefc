"""GPU checks of the torch custom operators (lastkv_amd.torch_ops): each equals the ctypes call it
wraps bit for bit, torch.library.opcheck accepts their schemas and fake implementations, and a
decode-step fragment compiled with torch.compile (aot_eager backend, full graph: dynamo and
AOTAutograd trace it, no code generation) gives the eager results."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lastkv_amd import ops
import lastkv_amd.torch_ops  # noqa: F401

pytestmark = pytest.mark.gpu

DEV = "cuda"
L = torch.ops.lastkv


def _r(g, shape, dtype=torch.bfloat16):
    return torch.randn(shape, generator=g, device=DEV).to(dtype)


def test_attention_ops_equal_the_ctypes_calls():
    g = torch.Generator(device=DEV).manual_seed(11)
    B, Hq, Hkv, T0, n1, start = 3, 16, 4, 150, 70, 9
    older = ops.TiledKV.zeros(B, Hkv, 160, DEV)
    ops.pack_kv(_r(g, (B, Hkv, T0, 128)), _r(g, (B, Hkv, T0, 128)), older)
    ring = ops.TiledKV.zeros(B, Hkv, 96, DEV)
    ops.pack_kv(_r(g, (B, Hkv, n1, 128)), _r(g, (B, Hkv, n1, 128)), ring, token0=start)
    vs = torch.rand(Hkv, generator=g, device=DEV) + 0.5
    q = _r(g, (B, Hq, 128))
    want = ops.decode_attention(q, older=older, older_len=T0, vscale=vs, local=ring, local_len=n1, local_start=start)
    got = L.decode_attention(q, older.k, older.v, None, T0, None, vs, ring.k, ring.v, None, n1, None, start, None, 0, 0.0, 0)
    assert torch.equal(got, want)
    lens = torch.full((B,), n1, dtype=torch.int32, device=DEV)
    got = L.decode_attention(q, older.k, older.v, None, T0, None, vs, ring.k, ring.v, lens, 0, None, start, None, 0, 0.0, 2)
    assert torch.equal(got, ops.decode_attention(q, older=older, older_len=T0, vscale=vs, local=ring, local_len=lens,
                                                 local_start=start, num_splits=2))
    Lq = 40
    qp = _r(g, (B, Lq, Hq, 128))
    want = ops.prefill_attention(qp, older=older, older_len=T0, vscale=vs, local=ring, local_len=n1, local_start=start,
                                 causal=True)
    got = L.prefill_attention(qp, older.k, older.v, None, T0, None, vs, ring.k, ring.v, None, n1, None, start, None, 0,
                              True, 0.0)
    assert torch.equal(got, want)
    # paged: the same keys through a head-major pool and block tables
    pages = B * 8 + 1
    pool = ops.PagedKV.zeros(pages, Hkv, DEV)
    perm = torch.randperm(pages - 1, generator=torch.Generator().manual_seed(2)).to(DEV).int().view(B, 8)
    for b in range(B):
        for j in range(5):  # older blocks 0-4 (150 tokens)
            pool.kp[perm[b, j]] = older.k[b, :, j]
            pool.vp[perm[b, j]] = older.v[b, :, j]
    got = L.decode_attention(q, pool.k, pool.v, None, T0, perm, vs, None, None, None, 0, None, 0, None, 0, 0.0, 0)
    assert torch.equal(got, ops.decode_attention(q, older=older, older_len=T0, vscale=vs))
    # the vLLM contract's output scale
    s = (torch.rand(Hkv, generator=g, device=DEV) + 0.5).bfloat16().float()
    got = L.decode_attention(q, older.k, older.v, None, T0, None, None, ring.k, ring.v, None, n1, None, start, None, 0,
                             0.0, 0, s)
    assert torch.equal(got, ops.decode_attention(q, older=older, older_len=T0, local=ring, local_len=n1,
                                                 local_start=start, out_scale=s))
    got = L.prefill_attention(qp, older.k, older.v, None, T0, None, None, ring.k, ring.v, None, n1, None, start, None, 0,
                              True, 0.0, s)
    assert torch.equal(got, ops.prefill_attention(qp, older=older, older_len=T0, local=ring, local_len=n1,
                                                  local_start=start, causal=True, out_scale=s))


def test_epilogue_merge_norm_ops_equal_the_ctypes_calls():
    g = torch.Generator(device=DEV).manual_seed(12)
    B, Lt, Hq, Hkv = 2, 37, 8, 2
    q, k, v = _r(g, (B, Lt, Hq * 128)), _r(g, (B, Lt, Hkv * 128)), _r(g, (B, Lt, Hkv * 128))
    cos, sin = _r(g, (1, Lt, 128)), _r(g, (1, Lt, 128))
    w = (torch.rand(128, generator=g, device=DEV) + 0.5).bfloat16()
    rings = [ops.TiledKV.zeros(B, Hkv, 64, DEV) for _ in range(2)]
    deeps = [ops.TiledKV.zeros(B, Hkv, 64, DEV) for _ in range(2)]
    q_outs = [torch.empty((B, Lt, Hq, 128), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    ops.qkv_epilogue(q, k, v, cos, sin, num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=w, k_norm_weight=w, eps=1e-6,
                     positions=5, ring=rings[0], deep=deeps[0], q_out=q_outs[0])
    L.qkv_epilogue(q, k, v, cos, sin, Hq, Hkv, w, w, 1e-6, None, 5, q_outs[1], rings[1].k, rings[1].v, None, 0,
                   deeps[1].k, deeps[1].v, None)
    assert torch.equal(q_outs[0], q_outs[1])
    for a, b in ((rings[0], rings[1]), (deeps[0], deeps[1])):
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    # the vLLM contract: fused-QKV rounding and V / s rings
    inv = 1.0 / (torch.rand(Hkv, generator=g, device=DEV) + 0.5).bfloat16().float()
    rings = [ops.TiledKV.zeros(B, Hkv, 64, DEV) for _ in range(2)]
    ops.qkv_epilogue(q, k, v, cos, sin, num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=w, k_norm_weight=w, eps=1e-6,
                     positions=5, ring=rings[0], q_out=q_outs[0], rounding="vllm", ring_v_mul=inv)
    L.qkv_epilogue(q, k, v, cos, sin, Hq, Hkv, w, w, 1e-6, None, 5, q_outs[1], rings[1].k, rings[1].v, None, 0,
                   None, None, None, 1, inv)
    assert torch.equal(q_outs[0], q_outs[1])
    assert torch.equal(rings[0].k, rings[1].k) and torch.equal(rings[0].v, rings[1].v)
    T, H = 33, 8
    o1, o2 = _r(g, (T, H, 128)), _r(g, (T, H, 128))
    l1, l2 = torch.randn((T, H), generator=g, device=DEV), torch.randn((T, H), generator=g, device=DEV)
    l1[::4] = -float("inf")
    want_o, want_l = ops.merge_state(o1, l1, o2, l2)
    got_o, got_l = L.merge_states(o1, l1, o2, l2, None)
    assert torch.equal(got_o, want_o) and torch.equal(got_l, want_l)
    x = _r(g, (17, 4096))
    wn = (torch.rand(4096, generator=g, device=DEV) + 0.5).bfloat16()
    assert torch.equal(L.rmsnorm(x, wn, 1e-5), ops.rmsnorm(x, wn, 1e-5))
    assert torch.equal(L.silu_mul(x, x), ops.silu_mul(x, x))


def test_ragged_ops_equal_the_ctypes_calls():
    """The varlen forms (cu_seqlens) of the prefill and epilogue operators: three sequences of 1, 40
    and 7 query tokens in one call each, equal to the ctypes calls bit for bit, and opcheck-clean."""

    g = torch.Generator(device=DEV).manual_seed(12)
    B, Hq, Hkv, T0 = 3, 8, 2, 200
    lengths = [1, 40, 7]
    T = sum(lengths)
    cu = torch.tensor([0, 1, 41, 48], dtype=torch.int32, device=DEV)
    older = ops.TiledKV.zeros(B, Hkv, 224, DEV)
    ops.pack_kv(_r(g, (B, Hkv, T0, 128)), _r(g, (B, Hkv, T0, 128)), older)
    ring = ops.TiledKV.zeros(B, Hkv, 96, DEV)
    ops.pack_kv(_r(g, (B, Hkv, 60, 128)), _r(g, (B, Hkv, 60, 128)), ring, token0=5)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    older_len, local_len, local_start = i32([T0, 150, 31]), i32([60, 60, 60]), i32([5, 5, 5])
    q = _r(g, (T, Hq, 128))
    want = ops.prefill_attention(q, older=older, older_len=older_len, local=ring, local_len=local_len,
                                 local_start=local_start, causal=True, cu_seqlens_q=cu, max_seqlen_q=40)
    args = (q, older.k, older.v, older_len, 0, None, None, ring.k, ring.v, local_len, 0, local_start, 0, None, 0, True,
            0.0, None, cu, 40, 0)
    assert torch.equal(L.prefill_attention(*args), want)
    torch.library.opcheck(L.prefill_attention, args)
    # the same with the host copy of the offsets (an int32 CPU tensor), which only plans the launches
    hargs = args + (cu.cpu(),)
    assert torch.equal(L.prefill_attention(*hargs), want)
    torch.library.opcheck(L.prefill_attention, hargs)
    qq, kk, vv = _r(g, (T, Hq * 128)), _r(g, (T, Hkv * 128)), _r(g, (T, Hkv * 128))
    cs = _r(g, (T, 128))
    pos = i32([300, 41, 77])
    rings = [ops.TiledKV.zeros(B, Hkv, 512, DEV) for _ in range(2)]
    q_outs = [torch.empty((T, Hq, 128), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    ops.qkv_epilogue(qq, kk, vv, cs, cs, num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=None, k_norm_weight=None,
                     eps=1e-6, positions=pos, ring=rings[0], q_out=q_outs[0], cu_seqlens=cu, max_seqlen=40)
    eargs = (qq, kk, vv, cs, cs, Hq, Hkv, None, None, 1e-6, pos, 0, q_outs[1], rings[1].k, rings[1].v, None, 0, None,
             None, None, 0, None, cu, 40)
    L.qkv_epilogue(*eargs)
    assert torch.equal(q_outs[0], q_outs[1])
    assert torch.equal(rings[0].k, rings[1].k) and torch.equal(rings[0].v, rings[1].v)
    torch.library.opcheck(L.qkv_epilogue, eargs)


def test_opcheck():
    g = torch.Generator(device=DEV).manual_seed(13)
    B, Hq, Hkv, T0 = 2, 8, 2, 96
    older = ops.TiledKV.zeros(B, Hkv, 96, DEV)
    ops.pack_kv(_r(g, (B, Hkv, T0, 128)), _r(g, (B, Hkv, T0, 128)), older)
    q = _r(g, (B, Hq, 128))
    torch.library.opcheck(L.decode_attention, (q, older.k, older.v, None, T0, None, None, None, None, None, 0, None, 0,
                                               None, 0, 0.0, 0))
    qp = _r(g, (B, 20, Hq, 128))
    ring = ops.TiledKV.zeros(B, Hkv, 32, DEV)
    ops.pack_kv(_r(g, (B, Hkv, 20, 128)), _r(g, (B, Hkv, 20, 128)), ring)
    torch.library.opcheck(L.prefill_attention, (qp, older.k, older.v, None, T0, None, None, ring.k, ring.v, None, 20,
                                                None, 0, None, 0, True, 0.0))
    T, H = 9, 4
    o = _r(g, (T, H, 128))
    lse = torch.randn((T, H), generator=g, device=DEV)
    torch.library.opcheck(L.merge_states, (o, lse, o, lse, None))
    x = _r(g, (5, 256))
    torch.library.opcheck(L.rmsnorm, (x, torch.ones(256, dtype=torch.bfloat16, device=DEV), 1e-5))
    torch.library.opcheck(L.silu_mul, (x, x))
    Lt = 3
    qq, kk, vv = _r(g, (B, Lt, Hq * 128)), _r(g, (B, Lt, Hkv * 128)), _r(g, (B, Lt, Hkv * 128))
    cs = _r(g, (1, Lt, 128))
    q_out = torch.empty((B, Lt, Hq, 128), dtype=torch.bfloat16, device=DEV)
    ring2 = ops.TiledKV.zeros(B, Hkv, 32, DEV)
    torch.library.opcheck(L.qkv_epilogue, (qq, kk, vv, cs, cs, Hq, Hkv, None, None, 1e-6, None, 0, q_out, ring2.k,
                                           ring2.v, None, 0, None, None, None))
    s = torch.full((Hkv,), 0.75, device=DEV)
    torch.library.opcheck(L.decode_attention, (q, older.k, older.v, None, T0, None, None, None, None, None, 0, None, 0,
                                               None, 0, 0.0, 0, s))
    torch.library.opcheck(L.qkv_epilogue, (qq, kk, vv, cs, cs, Hq, Hkv, None, None, 1e-6, None, 0, q_out, ring2.k,
                                           ring2.v, None, 0, None, None, None, 1, 1.0 / s))


def test_compiled_decode_fragment_equals_eager():
    g = torch.Generator(device=DEV).manual_seed(14)
    B, Hq, Hkv, T0 = 4, 32, 8, 200
    older = ops.TiledKV.zeros(B, Hkv, 224, DEV)
    ops.pack_kv(_r(g, (B, Hkv, T0, 128)), _r(g, (B, Hkv, T0, 128)), older)
    wn = (torch.rand(Hq * 128, generator=g, device=DEV) + 0.5).bfloat16()

    def fragment(h, wq):
        q = (h @ wq).view(B, Hq, 128)
        o = L.decode_attention(q, older.k, older.v, None, T0, None, None, None, None, None, 0, None, 0, None, 0, 0.0, 0)
        return L.rmsnorm(o.reshape(B, Hq * 128), wn, 1e-5) + h

    h = _r(g, (B, Hq * 128))
    wq = (_r(g, (Hq * 128, Hq * 128)) * 0.02).bfloat16()
    want = fragment(h, wq)
    compiled = torch.compile(fragment, backend="aot_eager", fullgraph=True)
    got = compiled(h, wq)
    torch.cuda.synchronize()
    assert torch.equal(got, want)

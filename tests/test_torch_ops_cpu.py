"""The torch custom operators of lastkv_amd.torch_ops, checked without a GPU: registration,
schemas (arguments, the caches each operator writes) and fake-tensor shape propagation, and a
trace of a caller through make_fx in fake mode (what torch.compile does before it runs anything)."""

from __future__ import annotations

import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import lastkv_amd.torch_ops  # noqa: F401  (registers torch.ops.lastkv.*)

OPS = ("decode_attention", "prefill_attention", "merge_states", "qkv_epilogue", "blend_chunk", "rmsnorm", "silu_mul")


def test_registered_with_schemas_that_name_the_written_caches():
    for name in OPS:
        assert hasattr(torch.ops.lastkv, name), name
    def written(name):
        schema = getattr(torch.ops.lastkv, name).default._schema
        return {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}

    assert written("qkv_epilogue") == {"q_out", "ring_k", "ring_v", "deep_k", "deep_v"}
    assert written("blend_chunk") == {"ring_k", "ring_v"}
    for name in ("decode_attention", "prefill_attention", "merge_states", "rmsnorm", "silu_mul"):
        assert written(name) == set(), f"{name} must be functional"


def test_fake_tensor_shapes():
    with FakeTensorMode():
        B, Hq, Hkv, L = 3, 32, 8, 5
        q = torch.empty((B, Hq, 128), dtype=torch.bfloat16)
        older = torch.empty((B, Hkv, 4, 4096), dtype=torch.bfloat16)
        out = torch.ops.lastkv.decode_attention(q, older, older, None, 100, None, None, None, None, None, 0, None, 0,
                                                None, 0, 0.0, 0)
        assert out.shape == (B, Hq, 128) and out.dtype == torch.bfloat16
        qp = torch.empty((B, L, Hq, 128), dtype=torch.bfloat16)
        ring = torch.empty((B, Hkv, 2, 4096), dtype=torch.bfloat16)
        out = torch.ops.lastkv.prefill_attention(qp, older, older, None, 100, None, None, ring, ring, None, 40, None, 0,
                                                 None, 0, True, 0.0)
        assert out.shape == (B, L, Hq, 128)
        o = torch.empty((7, Hq, 128), dtype=torch.bfloat16)
        lse = torch.empty((7, Hq), dtype=torch.float32)
        mo, ml = torch.ops.lastkv.merge_states(o, lse, o, lse, None)
        assert mo.shape == o.shape and ml.shape == lse.shape and ml.dtype == torch.float32
        x = torch.empty((9, 4096), dtype=torch.bfloat16)
        assert torch.ops.lastkv.rmsnorm(x, torch.empty(4096, dtype=torch.bfloat16), 1e-5).shape == x.shape
        assert torch.ops.lastkv.silu_mul(x, x).shape == x.shape


def test_a_caller_traces_into_one_graph_in_fake_mode():
    """A decode-step fragment (epilogue, attention, norm) traced with make_fx in fake mode: the
    custom operators appear as graph nodes and the cache writes as in-place operator calls."""

    Hq, Hkv, B = 32, 8, 2

    def step(q, k, v, cos, sin, w, ring_k, ring_v, older_k, older_v, q_out):
        torch.ops.lastkv.qkv_epilogue(q, k, v, cos, sin, Hq, Hkv, w, w, 1e-5, None, 7, q_out, ring_k, ring_v, None, 0,
                                      None, None, None)
        o = torch.ops.lastkv.decode_attention(q_out.view(B, Hq, 128), older_k, older_v, None, 64, None, None, ring_k,
                                              ring_v, None, 8, None, 0, None, 0, 0.0, 0)
        return torch.ops.lastkv.rmsnorm(o.reshape(B, Hq * 128), torch.ones(Hq * 128, dtype=torch.bfloat16), 1e-5)

    bf = dict(dtype=torch.bfloat16)
    args = (torch.zeros((B, 1, Hq * 128), **bf), torch.zeros((B, 1, Hkv * 128), **bf), torch.zeros((B, 1, Hkv * 128), **bf),
            torch.zeros((1, 1, 128), **bf), torch.zeros((1, 1, 128), **bf), torch.ones(128, **bf),
            torch.zeros((B, Hkv, 2, 4096), **bf), torch.zeros((B, Hkv, 2, 4096), **bf),
            torch.zeros((B, Hkv, 2, 4096), **bf), torch.zeros((B, Hkv, 2, 4096), **bf), torch.zeros((B, 1, Hq, 128), **bf))
    gm = make_fx(step, tracing_mode="fake")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    for name in ("qkv_epilogue", "decode_attention", "rmsnorm"):
        assert any(f"lastkv.{name}" in t for t in targets), (name, targets)

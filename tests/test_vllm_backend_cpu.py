"""The vLLM boundary adapter keeps the reference's pinned Impl signatures and fails closed (no GPU).

Signatures: vllm/src/lastkv/vllm/backends/rmarin_flashinfer/vllm_backend.py:60-85
(_EXPECTED_IMPL_INIT_PARAMETERS, _EXPECTED_IMPL_FORWARD_PARAMETERS); forward contract :648-655."""

from __future__ import annotations

import inspect
from types import SimpleNamespace

import pytest
import torch

from lastkv_amd import vllm_backend as VB

INIT = ("self", "num_heads", "head_size", "scale", "num_kv_heads", "alibi_slopes", "sliding_window",
        "kv_cache_dtype", "logits_soft_cap", "attn_type", "kv_sharing_target_layer_name", "sinks")
FORWARD = ("self", "layer", "query", "key", "value", "kv_cache", "attn_metadata", "output", "output_scale",
           "output_block_scale")


def _impl(**kw):
    args = dict(num_heads=32, head_size=128, scale=128 ** -0.5, num_kv_heads=8, alibi_slopes=None,
                sliding_window=None, kv_cache_dtype="auto")
    args.update(kw)
    return VB.LastKVAttentionImpl(**args)


def test_pinned_signatures():
    assert tuple(inspect.signature(VB.LastKVAttentionImpl.__init__).parameters) == INIT
    assert tuple(inspect.signature(VB.LastKVAttentionImpl.forward).parameters) == FORWARD
    assert tuple(inspect.signature(VB.merge_state).parameters) == ("v_a", "s_a", "v_b", "s_b")
    assert issubclass(VB.LastKVBackendContractError, RuntimeError)
    b = VB.LastKVAttentionBackend
    assert b.get_name() == "CUSTOM" and b.get_impl_cls() is VB.LastKVAttentionImpl
    assert b.forward_includes_kv_cache_update and not b.supports_non_causal() and not b.supports_sink()
    assert b.supported_dtypes == [torch.bfloat16]


@pytest.mark.parametrize("kw,message", [
    (dict(head_size=64), "head_size"), (dict(scale=0.1), "scale"), (dict(alibi_slopes=[1.0]), "ALiBi"),
    (dict(kv_cache_dtype="fp8"), "kv_cache_dtype"), (dict(logits_soft_cap=30.0), "soft-capping"),
    (dict(attn_type="encoder"), "decoder"), (dict(kv_sharing_target_layer_name="x"), "sharing"),
    (dict(sinks=torch.zeros(32)), "sinks"), (dict(num_kv_heads=5), "multiple")])
def test_init_rejects_what_the_path_cannot_honour(kw, message):
    with pytest.raises(VB.LastKVBackendContractError, match=message):
        _impl(**kw)


def test_forward_contract_before_any_kernel():
    impl = _impl()
    q = torch.ones(3, 32 * 128, dtype=torch.bfloat16)
    kv = torch.ones(3, 8 * 128, dtype=torch.bfloat16)
    out = torch.ones(3, 32, 128, dtype=torch.bfloat16)
    layer = SimpleNamespace(rmarin_layer_index=0)
    assert impl.forward(layer, q, kv, kv, None, None, out) is out and not out.any()  # no metadata: zeros
    meta = SimpleNamespace(num_actual_tokens=3)
    with pytest.raises(VB.LastKVBackendContractError, match="output quantization"):
        impl.forward(layer, q, kv, kv, None, meta, out, output_scale=torch.ones(1))
    with pytest.raises(VB.LastKVBackendContractError, match="output quantization"):
        impl.forward(layer, q, kv, kv, None, meta, out, output_block_scale=torch.ones(1))
    VB.set_current(None)
    with pytest.raises(VB.LastKVBackendContractError, match="no LastKV fast path"):
        impl.forward(layer, q, kv, kv, None, meta, out)
    fake = SimpleNamespace(tokens=3, pool=SimpleNamespace(num_layers=2))
    VB.set_current(fake)
    try:
        for bad in (None, True, 2, -1):
            with pytest.raises(VB.LastKVBackendContractError, match="rmarin_layer_index"):
                impl.forward(SimpleNamespace(rmarin_layer_index=bad), q, kv, kv, None, meta, out)
        for actual in (0, True, 4, None):
            with pytest.raises(VB.LastKVBackendContractError):
                impl.forward(layer, q, kv, kv, None, SimpleNamespace(num_actual_tokens=actual), out)
    finally:
        VB.set_current(None)

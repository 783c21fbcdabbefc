"""vLLM attention-backend boundary of the serving path, written against the reference's pinned API.

Mirrors vllm/src/lastkv/vllm/backends/rmarin_flashinfer/vllm_backend.py: the reference registers a
CUSTOM backend whose ``AttentionImpl`` (``RMarinFlashInferImpl``, :637-717) ignores vLLM's KV cache
(the composite source / ring caches belong to the model bridge), zero-fills the output when there
is no attention metadata (:650-651), rejects fused output quantization (:652-655), and hands the
layer to the decode fast path (``fast.run_layer``, :656-664), zero-filling output rows past the
step's real tokens (:714-716).  Every violation raises a contract error instead of falling back to
stock attention (runtime_contract.py:37-38, vllm_backend.py:19-21).

``LastKVAttentionImpl`` keeps the pinned ``__init__`` / ``forward`` parameter lists
(vllm_backend.py:60-85, ``_EXPECTED_IMPL_INIT_PARAMETERS`` / ``_EXPECTED_IMPL_FORWARD_PARAMETERS``)
and runs ``LastKVFastPath.run_layer`` (lastkv_amd/serving.py) of the fast path made current with
``set_current``.  vLLM is not a dependency of this module: a vLLM-ROCm install binds these classes
by class path through its CUSTOM backend registration (vllm_plugin.py:19-65 in the reference);
``merge_state`` is the FlashInfer-order LSE merge the reference passes to its executor
(flashinfer.cascade.merge_state).
"""

from __future__ import annotations

import math
import threading
from typing import Any

import torch

from . import ops

HEAD_SIZE = ops.HEAD_DIM
SUPPORTED_KV_CACHE_DTYPES = ("auto", "bfloat16")


class LastKVBackendContractError(RuntimeError):
    """Raised when a call could silently violate the LastKV recurrence (the reference's
    ``RMarinBackendContractError``, runtime_contract.py:37-38)."""


_state = threading.local()


def set_current(fast) -> None:
    """Make ``fast`` (a ``LastKVFastPath`` whose step the runner has ``prepare``d, or None) the
    fast path that attention layers of this thread run (the reference's ``fastpath.current()``)."""

    _state.fast = fast


def current():
    return getattr(_state, "fast", None)


class LastKVAttentionImpl:
    """vLLM ``AttentionImpl`` of the LastKV serving path (vllm_backend.py:637-717)."""

    can_return_lse_for_decode = False

    def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes, sliding_window, kv_cache_dtype,
                 logits_soft_cap=None, attn_type="decoder", kv_sharing_target_layer_name=None, sinks=None):
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        checks = [
            (head_size == HEAD_SIZE, f"head_size must be {HEAD_SIZE}, got {head_size}"),
            (num_heads > 0 and num_kv_heads > 0 and num_heads % num_kv_heads == 0,
             "num_heads must be a positive multiple of num_kv_heads"),
            (math.isclose(float(scale), HEAD_SIZE ** -0.5, rel_tol=1e-6),
             f"softmax scale must be 1/sqrt({HEAD_SIZE}), got {scale}"),
            (alibi_slopes is None, "ALiBi is not part of the LastKV attention"),
            (kv_cache_dtype in SUPPORTED_KV_CACHE_DTYPES, f"kv_cache_dtype must be one of {SUPPORTED_KV_CACHE_DTYPES}"),
            (not logits_soft_cap, "logits soft-capping is not part of the LastKV attention"),
            (str(getattr(attn_type, "value", attn_type)).lower() == "decoder", "LastKV attention is decoder attention"),
            (kv_sharing_target_layer_name is None, "vLLM KV sharing conflicts with the shared last-layer cache"),
            (sinks is None, "attention sinks are not part of the LastKV attention"),
        ]
        for ok, message in checks:
            if not ok:
                raise LastKVBackendContractError(message)
        self.num_heads = int(num_heads)
        self.head_size = int(head_size)
        self.scale = float(scale)
        self.num_kv_heads = int(num_kv_heads)
        # vLLM sizes its own (unused) cache from the model's placeholder KV spec; the LastKV caches
        # live in the fast path's page pool, so the window only describes that placeholder
        self.sliding_window = sliding_window
        self.kv_cache_dtype = kv_cache_dtype

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                output_block_scale=None):
        """Attention of one layer over the step the current fast path has prepared: ``query``
        ``[T, Hq * 128]`` (or ``[T, Hq, 128]``), ``key`` / ``value`` ``[T, Hkv * 128]``; writes
        ``output`` ``[T, Hq, 128]`` in place and returns it."""

        del kv_cache  # the LastKV caches belong to the fast path
        if attn_metadata is None:  # vLLM's profiling and dummy runs
            return output.fill_(0)
        if output_scale is not None or output_block_scale is not None:
            raise LastKVBackendContractError("LastKV attention disables fused output quantization")
        fast = current()
        if fast is None:
            raise LastKVBackendContractError("no LastKV fast path is current (set_current after prepare)")
        index = getattr(layer, "rmarin_layer_index", None)
        if isinstance(index, bool) or not isinstance(index, int) or not 0 <= index < fast.pool.num_layers:
            raise LastKVBackendContractError(f"layer.rmarin_layer_index is invalid: {index!r}")
        actual = getattr(attn_metadata, "num_actual_tokens", None)
        if isinstance(actual, bool) or not isinstance(actual, int) or actual < 1:
            raise LastKVBackendContractError("vLLM attention metadata num_actual_tokens is invalid")
        T = fast.tokens
        if not actual <= T <= min(query.shape[0], key.shape[0], value.shape[0], output.shape[0]):
            raise LastKVBackendContractError(
                f"the prepared step has {T} tokens; vLLM passes {actual} real of {query.shape[0]} rows")
        if query.dtype != torch.bfloat16 or output.dtype != torch.bfloat16:
            raise LastKVBackendContractError("LastKV attention runs in bfloat16")
        out = output.view(output.shape[0], self.num_heads, self.head_size)
        fast.run_layer(index, query.reshape(query.shape[0], -1), key, value, out)
        if out.shape[0] > actual:
            out[actual:].fill_(0)
        return output


class LastKVAttentionBackend:
    """The CUSTOM backend class (vllm_backend.py:719-750): bf16, causal, KV writes inside forward."""

    supported_dtypes = [torch.bfloat16]
    supported_kv_cache_dtypes = list(SUPPORTED_KV_CACHE_DTYPES)
    forward_includes_kv_cache_update = True

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls() -> type[Any]:
        return LastKVAttentionImpl

    @classmethod
    def supports_non_causal(cls) -> bool:
        return False

    @classmethod
    def supports_sink(cls) -> bool:
        return False


def merge_state(v_a, s_a, v_b, s_b):
    """FlashInfer ``cascade.merge_state`` order (the merger the reference's executor takes)."""

    return ops.merge_state(v_a, s_a, v_b, s_b)

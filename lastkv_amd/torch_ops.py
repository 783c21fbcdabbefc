"""The kernels as PyTorch custom operators (namespace ``lastkv``), with fake implementations.

``lastkv_amd.ops`` binds the C ABI through ctypes, which torch.compile and fake-tensor tracing
(vLLM-ROCm's compiled model path) cannot see into.  Importing this module registers the same
calls as ``torch.ops.lastkv.*`` operators whose schemas name their arguments, their outputs and
the caches they write, plus a meta ("fake") implementation of each that only computes output
shapes, so callers that use them can be traced and captured whole.  At run time each operator
calls the ``lastkv_amd.ops`` function of the same name (same kernels, same validation).

Caches enter as their tensors: a tiled cache ``[slots, H, blocks, 4096]`` (``ops.TiledKV``) or,
with a block table, a head-major page pool ``[H, pages, 4096]`` (``ops.PagedKV``).  Lengths and
ring starts are an optional per-sequence int32 tensor or, when it is None, the matching
``*_const`` integer.  Zero-valued ``num_splits`` / ``local_ring_blocks`` / ``sm_scale`` mean the
library default.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import ops

__all__ = ["decode_attention", "prefill_attention", "merge_states", "qkv_epilogue", "blend_chunk", "rmsnorm",
           "silu_mul"]


def _seg(k: Optional[Tensor], v: Optional[Tensor], table: Optional[Tensor]):
    if k is None:
        return None
    return ops.PagedKV(k, v) if table is not None else ops.TiledKV(k, v)


def _len(t: Optional[Tensor], const: int):
    return t if t is not None else const


@torch.library.custom_op("lastkv::decode_attention", mutates_args=())
def decode_attention(q: Tensor, older_k: Optional[Tensor], older_v: Optional[Tensor], older_len: Optional[Tensor],
                     older_len_const: int, older_table: Optional[Tensor], vscale: Optional[Tensor],
                     local_k: Optional[Tensor], local_v: Optional[Tensor], local_len: Optional[Tensor],
                     local_len_const: int, local_start: Optional[Tensor], local_start_const: int,
                     local_table: Optional[Tensor], local_ring_blocks: int, sm_scale: float, num_splits: int,
                     out_scale: Optional[Tensor] = None) -> Tensor:
    """``lkv_decode_attn``: q ``[B, Hq, 128]`` -> out ``[B, Hq, 128]`` over [older | local]
    (``out_scale`` [Hkv]: out = bf16(bf16(o) * s), the vLLM path's output rescale)."""

    return ops.decode_attention(
        q, older=_seg(older_k, older_v, older_table), older_len=_len(older_len, older_len_const), vscale=vscale,
        local=_seg(local_k, local_v, local_table), local_len=_len(local_len, local_len_const),
        local_start=_len(local_start, local_start_const), older_table=older_table, local_table=local_table,
        local_ring_blocks=local_ring_blocks or None, sm_scale=sm_scale or None, num_splits=num_splits or None,
        out_scale=out_scale)


@decode_attention.register_fake
def _(q, older_k, older_v, older_len, older_len_const, older_table, vscale, local_k, local_v, local_len,
      local_len_const, local_start, local_start_const, local_table, local_ring_blocks, sm_scale, num_splits,
      out_scale=None):
    return q.new_empty((q.shape[0], q.shape[1], ops.HEAD_DIM))


@torch.library.custom_op("lastkv::prefill_attention", mutates_args=())
def prefill_attention(q: Tensor, older_k: Optional[Tensor], older_v: Optional[Tensor], older_len: Optional[Tensor],
                      older_len_const: int, older_table: Optional[Tensor], vscale: Optional[Tensor],
                      local_k: Optional[Tensor], local_v: Optional[Tensor], local_len: Optional[Tensor],
                      local_len_const: int, local_start: Optional[Tensor], local_start_const: int,
                      local_table: Optional[Tensor], local_ring_blocks: int, causal: bool, sm_scale: float,
                      out_scale: Optional[Tensor] = None, cu_seqlens_q: Optional[Tensor] = None,
                      max_seqlen_q: int = 0, num_splits: int = 0, cu_seqlens_q_host: Optional[Tensor] = None) -> Tensor:
    """``lkv_prefill_attn``: q ``[B, L, Hq, 128]`` (the last L tokens of the local segment) ->
    out ``[B, L, Hq, 128]``; bottom-right causal over the local segment when ``causal``.  With
    ``cu_seqlens_q`` (int32 ``[B + 1]``) and ``max_seqlen_q`` q / out are ragged ``[T, Hq, 128]``
    (FlashAttention's varlen form), and ``cu_seqlens_q_host`` (the same offsets as an int32 CPU
    tensor, optional) lets the call plan its launches on the host; ``num_splits`` 0 lets the library
    choose the key splits."""

    return ops.prefill_attention(
        q, older=_seg(older_k, older_v, older_table), older_len=_len(older_len, older_len_const), vscale=vscale,
        local=_seg(local_k, local_v, local_table), local_len=_len(local_len, local_len_const),
        local_start=_len(local_start, local_start_const), older_table=older_table, local_table=local_table,
        local_ring_blocks=local_ring_blocks or None, causal=causal, sm_scale=sm_scale or None, out_scale=out_scale,
        cu_seqlens_q=cu_seqlens_q, max_seqlen_q=max_seqlen_q if cu_seqlens_q is not None else None,
        num_splits=num_splits, cu_seqlens_q_host=None if cu_seqlens_q_host is None else cu_seqlens_q_host.numpy())


@prefill_attention.register_fake
def _(q, older_k, older_v, older_len, older_len_const, older_table, vscale, local_k, local_v, local_len,
      local_len_const, local_start, local_start_const, local_table, local_ring_blocks, causal, sm_scale,
      out_scale=None, cu_seqlens_q=None, max_seqlen_q=0, num_splits=0, cu_seqlens_q_host=None):
    return q.new_empty(q.shape)


@torch.library.custom_op("lastkv::merge_states", mutates_args=())
def merge_states(prefix_out: Tensor, prefix_lse: Tensor, suffix_out: Tensor, suffix_lse: Tensor,
                 prefix_scale: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """``lkv_merge_states``: outputs bf16 ``[T, H, D]``, LSEs fp32 ``[T, H]`` -> (out, out_lse)."""

    out_lse = torch.empty(prefix_lse.shape, dtype=torch.float32, device=prefix_lse.device)
    out, _ = ops.merge_states(prefix_out, prefix_lse, suffix_out, suffix_lse, prefix_scale=prefix_scale,
                              out_lse=out_lse)
    return out, out_lse


@merge_states.register_fake
def _(prefix_out, prefix_lse, suffix_out, suffix_lse, prefix_scale):
    return suffix_out.new_empty(suffix_out.shape), prefix_lse.new_empty(prefix_lse.shape)


@torch.library.custom_op("lastkv::qkv_epilogue", mutates_args=("q_out", "ring_k", "ring_v", "deep_k", "deep_v"))
def qkv_epilogue(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor, num_q_heads: int, num_kv_heads: int,
                 q_norm_weight: Optional[Tensor], k_norm_weight: Optional[Tensor], eps: float,
                 positions: Optional[Tensor], positions_const: int, q_out: Tensor, ring_k: Tensor, ring_v: Tensor,
                 ring_table: Optional[Tensor], ring_tokens: int, deep_k: Optional[Tensor], deep_v: Optional[Tensor],
                 deep_table: Optional[Tensor], rounding: int = 0, ring_v_mul: Optional[Tensor] = None,
                 cu_seqlens: Optional[Tensor] = None, max_seqlen: int = 0) -> None:
    """``lkv_qkv_epilogue``: RoPE + q/k RMSNorm, q written to ``q_out`` ``[B, L, Hq, 128]``, K/V
    appended to the ring (and to the shared cache ``deep_*`` when given) at ``positions + i``;
    ``rounding`` 0 = the HF torch op order, 1 = the vLLM fused_qkv order; ``ring_v_mul`` [Hkv]
    scales the ring's V (the vLLM path's V / s rings).  With ``cu_seqlens`` (int32 ``[B + 1]``) and
    ``max_seqlen`` the rows are ragged: q / k / v ``[T, heads * 128]``, q_out ``[T, Hq, 128]``."""

    ops.qkv_epilogue(q, k, v, cos, sin, num_q_heads=num_q_heads, num_kv_heads=num_kv_heads,
                     q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight, eps=eps,
                     positions=_len(positions, positions_const), ring=_seg(ring_k, ring_v, ring_table),
                     deep=_seg(deep_k, deep_v, deep_table), q_out=q_out, ring_table=ring_table,
                     ring_tokens=ring_tokens or None, deep_table=deep_table,
                     rounding={v: k for k, v in ops.ROUNDINGS.items()}[rounding], ring_v_mul=ring_v_mul,
                     cu_seqlens=cu_seqlens, max_seqlen=max_seqlen if cu_seqlens is not None else None)


@qkv_epilogue.register_fake
def _(q, k, v, cos, sin, num_q_heads, num_kv_heads, q_norm_weight, k_norm_weight, eps, positions, positions_const,
      q_out, ring_k, ring_v, ring_table, ring_tokens, deep_k, deep_v, deep_table, rounding=0, ring_v_mul=None,
      cu_seqlens=None, max_seqlen=0):
    return None


@torch.library.custom_op("lastkv::blend_chunk", mutates_args=("ring_k", "ring_v"))
def blend_chunk(ring_k: Tensor, ring_v: Tensor, deep_k: Tensor, deep_v: Tensor, batch: int, chunk_start: int,
                chunk_len: int, alpha: Tensor, one_minus_alpha: Tensor, vscale: Optional[Tensor],
                ring_table: Optional[Tensor], ring_tokens: int, deep_table: Optional[Tensor]) -> None:
    """``lkv_blend_chunk``: the boundary commit, every layer's ring chunk blended in place."""

    ops.blend_chunk(ring_k, ring_v, _seg(deep_k, deep_v, deep_table), batch=batch, chunk_start=chunk_start,
                    chunk_len=chunk_len, alpha=alpha, one_minus_alpha=one_minus_alpha, vscale=vscale,
                    ring_table=ring_table, ring_tokens=ring_tokens or None, deep_table=deep_table)


@blend_chunk.register_fake
def _(ring_k, ring_v, deep_k, deep_v, batch, chunk_start, chunk_len, alpha, one_minus_alpha, vscale, ring_table,
      ring_tokens, deep_table):
    return None


@torch.library.custom_op("lastkv::rmsnorm", mutates_args=())
def rmsnorm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """``lkv_rmsnorm`` without a residual: LlamaRMSNorm of the rows of bf16 ``x``."""

    return ops.rmsnorm(x, weight, eps)


@rmsnorm.register_fake
def _(x, weight, eps):
    return x.new_empty(x.shape)


@torch.library.custom_op("lastkv::silu_mul", mutates_args=())
def silu_mul(gate: Tensor, up: Tensor) -> Tensor:
    """``lkv_silu_mul``: ``F.silu(gate) * up`` in bf16."""

    return ops.silu_mul(gate, up)


@silu_mul.register_fake
def _(gate, up):
    return gate.new_empty(gate.shape)

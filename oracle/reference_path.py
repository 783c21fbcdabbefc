"""The reference's attention composition + SDPA, restated with torch ops (test infrastructure only).

``lastkv_attention`` performs the steps of LastKVAttention.forward after the projections
(llm/src/lastkv/llm/modeling.py:109-146): concatenate the older (shared, V scaled), recent
(blended) and current regions with torch.cat, build the bottom-right causal mask for a partial
chunk, and call ``F.scaled_dot_product_attention`` with GQA.  It runs on any device and dtype:
  - on the CPU it is the timed CPU baseline of bench.py ("the reference CPU path");
  - on the GPU in bf16 it is "the reference PyTorch SDPA path";
  - with ``compute_dtype=torch.float32`` the composed bf16 K/V are attended in fp32 and the
    output rounded once to the input dtype, which isolates kernel error from torch-SDPA's own
    bf16 rounding.
Pinned by: tests/test_oracle_cpu.py checks it against the numpy fp64 oracle
(oracle.attention.compose_history_bf16 + attention) and, for chunk >= sequence length, against
plain GQA SDPA (LastKV then degenerates to a standard Llama attention).
"""

from __future__ import annotations

import torch
from torch.nn import functional as F


def compose(deep, previous, current, alpha_logits, vscale, chunk):
    """torch.cat composition of modeling.py:109-122; returns (full_k, full_v)."""

    cur_k, cur_v = current
    keys, values = [], []
    if deep is not None:
        deep_k, deep_v = deep
        older = deep_k.shape[2] - chunk
        s = vscale.to(deep_v.dtype).view(1, -1, 1, 1)
        if older:
            keys.append(deep_k[:, :, :older])
            values.append(deep_v[:, :, :older] * s)
        prev_k, prev_v = previous
        a = alpha_logits.sigmoid().to(cur_k.dtype).view(1, -1, 1, 1)
        keys.append(a * deep_k[:, :, older:] + (1 - a) * prev_k)
        values.append(a * (deep_v[:, :, older:] * s) + (1 - a) * prev_v)
    keys.append(cur_k)
    values.append(cur_v)
    return torch.cat(keys, dim=2), torch.cat(values, dim=2)


def sdpa_bottom_right(query, full_k, full_v, *, compute_dtype=None, scale=None, native_gqa=False):
    """SDPA with the reference's mask rule (modeling.py:124-130, :143-146).

    ``native_gqa`` passes ``enable_gqa=True`` as the reference does; otherwise K/V are expanded to
    the query heads first (every SDPA backend accepts that form).
    """

    length, key_length = query.shape[2], full_k.shape[2]
    causal = length == key_length
    mask = None
    if not causal and length > 1:
        qpos = torch.arange(length, device=query.device) + key_length - length
        mask = torch.arange(key_length, device=query.device)[None, :] <= qpos[:, None]
    out_dtype = query.dtype
    if compute_dtype is not None:
        query, full_k, full_v = query.to(compute_dtype), full_k.to(compute_dtype), full_v.to(compute_dtype)
    gqa = query.shape[1] != full_k.shape[1]
    if gqa and native_gqa:
        out = F.scaled_dot_product_attention(query, full_k, full_v, attn_mask=mask, is_causal=causal and length > 1,
                                             dropout_p=0.0, scale=scale, enable_gqa=True)
        return out.to(out_dtype)
    if gqa:
        # expand explicitly (contiguous) rather than rely on enable_gqa support of every backend
        group = query.shape[1] // full_k.shape[1]
        full_k = full_k.repeat_interleave(group, dim=1)
        full_v = full_v.repeat_interleave(group, dim=1)
    out = F.scaled_dot_product_attention(query, full_k, full_v, attn_mask=mask, is_causal=causal and length > 1,
                                         dropout_p=0.0, scale=scale)
    return out.to(out_dtype)


def lastkv_attention(query, deep, previous, current, alpha_logits, vscale, chunk, *, compute_dtype=None):
    """query [B, Hq, Lq, D] against one layer's composed history; returns [B, Hq, Lq, D]."""

    full_k, full_v = compose(deep, previous, current, alpha_logits, vscale, chunk)
    return sdpa_bottom_right(query, full_k, full_v, compute_dtype=compute_dtype)

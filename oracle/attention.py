"""fp64 attention and LastKV history composition (test infrastructure only; see oracle/__init__.py).

Restates, in numpy:
  - the region plan of one query position: older [0, rec), recent [rec, cur), current [cur, p]
    (vllm/src/lastkv/vllm/backends/rmarin_flashinfer/access_plan.py:237-253, :418-420);
  - the history composition of LastKVAttention.forward (llm/src/lastkv/llm/modeling.py:109-122)
    with the reference's bf16 rounding points (:96, :117-119);
  - softmax attention with GQA and the bottom-right causal mask (modeling.py:124-146,
    eager form :131-141), returning the natural-log LSE as FlashInfer / FA3 do;
  - the exact merge of two disjoint attention states
    (flashinfer_executor.py:185-231, `merge_state`; fastpath.py:717-720 masks a missing
    source with LSE -inf).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import bf16


@dataclass(frozen=True)
class Regions:
    """Half-open token ranges of the three history regions of query position ``p``."""

    older: tuple[int, int]
    recent: tuple[int, int]
    current: tuple[int, int]


def plan_regions(position: int, chunk: int) -> Regions:
    """access_plan.py:237-253: cur = floor(p / C) * C, rec = max(0, cur - C).

    Pinned by: tests/test_oracle_cpu.py enumerates every p < 5C for small C and checks the
    cache-shape invariants of the reference test (test_llm_inference.py:118-121) and that the
    local window never exceeds 2C (access_plan.py:272-273).
    """

    if position < 0 or chunk < 1:
        raise ValueError("position must be >= 0 and chunk >= 1")
    cur = (position // chunk) * chunk
    rec = max(0, cur - chunk)
    return Regions((0, rec), (rec, cur), (cur, position + 1))


def sigmoid(x):
    """Numerically stable logistic function (reference.py:134-141)."""

    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-x[pos]))
    e = np.exp(x[~pos])
    out[~pos] = e / (1.0 + e)
    return out


def compose_history_bf16(
    deep_k: np.ndarray,
    deep_v: np.ndarray,
    prev_k: np.ndarray | None,
    prev_v: np.ndarray | None,
    cur_k: np.ndarray,
    cur_v: np.ndarray,
    alpha_logits: np.ndarray,
    vscale: np.ndarray,
    chunk: int,
) -> tuple[np.ndarray, np.ndarray]:
    """Full K/V of one layer as the bf16 reference materialises them (modeling.py:109-122).

    deep_k/deep_v: final-layer K (post RoPE + k_norm) and raw V of the completed chunks,
    [B, Hkv, n_chunks * C, D] (n_chunks may be 0).  prev_k/prev_v: this layer's own K/V of the
    last completed chunk [B, Hkv, C, D] (None when no chunk is complete).  cur_k/cur_v: this
    layer's current-chunk K/V [B, Hkv, Lc, D].  alpha_logits, vscale: [Hkv] (bf16-valued when
    the model is bf16: parameters are cast with the model).  All inputs are bf16-representable
    float32 arrays; the result is bf16-representable float32.

    older  : K = deep_k,             V = bf16(deep_v * s)                      (:112-115, :96)
    recent : K = bf16(bf16(a*Kd) + bf16(bf16(1-a)*Kp))
             V = bf16(bf16(a*bf16(Vd*s)) + bf16(bf16(1-a)*Vp))                  (:117-119)
    current: own K/V                                                          (:120-121)
    with a = bf16(sigmoid(logit)) (:117).

    Pinned by: tests/test_oracle_cpu.py (a) compares against the same expression evaluated by
    torch in bf16, op for op; (b) checks alpha-logit -> +inf gives the shared chunk and -> -inf
    the layer's own chunk; (c) checks s = 1 leaves older V unscaled.
    """

    keys, values = [], []
    if deep_k.shape[2]:
        old_length = deep_k.shape[2] - chunk
        s = np.asarray(vscale, np.float32).reshape(1, -1, 1, 1)
        if old_length:
            keys.append(deep_k[:, :, :old_length])
            values.append(bf16.mul(deep_v[:, :, :old_length], s))
        alpha = bf16.round_bf16(sigmoid(alpha_logits).astype(np.float32)).reshape(1, -1, 1, 1)
        one_minus = bf16.rsub(alpha, 1.0)
        keys.append(bf16.add(bf16.mul(alpha, deep_k[:, :, old_length:]), bf16.mul(one_minus, prev_k)))
        scaled = bf16.mul(deep_v[:, :, old_length:], s)
        values.append(bf16.add(bf16.mul(alpha, scaled), bf16.mul(one_minus, prev_v)))
    keys.append(cur_k)
    values.append(cur_v)
    return np.concatenate(keys, axis=2), np.concatenate(values, axis=2)


def blend_chunk_bf16(shared: np.ndarray, own: np.ndarray, alpha_logits: np.ndarray, vscale=None) -> np.ndarray:
    """The recent-chunk blend of one of K or V, in the reference's bf16 op order (modeling.py:117-119).

    shared: final-layer chunk [.., Hkv, C, D]; own: this layer's chunk; vscale given -> the V form
    (shared side multiplied by s first).  Pinned as ``compose_history_bf16``.
    """

    alpha = bf16.round_bf16(sigmoid(alpha_logits).astype(np.float32)).reshape(1, -1, 1, 1)
    one_minus = bf16.rsub(alpha, 1.0)
    src = shared if vscale is None else bf16.mul(shared, np.asarray(vscale, np.float32).reshape(1, -1, 1, 1))
    return bf16.add(bf16.mul(alpha, src), bf16.mul(one_minus, own))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
              causal_bottom_right: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """fp64 softmax attention with GQA.  q [B, Hq, Lq, D], k/v [B, Hkv, S, D].

    Returns (out [B, Hq, Lq, D], lse [B, Hq, Lq]) with lse = log(sum exp(scores)) in natural log
    (-inf where a row has no visible key, whose output is 0).  ``causal_bottom_right`` applies
    modeling.py:124-130: query i of Lq sees keys j <= i + S - Lq.

    Pinned by: tests/test_oracle_cpu.py compares with torch's F.scaled_dot_product_attention in
    float64 (a library routine) and with a pure-Python loop on tiny shapes, including masked rows.
    """

    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, Lq, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    group = Hq // Hkv
    if group * Hkv != Hq:
        raise ValueError("Hq must be a multiple of Hkv")
    scale = D ** -0.5 if scale is None else scale
    kk = np.repeat(k, group, axis=1)
    vv = np.repeat(v, group, axis=1)
    scores = np.einsum("bhqd,bhkd->bhqk", q, kk) * scale
    if causal_bottom_right:
        qpos = np.arange(Lq)[:, None] + S - Lq
        visible = np.arange(S)[None, :] <= qpos
        scores = np.where(visible[None, None], scores, -np.inf)
    m = scores.max(axis=-1, keepdims=True)
    safe_m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(scores - safe_m)
    l = p.sum(axis=-1, keepdims=True)
    out = np.einsum("bhqk,bhkd->bhqd", p, vv) / np.where(l > 0, l, 1.0)
    lse = np.where(l[..., 0] > 0, np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)) + safe_m[..., 0], -np.inf)
    return out, lse


def merge_states(out_a, lse_a, out_b, lse_b) -> tuple[np.ndarray, np.ndarray]:
    """Exact merge of attention states over disjoint key sets (flashinfer_executor.py:185-231).

    out_*: [..., D]; lse_*: [...] natural log, -inf for an empty set.
    Pinned by: tests/test_oracle_cpu.py checks merge(attn(K1), attn(K2)) == attn(K1 u K2).
    """

    out_a, out_b = np.asarray(out_a, np.float64), np.asarray(out_b, np.float64)
    lse_a, lse_b = np.asarray(lse_a, np.float64), np.asarray(lse_b, np.float64)
    m = np.maximum(lse_a, lse_b)
    safe = np.where(np.isfinite(m), m, 0.0)
    wa = np.where(np.isfinite(lse_a), np.exp(lse_a - safe), 0.0)
    wb = np.where(np.isfinite(lse_b), np.exp(lse_b - safe), 0.0)
    tot = wa + wb
    denom = np.where(tot > 0, tot, 1.0)
    out = (out_a * wa[..., None] + out_b * wb[..., None]) / denom[..., None]
    lse = np.where(tot > 0, safe + np.log(denom), -np.inf)
    return out, lse


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    n = np.linalg.norm(e.ravel())
    return float(np.linalg.norm((a - e).ravel()) / (n if n > 0 else 1.0))


def max_abs(actual, expected) -> float:
    return float(np.max(np.abs(np.asarray(actual, np.float64) - np.asarray(expected, np.float64)))) if np.size(expected) else 0.0


def decode_history_bytes(batch: int, kv_heads: int, tokens: int, q_heads: int, head_dim: int = 128, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one decode layer-call: K+V of every key plus Q and O."""

    return 2 * batch * kv_heads * tokens * head_dim * elem + 2 * batch * q_heads * head_dim * elem


__all__ = [
    "Regions", "plan_regions", "sigmoid", "compose_history_bf16", "blend_chunk_bf16", "attention",
    "merge_states", "rel_l2", "max_abs", "decode_history_bytes",
]

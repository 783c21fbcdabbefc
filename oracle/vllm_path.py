"""The reference's vLLM serving-path rounding contract (test infrastructure only; see oracle/__init__.py).

The reference serves LastKV through a merged fast path whose numbers differ from the HF model's
(vllm/src/lastkv/vllm/backends/rmarin_flashinfer/):
  - fused_qkv.py:24-55 (_rope_rms): neox rotary as r1 = bf16(fma(x, c, -(y * s))),
    r2 = bf16(fma(y, c, x * s)) over the halves x = dims [0, 64), y = dims [64, 128); RMSNorm with
    a fixed summation order (16 groups of 8 consecutive dims, each group's squares accumulated in
    order with fused multiply-adds, adjacent groups then added pairwise 16 -> 8 -> 4 -> 2 -> 1),
    inv = rsqrt(var / 128 + eps), out = bf16(full * inv * w) in fp32;
  - fused_qkv.py:59-91 (_fused_qkv_kernel): the layer ring receives K and bf16(v * fp32(1 / s));
    the top layer also writes its K and raw V into the shared slab;
  - fastpath.py:644-651 (merged path): one causal attention over [slab pages | ring pages], then
    _head_scale: out = bf16(out_bf16 * s) (fused_qkv.py:130-156; fastpath.py:690, "s_l is
    bf16-exact");
  - batching.py:1124-1140 + fused_qkv.py:158-207 (commit with ring_v_scaled): the recent chunk of
    every ring := bf16(bf16(a * raw) + bf16(bf16(1 - a) * ring)), raw V unscaled (rings hold V / s).

Everything is float32 arithmetic in numpy with the reference's rounding points; fused
multiply-adds are emulated exactly (``fma_f32``).  The one deliberate difference: inv is computed
as fp32 1 / sqrt (correctly rounded square root and division), where the reference's Triton
``tl.math.rsqrt`` is a hardware approximation whose last bits are not specified; the GPU kernels
compute the same correctly rounded value.

Pinned by (tests/test_oracle_vllm_cpu.py): ``fma_f32`` against exact rational arithmetic rounded to
fp32 (random operands, constructed exact ties and cancellations); ``rope_rms`` by its special cases
(identity rotation, quarter turns) and by known answers of the summation order on inputs where the
documented order, and no nearby alternative order, yields a hand-derived sum; the per-layer merged
path by the algebraic identity s * attn(.., [V_old | V_ring / s]) = attn(.., [s V_old | V_ring])
(up to the rounding of V / s and the two output roundings) against ``attention.attention``.
"""

from __future__ import annotations

import numpy as np

from . import bf16
from .attention import attention, blend_chunk_bf16

HEAD_DIM = 128
HALF = HEAD_DIM // 2


def fma_f32(a, b, c) -> np.ndarray:
    """Exact fp32 fused multiply-add round(a * b + c) (round to nearest even) of float32 arrays.

    a * b is exact in float64; the float64 sum s and its TwoSum error e give the exact a * b + c =
    s + e.  Rounding s to fp32 is then correct except when s lies exactly halfway between two fp32
    values and e != 0 (double rounding), where the sign of e picks the neighbour.
    """

    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    c = np.asarray(c, np.float32)
    a, b, c = np.broadcast_arrays(a, b, c)
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)  # nearest-even fp32 of s
    r64 = r.astype(np.float64)
    toward = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
    n = np.nextafter(r, toward)  # the other fp32 neighbour of s
    tie = (s != r64) & np.isfinite(s) & (2.0 * s == r64 + n.astype(np.float64)) & (e != 0)
    # at a tie s is midway between r and n: the exact value lies on n's side when e points there
    pick_n = tie & (np.sign(e) == np.sign(n.astype(np.float64) - r64))
    return np.where(pick_n, n, r).astype(np.float32)


def rms_sum(full) -> np.ndarray:
    """The sum of squares of rows [..., 128] in fused_qkv.py:43-51's order: 16 groups of 8
    consecutive dims, each accumulated in order with fused multiply-adds from 0, then adjacent
    groups added pairwise (16 -> 8 -> 4 -> 2) and the two halves last."""

    full = np.asarray(full, np.float32)
    grp = full.reshape(full.shape[:-1] + (16, 8))
    acc = np.zeros(full.shape[:-1] + (16,), np.float32)
    for jj in range(8):
        acc = fma_f32(grp[..., jj], grp[..., jj], acc)
    t8 = (acc[..., 0::2] + acc[..., 1::2]).astype(np.float32)
    t4 = (t8[..., 0::2] + t8[..., 1::2]).astype(np.float32)
    t2 = (t4[..., 0::2] + t4[..., 1::2]).astype(np.float32)
    return (t2[..., 0] + t2[..., 1]).astype(np.float32)


def rope_rms(x, cos, sin, w=None, eps: float = 1e-6) -> np.ndarray:
    """fused_qkv.py:24-55 on rows x [..., 128] (bf16-valued float32) with cos / sin [..., 64]
    (the cos / sin of dims [0, 64) at the row's position) and norm weight w [128] or None.
    Returns bf16-valued float32 [..., 128]."""

    x = np.asarray(x, np.float32)
    c = np.asarray(cos, np.float32)
    s = np.asarray(sin, np.float32)
    x1, x2 = x[..., :HALF], x[..., HALF:]
    r1 = bf16.round_bf16(fma_f32(x1, c, -(x2 * s)))
    r2 = bf16.round_bf16(fma_f32(x2, c, x1 * s))
    full = np.concatenate([r1, r2], axis=-1).astype(np.float32)
    if w is None:
        return full
    var = rms_sum(full)
    inv = (np.float32(1.0) / np.sqrt((var / np.float32(HEAD_DIM) + np.float32(eps)).astype(np.float32))).astype(np.float32)
    wf = np.asarray(w, np.float32)
    return bf16.round_bf16((full * inv[..., None]).astype(np.float32) * wf)


def ring_value(v, inv_scale) -> np.ndarray:
    """fused_qkv.py:84-86: bf16(v * inv) with inv = fp32(1 / s) per kv head (v [..., Hkv, D])."""

    inv = np.asarray(inv_scale, np.float32)[:, None]
    return bf16.round_bf16(np.asarray(v, np.float32) * inv)


def inv_scale(s) -> np.ndarray:
    """fastpath.py:266: fp32 1 / s."""

    return (np.float32(1.0) / np.asarray(s, np.float32)).astype(np.float32)


def head_scale(out_bf16, s) -> np.ndarray:
    """fused_qkv.py:130-156: bf16(out * s), s per head of out [..., H, D]."""

    return bf16.round_bf16(np.asarray(out_bf16, np.float32) * np.asarray(s, np.float32)[:, None])


class MergedSequence:
    """One sequence through the reference's merged serving path, layer by layer (fastpath.py:619-651,
    batching.py:1099-1140): per-layer rings of (K, V / s) by position, the shared slab of the top
    layer's (K, raw V), the boundary commit at the first step after a chunk boundary.

    ``layer_params[l]`` = (q_norm_w [128] or None, k_norm_w or None, eps, s [Hkv] bf16-valued);
    ``alpha`` [L, Hkv] bf16-valued gates of the commit; ``rotary(positions) -> (cos, sin)`` [n, 64].
    """

    def __init__(self, layers: int, kv_heads: int, chunk: int, layer_params, alpha, rotary):
        self.layers, self.kv_heads, self.chunk = layers, kv_heads, chunk
        self.params = list(layer_params)
        self.alpha = np.asarray(alpha, np.float32).reshape(layers, kv_heads)
        self.rotary = rotary
        self.seen = 0
        self.committed = 0
        self.slab_k: dict[int, np.ndarray] = {}
        self.slab_v: dict[int, np.ndarray] = {}
        self.ring_k = [dict() for _ in range(layers)]
        self.ring_v = [dict() for _ in range(layers)]

    def begin_step(self) -> None:
        """The host prologue: commit the completed chunk if this step starts on a boundary."""

        C, p = self.chunk, self.seen
        if p > 0 and p % C == 0 and self.committed < p:
            one_minus = bf16.rsub(self.alpha, 1.0)
            for l in range(self.layers):
                a = self.alpha[l][:, None]
                om = one_minus[l][:, None]
                for t in range(p - C, p):
                    for ring, slab in ((self.ring_k[l], self.slab_k), (self.ring_v[l], self.slab_v)):
                        ring[t] = bf16.add(bf16.mul(a, slab[t]), bf16.mul(om, ring[t]))
            self.committed = p

    def layer(self, l: int, q, k, v, num_q_heads: int) -> np.ndarray:
        """This step's rows q [n, Hq, 128], k / v [n, Hkv, 128] (bf16-valued) through layer l; returns
        the bf16-valued output [n, Hq, 128] before the o projection (``last_attention`` keeps the
        attention's bf16 output before the head scale).  Attention in float64."""

        qn_w, kn_w, eps, s = self.params[l]
        n = q.shape[0]
        p0, C, Hkv = self.seen, self.chunk, self.kv_heads
        cos, sin = self.rotary(np.arange(p0, p0 + n))
        qn = rope_rms(q, cos[:, None], sin[:, None], qn_w, eps)
        kn = rope_rms(k, cos[:, None], sin[:, None], kn_w, eps)
        vr = ring_value(v, inv_scale(s))
        for i in range(n):
            self.ring_k[l][p0 + i] = kn[i]
            self.ring_v[l][p0 + i] = vr[i]
            if l == self.layers - 1:
                self.slab_k[p0 + i] = kn[i]
                self.slab_v[p0 + i] = np.asarray(v[i], np.float32)
        last = p0 + n - 1
        rec = max(0, last // C * C - C)
        keys = [self.slab_k[t] for t in range(rec)] + [self.ring_k[l][t] for t in range(rec, last + 1)]
        vals = [self.slab_v[t] for t in range(rec)] + [self.ring_v[l][t] for t in range(rec, last + 1)]
        K = np.stack(keys, axis=1)[None]  # [1, Hkv, S, D]
        V = np.stack(vals, axis=1)[None]
        out, _ = attention(np.transpose(qn, (1, 0, 2))[None], K, V, causal_bottom_right=True)
        o16 = bf16.round_bf16(np.transpose(out[0], (1, 0, 2)).astype(np.float32))
        self.last_attention = o16  # the attention output before the head scale
        group = num_q_heads // Hkv
        return head_scale(o16, np.repeat(np.asarray(s, np.float32), group))

    def end_step(self, n: int) -> None:
        self.seen += n


def blend_ring(raw, ring, alpha_logits) -> np.ndarray:
    """The commit blend with rings of V / s (batching.py:1126-1128: raw source unscaled)."""

    return blend_chunk_bf16(raw, ring, alpha_logits, vscale=None)


__all__ = ["fma_f32", "rms_sum", "rope_rms", "ring_value", "inv_scale", "head_scale", "MergedSequence", "blend_ring"]

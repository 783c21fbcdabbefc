"""Pins of oracle/vllm_path.py, the reference's vLLM serving-path rounding contract (CPU only).

- ``fma_f32`` against exact rational arithmetic rounded to fp32 (random operands of mixed
  magnitudes and signs, cancellations, and constructed cases whose float64 sum lands exactly on an
  fp32 midpoint, where a float64-then-fp32 evaluation double-rounds the wrong way).
- ``rms_sum``: known answers on inputs where the documented order (16 in-order FMA groups, then a
  pairwise tree, fused_qkv.py:43-51) gives a hand-derived value that a single sequential chain, a
  small-values-first order or a strided grouping do not.
- ``rope_rms``: rotation special cases (identity, quarter turn), closeness to the fp64 rotation and
  RMSNorm, and the V / s ring and head-scale roundings.
- ``MergedSequence``: s * attn([V_old | V_ring / s]) against attn([s V_old | V_ring]) in fp64.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

from oracle import attention as A
from oracle import bf16
from oracle import vllm_path as VP


def _round_f32(x: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to fp32 (normal and subnormal range)."""

    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    e = max(e, -126)  # subnormals share the exponent of the smallest normal
    q = x / Fraction(2) ** (e - 23)  # in [2^23, 2^24) for normals
    m = q.numerator // q.denominator
    rem = q - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return np.float32(sign * float(Fraction(m) * Fraction(2) ** (e - 23)))


def _fma_exact(a, b, c) -> np.float32:
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_fma_matches_exact_arithmetic_on_random_operands():
    rng = np.random.default_rng(0)
    n = 3000
    a = (rng.standard_normal(n) * 2.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 2.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    c = (rng.standard_normal(n) * 2.0 ** rng.integers(-60, 60, n)).astype(np.float32)
    # cancellations: c close to -a*b
    c[: n // 3] = (-(a[: n // 3].astype(np.float64) * b[: n // 3])).astype(np.float32)
    got = VP.fma_f32(a, b, c)
    want = np.array([_fma_exact(x, y, z) for x, y, z in zip(a, b, c)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fma_resolves_float64_midpoints():
    # a * b = 2^-24 + 2^-60 exactly (the factors (1 + 2^-12) and (1 - 2^-12 + 2^-24) are fp32), so
    # 1 + a * b lies just above the midpoint 1 + 2^-24: float64 drops the 2^-60 and then rounds to
    # the even neighbour 1.0, the exact FMA rounds up to 1 + 2^-23
    a = np.float32(2.0 ** -24 * (1 + 2.0 ** -12))
    b = np.float32(1 - 2.0 ** -12 + 2.0 ** -24)
    assert float(a) * float(b) != 2.0 ** -24 and np.float32(float(a) * float(b) + 1.0) == np.float32(1.0)
    cases = [(a, b, np.float32(1.0)), (-a, b, np.float32(-1.0)), (a, -b, np.float32(1.0)), (-a, -b, np.float32(1.0))]
    for x, y, z in cases:
        got = VP.fma_f32(x, y, z)
        assert got == _fma_exact(x, y, z), (x, y, z, got)
    assert VP.fma_f32(a, b, np.float32(1.0)) == np.float32(1 + 2.0 ** -23)
    # the same product below a midpoint: 1 + 2^-23 + 2^-24 - tiny rounds down to 1 + 2^-23
    lo = np.float32(1 + 2.0 ** -23)
    assert VP.fma_f32(-a, b, np.float32(1 + 2.0 ** -22)) == _fma_exact(-a, b, np.float32(1 + 2.0 ** -22))
    assert VP.fma_f32(a, b, lo) == _fma_exact(a, b, lo)


def test_rms_sum_order_known_answers():
    full = np.zeros(128, np.float32)
    # group 0 = [2^12, 1 x 7]: in order, 2^24 + 1 ties to the even 2^24 seven times -> 2^24
    # (small values first would give 2^24 + 8); group 1 = 1 x 8 -> 8; the tree adds them: 2^24 + 8
    full[0] = 2.0 ** 12
    full[1:8] = 1.0
    full[8:16] = 1.0
    assert VP.rms_sum(full) == np.float32(2.0 ** 24 + 8)
    # one sequential chain over all 16 ones after 2^24 would stay at 2^24
    chain = np.float32(0)
    for x in full:
        chain = VP.fma_f32(x, x, chain)
    assert chain == np.float32(2.0 ** 24)
    # groups are 8 consecutive dims, not strided: put the big value in dim 8 (group 1) and ones in
    # dims 0-7 (group 0) and 9-15: group 1 in order = 2^24 (its 7 ones tie away), group 0 = 8
    g = np.zeros(128, np.float32)
    g[0:8] = 1.0
    g[8] = 2.0 ** 12
    g[9:16] = 1.0
    assert VP.rms_sum(g) == np.float32(2.0 ** 24 + 8)
    # halves are summed last: 2^24 in the first half's tree, the second half's ones are separate
    h = np.zeros(128, np.float32)
    h[0] = 2.0 ** 12
    h[64:72] = 1.0
    h[72:80] = 1.0
    assert VP.rms_sum(h) == np.float32(2.0 ** 24 + 16)
    # against exact sums where no rounding occurs (small integers)
    rng = np.random.default_rng(1)
    x = rng.integers(-20, 20, (50, 128)).astype(np.float32)
    assert np.array_equal(VP.rms_sum(x), (x.astype(np.float64) ** 2).sum(-1).astype(np.float32))


def _rows(rng, n):
    x = bf16.round_bf16(rng.standard_normal((n, 128)).astype(np.float32))
    ang = rng.uniform(-np.pi, np.pi, (n, 64))
    c = bf16.round_bf16(np.cos(ang).astype(np.float32))
    s = bf16.round_bf16(np.sin(ang).astype(np.float32))
    return x, c, s


def test_rope_special_cases():
    rng = np.random.default_rng(2)
    x, _, _ = _rows(rng, 20)
    one, zero = np.ones((20, 64), np.float32), np.zeros((20, 64), np.float32)
    assert np.array_equal(VP.rope_rms(x, one, zero), x)  # identity rotation
    quarter = VP.rope_rms(x, zero, one)  # (x, y) -> (-y, x)
    assert np.array_equal(quarter[:, :64], -x[:, 64:]) and np.array_equal(quarter[:, 64:], x[:, :64])


def test_rope_rms_close_to_fp64_and_one_rounding_per_output():
    rng = np.random.default_rng(3)
    x, c, s = _rows(rng, 400)
    w = bf16.round_bf16((rng.random(128) + 0.5).astype(np.float32))
    x64, c64, s64 = x.astype(np.float64), c.astype(np.float64), s.astype(np.float64)
    rot = np.concatenate([x64[:, :64] * c64 - x64[:, 64:] * s64, x64[:, 64:] * c64 + x64[:, :64] * s64], -1)
    got = VP.rope_rms(x, c, s)
    # one rounding of a (nearly) exact value: within half a bf16 ulp of it, plus the fp32 error of
    # the separate product inside the FMA
    half_ulp = 2.0 ** (np.floor(np.log2(np.abs(rot) + 1e-300)) - 8)
    slack = 2.0 ** -23 * (np.abs(x64) * np.concatenate([np.abs(c64), np.abs(c64)], -1) +
                          np.abs(np.roll(x64, 64, axis=-1)) * np.concatenate([np.abs(s64), np.abs(s64)], -1))
    assert np.all(np.abs(got - rot) <= half_ulp + slack)
    normed = VP.rope_rms(x, c, s, w, 1e-6)
    ref = got.astype(np.float64) / np.sqrt((got.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(normed - ref) / (np.abs(ref) + 1e-3)) < 2.0 ** -8
    # the rounding points differ from the torch op order (three roundings): they disagree somewhere
    hf = bf16.add(bf16.mul(x[:, :64], c), bf16.mul(-x[:, 64:], s))
    assert not np.array_equal(hf, got[:, :64])


def test_ring_value_and_head_scale_roundings():
    rng = np.random.default_rng(4)
    v = bf16.round_bf16(rng.standard_normal((30, 2, 128)).astype(np.float32))
    s = bf16.round_bf16(np.array([0.75, 1.3], np.float32))
    inv = VP.inv_scale(s)
    assert inv.dtype == np.float32 and np.array_equal(inv, (np.float32(1) / s).astype(np.float32))
    vr = VP.ring_value(v, inv)
    assert np.array_equal(vr, bf16.round_bf16(v * inv[:, None]))
    # V / s carries one bf16 rounding: s * (V / s) is within one bf16 ulp of V
    assert np.all(np.abs(vr * s[:, None] - v) <= np.abs(v) * 2.0 ** -8 + 1e-30)
    assert np.array_equal(VP.head_scale(vr, s), bf16.round_bf16(vr * s[:, None]))
    assert np.array_equal(VP.ring_value(v, np.ones(2, np.float32)), v)


def test_merged_sequence_matches_scaled_history_attention():
    """The merged path's s * attn([V_old | V_ring / s]) against attn([s V_old | V_ring]) in fp64
    (identical up to the V / s rounding and the two output roundings), through a commit."""

    rng = np.random.default_rng(5)
    L, Hq, Hkv, C = 2, 4, 2, 8
    params = []
    for _ in range(L):
        w = bf16.round_bf16((rng.random(128) + 0.5).astype(np.float32))
        s = bf16.round_bf16((rng.random(Hkv) + 0.5).astype(np.float32))
        params.append((w, w[::-1].copy(), 1e-6, s))
    alpha = bf16.round_bf16(rng.random((L, Hkv)).astype(np.float32))
    inv_freq = 1.0 / (10000.0 ** (np.arange(0, 128, 2) / 128))

    def rotary(pos):
        f = np.asarray(pos, np.float64)[:, None] * inv_freq[None]
        return bf16.round_bf16(np.cos(f).astype(np.float32)), bf16.round_bf16(np.sin(f).astype(np.float32))

    seq = VP.MergedSequence(L, Hkv, C, params, alpha, rotary)
    k_raw, v_raw = {}, {}
    worst = 0.0
    for step, n in enumerate([5, 3, 8, 1, 1, 6]):
        seq.begin_step()
        p0 = seq.seen
        for l in range(L):
            q = bf16.round_bf16(rng.standard_normal((n, Hq, 128)).astype(np.float32))
            k = bf16.round_bf16(rng.standard_normal((n, Hkv, 128)).astype(np.float32))
            v = bf16.round_bf16(rng.standard_normal((n, Hkv, 128)).astype(np.float32))
            got = seq.layer(l, q, k, v, Hq)
            qn_w, kn_w, eps, s = params[l]
            cos, sin = rotary(np.arange(p0, p0 + n))
            qn = VP.rope_rms(q, cos[:, None], sin[:, None], qn_w, eps)
            last = p0 + n - 1
            rec = max(0, last // C * C - C)
            # the same keys; values as the HF contract sees them: s * V_old, the ring unscaled
            K = np.stack([seq.slab_k[t] for t in range(rec)] + [seq.ring_k[l][t] for t in range(rec, last + 1)], 1)[None]
            V = np.stack([seq.slab_v[t] * s[:, None] for t in range(rec)] +
                         [seq.ring_v[l][t] * s[:, None] for t in range(rec, last + 1)], 1)[None]
            want, _ = A.attention(np.transpose(qn, (1, 0, 2))[None], K, V, causal_bottom_right=True)
            want = np.transpose(want[0], (1, 0, 2))
            worst = max(worst, A.rel_l2(got, want))
            if l == L - 1:
                for i in range(n):
                    k_raw[p0 + i], v_raw[p0 + i] = seq.slab_k[p0 + i], v[i]
        seq.end_step(n)
    assert worst < 4e-3, worst  # two bf16 output roundings
    assert seq.committed == 16
    # the committed chunk [8, 16) of layer 0's ring is the V / s-domain blend with the raw slab
    assert all(np.array_equal(seq.slab_v[t], v_raw[t]) for t in range(8, 16))

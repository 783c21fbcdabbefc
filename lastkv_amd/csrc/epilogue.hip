// Fused QKV epilogue (RoPE + q/k RMSNorm + tiled K/V cache append) and the chunk-boundary blend.
//
// Epilogue, decode-sized calls: one wave per (token, head) of the Hq + Hkv heads; lane l owns dims
// l and l + 64, the two halves that rotate_half pairs, so RoPE needs no lane exchange and RMSNorm
// one wave sum.  Calls of many tokens: the block form below (16-byte accesses, V tiles written
// through LDS).  Two rounding contracts: the torch op order of the HF model (every intermediate
// rounded to bf16 where the reference's bf16 torch ops round) and the vLLM fused_qkv kernel's
// (fused multiply-adds, one rounding per output, a fixed RMSNorm summation order).
#include <algorithm>

#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

// Value of the bf16 nearest to x (round to nearest even), as fp32, in one v_cvt_pk_bf16_f32: with
// bf16(0) = 0 as the low half, the packed word is that fp32 value (no shift or mask to unpack it).
__device__ inline float rb(float x) { return __uint_as_float(pack_bf16x2(0.f, x)); }

// The torch-order RMSNorm's fp32 sum of squares of one row, in the order both epilogue forms share
// (the reference's own reduction order is torch's and not fixed): for each of the 8 groups of dims
// [8g, 8g + 8) with their partners 64 + 8g.., a fused multiply-add chain over the group's dims in
// order (dim 8g + j, then 64 + 8g + j), then the groups' sums added pairwise (g xor 1, 2, 4).  Here
// lane l holds dims l and l + 64 (the wave's row), so group g is lanes 8g .. 8g + 7.
__device__ inline float row_sumsq_lanes(float r0, float r1, int lane) {
  const int base = lane & ~7;
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float a = __shfl(r0, base + e), b = __shfl(r1, base + e);
    ss = __builtin_fmaf(a, a, ss);
    ss = __builtin_fmaf(b, b, ss);
  }
#pragma unroll
  for (int off = 8; off <= 32; off <<= 1) ss += __shfl_xor(ss, off);
  return ss;
}

struct QkvParams {
  int32_t batch, tokens, hq, hkv;
  float eps;
  int32_t pos_c;
  const int32_t* pos;
  const uint16_t *q, *k, *v;
  int64_t q_sb, q_st, k_sb, k_st, v_sb, v_st;
  const uint16_t *cos, *sin;
  int64_t cs_sb, cs_st;
  const uint16_t *qw, *kw;
  uint16_t* q_out;
  int64_t qo_sb, qo_st;
  uint16_t *rk, *rv;
  int64_t r_ss, r_hs;
  int32_t ring_tokens, ring_slots;
  const int32_t* ring_slot;
  uint16_t *dk, *dv;
  int64_t d_ss, d_hs;
  int32_t deep_cap, deep_slots;
  const int32_t* deep_slot;
  // optional page tables: block j of sequence b is page tab[b * tab_stride + j] of the pool
  const int32_t* r_tab;
  int64_t r_tab_stride, r_page;
  int32_t r_npages;
  const int32_t* d_tab;
  int64_t d_tab_stride, d_page;
  int32_t d_npages;
  int32_t rounding;      // 0: torch op order (HF model), 1: vLLM fused_qkv order
  const float* rv_mul;   // ring V := bf16(v * rv_mul[g]) (the vLLM path's V / s rings), or nullptr
  // ragged rows: sequence b's tokens are rows cu[b] .. cu[b + 1] - 1 (tokens = the call's total row
  // count, max_seqlen bounds a sequence's count); nullptr: `tokens` tokens per sequence
  const int32_t* cu;
  int32_t max_seqlen;
};

// First row and token count of sequence b (ragged calls; offsets clamped into [0, tokens]).
__device__ inline int2 ragged_rows(const QkvParams& p, int b) {
  const int s0 = min(max(p.cu[b], 0), p.tokens);
  return make_int2(s0, min(min(max(p.cu[b + 1], s0), p.tokens) - s0, p.max_seqlen));
}

// Sequence of ragged row t: the largest b with cu[b] <= t.
__device__ inline int ragged_seq(const QkvParams& p, int t) {
  int lo = 0, hi = p.batch;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.cu[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

// Element offset of token i of sequence b in a tensor with batch / token strides (sb, st); ragged
// calls address row `row` (= first row of b + i) instead.
__device__ inline int64_t tok_off(const QkvParams& p, int b, int i, int64_t row, int64_t sb, int64_t st) {
  return p.cu ? row * st : b * sb + i * st;
}

// Element offset of block blk of sequence b: contiguous per slot, or a clamped page of a pool.
__device__ inline int64_t write_block(const int32_t* tab, int64_t tab_stride, int64_t page, int32_t npages, int b,
                                      int blk) {
  if (tab == nullptr) return static_cast<int64_t>(blk) * kBlockElems;
  return static_cast<int64_t>(min(max(tab[b * tab_stride + blk], 0), npages - 1)) * page;
}

// vLLM fused_qkv arithmetic (fused_qkv.py:24-55) of one row, lane l holding dims l and l + 64:
// r = (bf16(fma(x0, c, -(x1 * s))), bf16(fma(x1, c, x0 * s))); the RMSNorm sum runs over the 16
// groups of 8 consecutive dims (lanes 8j..8j+7 of each half), the squares of a group accumulated
// in order with fused multiply-adds, then adjacent groups added pairwise (lane xor 8, 16, 32, then
// the two halves); out = bf16(r * inv * w) with fp32 products.  No contraction: every product and
// sum rounds where the reference's does.
__device__ inline void rope_norm_vllm_lane(float x0, float x1, float c, float s, const uint16_t* w, int lane,
                                           float eps, float& r0, float& r1) {
#pragma clang fp contract(off)
  r0 = rb(__builtin_fmaf(x0, c, -(x1 * s)));
  r1 = rb(__builtin_fmaf(x1, c, x0 * s));
  if (w == nullptr) return;
  const int base = lane & ~7;
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float ua = __shfl(r0, base + e), ub = __shfl(r1, base + e);
    sa = __builtin_fmaf(ua, ua, sa);
    sb = __builtin_fmaf(ub, ub, sb);
  }
#pragma unroll
  for (int off = 8; off <= 32; off <<= 1) {
    sa += __shfl_xor(sa, off);
    sb += __shfl_xor(sb, off);
  }
  const float inv = 1.0f / sqrtf((sa + sb) / static_cast<float>(kHeadDim) + eps);
  r0 = rb(r0 * inv * bf16_bits_to_f32(w[lane]));
  r1 = rb(r1 * inv * bf16_bits_to_f32(w[lane + 64]));
}

__global__ __launch_bounds__(256) void qkv_epilogue_kernel(const QkvParams p) {
  const int lane = threadIdx.x & 63;
  const int heads = p.hq + p.hkv;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= (p.cu ? 1 : static_cast<int64_t>(p.batch)) * p.tokens * heads) return;
  const int h = static_cast<int>(item % heads);
  const int64_t tok = item / heads;  // (ragged: the row)
  int i = static_cast<int>(tok % p.tokens);
  int b = static_cast<int>(tok / p.tokens);
  if (p.cu) {
    b = ragged_seq(p, static_cast<int>(tok));
    const int2 r = ragged_rows(p, b);
    i = static_cast<int>(tok) - r.x;
    if (i < 0 || i >= r.y) return;  // a row past a clamped sequence
  }
  const bool is_q = h < p.hq;
  const int g = h - p.hq;
  const uint16_t* src = is_q ? p.q + tok_off(p, b, i, tok, p.q_sb, p.q_st) + static_cast<int64_t>(h) * kHeadDim
                             : p.k + tok_off(p, b, i, tok, p.k_sb, p.k_st) + static_cast<int64_t>(g) * kHeadDim;
  const float x0 = bf16_bits_to_f32(src[lane]);
  const float x1 = bf16_bits_to_f32(src[lane + 64]);
  const uint16_t* cp = p.cos + tok_off(p, b, i, tok, p.cs_sb, p.cs_st);
  const uint16_t* sp = p.sin + tok_off(p, b, i, tok, p.cs_sb, p.cs_st);
  const float c0 = bf16_bits_to_f32(cp[lane]), c1 = bf16_bits_to_f32(cp[lane + 64]);
  const float s0 = bf16_bits_to_f32(sp[lane]), s1 = bf16_bits_to_f32(sp[lane + 64]);
  const uint16_t* w = is_q ? p.qw : p.kw;
  float r0, r1;
  if (p.rounding == 0) {
    // q * cos + rotate_half(q) * sin, rotate_half(q) = cat(-q[64:], q[:64]); three bf16 roundings
    r0 = rb(rb(x0 * c0) + rb(-x1 * s0));
    r1 = rb(rb(x1 * c1) + rb(x0 * s1));
    if (w != nullptr) {
      const float ss = row_sumsq_lanes(r0, r1, lane);
      const float inv = 1.0f / sqrtf(ss / static_cast<float>(kHeadDim) + p.eps);
      r0 = rb(bf16_bits_to_f32(w[lane]) * rb(r0 * inv));
      r1 = rb(bf16_bits_to_f32(w[lane + 64]) * rb(r1 * inv));
    }
  } else {
    rope_norm_vllm_lane(x0, x1, c0, s0, w, lane, p.eps, r0, r1);
  }
  const uint16_t o0 = f32_to_bf16_bits(r0), o1 = f32_to_bf16_bits(r1);
  if (is_q) {
    uint16_t* dst = p.q_out + tok_off(p, b, i, tok, p.qo_sb, p.qo_st) + static_cast<int64_t>(h) * kHeadDim;
    dst[lane] = o0;
    dst[lane + 64] = o1;
    return;
  }
  const int position = (p.pos ? p.pos[b] : p.pos_c) + i;
  if (position < 0) return;
  const uint16_t* vrow = p.v + tok_off(p, b, i, tok, p.v_sb, p.v_st) + static_cast<int64_t>(g) * kHeadDim;
  const uint16_t v0 = vrow[lane], v1 = vrow[lane + 64];
  {
    // the ring's V, scaled for the vLLM path (fp32 product, one rounding); the deep write is raw
    const float m = p.rv_mul != nullptr ? p.rv_mul[g] : 1.f;
    const uint16_t rv0 = p.rv_mul != nullptr ? f32_to_bf16_bits(bf16_bits_to_f32(v0) * m) : v0;
    const uint16_t rv1 = p.rv_mul != nullptr ? f32_to_bf16_bits(bf16_bits_to_f32(v1) * m) : v1;
    const int slot = p.r_tab ? 0 : (p.ring_slot ? p.ring_slot[b] : b);
    if (slot >= 0 && slot < p.ring_slots) {
      const int rt = position % p.ring_tokens;
      const int64_t off = slot * p.r_ss + g * p.r_hs + write_block(p.r_tab, p.r_tab_stride, p.r_page, p.r_npages, b, rt >> 5);
      uint16_t* kb = p.rk + off;
      uint16_t* vb = p.rv + off;
      const int wt = rt & 31;
      kb[k_tile_offset(wt, lane)] = o0;
      kb[k_tile_offset(wt, lane + 64)] = o1;
      vb[v_tile_offset(wt, lane)] = rv0;
      vb[v_tile_offset(wt, lane + 64)] = rv1;
    }
  }
  if (p.dk != nullptr && position < p.deep_cap) {
    const int slot = p.d_tab ? 0 : (p.deep_slot ? p.deep_slot[b] : b);
    if (slot >= 0 && slot < p.deep_slots) {
      const int64_t off = slot * p.d_ss + g * p.d_hs + write_block(p.d_tab, p.d_tab_stride, p.d_page, p.d_npages, b, position >> 5);
      uint16_t* kb = p.dk + off;
      uint16_t* vb = p.dv + off;
      const int wt = position & 31;
      kb[k_tile_offset(wt, lane)] = o0;
      kb[k_tile_offset(wt, lane + 64)] = o1;
      vb[v_tile_offset(wt, lane)] = v0;
      vb[v_tile_offset(wt, lane + 64)] = v1;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Block form of the epilogue for calls of many tokens (prefill pieces): the same arithmetic with
// 16-byte loads and stores.  Eight lanes own one 128-dim row; lane l of the eight holds dims
// [8l, 8l + 8) and [64 + 8l, 64 + 8l + 8), the pairs rotate_half combines, so RoPE needs no lane
// exchange and RMSNorm's sum three xor shuffles.  The first workgroups take one (sequence,
// 32-position block, kv head) each: K goes to its tile row by row (64-byte runs), V is transposed
// through LDS and written to its tile (d-major) with 16-byte stores, both to the ring block and, on
// the final layer, to the shared-store block.  The others take query rows, two heads of one token
// per 8-lane group.
constexpr int kRowLanes = 8;
constexpr int kVStride = 40;  // LDS row of one V dim: 32 tokens + 8 pad elements (80 bytes, 16-byte aligned)

__device__ inline void unpack8(uint4 u, float (&x)[8]) {
  x[0] = bf16_lo(u.x), x[1] = bf16_hi(u.x), x[2] = bf16_lo(u.y), x[3] = bf16_hi(u.y);
  x[4] = bf16_lo(u.z), x[5] = bf16_hi(u.z), x[6] = bf16_lo(u.w), x[7] = bf16_hi(u.w);
}

__device__ inline uint4 pack8(const float (&x)[8]) {
  return make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7]));
}

// Eight bf16 values kept packed (four registers instead of eight), unpacked where they are used:
// the block kernel then needs 92 VGPRs instead of 100, five waves per SIMD instead of four
// (measured at config 3's prefill call shape: 333-342 vs 340-347 us).
struct Packed8 {
  uint4 u;
  __device__ float operator[](int j) const {
    const uint32_t w = j < 2 ? u.x : j < 4 ? u.y : j < 6 ? u.z : u.w;
    return (j & 1) ? bf16_hi(w) : bf16_lo(w);
  }
};

// The norm weights of lane l's dims (loaded once per thread, ahead of its row loads: a load issued
// after them would make each row's s_waitcnt wait for every row load in flight).
struct NormW {
  Packed8 w0, w1;
  bool on;
};

// The same weights unpacked to fp32 once (the query rows: each thread normalises several rows with
// them; the K/V rows keep them packed, where the registers matter more).
struct Unpacked8 {
  float v[8];
  __device__ float operator[](int j) const { return v[j]; }
};
struct NormWU {
  Unpacked8 w0, w1;
  bool on;
};

__device__ inline NormW norm_weights(const uint16_t* w, int l);

__device__ inline NormWU norm_weights_unpacked(const uint16_t* w, int l) {
  const NormW p = norm_weights(w, l);
  NormWU r;
  r.on = p.on;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    r.w0.v[j] = p.w0[j];
    r.w1.v[j] = p.w1[j];
  }
  return r;
}

__device__ inline NormW norm_weights(const uint16_t* w, int l) {
  NormW r;
  r.on = w != nullptr;
  uint4 a = make_uint4(0, 0, 0, 0), b = a;
  if (w != nullptr) {
    a = *reinterpret_cast<const uint4*>(w + 8 * l);
    b = *reinterpret_cast<const uint4*>(w + 64 + 8 * l);
  }
  r.w0.u = a;
  r.w1.u = b;
  return r;
}

// One token's cos / sin values of lane l's dims, shared by every head of the token.
struct RopeCS {
  Packed8 c0, c1, s0, s1;
};

__device__ inline RopeCS rope_cs(uint4 ca, uint4 cb, uint4 sa, uint4 sb) {
  return RopeCS{{ca}, {cb}, {sa}, {sb}};
}

// Rounds a and b to bf16 (round to nearest even), one instruction each (rb): two conversions
// cost less than one v_cvt_pk_bf16_f32 of the pair and the two instructions unpacking it.
__device__ inline void rb2(float& a, float& b) {
  a = rb(a);
  b = rb(b);
}

// RoPE then RMSNorm of the row held by an 8-lane group (lane l: dims 8l.. in a / 64 + 8l.. in b),
// every bf16 operation of the reference rounded in the same order (rb; the last rounding is the
// packing of the output).
template <class NW>
__device__ inline void rope_norm_row(uint4& a, uint4& b, const RopeCS& cs, const NW& w, float eps) {
  float x0[8], x1[8], r0[8], r1[8];
  unpack8(a, x0), unpack8(b, x1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float p0 = x0[j] * cs.c0[j], p1 = -x1[j] * cs.s0[j], p2 = x1[j] * cs.c1[j], p3 = x0[j] * cs.s1[j];
    rb2(p0, p1);
    rb2(p2, p3);
    r0[j] = p0 + p1;
    r1[j] = p2 + p3;
    rb2(r0[j], r1[j]);
  }
  if (w.on) {
    // the sum of squares in the order row_sumsq_lanes takes (this lane is group l of the row)
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss = __builtin_fmaf(r0[j], r0[j], ss);
      ss = __builtin_fmaf(r1[j], r1[j], ss);
    }
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kHeadDim) + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float u0 = r0[j] * inv, u1 = r1[j] * inv;
      rb2(u0, u1);
      r0[j] = w.w0[j] * u0;  // rounded by the packing below
      r1[j] = w.w1[j] * u1;
    }
  }
  a = pack8(r0);
  b = pack8(r1);
}

// The vLLM fused_qkv order (fused_qkv.py:24-55) of the row held by an 8-lane group: lane l holds
// dims [8l, 8l + 8) and [64 + 8l, 64 + 8l + 8), i.e. groups l and 8 + l of the 16 groups of 8 dims
// whose squares the reference accumulates in order with fused multiply-adds; adjacent groups are
// then added pairwise (lane xor 1, 2, 4) and the two halves last.  cos / sin of dims [0, 64) rotate
// both halves.
template <class NW>
__device__ inline void rope_norm_row_vllm(uint4& a, uint4& b, const RopeCS& cs, const NW& w, float eps) {
#pragma clang fp contract(off)
  float x0[8], x1[8], r0[8], r1[8];
  unpack8(a, x0), unpack8(b, x1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    r0[j] = __builtin_fmaf(x0[j], cs.c0[j], -(x1[j] * cs.s0[j]));
    r1[j] = __builtin_fmaf(x1[j], cs.c0[j], x0[j] * cs.s0[j]);
    rb2(r0[j], r1[j]);
  }
  if (w.on) {
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sa = __builtin_fmaf(r0[j], r0[j], sa);
      sb = __builtin_fmaf(r1[j], r1[j], sb);
    }
#pragma unroll
    for (int off = 1; off <= 4; off <<= 1) {
      sa += __shfl_xor(sa, off);
      sb += __shfl_xor(sb, off);
    }
    const float inv = 1.0f / sqrtf((sa + sb) / static_cast<float>(kHeadDim) + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      r0[j] = r0[j] * inv * w.w0[j];  // rounded by the packing below
      r1[j] = r1[j] * inv * w.w1[j];
    }
  }
  a = pack8(r0);
  b = pack8(r1);
}

// kMode 1: the vLLM order (fixed at compile time); kMode 0: either order, by `rounding` at run time.
// (A block kernel specialised to the HF order measured slower for q, k, v as separate tensors:
// 311-316 against 305-310 us at config 3's prefill call, same box, four rounds.)
template <int kMode, class NW>
__device__ inline void rope_norm_row_any(uint4& a, uint4& b, const RopeCS& cs, const NW& w, float eps, int rounding) {
  if (kMode == 0 && rounding == 0)
    rope_norm_row(a, b, cs, w, eps);
  else
    rope_norm_row_vllm(a, b, cs, w, eps);
}

// 8 bf16 values times m (fp32 products, one rounding each).
__device__ inline uint4 scale8(uint4 x, float m) {
  float f[8];
  unpack8(x, f);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] *= m;
  return pack8(f);
}

__device__ inline void load_row(const uint16_t* row, int l, uint4& a, uint4& b) {
  a = *reinterpret_cast<const uint4*>(row + 8 * l);
  b = *reinterpret_cast<const uint4*>(row + 64 + 8 * l);
}

// Projection rows are read once and outputs written once per call: non-temporal accesses keep them
// from displacing the cos / sin rows and norm weights that every head rereads.
__device__ inline void load_row_nt(const uint16_t* row, int l, uint4& a, uint4& b) {
  a = load_nt(row + 8 * l);
  b = load_nt(row + 64 + 8 * l);
}

__device__ inline void store_nt(uint16_t* dst, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(dst));
}

// The cos or sin values of lane l's dims: dims [0, 64) only in the vLLM order, whose rotation takes
// them for both halves (the block kernel's vLLM instance then issues half the loads).
template <int kRounding>
__device__ inline void load_cs(const uint16_t* row, int l, uint4& a, uint4& b) {
  a = *reinterpret_cast<const uint4*>(row + 8 * l);
  if constexpr (kRounding == 0)
    b = *reinterpret_cast<const uint4*>(row + 64 + 8 * l);
  else
    b = make_uint4(0, 0, 0, 0);
}

// query heads of one token per 8-lane group (one cos / sin load for all; measured at config 3's
// prefill call shape: 2 heads 310 us, 4 heads 313 us, 8 heads 335 us per call)
constexpr int kQRows = 2;

// kv heads per K/V workgroup: they share each token's cos / sin loads (measured at config 3's
// prefill call, same box, four rounds: vLLM order 265-268 against 284-287 us with one head per
// workgroup, HF order 313-316 against 320-328 us with the fused projection's rows)
constexpr int kKvPerWg = 2;

// The query rows of one 8-lane group: kQRows heads of one token and the token's cos / sin rows.
struct QItem {
  uint4 xa[kQRows], xb[kQRows], ca, cb, sa, sb;
};

// grp = (b, i, head group).  The loads are unconditional (a group past the end rereads the last
// one, heads past Hq the last head) so that the compiler can count them for s_waitcnt and the next
// group's loads stay in flight while this one is computed.
template <int kRounding>
__device__ inline void q_item_load(const QkvParams& p, int32_t grp, int32_t groups, int hgroups, int l, QItem& it) {
  grp = grp < groups ? grp : groups - 1;
  const int h0 = grp % hgroups * kQRows;
  const int tok = grp / hgroups;  // (ragged: the row; the query rows need no sequence)
  const int i = p.cu ? tok : tok % p.tokens, b = p.cu ? 0 : tok / p.tokens;
  const uint16_t* qrow = p.q + b * p.q_sb + i * p.q_st;
#pragma unroll
  for (int r = 0; r < kQRows; ++r)
    load_row_nt(qrow + static_cast<int64_t>(min(h0 + r, p.hq - 1)) * kHeadDim, l, it.xa[r], it.xb[r]);
  load_cs<kRounding>(p.cos + b * p.cs_sb + i * p.cs_st, l, it.ca, it.cb);
  load_cs<kRounding>(p.sin + b * p.cs_sb + i * p.cs_st, l, it.sa, it.sb);
}

template <int kRounding, class NW>
__device__ inline void q_item_store(const QkvParams& p, int32_t grp, int32_t groups, int hgroups, int l, const NW& w,
                                    QItem& it) {
  if (grp >= groups) return;
  const int h0 = grp % hgroups * kQRows;
  const int tok = grp / hgroups;
  const int i = p.cu ? tok : tok % p.tokens, b = p.cu ? 0 : tok / p.tokens;
  uint16_t* dst = p.q_out + b * p.qo_sb + i * p.qo_st + static_cast<int64_t>(h0) * kHeadDim;
  const RopeCS cs = rope_cs(it.ca, it.cb, it.sa, it.sb);
#pragma unroll
  for (int r = 0; r < kQRows; ++r) {
    if (h0 + r >= p.hq) break;
    rope_norm_row_any<kRounding>(it.xa[r], it.xb[r], cs, w, p.eps, p.rounding);
    store_nt(dst + r * kHeadDim + 8 * l, it.xa[r]);
    store_nt(dst + r * kHeadDim + 64 + 8 * l, it.xb[r]);
  }
}

// Workgroups [0, kv_wgs) take one (sequence, 32-position block, pair of kv heads) each; the rest 32 groups of
// kQRows query rows (heads [kQRows j, kQRows j + kQRows) of one token, j < ceil(Hq / kQRows)).  The
// vLLM order runs instance 1 (half the cos / sin loads, 74 instead of 92 VGPRs: 280-282 against
// 284-287 us at config 3's prefill call), the HF order instance 0.
template <int kRounding>
__global__ __launch_bounds__(256) void qkv_block_kernel(const QkvParams p, int32_t kv_wgs, int32_t kv_blocks) {
  __shared__ uint16_t sv[kKvPerWg * kHeadDim * kVStride];
  const int t = threadIdx.x, l = t & (kRowLanes - 1);
  if (static_cast<int>(blockIdx.x) >= kv_wgs) {
    const int hgroups = (p.hq + kQRows - 1) / kQRows;
    const int32_t groups = (p.cu ? 1 : p.batch) * p.tokens * hgroups;  // < 2^31 (checked by the host)
    const int32_t grp = (static_cast<int32_t>(blockIdx.x) - kv_wgs) * 32 + (t >> 3);
    if (grp >= groups) return;
    const NormWU w = norm_weights_unpacked(p.qw, l);
    QItem it;
    q_item_load<kRounding>(p, grp, groups, hgroups, l, it);
    q_item_store<kRounding>(p, grp, groups, hgroups, l, w, it);
    return;
  }
  // kv heads 2 gp and 2 gp + 1 (if present) of one (sequence, 32-position block): each token's
  // cos / sin rows are loaded once for both
  const int kv = static_cast<int>(blockIdx.x);
  const int hpairs = (p.hkv + kKvPerWg - 1) / kKvPerWg;
  const int jr = kv % kv_blocks, gp = (kv / kv_blocks) % hpairs, b = kv / (kv_blocks * hpairs);
  const int p0 = p.pos ? p.pos[b] : p.pos_c;
  if (p0 < 0) return;  // (uniform over the workgroup)
  // this sequence's tokens: rows [r0, r0 + n) of a ragged call, else tokens [0, p.tokens)
  const int2 rr = p.cu ? ragged_rows(p, b) : make_int2(0, p.tokens);
  const int n = rr.y;
  const int blk = (p0 >> 5) + jr;             // positions [32 blk, 32 blk + 32)
  if (blk * kBlockTokens >= p0 + n) return;   // past this sequence's tokens (uniform)
  const int w = t >> 3;                       // this thread's token of the block
  const int i = blk * kBlockTokens + w - p0;  // its index in the sequence
  const bool valid = i >= 0 && i < n;
  const int64_t row = static_cast<int64_t>(rr.x) + i;  // (ragged calls)
  const int rslot = p.r_tab ? 0 : (p.ring_slot ? p.ring_slot[b] : b);
  const bool ring_ok = rslot >= 0 && rslot < p.ring_slots;
  const int dslot = p.d_tab ? 0 : (p.deep_slot ? p.deep_slot[b] : b);
  const bool deep_ok = p.dk != nullptr && dslot >= 0 && dslot < p.deep_slots && blk * kBlockTokens < p.deep_cap;
  const int rblk = ((blk * kBlockTokens) % p.ring_tokens) >> 5;
  const int64_t rbase = ring_ok ? rslot * p.r_ss + write_block(p.r_tab, p.r_tab_stride, p.r_page, p.r_npages, b, rblk) : 0;
  const int64_t dbase = deep_ok ? dslot * p.d_ss + write_block(p.d_tab, p.d_tab_stride, p.d_page, p.d_npages, b, blk) : 0;
  const int g0 = gp * kKvPerWg, ng = min(kKvPerWg, p.hkv - g0);  // (uniform)
  const NormW kw = norm_weights(p.kw, l);
  if (valid) {
    static_assert(kKvPerWg == 2, "the K/V path below holds two heads");
    uint4 ka0, kb0, va0, vb0, ka1, kb1, va1, vb1, ca, cb, sa, sb;
    const int64_t go0 = static_cast<int64_t>(g0) * kHeadDim, go1 = static_cast<int64_t>(min(g0 + 1, p.hkv - 1)) * kHeadDim;
    const uint16_t* krow = p.k + tok_off(p, b, i, row, p.k_sb, p.k_st);
    const uint16_t* vrow = p.v + tok_off(p, b, i, row, p.v_sb, p.v_st);
    load_row_nt(krow + go0, l, ka0, kb0);
    load_row_nt(vrow + go0, l, va0, vb0);
    load_row_nt(krow + go1, l, ka1, kb1);  // (a missing second head rereads the first)
    load_row_nt(vrow + go1, l, va1, vb1);
    load_cs<kRounding>(p.cos + tok_off(p, b, i, row, p.cs_sb, p.cs_st), l, ca, cb);
    load_cs<kRounding>(p.sin + tok_off(p, b, i, row, p.cs_sb, p.cs_st), l, sa, sb);
    const RopeCS cs = rope_cs(ca, cb, sa, sb);
    // dims [8l, 8l + 8) and [64 + 8l, 64 + 8l + 8) of token w are 16 contiguous bytes each in a K tile
    const int ko0 = k_tile_offset(w, 8 * l), ko1 = k_tile_offset(w, 64 + 8 * l);
    auto head = [&](int h, uint4 ka, uint4 kb, uint4 va, uint4 vb) __attribute__((always_inline)) {
      rope_norm_row_any<kRounding>(ka, kb, cs, kw, p.eps, p.rounding);
      const int g = g0 + h;
      if (ring_ok) {
        store_nt(p.rk + rbase + g * p.r_hs + ko0, ka);
        store_nt(p.rk + rbase + g * p.r_hs + ko1, kb);
      }
      if (deep_ok) {
        store_nt(p.dk + dbase + g * p.d_hs + ko0, ka);
        store_nt(p.dk + dbase + g * p.d_hs + ko1, kb);
      }
      const uint16_t* ea = reinterpret_cast<const uint16_t*>(&va);
      const uint16_t* eb = reinterpret_cast<const uint16_t*>(&vb);
      uint16_t* svh = sv + h * (kHeadDim * kVStride);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        svh[(8 * l + e) * kVStride + w] = ea[e];
        svh[(64 + 8 * l + e) * kVStride + w] = eb[e];
      }
    };
    head(0, ka0, kb0, va0, vb0);
    if (ng > 1) head(1, ka1, kb1, va1, vb1);
  }
  __syncthreads();
  // V tiles: element (token w, dim d) at d * 32 + w; 512 runs of 8 tokens of one dim per head.  The
  // ring takes bf16(v * rv_mul[g]) on the vLLM path, the deep store the raw V.
  const int lo = max(0, p0 - blk * kBlockTokens), hi = min(kBlockTokens, p0 + n - blk * kBlockTokens);
#pragma unroll
  for (int h = 0; h < kKvPerWg; ++h) {
    if (h >= ng) break;
    const int g = g0 + h;
    const int64_t roff = rbase + g * p.r_hs, doff = dbase + g * p.d_hs;
    const float vm = p.rv_mul != nullptr ? p.rv_mul[g] : 1.f;
    const uint16_t* svh = sv + h * (kHeadDim * kVStride);
#pragma unroll
    for (int run = t; run < kHeadDim * 4; run += 256) {
      const int d = run >> 2, w0 = 8 * (run & 3);
      if (w0 + 8 <= lo || w0 >= hi) continue;
      const uint4 x = *reinterpret_cast<const uint4*>(svh + d * kVStride + w0);
      const uint4 xr = p.rv_mul != nullptr ? scale8(x, vm) : x;
      if (w0 >= lo && w0 + 8 <= hi) {
        if (ring_ok) store_nt(p.rv + roff + d * kBlockTokens + w0, xr);
        if (deep_ok) store_nt(p.dv + doff + d * kBlockTokens + w0, x);
      } else {  // a block edge of the call: only its own tokens
        const uint16_t* e = reinterpret_cast<const uint16_t*>(&x);
        const uint16_t* er = reinterpret_cast<const uint16_t*>(&xr);
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // (constant indices: the 8 values stay in registers)
          if (w0 + j < lo || w0 + j >= hi) continue;
          if (ring_ok) p.rv[roff + d * kBlockTokens + w0 + j] = er[j];
          if (deep_ok) p.dv[doff + d * kBlockTokens + w0 + j] = e[j];
        }
      }
    }
  }
}

struct BlendParams {
  int32_t layers, batch, heads;
  int32_t start, end;  // chunk tokens [start, end)
  int32_t blk0, nblk;  // blocks covering the chunk
  uint16_t *rk, *rv;
  int64_t r_ls, r_ss, r_hs;
  int32_t ring_tokens;
  const uint16_t *dk, *dv;
  int64_t d_ss, d_hs;
  const float *alpha, *om, *vs;
  const int32_t* r_tab;  // [layers, batch, .] ring pages, or nullptr
  int64_t r_tab_ls, r_tab_stride, r_page;
  int32_t r_npages;
  const int32_t* d_tab;  // [batch, .] shared-store pages, or nullptr
  int64_t d_tab_stride, d_page;
  int32_t d_npages;
};

// One thread per 8-element (16-byte) run of one block of one (layer, sequence, head).  K and
// V runs are handled by separate threads (kind = item parity).
__global__ __launch_bounds__(256) void blend_kernel(const BlendParams p) {
  const int64_t per_block = kBlockElems / 8;
  const int64_t total = static_cast<int64_t>(p.layers) * p.batch * p.heads * p.nblk * per_block * 2;
  for (int64_t item = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; item < total;
       item += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int kind = static_cast<int>(item & 1);
    int64_t rest = item >> 1;
    const int run = static_cast<int>(rest % per_block);
    rest /= per_block;
    const int blk = p.blk0 + static_cast<int>(rest % p.nblk);
    rest /= p.nblk;
    const int g = static_cast<int>(rest % p.heads);
    rest /= p.heads;
    const int b = static_cast<int>(rest % p.batch);
    const int l = static_cast<int>(rest / p.batch);
    const int off = run * 8;
    const int base_tok = blk * kBlockTokens;
    const int ring_blk = (base_tok % p.ring_tokens) >> 5;
    const int lh = l * p.heads + g;
    const float a = p.alpha[lh], om = p.om[lh];
    const float s = (kind == 1 && p.vs != nullptr) ? p.vs[lh] : 1.f;
    const int64_t doff = (p.d_tab ? 0 : b * p.d_ss) + g * p.d_hs +
                         write_block(p.d_tab, p.d_tab_stride, p.d_page, p.d_npages, b, blk);
    const int64_t roff = p.r_tab ? g * p.r_hs + write_block(p.r_tab + l * p.r_tab_ls, p.r_tab_stride, p.r_page,
                                                            p.r_npages, b, ring_blk)
                                 : l * p.r_ls + b * p.r_ss + g * p.r_hs + static_cast<int64_t>(ring_blk) * kBlockElems;
    const uint16_t* dsrc = (kind == 0 ? p.dk : p.dv) + doff + off;
    uint16_t* rdst = (kind == 0 ? p.rk : p.rv) + roff + off;
    const uint4 dv4 = *reinterpret_cast<const uint4*>(dsrc);
    uint4 rv4 = *reinterpret_cast<const uint4*>(rdst);
    const uint16_t* de = reinterpret_cast<const uint16_t*>(&dv4);
    uint16_t* re = reinterpret_cast<uint16_t*>(&rv4);
    // token index of each element of the run: K runs hold 8 dims of one token, V runs 8 tokens
    int w_k = 0;
    if (kind == 0) {
      const int r = (off >> 5) & 15, u = (off >> 11) & 1;
      w_k = 8 * (r >> 2) + 4 * u + (r & 3);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int tokpos = base_tok + (kind == 0 ? w_k : ((off & 31) + j));
      if (tokpos < p.start || tokpos >= p.end) continue;
      const float src = bf16_bits_to_f32(de[j]);
      const float own = bf16_bits_to_f32(re[j]);
      const float scaled = kind == 1 ? rb(src * s) : src;
      re[j] = f32_to_bf16_bits(rb(a * scaled) + rb(om * own));
    }
    *reinterpret_cast<uint4*>(rdst) = rv4;
  }
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_qkv_epilogue(const lkv_qkv_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_qkv_args)), "lkv_qkv_args size mismatch");
  LKV_REQUIRE(a->head_dim == kHeadDim, "head_dim must be 128, got %d", a->head_dim);
  LKV_REQUIRE(a->batch >= 0 && a->tokens >= 0 && a->num_q_heads > 0 && a->num_kv_heads > 0, "bad sizes");
  LKV_REQUIRE(a->q && a->k && a->v && a->cos && a->sin && a->q_out, "null tensor pointer");
  LKV_REQUIRE(a->ring_k && a->ring_v, "ring cache required");
  LKV_REQUIRE(a->ring_tokens > 0 && a->ring_tokens % kBlockTokens == 0, "ring_tokens must be a positive multiple of 32");
  const bool rpaged = a->ring_block_table != nullptr, dpaged = a->deep_block_table != nullptr;
  if (rpaged) {
    LKV_REQUIRE(a->ring_num_pages > 0 && a->ring_table_stride * kBlockTokens >= a->ring_tokens,
                "ring page table must hold ring_tokens / 32 pages of a non-empty pool");
  } else {
    LKV_REQUIRE(a->ring_num_slots > 0, "ring_num_slots must be positive");
    LKV_REQUIRE(a->ring_slot != nullptr || a->ring_num_slots >= a->batch, "ring has fewer slots than sequences");
  }
  LKV_REQUIRE((a->deep_k == nullptr) == (a->deep_v == nullptr), "deep_k and deep_v must both be set");
  LKV_REQUIRE(a->deep_k == nullptr || a->deep_capacity_tokens % kBlockTokens == 0, "deep capacity must be a multiple of 32");
  if (a->deep_k != nullptr && dpaged) {
    LKV_REQUIRE(a->deep_num_pages > 0 && a->deep_table_stride * kBlockTokens >= a->deep_capacity_tokens,
                "deep page table must hold deep_capacity_tokens / 32 pages of a non-empty pool");
  } else if (a->deep_k != nullptr) {
    LKV_REQUIRE(a->deep_slot != nullptr || a->deep_num_slots >= a->batch, "deep cache has fewer slots than sequences");
  }
  LKV_REQUIRE(a->positions != nullptr || a->position_const >= 0, "negative position");
  LKV_REQUIRE(a->rounding == 0 || a->rounding == 1, "rounding must be 0 (torch op order) or 1 (vLLM fused_qkv), got %d",
              a->rounding);
  const bool ragged = a->cu_seqlens != nullptr;
  LKV_REQUIRE(!ragged || a->batch == 0 || a->tokens == 0 || a->max_seqlen >= 1,
              "ragged calls need max_seqlen >= 1, got %d", a->max_seqlen);
  // token rows of the call: tokens per sequence x batch, or the ragged call's total
  const int64_t rows = ragged ? (a->batch > 0 ? a->tokens : 0) : static_cast<int64_t>(a->batch) * a->tokens;
  // tokens of the longest sequence
  const int64_t seq_tokens = ragged ? std::min(a->max_seqlen, a->tokens) : a->tokens;
  const int64_t items = rows * (a->num_q_heads + a->num_kv_heads);
  if (items == 0) return LKV_OK;
  LKV_REQUIRE(items / 4 + 1 < (1LL << 31), "too many tokens in one call");
  QkvParams p;
  p.batch = a->batch;
  p.tokens = a->tokens;
  p.hq = a->num_q_heads;
  p.hkv = a->num_kv_heads;
  p.eps = a->eps;
  p.pos_c = a->position_const;
  p.pos = a->positions;
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.q_sb = a->q_stride_b;
  p.q_st = a->q_stride_t;
  p.k_sb = a->k_stride_b;
  p.k_st = a->k_stride_t;
  p.v_sb = a->v_stride_b;
  p.v_st = a->v_stride_t;
  p.cos = static_cast<const uint16_t*>(a->cos);
  p.sin = static_cast<const uint16_t*>(a->sin);
  p.cs_sb = a->cs_stride_b;
  p.cs_st = a->cs_stride_t;
  p.qw = static_cast<const uint16_t*>(a->q_norm_w);
  p.kw = static_cast<const uint16_t*>(a->k_norm_w);
  p.q_out = static_cast<uint16_t*>(a->q_out);
  p.qo_sb = a->q_out_stride_b;
  p.qo_st = a->q_out_stride_t;
  p.rk = static_cast<uint16_t*>(a->ring_k);
  p.rv = static_cast<uint16_t*>(a->ring_v);
  p.r_ss = a->ring_seq_stride;
  p.r_hs = a->ring_head_stride;
  p.ring_tokens = a->ring_tokens;
  p.ring_slots = a->ring_num_slots;
  p.ring_slot = a->ring_slot;
  p.dk = static_cast<uint16_t*>(a->deep_k);
  p.dv = static_cast<uint16_t*>(a->deep_v);
  p.d_ss = a->deep_seq_stride;
  p.d_hs = a->deep_head_stride;
  p.deep_cap = a->deep_k ? a->deep_capacity_tokens : 0;
  p.deep_slots = dpaged ? 1 : a->deep_num_slots;
  p.deep_slot = a->deep_slot;
  p.ring_slots = rpaged ? 1 : a->ring_num_slots;
  p.r_tab = a->ring_block_table;
  p.r_tab_stride = a->ring_table_stride;
  p.r_page = a->ring_page_stride;
  p.r_npages = a->ring_num_pages;
  p.d_tab = a->deep_block_table;
  p.d_tab_stride = a->deep_table_stride;
  p.d_page = a->deep_page_stride;
  p.d_npages = a->deep_num_pages;
  p.rounding = a->rounding;
  p.rv_mul = a->ring_v_mul;
  p.cu = a->cu_seqlens;
  p.max_seqlen = static_cast<int32_t>(seq_tokens);
  // Calls of many tokens per sequence (16 or more; ragged calls: the longest sequence) with
  // 16-byte-aligned rows take the block form (16-byte accesses, V tiles written through LDS),
  // provided the call's 32-position blocks do not wrap onto each other in the ring; decode-sized
  // calls keep one wave per (token, head) however many sequences they hold (B = 32 one-token rows:
  // 7 us against 22 us in block form, whose workgroups would each hold one token of a block).
  auto aligned = [](const void* ptr, int64_t s0, int64_t s1) {
    return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0 && s0 % 8 == 0 && s1 % 8 == 0;
  };
  // 32-position blocks one sequence's tokens span (exact for host-constant positions)
  const int64_t kv_blocks = a->positions != nullptr || ragged
                                ? (seq_tokens + kBlockTokens - 1) / kBlockTokens + 1
                                : (a->position_const + a->tokens - 1) / kBlockTokens - a->position_const / kBlockTokens + 1;
  const bool block_form = seq_tokens >= 16 && kv_blocks <= a->ring_tokens / kBlockTokens &&
                          aligned(a->q, a->q_stride_b, a->q_stride_t) && aligned(a->k, a->k_stride_b, a->k_stride_t) &&
                          aligned(a->v, a->v_stride_b, a->v_stride_t) && aligned(a->cos, a->cs_stride_b, a->cs_stride_t) &&
                          aligned(a->sin, a->cs_stride_b, a->cs_stride_t) &&
                          aligned(a->q_out, a->q_out_stride_b, a->q_out_stride_t) && aligned(a->q_norm_w, 0, 0) &&
                          aligned(a->k_norm_w, 0, 0) && aligned(a->ring_k, a->ring_seq_stride, a->ring_head_stride) &&
                          aligned(a->ring_v, a->ring_page_stride, 0) &&
                          aligned(a->deep_k, a->deep_seq_stride, a->deep_head_stride) &&
                          aligned(a->deep_v, a->deep_page_stride, 0);
  if (block_form) {
    const int64_t q_groups = rows * ((a->num_q_heads + kQRows - 1) / kQRows);
    const int64_t kv_wgs = static_cast<int64_t>(a->batch) * ((a->num_kv_heads + kKvPerWg - 1) / kKvPerWg) * kv_blocks;
    const int64_t wgs = kv_wgs + (q_groups + 31) / 32;
    LKV_REQUIRE(wgs < (1LL << 31) && q_groups < (1LL << 31) - 32, "too many tokens in one call");
    if (p.rounding == 0)
      qkv_block_kernel<0><<<static_cast<unsigned>(wgs), 256, 0, as_stream(stream)>>>(p, static_cast<int32_t>(kv_wgs),
                                                                                 static_cast<int32_t>(kv_blocks));
    else
      qkv_block_kernel<1><<<static_cast<unsigned>(wgs), 256, 0, as_stream(stream)>>>(p, static_cast<int32_t>(kv_wgs),
                                                                                 static_cast<int32_t>(kv_blocks));
  } else {
    const int blocks = static_cast<int>((items + 3) / 4);
    qkv_epilogue_kernel<<<blocks, 256, 0, as_stream(stream)>>>(p);
  }
  return check_launch("lkv_qkv_epilogue");
}

extern "C" int32_t lkv_blend_chunk(const lkv_blend_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_blend_args)), "lkv_blend_args size mismatch");
  LKV_REQUIRE(a->layers >= 0 && a->batch >= 0 && a->kv_heads > 0, "bad sizes");
  LKV_REQUIRE(a->chunk_start >= 0 && a->chunk_len >= 0, "bad chunk range");
  LKV_REQUIRE(a->ring_tokens > 0 && a->ring_tokens % kBlockTokens == 0, "ring_tokens must be a positive multiple of 32");
  LKV_REQUIRE(a->chunk_len <= a->ring_tokens, "chunk longer than the ring");
  LKV_REQUIRE(static_cast<int64_t>(a->chunk_start) + a->chunk_len <= a->deep_capacity_tokens, "chunk beyond the deep capacity");
  LKV_REQUIRE(a->ring_k && a->ring_v && a->deep_k && a->deep_v && a->alpha && a->one_minus_alpha, "null pointer");
  LKV_REQUIRE(a->ring_block_table == nullptr ||
                  (a->ring_num_pages > 0 && a->ring_table_stride * kBlockTokens >= a->ring_tokens),
              "ring page table must hold ring_tokens / 32 pages of a non-empty pool");
  LKV_REQUIRE(a->deep_block_table == nullptr ||
                  (a->deep_num_pages > 0 && a->deep_table_stride * kBlockTokens >= a->deep_capacity_tokens),
              "deep page table must hold deep_capacity_tokens / 32 pages of a non-empty pool");
  if (a->layers == 0 || a->batch == 0 || a->chunk_len == 0) return LKV_OK;
  // two blocks of the chunk must not share a ring block, or their threads would race on it
  const int first_blk = a->chunk_start / kBlockTokens;
  const int last_blk = (a->chunk_start + a->chunk_len - 1) / kBlockTokens;
  LKV_REQUIRE(last_blk - first_blk + 1 <= a->ring_tokens / kBlockTokens,
              "chunk [%d, %d) spans more 32-token blocks than the ring holds (%d tokens)", a->chunk_start,
              a->chunk_start + a->chunk_len, a->ring_tokens);
  BlendParams p;
  p.layers = a->layers;
  p.batch = a->batch;
  p.heads = a->kv_heads;
  p.start = a->chunk_start;
  p.end = a->chunk_start + a->chunk_len;
  p.blk0 = first_blk;
  p.nblk = last_blk - first_blk + 1;
  p.rk = static_cast<uint16_t*>(a->ring_k);
  p.rv = static_cast<uint16_t*>(a->ring_v);
  p.r_ls = a->ring_layer_stride;
  p.r_ss = a->ring_seq_stride;
  p.r_hs = a->ring_head_stride;
  p.ring_tokens = a->ring_tokens;
  p.dk = static_cast<const uint16_t*>(a->deep_k);
  p.dv = static_cast<const uint16_t*>(a->deep_v);
  p.d_ss = a->deep_seq_stride;
  p.d_hs = a->deep_head_stride;
  p.alpha = a->alpha;
  p.om = a->one_minus_alpha;
  p.vs = a->vscale;
  p.r_tab = a->ring_block_table;
  p.r_tab_ls = a->ring_table_layer_stride;
  p.r_tab_stride = a->ring_table_stride;
  p.r_page = a->ring_page_stride;
  p.r_npages = a->ring_num_pages;
  p.d_tab = a->deep_block_table;
  p.d_tab_stride = a->deep_table_stride;
  p.d_page = a->deep_page_stride;
  p.d_npages = a->deep_num_pages;
  const int64_t total = static_cast<int64_t>(a->layers) * a->batch * a->kv_heads * p.nblk * (kBlockElems / 8) * 2;
  const int64_t want = (total + 255) / 256;
  const int grid = static_cast<int>(want < 65536 ? want : 65536);
  blend_kernel<<<grid, 256, 0, as_stream(stream)>>>(p);
  return check_launch("lkv_blend_chunk");
}

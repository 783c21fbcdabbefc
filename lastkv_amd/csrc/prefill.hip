// Chunked-prefill attention on MFMA for gfx950: several query tokens per sequence attend to
// [older shared segment (non-causal) | local ring segment (bottom-right causal or bidirectional)].
//
// Workgroup = NW waves = one (sequence, kv head, query tile); workgroups are numbered so that the
// tiles of one (sequence, kv head) run on one XCD and share its L2.  Query rows are (token, head)
// pairs of the GQA group, row = token * G + head, so every K/V block feeds all heads of the group.
// Each wave owns 32 rows (two 16-column groups of the 16x16x32 MFMA tiles), few enough registers
// (< 256 VGPRs, accumulators in VGPRs) for two waves per SIMD.
// Per 32-token key block:
//   - the NW waves each fetch 16 / NW of the block's 16 one-KiB fragments from HBM/L2 into
//     registers one block ahead (one contiguous 1 KiB run per load instruction), convert V to
//     fp16 (applying bf16(V * s) on the older segment) and publish the block to an LDS double
//     buffer in lane order, so every MFMA operand is one conflict-free ds_read_b128;
//   - S^T = K * Q^T with 16x16x32 bf16 MFMAs (exact products, fp32 sums);
//   - online softmax in the exp2 domain (scale and offset folded into one FMA), row max over the
//     four 16-lane rows with VALU lane swaps, row sums kept per lane and reduced once at the end,
//     O rescaled (a branch taken only when some row's offset moved) with the factor each lane
//     already holds;
//   - O^T += V^T * P^T with 16x16x32 fp16 MFMAs: P in [0, 1] carries 11 mantissa bits (bf16
//     would carry 8, a 1.7e-3 relative error the rel-L2 1e-3 bound does not allow), and bf16 V
//     converts to fp16 exactly for |V| < 65504 (larger values saturate).
#include "attn_common.h"
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr float kNegInf = -__builtin_inff();
// log2 of the largest unnormalised probability.  0 keeps the exact running maximum: a larger
// slack skips rescales but lets fp16 P round relative to a stale offset, which measurably
// raises the output error (rel-L2 6e-4 -> 1.1e-3 on random data at slack 8).
constexpr float kSlack = 0.f;

struct PrefillParams {
  const uint16_t* q;
  int64_t q_sb, q_st;
  uint16_t* out;
  int64_t out_sb, out_st;
  float* lse;
  const uint16_t* ok;
  const uint16_t* ov;
  int64_t o_ss, o_hs;
  const int32_t* o_len;
  int32_t o_len_c, o_cap;
  const int32_t* o_slot;
  int32_t o_nslots;
  const float* vscale;
  const uint16_t* lk;
  const uint16_t* lv;
  int64_t l_ss, l_hs;
  int32_t ring_blocks;
  const int32_t* l_len;
  int32_t l_len_c;
  const int32_t* l_start;
  int32_t l_start_c;
  const int32_t* l_slot;
  int32_t l_nslots;
  int32_t L, hq, hkv, group, causal, tiles;
  float scale_log2;
};

__device__ inline uint32_t f16x2_bits(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// 8 bf16 -> 8 fp16 (exact in range); with kScale the value is bf16(v * s) first.
template <bool kScale>
__device__ inline uint4 v_to_f16(uint4 v, float s) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  auto cv = [s](uint32_t w) -> uint32_t {
    float lo = bf16_lo(w), hi = bf16_hi(w);
    if (kScale) {  // one v_cvt_pk_bf16_f32 rounds both products
      const uint32_t packed = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo * s, hi * s}), bf16x2));
      lo = bf16_lo(packed);
      hi = bf16_hi(packed);
    }
    return f16x2_bits(lo, hi);
  };
  return make_uint4(cv(v.x), cv(v.y), cv(v.z), cv(v.w));
}

__device__ inline uint32_t pack_f16_rne(float lo, float hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 r;
  r.x = static_cast<_Float16>(lo);
  r.y = static_cast<_Float16>(hi);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ inline SeqView make_view(const PrefillParams& p, int b, int kvh) {
  SeqView sv;
  const int oslot = p.o_slot ? p.o_slot[b] : b;
  const int lslot = p.l_slot ? p.l_slot[b] : b;
  int n0 = p.o_len ? p.o_len[b] : p.o_len_c;
  int n1 = p.lk ? (p.l_len ? p.l_len[b] : p.l_len_c) : 0;
  n0 = (oslot < 0 || oslot >= p.o_nslots || p.ok == nullptr) ? 0 : min(max(n0, 0), p.o_cap);
  n1 = (lslot < 0 || lslot >= p.l_nslots) ? 0 : min(max(n1, 0), p.ring_blocks * kBlockTokens);
  int ls = p.l_start ? p.l_start[b] : p.l_start_c;
  ls = (ls < 0 || ls >= p.ring_blocks * kBlockTokens) ? 0 : ls;
  sv.ok = p.ok ? p.ok + static_cast<int64_t>(oslot) * p.o_ss + kvh * p.o_hs : nullptr;
  sv.ov = p.ov ? p.ov + static_cast<int64_t>(oslot) * p.o_ss + kvh * p.o_hs : nullptr;
  sv.lk = p.lk ? p.lk + static_cast<int64_t>(lslot) * p.l_ss + kvh * p.l_hs : nullptr;
  sv.lv = p.lv ? p.lv + static_cast<int64_t>(lslot) * p.l_ss + kvh * p.l_hs : nullptr;
  sv.n0 = n0;
  sv.n1 = n1;
  sv.nb0 = (n0 + kBlockTokens - 1) / kBlockTokens;
  sv.lblk0 = ls >> 5;
  sv.lead = ls & (kBlockTokens - 1);
  sv.ring_blocks = p.ring_blocks;
  return sv;
}

// Local-segment tokens visible to a query token (causal: bottom-right aligned).
__device__ inline int visible_local(const PrefillParams& p, const SeqView& sv, int token) {
  const int v = p.causal ? sv.n1 - p.L + token + 1 : sv.n1;
  return min(max(v, 0), sv.n1);
}

// One fragment = one 16-byte-per-lane MFMA operand = 1 KiB; a 32-token block is 16 fragments:
// K fragments f = u * 4 + kb (u: 16-token half, kb: 32-dim slice) and V fragments 8 + nb (nb:
// 16-dim slice).  Wave w of NW stages fragments w, w + NW, ... of each block.
template <int NW>
struct Stage {
  uint4 r[16 / NW];
};

template <int NW>
__device__ inline void stage_load(Stage<NW>& st, const BlockRef& r, int wave, int n16, int g4) {
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int f = wave + j * NW;
    const uint16_t* src = f < 8 ? r.k + (f * 16 + n16) * 32 + 8 * g4 : r.v + (16 * (f - 8) + n16) * 32 + 8 * g4;
    st.r[j] = *reinterpret_cast<const uint4*>(src);
  }
}

template <int NW, bool kVScale>
__device__ inline void stage_store(const Stage<NW>& st, uint4* buf, bool older, float vs, int wave, int lane) {
  // bf16(v * 1) == v, so local blocks take the same instructions with s = 1 (no branch)
  const float s = (kVScale && older) ? vs : 1.f;
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int f = wave + j * NW;
    uint4 x = st.r[j];
    if (f >= 8) x = kVScale ? v_to_f16<true>(x, s) : v_to_f16<false>(x, 1.f);
    buf[f * 64 + lane] = x;
  }
}

// Scores of one 16-column group for one block: s0 (tokens 8*g4 + 0..3) and s1 (8*g4 + 4..7) of
// column n16.
__device__ inline void gather_scores(f32x4 s0, f32x4 s1, float (&s)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = s0[i];
    s[4 + i] = s1[i];
  }
}

// -inf for tokens outside the block's valid range or past the column's causal limit.
__device__ inline void mask_scores(float (&s)[8], const BlockRef& r, int lim, int g4) {
  const int w0 = 8 * g4;
  const int hi = r.older ? r.hi : min(r.hi, lim - r.seg_tok + 1);
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = (w0 + j >= r.lo && w0 + j < hi) ? s[j] : kNegInf;
}

// Online-softmax update of one column group -> fp16 probabilities; m in the scaled exp2 domain,
// l partial (this lane's 8 tokens only; the four rows are summed once at the end).
__device__ inline uint4 softmax_core(const float (&s)[8], float c, float& m, float& l, float& alpha) {
  float mx = fmax3_nan(fmax3_nan(s[0], s[1], s[2]), fmax3_nan(s[3], s[4], s[5]), fmax_nan(s[6], s[7]));
  mx = wave_max_across_rows(mx) * c;
  // The row keeps its exp2 offset m until a block's maximum exceeds it by more than kSlack, so
  // P <= 2^kSlack; the final O / l ratio does not depend on the offset.
  const bool raise = mx > m + kSlack;  // m = -inf: true for the first finite maximum
  const float m_new = raise ? mx : m;
  // with no visible key yet m_new is -inf: subtract 0 instead, so exp2 gives 0 for every -inf
  const float m_sub = m_new == kNegInf ? 0.f : m_new;
  alpha = raise ? fast_exp2(m - m_sub) : 1.f;
  float pr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(__builtin_fmaf(s[j], c, -m_sub));
  l = l * alpha + (((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7])));
  m = m_new;
  return make_uint4(pack_f16_rne(pr[0], pr[1]), pack_f16_rne(pr[2], pr[3]), pack_f16_rne(pr[4], pr[5]),
                    pack_f16_rne(pr[6], pr[7]));
}

// O is accumulated transposed (O^T = V^T * P^T): lane (n16, g4) holds dims 16 * nb + 4 * g4 + i
// of query row n16, the row whose offset and factor the lane itself holds.
__device__ inline void rescale_rows(float alpha, f32x4 (&o)[8]) {
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[nb] *= alpha;
  }
}

// Workgroup = NW waves x 32 query rows (two 16-column groups per wave); K/V of each 32-token block
// go through a two-buffer LDS ring, fetched two blocks ahead.
template <int NW, bool kVScale>
__global__ __launch_bounds__(NW * 64) void prefill_kernel(const PrefillParams p) {
  __shared__ uint4 lds[2][1024];
  constexpr int kRowsPerWave = 32;
  constexpr int kRowsPerWg = NW * kRowsPerWave;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;
  const int logical = xcd_logical_index(blockIdx.x, gridDim.x);
  const int tile = logical % p.tiles;
  const int kvh = (logical / p.tiles) % p.hkv;
  const int b = logical / (p.tiles * p.hkv);
  const int G = p.group;
  const int rows_total = p.L * G;
  const int wg_row0 = tile * kRowsPerWg;
  const int row0 = wg_row0 + wave * kRowsPerWave;

  const SeqView sv = make_view(p, b, kvh);
  const int wg_last_row = min(rows_total, wg_row0 + kRowsPerWg) - 1;
  const int nbt = sv.nb0 + local_blocks(sv, visible_local(p, sv, wg_last_row / G));
  int w_nbt = 0;
  if (row0 < rows_total) {
    const int w_last_row = min(rows_total, row0 + kRowsPerWave) - 1;
    w_nbt = sv.nb0 + local_blocks(sv, visible_local(p, sv, w_last_row / G));
  }

  uint4 qf[2][4];
  int lim[2];  // last visible local-segment token of this lane's column
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    const int row = row0 + 16 * cg + n16;
    if (row < rows_total) {
      const int tok = row / G, h = row - tok * G;
      const uint16_t* qrow = p.q + b * p.q_sb + tok * p.q_st + static_cast<int64_t>(kvh * G + h) * kHeadDim;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qf[cg][kb] = *reinterpret_cast<const uint4*>(qrow + 32 * kb + 8 * g4);
      lim[cg] = visible_local(p, sv, tok) - 1;
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qf[cg][kb] = make_uint4(0, 0, 0, 0);
      lim[cg] = -1;
    }
  }
  const float vs = kVScale ? p.vscale[kvh] : 1.f;
  const float c = p.scale_log2;
  // smallest causal limit among the wave's rows (its first row); blocks past it need masking
  const int w_min_lim = row0 < rows_total ? visible_local(p, sv, row0 / G) - 1 : -1;

  float m[2] = {kNegInf, kNegInf}, l[2] = {0.f, 0.f};
  f32x4 o[2][8];
#pragma unroll
  for (int cg = 0; cg < 2; ++cg)
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[cg][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (nbt > 0) {
    // Loads are unconditional (indices past the end re-read the last block, an L2 hit) so that
    // the compiler can count outstanding loads for s_waitcnt.
    const int last = nbt - 1;
    Stage<NW> st;
    stage_load<NW>(st, block_ref(sv, 0), wave, n16, g4);
    stage_store<NW, kVScale>(st, lds[0], 0 < sv.nb0, vs, wave, lane);
    stage_load<NW>(st, block_ref(sv, min(1, last)), wave, n16, g4);
    __syncthreads();

    // step(blk): block blk is in `cur`, block blk + 1 is in flight into `st`; at the end it is
    // published into `nxt` and block blk + 2 is requested.
    auto step = [&](int blk, const uint4* cur, uint4* nxt) {
      if (blk < w_nbt) {
        const BlockRef r = block_ref(sv, blk);
        f32x4 s00 = {0.f, 0.f, 0.f, 0.f}, s01 = s00, s10 = s00, s11 = s00;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const uint4 k0 = cur[kb * 64 + lane];
          const uint4 k1 = cur[(4 + kb) * 64 + lane];
          s00 = mfma_bf16(k0, qf[0][kb], s00);
          s10 = mfma_bf16(k0, qf[1][kb], s10);
          s01 = mfma_bf16(k1, qf[0][kb], s01);
          s11 = mfma_bf16(k1, qf[1][kb], s11);
        }
        float sc0[8], sc1[8];
        gather_scores(s00, s01, sc0);
        gather_scores(s10, s11, sc1);
        // partial block, or a local block crossing the causal limit of some row of this wave
        if (r.lo > 0 || r.hi < kBlockTokens || (!r.older && r.seg_tok + kBlockTokens - 1 > w_min_lim)) {
          mask_scores(sc0, r, lim[0], g4);
          mask_scores(sc1, r, lim[1], g4);
        }
        float a0, a1;
        const uint4 p0 = softmax_core(sc0, c, m[0], l[0], a0);
        const uint4 p1 = softmax_core(sc1, c, m[1], l[1], a1);
        rescale_rows(a0, o[0]);
        rescale_rows(a1, o[1]);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const uint4 vf = cur[512 + nb * 64 + lane];
          o[0][nb] = mfma_f16(vf, p0, o[0][nb]);
          o[1][nb] = mfma_f16(vf, p1, o[1][nb]);
        }
      }
      // rows of this wave that see no more keys skip the math but keep the workgroup's staging;
      // the store is unconditional (after the last block it rewrites a clamped copy nobody reads),
      // so every path through the loop has the same loads outstanding and the waits stay partial
      stage_store<NW, kVScale>(st, nxt, blk + 1 < sv.nb0, vs, wave, lane);
      stage_load<NW>(st, block_ref(sv, min(blk + 2, last)), wave, n16, g4);
      __syncthreads();
    };
    for (int blk = 0; blk < nbt; blk += 2) {
      step(blk, lds[0], lds[1]);
      if (blk + 1 >= nbt) break;
      step(blk + 1, lds[1], lds[0]);
    }
  }

  // normalise and write: lane (n16, g4) holds dims 16 * nb + 4 * g4 + i of row n16 of each group
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    const float lt = wave_sum_across_rows(l[cg]);
    const float linv = lt > 0.f ? 1.f / lt : 0.f;
    const int row = row0 + 16 * cg + n16;
    if (row < rows_total) {
      const int tok = row / G, h = row - tok * G;
      uint16_t* orow = p.out + b * p.out_sb + tok * p.out_st + static_cast<int64_t>(kvh * G + h) * kHeadDim;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const f32x4 x = o[cg][nb] * linv;
        *reinterpret_cast<uint2*>(orow + 16 * nb + 4 * g4) = make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]));
      }
      if (p.lse != nullptr && g4 == 0)
        p.lse[(static_cast<int64_t>(b) * p.L + tok) * p.hq + kvh * G + h] =
            lt > 0.f ? (m[cg] + __log2f(lt)) * kLn2 : kNegInf;
    }
  }
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_prefill_attn(const lkv_prefill_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_prefill_args)),
              "lkv_prefill_args size mismatch (caller %d, library %d)", a->struct_size,
              static_cast<int32_t>(sizeof(lkv_prefill_args)));
  LKV_REQUIRE(a->head_dim == kHeadDim, "head_dim must be 128, got %d", a->head_dim);
  LKV_REQUIRE(a->batch >= 0 && a->tokens >= 0 && a->num_kv_heads > 0 && a->num_q_heads > 0, "bad sizes");
  LKV_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  const int group = a->num_q_heads / a->num_kv_heads;
  LKV_REQUIRE(a->causal == 0 || a->causal == 1, "causal must be 0 or 1");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->older_vscale_mode == 1, "older_vscale_mode must be 0 or 1");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->vscale != nullptr, "older_vscale_mode 1 needs vscale");
  LKV_REQUIRE(a->q != nullptr && a->out != nullptr, "null q/out");
  LKV_REQUIRE((a->older_k == nullptr) == (a->older_v == nullptr), "older_k and older_v must both be set");
  LKV_REQUIRE((a->local_k == nullptr) == (a->local_v == nullptr), "local_k and local_v must both be set");
  LKV_REQUIRE(a->older_k == nullptr || a->older_capacity_tokens % kBlockTokens == 0,
              "older capacity must be a multiple of 32 tokens");
  LKV_REQUIRE(a->older_k == nullptr || a->older_num_slots > 0, "older_num_slots must be positive");
  LKV_REQUIRE(a->older_k == nullptr || a->older_slot != nullptr || a->older_num_slots >= a->batch,
              "older_num_slots < batch with identity slots");
  LKV_REQUIRE(a->local_k == nullptr || a->local_ring_blocks > 0, "local ring needs at least one block");
  LKV_REQUIRE(a->local_k == nullptr || a->local_num_slots > 0, "local_num_slots must be positive");
  LKV_REQUIRE(a->local_k == nullptr || a->local_slot != nullptr || a->local_num_slots >= a->batch,
              "local_num_slots < batch with identity slots");
  LKV_REQUIRE((a->q_stride_b % 8) == 0 && (a->q_stride_t % 8) == 0 && (reinterpret_cast<uintptr_t>(a->q) & 15) == 0,
              "q rows must be 16-byte aligned");
  LKV_REQUIRE((a->out_stride_b % 4) == 0 && (a->out_stride_t % 4) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 7) == 0,
              "out rows must be 8-byte aligned");
  const uintptr_t align_or = reinterpret_cast<uintptr_t>(a->older_k) | reinterpret_cast<uintptr_t>(a->older_v) |
                             reinterpret_cast<uintptr_t>(a->local_k) | reinterpret_cast<uintptr_t>(a->local_v);
  LKV_REQUIRE((align_or & 15) == 0, "caches must be 16-byte aligned");
  LKV_REQUIRE((a->older_seq_stride | a->older_head_stride | a->local_seq_stride | a->local_head_stride) % 8 == 0,
              "cache strides must be multiples of 8 elements");
  if (a->batch == 0 || a->tokens == 0) return LKV_OK;
  PrefillParams p;
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_stride_b;
  p.q_st = a->q_stride_t;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_sb = a->out_stride_b;
  p.out_st = a->out_stride_t;
  p.lse = a->lse;
  p.ok = static_cast<const uint16_t*>(a->older_k);
  p.ov = static_cast<const uint16_t*>(a->older_v);
  p.o_ss = a->older_seq_stride;
  p.o_hs = a->older_head_stride;
  p.o_len = a->older_len;
  p.o_len_c = a->older_len_const;
  p.o_cap = a->older_capacity_tokens;
  p.o_slot = a->older_slot;
  p.o_nslots = a->older_num_slots;
  p.vscale = a->vscale;
  p.lk = static_cast<const uint16_t*>(a->local_k);
  p.lv = static_cast<const uint16_t*>(a->local_v);
  p.l_ss = a->local_seq_stride;
  p.l_hs = a->local_head_stride;
  p.ring_blocks = a->local_k ? a->local_ring_blocks : 1;
  p.l_len = a->local_len;
  p.l_len_c = a->local_len_const;
  p.l_start = a->local_start;
  p.l_start_c = a->local_start_const;
  p.l_slot = a->local_slot;
  p.l_nslots = a->local_num_slots;
  p.L = a->tokens;
  p.hq = a->num_q_heads;
  p.group = group;
  p.causal = a->causal;
  p.scale_log2 = a->sm_scale * kLog2e;
  const int64_t rows = static_cast<int64_t>(a->tokens) * group;
  // wide: 8 waves x 32 rows (two waves per SIMD); narrow: 2 waves x 32 rows
  const bool wide = rows > 64;
  const int64_t rows_per_wg = wide ? 8 * 32 : 2 * 32;
  const int64_t tiles = (rows + rows_per_wg - 1) / rows_per_wg;
  const int64_t wgs = tiles * a->num_kv_heads * a->batch;
  LKV_REQUIRE(wgs < (1LL << 31), "too many query rows");
  p.tiles = static_cast<int32_t>(tiles);
  p.hkv = a->num_kv_heads;
  hipStream_t s = as_stream(stream);
  const bool vsc = a->older_vscale_mode == 1;
  const dim3 grid(static_cast<unsigned>(wgs));
  if (wide) {
    if (vsc)
      prefill_kernel<8, true><<<grid, 8 * 64, 0, s>>>(p);
    else
      prefill_kernel<8, false><<<grid, 8 * 64, 0, s>>>(p);
  } else {
    if (vsc)
      prefill_kernel<2, true><<<grid, 2 * 64, 0, s>>>(p);
    else
      prefill_kernel<2, false><<<grid, 2 * 64, 0, s>>>(p);
  }
  return check_launch("lkv_prefill_attn");
}

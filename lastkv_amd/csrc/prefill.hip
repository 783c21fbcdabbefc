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
//     registers two blocks ahead (one contiguous 1 KiB run per load instruction), convert V to
//     fp16 (applying bf16(V * s) on the older segment) and publish the block to an LDS double
//     buffer in lane order, so every MFMA operand is one conflict-free ds_read_b128;
//   - S^T = K * Q^T with 16x16x32 bf16 MFMAs (exact products, fp32 sums);
//   - online softmax in the exp2 domain (scale and max folded into one FMA), row max over the
//     four 16-lane rows with VALU lane swaps, row sums kept per lane and reduced once at the end,
//     O rescaled only when some row's running max moved;
//   - O += P * V with 16x16x32 fp16 MFMAs: P in [0, 1] carries 11 mantissa bits (bf16 would
//     carry 8, a 1.7e-3 relative error the rel-L2 1e-3 bound does not allow), and bf16 V
//     converts to fp16 exactly for |V| < 65504 (larger values saturate).
#include "attn_common.h"
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr float kNegInf = -__builtin_inff();

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
  auto cv = [s](uint32_t w) -> uint32_t {
    float lo = bf16_lo(w), hi = bf16_hi(w);
    if (kScale) {
      const uint32_t packed = pack_bf16x2(lo * s, hi * s);
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
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int f = wave + j * NW;
    uint4 x = st.r[j];
    if (f >= 8) x = (kVScale && older) ? v_to_f16<true>(x, vs) : v_to_f16<false>(x, 1.f);
    buf[f * 64 + lane] = x;
  }
}

// Softmax step of one 16-column group for one block: scores s0 (tokens 8*g4 + 0..3) and s1
// (8*g4 + 4..7) of column n16 -> fp16 probabilities; m in the scaled exp2 domain, l partial
// (this lane's 8 tokens only; the four rows are summed once at the end).
__device__ inline uint4 softmax_step(f32x4 s0, f32x4 s1, const BlockRef& r, bool need_mask, int lim, int g4,
                                     float c, float& m, float& l, f32x4 (&o)[8]) {
  float s[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = s0[i];
    s[4 + i] = s1[i];
  }
  if (need_mask) {  // wave-uniform: partial block or a local block that crosses some row's causal limit
    const int w0 = 8 * g4;
    const int hi = r.older ? r.hi : min(r.hi, lim - r.seg_tok + 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = (w0 + j >= r.lo && w0 + j < hi) ? s[j] : kNegInf;
  }
  float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
  mx = wave_max_across_rows(mx) * c;
  const float m_new = fmaxf(m, mx);
  // with no visible key yet m_new is -inf: subtract 0 instead, so exp2 gives 0 for every -inf
  const float m_sub = m_new == kNegInf ? 0.f : m_new;
  const float alpha = fast_exp2(m - m_sub);
  float pr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(__builtin_fmaf(s[j], c, -m_sub));
  l = l * alpha + (((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7])));
  m = m_new;
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
    // O rows of this lane are columns 4*g4 + i, whose factors live in lanes 4*g4 + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __shfl(alpha, 4 * g4 + i);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) o[nb][i] *= a;
    }
  }
  return make_uint4(pack_f16_rne(pr[0], pr[1]), pack_f16_rne(pr[2], pr[3]), pack_f16_rne(pr[4], pr[5]),
                    pack_f16_rne(pr[6], pr[7]));
}

// Workgroup = NW waves x 32 query rows (two 16-column groups per wave); K/V of each 32-token
// block are staged through a three-buffer LDS ring, loaded three blocks ahead.
template <int NW, bool kVScale>
__global__ __launch_bounds__(NW * 64) void prefill_kernel(const PrefillParams p) {
  __shared__ uint4 lds[3][1024];
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
  int lim[2];
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
    // Software pipeline over blocks j (block j lives in LDS buffer j % 3, in registers set j % 2):
    //   iteration i: load block i + 3 -> registers; S(i + 1) = K(i + 1) Q^T (MFMA) while the
    //   softmax of S(i) runs on the VALU; O += P(i) V(i) (MFMA); publish block i + 2 to LDS.
    // Loads are unconditional (indices past the end re-read the last block, an L2 hit) so the
    // compiler can count outstanding loads for s_waitcnt.
    const int last = nbt - 1;
    Stage<NW> r0, r1;
    stage_load<NW>(r0, block_ref(sv, 0), wave, n16, g4);
    stage_load<NW>(r1, block_ref(sv, min(1, last)), wave, n16, g4);
    stage_store<NW, kVScale>(r0, lds[0], 0 < sv.nb0, vs, wave, lane);
    stage_store<NW, kVScale>(r1, lds[1], 1 < sv.nb0, vs, wave, lane);
    stage_load<NW>(r0, block_ref(sv, min(2, last)), wave, n16, g4);
    __syncthreads();

    auto qk = [&](const uint4* buf, f32x4& s00, f32x4& s01, f32x4& s10, f32x4& s11) {
      s00 = s01 = s10 = s11 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const uint4 k0 = buf[kb * 64 + lane];
        const uint4 k1 = buf[(4 + kb) * 64 + lane];
        s00 = mfma_bf16(k0, qf[0][kb], s00);
        s10 = mfma_bf16(k0, qf[1][kb], s10);
        s01 = mfma_bf16(k1, qf[0][kb], s01);
        s11 = mfma_bf16(k1, qf[1][kb], s11);
      }
    };
    f32x4 c00, c01, c10, c11;  // S of the block being softmaxed
    if (0 < w_nbt) qk(lds[0], c00, c01, c10, c11);
    // step(i): `ld` receives block i + 3, `st` (holding block i + 2) is published to LDS
    auto step = [&](int i, Stage<NW>& ld, Stage<NW>& st) {
      stage_load<NW>(ld, block_ref(sv, min(i + 3, last)), wave, n16, g4);
      f32x4 n00, n01, n10, n11;
      const bool next = i + 1 < w_nbt;
      if (next) qk(lds[(i + 1) % 3], n00, n01, n10, n11);
      if (i < w_nbt) {
        const BlockRef r = block_ref(sv, i);
        const bool need_mask = r.lo > 0 || r.hi < kBlockTokens || (!r.older && r.seg_tok + kBlockTokens - 1 > w_min_lim);
        const uint4 p0 = softmax_step(c00, c01, r, need_mask, lim[0], g4, c, m[0], l[0], o[0]);
        const uint4 p1 = softmax_step(c10, c11, r, need_mask, lim[1], g4, c, m[1], l[1], o[1]);
        const uint4* vb = lds[i % 3] + 512;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const uint4 vf = vb[nb * 64 + lane];
          o[0][nb] = mfma_f16(p0, vf, o[0][nb]);
          o[1][nb] = mfma_f16(p1, vf, o[1][nb]);
        }
      }
      if (next) {
        c00 = n00;
        c01 = n01;
        c10 = n10;
        c11 = n11;
      }
      if (i + 2 < nbt) stage_store<NW, kVScale>(st, lds[(i + 2) % 3], i + 2 < sv.nb0, vs, wave, lane);
      __syncthreads();
    };
    for (int i = 0; i < nbt; i += 2) {
      step(i, r1, r0);
      if (i + 1 >= nbt) break;
      step(i + 1, r0, r1);
    }
  }

  // normalise and write: lane (n16 = dim in slice nb, g4) holds rows 4*g4 + i of each column group
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    const float lt = wave_sum_across_rows(l[cg]);
    const float linv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = __shfl(linv, 4 * g4 + i);
      const int row = row0 + 16 * cg + 4 * g4 + i;
      if (row < rows_total) {
        const int tok = row / G, h = row - tok * G;
        uint16_t* orow = p.out + b * p.out_sb + tok * p.out_st + static_cast<int64_t>(kvh * G + h) * kHeadDim;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) orow[16 * nb + n16] = f32_to_bf16_bits(o[cg][nb][i] * f);
      }
    }
    if (p.lse != nullptr && g4 == 0) {
      const int row = row0 + 16 * cg + n16;
      if (row < rows_total) {
        const int tok = row / G, h = row - tok * G;
        p.lse[(static_cast<int64_t>(b) * p.L + tok) * p.hq + kvh * G + h] =
            lt > 0.f ? (m[cg] + __log2f(lt)) * kLn2 : kNegInf;
      }
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

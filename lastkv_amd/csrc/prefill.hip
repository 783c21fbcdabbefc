// Chunked-prefill attention on MFMA for gfx950: several query tokens per sequence attend to
// [older shared segment (non-causal) | local ring segment (bottom-right causal or bidirectional)].
//
// Workgroup = 4 waves = one (sequence, kv head, query tile).  Query rows are (token, head) pairs
// of the GQA group, row = token * G + head, so every K/V block feeds all heads of the group.
// Each wave owns 16 * CG rows (CG column groups of the 16-column MFMA tiles).
// Per 32-token key block:
//   - the four waves each fetch a quarter of the block from HBM/L2 (16-byte loads, one
//     contiguous 1 KiB run per load instruction) into registers one block ahead, convert V to
//     fp16 (applying bf16(V * s) on the older segment) and publish it to an LDS double buffer in
//     lane order, so every MFMA operand is one conflict-free ds_read_b128;
//   - S^T = K * Q^T with 16x16x32 bf16 MFMAs (exact products, fp32 sums);
//   - online softmax in the exp2 domain (scale and max folded into one FMA), O rescaled only
//     when some row's running max moved;
//   - O += P * V with 16x16x32 fp16 MFMAs: P in [0, 1] carries 11 mantissa bits (bf16 would
//     carry 8, a 1.7e-3 relative error the rel-L2 1e-3 bound does not allow), and bf16 V
//     converts to fp16 exactly for |V| < 65504 (larger values saturate).
#include "attn_common.h"
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr int kWaves = 4;
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
  int32_t L, hq, group, causal;
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

template <int CG, bool kVScale>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillParams p) {
  __shared__ uint4 lds[2][1024];  // per buffer: 8 K fragments x 64 lanes, then 8 V fragments

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;
  const int tile = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = p.group;
  const int rows_total = p.L * G;
  constexpr int kRows = 16 * CG;
  const int wg_row0 = tile * kWaves * kRows;
  const int row0 = wg_row0 + wave * kRows;

  const SeqView sv = make_view(p, b, kvh);
  const int wg_last_row = min(rows_total, wg_row0 + kWaves * kRows) - 1;
  const int nbt = sv.nb0 + local_blocks(sv, visible_local(p, sv, wg_last_row / G));
  int w_nbt = 0;
  if (row0 < rows_total) {
    const int w_last_row = min(rows_total, row0 + kRows) - 1;
    w_nbt = sv.nb0 + local_blocks(sv, visible_local(p, sv, w_last_row / G));
  }

  uint4 qf[CG][4];
  int lim[CG];  // last visible local-segment token of this lane's column
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
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

  float m[CG], l[CG];
  f32x4 o[CG][8];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    m[cg] = kNegInf;
    l[cg] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[cg][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // this wave's quarter of a block: K fragments 2w, 2w+1 and V fragments 2w, 2w+1
  uint4 rk0, rk1, rv0, rv1;
  auto load_share = [&](int blk) {
    const BlockRef r = block_ref(sv, blk);
    const int i = 2 * wave;
    rk0 = *reinterpret_cast<const uint4*>(r.k + (i * 16 + n16) * 32 + 8 * g4);
    rk1 = *reinterpret_cast<const uint4*>(r.k + ((i + 1) * 16 + n16) * 32 + 8 * g4);
    rv0 = *reinterpret_cast<const uint4*>(r.v + (16 * i + n16) * 32 + 8 * g4);
    rv1 = *reinterpret_cast<const uint4*>(r.v + (16 * (i + 1) + n16) * 32 + 8 * g4);
  };
  auto store_share = [&](int blk, int buf) {
    const int i = 2 * wave;
    lds[buf][i * 64 + lane] = rk0;
    lds[buf][(i + 1) * 64 + lane] = rk1;
    if (kVScale && blk < sv.nb0) {
      lds[buf][512 + i * 64 + lane] = v_to_f16<true>(rv0, vs);
      lds[buf][512 + (i + 1) * 64 + lane] = v_to_f16<true>(rv1, vs);
    } else {
      lds[buf][512 + i * 64 + lane] = v_to_f16<false>(rv0, 1.f);
      lds[buf][512 + (i + 1) * 64 + lane] = v_to_f16<false>(rv1, 1.f);
    }
  };

  if (nbt > 0) {
    load_share(0);
    store_share(0, 0);
  }
  __syncthreads();
  const float c = p.scale_log2;
  for (int blk = 0; blk < nbt; ++blk) {
    const int buf = blk & 1;
    const bool has_next = blk + 1 < nbt;
    if (has_next) load_share(blk + 1);
    if (blk < w_nbt) {
      const BlockRef r = block_ref(sv, blk);
      uint4 kf[8], vf[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) kf[i] = lds[buf][i * 64 + lane];
#pragma unroll
      for (int i = 0; i < 8; ++i) vf[i] = lds[buf][512 + i * 64 + lane];
      const bool edge = r.lo > 0 || r.hi < kBlockTokens;
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          s0 = mfma_bf16(kf[kb], qf[cg][kb], s0);
          s1 = mfma_bf16(kf[4 + kb], qf[cg][kb], s1);
        }
        float s[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[i] = s0[i];
          s[4 + i] = s1[i];
        }
        // token w = 8*g4 + j of the block; local tokens past the column's causal limit are hidden
        if (edge || (!r.older && r.seg_tok + kBlockTokens - 1 > lim[cg])) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int w = 8 * g4 + j;
            if (w < r.lo || w >= r.hi || (!r.older && r.seg_tok + w > lim[cg])) s[j] = kNegInf;
          }
        }
        float mx = s[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) mx = fmaxf(mx, s[j]);
        mx = wave_max_across_rows(mx) * c;
        const float m_new = fmaxf(m[cg], mx);
        float alpha = 1.f, pr[8];
        if (m_new == kNegInf) {
#pragma unroll
          for (int j = 0; j < 8; ++j) pr[j] = 0.f;
        } else {
          alpha = fast_exp2(m[cg] - m_new);
#pragma unroll
          for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(__builtin_fmaf(s[j], c, -m_new));
        }
        float rs = ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
        rs = wave_sum_across_rows(rs);
        l[cg] = l[cg] * alpha + rs;
        m[cg] = m_new;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float a = __shfl(alpha, 4 * g4 + i);
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) o[cg][nb][i] *= a;
          }
        }
        const uint4 ph = make_uint4(pack_f16_rne(pr[0], pr[1]), pack_f16_rne(pr[2], pr[3]),
                                    pack_f16_rne(pr[4], pr[5]), pack_f16_rne(pr[6], pr[7]));
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) o[cg][nb] = mfma_f16(ph, vf[nb], o[cg][nb]);
      }
    }
    if (has_next) store_share(blk + 1, buf ^ 1);
    __syncthreads();
  }

  // normalise and write: lane (n16 = dim in group nb, g4) holds rows 4*g4 + i of each column group
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const float linv = l[cg] > 0.f ? 1.f / l[cg] : 0.f;
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
            l[cg] > 0.f ? (m[cg] + __log2f(l[cg])) * kLn2 : kNegInf;
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
  const bool wide = rows > 4 * 16;
  const int64_t rows_per_wg = kWaves * 16 * (wide ? 4 : 1);
  const int64_t tiles = (rows + rows_per_wg - 1) / rows_per_wg;
  LKV_REQUIRE(tiles < (1LL << 31), "too many query rows");
  const dim3 grid(static_cast<unsigned>(tiles), a->num_kv_heads, a->batch);
  hipStream_t s = as_stream(stream);
  const bool vsc = a->older_vscale_mode == 1;
  if (wide) {
    if (vsc)
      prefill_kernel<4, true><<<grid, 256, 0, s>>>(p);
    else
      prefill_kernel<4, false><<<grid, 256, 0, s>>>(p);
  } else {
    if (vsc)
      prefill_kernel<1, true><<<grid, 256, 0, s>>>(p);
    else
      prefill_kernel<1, false><<<grid, 256, 0, s>>>(p);
  }
  return check_launch("lkv_prefill_attn");
}

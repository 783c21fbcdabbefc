// Split-K shared-KV decode attention for gfx950.
//
// One workgroup = 4 waves = one (sequence, kv head, key split).  Each wave streams 32-token
// blocks of the tiled K/V cache straight from HBM into registers with 16-byte loads (each load
// instruction of the wave covers one contiguous 1 KiB run), double-buffered so that the next
// block is in flight while the current one is computed:
//   S^T[32 tok x 16 col] = K_tile * Q^T   two 16x16x32 bf16 MFMAs per 32 dims, 8 per block;
//                                          columns are the (<=16) query heads of the GQA group
//   online softmax in the exp2 domain, row max / row sum over the four 16-lane rows (DPP)
//   O[16 x 128] += P * V                  P split into bf16 hi + lo parts, 16 MFMAs per block,
//                                          so P*V carries ~16 mantissa bits instead of 8
// The waves of a workgroup merge their (m, l, O) states through LDS.  With one split the
// workgroup writes the normalised bf16 output; otherwise it writes an unnormalised partial
// state and lkv_decode_combine merges the splits.
#include <algorithm>

#include "attn_common.h"
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr int kWaves = 4;
constexpr float kNegInf = -__builtin_inff();

struct DecodeParams {
  const uint16_t* q;
  int64_t q_sb;
  uint16_t* out;
  int64_t out_sb;
  float* lse;
  SegParams seg;
  const float* vscale;
  float* ws_o;
  float* ws_ml;
  int32_t hq, group, splits;
  float scale_log2;
};

struct BlockFrags {
  uint4 k[2][4];
  uint4 v[8];
};

template <bool kNT>
__device__ inline uint4 load_frag(const uint16_t* p) {
  return kNT ? load_nt(p) : *reinterpret_cast<const uint4*>(p);
}

// kNT: non-temporal loads (K/V read once and not again before they would be evicted anyway).
template <bool kNT>
__device__ inline void load_block(BlockFrags& f, const BlockRef& r, int n16, int g4) {
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      f.k[u][kb] = load_frag<kNT>(r.k + ((u * 4 + kb) * 16 + n16) * 32 + 8 * g4);
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) f.v[nb] = load_frag<kNT>(r.v + (16 * nb + n16) * 32 + 8 * g4);
}

struct SoftmaxState {
  float m, l;
  f32x4 o[8];  // O rows (heads 4*g4 + i) x dims 16*nb + n16
};

template <bool kVScale>
__device__ inline void compute_block(const BlockFrags& f, const BlockRef& r, const uint4 (&qf)[4], float vs,
                                     float scale_log2, int n16, int g4, SoftmaxState& st) {
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    s0 = mfma_bf16(f.k[0][kb], qf[kb], s0);
    s1 = mfma_bf16(f.k[1][kb], qf[kb], s1);
  }
  // lane (n16 = head column, g4) holds the scores of tokens 8*g4 + j, j = 0..7
  float s[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = s0[i] * scale_log2;
    s[4 + i] = s1[i] * scale_log2;
  }
  if (r.lo > 0 || r.hi < kBlockTokens) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (8 * g4 + j < r.lo || 8 * g4 + j >= r.hi) s[j] = kNegInf;
  }
  float mx = s[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) mx = fmaxf(mx, s[j]);
  mx = wave_max_across_rows(mx);
  const float m_new = fmaxf(st.m, mx);
  float alpha = 1.f;
  float p[8];
  if (m_new == kNegInf) {
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = 0.f;
  } else {
    alpha = fast_exp2(st.m - m_new);
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = fast_exp2(s[j] - m_new);
  }
  float rs = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  rs = wave_sum_across_rows(rs);
  st.l = st.l * alpha + rs;
  st.m = m_new;
  // rows of this lane's O accumulators are heads 4*g4 + i; their factors live in lanes 4*g4 + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = __shfl(alpha, 4 * g4 + i);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st.o[nb][i] *= a;
  }
  uint4 phi, plo;
  float hi[8];
  phi.x = pack_bf16x2(p[0], p[1]);
  phi.y = pack_bf16x2(p[2], p[3]);
  phi.z = pack_bf16x2(p[4], p[5]);
  phi.w = pack_bf16x2(p[6], p[7]);
  hi[0] = bf16_lo(phi.x);
  hi[1] = bf16_hi(phi.x);
  hi[2] = bf16_lo(phi.y);
  hi[3] = bf16_hi(phi.y);
  hi[4] = bf16_lo(phi.z);
  hi[5] = bf16_hi(phi.z);
  hi[6] = bf16_lo(phi.w);
  hi[7] = bf16_hi(phi.w);
  plo.x = pack_bf16x2(p[0] - hi[0], p[1] - hi[1]);
  plo.y = pack_bf16x2(p[2] - hi[2], p[3] - hi[3]);
  plo.z = pack_bf16x2(p[4] - hi[4], p[5] - hi[5]);
  plo.w = pack_bf16x2(p[6] - hi[6], p[7] - hi[7]);
  const bool scale_v = kVScale && r.older;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const uint4 v = scale_v ? scale_frag(f.v[nb], vs) : f.v[nb];
    st.o[nb] = mfma_bf16(phi, v, st.o[nb]);
    st.o[nb] = mfma_bf16(plo, v, st.o[nb]);
  }
}

template <bool kVScale, bool kNT>
__global__ __launch_bounds__(256) void decode_split_kernel(const DecodeParams p) {
  __shared__ float sm_m[kWaves][16];
  __shared__ float sm_l[kWaves][16];
  __shared__ float sm_o[kWaves][16][kHeadDim];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = p.group;

  const SeqView sv = make_seq_view(p.seg, b, kvh);
  const int nbt = sv.nb0 + (sv.n1 > 0 ? (sv.lead + sv.n1 + kBlockTokens - 1) / kBlockTokens : 0);
  const int bps = (nbt + p.splits - 1) / p.splits;
  const int blk_begin = split * bps;
  const int blk_end = min(blk_begin + bps, nbt);

  uint4 qf[4];
  {
    const uint16_t* qrow = p.q + b * p.q_sb + static_cast<int64_t>(kvh * G + n16) * kHeadDim;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qf[kb] = n16 < G ? *reinterpret_cast<const uint4*>(qrow + 32 * kb + 8 * g4) : make_uint4(0, 0, 0, 0);
  }
  const float vs = kVScale ? p.vscale[kvh] : 1.f;

  SoftmaxState st;
  st.m = kNegInf;
  st.l = 0.f;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) st.o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // this wave's blocks: blk_begin + wave + kWaves * t, t < nw; block t + 1 is loaded while block
  // t is computed.  The loop runs while two or more blocks remain, so its loads are unconditional
  // (the compiler then counts them exactly for s_waitcnt); the last one or two blocks follow it.
  const int first = blk_begin + wave;
  if (first < blk_end) {
    const int nw = (blk_end - 1 - first) / kWaves + 1;
    BlockFrags fa, fb;
    BlockRef ra = block_ref(sv, first);
    load_block<kNT>(fa, ra, n16, g4);
    int t = 0;
    // (the scheduling barriers keep the block being computed from moving above the next block's
    // loads, where reusing its registers would make the loads wait for it)
    for (; t + 2 < nw; t += 2) {
      const BlockRef rb = block_ref(sv, first + kWaves * (t + 1));
      load_block<kNT>(fb, rb, n16, g4);
      __builtin_amdgcn_sched_barrier(0);
      compute_block<kVScale>(fa, ra, qf, vs, p.scale_log2, n16, g4, st);
      ra = block_ref(sv, first + kWaves * (t + 2));
      load_block<kNT>(fa, ra, n16, g4);
      __builtin_amdgcn_sched_barrier(0);
      compute_block<kVScale>(fb, rb, qf, vs, p.scale_log2, n16, g4, st);
    }
    if (t + 1 < nw) {
      const BlockRef rb = block_ref(sv, first + kWaves * (t + 1));
      load_block<kNT>(fb, rb, n16, g4);
      compute_block<kVScale>(fa, ra, qf, vs, p.scale_log2, n16, g4, st);
      compute_block<kVScale>(fb, rb, qf, vs, p.scale_log2, n16, g4, st);
    } else {
      compute_block<kVScale>(fa, ra, qf, vs, p.scale_log2, n16, g4, st);
    }
  }

  // merge the four waves' states
  if (g4 == 0 && n16 < G) {
    sm_m[wave][n16] = st.m;
    sm_l[wave][n16] = st.l;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * g4 + i;
    if (h < G) {
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) sm_o[wave][h][16 * nb + n16] = st.o[nb][i];
    }
  }
  __syncthreads();
  const int bh0 = b * p.hq + kvh * G;
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += 256) {
    const int h = idx >> 7, d = idx & (kHeadDim - 1);
    float M = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = sm_m[w][h] == kNegInf ? 0.f : fast_exp2(sm_m[w][h] - M);
      L += f * sm_l[w][h];
      O += f * sm_o[w][h][d];
    }
    if (p.splits == 1) {
      p.out[b * p.out_sb + static_cast<int64_t>(kvh * G + h) * kHeadDim + d] = f32_to_bf16_bits(L > 0.f ? O / L : 0.f);
      if (p.lse != nullptr && d == 0) p.lse[bh0 + h] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
    } else {
      const int64_t row = static_cast<int64_t>(bh0 + h) * p.splits + split;
      p.ws_o[row * kHeadDim + d] = O;
      if (d == 0) {
        p.ws_ml[row * 2] = M;
        p.ws_ml[row * 2 + 1] = L;
      }
    }
  }
}

// Merges the per-split states of one (sequence, query head); one thread per head dim.  The splits'
// (m, l) pairs are staged in LDS and reduced in parallel (maximum, then the weights 2^(m_s - M)
// and L), so the per-dim accumulation over the splits has no dependent loads and keeps several
// partial-O loads in flight.
constexpr int kCombineThreads = kHeadDim;
constexpr int kMaxSplits = 1024;

__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const DecodeParams p) {
  __shared__ float sm_w[kMaxSplits];
  __shared__ float sm_red[kCombineThreads / 64];
  const int bh = blockIdx.x;
  const int d = threadIdx.x;
  const int b = bh / p.hq, h = bh % p.hq;
  const int S = p.splits;
  const float* ml = p.ws_ml + static_cast<int64_t>(bh) * S * 2;
  const float* o = p.ws_o + static_cast<int64_t>(bh) * S * kHeadDim;
  float mx = kNegInf;
  for (int s = d; s < S; s += kCombineThreads) {
    const float m = ml[2 * s];
    sm_w[s] = m;
    mx = fmaxf(mx, m);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((d & 63) == 0) sm_red[d >> 6] = mx;
  __syncthreads();
  const float M = fmaxf(sm_red[0], sm_red[1]);
  __syncthreads();
  float lsum = 0.f;
  for (int s = d; s < S; s += kCombineThreads) {
    const float m = sm_w[s];
    const float f = m == kNegInf ? 0.f : fast_exp2(m - M);
    sm_w[s] = f;
    lsum += f * ml[2 * s + 1];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off);
  if ((d & 63) == 0) sm_red[d >> 6] = lsum;
  __syncthreads();
  const float L = sm_red[0] + sm_red[1];
  float O[4] = {0.f, 0.f, 0.f, 0.f};
  int s = 0;
  for (; s + 4 <= S; s += 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) O[j] += sm_w[s + j] * o[(s + j) * kHeadDim + d];
  }
  for (; s < S; ++s) O[0] += sm_w[s] * o[s * kHeadDim + d];
  const float Ot = (O[0] + O[1]) + (O[2] + O[3]);
  p.out[b * p.out_sb + static_cast<int64_t>(h) * kHeadDim + d] = f32_to_bf16_bits(L > 0.f ? Ot / L : 0.f);
  if (p.lse != nullptr && d == 0) p.lse[bh] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
}

}  // namespace
}  // namespace lkv

extern "C" int64_t lkv_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || num_splits <= 1) return 0;
  return static_cast<int64_t>(batch) * num_q_heads * num_splits * (lkv::kHeadDim + 2) * 4;
}

extern "C" int32_t lkv_decode_attn(const lkv_decode_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_decode_args)),
              "lkv_decode_args size mismatch (caller %d, library %d)", a->struct_size,
              static_cast<int32_t>(sizeof(lkv_decode_args)));
  LKV_REQUIRE(a->head_dim == kHeadDim, "head_dim must be 128, got %d", a->head_dim);
  LKV_REQUIRE(a->batch >= 0 && a->num_kv_heads > 0 && a->num_q_heads > 0, "bad sizes");
  LKV_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  const int group = a->num_q_heads / a->num_kv_heads;
  LKV_REQUIRE(group <= 16, "GQA group %d exceeds 16", group);
  LKV_REQUIRE(a->num_splits >= 1 && a->num_splits <= 1024, "num_splits must be in [1, 1024]");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->older_vscale_mode == 1, "older_vscale_mode must be 0 or 1");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->vscale != nullptr, "older_vscale_mode 1 needs vscale");
  LKV_REQUIRE(a->kv_cache_hint >= 0 && a->kv_cache_hint <= 2, "kv_cache_hint must be 0, 1 or 2, got %d", a->kv_cache_hint);
  LKV_REQUIRE(a->q != nullptr && a->out != nullptr, "null q/out");
  LKV_REQUIRE((a->q_stride_b % 8) == 0 && (reinterpret_cast<uintptr_t>(a->q) & 15) == 0,
              "q rows must be 16-byte aligned");
  DecodeParams p;
  if (const int32_t st = fill_segments(a, p.seg)) return st;
  if (a->batch == 0) return LKV_OK;
  const int64_t need = lkv_decode_workspace_bytes(a->batch, a->num_q_heads, a->num_splits);
  if (need > 0) {
    if (a->workspace == nullptr || a->workspace_bytes < need)
      return fail(LKV_ERR_WORKSPACE, "decode workspace needs %lld bytes, got %lld", static_cast<long long>(need),
                  static_cast<long long>(a->workspace_bytes));
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 15) != 0)
      return fail(LKV_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_stride_b;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_sb = a->out_stride_b;
  p.lse = a->lse;
  p.vscale = a->vscale;
  p.ws_o = static_cast<float*>(a->workspace);
  p.ws_ml = need > 0 ? p.ws_o + static_cast<int64_t>(a->batch) * a->num_q_heads * a->num_splits * kHeadDim : nullptr;
  p.hq = a->num_q_heads;
  p.group = group;
  p.splits = a->num_splits;
  p.scale_log2 = a->sm_scale * kLog2e;
  const dim3 grid(a->num_splits, a->num_kv_heads, a->batch);
  hipStream_t s = as_stream(stream);
  // K/V bytes the call can read (lengths read from device memory bounded by the capacities)
  const int64_t ring_tokens = static_cast<int64_t>(a->local_ring_blocks) * kBlockTokens;
  const int64_t older_tokens =
      a->older_k == nullptr ? 0
                            : (a->older_len != nullptr ? a->older_capacity_tokens
                                                       : std::min(a->older_len_const, a->older_capacity_tokens));
  const int64_t local_tokens =
      a->local_k == nullptr ? 0
                            : (a->local_len != nullptr ? ring_tokens : std::min<int64_t>(a->local_len_const, ring_tokens));
  const int64_t kv_bytes = static_cast<int64_t>(a->batch) * a->num_kv_heads *
                           (std::max<int64_t>(older_tokens, 0) + std::max<int64_t>(local_tokens, 0)) * kHeadDim * 2 * 2;
  const bool nt = a->kv_cache_hint == 2 || (a->kv_cache_hint == 0 && kv_bytes > (int64_t{384} << 20));
  if (a->older_vscale_mode == 1 && nt)
    decode_split_kernel<true, true><<<grid, 256, 0, s>>>(p);
  else if (a->older_vscale_mode == 1)
    decode_split_kernel<true, false><<<grid, 256, 0, s>>>(p);
  else if (nt)
    decode_split_kernel<false, true><<<grid, 256, 0, s>>>(p);
  else
    decode_split_kernel<false, false><<<grid, 256, 0, s>>>(p);
  if (int32_t st = check_launch("lkv_decode_attn split kernel")) return st;
  if (a->num_splits > 1) {
    decode_combine_kernel<<<a->batch * a->num_q_heads, kCombineThreads, 0, s>>>(p);
    return check_launch("lkv_decode_attn combine kernel");
  }
  return LKV_OK;
}

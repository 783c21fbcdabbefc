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
#include <atomic>

#include "attn_common.h"
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr int kWaves = 4;
constexpr float kNegInf = -__builtin_inff();
constexpr float kLazyRaise = 8.f;  // exp2 units a block maximum may exceed m before m is raised

struct DecodeParams {
  const uint16_t* q;
  int64_t q_sb, q_st;
  uint16_t* out;
  int64_t out_sb, out_st;
  float* lse;
  SegParams seg;
  const float* vscale;
  const float* out_scale;  // [Hkv] or nullptr: out = bf16(bf16(o) * out_scale[kvh])
  float* ws_o;
  float* ws_ml;
  int32_t batch, hq, group, splits;
  int32_t L, causal;  // query tokens per sequence (1 for decode calls) and bottom-right causality
  float scale_log2;
  // ragged query rows (short-prefill calls): sequence b's tokens are rows cu[b] .. cu[b + 1] - 1 of
  // q / out (nullptr: L tokens per sequence); rows = the call's total row count.  Only sequences
  // with col_lo < tokens * group <= col_hi run in this launch.  Their split count is `splits` when
  // dyn_splits is 0, else chosen per launch on the device from the number n of sequences in the
  // class, min(splits, max(1, floor(cus / (n * Hkv)))); their split states are laid out by the sequence's
  // rank in the class, lmax token rows each.
  const int32_t* cu;
  int32_t rows, col_lo, col_hi;
  int32_t dyn_splits, cus, lmax;
};

// Query tokens of sequence b (kMulti calls) and the flattened row of its token 0 (the q / out / lse
// / split-state row index is row0 + token).
struct MultiRows {
  int L;
  int64_t row0;
};

__device__ inline MultiRows multi_rows(const DecodeParams& p, int b) {
  if (p.cu == nullptr) return MultiRows{p.L, static_cast<int64_t>(b) * p.L};
  const int s0 = min(max(p.cu[b], 0), p.rows);
  return MultiRows{min(min(max(p.cu[b + 1], s0), p.rows) - s0, p.L), s0};
}

__device__ inline bool in_column_class(const DecodeParams& p, int L) {
  const int cols = L * p.group;
  return L > 0 && cols > p.col_lo && cols <= p.col_hi;
}

// Ragged calls: the number of sequences in this launch's column class and b's rank among them (every
// wave counts them itself, 64 sequences per ballot), and the class's split count.
struct ClassRank {
  int n, rank, splits;
};

__device__ inline ClassRank class_rank(const DecodeParams& p, int b, int hkv) {
  const int lane = threadIdx.x & 63;
  int n = 0, rank = 0;
  for (int i0 = 0; i0 < p.batch; i0 += 64) {
    const int i = i0 + lane;
    const bool in = i < p.batch && in_column_class(p, multi_rows(p, i).L);
    const uint64_t m = __builtin_amdgcn_ballot_w64(in);
    n += __builtin_popcountll(m);
    if (b >= i0) rank += __builtin_popcountll(b - i0 >= 64 ? m : (m & ((uint64_t{1} << (b - i0)) - 1)));
  }
  int splits = p.splits;
  if (p.dyn_splits && n > 0) splits = min(p.splits, max(1, p.cus / (n * hkv)));
  return ClassRank{n, rank, splits};
}

// Ragged calls with the split count chosen on the device run on a compact grid: workgroup
// (kv head fastest) u-th (sequence, split) pair of the class, sequences in order, each with the
// class's split count S.  Returns false past the class's n * S pairs.
struct ClassPick {
  int b, rank, split, splits;
};

__device__ inline bool class_pick(const DecodeParams& p, int u, int hkv, ClassPick& r) {
  const int lane = threadIdx.x & 63;
  int n = 0;
  for (int i0 = 0; i0 < p.batch; i0 += 64) {
    const int i = i0 + lane;
    n += __builtin_popcountll(__builtin_amdgcn_ballot_w64(i < p.batch && in_column_class(p, multi_rows(p, i).L)));
  }
  if (n == 0) return false;
  r.splits = min(p.splits, max(1, p.cus / (n * hkv)));
  r.rank = u / r.splits;
  r.split = u - r.rank * r.splits;
  if (r.rank >= n) return false;
  int base = 0;  // class sequences before this step's 64
  for (int i0 = 0; i0 < p.batch; i0 += 64) {
    const int i = i0 + lane;
    const bool in = i < p.batch && in_column_class(p, multi_rows(p, i).L);
    const uint64_t m = __builtin_amdgcn_ballot_w64(in);
    const int c = __builtin_popcountll(m);
    if (r.rank < base + c) {  // the (rank - base)-th class sequence of these 64
      const int below = __builtin_popcountll(m & ((uint64_t{1} << lane) - 1));
      r.b = i0 + __builtin_ctzll(__builtin_amdgcn_ballot_w64(in && below == r.rank - base));
      return true;
    }
    base += c;
  }
  return false;
}

// The bf16 output of a normalised fp32 value x of kv head kvh: bf16(x), or bf16(bf16(x) * s) with
// an output scale (the reference rescales its bf16 attention output by s in fp32).
__device__ inline uint16_t out_bits(float x, const float* out_scale, int kvh) {
  if (out_scale == nullptr) return f32_to_bf16_bits(x);
  return f32_to_bf16_bits(bf16_bits_to_f32(f32_to_bf16_bits(x)) * out_scale[kvh]);
}

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

// kMulti: the columns are (query token, head) pairs; lim is this lane's column's last visible local
// token and lim_min the smallest over the columns (local blocks past it need the causal mask).
template <bool kVScale, bool kMulti>
__device__ inline void compute_block(const BlockFrags& f, const BlockRef& r, const uint4 (&qf)[4], float vs,
                                     float scale_log2, int n16, int g4, int lim, int lim_min, SoftmaxState& st) {
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
  if (r.lo > 0 || r.hi < kBlockTokens || (kMulti && !r.older && r.seg_tok + kBlockTokens - 1 > lim_min)) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (8 * g4 + j < r.lo || 8 * g4 + j >= r.hi || (kMulti && !r.older && r.seg_tok + 8 * g4 + j > lim)) s[j] = kNegInf;
  }
  float mx = s[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) mx = fmaxf(mx, s[j]);
  mx = wave_max_across_rows(mx);
  // Lazy reference: a column's m moves (and O and l are rescaled) only in a wave-uniform branch
  // taken when some column's block maximum exceeds its m by more than kLazyRaise (exp2 units), the
  // first block with a visible key included (m = -inf).  Otherwise P = 2^(s - m) stays below
  // 2^kLazyRaise; its bf16 hi + lo split keeps ~16 bits at any magnitude and O, l are fp32.
  float alpha = 1.f;
  if (__builtin_amdgcn_ballot_w64(mx > st.m + kLazyRaise)) {
    const float m_new = fmaxf(st.m, mx);
    alpha = m_new == kNegInf ? 1.f : fast_exp2(st.m - m_new);
    st.m = m_new;
    // rows of this lane's O accumulators are heads 4*g4 + i; their factors live in lanes 4*g4 + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __shfl(alpha, 4 * g4 + i);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) st.o[nb][i] *= a;
    }
  }
  float p[8];
  if (st.m == kNegInf) {
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = 0.f;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = fast_exp2(s[j] - st.m);
  }
  float rs = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  rs = wave_sum_across_rows(rs);
  st.l = st.l * alpha + rs;
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

// kMulti: L > 1 query tokens per sequence, column c = (token c / G, head c % G) for c < G * L <=
// 16 * CG (CG <= 2 per wave: four groups spill), in CG groups of 16 columns that share each block's K/V fragments (short prefill calls);
// otherwise column c = head c (L = 1, CG = 1).
// kPairs (with kMulti): 32 * CG columns; waves 0-1 take column groups [0, CG), waves 2-3 groups
// [CG, 2 CG), and each pair walks all of the split's blocks (every block is fetched by both pairs,
// the second time normally from L2), so no wave holds more than CG groups of state.
template <bool kVScale, bool kNT, bool kMulti, int CG = 1, bool kPairs = false>
__global__ __launch_bounds__(256) void decode_split_kernel(const DecodeParams p) {
  constexpr int kWaveCols = 16 * CG;  // columns one wave holds (a pair's share with kPairs)
  constexpr int kStride = kPairs ? 2 : kWaves;  // block stride of one wave
  // indexed by the column inside the wave's own range: with kPairs each wave pair stages only its
  // half of the columns, so the staging takes 64 KiB at most and two workgroups fit on a CU
  __shared__ float sm_m[kWaves][kWaveCols];
  __shared__ float sm_l[kWaves][kWaveCols];
  __shared__ float sm_o[kWaves][kWaveCols][kHeadDim];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;
  const int G = p.group;
  int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  int S = p.splits;
  int64_t ws_row0 = 0;  // ragged calls: split-state row of the sequence's token 0 (its rank in the class)
  if (kMulti && p.dyn_splits) {
    // the class's (sequence, split) pairs on a compact 1-D grid (the split count, chosen from the
    // number of sequences in the class, is not known to the host; a grid of every sequence at the
    // largest count would mostly exit, and with the split as its fastest dimension the exiting
    // workgroups were whole XCDs: 2 splits left 6 of 8 idle)
    const int hkv = p.hq / G;
    kvh = static_cast<int>(blockIdx.x) % hkv;
    ClassPick cp;
    if (!class_pick(p, static_cast<int>(blockIdx.x) / hkv, hkv, cp)) return;  // (workgroup-uniform)
    b = cp.b;
    split = cp.split;
    S = cp.splits;
    ws_row0 = static_cast<int64_t>(cp.rank) * p.lmax;
  }

  // ragged calls: this sequence's query tokens (workgroup-uniform; sequences of another column
  // class run in another launch)
  const MultiRows mr = kMulti ? multi_rows(p, b) : MultiRows{1, b};
  if (kMulti && !in_column_class(p, mr.L)) return;
  const int Lq = mr.L;
  if (!(kMulti && p.cu != nullptr)) {
    ws_row0 = mr.row0;
  } else if (!p.dyn_splits) {  // a fixed split count over a (splits, Hkv, B) grid
    ws_row0 = static_cast<int64_t>(class_rank(p, b, gridDim.y).rank) * p.lmax;
  }

  const SeqView sv = make_seq_view(p.seg, b, kvh);
  const int nbt = sv.nb0 + (sv.n1 > 0 ? (sv.lead + sv.n1 + kBlockTokens - 1) / kBlockTokens : 0);
  const int bps = (nbt + S - 1) / S;
  const int blk_begin = split * bps;
  const int blk_end = min(blk_begin + bps, nbt);

  const int cols = kMulti ? G * Lq : G;
  uint4 qf[CG][4];
  int lim[CG], lim_min = 0;  // causal limits (local token index) of this lane's columns and of column 0
  if (kMulti) lim_min = p.causal ? sv.n1 - Lq : sv.n1 - 1;
  const int cg0 = kPairs ? (wave >> 1) * CG : 0;  // this wave's first column group
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int c = 16 * (cg0 + cg) + n16;
    const int t = kMulti ? c / G : 0, h = c - t * G;
    const uint16_t* qrow = p.q + (kMulti && p.cu ? mr.row0 * p.q_st : b * p.q_sb) + (kMulti ? t * p.q_st : 0) +
                           static_cast<int64_t>(kvh * G + h) * kHeadDim;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qf[cg][kb] = c < cols ? *reinterpret_cast<const uint4*>(qrow + 32 * kb + 8 * g4) : make_uint4(0, 0, 0, 0);
    lim[cg] = kMulti && p.causal ? lim_min + t : lim_min;
  }
  const float vs = kVScale ? p.vscale[kvh] : 1.f;

  SoftmaxState st[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    st[cg].m = kNegInf;
    st[cg].l = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st[cg].o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto compute = [&](const BlockFrags& f, const BlockRef& r) __attribute__((always_inline)) {
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
      compute_block<kVScale, kMulti>(f, r, qf[cg], vs, p.scale_log2, n16, g4, lim[cg], lim_min, st[cg]);
  };

  // this wave's blocks: blk_begin + wave + kWaves * t, t < nw; block t + 1 is loaded while block
  // t is computed.  The loop runs while two or more blocks remain, so its loads are unconditional
  // (the compiler then counts them exactly for s_waitcnt); the last one or two blocks follow it.
  const int first = blk_begin + (kPairs ? (wave & 1) : wave);
  if (first < blk_end) {
    int nw = (blk_end - 1 - first) / kStride + 1;
    // A wave with one block more than the workgroup's last wave (the split's block count is not a
    // multiple of the waves) fetches that last block together with its first one and computes it
    // after the loop, so its extra block adds compute but no round trip to memory: the loop, whose
    // iterations are bound by load latency, then runs as many iterations in every wave.
    const int last_first = blk_begin + (kPairs ? 1 : kWaves - 1);
    const int nw_last = last_first < blk_end ? (blk_end - 1 - last_first) / kStride + 1 : 0;
    const bool fold = nw > nw_last && nw >= 2;
    BlockFrags fa, fb, fc;
    BlockRef ra = block_ref(sv, first), rc{};
    load_block<kNT>(fa, ra, n16, g4);
    if (fold) {
      rc = block_ref(sv, first + kStride * (nw - 1));
      load_block<kNT>(fc, rc, n16, g4);
      --nw;
    }
    int t = 0;
    // (the scheduling barriers keep the block being computed from moving above the next block's
    // loads, where reusing its registers would make the loads wait for it)
    for (; t + 2 < nw; t += 2) {
      const BlockRef rb = block_ref(sv, first + kStride * (t + 1));
      load_block<kNT>(fb, rb, n16, g4);
      __builtin_amdgcn_sched_barrier(0);
      compute(fa, ra);
      ra = block_ref(sv, first + kStride * (t + 2));
      load_block<kNT>(fa, ra, n16, g4);
      __builtin_amdgcn_sched_barrier(0);
      compute(fb, rb);
    }
    if (t + 1 < nw) {
      const BlockRef rb = block_ref(sv, first + kStride * (t + 1));
      load_block<kNT>(fb, rb, n16, g4);
      compute(fa, ra);
      compute(fb, rb);
    } else {
      compute(fa, ra);
    }
    if (fold) compute(fc, rc);
  }

  // merge the four waves' states
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    if (g4 == 0 && 16 * (cg0 + cg) + n16 < cols) {
      sm_m[wave][16 * cg + n16] = st[cg].m;
      sm_l[wave][16 * cg + n16] = st[cg].l;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hl = 16 * cg + 4 * g4 + i;  // column 16 * cg0 + hl
      if (16 * cg0 + hl < cols) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) sm_o[wave][hl][16 * nb + n16] = st[cg].o[nb][i];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < cols * kHeadDim; idx += 256) {
    const int h = idx >> 7, d = idx & (kHeadDim - 1);  // column h = (token tq, head hh)
    const int tq = kMulti ? h / G : 0, hh = h - tq * G;
    const int64_t row_q = (mr.row0 + tq) * p.hq + kvh * G + hh;  // [rows, Hq] row
    // the waves that hold column h: all four, or the pair of its column group
    const int pair = kPairs ? h / kWaveCols : 0;
    const int w0 = 2 * pair, hl = h - pair * kWaveCols;  // its waves and its column inside their range
    constexpr int kMergeWaves = kPairs ? 2 : kWaves;
    float M = sm_m[w0][hl];
#pragma unroll
    for (int w = w0 + 1; w < w0 + kMergeWaves; ++w) M = fmaxf(M, sm_m[w][hl]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = w0; w < w0 + kMergeWaves; ++w) {
      const float f = sm_m[w][hl] == kNegInf ? 0.f : fast_exp2(sm_m[w][hl] - M);
      L += f * sm_l[w][hl];
      O += f * sm_o[w][hl][d];
    }
    if (S == 1) {
      p.out[(kMulti && p.cu ? mr.row0 * p.out_st : b * p.out_sb) + (kMulti ? tq * p.out_st : 0) +
            static_cast<int64_t>(kvh * G + hh) * kHeadDim + d] =
          out_bits(L > 0.f ? O / L : 0.f, p.out_scale, kvh);
      if (p.lse != nullptr && d == 0) p.lse[row_q] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
    } else {
      const int64_t row = ((ws_row0 + tq) * p.hq + kvh * G + hh) * S + split;
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

// Merges the S split states (ml: (m, l) pairs, o: partial O rows) of one (query token, head) into
// its output row and optional LSE; every thread of the block calls it (one per head dim).
__device__ inline void combine_row(const DecodeParams& p, const float* ml, const float* o, int S, uint16_t* out_row,
                                   float* lse, int kvh, float* sm_w, float* sm_red) {
  const int d = threadIdx.x;
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
  out_row[d] = out_bits(L > 0.f ? Ot / L : 0.f, p.out_scale, kvh);
  if (lse != nullptr && d == 0) *lse = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
  __syncthreads();  // (sm_w and sm_red are reused by the caller's next row)
}

// Uniform calls: one block per [B, L, Hq] row.  Ragged calls: one block per (head, sequence, query
// token) of the launch's column class (its split count and split-state rows come from the
// sequence's rank in the class, as in the split kernel; with one split that kernel wrote the output).
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const DecodeParams p) {
  __shared__ float sm_w[kMaxSplits];
  __shared__ float sm_red[kCombineThreads / 64];
  if (p.cu != nullptr) {
    const int h = blockIdx.x, b = blockIdx.y, tq = blockIdx.z;
    const MultiRows mr = multi_rows(p, b);
    if (!in_column_class(p, mr.L) || tq >= mr.L) return;  // (uniform over the block)
    const ClassRank cr = class_rank(p, b, p.hq / p.group);
    const int S = cr.splits;
    if (S == 1) return;
    const int64_t ws_row = (static_cast<int64_t>(cr.rank) * p.lmax + tq) * p.hq + h;
    const int64_t out_row = mr.row0 + tq;
    combine_row(p, p.ws_ml + ws_row * S * 2, p.ws_o + ws_row * S * kHeadDim, S,
                p.out + out_row * p.out_st + static_cast<int64_t>(h) * kHeadDim,
                p.lse != nullptr ? p.lse + out_row * p.hq + h : nullptr, h / p.group, sm_w, sm_red);
    return;
  }
  const int bh = blockIdx.x;  // [B, L, Hq] row
  const int row = bh / p.hq, h = bh % p.hq;
  const int b = row / p.L, tq = row % p.L;
  const int S = p.splits;
  combine_row(p, p.ws_ml + static_cast<int64_t>(bh) * S * 2, p.ws_o + static_cast<int64_t>(bh) * S * kHeadDim, S,
              p.out + b * p.out_sb + tq * p.out_st + static_cast<int64_t>(h) * kHeadDim,
              p.lse != nullptr ? p.lse + bh : nullptr, h / p.group, sm_w, sm_red);
}

// Key tokens a call can read per sequence (lengths read from device memory bounded by the
// capacities); Args is lkv_decode_args or lkv_prefill_args (same segment fields).
template <typename Args>
int64_t call_key_tokens(const Args* a) {
  const int64_t ring_tokens = static_cast<int64_t>(a->local_ring_blocks) * kBlockTokens;
  const int64_t older = a->older_k == nullptr ? 0
                                              : (a->older_len != nullptr ? a->older_capacity_tokens
                                                                         : std::min(a->older_len_const, a->older_capacity_tokens));
  const int64_t local = a->local_k == nullptr
                            ? 0
                            : (a->local_len != nullptr ? ring_tokens : std::min<int64_t>(a->local_len_const, ring_tokens));
  return std::max<int64_t>(older, 0) + std::max<int64_t>(local, 0);
}

// Non-temporal K/V loads when a call's K/V exceed 384 MiB (more than the 256 MB last-level cache
// could keep for the next layer's call over the same shared cache); hint 1 / 2 force a policy.
bool use_nontemporal(int32_t hint, int64_t kv_bytes) { return hint == 2 || (hint == 0 && kv_bytes > (int64_t{384} << 20)); }

template <int CG, bool kPairs = false>
void launch_multi(const DecodeParams& p, dim3 grid, bool vscale, bool nt, hipStream_t s) {
  if (vscale && nt)
    decode_split_kernel<true, true, true, CG, kPairs><<<grid, 256, 0, s>>>(p);
  else if (vscale)
    decode_split_kernel<true, false, true, CG, kPairs><<<grid, 256, 0, s>>>(p);
  else if (nt)
    decode_split_kernel<false, true, true, CG, kPairs><<<grid, 256, 0, s>>>(p);
  else
    decode_split_kernel<false, false, true, CG, kPairs><<<grid, 256, 0, s>>>(p);
}

// cg: 0 for decode calls (one column per head), else the 16-column groups of a short prefill call
int32_t launch_decode(const DecodeParams& p, dim3 grid, bool vscale, bool nt, int cg, int rows, hipStream_t s,
                      const char* what) {
  if (cg == 1) {
    launch_multi<1>(p, grid, vscale, nt, s);
  } else if (cg == 2) {
    launch_multi<2>(p, grid, vscale, nt, s);
  } else if (cg == 4) {  // two wave pairs of two groups each
    launch_multi<2, true>(p, grid, vscale, nt, s);
  } else {
    if (vscale && nt)
      decode_split_kernel<true, true, false><<<grid, 256, 0, s>>>(p);
    else if (vscale)
      decode_split_kernel<true, false, false><<<grid, 256, 0, s>>>(p);
    else if (nt)
      decode_split_kernel<false, true, false><<<grid, 256, 0, s>>>(p);
    else
      decode_split_kernel<false, false, false><<<grid, 256, 0, s>>>(p);
  }
  if (const int32_t st = check_launch(what)) return st;
  if (p.splits > 1) {
    const dim3 grid = p.cu != nullptr ? dim3(p.hq, p.batch, p.lmax) : dim3(rows);
    decode_combine_kernel<<<grid, kCombineThreads, 0, s>>>(p);
    return check_launch(what);
  }
  return LKV_OK;
}

}  // namespace

int64_t ragged_split_state_rows(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t lmax, int32_t cap,
                                int32_t fixed, int32_t cus) {
  int64_t worst = 0;
  for (int64_t n = 1; n <= batch; ++n) {
    const int64_t S = fixed > 0 ? fixed : std::min<int64_t>(cap, std::max<int64_t>(1, cus / (n * num_kv_heads)));
    if (S > 1) worst = std::max(worst, n * lmax * num_q_heads * S);
  }
  return worst;
}

int32_t prefill_on_decode_kernel(const lkv_prefill_args* a, const SegParams& seg, int32_t group, int32_t col_lo,
                                 int32_t col_hi, int32_t class_n, hipStream_t s) {
  DecodeParams p;
  p.seg = seg;
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_stride_b;
  p.q_st = a->q_stride_t;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_sb = a->out_stride_b;
  p.out_st = a->out_stride_t;
  p.lse = a->lse;
  p.vscale = a->vscale;
  p.out_scale = a->out_scale;
  p.batch = a->batch;
  p.hq = a->num_q_heads;
  p.group = group;
  p.cu = a->cu_seqlens_q;
  p.rows = a->tokens;
  p.L = a->cu_seqlens_q ? std::min(a->max_seqlen_q, a->tokens) : a->tokens;
  p.col_lo = col_lo;
  p.col_hi = col_hi;
  p.causal = a->causal;
  p.scale_log2 = a->sm_scale * kLog2e;
  const bool ragged = p.cu != nullptr;
  // a ragged call's sequences of this class have at most lmax query tokens
  p.lmax = ragged ? std::min(col_hi / group, p.L) : p.L;
  if (p.lmax < 1) return LKV_OK;  // (no sequence fits the class)
  const int64_t tokens = call_key_tokens(a);
  const int64_t blocks = (tokens + 2 * kBlockTokens - 1) / kBlockTokens;  // (+1 for a ring start inside a block)
  const int64_t pairs = static_cast<int64_t>(a->batch) * a->num_kv_heads;
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  p.cus = static_cast<int32_t>(cus);
  // as many splits as fit one round of workgroups (one per CU), at least 4 blocks per split, partial
  // states within the workspace; a ragged call's launch caps the count at what one sequence alone
  // would take (and kRaggedSplitCap) and each launch divides the CUs among the sequences it finds in
  // its class
  int64_t splits = std::min<int64_t>({ragged ? std::min<int64_t>(std::max<int64_t>(1, cus / a->num_kv_heads), kRaggedSplitCap)
                                             : std::max<int64_t>(1, cus / pairs),
                                      std::max<int64_t>(blocks / 4, 1), 1024});
  // split-state rows x splits: [B, L, Hq] rows for uniform calls, the class's sequences by rank
  // (lmax rows each) for ragged ones
  auto state = [&](int64_t cap, int32_t fixed) -> int64_t {
    if (ragged) return ragged_split_state_rows(a->batch, a->num_q_heads, a->num_kv_heads, p.lmax, cap, fixed, p.cus);
    const int64_t S = fixed > 0 ? fixed : cap;
    return S > 1 ? static_cast<int64_t>(a->batch) * a->tokens * a->num_q_heads * S : 0;
  };
  if (a->num_splits > 0) {  // fixed by the caller (lkv_prefill_workspace_bytes counted its states)
    splits = a->num_splits;
    const int64_t need = state(splits, a->num_splits) * (kHeadDim + 2) * 4;
    if (need > a->workspace_bytes)
      return fail(LKV_ERR_WORKSPACE, "prefill with %d decode splits needs %lld bytes of workspace, got %lld", a->num_splits,
                  static_cast<long long>(need), static_cast<long long>(a->workspace_bytes));
  }
  while (splits > 1 && state(splits, a->num_splits > 0 ? static_cast<int32_t>(splits) : 0) * (kHeadDim + 2) * 4 >
                           a->workspace_bytes)
    splits = (splits + 1) / 2;
  p.splits = static_cast<int32_t>(splits);
  p.dyn_splits = ragged && a->num_splits == 0;
  const int64_t state_rows = state(splits, a->num_splits > 0 ? static_cast<int32_t>(splits) : 0);
  p.ws_o = state_rows > 0 ? static_cast<float*>(a->workspace) : nullptr;
  p.ws_ml = state_rows > 0 ? p.ws_o + state_rows * kHeadDim : nullptr;
  // the class's split count when the host knows how many sequences it holds: the count the split
  // kernel derives from them (so one split launches no merge); a cap the kernel cannot exceed
  if (p.dyn_splits && class_n > 0)
    p.splits = static_cast<int32_t>(std::min<int64_t>(p.splits, std::max<int64_t>(1, cus / (int64_t{class_n} * a->num_kv_heads))));
  const bool nt = use_nontemporal(0, pairs * tokens * kHeadDim * 2 * 2);
  // the instance holds the class's widest sequence: 16, 32 or 64 columns
  const int64_t cols = std::min<int64_t>(col_hi, static_cast<int64_t>(group) * p.L);
  const int cg = cols <= 16 ? 1 : cols <= 32 ? 2 : 4;
  // combine grid: one block per output row ([rows, Hq] ragged, [B, L, Hq] uniform)
  const int64_t out_rows = (ragged ? static_cast<int64_t>(a->tokens) : static_cast<int64_t>(a->batch) * a->tokens) *
                           a->num_q_heads;
  // split counts chosen on the device: n sequences x S(n) splits <= ceil(CUs / Hkv) + B pairs per kv head
  const dim3 grid = p.dyn_splits
                        ? dim3(static_cast<unsigned>(a->num_kv_heads * ((cus + a->num_kv_heads - 1) / a->num_kv_heads + a->batch)))
                        : dim3(p.splits, a->num_kv_heads, a->batch);
  return launch_decode(p, grid, a->older_vscale_mode == 1, nt, cg, static_cast<int>(out_rows), s,
                       "lkv_prefill_attn (short call on the decode kernel)");
}

}  // namespace lkv

extern "C" int64_t lkv_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || num_splits <= 1) return 0;
  return static_cast<int64_t>(batch) * num_q_heads * num_splits * (lkv::kHeadDim + 2) * 4;
}

namespace lkv {
namespace {

// Argument checks of lkv_decode_attn and lkv_decode_attn_noalloc (no device calls).
int32_t check_decode_args(const lkv_decode_args* a) {
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_decode_args)),
              "lkv_decode_args size mismatch (caller %d, library %d)", a->struct_size,
              static_cast<int32_t>(sizeof(lkv_decode_args)));
  LKV_REQUIRE(a->head_dim == kHeadDim, "head_dim must be 128, got %d", a->head_dim);
  LKV_REQUIRE(a->batch >= 0 && a->num_kv_heads > 0 && a->num_q_heads > 0, "bad sizes");
  LKV_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  LKV_REQUIRE(a->num_q_heads / a->num_kv_heads <= 64, "GQA group %d exceeds 64", a->num_q_heads / a->num_kv_heads);
  LKV_REQUIRE(a->num_splits >= 1 && a->num_splits <= 1024, "num_splits must be in [1, 1024]");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->older_vscale_mode == 1, "older_vscale_mode must be 0 or 1");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->vscale != nullptr, "older_vscale_mode 1 needs vscale");
  LKV_REQUIRE(a->kv_cache_hint >= 0 && a->kv_cache_hint <= 2, "kv_cache_hint must be 0, 1 or 2, got %d", a->kv_cache_hint);
  LKV_REQUIRE(a->q != nullptr && a->out != nullptr, "null q/out");
  LKV_REQUIRE((a->q_stride_b % 8) == 0 && (reinterpret_cast<uintptr_t>(a->q) & 15) == 0,
              "q rows must be 16-byte aligned");
  return LKV_OK;
}

// The decode call of checked args with the split partials in `ws` (ws_bytes bytes).
int32_t run_decode(const lkv_decode_args* a, void* ws, int64_t ws_bytes, hipStream_t stream) {
  DecodeParams p;
  if (const int32_t st = fill_segments(a, p.seg)) return st;
  if (a->batch == 0) return LKV_OK;
  const int group = a->num_q_heads / a->num_kv_heads;
  const int64_t need = lkv_decode_workspace_bytes(a->batch, a->num_q_heads, a->num_splits);
  if (need > 0) {
    if (ws == nullptr || ws_bytes < need)
      return fail(LKV_ERR_WORKSPACE, "decode workspace needs %lld bytes, got %lld", static_cast<long long>(need),
                  static_cast<long long>(ws_bytes));
    if ((reinterpret_cast<uintptr_t>(ws) & 15) != 0) return fail(LKV_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_stride_b;
  p.q_st = 0;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_sb = a->out_stride_b;
  p.out_st = 0;
  p.L = 1;
  p.causal = 0;
  p.cu = nullptr;
  p.rows = a->batch;
  p.col_lo = 0;
  p.col_hi = 1 << 30;
  p.dyn_splits = 0;
  p.cus = 0;
  p.lmax = 1;
  p.batch = a->batch;
  p.lse = a->lse;
  p.vscale = a->vscale;
  p.out_scale = a->out_scale;
  p.ws_o = static_cast<float*>(ws);
  p.ws_ml = need > 0 ? p.ws_o + static_cast<int64_t>(a->batch) * a->num_q_heads * a->num_splits * kHeadDim : nullptr;
  p.hq = a->num_q_heads;
  p.group = group;
  p.splits = a->num_splits;
  p.scale_log2 = a->sm_scale * kLog2e;
  const int64_t kv_bytes = static_cast<int64_t>(a->batch) * a->num_kv_heads * call_key_tokens(a) * kHeadDim * 2 * 2;
  // groups above 16 query heads per kv head take the multi-column instances (columns = heads)
  const int cg = group <= 16 ? 0 : group <= 32 ? 2 : 4;
  return launch_decode(p, dim3(a->num_splits, a->num_kv_heads, a->batch), a->older_vscale_mode == 1,
                       use_nontemporal(a->kv_cache_hint, kv_bytes), cg, a->batch * a->num_q_heads, stream,
                       "lkv_decode_attn");
}

// Scratch of the allocation-free entry point: the split partials of one call, in a static device
// array that each GPU holds for the life of the process.  Host code must not use the array's name
// as a device address (it is a host-side stand-in): the address on a device comes from
// hipGetSymbolAddress, taken once per device with that device current and kept here.
constexpr int64_t kNoAllocScratchBytes = LKV_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];

// Device address of the current device's scratch.
int32_t current_device_scratch(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(LKV_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxScratchDevices) return fail(LKV_ERR_UNSUPPORTED, "device %d beyond the scratch table", dev);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(LKV_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(err));
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return LKV_OK;
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_decode_attn(const lkv_decode_args* a, lkv_stream_t stream) {
  using namespace lkv;
  if (const int32_t st = check_decode_args(a)) return st;
  return run_decode(a, a->workspace, a->workspace_bytes, as_stream(stream));
}

extern "C" int32_t lkv_decode_attn_noalloc(const lkv_decode_args* a, lkv_stream_t stream) {
  using namespace lkv;
  if (const int32_t st = check_decode_args(a)) return st;
  LKV_REQUIRE(a->workspace == nullptr && a->workspace_bytes == 0,
              "lkv_decode_attn_noalloc uses the library's static scratch: workspace must be NULL and workspace_bytes 0");
  const int64_t need = lkv_decode_workspace_bytes(a->batch, a->num_q_heads, a->num_splits);
  LKV_REQUIRE(need <= kNoAllocScratchBytes,
              "%d splits of %d x %d query heads need %lld bytes of split state, more than the %lld bytes of static "
              "scratch: use fewer splits, or lkv_decode_attn with a workspace",
              a->num_splits, a->batch, a->num_q_heads, static_cast<long long>(need),
              static_cast<long long>(kNoAllocScratchBytes));
  void* ws = nullptr;
  if (need > 0 && a->batch > 0) {
    if (const int32_t st = current_device_scratch(&ws)) return st;
  }
  return run_decode(a, ws, kNoAllocScratchBytes, as_stream(stream));
}

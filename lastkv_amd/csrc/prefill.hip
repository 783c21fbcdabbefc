// Chunked-prefill attention on MFMA for gfx950: several query tokens per sequence attend to
// [older shared segment (non-causal) | local ring segment (bottom-right causal or bidirectional)].
//
// Workgroup = NW waves = one (sequence, kv head, query tile); workgroups are numbered so that the
// tiles of one (sequence, kv head) run on one XCD and share its L2.  Query rows are (token, head)
// pairs of the GQA group, row = token * G + head, so every K/V block feeds all heads of the group.
// Each wave owns 32 rows (two 16-column groups of the 16x16x32 MFMA tiles), few enough registers
// (< 256 VGPRs, accumulators in VGPRs) for two waves per SIMD.
// Per 32-token key block:
//   - the NW waves each fetch 16 / NW of the block's 16 one-KiB fragments (K bf16 from the cache,
//     V fp16 from the call's V pre-pass) from HBM/L2 into registers two blocks ahead (one
//     contiguous 1 KiB run per load instruction) and publish them to a ring of LDS buffers in
//     lane order, so every MFMA operand is one conflict-free ds_read_b128;
//   - S^T = K * Q^T with 16x16x32 bf16 MFMAs (exact products, fp32 sums);
//   - online softmax in the exp2 domain (scale and offset folded into one FMA), row max over the
//     four 16-lane rows with VALU lane swaps, O rescaled (a branch taken only when some row's
//     offset moved) with the factor each lane already holds;
//   - O^T += V^T * P^T with 16x16x32 fp16 MFMAs, and the row sums as P times a tile of ones on
//     the same pipe: P in (0, 512) carries 11 mantissa bits (bf16 would carry 8, a 1.7e-3 relative
//     error the rel-L2 1e-3 bound does not allow); the 2-wave instance adds the fp16 residual of
//     P (hi + lo, ~22 bits).  bf16 V converts to fp16 exactly for 2^-17 <= |V| <= 65280 and 0;
//     smaller magnitudes are truncated toward zero (absolute error < 2^-24), larger ones
//     saturate at 65504.
#include <algorithm>
#include <utility>

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
  SegParams seg;
  const float* vscale;
  const float* out_scale;  // [Hkv] or nullptr: out = bf16(bf16(o) * out_scale[kvh])
  int32_t L, hq, hkv, group, causal, tiles;
  int32_t batch;
  float scale_log2;
  int32_t vscale_mode;
  uint16_t* v16;       // fp16 V of every key block, [B, Hkv, v16_blocks, 4096]
  int32_t v16_blocks;  // blocks per (sequence, kv head) in v16
  // per key block of v16: 1 when some V value (older: bf16(V * s)) is finite with magnitude >= 65536,
  // which fp16 cannot hold ([B, Hkv, vflag_stride] bytes after v16); the tiles that read such a block
  // run on the wide instance instead (bf16 V, P as bf16 hi + lo)
  uint8_t* vflags;
  int32_t vflag_stride;
  // set to 1 by the fp16 instance when it skips a tile for the wide one (cleared by the pre-pass).
  // A float: a store of int32 type in the tile kernel may alias the int32 page tables for the
  // compiler, which then reads every page id with a vector load instead of a scalar one.
  float* any_wide;
  // ragged query rows: sequence b's tokens are rows cu[b] .. cu[b + 1] - 1 of q / out (nullptr:
  // L tokens per sequence); rows = the call's total row count.  Sequences with at most
  // decode_rows query rows per kv head run on the decode kernel and are skipped here.
  const int32_t* cu;
  int32_t rows, decode_rows;
  // split-K over the keys for grids that would leave CUs idle: tile_splits key ranges per tile, each
  // writing its rows' normalised fp32 O and base-2 LSE to ws_o [row, Hq, S, 128] / ws_lse
  // [row, Hq, S] (row = the lse row), merged by prefill_split_combine_kernel; 1 = no split
  int32_t tile_splits;
  float* ws_o;
  float* ws_lse;
};

// Query tokens of sequence b and the q / out / lse row of its token 0.
struct SeqRows {
  int L;
  int64_t q0, o0, lse0;
};

__device__ inline SeqRows seq_rows(const PrefillParams& p, int b) {
  SeqRows r;
  if (p.cu == nullptr) {
    r.L = p.L;
    r.q0 = b * p.q_sb;
    r.o0 = b * p.out_sb;
    r.lse0 = static_cast<int64_t>(b) * p.L;
    return r;
  }
  const int s0 = min(max(p.cu[b], 0), p.rows);
  r.L = min(min(max(p.cu[b + 1], s0), p.rows) - s0, p.L);
  r.q0 = s0 * p.q_st;
  r.o0 = s0 * p.out_st;
  r.lse0 = s0;
  return r;
}

// Whether sequence b's queries run in this kernel (ragged calls hand short sequences to the decode
// kernel).
__device__ inline bool on_tile_path(const PrefillParams& p, const SeqRows& sr) {
  return sr.L > 0 && static_cast<int64_t>(sr.L) * p.group > p.decode_rows;
}

// Two values as packed fp16, rounded toward zero: exact for bf16 values of magnitude 2^-17 to 65280
// and for zero (below 2^-17 fp16's subnormals keep them to a multiple of 2^-24).
__device__ inline uint32_t f16x2_bits(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// Whether either bf16 of a packed pair is finite with magnitude >= 65536 (exponent field 143-254):
// fp16 cannot represent it (its largest finite value is 65504; bf16 has none between 65280 and 65536).
__device__ inline bool f16_overflow(uint32_t w) {
  const uint32_t e_lo = (w >> 7) & 0xffu, e_hi = (w >> 23) & 0xffu;
  return (e_lo >= 143u && e_lo < 255u) || (e_hi >= 143u && e_hi < 255u);
}

__device__ inline uint32_t pack_f16_rne(float lo, float hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  h2 r;
  r.x = static_cast<_Float16>(lo);
  r.y = static_cast<_Float16>(hi);
  return __builtin_bit_cast(uint32_t, r);
}

// Local-segment tokens visible to query token `token` of a sequence of L query tokens (causal:
// bottom-right aligned).
__device__ inline int visible_local(const PrefillParams& p, const SeqView& sv, int L, int token) {
  const int v = p.causal ? sv.n1 - L + token + 1 : sv.n1;
  return min(max(v, 0), sv.n1);
}

// One fragment = one 16-byte-per-lane MFMA operand = 1 KiB; a 32-token block is 16 fragments:
// K fragments f = u * 4 + kb (u: 16-token half, kb: 32-dim slice) and V fragments 8 + nb (nb:
// 16-dim slice).  Wave w of NW stages fragments w, w + NW, ... of each block.  Inside a fragment
// lane (n16, g4) holds the 16 bytes at n16 * 64 + g4 * 16.
template <int NW>
struct Stage {
  uint4 r[16 / NW];
};

// Wave-uniform base of the fp16 V workspace of one (sequence, kv head) and its byte range.
struct SegBase {
  const uint16_t* v16;
  int32_t v16_bytes;
};

__device__ inline const uint16_t* uniform_ptr(const uint16_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint16_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t* base, int32_t bytes) {
  // word 3 = 0x00020000: raw (untyped) 32-bit data format, the gfx9 setting for byte-addressed loads
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, base ? bytes : 0, 0x00020000);
}

// Wave w of NW loads fragments w, w + NW, ... of block blk: K (bf16) from the block's cache or
// pool page (a buffer resource over that one 8 KiB block, built with scalar instructions) and V
// (fp16) from the workspace, which holds the blocks in order.
// Wave-uniform address of block blk's K (cache block or pool page).
template <bool kPaged>
__device__ inline const uint16_t* k_block(const SeqView& sv, int blk) {
  return uniform_ptr((blk < sv.nb0 ? sv.ok : sv.lk) + block_offset<kPaged>(sv, blk));
}

// Wave-uniform address of block blk's V in the cache (the wide instance reads bf16 V from there).
template <bool kPaged>
__device__ inline const uint16_t* v_block(const SeqView& sv, int blk) {
  return uniform_ptr((blk < sv.nb0 ? sv.ov : sv.lv) + block_offset<kPaged>(sv, blk));
}

// kblk = k_block<kPaged>(sv, blk), computed by the caller outside the scheduled region (the page-table
// lookup branches).  kWide: V (bf16) from the cache block vblk instead of the fp16 workspace.
template <int NW, bool kWide = false>
__device__ inline void stage_load(Stage<NW>& st, const SegBase sb, const uint16_t* kblk, const uint16_t* vblk, int blk,
                                  int wave, int lane_off) {
  const int voff = blk * (kBlockElems * 2);
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j) {
    const int f = wave + j * NW;  // wave < NW, so f < 8 exactly when j < 8 / NW
    const bool is_k = j < 8 / NW;
    const __amdgpu_buffer_rsrc_t r = is_k ? make_rsrc(kblk, kBlockElems * 2)
                                          : (kWide ? make_rsrc(vblk, kBlockElems * 2) : make_rsrc(sb.v16, sb.v16_bytes));
    const int off = (is_k || kWide ? 0 : voff) + (f & 7) * 1024;
    st.r[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, off, 0));
  }
}

// kWide: the V fragments are bf16 from the cache; an older block's become bf16(V * vs) here (vs = 1:
// unchanged), the value the V pre-pass gives the fp16 instance.
template <int NW, bool kWide = false>
__device__ inline void stage_store(const Stage<NW>& st, uint4* buf, int wave, int lane, float vs = 1.f) {
#pragma unroll
  for (int j = 0; j < 16 / NW; ++j)
    buf[(wave + j * NW) * 64 + lane] = (kWide && j >= 8 / NW) ? scale_frag(st.r[j], vs) : st.r[j];
}

// -inf for tokens outside the block's valid range or past the column's causal limit.
__device__ inline void mask_scores(float (&s)[8], const BlockRef& r, int lim, int g4) {
  const int w0 = 8 * g4;
  const int hi = r.older ? r.hi : min(r.hi, lim - r.seg_tok + 1);
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = (w0 + j >= r.lo && w0 + j < hi) ? s[j] : kNegInf;
}

__device__ inline float max8(const float (&s)[8]) {
  return fmax_nan(fmax3_nan(fmax3_nan(s[0], s[1], s[2]), fmax3_nan(s[3], s[4], s[5]), s[6]), s[7]);
}

// Online-softmax state of one 16-row column group: m = the row's score reference (raw scores),
// mc = m * c, the exp2 offset (0 while m = -inf).
// Probabilities are P = 2^(s c - mc).  m is the exact row maximum after the first block; later it
// is raised only when some P reaches 2^9 (a new maximum more than 9 / c above m), so P < 512
// always: fp16 keeps its full 11-bit precision (P V and the row sums accumulate in fp32), and
// later blocks rarely pay for a rescale.  O / l does not depend on the offset.
struct RowState {
  float m, mc;
};

// Raises each row's reference to its maximum over this block (lm = lane maxima) and rescales O
// and the row sums by 2^(mc_old - mc_new).  Runs for the first block and in a wave-uniform branch
// taken whenever some P reached 2^9.
__device__ inline void raise_rows(RowState& rs, float lm, float c, f32x4 (&o)[8], f32x4& ol) {
  const float bm = wave_max_across_rows(lm);
  const bool up = bm > rs.m;  // m = -inf: true for the first finite maximum
  const float mc_new = up ? bm * c : rs.mc;
  // l and O are 0 while m = -inf: scale them by 0, not by 2^(0 - mc_new), which overflows to inf
  // (and 0 * inf = NaN) when the first maximum is below -128 / c
  const float alpha = up ? (rs.m == kNegInf ? 0.f : fast_exp2(rs.mc - mc_new)) : 1.f;
  rs.m = up ? bm : rs.m;
  rs.mc = rs.m == kNegInf ? 0.f : mc_new;
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[nb] *= alpha;
    ol *= alpha;
  }
}

// fp32 probabilities of 8 scores and their fp16 packing.
__device__ inline void probs(const float (&s)[8], float c, float mc, float (&pr)[8], uint32_t (&w)[4]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(__builtin_fmaf(s[j], c, -mc));
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = pack_f16_rne(pr[2 * j], pr[2 * j + 1]);
}

// The fp16 residuals pr - fp16(pr) of the probabilities packed in w (exact in fp32; fp16
// subnormals keep them to 2^-24 absolute), so hi + lo carries ~22 bits of each probability.
__device__ inline void probs_lo(const float (&pr)[8], const uint32_t (&w)[4], uint32_t (&lo)[4]) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const h2 hi = __builtin_bit_cast(h2, w[j]);
    lo[j] = pack_f16_rne(pr[2 * j] - static_cast<float>(hi.x), pr[2 * j + 1] - static_cast<float>(hi.y));
  }
}

// The wide instance's probabilities: bf16 hi + lo of each (~16 bits, the decode kernel's split) and
// the lane's largest (NaN-propagating).
__device__ inline void probs_bf16(const float (&s)[8], float c, float mc, uint32_t (&hi)[4], uint32_t (&lo)[4],
                                  float& pm) {
  float pr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(__builtin_fmaf(s[j], c, -mc));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hi[j] = pack_bf16x2(pr[2 * j], pr[2 * j + 1]);
    lo[j] = pack_bf16x2(pr[2 * j] - bf16_lo(hi[j]), pr[2 * j + 1] - bf16_hi(hi[j]));
  }
  pm = max8(pr);
}

// The lane's largest packed fp16 probabilities of a block (one per half, NaN-propagating).
__device__ inline uint32_t probs_max(uint32_t a, uint32_t b, uint32_t c) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 x = __builtin_elementwise_maximum(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_maximum(x, __builtin_bit_cast(h2, c)));
}

// A rescale is due when some probability of the block is >= 2^9 (fp16 exponent field >= 24:
// bits 14 and 13 of a half both set), infinite or NaN; pm = probs_max over the block's words.
__device__ inline bool probs_overflow(uint32_t pm) { return (pm & (pm << 1) & 0x40004000u) != 0; }

template <int N>
struct IC {
  static constexpr int value = N;
};

// f(IC<0>{}), f(IC<1>{}), ... in order.
template <int... J, class F>
__device__ __attribute__((always_inline)) inline void unroll_steps(std::integer_sequence<int, J...>, F&& f) {
  (f(IC<J>{}), ...);
}

// V pre-pass: every key block of every (sequence, kv head) as fp16 in block order [older |
// local], with the older segment as bf16(V * s) (the reference's rounded _scale()).  The
// attention kernel's query tiles then stage V as plain copies instead of each converting it.
// Each block also gets its flag: whether some value does not fit fp16 (magnitude 65536 or more).
// Blocks [x kBlocks, (x + 1) kBlocks) of (kv head y, sequence b), 256 threads x 16 values per block.
template <bool kPaged, int kBlocks>
__device__ __attribute__((always_inline)) inline void v16_stage_blocks(const PrefillParams& p, int b, int kvh, int x);

// Uniform calls (kBlocks 1): one workgroup per (block, kv head, sequence).  Ragged calls (kBlocks
// 8): one per (8 blocks, kv head, z < Z) that converts those blocks of the tile-path sequences of
// rank z, z + Z, ... (a
// wave scan of cu_seqlens finds them): a grid over every sequence had mostly exiting workgroups
// (a serving step of 31 decode rows and one 1024-token row: 33 us with one block per workgroup, 25
// with 8 and every sequence in the grid).
template <bool kPaged, int kBlocks>
__global__ __launch_bounds__(256) void v16_stage_kernel(const PrefillParams p) {
  const int kvh = blockIdx.y;
  if ((blockIdx.x | blockIdx.y | blockIdx.z) == 0 && threadIdx.x == 0) *p.any_wide = 0.f;  // (the tile kernels run after this one)
  if constexpr (kBlocks == 1) {  // (uniform calls)
    if (on_tile_path(p, seq_rows(p, blockIdx.z))) v16_stage_blocks<kPaged, kBlocks>(p, blockIdx.z, kvh, blockIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  int rank = 0;
  for (int i0 = 0; i0 < p.batch; i0 += 64) {
    const int i = i0 + lane;
    uint64_t m = __builtin_amdgcn_ballot_w64(i < p.batch && on_tile_path(p, seq_rows(p, i)));
    while (m != 0) {  // (wave-uniform)
      const int l = __builtin_ctzll(m);
      m &= m - 1;
      if (rank++ % static_cast<int>(gridDim.z) == static_cast<int>(blockIdx.z))
        v16_stage_blocks<kPaged, kBlocks>(p, i0 + l, kvh, blockIdx.x);
    }
  }
}

template <bool kPaged, int kBlocks>
__device__ __attribute__((always_inline)) inline void v16_stage_blocks(const PrefillParams& p, int b, int kvh, int x) {
  const SeqView sv = make_seq_view(p.seg, b, kvh);
  const int nb = sv.nb0 + local_blocks(sv, sv.n1);
  const float vs = p.vscale_mode ? p.vscale[kvh] : 1.f;
  const int blk0 = x * kBlocks;
  const int n = min(kBlocks, nb - blk0);  // (workgroup-uniform)
  if (n <= 0) return;
  // every block's loads first (one round trip for all of them), then the conversions and stores
  uint4 raw[kBlocks][2];
#pragma unroll
  for (int k = 0; k < kBlocks; ++k) {
    if (k >= n) break;
    const int blk = blk0 + k;
    const uint16_t* src = (blk < sv.nb0 ? sv.ov : sv.lv) + block_offset<kPaged>(sv, blk);
#pragma unroll
    for (int j = 0; j < 2; ++j) raw[k][j] = *reinterpret_cast<const uint4*>(src + (threadIdx.x + j * 256) * 8);
  }
  uint32_t over = 0;  // bit k: block k holds a value fp16 cannot
#pragma unroll
  for (int k = 0; k < kBlocks; ++k) {
    if (k >= n) break;
    const int blk = blk0 + k;
    uint16_t* dst = p.v16 + ((static_cast<int64_t>(b) * p.hkv + kvh) * p.v16_blocks + blk) * kBlockElems;
    const float s = blk < sv.nb0 ? vs : 1.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // bf16(v * s); bf16(v * 1) == v, so the unscaled blocks take the same instructions
      const uint4 y = scale_frag(raw[k][j], s);
      if (f16_overflow(y.x) || f16_overflow(y.y) || f16_overflow(y.z) || f16_overflow(y.w)) over |= 1u << k;
      *reinterpret_cast<uint4*>(dst + (threadIdx.x + j * 256) * 8) =
          make_uint4(f16x2_bits(bf16_lo(y.x), bf16_hi(y.x)), f16x2_bits(bf16_lo(y.y), bf16_hi(y.y)),
                     f16x2_bits(bf16_lo(y.z), bf16_hi(y.z)), f16x2_bits(bf16_lo(y.w), bf16_hi(y.w)));
    }
  }
  // the blocks' flags: an OR over the workgroup of each thread's bits
  __shared__ uint32_t sm_over;
  if (threadIdx.x == 0) sm_over = 0;
  __syncthreads();
  if (over != 0) atomicOr(&sm_over, over);
  __syncthreads();
  if (threadIdx.x < n)
    p.vflags[(static_cast<int64_t>(b) * p.hkv + kvh) * p.vflag_stride + blk0 + threadIdx.x] =
        (sm_over >> threadIdx.x) & 1u;
  __syncthreads();  // (sm_over is reused by the next sequence's call)
}

// Whether some block in [0, nbt) of (b, kvh) holds a V value fp16 cannot (the pre-pass's flags),
// read 16 flags per load over the wave.
// The flags of blocks [i, i + 16) of a flag row, those at or past nbt cleared (by masks, not by an
// indexed write, which would put the word in LDS).
__device__ inline uint4 flags_below(uint4 w, int i, int nbt) {
  const int valid = nbt - i;  // flags of this word that count (0-16)
  auto mask = [valid](int word) {
    const int n = min(max(valid - 4 * word, 0), 4);  // bytes of this 32-bit word that count
    return n == 4 ? 0xffffffffu : (1u << (8 * n)) - 1u;
  };
  return make_uint4(w.x & mask(0), w.y & mask(1), w.z & mask(2), w.w & mask(3));
}

// Whether some block in [0, nbt) of (b, kvh) holds a V value fp16 cannot (the pre-pass's flags), in
// two parts so that the load's latency can pass under other loads: flags_peek issues each lane's
// first 16 flags (the row's first 1024 blocks), flags_any masks them, reads any further ones and
// takes the wave's ballot.
struct FlagPeek {
  uint4 w;
};

__device__ inline FlagPeek flags_peek(const PrefillParams& p, int b, int kvh, int nbt) {
  const uint8_t* f = p.vflags + (static_cast<int64_t>(b) * p.hkv + kvh) * p.vflag_stride;
  const int i = (threadIdx.x & 63) * 16;
  FlagPeek r{make_uint4(0, 0, 0, 0)};
  if (i < nbt) r.w = *reinterpret_cast<const uint4*>(f + i);
  return r;
}

__device__ inline bool flags_any(const FlagPeek& pk, const PrefillParams& p, int b, int kvh, int nbt) {
  const uint8_t* f = p.vflags + (static_cast<int64_t>(b) * p.hkv + kvh) * p.vflag_stride;
  const int lane = threadIdx.x & 63;
  uint4 w = flags_below(pk.w, lane * 16, nbt);
  bool any = (w.x | w.y | w.z | w.w) != 0;
  for (int i = lane * 16 + 64 * 16; i < nbt; i += 64 * 16) {
    w = flags_below(*reinterpret_cast<const uint4*>(f + i), i, nbt);
    any |= (w.x | w.y | w.z | w.w) != 0;
  }
  return __builtin_amdgcn_ballot_w64(any) != 0;
}

__device__ inline bool tile_needs_wide(const PrefillParams& p, int b, int kvh, int nbt) {
  return flags_any(flags_peek(p, b, kvh, nbt), p, b, kvh, nbt);
}

// Whether some key block of (b, kvh) holds a V value fp16 cannot, over all nb of its blocks.
__device__ inline bool pair_needs_wide(const PrefillParams& p, int b, int kvh) {
  if (!on_tile_path(p, seq_rows(p, b))) return false;  // (the pre-pass wrote no flags for it)
  const SeqView sv = make_seq_view(p.seg, b, kvh);
  return tile_needs_wide(p, b, kvh, sv.nb0 + local_blocks(sv, sv.n1));
}

constexpr int kMaxTileSplits = 4;  // key splits of a tile (the wide instance marks the others of its rows empty)
constexpr int kTileRing = 4;       // LDS block buffers of the tile kernel
constexpr int kTileBuf = 1024;     // uint4 per block buffer (16 KiB)

// Workgroup = NW waves x 16 * CG query rows (CG 16-column groups per wave).  K (bf16, from the caches)
// and V (fp16, from the pre-pass) blocks go through a ring of kRing LDS buffers; two register
// stage sets keep the global loads two steps ahead of their LDS store.  Step i (block i in
// buffer i % 4, block i + 1 in buffer (i + 1) % 4): probabilities of block i from the scores
// computed in step i - 1, QK^T of block i + 1, P V of block i, store block i + 2 into buffer
// (i + 2) % 4, load block i + 4, one barrier.
// The 2-wave instance (calls of at most 64 query rows per kv head, bound by HBM, not by the matrix
// pipe) splits P into fp16 hi + lo and runs P V twice, so its probabilities carry ~22 bits
// instead of 11.  prefill_tile runs query tile `tile` of (sequence b, kv head kvh), over key split
// `split` of p.tile_splits: split s of S' covers blocks [s q, (s + 1) q), q = ceil(nbt / S'), the
// last one to nbt, with S' <= S the most splits that all start in the older segment ((S' - 1) q <
// nb0), so every split begins with an older block that every row sees (the exact maximum of its
// first block is then finite for every row); splits from S' on are empty (their states say so).
// kWide: the instance for tiles whose V does not fit fp16 (the pre-pass flagged one of their blocks):
// V staged as bf16 from the caches (older blocks as bf16(V * s)), P split into bf16 hi + lo, P V and
// the row sums on bf16 MFMAs; the fp16 instance skips those tiles and this one runs only them.
template <int NW, int CG, bool kPaged, bool kWide = false>
__device__ __attribute__((always_inline)) inline void prefill_tile(const PrefillParams& p, const int b, const int kvh,
                                                                   const int tile, const int split, uint4* lds) {
  constexpr bool kSplitP = NW == 2 || kWide;
  constexpr int kStages = 2;  // register stage sets (global loads run kStages steps ahead of their LDS store)
  constexpr int kDist = 2;    // step i stores block i + kDist into the LDS ring
  constexpr int kRing = kTileRing;
  constexpr int kBuf = kTileBuf;
  constexpr int kRowsPerWave = 16 * CG;
  constexpr int kRowsPerWg = NW * kRowsPerWave;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;
  const int G = p.group;
  const SeqRows sr = seq_rows(p, b);
  const int rows_total = sr.L * G;
  const int wg_row0 = tile * kRowsPerWg;
  const int row0 = wg_row0 + wave * kRowsPerWave;
  // (workgroup-uniform: a ragged call's tiles past a sequence's rows, or its short sequences)
  if (!on_tile_path(p, sr) || wg_row0 >= rows_total) return;

  SeqView sv = make_seq_view(p.seg, b, kvh);
  // these are wave-uniform; keeping them in scalar registers keeps every block offset scalar
  sv.n0 = __builtin_amdgcn_readfirstlane(sv.n0);
  sv.n1 = __builtin_amdgcn_readfirstlane(sv.n1);
  sv.nb0 = __builtin_amdgcn_readfirstlane(sv.nb0);
  sv.lblk0 = __builtin_amdgcn_readfirstlane(sv.lblk0);
  sv.lead = __builtin_amdgcn_readfirstlane(sv.lead);
  const int wg_last_row = min(rows_total, wg_row0 + kRowsPerWg) - 1;
  const int nbt = __builtin_amdgcn_readfirstlane(sv.nb0 + local_blocks(sv, visible_local(p, sv, sr.L, wg_last_row / G)));
  // The tiles that read a V block fp16 cannot hold belong to the wide instance: it leaves the other
  // tiles at once, and the fp16 instance leaves these at its prologue's barrier, reducing the flags
  // only after its first Q and K / V loads are issued, so that the flag load's latency passes under
  // theirs.  (Both workgroup-uniform.)
  const FlagPeek flag_peek = flags_peek(p, b, kvh, nbt);
  bool needs_wide = false;
  if (kWide) {
    needs_wide = flags_any(flag_peek, p, b, kvh, nbt);
    if (!needs_wide) return;
  }
  const float vs_older = p.vscale_mode ? p.vscale[kvh] : 1.f;  // (the wide instance's V scale)
  // this split's blocks [kb0, kb1) (the wide instance runs every block as split 0)
  const int S = kWide ? 1 : p.tile_splits;
  int kb0 = 0, kb1 = nbt;
  if (S > 1) {
    // as many equal splits as start inside the older segment (a short older segment would leave
    // the last split most of the keys: slower than no split)
    int se = min(S, sv.nb0);
    while (se > 1 && (se - 1) * ((nbt + se - 1) / se) > sv.nb0 - 1) --se;
    if (split >= max(se, 1)) {
      kb1 = 0;
    } else if (se > 1) {
      const int q = (nbt + se - 1) / se;
      kb0 = split * q;
      if (split + 1 < se) kb1 = (split + 1) * q;
    }
  }
  kb0 = __builtin_amdgcn_readfirstlane(kb0);
  kb1 = __builtin_amdgcn_readfirstlane(kb1);

  uint4 qf[CG][4];
  int lim[CG];  // last visible local-segment token of this lane's column
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int row = row0 + 16 * cg + n16;
    if (row < rows_total) {
      const int tok = row / G, h = row - tok * G;
      const uint16_t* qrow = p.q + sr.q0 + tok * p.q_st + static_cast<int64_t>(kvh * G + h) * kHeadDim;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qf[cg][kb] = *reinterpret_cast<const uint4*>(qrow + 32 * kb + 8 * g4);
      lim[cg] = visible_local(p, sv, sr.L, tok) - 1;
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qf[cg][kb] = make_uint4(0, 0, 0, 0);
      lim[cg] = -1;
    }
  }
  const float c = p.scale_log2;
  // smallest causal limit among the wave's rows (its first row); blocks past it need masking
  const int w_min_lim =
      __builtin_amdgcn_readfirstlane(row0 < rows_total ? visible_local(p, sv, sr.L, row0 / G) - 1 : -1);

  RowState rs[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) rs[cg] = RowState{kNegInf, 0.f};
  // O^T tiles (lane (n16, g4): dims 16 nb + 4 g4 + i of row n16) and the row sums of the fp16 P,
  // accumulated on the matrix pipe as P times a tile of ones (each lane holds its row's sum).
  f32x4 o[CG][8], ol[CG];
  const uint4 kOnes = make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
  const uint4 kOnesBf16 = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    ol[cg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[cg][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  if (kb1 > kb0) {
    SegBase rsrc;
    rsrc.v16 = uniform_ptr(p.v16 + (static_cast<int64_t>(b) * p.hkv + kvh) * p.v16_blocks * kBlockElems);
    rsrc.v16_bytes = p.v16_blocks * (kBlockElems * 2);
    const int lane_off = n16 * 64 + g4 * 16;
    // Loads are unconditional (indices past the end re-read the last block, an L2 hit) so that
    // the compiler can count outstanding loads for s_waitcnt.
    const int last = kb1 - 1;

    Stage<NW> sets[kStages];
    // (the V blocks of the wide instance; the fp16 instance reads V from the workspace)
    auto vb = [&](int blk) __attribute__((always_inline)) { return kWide ? v_block<kPaged>(sv, blk) : nullptr; };
    auto vs_of = [&](int blk) __attribute__((always_inline)) { return kWide && blk < sv.nb0 ? vs_older : 1.f; };
#pragma unroll
    for (int j = 0; j < kStages; ++j)
      stage_load<NW, kWide>(sets[j], rsrc, k_block<kPaged>(sv, min(kb0 + j, last)), vb(min(kb0 + j, last)),
                            min(kb0 + j, last), wave, lane_off);
#pragma unroll
    for (int j = 0; j < kDist; ++j) {
      stage_store<NW, kWide>(sets[j % kStages], lds + j * kBuf, wave, lane, vs_of(min(kb0 + j, last)));
      const int lb = min(kb0 + j + kStages, last);
      stage_load<NW, kWide>(sets[j % kStages], rsrc, k_block<kPaged>(sv, lb), vb(lb), lb, wave, lane_off);
    }
    if (!kWide) needs_wide = flags_any(flag_peek, p, b, kvh, nbt);
    if (!kWide && needs_wide) {
      if (threadIdx.x == 0) *p.any_wide = 1.f;
      return;
    }
    __syncthreads();

    // S^T of block kb0: sc[cg][u] holds tokens 8 * g4 + 4u .. + 3 of this lane's column n16 of
    // group cg
    f32x4 sc[CG][2];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
#pragma unroll
      for (int u = 0; u < 2; ++u) sc[cg][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint4 k0 = lds[kb * 64 + lane];
      const uint4 k1 = lds[(4 + kb) * 64 + lane];
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        sc[cg][0] = mfma_bf16(k0, qf[cg][kb], sc[cg][0]);
        sc[cg][1] = mfma_bf16(k1, qf[cg][kb], sc[cg][1]);
      }
    }
    // Block 0 sets every row's reference to its exact maximum (a row that sees any key sees one
    // in block 0: visible keys are a prefix of [older | local]).  Inside the loop the only rescale
    // test is then the packed-probability overflow check, so the compiler keeps the QK^T MFMAs of
    // block i + 1 and the probabilities of block i in one scheduling region and interleaves them.
    {
      const BlockRef r0 = block_range(sv, kb0);
      float s0[CG][8];
#pragma unroll
      for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s0[cg][i] = sc[cg][0][i];
          s0[cg][4 + i] = sc[cg][1][i];
        }
      if (r0.lo > 0 || r0.hi < kBlockTokens || (!r0.older && r0.seg_tok + kBlockTokens - 1 > w_min_lim)) {
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) mask_scores(s0[cg], r0, lim[cg], g4);
      }
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) raise_rows(rs[cg], max8(s0[cg]), c, o[cg], ol[cg]);
    }

    // Step i: the 16 LDS reads (K of block i + 1, V of block i) are issued first so their latency
    // passes under the mask work; then the QK^T MFMAs of block i + 1 are interleaved with the
    // probabilities of block i (1 MFMA : 2 VALU : 1 exp), and the P V MFMAs of block i with the
    // row sums and the staging of block i + 2.  A wave whose rows see no keys in a block still
    // runs it: the mask makes every score -inf, so P = 0 and O, l, m do not change (at most two
    // blocks per wave at the causal edge).
    auto step = [&](auto rc, int blk) __attribute__((always_inline)) {
      constexpr int R = decltype(rc)::value;
      const uint4* cur = lds + R * kBuf;
      const uint4* nxt = lds + ((R + 1) % kRing) * kBuf;
      uint4* wr = lds + ((R + kDist) % kRing) * kBuf;
      // the register set holding block i + kDist (loaded kStages steps ago)
      Stage<NW>& st = sets[(R + kDist) % kStages];
      const int ld_blk = min(blk + kDist + kStages, last);
      const uint16_t* ld_k = k_block<kPaged>(sv, ld_blk);
      const uint16_t* ld_v = vb(ld_blk);
      const float st_vs = vs_of(min(blk + kDist, last));  // (the block st holds)
      uint4 kf[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) kf[t] = nxt[t * 64 + lane];
      const BlockRef r = block_range(sv, blk);
      float s[CG][8];
#pragma unroll
      for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[cg][i] = sc[cg][0][i];
          s[cg][4 + i] = sc[cg][1][i];
        }
      // partial block, or a local block crossing the causal limit of some row of this wave
      if (r.lo > 0 || r.hi < kBlockTokens || (!r.older && r.seg_tok + kBlockTokens - 1 > w_min_lim)) {
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) mask_scores(s[cg], r, lim[cg], g4);
      }
      // QK^T of block i + 1 (past the last block it multiplies a stale buffer; never used)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int u = 0; u < 2; ++u) sc[cg][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
          sc[cg][0] = mfma_bf16(kf[kb], qf[cg][kb], sc[cg][0]);
          sc[cg][1] = mfma_bf16(kf[4 + kb], qf[cg][kb], sc[cg][1]);
        }
      uint32_t pw[CG][4], pl[CG][4];
      uint32_t pmax;  // the lane's largest probabilities of this block (packed fp16)
      float pmf = 0.f;  // (the wide instance: the largest as fp32)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        if constexpr (kWide) {
          float pm;
          probs_bf16(s[cg], c, rs[cg].mc, pw[cg], pl[cg], pm);
          pmf = fmax_nan(pmf, pm);
        } else {
          float pr[8];
          probs(s[cg], c, rs[cg].mc, pr, pw[cg]);
          if (kSplitP) probs_lo(pr, pw[cg], pl[cg]);
          pmax = cg == 0 ? probs_max(pw[cg][0], pw[cg][1], probs_max(pw[cg][2], pw[cg][3], pw[cg][3]))
                         : probs_max(pmax, probs_max(pw[cg][0], pw[cg][1], pw[cg][2]), pw[cg][3]);
        }
      }
      uint4 vf[8];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) vf[nb] = cur[512 + nb * 64 + lane];
      // the first probabilities go ahead of the first MFMA, which waits for the K fragments
      // just read from LDS (in-order issue would otherwise hold every exp behind that wait);
      // measured best: 4 with 4-wave tiles, 2 with 8-wave tiles
      __builtin_amdgcn_sched_group_barrier(0x002, NW == 8 ? 2 : 4, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x400, NW == 8 ? 2 : 4, 0);  // exp
#pragma unroll
      for (int i = 0; i < 8 * CG; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (QK^T of block i + 1)
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);  // exp
      }
      // a new row maximum: exact maxima, rescale, recompute this block's P
      if (__builtin_amdgcn_ballot_w64(kWide ? !(pmf < 512.f) : probs_overflow(pmax))) {
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
          raise_rows(rs[cg], max8(s[cg]), c, o[cg], ol[cg]);
          if constexpr (kWide) {
            float pm;
            probs_bf16(s[cg], c, rs[cg].mc, pw[cg], pl[cg], pm);
          } else {
            float pr[8];
            probs(s[cg], c, rs[cg].mc, pr, pw[cg]);
            if (kSplitP) probs_lo(pr, pw[cg], pl[cg]);
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
          const uint4 ph = make_uint4(pw[cg][0], pw[cg][1], pw[cg][2], pw[cg][3]);
          if constexpr (kWide) {
            o[cg][nb] = mfma_bf16(vf[nb], ph, o[cg][nb]);
            o[cg][nb] = mfma_bf16(vf[nb], make_uint4(pl[cg][0], pl[cg][1], pl[cg][2], pl[cg][3]), o[cg][nb]);
          } else {
            o[cg][nb] = mfma_f16(vf[nb], ph, o[cg][nb]);
            if constexpr (kSplitP)
              o[cg][nb] = mfma_f16(vf[nb], make_uint4(pl[cg][0], pl[cg][1], pl[cg][2], pl[cg][3]), o[cg][nb]);
          }
        }
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        const uint4 ph = make_uint4(pw[cg][0], pw[cg][1], pw[cg][2], pw[cg][3]);
        if constexpr (kWide) {
          ol[cg] = mfma_bf16(kOnesBf16, ph, ol[cg]);
          ol[cg] = mfma_bf16(kOnesBf16, make_uint4(pl[cg][0], pl[cg][1], pl[cg][2], pl[cg][3]), ol[cg]);
        } else {
          ol[cg] = mfma_f16(kOnes, ph, ol[cg]);
          if constexpr (kSplitP) ol[cg] = mfma_f16(kOnes, make_uint4(pl[cg][0], pl[cg][1], pl[cg][2], pl[cg][3]), ol[cg]);
        }
      }
      stage_store<NW, kWide>(st, wr, wave, lane, st_vs);
      stage_load<NW, kWide>(st, rsrc, ld_k, ld_v, ld_blk, wave, lane_off);
#pragma unroll
      for (int i = 0; i < (kSplitP ? 18 : 9) * CG; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (P V and P 1 of block i)
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write (staging of block i + 2)
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (load of block i + 4)
      }
      __syncthreads();
    };
    // Whole rounds of the ring in the loop, the 0-3 remaining blocks after it: an exit from the
    // middle of a round gives the loop header a second predecessor on which that round's stage
    // loads are still in flight, and the header then waits for every load each round.
    int blk = kb0;
    // (the remaining blocks as independent tests, not nested ones: 0.5 points faster on configs 3-5)
    for (; blk + kRing <= kb1; blk += kRing)
      unroll_steps(std::make_integer_sequence<int, kRing>{},
                   [&](auto jc) __attribute__((always_inline)) { step(jc, blk + decltype(jc)::value); });
    unroll_steps(std::make_integer_sequence<int, kRing - 1>{}, [&](auto jc) __attribute__((always_inline)) {
      if (blk + decltype(jc)::value < kb1) step(jc, blk + decltype(jc)::value);
    });
  }

  // normalise and write: lane (n16, g4) holds dims 16 * nb + 4 * g4 + i of row n16 of each group
  const float os = p.out_scale != nullptr ? p.out_scale[kvh] : 1.f;
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const float lt = ol[cg][0];
    const float linv = lt > 0.f ? 1.f / lt : 0.f;
    const int row = row0 + 16 * cg + n16;
    if (row < rows_total && p.tile_splits > 1) {  // this split's state (the wide instance: split 0)
      const int tok = row / G, h = row - tok * G;
      const int64_t srow = ((sr.lse0 + tok) * p.hq + kvh * G + h) * p.tile_splits + (kWide ? 0 : split);
      float* orow = p.ws_o + srow * kHeadDim;
      if (lt > 0.f) {  // (an empty split's O is never read: its LSE says so)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
          *reinterpret_cast<f32x4*>(orow + 16 * nb + 4 * g4) = o[cg][nb] * linv;
      }
      if (g4 == 0) p.ws_lse[srow] = lt > 0.f ? rs[cg].mc + __log2f(lt) : kNegInf;
      if (kWide && g4 < p.tile_splits - 1) p.ws_lse[srow + 1 + g4] = kNegInf;  // (the other splits, <= 3: empty)
    } else if (row < rows_total) {
      const int tok = row / G, h = row - tok * G;
      uint16_t* orow = p.out + sr.o0 + tok * p.out_st + static_cast<int64_t>(kvh * G + h) * kHeadDim;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const f32x4 x = o[cg][nb] * linv;
        uint32_t w01 = pack_bf16x2(x[0], x[1]), w23 = pack_bf16x2(x[2], x[3]);
        if (p.out_scale != nullptr) {  // bf16(bf16(o) * s), the reference's rescale of its bf16 output
          w01 = pack_bf16x2(bf16_lo(w01) * os, bf16_hi(w01) * os);
          w23 = pack_bf16x2(bf16_lo(w23) * os, bf16_hi(w23) * os);
        }
        *reinterpret_cast<uint2*>(orow + 16 * nb + 4 * g4) = make_uint2(w01, w23);
      }
      if (p.lse != nullptr && g4 == 0)
        p.lse[(sr.lse0 + tok) * p.hq + kvh * G + h] =
            lt > 0.f ? (rs[cg].mc + __log2f(lt)) * kLn2 : kNegInf;
    }
  }
}

// Ragged calls: the sequence and tile of the call's tile number gt, counting the tiles of the
// sequences on the tile path in order (ceil(rows / rows_per_wg) each); false past the last one.
// Every wave scans the sequences itself, 64 per step (an inclusive scan of the tile counts over the
// lanes, then a ballot for the first lane whose running total exceeds gt).
__device__ inline bool ragged_tile(const PrefillParams& p, int gt, int rows_per_wg, int& b, int& tile) {
  const int lane = threadIdx.x & 63;
  int base = 0;  // tiles of the sequences before this step's 64
  for (int i0 = 0; i0 < p.batch; i0 += 64) {
    const int i = i0 + lane;
    int nt = 0;
    if (i < p.batch) {
      const SeqRows sr = seq_rows(p, i);
      if (on_tile_path(p, sr)) nt = (sr.L * p.group + rows_per_wg - 1) / rows_per_wg;
    }
    int incl = nt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    const int total = __shfl(incl, 63);
    if (gt < base + total) {
      const int l = __builtin_ctzll(__builtin_amdgcn_ballot_w64(base + incl > gt));
      b = i0 + l;
      tile = gt - base - __shfl(incl - nt, l);
      return true;
    }
    base += total;
  }
  return false;
}

// One workgroup per query tile.  Workgroup ids map to tiles so that the tiles of one (sequence, kv
// head) run on one XCD; in causal calls a tile's key count grows with its index, and the tiles are
// dispatched longest first (largest index first), which shortens the tail of the last workgroups
// (config-3 chunk pieces: 41.9 -> 43.1 % of the MFMA peak in a same-box A/B; the bidirectional Wan
// block's tiles are all alike and keep their order).  A ragged call's grid holds (an upper bound of)
// the tiles its sequences need, kv head fastest, each workgroup finding its sequence and tile by a
// scan of cu_seqlens: a grid sized by the longest sequence for every sequence mostly exits, and the
// exits delayed the working tiles (a serving step of 31 decode rows, a 1024-token row and a 7-token
// row: 258 us for the one long row against 206 us for the same tiles alone).
template <int NW, int CG, int WPE, bool kPaged>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE))) void prefill_kernel(
    const PrefillParams p) {
  __shared__ uint4 lds[kTileRing * kTileBuf];
  // key splits: the grid is tile_splits copies of the tile grid, the split the slowest index
  const int per_split = static_cast<int>(gridDim.x) / p.tile_splits;
  const int split = static_cast<int>(blockIdx.x) / per_split;
  const int id = static_cast<int>(blockIdx.x) - split * per_split;
  int b, kvh, tile, tiles;
  if (p.cu != nullptr) {
    kvh = id % p.hkv;
    if (!ragged_tile(p, id / p.hkv, NW * 32, b, tile)) return;  // (workgroup-uniform)
    tiles = (seq_rows(p, b).L * p.group + NW * 32 - 1) / (NW * 32);
  } else {
    const int logical = xcd_logical_index(id, per_split);
    tiles = p.tiles;
    tile = logical % tiles;
    kvh = (logical / tiles) % p.hkv;
    b = logical / (tiles * p.hkv);
  }
  // (one call site: the tile body is inlined once)
  prefill_tile<NW, CG, kPaged>(p, __builtin_amdgcn_readfirstlane(b), __builtin_amdgcn_readfirstlane(kvh),
                               __builtin_amdgcn_readfirstlane(p.causal ? tiles - 1 - tile : tile),
                               __builtin_amdgcn_readfirstlane(split), lds);
}

// Merges the key splits of one (row, query head) per wave: O = sum_s 2^(lse_s - lse) O_s with
// lse = log2(sum_s 2^lse_s) (splits with no visible key have lse_s = -inf and weight 0), then
// the output rounding of the unsplit path (bf16, optional bf16(bf16(o) * s)) and the natural-log
// LSE.  Rows of sequences that are not on the tile path (a ragged call's decode rows) are skipped.
__global__ __launch_bounds__(256) void prefill_split_combine_kernel(const PrefillParams p, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // (row, head)
  if (item >= rows * p.hq) return;
  const int64_t row = item / p.hq;  // the lse row: b * L + token, or the ragged row
  const int h = static_cast<int>(item - row * p.hq);
  const int S = p.tile_splits;
  const int64_t s0 = item * S;
  // every split's state is loaded up front, beside the sequence lookup
  float ls[kMaxTileSplits];
  float2 x[kMaxTileSplits];
#pragma unroll
  for (int s = 0; s < kMaxTileSplits; ++s) {
    ls[s] = s < S ? p.ws_lse[s0 + s] : kNegInf;
    x[s] = s < S ? *reinterpret_cast<const float2*>(p.ws_o + (s0 + s) * kHeadDim + 2 * lane) : float2{0.f, 0.f};
  }
  int b = 0;
  int64_t tok = row;
  SeqRows sr;
  if (p.cu == nullptr) {
    b = static_cast<int>(row / p.L);
    tok = row - static_cast<int64_t>(b) * p.L;
    sr = seq_rows(p, b);
  } else {  // the sequence holding this row: the last b with cu[b] <= row (a wave scan, 64 per step)
    int c_lo = 0, c_hi = 0;
    for (int i0 = 0; i0 < p.batch; i0 += 64) {
      const int i = i0 + lane;
      const int c = i <= p.batch ? min(max(p.cu[i], 0), p.rows) : p.rows;  // cu[b], clamped as seq_rows does
      const uint64_t m = __builtin_amdgcn_ballot_w64(i < p.batch && c <= row);
      if (m == 0) break;
      const int l = 63 - __builtin_clzll(m);
      b = i0 + l;
      c_lo = __shfl(c, l);
      c_hi = l < 63 ? __shfl(c, l + 1) : min(max(p.cu[b + 1], 0), p.rows);
    }
    sr.L = min(max(c_hi, c_lo) - c_lo, p.L);
    sr.o0 = static_cast<int64_t>(c_lo) * p.out_st;
    sr.lse0 = c_lo;
    tok = row - sr.lse0;
    if (tok < 0 || tok >= sr.L) return;
  }
  if (!on_tile_path(p, sr)) return;  // (a ragged call's decode rows)
  float m = kNegInf;
#pragma unroll
  for (int s = 0; s < kMaxTileSplits; ++s) m = fmaxf(m, ls[s]);
  float l = 0.f, o0 = 0.f, o1 = 0.f;
  if (m != kNegInf) {
#pragma unroll
    for (int s = 0; s < kMaxTileSplits; ++s) {
      if (ls[s] == kNegInf) continue;  // (no visible key, or no such split: weight 0)
      const float w = fast_exp2(ls[s] - m);
      l += w;
      o0 += w * x[s].x;
      o1 += w * x[s].y;
    }
  }
  const float linv = l > 0.f ? 1.f / l : 0.f;
  uint32_t w01 = pack_bf16x2(o0 * linv, o1 * linv);
  const int kvh = h / p.group;
  if (p.out_scale != nullptr) w01 = pack_bf16x2(bf16_lo(w01) * p.out_scale[kvh], bf16_hi(w01) * p.out_scale[kvh]);
  uint16_t* orow = p.out + sr.o0 + tok * p.out_st + static_cast<int64_t>(h) * kHeadDim;
  *reinterpret_cast<uint32_t*>(orow + 2 * lane) = w01;
  if (p.lse != nullptr && lane == 0) p.lse[row * p.hq + h] = l > 0.f ? (m + __log2f(l)) * kLn2 : kNegInf;
}

// The wide instance: one workgroup per (sequence, kv head) pair at a time, min(pairs, CUs) of them.
// Unless the fp16 instance skipped a tile, every workgroup exits after one load (the launch costs a
// few microseconds instead of a full grid of tile workgroups that each check their flags and exit).
// Otherwise a pair none of whose V blocks the pre-pass flagged is skipped after one flag scan, and a
// flagged pair's tiles run here one after another, each tile again checking whether its own blocks
// reach a flagged one (the fp16 instance ran the others).
template <int NW, int CG, int WPE, bool kPaged>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE))) void prefill_wide_kernel(
    const PrefillParams p) {
  __shared__ uint4 lds[kTileRing * kTileBuf];
  if (*p.any_wide == 0.f) return;  // the fp16 instance ran every tile (workgroup-uniform)
  const int pairs = p.batch * p.hkv;
  for (int pair = blockIdx.x; pair < pairs; pair += gridDim.x) {
    if (!pair_needs_wide(p, pair / p.hkv, pair % p.hkv)) continue;  // (workgroup-uniform)
    for (int tile = 0; tile < p.tiles; ++tile) {
      prefill_tile<NW, CG, kPaged, true>(p, pair / p.hkv, pair % p.hkv, tile, 0, lds);
      __syncthreads();  // the next tile's staging reuses the LDS ring
    }
  }
}

}  // namespace
}  // namespace lkv

namespace {

// Key blocks per (sequence, kv head) the fp16 V workspace must hold: exact when the lengths and
// the ring start are host constants, else bounded by the capacities.
int64_t v16_blocks(const lkv_prefill_args* a) {
  using namespace lkv;
  int64_t n0 = 0, lblocks = 0;
  if (a->older_k != nullptr)
    n0 = a->older_len ? a->older_capacity_tokens
                      : std::min<int64_t>(std::max(a->older_len_const, 0), a->older_capacity_tokens);
  if (a->local_k != nullptr) {
    const int64_t ring = static_cast<int64_t>(a->local_ring_blocks) * kBlockTokens;
    const int64_t n1 = a->local_len ? ring : std::min<int64_t>(std::max(a->local_len_const, 0), ring);
    const int64_t lead = a->local_start ? kBlockTokens - 1 : (a->local_start_const & (kBlockTokens - 1));
    lblocks = n1 > 0 ? (lead + n1 + kBlockTokens - 1) / kBlockTokens : 0;
  }
  return (n0 + kBlockTokens - 1) / kBlockTokens + lblocks;
}

// Bytes of the V pre-pass's output: the fp16 V blocks, then one overflow flag per block (rows of a
// multiple of 16 bytes per (sequence, kv head)), then a 16-byte word that says whether the fp16
// tile instance skipped a tile.
int64_t v16_region_bytes(const lkv_prefill_args* a, int64_t vblocks) {
  const int64_t heads = static_cast<int64_t>(a->batch) * a->num_kv_heads;
  return heads * vblocks * (lkv::kBlockElems * 2) + heads * ((vblocks + 15) / 16 * 16) + 16;
}

}  // namespace

namespace {

// The tile kernel's plan for a call: waves per workgroup, tiles per (sequence, kv head), the grid,
// and the key splits it would take with room for their states.  Each wave takes 32 query rows.
// Short calls (<= 64 rows per kv head) would take 2 waves (with tile_waves 0 they run on the decode
// kernel instead).  Otherwise 8 waves (two per SIMD, one workgroup per CU), or 4 waves (two
// workgroups per CU) when the 4-wave grid still leaves at most one workgroup per CU, which keeps
// twice the CUs busy (measured on 256 CUs: at B = 1 of a config-3 piece 23 vs 18 %; from B = 2 up
// the 8-wave tile is 0.5-1.5 points ahead).  A ragged call takes 4-wave tiles (the host does not
// know how many of its sequences are long, and a step of decode rows and one or two prefill pieces
// would leave half the CUs idle with 8-wave tiles) over a grid of at most ceil(T * G / rows_per_wg)
// + B tiles per kv head.  A grid of fewer 4-wave workgroups than two per CU, or of 8-wave ones for
// at most half the CUs, splits each tile's keys over up to 4 workgroups when the call has an older
// segment and leaves the split counts to the library (num_splits 0): a 1024-token piece of one
// sequence over 8K keys runs 256 4-wave workgroups, one wave per SIMD, and its key splits let a
// second workgroup share each CU.
struct TilePlan {
  bool runs;          // the tile kernel runs (some sequence has > 64 rows per kv head, or tile_waves)
  int waves;
  int64_t tiles, wgs, rows_all;  // rows_all: the output rows (B * L, or T ragged)
  int splits;         // key splits with room for their states
};

TilePlan tile_plan(const lkv_prefill_args* a) {
  using namespace lkv;
  TilePlan t{};
  const bool ragged = a->cu_seqlens_q != nullptr;
  const int group = a->num_q_heads / a->num_kv_heads;
  const int64_t seq_tokens = ragged ? std::min(a->max_seqlen_q, a->tokens) : a->tokens;
  const int64_t rows = seq_tokens * group;
  const int64_t heads = static_cast<int64_t>(a->num_kv_heads) * a->batch;
  t.runs = rows > 64 || a->tile_waves != 0;
  const bool wide = rows > 64;
  t.waves = wide ? 8 : 2;
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  if (wide && a->tile_waves != 0) {
    t.waves = a->tile_waves;
  } else if (wide && ragged) {
    t.waves = 4;
  } else if (wide) {
    const int64_t wgs4 = (rows + 127) / 128 * heads;
    if (wgs4 <= cus) t.waves = 4;
  }
  const int64_t rows_per_wg = t.waves * 32;
  t.tiles = (rows + rows_per_wg - 1) / rows_per_wg;
  const int64_t ragged_tiles = (static_cast<int64_t>(a->tokens) * group + rows_per_wg - 1) / rows_per_wg;
  t.wgs = ragged ? (ragged_tiles + a->batch) * a->num_kv_heads : t.tiles * heads;
  t.rows_all = ragged ? a->tokens : static_cast<int64_t>(a->batch) * a->tokens;
  t.splits = 1;
  const int64_t est = ragged ? ragged_tiles * a->num_kv_heads : t.wgs;  // the tiles that work
  // 4-wave tiles: below two workgroups per CU; 8-wave tiles (one per CU): at most half the CUs busy
  const bool idle = t.waves == 4 ? est < 2 * cus : (t.waves == 8 && est * 2 <= cus);
  if (t.runs && idle && a->num_splits == 0 && a->older_k != nullptr && est > 0) {
    // enough splits to fill the CUs' workgroup slots, rounded up to a power of two (a 768-token call
    // of one sequence, 32 query and 8 kv heads, over 8K keys: 192 4-wave tiles; 3 splits 156 us,
    // 4 splits 134 us, 2 splits 147 us)
    int64_t want = (cus * (t.waves == 4 ? 2 : 1) + est - 1) / est;
    int64_t pow2 = 1;
    while (pow2 < want) pow2 *= 2;
    t.splits = static_cast<int>(std::min<int64_t>(kMaxTileSplits, pow2));
  }
  if (t.splits > 1 && a->older_len == nullptr && (a->local_k == nullptr || a->local_len == nullptr)) {
    // host-constant lengths: as many equal splits as start inside the older segment for the last
    // tile (the kernel applies the same rule per tile; a grid of splits that would all be empty
    // would only cost their launch and the merge)
    const int64_t nb0 = (std::min<int64_t>(std::max(a->older_len_const, 0), a->older_capacity_tokens) + kBlockTokens - 1) /
                        kBlockTokens;
    const int64_t lead = a->local_start ? kBlockTokens - 1 : (a->local_start_const & (kBlockTokens - 1));
    const int64_t n1 = a->local_k == nullptr ? 0 : std::max(a->local_len_const, 0);
    const int64_t nbt = nb0 + (n1 > 0 ? (lead + n1 + kBlockTokens - 1) / kBlockTokens : 0);
    while (t.splits > 1 && (t.splits - 1) * ((nbt + t.splits - 1) / t.splits) > nb0 - 1) --t.splits;
  }
  return t;
}

// Bytes of the key splits' states: fp32 O and LSE per (output row, query head, split).
int64_t tile_split_bytes(const lkv_prefill_args* a, const TilePlan& t, int splits) {
  return splits > 1 ? t.rows_all * a->num_q_heads * splits * (lkv::kHeadDim + 1) * 4 : 0;
}

// A ragged call's plan from the host copy of its offsets (cu_seqlens_q_host): the number of its
// sequences in each decode-kernel column class (1-16, 17-32, 33-64 columns) and whether any has
// more rows per kv head, counted as the kernels count them (offsets clamped into [0, tokens],
// counts to max_seqlen_q).
struct HostPlan {
  bool known;
  int32_t class_n[3];
  bool any_tile;
};

HostPlan host_plan(const lkv_prefill_args* a, int64_t group) {
  HostPlan h{};
  const int32_t* cu = a->cu_seqlens_q_host;
  if (a->cu_seqlens_q == nullptr || cu == nullptr) return h;
  h.known = true;
  const int32_t lmax = std::min(a->max_seqlen_q, a->tokens);
  for (int32_t b = 0; b < a->batch; ++b) {
    const int32_t s0 = std::min(std::max(cu[b], 0), a->tokens);
    const int32_t L = std::min(std::min(std::max(cu[b + 1], s0), a->tokens) - s0, lmax);
    if (L <= 0) continue;
    const int64_t cols = L * group;
    if (cols > 64)
      h.any_tile = true;
    else
      ++h.class_n[cols <= 16 ? 0 : cols <= 32 ? 1 : 2];
  }
  return h;
}

// Whether a ragged call runs its sequences of at most 64 query rows per kv head on the decode kernel:
// with tile_waves 0, and with tile_waves 4 or 8 too when its longest sequence has more rows.  The 4-
// and 8-wave tiles carry each probability as one fp16, whose rel-L2 over a short sequence's few
// outputs can pass 1e-3; only a call of short sequences alone takes the 2-wave tiles (fp16 hi + lo).
bool ragged_short_on_decode(const lkv_prefill_args* a) {
  if (a->cu_seqlens_q == nullptr) return false;
  const int64_t group = a->num_q_heads / a->num_kv_heads;
  return a->tile_waves == 0 || std::min(a->max_seqlen_q, a->tokens) * group > 64;
}

// The workspace a call cannot run without: the V pre-pass's region, or the decode kernel's split
// states if larger (they are used before the pre-pass runs, in the same bytes).
int64_t min_workspace_bytes(const lkv_prefill_args* a) {
  using namespace lkv;
  const int64_t v16 = v16_region_bytes(a, v16_blocks(a));
  const int64_t per_row = (kHeadDim + 2) * 4;  // one split state
  if (ragged_short_on_decode(a) && a->max_seqlen_q >= 1 && a->tokens > 0) {
    // a ragged call's decode-kernel classes: split states of their sequences, by rank in the class
    const int group = a->num_q_heads / a->num_kv_heads;
    const int L = std::min(a->max_seqlen_q, a->tokens);
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int cap = std::min(kRaggedSplitCap, std::max(1, cus / a->num_kv_heads));
    int64_t states = 0;
    for (const int col_hi : {16, 32, 64}) {
      const int lmax = std::min(col_hi / std::max(group, 1), L);
      if (lmax >= 1)
        states = std::max(states, ragged_split_state_rows(a->batch, a->num_q_heads, a->num_kv_heads, lmax, cap,
                                                          a->num_splits, cus));
    }
    return std::max(v16, states * per_row);
  }
  if (a->num_splits <= 1) return v16;
  // split states of the decode kernel's sequences: [B, L, Hq] rows
  return std::max(v16, static_cast<int64_t>(a->batch) * std::max(a->tokens, 0) * a->num_q_heads * a->num_splits * per_row);
}

}  // namespace

extern "C" int64_t lkv_prefill_workspace_bytes(const lkv_prefill_args* a) {
  using namespace lkv;
  if (a == nullptr || a->batch <= 0 || a->num_kv_heads <= 0 || a->num_q_heads <= 0) return 0;
  const TilePlan t = tile_plan(a);
  // the tile kernel's key-split states follow the V pre-pass's region
  return std::max(min_workspace_bytes(a), v16_region_bytes(a, v16_blocks(a)) + tile_split_bytes(a, t, t.splits));
}

extern "C" int64_t lkv_prefill_workspace_min_bytes(const lkv_prefill_args* a) {
  if (a == nullptr || a->batch <= 0 || a->num_kv_heads <= 0 || a->num_q_heads <= 0) return 0;
  return min_workspace_bytes(a);
}

// The tile kernel instance for this call's wave count and addressing.
void launch_tiles(int waves, bool paged, dim3 grid, const lkv::PrefillParams& p, hipStream_t s) {
  using namespace lkv;
  if (waves == 8 && paged)
    prefill_kernel<8, 2, 2, true><<<grid, 8 * 64, 0, s>>>(p);
  else if (waves == 8)
    prefill_kernel<8, 2, 2, false><<<grid, 8 * 64, 0, s>>>(p);
  else if (waves == 4 && paged)
    prefill_kernel<4, 2, 2, true><<<grid, 4 * 64, 0, s>>>(p);
  else if (waves == 4)
    prefill_kernel<4, 2, 2, false><<<grid, 4 * 64, 0, s>>>(p);
  else if (paged)
    prefill_kernel<2, 2, 1, true><<<grid, 2 * 64, 0, s>>>(p);
  else
    prefill_kernel<2, 2, 1, false><<<grid, 2 * 64, 0, s>>>(p);
}

// The wide-range V instance for the same wave count and addressing, over `pair_wgs` workgroups
// (4-wave tiles at one wave per SIMD: the bf16 instance needs more than 256 registers).
void launch_wide(int waves, bool paged, int pair_wgs, const lkv::PrefillParams& p, hipStream_t s) {
  using namespace lkv;
  const dim3 grid(static_cast<unsigned>(pair_wgs));
  if (waves == 8 && paged)
    prefill_wide_kernel<8, 2, 2, true><<<grid, 8 * 64, 0, s>>>(p);
  else if (waves == 8)
    prefill_wide_kernel<8, 2, 2, false><<<grid, 8 * 64, 0, s>>>(p);
  else if (waves == 4 && paged)
    prefill_wide_kernel<4, 2, 1, true><<<grid, 4 * 64, 0, s>>>(p);
  else if (waves == 4)
    prefill_wide_kernel<4, 2, 1, false><<<grid, 4 * 64, 0, s>>>(p);
  else if (paged)
    prefill_wide_kernel<2, 2, 1, true><<<grid, 2 * 64, 0, s>>>(p);
  else
    prefill_wide_kernel<2, 2, 1, false><<<grid, 2 * 64, 0, s>>>(p);
}

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
  LKV_REQUIRE(a->tile_waves == 0 || a->tile_waves == 4 || a->tile_waves == 8, "tile_waves must be 0, 4 or 8, got %d",
              a->tile_waves);
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->older_vscale_mode == 1, "older_vscale_mode must be 0 or 1");
  LKV_REQUIRE(a->older_vscale_mode == 0 || a->vscale != nullptr, "older_vscale_mode 1 needs vscale");
  LKV_REQUIRE(a->q != nullptr && a->out != nullptr, "null q/out");
  const bool ragged = a->cu_seqlens_q != nullptr;
  LKV_REQUIRE(!ragged || a->tokens == 0 || a->max_seqlen_q >= 1, "ragged calls need max_seqlen_q >= 1, got %d",
              a->max_seqlen_q);
  LKV_REQUIRE(a->num_splits >= 0 && a->num_splits <= 1024, "num_splits must be in [0, 1024], got %d", a->num_splits);
  LKV_REQUIRE((a->q_stride_b % 8) == 0 && (a->q_stride_t % 8) == 0 && (reinterpret_cast<uintptr_t>(a->q) & 15) == 0,
              "q rows must be 16-byte aligned");
  LKV_REQUIRE((a->out_stride_b % 4) == 0 && (a->out_stride_t % 4) == 0 && (reinterpret_cast<uintptr_t>(a->out) & 7) == 0,
              "out rows must be 8-byte aligned");
  // causal = 1 masks the local segment bottom-right, the queries' own keys being its last `tokens`
  // tokens; a non-empty local segment shorter than that would need the mask to reach into the older
  // segment (without a local segment, or with an empty one, the older segment is fully visible)
  LKV_REQUIRE(ragged || a->causal == 0 || a->local_k == nullptr || a->local_len != nullptr || a->local_len_const <= 0 ||
                  a->local_len_const >= a->tokens,
              "causal calls need local_len >= tokens (the queries' own keys end the local segment), got %d < %d",
              a->local_len_const, a->tokens);
  PrefillParams p;
  if (const int32_t st = fill_segments(a, p.seg)) return st;
  LKV_REQUIRE(a->batch <= 65535 && a->num_kv_heads <= 65535, "batch and num_kv_heads must be <= 65535");
  if (a->batch == 0 || a->tokens == 0) return LKV_OK;
  // query tokens per sequence (ragged: an upper bound)
  const int64_t seq_tokens = ragged ? std::min(a->max_seqlen_q, a->tokens) : a->tokens;
  const int64_t vblocks = v16_blocks(a);
  const int64_t need = min_workspace_bytes(a);
  LKV_REQUIRE(vblocks * kBlockElems * 2 < (1LL << 31), "too many key blocks per sequence");
  LKV_REQUIRE(vblocks == 0 || (a->workspace != nullptr && a->workspace_bytes >= need),
              "prefill needs a workspace of at least %lld bytes (lkv_prefill_workspace_bytes: %lld with the key "
              "splits' states), got %lld",
              static_cast<long long>(need), static_cast<long long>(lkv_prefill_workspace_bytes(a)),
              static_cast<long long>(a->workspace_bytes));
  LKV_REQUIRE((reinterpret_cast<uintptr_t>(a->workspace) & 15) == 0, "workspace must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  // Sequences of at most 64 query rows per kv head (e.g. decode tokens, or up to 16 tokens of a GQA
  // group of 4) read every key once on the decode kernel (one score column per (token, head))
  // instead of converting V to fp16 and running 2-wave tiles; tile_waves 4 or 8 keep a uniform call
  // on the tile kernel.  A ragged call runs its sequences of 1-16, 17-32 and 33-64 columns on the
  // decode instance of that width (one launch per class present) and the longer ones on the tile
  // kernel, also with tile_waves 4 or 8 unless all of its sequences are short.
  const int64_t max_cols = seq_tokens * group;
  const bool short_on_decode = a->tile_waves == 0 || ragged_short_on_decode(a);
  if (short_on_decode) {
    // (with the host copy of a ragged call's offsets: only the classes that hold a sequence)
    const HostPlan hp = host_plan(a, group);
    const int32_t bounds[4] = {0, 16, 32, 64};
    for (int c = 0; c < 3; ++c) {
      if (max_cols <= bounds[c]) break;
      // a uniform call is one class: the one its width falls in
      if (!ragged && max_cols > bounds[c + 1]) continue;
      if (hp.known && hp.class_n[c] == 0) continue;
      if (const int32_t st = prefill_on_decode_kernel(a, p.seg, group, bounds[c], bounds[c + 1],
                                                      hp.known ? hp.class_n[c] : -1, s))
        return st;
    }
    if (max_cols <= 64 || (hp.known && !hp.any_tile)) return LKV_OK;
  }
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_stride_b;
  p.q_st = a->q_stride_t;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_sb = a->out_stride_b;
  p.out_st = a->out_stride_t;
  p.lse = a->lse;
  p.vscale = a->vscale;
  p.out_scale = a->out_scale;
  p.L = static_cast<int32_t>(seq_tokens);
  p.hq = a->num_q_heads;
  p.group = group;
  p.causal = a->causal;
  p.scale_log2 = a->sm_scale * kLog2e;
  p.vscale_mode = a->older_vscale_mode;
  p.v16 = static_cast<uint16_t*>(a->workspace);
  p.v16_blocks = static_cast<int32_t>(vblocks);
  p.vflag_stride = static_cast<int32_t>((vblocks + 15) / 16 * 16);
  p.vflags = static_cast<uint8_t*>(a->workspace) + static_cast<int64_t>(a->batch) * a->num_kv_heads * vblocks * (kBlockElems * 2);
  p.any_wide = reinterpret_cast<float*>(p.vflags + static_cast<int64_t>(a->batch) * a->num_kv_heads * p.vflag_stride);
  p.cu = a->cu_seqlens_q;
  p.rows = a->tokens;
  p.decode_rows = ragged && short_on_decode ? 64 : -1;
  const int64_t heads = static_cast<int64_t>(a->num_kv_heads) * a->batch;
  const TilePlan plan = tile_plan(a);
  const int waves = plan.waves;
  const int64_t tiles = plan.tiles, wgs = plan.wgs;
  // key splits: as many as the workspace holds the states of (1 without room)
  int splits = plan.splits;
  const int64_t v16_bytes = v16_region_bytes(a, vblocks);
  while (splits > 1 && v16_bytes + tile_split_bytes(a, plan, splits) > a->workspace_bytes) --splits;
  if (vblocks == 0) splits = 1;
  LKV_REQUIRE(wgs * splits < (1LL << 31), "too many query rows");
  p.tile_splits = splits;
  p.ws_o = splits > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(a->workspace) + v16_bytes) : nullptr;
  p.ws_lse = splits > 1 ? p.ws_o + plan.rows_all * a->num_q_heads * splits * kHeadDim : nullptr;
  p.tiles = static_cast<int32_t>(tiles);
  p.hkv = a->num_kv_heads;
  p.batch = a->batch;
  const bool paged = a->older_block_table != nullptr || a->local_block_table != nullptr;
  if (vblocks > 0) {  // (no keys at all: every row's output is zero; the main kernel skips its loop)
    const int per_wg = ragged ? 8 : 1;
    const dim3 vgrid(static_cast<unsigned>((vblocks + per_wg - 1) / per_wg), a->num_kv_heads,
                     ragged ? std::min(a->batch, 4) : a->batch);
    if (paged && ragged)
      v16_stage_kernel<true, 8><<<vgrid, 256, 0, s>>>(p);
    else if (paged)
      v16_stage_kernel<true, 1><<<vgrid, 256, 0, s>>>(p);
    else if (ragged)
      v16_stage_kernel<false, 8><<<vgrid, 256, 0, s>>>(p);
    else
      v16_stage_kernel<false, 1><<<vgrid, 256, 0, s>>>(p);
    if (const int32_t e = check_launch("lkv_prefill_attn (V pre-pass)")) return e;
  }
  const dim3 grid(static_cast<unsigned>(wgs * splits));
  launch_tiles(waves, paged, grid, p, s);
  if (const int32_t e = check_launch("lkv_prefill_attn")) return e;
  if (vblocks == 0) return LKV_OK;
  // the tiles that read a V value of magnitude 65536 or more (flagged by the pre-pass; the instance
  // above skipped them), exactly in bf16, by workgroups that each scan one (sequence, kv head)'s
  // flags at a time
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  launch_wide(waves, paged, static_cast<int>(std::min(heads, cus)), p, s);
  if (const int32_t e = check_launch("lkv_prefill_attn (wide-range V)")) return e;
  if (splits == 1) return LKV_OK;
  const int64_t items = plan.rows_all * a->num_q_heads;  // (row, query head) pairs, 4 per workgroup
  LKV_REQUIRE((items + 3) / 4 < (1LL << 31), "too many query rows");
  prefill_split_combine_kernel<<<static_cast<unsigned>((items + 3) / 4), 256, 0, s>>>(p, plan.rows_all);
  return check_launch("lkv_prefill_attn (key-split merge)");
}

// Shared device helpers for the gfx950 LastKV kernels.
//
// Cache layout ("tiled", one 32-token block = 4096 bf16 = 8 KiB per (sequence, kv head)):
//   K block: element (w, d), w = token in block, d = head dim, is stored at
//            ((u * 4 + kb) * 16 + r) * 32 + (d & 31)
//            with kb = d >> 5, u = (w >> 2) & 1, r = ((w >> 3) << 2) | (w & 3).
//            A wave reads a 16-token x 32-dim MFMA operand tile as one contiguous 1 KiB run.
//   V block: element (w, d) is stored at d * 32 + w (the block is V transposed),
//            so the PV operand (8 consecutive tokens of one dim per lane) is a 16-byte load.
// The token permutation inside K tiles makes the QK^T accumulator of lane (n, g) hold
// exactly the tokens 8g..8g+7 that the PV MFMA wants as its A operand in that lane, so
// the probabilities never cross lanes.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lkv {

constexpr int kHeadDim = 128;
constexpr int kBlockTokens = 32;
constexpr int kBlockElems = kBlockTokens * kHeadDim;  // 4096
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte global load with the non-temporal hint, for data read once per launch.  On gfx950 a read
// stream of such loads sustains ~7.1 TB/s against ~6.3 TB/s with the default cache policy.
__device__ inline uint4 load_nt(const void* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}

__host__ __device__ inline int k_tile_offset(int w, int d) {
  const int u = (w >> 2) & 1;
  const int r = ((w >> 3) << 2) | (w & 3);
  const int kb = d >> 5;
  return ((u * 4 + kb) * 16 + r) * 32 + (d & 31);
}

__host__ __device__ inline int v_tile_offset(int w, int d) { return d * 32 + w; }

__device__ inline float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ inline float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ inline float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950), NaN preserved.
__device__ inline uint16_t f32_to_bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

// Both halves rounded by one v_cvt_pk_bf16_f32 (NaN preserved).
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}

__device__ inline bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

__device__ inline f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ inline f32x4 mfma_f16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// IEEE-754 maximum (NaN-propagating): one v_maximum3_f32 for up to three inputs and no NaN
// quieting instructions, unlike fmaxf in IEEE mode.
__device__ inline float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ inline float fmax3_nan(float a, float b, float c) { return fmax_nan(fmax_nan(a, b), c); }

// Reductions over the four 16-lane rows of a wave (lanes n, n+16, n+32, n+48) with the gfx950
// VALU lane swaps: permlane16_swap(x, x) yields rows (0,0,2,2) and (1,1,3,3), permlane32_swap(x, x)
// yields the lower and the upper half on both halves.  No LDS traffic, no bpermute latency.
__device__ inline float wave_max_across_rows(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = fmax_nan(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmax_nan(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ inline float wave_sum_across_rows(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Workgroup id -> logical work index such that consecutive logical indices run on the same XCD:
// the dispatcher hands workgroup i to XCD i % 8, so logical ranges [x * n / 8, (x + 1) * n / 8)
// land on XCD x and tiles that share K/V share that XCD's L2.
__device__ inline int xcd_logical_index(int id, int n) {
  constexpr int kXcds = 8;
  const int xcd = id % kXcds, k = id / kXcds;
  const int q = n / kXcds, r = n % kXcds;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
}

}  // namespace lkv

// Achievable-peak probes of the part the library runs on: the rates the hot-path kernels are
// compared with beside the nominal peaks (8 TB/s HBM, 2.5 PFLOP/s dense bf16).
//
// probe_read_kernel: the decode kernel's access pattern at its best -- 16-byte non-temporal loads,
// every load instruction of a wave one contiguous 1 KiB run, 8 loads in flight per thread over a
// grid-stride walk of the buffer.
// probe_mfma_kernel: independent 16x16x32 bf16 MFMA chains, 8 per wave, whose operands change from
// one MFMA to the next (pseudo-random bf16 values of magnitude [0.5, 1) with random signs, the
// bit activity of N(0, 1) data), so the matrix pipe draws the power it draws on real data.
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr int kProbeThreads = 256;

__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const uint4* src, int64_t n16, uint32_t* sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = load_nt(src + i + j * stride);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = load_nt(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

__device__ inline uint32_t xorshift(uint32_t& x) {
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  return x;
}

// Two bf16 values of magnitude [0.5, 1) with random mantissas and signs.
__device__ inline uint32_t random_bf16x2(uint32_t& x) { return (xorshift(x) & 0x807f807fu) | 0x3f003f00u; }

__global__ __launch_bounds__(kProbeThreads) void probe_mfma_kernel(uint32_t* sink, int32_t iters, uint32_t seed) {
  constexpr int kChains = 8;
  uint32_t x = seed ^ ((blockIdx.x * kProbeThreads + threadIdx.x + 1) * 0x9e3779b9u);
  uint4 a[kChains], b[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
    a[c] = make_uint4(random_bf16x2(x), random_bf16x2(x), random_bf16x2(x), random_bf16x2(x));
    b[c] = make_uint4(random_bf16x2(x), random_bf16x2(x), random_bf16x2(x), random_bf16x2(x));
  }
  f32x4 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; it += 8) {
    // round it + k: chain c multiplies a[c] by b[(c + k) mod 8], so consecutive MFMAs never repeat
    // an operand pair (all indices compile-time: the operands stay in registers)
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int c = 0; c < kChains; ++c) acc[c] = mfma_bf16(a[c], b[(c + k) & 7], acc[c]);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += (acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3]);
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = __float_as_uint(s);
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_probe_read(const void* src, int64_t bytes, uint32_t* sink, int32_t workgroups,
                                  lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(src != nullptr && sink != nullptr, "null pointer");
  LKV_REQUIRE(bytes > 0 && bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0,
              "src must be 16-byte aligned and bytes a positive multiple of 16");
  LKV_REQUIRE(workgroups > 0 && workgroups <= 65536, "workgroups must be in [1, 65536]");
  probe_read_kernel<<<workgroups, kProbeThreads, 0, as_stream(stream)>>>(static_cast<const uint4*>(src), bytes / 16, sink);
  return check_launch("lkv_probe_read");
}

extern "C" int32_t lkv_probe_mfma(uint32_t* sink, int32_t workgroups, int32_t iters, uint32_t seed, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(sink != nullptr, "null sink");
  LKV_REQUIRE(workgroups > 0 && workgroups <= 65536, "workgroups must be in [1, 65536]");
  LKV_REQUIRE(iters > 0 && iters <= (1 << 24) && iters % 8 == 0, "iters must be a positive multiple of 8 up to 2^24");
  probe_mfma_kernel<<<workgroups, kProbeThreads, 0, as_stream(stream)>>>(sink, iters, seed);
  return check_launch("lkv_probe_mfma");
}

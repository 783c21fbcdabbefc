// Row-wise RMSNorm with an optional fused residual add, and the SwiGLU product, for the decoder
// layers of the serving path (the roles of vLLM's fused_add_rms_norm and silu_and_mul around the
// attention backend).  Both keep the rounding points of the torch expressions they replace, so a
// row computed here differs from torch's only where torch's own reduction order would.
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxHidden = 16384;  // 8 chunks of 8 elements per thread
constexpr int kNormChunks = kNormMaxHidden / (kNormThreads * 8);

struct NormParams {
  const uint16_t* x;
  int64_t x_stride;
  uint16_t* residual;
  int64_t res_stride;
  const uint16_t* w;
  uint16_t* out;
  int64_t out_stride;
  int32_t hidden;
  float eps;
};

__device__ inline void unpack8(uint4 u, float (&f)[8]) {
  f[0] = bf16_lo(u.x);
  f[1] = bf16_hi(u.x);
  f[2] = bf16_lo(u.y);
  f[3] = bf16_hi(u.y);
  f[4] = bf16_lo(u.z);
  f[5] = bf16_hi(u.z);
  f[6] = bf16_lo(u.w);
  f[7] = bf16_hi(u.w);
}

__device__ inline uint4 pack8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// One workgroup per row; thread t owns the 8-element chunks t, t + 256, ...  With kAdd the row is
// residual := bf16(residual + x) first (torch's bf16 add) and the normalised row is that sum.
// Then, as transformers' LlamaRMSNorm: h = float(row); r = rsqrt(sum(h^2) * (1 / hidden) + eps);
// out = bf16(w * bf16(h * r)).
template <bool kAdd>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const NormParams p) {
  __shared__ float part[kNormThreads / 64];
  const int row = blockIdx.x;
  const int chunks = p.hidden >> 3;
  const uint4* x = reinterpret_cast<const uint4*>(p.x + row * p.x_stride);
  uint4* res = kAdd ? reinterpret_cast<uint4*>(p.residual + row * p.res_stride) : nullptr;
  float v[kNormChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormChunks; ++k) {
    const int c = threadIdx.x + k * kNormThreads;
    if (c < chunks) {
      unpack8(x[c], v[k]);
      if (kAdd) {
        float r[8];
        unpack8(res[c], r);
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] += v[k][j];
        const uint4 s = pack8(r);
        res[c] = s;
        unpack8(s, v[k]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(v[k][j], v[k][j], ss);
    }
  }
  // row sum: within the wave (DPP through the shuffle builtins), then across the 4 waves
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = rsqrtf(total * (1.f / static_cast<float>(p.hidden)) + p.eps);
  const uint4* w = reinterpret_cast<const uint4*>(p.w);
  uint4* out = reinterpret_cast<uint4*>(p.out + row * p.out_stride);
#pragma unroll
  for (int k = 0; k < kNormChunks; ++k) {
    const int c = threadIdx.x + k * kNormThreads;
    if (c < chunks) {
      float h[8], wf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = v[k][j] * r;
      unpack8(pack8(h), h);  // h.to(bf16)
      unpack8(w[c], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = wf[j] * h[j];
      out[c] = pack8(h);
    }
  }
}

// out = bf16(bf16(silu(gate)) * up), silu(g) = g / (1 + exp(-g)) in fp32 as torch's kernel
// evaluates it; one thread per 8 elements.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gate, int64_t g_stride, const uint16_t* up,
                                                       int64_t u_stride, uint16_t* out, int64_t o_stride, int32_t rows,
                                                       int32_t width) {
  const int chunks = width >> 3;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(rows) * chunks) return;
  const int row = static_cast<int>(i / chunks), c = static_cast<int>(i - static_cast<int64_t>(row) * chunks);
  float g[8], u[8];
  unpack8(reinterpret_cast<const uint4*>(gate + row * g_stride)[c], g);
  unpack8(reinterpret_cast<const uint4*>(up + row * u_stride)[c], u);
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = g[j] / (1.f + expf(-g[j]));
  unpack8(pack8(g), g);  // silu's bf16 result
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] *= u[j];
  reinterpret_cast<uint4*>(out + row * o_stride)[c] = pack8(g);
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_rmsnorm(const lkv_rmsnorm_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_rmsnorm_args)),
              "lkv_rmsnorm_args size mismatch (caller %d, library %d)", a->struct_size,
              static_cast<int32_t>(sizeof(lkv_rmsnorm_args)));
  LKV_REQUIRE(a->rows >= 0, "rows must be non-negative");
  LKV_REQUIRE(a->hidden > 0 && a->hidden % 8 == 0 && a->hidden <= kNormMaxHidden,
              "hidden must be a positive multiple of 8 up to %d, got %d", kNormMaxHidden, a->hidden);
  LKV_REQUIRE(a->x != nullptr && a->weight != nullptr && a->out != nullptr, "null x/weight/out");
  const uintptr_t align = reinterpret_cast<uintptr_t>(a->x) | reinterpret_cast<uintptr_t>(a->weight) |
                          reinterpret_cast<uintptr_t>(a->out) | reinterpret_cast<uintptr_t>(a->residual);
  LKV_REQUIRE((align & 15) == 0, "rows must be 16-byte aligned");
  LKV_REQUIRE((a->x_stride | a->out_stride | a->residual_stride) % 8 == 0, "row strides must be multiples of 8 elements");
  if (a->rows == 0) return LKV_OK;
  NormParams p;
  p.x = static_cast<const uint16_t*>(a->x);
  p.x_stride = a->x_stride;
  p.residual = static_cast<uint16_t*>(a->residual);
  p.res_stride = a->residual_stride;
  p.w = static_cast<const uint16_t*>(a->weight);
  p.out = static_cast<uint16_t*>(a->out);
  p.out_stride = a->out_stride;
  p.hidden = a->hidden;
  p.eps = a->eps;
  hipStream_t s = as_stream(stream);
  if (a->residual != nullptr)
    rmsnorm_kernel<true><<<a->rows, kNormThreads, 0, s>>>(p);
  else
    rmsnorm_kernel<false><<<a->rows, kNormThreads, 0, s>>>(p);
  return check_launch("lkv_rmsnorm");
}

extern "C" int32_t lkv_silu_mul(const void* gate, int64_t gate_stride, const void* up, int64_t up_stride, void* out,
                                int64_t out_stride, int32_t rows, int32_t width, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(gate != nullptr && up != nullptr && out != nullptr, "null gate/up/out");
  LKV_REQUIRE(rows >= 0 && width > 0 && width % 8 == 0, "width must be a positive multiple of 8");
  const uintptr_t align = reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(out);
  LKV_REQUIRE((align & 15) == 0, "rows must be 16-byte aligned");
  LKV_REQUIRE((gate_stride | up_stride | out_stride) % 8 == 0, "row strides must be multiples of 8 elements");
  const int64_t threads = static_cast<int64_t>(rows) * (width / 8);
  LKV_REQUIRE(threads / 256 < (1LL << 31), "too many elements");
  if (threads == 0) return LKV_OK;
  silu_mul_kernel<<<static_cast<unsigned>((threads + 255) / 256), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(gate), gate_stride, static_cast<const uint16_t*>(up), up_stride,
      static_cast<uint16_t*>(out), out_stride, rows, width);
  return check_launch("lkv_silu_mul");
}

// Conversion between [B, H, T, 128] bf16 tensors and the tiled K/V cache layout.
// These run off the hot path (cache import/export, inspection, tests); one thread moves one
// 8-element run, which is a 16-byte store on the K side and a 16-byte load on the V side.
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

// Tiled offset of cache token t (absolute within the (seq, head) run), dim d.
__device__ inline int64_t tiled_offset(int kind, int t, int d) {
  const int64_t block = t >> 5;
  const int w = t & 31;
  return block * kBlockElems + (kind == 0 ? k_tile_offset(w, d) : v_tile_offset(w, d));
}

template <bool kPack>
__global__ void convert_kernel(const uint16_t* __restrict__ a, int64_t a_sb, int64_t a_sh, int64_t a_st,
                               uint16_t* __restrict__ cache, int64_t c_ss, int64_t c_hs, int32_t token0,
                               int32_t batch, int32_t heads, int32_t tokens, int32_t kind) {
  // work item = (b, h, t, 8-dim group)
  const int64_t total = static_cast<int64_t>(batch) * heads * tokens * (kHeadDim / 8);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int dg = static_cast<int>(i % (kHeadDim / 8));
    int64_t rest = i / (kHeadDim / 8);
    const int t = static_cast<int>(rest % tokens);
    rest /= tokens;
    const int h = static_cast<int>(rest % heads);
    const int b = static_cast<int>(rest / heads);
    const uint16_t* arow = a + b * a_sb + h * a_sh + t * a_st + dg * 8;
    uint16_t* crow = cache + b * c_ss + h * c_hs;
    const int ct = token0 + t;
    if (kPack) {
      const uint4 v = *reinterpret_cast<const uint4*>(arow);
      const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
      if (kind == 0) {
        *reinterpret_cast<uint4*>(crow + tiled_offset(0, ct, dg * 8)) = v;
      } else {
        for (int j = 0; j < 8; ++j) crow[tiled_offset(1, ct, dg * 8 + j)] = e[j];
      }
    } else {
      uint16_t* out = const_cast<uint16_t*>(arow);
      if (kind == 0) {
        *reinterpret_cast<uint4*>(out) = *reinterpret_cast<const uint4*>(crow + tiled_offset(0, ct, dg * 8));
      } else {
        uint4 v;
        uint16_t* e = reinterpret_cast<uint16_t*>(&v);
        for (int j = 0; j < 8; ++j) e[j] = crow[tiled_offset(1, ct, dg * 8 + j)];
        *reinterpret_cast<uint4*>(out) = v;
      }
    }
  }
}

int32_t validate(const void* a, int64_t a_st, const void* cache, int32_t batch, int32_t heads, int32_t tokens,
                 int32_t kind, int32_t token0, int32_t capacity) {
  LKV_REQUIRE(a != nullptr && cache != nullptr, "null tensor pointer");
  LKV_REQUIRE(batch >= 0 && heads >= 0 && tokens >= 0, "negative size");
  LKV_REQUIRE(kind == 0 || kind == 1, "kind must be 0 (K) or 1 (V), got %d", kind);
  LKV_REQUIRE(token0 >= 0 && capacity % kBlockTokens == 0, "capacity must be a multiple of 32 tokens");
  LKV_REQUIRE(static_cast<int64_t>(token0) + tokens <= capacity, "tokens [%d, %d) exceed the cache capacity %d",
              token0, token0 + tokens, capacity);
  LKV_REQUIRE((reinterpret_cast<uintptr_t>(a) & 15) == 0 && (a_st % 8) == 0,
              "tensor rows must be 16-byte aligned");
  LKV_REQUIRE((reinterpret_cast<uintptr_t>(cache) & 15) == 0, "cache must be 16-byte aligned");
  return LKV_OK;
}

int launch_blocks(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return static_cast<int>(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_cache_pack(const void* src, int64_t src_stride_b, int64_t src_stride_h, int64_t src_stride_t,
                                  int32_t batch, int32_t heads, int32_t tokens, int32_t kind, void* dst,
                                  int64_t dst_seq_stride, int64_t dst_head_stride, int32_t dst_token0,
                                  int32_t dst_capacity_tokens, lkv_stream_t stream) {
  using namespace lkv;
  if (int32_t st = validate(src, src_stride_t, dst, batch, heads, tokens, kind, dst_token0, dst_capacity_tokens))
    return st;
  LKV_REQUIRE((src_stride_b % 8) == 0 && (src_stride_h % 8) == 0, "tensor rows must be 16-byte aligned");
  const int64_t items = static_cast<int64_t>(batch) * heads * tokens * (kHeadDim / 8);
  if (items == 0) return LKV_OK;
  convert_kernel<true><<<launch_blocks(items), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(src), src_stride_b, src_stride_h, src_stride_t, static_cast<uint16_t*>(dst),
      dst_seq_stride, dst_head_stride, dst_token0, batch, heads, tokens, kind);
  return check_launch("lkv_cache_pack");
}

extern "C" int32_t lkv_cache_unpack(const void* src, int64_t src_seq_stride, int64_t src_head_stride,
                                    int32_t src_token0, int32_t src_capacity_tokens, int32_t batch, int32_t heads,
                                    int32_t tokens, int32_t kind, void* dst, int64_t dst_stride_b,
                                    int64_t dst_stride_h, int64_t dst_stride_t, lkv_stream_t stream) {
  using namespace lkv;
  if (int32_t st = validate(dst, dst_stride_t, src, batch, heads, tokens, kind, src_token0, src_capacity_tokens))
    return st;
  LKV_REQUIRE((dst_stride_b % 8) == 0 && (dst_stride_h % 8) == 0, "tensor rows must be 16-byte aligned");
  const int64_t items = static_cast<int64_t>(batch) * heads * tokens * (kHeadDim / 8);
  if (items == 0) return LKV_OK;
  convert_kernel<false><<<launch_blocks(items), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(dst), dst_stride_b, dst_stride_h, dst_stride_t,
      const_cast<uint16_t*>(static_cast<const uint16_t*>(src)), src_seq_stride, src_head_stride, src_token0, batch,
      heads, tokens, kind);
  return check_launch("lkv_cache_unpack");
}

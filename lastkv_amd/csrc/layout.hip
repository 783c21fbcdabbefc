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

// ---------------------------------------------------------------------------------------------
// Paged append: K/V rows -> pool pages.  One thread moves one (sequence, head, 8-token group,
// 8-dim group): eight 16-byte K stores, and for V an 8x8 register transpose so that each of the
// eight dims is one 16-byte store of 8 consecutive tokens (V tiles are dim-major).  Groups are
// 8-aligned in absolute positions; a ring wrap (a multiple of 32 tokens) keeps that alignment.
namespace lkv {
namespace {

struct AppendParams {
  const uint16_t* k;
  int64_t ksb, kst, ksh;
  const uint16_t* v;
  int64_t vsb, vst, vsh;
  uint16_t* pk;
  uint16_t* pv;
  int64_t page_stride, head_stride;
  const int32_t* table;
  int64_t table_stride;
  int32_t num_pages, token0, tokens, wrap, heads, groups;
};

__global__ __launch_bounds__(256) void append_paged_kernel(const AppendParams p, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int d8 = static_cast<int>(i & 15);
  int64_t rest = i >> 4;
  const int g = static_cast<int>(rest % p.groups);
  rest /= p.groups;
  const int h = static_cast<int>(rest % p.heads);
  const int b = static_cast<int>(rest / p.heads);
  const int a0 = ((p.token0 >> 3) + g) * 8;  // absolute position of the group's first token
  const int c0 = p.wrap > 0 ? a0 % p.wrap : a0;
  int page = p.table[b * p.table_stride + (c0 >> 5)];
  page = page < 0 ? 0 : (page >= p.num_pages ? p.num_pages - 1 : page);
  const int64_t base = page * p.page_stride + h * p.head_stride;
  const int w0 = c0 & 31;
  uint16_t vt[8][8];  // [token j][dim e]
  bool all = true;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int t = a0 + j - p.token0;
    const bool ok = t >= 0 && t < p.tokens;
    all = all && ok;
    uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
    if (ok) {
      kv = *reinterpret_cast<const uint4*>(p.k + b * p.ksb + t * p.kst + h * p.ksh + d8 * 8);
      vv = *reinterpret_cast<const uint4*>(p.v + b * p.vsb + t * p.vst + h * p.vsh + d8 * 8);
      *reinterpret_cast<uint4*>(p.pk + base + k_tile_offset(w0 + j, d8 * 8)) = kv;
    }
    const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vt[j][2 * e] = static_cast<uint16_t>(w[e] & 0xffffu);
      vt[j][2 * e + 1] = static_cast<uint16_t>(w[e] >> 16);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint16_t* dst = p.pv + base + v_tile_offset(w0, d8 * 8 + e);
    if (all) {
      uint4 o;
      o.x = vt[0][e] | (static_cast<uint32_t>(vt[1][e]) << 16);
      o.y = vt[2][e] | (static_cast<uint32_t>(vt[3][e]) << 16);
      o.z = vt[4][e] | (static_cast<uint32_t>(vt[5][e]) << 16);
      o.w = vt[6][e] | (static_cast<uint32_t>(vt[7][e]) << 16);
      *reinterpret_cast<uint4*>(dst) = o;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = a0 + j - p.token0;
        if (t >= 0 && t < p.tokens) dst[j] = vt[j][e];
      }
    }
  }
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_append_paged(const lkv_append_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_append_args)),
              "lkv_append_args size mismatch (caller %d, library %d)", a->struct_size,
              static_cast<int32_t>(sizeof(lkv_append_args)));
  LKV_REQUIRE(a->head_dim == kHeadDim, "head_dim must be 128, got %d", a->head_dim);
  LKV_REQUIRE(a->batch >= 0 && a->heads > 0 && a->tokens >= 0 && a->token0 >= 0, "bad sizes");
  LKV_REQUIRE(a->k && a->v && a->pool_k && a->pool_v && a->block_table, "null tensor");
  LKV_REQUIRE(a->num_pages > 0 && a->table_width > 0, "empty pool or table");
  LKV_REQUIRE(a->wrap_tokens >= 0 && a->wrap_tokens % kBlockTokens == 0, "wrap_tokens must be a multiple of 32");
  const int64_t cap = static_cast<int64_t>(a->table_width) * kBlockTokens;
  if (a->wrap_tokens > 0) {
    LKV_REQUIRE(a->tokens <= a->wrap_tokens && a->wrap_tokens <= cap,
                "a ring append needs tokens (%d) <= wrap_tokens (%d) <= 32 * table_width (%lld)", a->tokens,
                a->wrap_tokens, static_cast<long long>(cap));
  } else {
    LKV_REQUIRE(static_cast<int64_t>(a->token0) + a->tokens <= cap, "positions [%d, %d) exceed the table (%lld tokens)",
                a->token0, a->token0 + a->tokens, static_cast<long long>(cap));
  }
  const uintptr_t align = reinterpret_cast<uintptr_t>(a->k) | reinterpret_cast<uintptr_t>(a->v) |
                          reinterpret_cast<uintptr_t>(a->pool_k) | reinterpret_cast<uintptr_t>(a->pool_v);
  LKV_REQUIRE((align & 15) == 0, "tensors must be 16-byte aligned");
  LKV_REQUIRE(((a->k_stride_b | a->k_stride_t | a->k_stride_h | a->v_stride_b | a->v_stride_t | a->v_stride_h |
                a->page_stride | a->head_stride) & 7) == 0,
              "strides must be multiples of 8 elements");
  if (a->batch == 0 || a->tokens == 0) return LKV_OK;
  AppendParams p;
  p.k = static_cast<const uint16_t*>(a->k);
  p.ksb = a->k_stride_b;
  p.kst = a->k_stride_t;
  p.ksh = a->k_stride_h;
  p.v = static_cast<const uint16_t*>(a->v);
  p.vsb = a->v_stride_b;
  p.vst = a->v_stride_t;
  p.vsh = a->v_stride_h;
  p.pk = static_cast<uint16_t*>(a->pool_k);
  p.pv = static_cast<uint16_t*>(a->pool_v);
  p.page_stride = a->page_stride;
  p.head_stride = a->head_stride;
  p.table = a->block_table;
  p.table_stride = a->table_stride;
  p.num_pages = a->num_pages;
  p.token0 = a->token0;
  p.tokens = a->tokens;
  p.wrap = a->wrap_tokens;
  p.heads = a->heads;
  p.groups = ((a->token0 + a->tokens + 7) >> 3) - (a->token0 >> 3);
  const int64_t total = static_cast<int64_t>(a->batch) * a->heads * p.groups * 16;
  const int64_t blocks = (total + 255) / 256;
  LKV_REQUIRE(blocks < (1LL << 31), "too many elements");
  append_paged_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, as_stream(stream)>>>(p, total);
  return check_launch("lkv_append_paged");
}

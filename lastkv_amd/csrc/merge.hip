// Exact merge of two attention states over disjoint key sets (log-sum-exp merge).
//
// For each (token t, head h):
//   a = prefix output (optionally bf16(prefix * scale[h]) first), la = its natural-log LSE,
//   b = suffix output, lb = its LSE (an LSE of -inf marks an empty key set; +inf is read as -inf),
//   m = max(la, lb), wa = e^(la - m), wb = e^(lb - m),
//   out = (a wa + b wb) / (wa + wb),  out_lse = m + ln(wa + wb)
// computed in fp32, out rounded to bf16.  Both sets empty: out = 0, out_lse = -inf.
// Memory-bound: one thread per 8 output elements, 16-byte loads and stores.
#include "common.h"
#include "runtime.h"

namespace lkv {
namespace {

struct MergeParams {
  const uint16_t* pa;
  int64_t pa_st, pa_sh;
  const float* la;
  int64_t la_st, la_sh;
  const uint16_t* pb;
  int64_t pb_st, pb_sh;
  const float* lb;
  int64_t lb_st, lb_sh;
  const float* scale;
  uint16_t* out;
  int64_t o_st, o_sh;
  float* out_lse;
  int64_t ol_st, ol_sh;
  int32_t T, H, chunks;  // chunks = head_dim / 8
};

__device__ inline float lse_in(float x) { return x == __builtin_inff() ? -__builtin_inff() : x; }

__global__ __launch_bounds__(256) void merge_kernel(const MergeParams p) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(p.T) * p.H * p.chunks;
  if (i >= total) return;
  const int c = static_cast<int>(i % p.chunks);
  const int64_t th = i / p.chunks;
  const int h = static_cast<int>(th % p.H);
  const int64_t t = th / p.H;
  const float la = lse_in(p.la[t * p.la_st + h * p.la_sh]);
  const float lb = lse_in(p.lb[t * p.lb_st + h * p.lb_sh]);
  const float m = fmaxf(la, lb);
  const bool any = m != -__builtin_inff();
  // with both sets empty the weights are 0 and the output is 0
  const float wa = any ? fast_exp2((la - m) * kLog2e) : 0.f;
  const float wb = any ? fast_exp2((lb - m) * kLog2e) : 0.f;
  const float tot = wa + wb;
  const float inv = any ? 1.f / tot : 0.f;
  const float sa = wa * inv, sb = wb * inv;
  const uint4 a = *reinterpret_cast<const uint4*>(p.pa + t * p.pa_st + h * p.pa_sh + 8 * c);
  const uint4 b = *reinterpret_cast<const uint4*>(p.pb + t * p.pb_st + h * p.pb_sh + 8 * c);
  const float s = p.scale ? p.scale[h] : 1.f;
  auto mix = [&](uint32_t wa2, uint32_t wb2) -> uint32_t {
    float a0 = bf16_lo(wa2), a1 = bf16_hi(wa2);
    if (p.scale) {  // the reference scales the prefix output in bf16 before merging
      a0 = bf16_bits_to_f32(f32_to_bf16_bits(a0 * s));
      a1 = bf16_bits_to_f32(f32_to_bf16_bits(a1 * s));
    }
    return pack_bf16x2(a0 * sa + bf16_lo(wb2) * sb, a1 * sa + bf16_hi(wb2) * sb);
  };
  *reinterpret_cast<uint4*>(p.out + t * p.o_st + h * p.o_sh + 8 * c) =
      make_uint4(mix(a.x, b.x), mix(a.y, b.y), mix(a.z, b.z), mix(a.w, b.w));
  if (p.out_lse != nullptr && c == 0) p.out_lse[t * p.ol_st + h * p.ol_sh] = any ? m + __logf(tot) : -__builtin_inff();
}

}  // namespace
}  // namespace lkv

extern "C" int32_t lkv_merge_states(const lkv_merge_args* a, lkv_stream_t stream) {
  using namespace lkv;
  LKV_REQUIRE(a != nullptr, "null args");
  LKV_REQUIRE(a->struct_size == static_cast<int32_t>(sizeof(lkv_merge_args)),
              "lkv_merge_args size mismatch (caller %d, library %d)", a->struct_size,
              static_cast<int32_t>(sizeof(lkv_merge_args)));
  LKV_REQUIRE(a->tokens >= 0 && a->num_heads > 0, "bad sizes");
  LKV_REQUIRE(a->head_dim > 0 && a->head_dim % 8 == 0, "head_dim must be a positive multiple of 8");
  LKV_REQUIRE(a->prefix_out && a->prefix_lse && a->suffix_out && a->suffix_lse && a->out, "null tensor");
  const uintptr_t align = reinterpret_cast<uintptr_t>(a->prefix_out) | reinterpret_cast<uintptr_t>(a->suffix_out) |
                          reinterpret_cast<uintptr_t>(a->out);
  LKV_REQUIRE((align & 15) == 0, "outputs must be 16-byte aligned");
  LKV_REQUIRE(((a->prefix_out_stride_t | a->prefix_out_stride_h | a->suffix_out_stride_t | a->suffix_out_stride_h |
                a->out_stride_t | a->out_stride_h) & 7) == 0,
              "output strides must be multiples of 8 elements");
  if (a->tokens == 0) return LKV_OK;
  MergeParams p;
  p.pa = static_cast<const uint16_t*>(a->prefix_out);
  p.pa_st = a->prefix_out_stride_t;
  p.pa_sh = a->prefix_out_stride_h;
  p.la = a->prefix_lse;
  p.la_st = a->prefix_lse_stride_t;
  p.la_sh = a->prefix_lse_stride_h;
  p.pb = static_cast<const uint16_t*>(a->suffix_out);
  p.pb_st = a->suffix_out_stride_t;
  p.pb_sh = a->suffix_out_stride_h;
  p.lb = a->suffix_lse;
  p.lb_st = a->suffix_lse_stride_t;
  p.lb_sh = a->suffix_lse_stride_h;
  p.scale = a->prefix_scale;
  p.out = static_cast<uint16_t*>(a->out);
  p.o_st = a->out_stride_t;
  p.o_sh = a->out_stride_h;
  p.out_lse = a->out_lse;
  p.ol_st = a->out_lse_stride_t;
  p.ol_sh = a->out_lse_stride_h;
  p.T = a->tokens;
  p.H = a->num_heads;
  p.chunks = a->head_dim / 8;
  const int64_t total = static_cast<int64_t>(p.T) * p.H * p.chunks;
  const int64_t blocks = (total + 255) / 256;
  LKV_REQUIRE(blocks < (1LL << 31), "too many elements");
  merge_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, as_stream(stream)>>>(p);
  return check_launch("lkv_merge_states");
}

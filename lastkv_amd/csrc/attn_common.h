// Key-segment addressing shared by the decode and prefill attention kernels.
//
// A sequence's keys are the concatenation [older | local]:
//   older: tokens [0, n0) of the shared last-layer cache (tiled blocks 0, 1, ..., contiguous per
//          (slot, head) or listed in a page table);
//   local: n1 tokens of a ring of ring_blocks tiled blocks, starting at ring token lstart
//          (block lstart / 32, token lstart % 32) and wrapping at the ring's end (ring block rb
//          contiguous, or page ltab[rb] of a pool).
// Blocks are numbered over the concatenation: older blocks first, then local blocks.
#pragma once
#include "common.h"
#include "runtime.h"

namespace lkv {

struct BlockRef {
  const uint16_t* k;
  const uint16_t* v;
  int lo, hi;   // valid tokens [lo, hi) of the block
  int seg_tok;  // local segment index of token 0 of the block (older: -1)
  bool older;
};

// A segment is either contiguous (block j of the (slot, head) at j * kBlockElems) or paged: block j
// lives in page tab[j] of a pool, page stride `page` elements (page ids are clamped into
// [0, npages), so corrupt tables cannot address outside the pool).
struct SeqView {
  const uint16_t* ok;
  const uint16_t* ov;
  const uint16_t* lk;
  const uint16_t* lv;
  const int32_t* otab;  // this sequence's older page list, or nullptr
  const int32_t* ltab;  // this sequence's ring page list, or nullptr
  int64_t opage, lpage;
  int32_t onpages, lnpages;
  int n0, n1, nb0;
  int lblk0, lead;  // local segment: first ring block, first token inside it
  int ring_blocks;
};

__device__ inline int64_t page_offset(const int32_t* tab, int idx, int64_t page, int32_t npages) {
  if (tab == nullptr) return static_cast<int64_t>(idx) * kBlockElems;
  const int pg = min(max(tab[idx], 0), npages - 1);
  return static_cast<int64_t>(pg) * page;
}

// Ring block of local block j (the segment spans at most ring_blocks + 1 blocks).
__device__ inline int ring_block(const SeqView& s, int j) {
  const int rb = s.lblk0 + j;
  return rb >= s.ring_blocks ? rb - s.ring_blocks : rb;
}

// Element offset of block blk (older or local) inside its segment's (slot, head) or pool base.
// kMayPage = false compiles the contiguous addressing only (the caller has no page tables).
template <bool kMayPage = true>
__device__ inline int64_t block_offset(const SeqView& s, int blk) {
  if (!kMayPage)
    return static_cast<int64_t>(blk < s.nb0 ? blk : ring_block(s, blk - s.nb0)) * kBlockElems;
  return blk < s.nb0 ? page_offset(s.otab, blk, s.opage, s.onpages)
                     : page_offset(s.ltab, ring_block(s, blk - s.nb0), s.lpage, s.lnpages);
}

// Token range of block blk without its address (no page-table lookup).
__device__ inline BlockRef block_range(const SeqView& s, int blk) {
  const bool older = blk < s.nb0;
  const int j = blk - s.nb0;
  BlockRef r;
  r.k = nullptr;
  r.v = nullptr;
  r.lo = (older || j != 0) ? 0 : s.lead;
  r.hi = min(kBlockTokens, older ? s.n0 - blk * kBlockTokens : s.lead + s.n1 - j * kBlockTokens);
  r.seg_tok = older ? -1 : j * kBlockTokens - s.lead;
  r.older = older;
  return r;
}

__device__ inline BlockRef block_ref(const SeqView& s, int blk) {
  const bool older = blk < s.nb0;
  const int j = blk - s.nb0;
  const int64_t off = block_offset(s, blk);
  BlockRef r;
  r.k = (older ? s.ok : s.lk) + off;
  r.v = (older ? s.ov : s.lv) + off;
  r.lo = (older || j != 0) ? 0 : s.lead;
  r.hi = min(kBlockTokens, older ? s.n0 - blk * kBlockTokens : s.lead + s.n1 - j * kBlockTokens);
  r.seg_tok = older ? -1 : j * kBlockTokens - s.lead;
  r.older = older;
  return r;
}

// Segment arguments shared by the decode and prefill entry points (the lkv_*_args fields of the
// same names).  Paged segments (a block table) address one pool for all sequences: page p of
// kv head h is at base + p * page + h * head_stride, and block j of sequence b is page
// tab[b * tab_stride + j]; slots and seq strides are then unused.
struct SegParams {
  const uint16_t* ok;
  const uint16_t* ov;
  int64_t o_ss, o_hs;
  const int32_t* o_len;
  int32_t o_len_c, o_cap;
  const int32_t* o_slot;
  int32_t o_nslots;
  const int32_t* o_tab;
  int64_t o_tab_stride, o_page;
  int32_t o_npages;
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
  const int32_t* l_tab;
  int64_t l_tab_stride, l_page;
  int32_t l_npages;
};

// Lengths read from device memory are clamped to the capacities, and a slot outside [0, slots)
// gives that sequence an empty segment, so corrupt metadata cannot address outside the caches.
__device__ inline SeqView make_seq_view(const SegParams& g, int b, int kvh) {
  SeqView sv;
  const bool opaged = g.o_tab != nullptr, lpaged = g.l_tab != nullptr;
  const int oslot = opaged ? b : (g.o_slot ? g.o_slot[b] : b);
  const int lslot = lpaged ? b : (g.l_slot ? g.l_slot[b] : b);
  const bool oslot_ok = opaged || (oslot >= 0 && oslot < g.o_nslots);
  const bool lslot_ok = lpaged || (lslot >= 0 && lslot < g.l_nslots);
  int n0 = g.o_len ? g.o_len[b] : g.o_len_c;
  int n1 = g.lk ? (g.l_len ? g.l_len[b] : g.l_len_c) : 0;
  n0 = (!oslot_ok || g.ok == nullptr) ? 0 : min(max(n0, 0), g.o_cap);
  n1 = !lslot_ok ? 0 : min(max(n1, 0), g.ring_blocks * kBlockTokens);
  int ls = g.l_start ? g.l_start[b] : g.l_start_c;
  ls = (ls < 0 || ls >= g.ring_blocks * kBlockTokens) ? 0 : ls;
  const int64_t obase = (opaged ? 0 : static_cast<int64_t>(oslot) * g.o_ss) + kvh * g.o_hs;
  const int64_t lbase = (lpaged ? 0 : static_cast<int64_t>(lslot) * g.l_ss) + kvh * g.l_hs;
  sv.ok = g.ok ? g.ok + obase : nullptr;
  sv.ov = g.ov ? g.ov + obase : nullptr;
  sv.lk = g.lk ? g.lk + lbase : nullptr;
  sv.lv = g.lv ? g.lv + lbase : nullptr;
  sv.otab = opaged ? g.o_tab + b * g.o_tab_stride : nullptr;
  sv.ltab = lpaged ? g.l_tab + b * g.l_tab_stride : nullptr;
  sv.opage = g.o_page;
  sv.lpage = g.l_page;
  sv.onpages = g.o_npages;
  sv.lnpages = g.l_npages;
  sv.n0 = n0;
  sv.n1 = n1;
  sv.nb0 = (n0 + kBlockTokens - 1) / kBlockTokens;
  sv.lblk0 = ls >> 5;
  sv.lead = ls & (kBlockTokens - 1);
  sv.ring_blocks = g.ring_blocks;
  return sv;
}

// Validates and copies the segment fields of an lkv_decode_args / lkv_prefill_args.
template <class Args>
inline int32_t fill_segments(const Args* a, SegParams& g) {
  LKV_REQUIRE(a->older_k != nullptr || a->local_k != nullptr, "at least one key segment is required");
  LKV_REQUIRE((a->older_k == nullptr) == (a->older_v == nullptr), "older_k and older_v must both be set");
  LKV_REQUIRE((a->local_k == nullptr) == (a->local_v == nullptr), "local_k and local_v must both be set");
  const bool opaged = a->older_block_table != nullptr, lpaged = a->local_block_table != nullptr;
  LKV_REQUIRE(!opaged || a->older_k != nullptr, "older_block_table without an older pool");
  LKV_REQUIRE(!lpaged || a->local_k != nullptr, "local_block_table without a local pool");
  LKV_REQUIRE(a->older_k == nullptr || (a->older_capacity_tokens >= 0 && a->older_capacity_tokens % kBlockTokens == 0),
              "older capacity must be a multiple of 32 tokens");
  if (a->older_k != nullptr && opaged) {
    LKV_REQUIRE(a->older_num_pages > 0, "older_num_pages must be positive");
    LKV_REQUIRE(a->older_table_stride * kBlockTokens >= a->older_capacity_tokens,
                "older_table_stride must hold older_capacity_tokens / 32 pages");
    LKV_REQUIRE(a->older_page_stride > 0 && a->older_page_stride % 8 == 0, "older_page_stride must be a positive multiple of 8");
  } else if (a->older_k != nullptr) {
    LKV_REQUIRE(a->older_num_slots > 0, "older_num_slots must be positive");
    LKV_REQUIRE(a->older_slot != nullptr || a->older_num_slots >= a->batch, "older_num_slots < batch with identity slots");
  }
  if (a->local_k != nullptr) {
    LKV_REQUIRE(a->local_ring_blocks > 0, "local ring needs at least one block");
    if (lpaged) {
      LKV_REQUIRE(a->local_num_pages > 0, "local_num_pages must be positive");
      LKV_REQUIRE(a->local_table_stride >= a->local_ring_blocks, "local_table_stride must hold local_ring_blocks pages");
      LKV_REQUIRE(a->local_page_stride > 0 && a->local_page_stride % 8 == 0, "local_page_stride must be a positive multiple of 8");
    } else {
      LKV_REQUIRE(a->local_num_slots > 0, "local_num_slots must be positive");
      LKV_REQUIRE(a->local_slot != nullptr || a->local_num_slots >= a->batch, "local_num_slots < batch with identity slots");
    }
  }
  const uintptr_t align_or = reinterpret_cast<uintptr_t>(a->older_k) | reinterpret_cast<uintptr_t>(a->older_v) |
                             reinterpret_cast<uintptr_t>(a->local_k) | reinterpret_cast<uintptr_t>(a->local_v);
  LKV_REQUIRE((align_or & 15) == 0, "caches must be 16-byte aligned");
  LKV_REQUIRE((a->older_seq_stride | a->older_head_stride | a->local_seq_stride | a->local_head_stride) % 8 == 0,
              "cache strides must be multiples of 8 elements");
  g.ok = static_cast<const uint16_t*>(a->older_k);
  g.ov = static_cast<const uint16_t*>(a->older_v);
  g.o_ss = a->older_seq_stride;
  g.o_hs = a->older_head_stride;
  g.o_len = a->older_len;
  g.o_len_c = a->older_len_const;
  g.o_cap = a->older_capacity_tokens;
  g.o_slot = a->older_slot;
  g.o_nslots = a->older_num_slots;
  g.o_tab = opaged ? a->older_block_table : nullptr;
  g.o_tab_stride = a->older_table_stride;
  g.o_page = opaged ? a->older_page_stride : kBlockElems;
  g.o_npages = opaged ? a->older_num_pages : 1;
  g.lk = static_cast<const uint16_t*>(a->local_k);
  g.lv = static_cast<const uint16_t*>(a->local_v);
  g.l_ss = a->local_seq_stride;
  g.l_hs = a->local_head_stride;
  g.ring_blocks = a->local_k ? a->local_ring_blocks : 1;
  g.l_len = a->local_len;
  g.l_len_c = a->local_len_const;
  g.l_start = a->local_start;
  g.l_start_c = a->local_start_const;
  g.l_slot = a->local_slot;
  g.l_nslots = a->local_num_slots;
  g.l_tab = lpaged ? a->local_block_table : nullptr;
  g.l_tab_stride = a->local_table_stride;
  g.l_page = lpaged ? a->local_page_stride : kBlockElems;
  g.l_npages = lpaged ? a->local_num_pages : 1;
  return LKV_OK;
}

__device__ inline int local_blocks(const SeqView& s, int n_local_used) {
  return n_local_used > 0 ? (s.lead + n_local_used + kBlockTokens - 1) / kBlockTokens : 0;
}

// bf16(v * s) for the 8 bf16 values of one fragment (the reference materialises s * V in bf16).
__device__ inline uint4 scale_frag(uint4 v, float s) {
  uint4 r;
  r.x = pack_bf16x2(bf16_lo(v.x) * s, bf16_hi(v.x) * s);
  r.y = pack_bf16x2(bf16_lo(v.y) * s, bf16_hi(v.y) * s);
  r.z = pack_bf16x2(bf16_lo(v.z) * s, bf16_hi(v.z) * s);
  r.w = pack_bf16x2(bf16_lo(v.w) * s, bf16_hi(v.w) * s);
  return r;
}

// The sequences of a prefill call with col_lo < group * tokens <= col_hi <= 64 query rows per kv head
// (tokens: the call's count, or each sequence's own in a ragged call), run on the decode kernel with
// one score column per (query token, head) (decode.hip).  The arguments have passed
// lkv_prefill_attn's checks; seg was filled from them.  class_n: the number of the ragged call's
// sequences in the class when the host knows it (from cu_seqlens_q_host), else -1.
int32_t prefill_on_decode_kernel(const lkv_prefill_args* a, const SegParams& seg, int32_t group, int32_t col_lo,
                                 int32_t col_hi, int32_t class_n, hipStream_t s);

// The largest split count a ragged call's decode-kernel classes take (a lone sequence of the class
// then spreads over 32 workgroups per kv head: 256 at Hkv 8).
constexpr int kRaggedSplitCap = 32;

// Split-state rows x splits a ragged call's decode-kernel class needs in the worst case over the
// number n <= batch of its sequences (lmax query tokens each): the split count is `fixed` when
// positive, else min(cap, max(1, floor(cus / (n * num_kv_heads)))); rows of one split count nothing.
int64_t ragged_split_state_rows(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t lmax, int32_t cap,
                                int32_t fixed, int32_t cus);

}  // namespace lkv

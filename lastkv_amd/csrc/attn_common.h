// Key-segment addressing shared by the decode and prefill attention kernels.
//
// A sequence's keys are the concatenation [older | local]:
//   older: tokens [0, n0) of the shared last-layer cache (tiled blocks 0, 1, ...);
//   local: n1 tokens of a ring of ring_blocks tiled blocks, starting at ring token lstart
//          (block lstart / 32, token lstart % 32) and wrapping at the ring's end.
// Blocks are numbered over the concatenation: older blocks first, then local blocks.
#pragma once
#include "common.h"

namespace lkv {

struct BlockRef {
  const uint16_t* k;
  const uint16_t* v;
  int lo, hi;   // valid tokens [lo, hi) of the block
  int seg_tok;  // local segment index of token 0 of the block (older: -1)
  bool older;
};

struct SeqView {
  const uint16_t* ok;
  const uint16_t* ov;
  const uint16_t* lk;
  const uint16_t* lv;
  int n0, n1, nb0;
  int lblk0, lead;  // local segment: first ring block, first token inside it
  int ring_blocks;
};

// Branch-free (selects only), so it can sit inside straight-line scheduling regions.
__device__ inline BlockRef block_ref(const SeqView& s, int blk) {
  const bool older = blk < s.nb0;
  const int j = blk - s.nb0;
  int rb = s.lblk0 + j;  // < 2 * ring_blocks: the segment spans at most ring_blocks + 1 blocks
  rb = rb >= s.ring_blocks ? rb - s.ring_blocks : rb;
  const int64_t off = static_cast<int64_t>(older ? blk : rb) * kBlockElems;
  BlockRef r;
  r.k = (older ? s.ok : s.lk) + off;
  r.v = (older ? s.ov : s.lv) + off;
  r.lo = (older || j != 0) ? 0 : s.lead;
  r.hi = min(kBlockTokens, older ? s.n0 - blk * kBlockTokens : s.lead + s.n1 - j * kBlockTokens);
  r.seg_tok = older ? -1 : j * kBlockTokens - s.lead;
  r.older = older;
  return r;
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

}  // namespace lkv

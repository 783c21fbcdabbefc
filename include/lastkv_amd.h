/*
 * lastkv_amd.h -- C ABI of the MI355X (gfx950) LastKV shared last-layer KV attention path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, launches on the
 * given HIP stream, never allocates, never synchronises the host, and returns an lkv_status.
 * On failure lkv_last_error() returns a thread-local message.  bf16 tensors are passed as
 * pointers to uint16 storage.
 *
 * K/V caches use the tiled block layout: per (sequence, kv head) a run of 32-token blocks of
 * 4096 bf16 each (head_dim 128).  Inside a block, K element (w, d) sits at
 *   ((((w >> 2) & 1) * 4 + (d >> 5)) * 16 + (((w >> 3) << 2) | (w & 3))) * 32 + (d & 31)
 * and V element (w, d) at d * 32 + w.  lkv_cache_pack / lkv_cache_unpack convert from / to the
 * reference's [B, H, T, D] tensors (llm/src/lastkv/llm/modeling.py:37-67 keeps K/V that way).
 */
#ifndef LASTKV_AMD_H
#define LASTKV_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *lkv_stream_t; /* hipStream_t; NULL means the legacy default stream */

typedef enum lkv_status {
  LKV_OK = 0,
  LKV_ERR_INVALID_ARGUMENT = 1,
  LKV_ERR_UNSUPPORTED = 2,
  LKV_ERR_WORKSPACE = 3,
  LKV_ERR_HIP = 4
} lkv_status;

#define LKV_HEAD_DIM 128
#define LKV_BLOCK_TOKENS 32
#define LKV_BLOCK_ELEMS 4096
#define LKV_ABI_VERSION 1

/* Version of this ABI (LKV_ABI_VERSION). */
int32_t lkv_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char *lkv_last_error(void);

/* ---------------------------------------------------------------------------------------
 * Cache layout conversion.  No reference counterpart: the reference keeps K/V as
 * [B, Hkv, T, D] tensors (llm/src/lastkv/llm/modeling.py:31-34, :107, :205).
 * kind: 0 = K layout, 1 = V layout.  src is bf16 [B, H, T, 128] with element strides
 * (src_stride_b, src_stride_h, src_stride_t; the dim stride must be 1).  Tokens [0, T) of src
 * are written to cache tokens [dst_token0, dst_token0 + T) of sequence b, kv head h at
 * dst + b * dst_seq_stride + h * dst_head_stride; dst_capacity_tokens bounds the write.
 * ------------------------------------------------------------------------------------- */
int32_t lkv_cache_pack(const void *src, int64_t src_stride_b, int64_t src_stride_h, int64_t src_stride_t,
                       int32_t batch, int32_t heads, int32_t tokens, int32_t kind, void *dst,
                       int64_t dst_seq_stride, int64_t dst_head_stride, int32_t dst_token0,
                       int32_t dst_capacity_tokens, lkv_stream_t stream);

/* Inverse of lkv_cache_pack: cache tokens [src_token0, src_token0 + T) -> dst [B, H, T, 128]. */
int32_t lkv_cache_unpack(const void *src, int64_t src_seq_stride, int64_t src_head_stride, int32_t src_token0,
                         int32_t src_capacity_tokens, int32_t batch, int32_t heads, int32_t tokens, int32_t kind,
                         void *dst, int64_t dst_stride_b, int64_t dst_stride_h, int64_t dst_stride_t,
                         lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Shared-KV decode attention (one query token per sequence).
 *
 * Replaces, for decode steps (Lq = 1):
 *   - the region composition + SDPA of LastKVAttention.forward
 *     (llm/src/lastkv/llm/modeling.py:109-122 torch.cat of older/recent/current, :143-146 SDPA);
 *   - the merged paged FA3 call of the serving fast path
 *     (vllm/src/lastkv/vllm/backends/rmarin_flashinfer/fastpath.py:644-651, FA3 + head_scale_).
 * Softmax runs over the union of two key segments of sequence b:
 *   older : tokens [0, older_len[b]) of the shared last-layer cache (slot older_slot[b]);
 *           with older_vscale_mode 1 its V is used as bf16(V * vscale[h]), the reference's
 *           _scale() (modeling.py:93-96); with mode 0 V is used as stored.
 *   local : local_len[b] tokens of a per-layer ring of local_ring_blocks blocks starting at
 *           ring block local_start_block[b] (wrapping), e.g. the recent (already blended)
 *           chunk followed by the current chunk.
 * out[b, h, :] = softmax(q[b, h] . K^T * sm_scale) V for query head h, GQA group
 * Hq / Hkv <= 16 (query head h reads kv head h / group).  Optional lse[b * Hq + h] receives the
 * natural-log log-sum-exp of the scaled scores (-inf when there are no keys).
 * num_splits > 1 splits each sequence's keys across workgroups; the workspace must then hold
 * lkv_decode_workspace_bytes(batch, num_q_heads, num_splits) bytes.
 * Lengths read from device memory are clamped to the capacities, and a slot index outside
 * [0, num_slots) makes that sequence attend to no keys (its output is zero), so corrupt
 * metadata cannot make the kernel read outside the caches.
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_decode_args {
  int32_t struct_size; /* sizeof(lkv_decode_args) */
  int32_t batch;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim; /* must be 128 */
  int32_t num_splits;
  float sm_scale;
  int32_t older_vscale_mode; /* 0 or 1 */
  const void *q;             /* bf16 [B, Hq, 128], head stride 128 */
  int64_t q_stride_b;
  void *out; /* bf16 [B, Hq, 128], head stride 128 */
  int64_t out_stride_b;
  float *lse; /* optional fp32 [B, Hq] */
  const void *older_k;
  const void *older_v;
  int64_t older_seq_stride;
  int64_t older_head_stride;
  const int32_t *older_len; /* device [B] or NULL -> older_len_const */
  int32_t older_len_const;
  int32_t older_capacity_tokens; /* tokens per (slot, head); older_len is clamped to it */
  const int32_t *older_slot;     /* device [B] or NULL -> slot b */
  int32_t older_num_slots;       /* slots addressable through older_slot (>= batch if NULL) */
  const float *vscale;       /* device [Hkv] fp32, required for older_vscale_mode 1 */
  const void *local_k;       /* NULL: no local segment */
  const void *local_v;
  int64_t local_seq_stride;
  int64_t local_head_stride;
  int32_t local_ring_blocks;
  int32_t local_len_const;
  const int32_t *local_len;         /* device [B] or NULL -> local_len_const */
  const int32_t *local_start_block; /* device [B] or NULL -> 0 */
  const int32_t *local_slot;        /* device [B] or NULL -> slot b */
  int32_t local_num_slots;          /* slots addressable through local_slot */
  void *workspace;
  int64_t workspace_bytes;
} lkv_decode_args;

int64_t lkv_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_splits);

int32_t lkv_decode_attn(const lkv_decode_args *args, lkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LASTKV_AMD_H */

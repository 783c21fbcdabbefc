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
#define LKV_ABI_VERSION 11

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
 *           ring token local_start[b] (wrapping at 32 * local_ring_blocks), e.g. the recent
 *           (already blended) chunk followed by the current chunk.
 * out[b, h, :] = softmax(q[b, h] . K^T * sm_scale) V for query head h, GQA group
 * Hq / Hkv <= 64 (query head h reads kv head h / group).  Optional lse[b * Hq + h] receives the
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
  const int32_t *local_start;       /* device [B] ring token or NULL -> local_start_const */
  int32_t local_start_const;
  const int32_t *local_slot;        /* device [B] or NULL -> slot b */
  int32_t local_num_slots;          /* slots addressable through local_slot */
  void *workspace;
  int64_t workspace_bytes;
  /* Optional paging (NULL tables: contiguous segments as above).  With older_block_table, block j
   * (tokens 32j..32j+31) of sequence b's older segment is page older_block_table[b *
   * older_table_stride + j] of the pool at older_k / older_v: page p of kv head h starts at element
   * p * older_page_stride + h * older_head_stride; older_slot and older_seq_stride are unused and
   * older_capacity_tokens <= 32 * older_table_stride.  With local_block_table, ring block rb of
   * sequence b is page local_block_table[b * local_table_stride + rb] (rb < local_ring_blocks <=
   * local_table_stride).  Page ids are clamped into [0, num_pages). */
  const int32_t *older_block_table;
  int64_t older_table_stride;
  int64_t older_page_stride;
  int32_t older_num_pages;
  const int32_t *local_block_table;
  int64_t local_table_stride;
  int64_t local_page_stride;
  int32_t local_num_pages;
  /* Cache policy of the K/V loads: 0 = automatic (non-temporal when the call's K/V, bounded by the
   * segment lengths or capacities, exceed 384 MiB: more than the 256 MB last-level cache could
   * keep for the next layer's call over the same shared cache), 1 = default policy, 2 =
   * non-temporal.  Results do not depend on it. */
  int32_t kv_cache_hint;
  /* Optional output scale, fp32 [Hkv] (bf16-valued) or NULL: the output of query head h becomes
   * bf16(bf16(o) * out_scale[h / group]), the serving path's per-head rescale of an attention over
   * rings that hold V / s (fastpath.py:650 _head_scale / :690 output.mul_(out_scale),
   * fused_qkv.py:130-156 head_scale_: the bf16 output times s in fp32, one rounding).  lse is not
   * scaled. */
  const float *out_scale;
} lkv_decode_args;

int64_t lkv_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_splits);

int32_t lkv_decode_attn(const lkv_decode_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Allocation-free variant of lkv_decode_attn.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc) and cannot keep a workspace of their own.  Same arguments, kernels and
 * results as lkv_decode_attn, except that args->workspace must be NULL and workspace_bytes 0: the
 * split-K partial states live in a static device array of LKV_NOALLOC_SCRATCH_BYTES that the
 * library holds on every GPU it runs on until the process ends.  Calls whose
 * lkv_decode_workspace_bytes(batch, num_q_heads, num_splits) exceeds it are rejected
 * (LKV_ERR_INVALID_ARGUMENT).  Nothing is allocated and nothing needs clearing (every split writes
 * its whole partial state), but every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (streams or host threads running concurrently) race and must be serialised by the
 * caller.  Call it with the stream's device current.
 * ------------------------------------------------------------------------------------- */
#define LKV_NOALLOC_SCRATCH_BYTES (16 << 20)

int32_t lkv_decode_attn_noalloc(const lkv_decode_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Chunked-prefill attention (L >= 1 query tokens per sequence, MFMA).
 *
 * Replaces, for prefill calls (Lq > 1): the region composition + masked SDPA of
 * LastKVAttention.forward (modeling.py:109-146, bottom-right causal mask :124-130), the merged
 * FA3 varlen call of the serving fast path over [older pages | ring pages] (fastpath.py:644-651),
 * and, with causal = 0, the Wan block attention over [history | current block] whose current
 * block is bidirectional (videogen/src/lastkv/videogen/attention.py:9-32).
 * Query token i of sequence b (q[b, i, h, :], bf16 [B, L, Hq, 128]) attends to the older
 * segment (all of it) and to local tokens [0, local_len[b] - L + i] (causal = 1) or to all
 * local tokens (causal = 0); the last L local tokens are the queries' own K/V.  Segments,
 * slots, clamping and vscale are as in lkv_decode_args.  out is bf16 [B, L, Hq, 128] with
 * 8-byte-aligned rows (q: 16-byte-aligned rows); optional lse is fp32 [B, L, Hq] (natural log).
 * The tile kernel runs P*V in fp16, which represents bf16 V exactly for 2^-17 <= |V| <= 65280 and 0
 * (smaller magnitudes are truncated toward zero, an absolute error below 2^-24); a query tile whose
 * keys include a finite V (older: bf16(V * vscale)) of magnitude 65536 or more runs instead on a
 * second instance with bf16 V and the probabilities split into bf16 hi + lo, so no value
 * saturates.  causal = 1 masks only the local segment, whose last `tokens` tokens are the queries' own
 * keys: a host-constant local_len in [1, tokens) is rejected (the mask would have to reach into
 * the older segment); without a local segment, or with local_len 0, the older segment is fully
 * visible (the two-pass path's source pass).  Device lengths are not checked: a row then sees the
 * local tokens up to its bottom-right limit, if any.  The call first writes the fp16 V (older segment as bf16(V * vscale)) of every key
 * block and a flag per block (does some value exceed fp16's range) into the caller's workspace
 * (lkv_prefill_workspace_bytes), then runs the attention over it (the fp16 instance, then the
 * wide instance for the flagged tiles); all launches go on `stream`, and the workspace may be
 * reused once the call has run.
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_prefill_args {
  int32_t struct_size; /* sizeof(lkv_prefill_args) */
  int32_t batch;
  int32_t tokens; /* L */
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim; /* must be 128 */
  float sm_scale;
  int32_t causal;
  int32_t older_vscale_mode;
  const void *q;
  int64_t q_stride_b;
  int64_t q_stride_t;
  void *out;
  int64_t out_stride_b;
  int64_t out_stride_t;
  float *lse;
  const void *older_k;
  const void *older_v;
  int64_t older_seq_stride;
  int64_t older_head_stride;
  const int32_t *older_len;
  int32_t older_len_const;
  int32_t older_capacity_tokens;
  const int32_t *older_slot;
  int32_t older_num_slots;
  const float *vscale;
  const void *local_k;
  const void *local_v;
  int64_t local_seq_stride;
  int64_t local_head_stride;
  int32_t local_ring_blocks;
  int32_t local_len_const;
  const int32_t *local_len;
  const int32_t *local_start;
  int32_t local_start_const;
  const int32_t *local_slot;
  int32_t local_num_slots;
  void *workspace; /* >= lkv_prefill_workspace_bytes(args) bytes, 16-byte aligned */
  int64_t workspace_bytes;
  /* Optional paging, with the same meaning as in lkv_decode_args. */
  const int32_t *older_block_table;
  int64_t older_table_stride;
  int64_t older_page_stride;
  int32_t older_num_pages;
  const int32_t *local_block_table;
  int64_t local_table_stride;
  int64_t local_page_stride;
  int32_t local_num_pages;
  /* Kernel choice.  0: calls of at most 64 query rows per kv head (tokens * Hq / Hkv <= 64) run on
   * the decode kernel (one score column per (token, head), each key read once); larger calls on the
   * MFMA tile kernel with 4 or 8 waves per workgroup chosen from the grid and the device's CU
   * count.  4 / 8: always the tile kernel, with that many waves (32 rows each) above 64 rows per
   * kv head and 2 waves at or below.  In a ragged call (cu_seqlens_q) 4 / 8 set the waves of its
   * sequences above 64 rows per kv head; its shorter sequences stay on the decode kernel unless
   * every sequence is short, in which case all take the 2-wave tiles. */
  int32_t tile_waves;
  /* Optional output scale, fp32 [Hkv] (bf16-valued) or NULL, as in lkv_decode_args. */
  const float *out_scale;
  /* Optional ragged query rows (varlen; the cu_seqlens_q / max_seqlen_q of the FlashAttention varlen
   * call the serving fast path makes for mixed prefill + decode steps, fastpath.py:643-648).  NULL:
   * every sequence has `tokens` query tokens, q[b, i] at q + b * q_stride_b + i * q_stride_t.  Else a
   * device int32 [batch + 1] array, non-decreasing from cu_seqlens_q[0] = 0: sequence b's query
   * tokens are rows cu_seqlens_q[b] .. cu_seqlens_q[b + 1] - 1 of a [tokens, Hq, 128] q (row t at
   * q + t * q_stride_t; q_stride_b and out_stride_b are unused; out and lse likewise by row, lse fp32
   * [tokens, Hq]), `tokens` is the total row count and max_seqlen_q (>= 1) bounds every sequence's
   * count.  Sequence b's L_b query tokens are the last L_b tokens of its local segment (causal).
   * Entries are clamped into [0, tokens] and counts to max_seqlen_q, so corrupt offsets cannot
   * address outside q / out.  With tile_waves 0, sequences of at most 64 query rows per kv head run
   * on the decode kernel and the others on the tile kernel, in one call. */
  const int32_t *cu_seqlens_q;
  int32_t max_seqlen_q;
  /* Key splits of the sequences that run on the decode kernel (at most 64 query rows per kv head):
   * 0 chooses them from the grid and the workspace, and lets the tile kernel split its tiles' keys
   * (at most 4 ways, merged by LSE) when its grid would leave CUs idle and the workspace holds the
   * states; n in [1, 1024] fixes n (the workspace must then also hold their split states, which
   * lkv_prefill_workspace_bytes includes) and runs the tiles unsplit, so that a caller that fixes
   * the split count gets the same arithmetic whatever the batch. */
  int32_t num_splits;
  /* Optional host copy of cu_seqlens_q (the same batch + 1 offsets, in host memory), or NULL.  With
   * it a ragged call plans on the host, as FlashInfer's plan() does from its host-side indptr: it
   * launches only the decode-kernel column classes that hold a sequence, merges a class's key
   * splits only when it has more than one, and skips the tile kernel when no sequence needs it.
   * It must hold the device array's values (the kernels read cu_seqlens_q); a class it shows empty
   * is not computed.  The reference's FA3 varlen call plans inside that library; no counterpart. */
  const int32_t *cu_seqlens_q_host;
} lkv_prefill_args;

/* Workspace bytes lkv_prefill_attn wants for these args: the fp16 V of every key block of every
 * (sequence, kv head), 8 KiB per 32-token block (exact when the lengths and the ring start are
 * host constants, else bounded by the capacities), one flag byte per block (rows padded to 16
 * bytes) and one 16-byte word, then the states of the tile kernel's key splits (fp32 O and LSE per
 * output row, query head and split) when its grid would leave CUs idle; or the decode kernel's
 * split states (ragged calls, or num_splits > 1) if those are larger.  Takes the same filled-in
 * struct. */
int64_t lkv_prefill_workspace_bytes(const lkv_prefill_args *args);

/* The smallest workspace lkv_prefill_attn accepts for these args: lkv_prefill_workspace_bytes
 * without the key splits' states (with less room than those need, a call splits its tiles' keys
 * fewer ways, down to none).  No counterpart in the reference (its FA3 / FlashInfer calls manage
 * their own scratch); for callers that size one workspace for many calls. */
int64_t lkv_prefill_workspace_min_bytes(const lkv_prefill_args *args);

int32_t lkv_prefill_attn(const lkv_prefill_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Fused per-layer QKV epilogue: RoPE, q/k RMSNorm and the K/V cache append in one launch.
 *
 * Replaces modeling.py:103-108 (apply_rotary_pos_emb, q_norm / k_norm, append of the new K/V to
 * current[l]) and, on the serving path, fused_qkv.py:58-126 (_fused_qkv_kernel: rotary + RMSNorm
 * + ring / slab K,V writes).  With rounding = 0 the arithmetic follows the torch op order of the
 * reference's bf16 model: rope = bf16(bf16(x*cos) + bf16(rotate_half(x)*sin)); norm =
 * bf16(w * bf16(x * r)) with r = 1 / sqrt(mean(x^2) + eps) in fp32 (transformers LlamaRMSNorm,
 * modeling.py:90-91); rounding = 1 follows the fused_qkv kernel instead (see the field).
 * For new token i of sequence b at cache position p = pos(b) + i (pos(b) = positions[b], or
 * position_const when positions is NULL):
 *   q_out[b, i, h, :] = norm_q(rope(q[b, i, h, :]))                  for h < Hq
 *   K = norm_k(rope(k[b, i, g, :])); V = v[b, i, g, :]               for g < Hkv
 *   ring (tiled, ring_tokens a multiple of 32): token p mod ring_tokens of (ring slot, g) := K, V
 *   deep (optional, tiled): token p of (deep slot, g) := K, V            (the final layer)
 * cos/sin are bf16 [Bc, L, 128] with Bc in {1, B} (cs_stride_b 0 broadcasts), as produced by the
 * model's rotary embedding for positions p.  q_norm_w / k_norm_w NULL skips that norm.
 * Writes to positions outside the deep capacity are dropped.
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_qkv_args {
  int32_t struct_size;
  int32_t batch;
  int32_t tokens; /* new tokens per sequence, L */
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim; /* must be 128 */
  float eps;
  int32_t position_const;
  const int32_t *positions; /* device [B] or NULL */
  const void *q;            /* bf16, row (b, i) at b * q_stride_b + i * q_stride_t, heads contiguous */
  int64_t q_stride_b;
  int64_t q_stride_t;
  const void *k;
  int64_t k_stride_b;
  int64_t k_stride_t;
  const void *v;
  int64_t v_stride_b;
  int64_t v_stride_t;
  const void *cos;
  const void *sin;
  int64_t cs_stride_b;
  int64_t cs_stride_t;
  const void *q_norm_w; /* bf16 [128] or NULL */
  const void *k_norm_w; /* bf16 [128] or NULL */
  void *q_out;          /* bf16 [B, L, Hq, 128] */
  int64_t q_out_stride_b;
  int64_t q_out_stride_t;
  void *ring_k;
  void *ring_v;
  int64_t ring_seq_stride;
  int64_t ring_head_stride;
  int32_t ring_tokens;
  int32_t ring_num_slots;
  const int32_t *ring_slot; /* device [B] or NULL -> slot b */
  void *deep_k;             /* NULL: no deep write */
  void *deep_v;
  int64_t deep_seq_stride;
  int64_t deep_head_stride;
  int32_t deep_capacity_tokens;
  int32_t deep_num_slots;
  const int32_t *deep_slot; /* device [B] or NULL -> slot b */
  /* Optional paging (the serving path's page pool): with ring_block_table, ring block rb of
   * sequence b is page ring_block_table[b * ring_table_stride + rb] of the pool at ring_k /
   * ring_v (page p of kv head g at p * ring_page_stride + g * ring_head_stride; ring slots and
   * ring_seq_stride unused); deep_block_table likewise maps deep block j of sequence b.  Page ids
   * are clamped into [0, num_pages). */
  const int32_t *ring_block_table;
  int64_t ring_table_stride;
  int64_t ring_page_stride;
  int32_t ring_num_pages;
  const int32_t *deep_block_table;
  int64_t deep_table_stride;
  int64_t deep_page_stride;
  int32_t deep_num_pages;
  /* Rounding contract of RoPE and RMSNorm: 0 = the torch op order above (the HF model); 1 = the
   * vLLM fused_qkv kernel (fused_qkv.py:24-55): rope = (bf16(fma(x, c, -(y * s))), bf16(fma(y, c,
   * x * s))) over the halves x = dims [0, 64), y = dims [64, 128) with c, s the cos / sin of dims
   * [0, 64); RMSNorm sums the squares as 16 groups of 8 consecutive dims, each accumulated in order
   * with fused multiply-adds, then adjacent groups pairwise (16 -> 8 -> 4 -> 2 -> 1), and writes
   * bf16(x * r * w) with fp32 products.  r = 1 / sqrt(sum / 128 + eps) in both contracts (fp32,
   * correctly rounded square root and division; the reference's rsqrt.approx is hardware-specific). */
  int32_t rounding;
  /* Optional fp32 [Hkv] or NULL: the ring receives V as bf16(v * ring_v_mul[g]) (the vLLM path's
   * rings of V / s with ring_v_mul = fp32(1 / s), fused_qkv.py:84-86); the deep write keeps the
   * raw V (fused_qkv.py:87-90). */
  const float *ring_v_mul;
  /* Optional ragged rows (the fused QKV kernel's per-token form over a mixed step's flattened rows,
   * fused_qkv.py:58-126).  NULL: `tokens` new tokens per sequence as above.  Else a device int32
   * [batch + 1] array, non-decreasing from cu_seqlens[0] = 0: sequence b's new tokens are rows
   * cu_seqlens[b] .. cu_seqlens[b + 1] - 1 (row t of q, k, v, cos, sin and q_out at t * *_stride_t;
   * the *_stride_b fields are unused), its token i at position positions[b] + i (or position_const
   * + i); `tokens` is the total row count and max_seqlen (>= 1) bounds every sequence's count.
   * Offsets are clamped into [0, tokens] and counts to max_seqlen. */
  const int32_t *cu_seqlens;
  int32_t max_seqlen;
} lkv_qkv_args;

int32_t lkv_qkv_epilogue(const lkv_qkv_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Chunk-boundary commit: materialise the recent-chunk blend of every layer once.
 *
 * Replaces the per-step recomputation of modeling.py:116-119 and the serving commit
 * fused_qkv.py:158-201 (blend_chunk_) / batching.py:1099-1155 (_commit_previous_boundary).
 * For layer l < layers, sequence b < batch, kv head g and tokens p in
 * [chunk_start, chunk_start + chunk_len), with a = alpha[l*Hkv+g], om = one_minus_alpha[..],
 * s = vscale[..] (bf16 values carried as fp32; vscale NULL means s = 1):
 *   ringK[l][b][g][p mod R] = bf16(bf16(a * deepK[b][g][p]) + bf16(om * ringK[l][b][g][p mod R]))
 *   ringV[l][b][g][p mod R] = bf16(bf16(a * bf16(deepV[b][g][p] * s)) + bf16(om * ringV[..]))
 * which is the reference's bf16 expression evaluated op by op.  Both caches are tiled; R =
 * ring_tokens (a multiple of 32).  Layer l's ring is ring + l * ring_layer_stride.
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_blend_args {
  int32_t struct_size; /* sizeof(lkv_blend_args) */
  int32_t layers;
  int32_t batch;
  int32_t kv_heads;
  int32_t chunk_start;
  int32_t chunk_len;
  void *ring_k; /* tiled rings, layer l at ring + l * ring_layer_stride (or a page pool, below) */
  void *ring_v;
  int64_t ring_layer_stride;
  int64_t ring_seq_stride;
  int64_t ring_head_stride;
  int32_t ring_tokens;
  const void *deep_k; /* tiled shared store (or a page pool, below) */
  const void *deep_v;
  int64_t deep_seq_stride;
  int64_t deep_head_stride;
  int32_t deep_capacity_tokens;
  const float *alpha;           /* [layers * kv_heads] */
  const float *one_minus_alpha; /* [layers * kv_heads] */
  const float *vscale;          /* [layers * kv_heads] or NULL (s = 1) */
  /* Optional paging: ring block rb of (layer l, sequence b) is page ring_block_table[l *
   * ring_table_layer_stride + b * ring_table_stride + rb] of the ring pool (page stride
   * ring_page_stride; ring_layer_stride / ring_seq_stride unused); deep block j of sequence b is
   * page deep_block_table[b * deep_table_stride + j] of the deep pool.  Ids are clamped. */
  const int32_t *ring_block_table;
  int64_t ring_table_layer_stride;
  int64_t ring_table_stride;
  int64_t ring_page_stride;
  int32_t ring_num_pages;
  const int32_t *deep_block_table;
  int64_t deep_table_stride;
  int64_t deep_page_stride;
  int32_t deep_num_pages;
} lkv_blend_args;

int32_t lkv_blend_chunk(const lkv_blend_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Exact merge of two attention states over disjoint key sets.
 *
 * Replaces the serving path's merge of the older-source pass with the local pass:
 *   - vllm/src/lastkv/vllm/backends/rmarin_flashinfer/flashinfer_executor.py:185-231
 *     (merge_attention_states -> flashinfer.cascade.merge_state, LSE [T, H]);
 *   - fastpath.py:709-719 (two-pass FA3: source_out *= s_l, then vLLM merge_attn_states with
 *     LSE [H, T]; rows without older history get a source LSE of -inf);
 *   - batching.py:1835-1861 (source_out * source_out_scale, merge, index_copy into the output).
 * For token t and head h (strides in elements, so either LSE layout works):
 *   a = prefix_out[t, h, :], or bf16(prefix_out[t, h, :] * prefix_scale[h]) when prefix_scale is
 *       set (the reference scales the bf16 source output before merging);
 *   m = max(la, lb); wa = e^(la - m); wb = e^(lb - m)      (natural-log LSEs; +inf reads as -inf)
 *   out[t, h, :] = bf16((a * wa + suffix_out[t, h, :] * wb) / (wa + wb))
 *   out_lse[t, h] = m + ln(wa + wb)                          (optional)
 * Both LSEs -inf (no keys on either side): out = 0 and out_lse = -inf.  Outputs are bf16 with
 * 16-byte-aligned rows; head_dim is a multiple of 8.  out may alias suffix_out (each element is
 * read before it is written by the same thread).
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_merge_args {
  int32_t struct_size; /* sizeof(lkv_merge_args) */
  int32_t tokens;
  int32_t num_heads;
  int32_t head_dim;
  const void *prefix_out; /* bf16 */
  int64_t prefix_out_stride_t;
  int64_t prefix_out_stride_h;
  const float *prefix_lse;
  int64_t prefix_lse_stride_t;
  int64_t prefix_lse_stride_h;
  const void *suffix_out; /* bf16 */
  int64_t suffix_out_stride_t;
  int64_t suffix_out_stride_h;
  const float *suffix_lse;
  int64_t suffix_lse_stride_t;
  int64_t suffix_lse_stride_h;
  const float *prefix_scale; /* optional fp32 [H] (bf16 values) */
  void *out;                 /* bf16 */
  int64_t out_stride_t;
  int64_t out_stride_h;
  float *out_lse; /* optional */
  int64_t out_lse_stride_t;
  int64_t out_lse_stride_h;
} lkv_merge_args;

int32_t lkv_merge_states(const lkv_merge_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Append K and V rows into pages of a tiled pool.
 *
 * Replaces the cache writes of:
 *   - the Wan model's cache append (videogen/src/lastkv/videogen/cache.py:33-50 append_shared,
 *     model.py:621-645 _append_current_history, model.py:67-84 append_to_cache);
 *   - vLLM's reshape_and_cache_flash into the fast path's ring / source pages
 *     (vllm/src/lastkv/vllm/backends/rmarin_flashinfer/fastpath.py:659-663).
 * Token t of sequence b (k / v rows at b * stride_b + t * stride_t + h * stride_h, 128 bf16
 * each, 16-byte aligned) goes to absolute position p = token0 + t; with wrap_tokens > 0 (a ring,
 * a multiple of 32) the cache position is p mod wrap_tokens, else p.  Cache position c of
 * sequence b lives in page block_table[b * table_stride + c / 32] (ids clamped to the pool)
 * at offset c mod 32 of the tiled block of head h.  Requires token0 + tokens <= 32 * table_width
 * without wrap, tokens <= wrap_tokens <= 32 * table_width with it.
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_append_args {
  int32_t struct_size; /* sizeof(lkv_append_args) */
  int32_t batch;
  int32_t tokens;
  int32_t heads;
  int32_t head_dim; /* 128 */
  int32_t token0;
  int32_t wrap_tokens;
  const void *k; /* bf16 */
  int64_t k_stride_b;
  int64_t k_stride_t;
  int64_t k_stride_h;
  const void *v; /* bf16 */
  int64_t v_stride_b;
  int64_t v_stride_t;
  int64_t v_stride_h;
  void *pool_k; /* bf16 pool: page p of head h at p * page_stride + h * head_stride (4096 each) */
  void *pool_v;
  int64_t page_stride;
  int64_t head_stride;
  int32_t num_pages;
  const int32_t *block_table;
  int64_t table_stride;
  int32_t table_width;
} lkv_append_args;

int32_t lkv_append_paged(const lkv_append_args *args, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Decoder-layer glue of the serving path: RMSNorm with a fused residual add, and SwiGLU.
 *
 * lkv_rmsnorm replaces the serving model's input / post-attention / final norms and the
 * residual adds before them (the reference's vLLM model uses vLLM's fused_add_rms_norm there;
 * its HF model, modeling.py:150-171, uses transformers' LlamaRMSNorm, whose arithmetic this keeps):
 * for each of `rows` rows of `hidden` bf16 values,
 *   if residual != NULL: residual := bf16(residual + x), and the normalised row is residual;
 *   h = float(row); r = rsqrt(sum(h^2) * (1 / hidden) + eps); out = bf16(weight * bf16(h * r)).
 * hidden is a multiple of 8 up to 16384; rows are 16-byte aligned, strides in elements.
 * ------------------------------------------------------------------------------------- */
typedef struct lkv_rmsnorm_args {
  int32_t struct_size; /* sizeof(lkv_rmsnorm_args) */
  int32_t rows;
  int32_t hidden;
  float eps;
  const void *x; /* bf16 [rows, hidden] */
  int64_t x_stride;
  void *residual; /* optional bf16 [rows, hidden], updated in place */
  int64_t residual_stride;
  const void *weight; /* bf16 [hidden] */
  void *out;          /* bf16 [rows, hidden]; may alias x when residual is NULL */
  int64_t out_stride;
} lkv_rmsnorm_args;

int32_t lkv_rmsnorm(const lkv_rmsnorm_args *args, lkv_stream_t stream);

/* out = bf16(bf16(silu(gate)) * up) over rows x width bf16 values (torch's
 * F.silu(gate_proj(x)) * up_proj(x) in the Llama MLP, with both of its roundings); width is a
 * multiple of 8, rows 16-byte aligned, strides in elements. */
int32_t lkv_silu_mul(const void *gate, int64_t gate_stride, const void *up, int64_t up_stride, void *out,
                     int64_t out_stride, int32_t rows, int32_t width, lkv_stream_t stream);

/* ---------------------------------------------------------------------------------------
 * Achievable-peak probes.  No counterpart in the reference: measurement support for the bench,
 * which reports the kernels' rates against what these reach on the same part, beside the nominal
 * 8 TB/s and 2.5 PFLOP/s.
 *   lkv_probe_read: reads `bytes` (a positive multiple of 16, src 16-byte aligned) with 16-byte
 *     non-temporal loads, 8 in flight per thread, `workgroups` x 256 threads in a grid-stride walk
 *     (each load instruction of a wave one contiguous 1 KiB run), and writes one word per thread to
 *     `sink` (workgroups * 256 uint32).
 *   lkv_probe_mfma: `workgroups` x 4 waves, each running `iters` (a multiple of 8) rounds of 8 independent
 *     16x16x32 bf16 MFMA chains whose operands change from one MFMA to the next (pseudo-random
 *     bf16 values of magnitude [0.5, 1) with random signs, from `seed`); workgroups * 4 * iters *
 *     8 * 16384 FLOP in total; one word per thread to `sink`.
 * ------------------------------------------------------------------------------------- */
int32_t lkv_probe_read(const void *src, int64_t bytes, uint32_t *sink, int32_t workgroups, lkv_stream_t stream);

int32_t lkv_probe_mfma(uint32_t *sink, int32_t workgroups, int32_t iters, uint32_t seed, lkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LASTKV_AMD_H */

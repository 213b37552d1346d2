/*
 * gllm_attn — MI355X (gfx950) attention hot path for gLLM, C ABI.
 *
 * Drop-in boundary for the attention path of TheEpicDolphin/gllm.  The
 * reference is pure Python and binds no FFI; these entry points are what its
 * call sites would bind (through ctypes; gllm_amd/_lib.py is such a binding):
 *
 *   gllm_rope_kv_write    replaces gllm/model/layers/attention.py:151-161
 *                         (Attention.apply_rope :76-119 on k [and q], then the
 *                         index_put_ of k/v through query_slot_mapping)
 *   gllm_qkv_rope_kv_write replaces gllm/model/layers/attention.py:139-161
 *                         (linear_q/k/v = F.linear, linear.py:13-19, then the
 *                         same RoPE and KV write) with one fused launch
 *   gllm_paged_attention  replaces gllm/model/layers/attention.py:163-178
 *                         (the dense KV gather through slot_mapping plus
 *                         reference_attention with the 0/-inf bias of
 *                         gllm/llm/llm.py:249-274) for decode, prefill and
 *                         mixed batches; q rotation may be fused in
 *   gllm_attention_dense  replaces gllm/ops/attention/reference_attention.py:5-51
 *                         and flash_attention.py:155-192 (same contract:
 *                         q[B,T_q,Hq,D], k/v[B,T,Hkv,D], bias[B,T_q,T])
 *   gllm_attn_plan_*      host-side work planning for one batch (the lengths
 *                         gllm/llm/llm.py:233-241 derives), built once per
 *                         engine step and reused by every layer
 *   gllm_build_metadata   replaces gllm/llm/llm.py:245-281 (slot mapping of the
 *                         query rows and positions, built on the device from
 *                         the block table and lengths instead of the per-row
 *                         host loop; the paged kernels need no dense bias)
 *
 * Conventions: every data pointer is a device pointer the caller owns; the
 * library never allocates device memory (the paged path uses a caller-sized
 * workspace).  `stream` is a hipStream_t (NULL = default stream).  Every
 * function returns GLLM_ATTN_OK or an error code and records a message for
 * gllm_attn_last_error() (thread-local).  Strides are in elements.
 */
#ifndef GLLM_ATTN_H_
#define GLLM_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GLLM_ATTN_OK = 0,
  GLLM_ATTN_EINVAL = 1,       /* bad argument (shape, stride, null pointer) */
  GLLM_ATTN_EUNSUPPORTED = 2, /* valid but not implemented (dtype, head_dim) */
  GLLM_ATTN_EHIP = 3          /* HIP runtime error */
};

enum {
  GLLM_DTYPE_F32 = 0,
  GLLM_DTYPE_BF16 = 1,
  GLLM_DTYPE_FP8_E4M3 = 2, /* torch.float8_e4m3fn, KV cache only */
  GLLM_DTYPE_F16 = 3
};

enum {
  GLLM_ROPE_NONE = 0,        /* q already rotated */
  GLLM_ROPE_BY_POSITION = 1, /* cos/sin table row = c_i + r (model.py:117-128 table) */
  GLLM_ROPE_BY_ROW = 2       /* cos/sin row = query row index (model.py:195-196 gathered cos_pos) */
};

/* split_tokens value of gllm_attn_plan_create: page-balanced decode plan */
enum { GLLM_SPLIT_BALANCED = -1 };

typedef struct gllm_attn_plan gllm_attn_plan;

/* Thread-local message of the last failing call ("" if none). */
const char* gllm_attn_last_error(void);
int gllm_attn_version(void);

/*
 * Query-row metadata on the device (gllm/llm/llm.py:245-281).  For query row
 * r of sequence i, with c_i = seq_lens[i] - query_lens[i]:
 *   positions[row]    = c_i + r for r < query_lens[i] (llm.py:281); padded rows get the
 *                       sequence's last position seq_lens[i] - 1 (llm.py:281 gives them
 *                       c_i + r, which can pass the RoPE table's end in mixed batches),
 *                       so every position is < max(seq_lens) and indexes the table.
 *   slot_mapping[row] = block_table[i][(c_i+r)/bs]*bs + (c_i+r)%bs for r < query_lens[i],
 *                       0 (the reserved dummy slot) for padded rows, as llm.py:277 gives.
 * q_seq_stride > 0: padded layout, row = i*q_seq_stride + r for r < q_seq_stride.
 * q_seq_stride == 0: packed rows, row = cu_seqlens[i] + r for r < query_lens[i], and
 * cu_seqlens[0..num_seqs] (int32, optional) receives the running sums of query_lens.
 * Rows >= num_rows are not written; block-table columns >= block_table_width
 * (and inconsistent lengths) give slot 0.  Any output pointer may be NULL.
 * block_size: any value in [1, 65536] (the reference's block size is a free
 * config value).
 * Lengths and table are device pointers: nothing is read back to the host.
 */
int gllm_build_metadata(const int32_t* block_table, int64_t block_table_stride, int64_t block_table_width,
                        const int32_t* seq_lens, const int32_t* query_lens, int32_t num_seqs,
                        int64_t q_seq_stride, int32_t block_size, int64_t* slot_mapping, int64_t* positions,
                        int32_t* cu_seqlens, int64_t num_rows, void* stream);

/*
 * Fused QKV projection + RoPE + paged KV write (bf16 model only; replaces
 * attention.py:139-161).  For token t: q = x[t] @ w_q^T, k = x[t] @ w_k^T,
 * v = x[t] @ w_v^T (w_* row-major [heads * head_dim, hidden] as the
 * checkpoint stores them; fp32 accumulation, rounded to bf16 as F.linear
 * stores its result), then k (and q if rotate_q) rotated exactly as
 * gllm_rope_kv_write does and k/v stored at slot_mapping[t] in kv_dtype
 * (bf16 or fp8 e4m3fn).  q is written to q_out if q_out != NULL (rotated or
 * not: the paged attention kernels can rotate it on load).  query_lens /
 * tokens_per_seq / rope_rows and the slot range check as in
 * gllm_rope_kv_write (padded rows: nothing written, q_out included).  hidden must be a positive multiple of 32; x, the
 * weights and their row strides 16-byte aligned.  workspace (may be NULL,
 * 16-byte aligned) see gllm_qkv_workspace_bytes.  Results equal the
 * reference within the GEMM's accumulation order (fp32 sums in another
 * order, so a bf16 output may differ by one ulp); RoPE and the casts applied
 * to those bf16 values are bit-identical.
 */
int gllm_qkv_rope_kv_write(const void* x, int64_t x_row_stride, int64_t num_tokens, int32_t hidden,
                           const void* w_q, int64_t w_q_row_stride, const void* w_k, int64_t w_k_row_stride,
                           const void* w_v, int64_t w_v_row_stride, void* q_out, int64_t q_out_row_stride,
                           int32_t rotate_q, void* k_cache, void* v_cache, int64_t cache_slot_stride,
                           int64_t num_slots, const int64_t* slot_mapping, const int32_t* query_lens,
                           int64_t tokens_per_seq, const void* cos, const void* sin, const int64_t* rope_rows,
                           int64_t rope_row_stride, int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t dtype, int32_t kv_dtype, void* workspace,
                           size_t workspace_bytes, void* stream);
/* Device bytes gllm_qkv_rope_kv_write can use as `workspace` for this batch
 * (0: none).  Up to 32 tokens (hidden a multiple of 256, at most 4096) the
 * projection runs in one launch with no workspace (each workgroup the whole
 * hidden dimension of 16 or 32 output columns).  Otherwise, with a
 * workspace of at least that size, batches too small to fill the GPU with
 * (128-token x head) tiles (decode) split the hidden dimension over more
 * workgroups: fp32 partial sums go to the workspace and a second small
 * launch sums them in fixed order (deterministic) before the RoPE and the
 * stores.  Without it the tile kernel runs (same results up to the fp32
 * summation order of the projections).  No library counterpart in the
 * reference: F.linear needs none. */
size_t gllm_qkv_workspace_bytes(int64_t num_tokens, int32_t hidden, int32_t num_q_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t with_q);

/*
 * gllm_qkv_rope_kv_write without a workspace argument and without any
 * allocation (no hipMalloc/hipFree, no allocating library call).  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, serving loops and harnesses that forbid it).  The
 * split-K partial sums of few-token batches go to a static 24 MiB device
 * array inside the library, one per GPU, held until the process ends; a
 * batch whose partials would need more (gllm_qkv_workspace_bytes > 24 MiB; every Llama-3 decode shape fits)
 * is rejected with GLLM_ATTN_EUNSUPPORTED.  Every call on one GPU shares that
 * GPU's array: calls that overlap on the same GPU (different streams, or
 * threads) race.  Results equal gllm_qkv_rope_kv_write's with a workspace of
 * gllm_qkv_workspace_bytes bytes.
 */
int gllm_qkv_rope_kv_write_noalloc(const void* x, int64_t x_row_stride, int64_t num_tokens, int32_t hidden,
                                   const void* w_q, int64_t w_q_row_stride, const void* w_k, int64_t w_k_row_stride,
                                   const void* w_v, int64_t w_v_row_stride, void* q_out, int64_t q_out_row_stride,
                                   int32_t rotate_q, void* k_cache, void* v_cache, int64_t cache_slot_stride,
                                   int64_t num_slots, const int64_t* slot_mapping, const int32_t* query_lens,
                                   int64_t tokens_per_seq, const void* cos, const void* sin, const int64_t* rope_rows,
                                   int64_t rope_row_stride, int32_t num_q_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t dtype, int32_t kv_dtype, void* stream);

/*
 * Rotate k (and, if q_out != NULL, q) with rotate-half RoPE and write k/v rows
 * into the paged cache.  Token t (0 <= t < num_tokens) writes slot
 * slot_mapping[t] of k_cache / v_cache (each [num_slots, cache_slot_stride]).
 * If query_lens != NULL, token t is row t % tokens_per_seq of sequence
 * t / tokens_per_seq and rows past query_lens[seq] (the reference's padded
 * rows, which it sends to dummy slot 0) are skipped whole: nothing is
 * written for them (their q_out rows included) and their cos/sin rows are
 * not read.  Slots outside
 * [0, num_slots) are never written.  cos/sin rows: rope_rows[t] if given,
 * else t.  dtype is the model dtype of q/k/v/cos/sin (f32, bf16 or f16);
 * kv_dtype the cache's (f32, bf16, f16 or fp8 e4m3fn, any pairing, as
 * model.py:64,75 allow): each written value is cast like torch's
 * .to(kv_dtype) (round to nearest even; fp8: NaN -> 0x7f|sign,
 * |x| > 464 -> NaN).
 * Every op is rounded to the model dtype in the reference's order, so the
 * written K/V are bit-identical to attention.py:151-161.  With k == v == NULL
 * only q is rotated into q_out (Attention.apply_rope on one tensor).
 */
int gllm_rope_kv_write(const void* q, void* q_out, const void* k, const void* v,
                       void* k_cache, void* v_cache, const int64_t* slot_mapping,
                       const int32_t* query_lens, int64_t tokens_per_seq,
                       const void* cos, const void* sin, const int64_t* rope_rows,
                       int64_t rope_row_stride, int64_t num_tokens, int32_t num_q_heads,
                       int32_t num_kv_heads, int32_t head_dim, int64_t q_row_stride,
                       int64_t k_row_stride, int64_t v_row_stride, int64_t q_out_row_stride,
                       int64_t cache_slot_stride, int64_t num_slots, int32_t dtype,
                       int32_t kv_dtype, void* stream);

/*
 * Plan the work for one batch from HOST lengths.  Sequence i has
 * query_lens[i] query rows starting at row i * q_seq_stride of q/out
 * (q_seq_stride = the padded T_q of the reference's [B, T_q, ...] layout), or,
 * if q_seq_stride == 0, packed rows (cumulative query_lens).  seq_lens[i] =
 * context + query length, as llm.py:233-236.  block_size: any value in
 * [1, 65536] (the kernels divide by it exactly; powers of two are not
 * required).  split_tokens = context tokens
 * per decode split (multiple of 32) and decode_heads_per_wg = kv heads one
 * decode workgroup serves (1, 2, 4 or 8); 0 lets the planner choose both from
 * the batch and the CU count.  split_tokens == GLLM_SPLIT_BALANCED (-1) plans
 * the decode sequences page-balanced: their keys (16-key units per sequence
 * and kv-head group) are dealt out evenly to one workgroup per resident CU
 * slot, and sequences spread over several workgroups are merged inside the
 * same launch (split tickets); 0 picks it for decode-only batches whose
 * workgroups would each stream >= 2048 keys.  In a mixed batch (only on
 * request) the decode share goes to a multiple of 8 workgroups sized by a
 * cost model, and one workgroup per prefill item follows them on the other
 * CUs.  No device work happens here.
 */
int gllm_attn_plan_create(gllm_attn_plan** plan, const int32_t* query_lens,
                          const int32_t* seq_lens, int32_t num_seqs, int64_t q_seq_stride,
                          int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t dtype, int32_t split_tokens,
                          int32_t decode_heads_per_wg);
/* Device bytes the plan needs (work list, split partials, tickets). */
size_t gllm_attn_plan_workspace_bytes(const gllm_attn_plan* plan);
/* Stream-ordered upload of the plan into `workspace` (>= workspace_bytes).
 * The workspace must stay alive and untouched while launches use the plan. */
int gllm_attn_plan_upload(gllm_attn_plan* plan, void* workspace, size_t workspace_bytes, void* stream);
/* Plan facts: [0] work items, [1] split length, [2] decode-path sequences,
 * [3] prefill-path sequences, [4] split partials, [5] total query rows,
 * [6] kv heads per decode workgroup, [7] waves per decode workgroup,
 * [8] waves per prefill workgroup, [9] page-balanced decode segments (0:
 * split planner).  [0] counts workgroups for a page-balanced plan. */
int gllm_attn_plan_info(const gllm_attn_plan* plan, int64_t* info, int32_t n);
int gllm_attn_plan_destroy(gllm_attn_plan* plan);

/*
 * Paged attention for every query row the plan describes.  q/out rows are
 * [rows, num_q_heads * head_dim] with row strides in elements (heads at
 * h * head_dim, head dim contiguous).  k_cache/v_cache: [num_blocks *
 * block_size, cache_slot_stride] (one layer of the reference's
 * [2, L, NB, bs, Hkv, D] pool).  block_table: int32 rows of
 * block_table_stride, row i covering sequence i's ceil(seq_len / bs) blocks.
 * Key p of sequence i is visible to query row r iff p <= c_i + r.
 * Query head h reads kv head h / (num_q_heads / num_kv_heads).
 * rope_mode != NONE rotates q on load (bit-identical to apply_rope).
 * A bf16 or f16 model dtype runs the MFMA kernels (head_dim 64 or 128) over
 * a cache in the model dtype or fp8 e4m3fn; every other pairing (f32 model;
 * a 16-bit model over an f32 or the other 16-bit cache; other even head dims
 * up to 256) runs a generic kernel (fp32 arithmetic, model dtype in and
 * out).  Cached values are read as the reference reads them: cast to the
 * model dtype (attention.py:169-170's .to(q.dtype); exact for fp8, rounded
 * to nearest even where the cache is wider).
 * Returns after enqueueing on `stream`.
 */
int gllm_paged_attention(const gllm_attn_plan* plan, const void* q, int64_t q_row_stride,
                         void* out, int64_t out_row_stride, const void* k_cache,
                         const void* v_cache, int64_t cache_slot_stride, int64_t num_blocks,
                         const int32_t* block_table, int64_t block_table_stride,
                         const void* rope_cos, const void* rope_sin, int64_t rope_row_stride,
                         int32_t rope_mode, float scale, int32_t dtype, int32_t kv_dtype,
                         void* stream);

/*
 * gllm_rope_kv_write followed by gllm_paged_attention in one launch, for
 * plans whose sequences are all on the decode path (query_len x G <= 16 on
 * the MFMA kernels; query_len <= 16 on the generic kernel; other plans give
 * GLLM_ATTN_EINVAL).  Replaces gllm/model/layers/attention.py:151-178 for a
 * decode step (the reference's RoPE of k, its index_put_ into the cache and
 * the attention), i.e. model.py:202-222's per-layer write + attention pair.
 * k_new / v_new: one row per query row of q (same row layout, row strides in
 * elements, Hkv heads at h * head_dim, model dtype).  The new key of query
 * row r of sequence i is key c_i + r: k is rotated with the cos/sin rows
 * rope_mode selects for q (bit-identical to apply_rope), k and v are cast to
 * kv_dtype as .to(kv_dtype) rounds and stored at that key's slot
 * (block_table[i][p / bs] * bs + p % bs, the reference's query_slot_mapping),
 * and the attention reads them from there (MFMA kernels) or from the same
 * values kept in the kernel (generic kernel).  Cache contents and outputs
 * equal the two-call sequence's; on the MFMA kernels bit for bit.
 */
int gllm_paged_attention_write_kv(const gllm_attn_plan* plan, const void* q, int64_t q_row_stride,
                                  void* out, int64_t out_row_stride, void* k_cache, void* v_cache,
                                  int64_t cache_slot_stride, int64_t num_blocks,
                                  const int32_t* block_table, int64_t block_table_stride,
                                  const void* k_new, int64_t k_new_row_stride, const void* v_new,
                                  int64_t v_new_row_stride, const void* rope_cos, const void* rope_sin,
                                  int64_t rope_row_stride, int32_t rope_mode, float scale, int32_t dtype,
                                  int32_t kv_dtype, void* stream);

/*
 * reference_attention(q, k, v, bias): softmax(q k^T * scale + bias) v with
 * GQA.  q/out [B, T_q, Hq, D] (row stride q_row_stride, batch = T_q rows),
 * k/v [B, T, Hkv, D] with the given batch / row strides, bias [B, T_q, T]
 * (model dtype: f32, bf16 or f16) with batch / row strides, last dim
 * contiguous.  A row whose bias is -inf everywhere comes out NaN, as torch's
 * softmax makes it.
 */
int gllm_attention_dense(const void* q, int64_t q_row_stride, const void* k, int64_t k_batch_stride,
                         int64_t k_row_stride, const void* v, int64_t v_batch_stride,
                         int64_t v_row_stride, const void* bias, int64_t bias_batch_stride,
                         int64_t bias_row_stride, void* out, int64_t out_row_stride, int32_t batch,
                         int32_t q_len, int32_t kv_len, int32_t num_q_heads, int32_t num_kv_heads,
                         int32_t head_dim, float scale, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GLLM_ATTN_H_ */

// Host-visible argument blocks and launchers shared by the C ABI and kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace gllm {

enum : int32_t { kF32 = 0, kBF16 = 1, kFP8 = 2, kF16 = 3 };   // kFP8: OCP e4m3fn (KV cache only)

struct RopeKVWriteArgs {
  const void* q;            // [N, q_row_stride] model dtype, heads at h*D
  void* q_out;              // nullable: rotated q (same layout, q_out_row_stride)
  const void* k;            // [N, k_row_stride]
  const void* v;            // [N, v_row_stride]
  void* k_cache;            // [num_slots, cache_slot_stride] kv dtype
  void* v_cache;
  const int64_t* slot_mapping;   // [N]
  const int32_t* query_lens;     // nullable: skip row r >= query_lens[tok / tokens_per_seq]
  int64_t tokens_per_seq;
  const void* cos;               // [rows, rope_row_stride] model dtype
  const void* sin;
  const int64_t* rope_rows;      // nullable: cos/sin row per token (else the token index)
  int64_t rope_row_stride;
  int64_t num_tokens;
  int32_t num_q_heads, num_kv_heads, head_dim;
  int64_t q_row_stride, k_row_stride, v_row_stride, q_out_row_stride;
  int64_t cache_slot_stride, num_slots;
  int32_t dtype, kv_dtype;
};

enum : int32_t { kRopeNone = 0, kRopeByPosition = 1, kRopeByRow = 2 };

// Prefill-only launches (prefill_kernel): waves per workgroup and LDS ring
// stages, as in a mixed launch's prefill items.  Measured on config (c): two
// 4-wave workgroups per CU with 2-stage rings (so one workgroup's start
// overlaps the other's compute) 550-557 us against 516-518 us.
constexpr int kPrefillOnlyWaves = 8;
constexpr int kPrefillOnlyStages = 4;

// Paged attention (decode / prefill / mixed) and the dense-bias op share it.
struct AttnArgs {
  const void* q;             // query rows, heads at h*D within a row
  int64_t q_row_stride;      // elements between consecutive query rows
  void* out;
  int64_t out_row_stride;
  // paged source
  const void* k_cache;
  const void* v_cache;
  int64_t cache_slot_stride;  // elements between slots (Hkv * D)
  int64_t num_blocks;
  const int32_t* block_table;
  int64_t block_table_stride;
  int32_t block_size;         // any size >= 1
  uint32_t block_magic;       // floor(p / block_size) = div_bs(p, block_magic, block_shift)
  int32_t block_shift;
  // dense source (reference_attention contract); q/out rows are b * q_seq_stride + r
  const void* k;
  const void* v;
  int64_t k_batch_stride, k_row_stride, v_batch_stride, v_row_stride;
  const void* bias;           // [B, T_q, T] model dtype
  int64_t bias_batch_stride, bias_row_stride;
  int32_t dense_T;            // keys per batch entry
  int32_t dense_Tq;           // query rows per batch entry (q/out row = b * dense_Tq + r)
  // rope applied to q on load
  const void* rope_cos;
  const void* rope_sin;
  int64_t rope_row_stride;
  int32_t rope_mode;
  // work description
  const SeqInfo* seqs;
  const WorkItem* items;
  int32_t n_items;
  int32_t num_seqs;
  int64_t n_partials;
  float* partials;            // [n_partials][16][D] fp32
  float* partial_ml;          // [n_partials][16][2] fp32 (running max in log2 units, sum)
  int32_t* counters;          // [num_seqs * Hkv] split tickets, zero between launches
  // page-balanced decode (n_segs > 0): workgroup w runs segs[seg_ptr[w] .. seg_ptr[w + 1])
  const DecodeSeg* segs;
  const int32_t* seg_ptr;
  int32_t n_segs;
  int32_t n_seg_wgs;          // workgroups running segments; a mixed launch's prefill items follow them
  int32_t split_len;
  int32_t heads_per_wg;       // decode: kv heads per workgroup (1, 2, 4, 8)
  int32_t decode_waves;       // decode: waves per workgroup (8)
  int32_t prefill_waves;      // prefill: waves per workgroup (8)
  int32_t num_q_heads, num_kv_heads, head_dim;
  float scale;
  int32_t dtype, kv_dtype;
  // new tokens written by the attention launch itself (decode-path plans;
  // null otherwise): row q_row_start + r of k_new / v_new (model dtype, Hkv
  // heads at h * D) is key ctx_len + r of its sequence; k is rotated with the
  // q rows' cos/sin rows, both are cast to the cache dtype and stored at the
  // key's slot (block table).
  const void* k_new;
  const void* v_new;
  int64_t k_new_row_stride, v_new_row_stride;
};

struct MetadataArgs {
  const int32_t* block_table;
  int64_t block_table_stride;   // elements between rows
  int64_t bt_width;             // valid columns per row
  const int32_t* seq_lens;
  const int32_t* query_lens;
  int32_t num_seqs;
  int64_t q_seq_stride;         // > 0: padded [B, q_seq_stride] rows; 0: packed
  int32_t block_size, block_shift;   // div_bs(p, block_magic, block_shift) = p / block_size
  uint32_t block_magic;
  int64_t* slot_mapping;        // [num_rows] (may be NULL)
  int64_t* positions;           // [num_rows] (may be NULL)
  int32_t* cu_seqlens;          // [num_seqs + 1], packed layout only (may be NULL)
  int64_t num_rows;
};

// Fused QKV projection + RoPE + paged KV write (bf16 model).
struct QKVArgs {
  const void* x;                 // [num_tokens, x_row_stride] bf16
  int64_t x_row_stride;
  int64_t num_tokens;
  int32_t hidden;                // K of the projection (multiple of 32)
  const void* w_q;               // [Hq * D, hidden] bf16, row stride w_q_row_stride
  const void* w_k;               // [Hkv * D, hidden]
  const void* w_v;               // [Hkv * D, hidden]
  int64_t w_q_row_stride, w_k_row_stride, w_v_row_stride;
  void* q_out;                   // nullable: [num_tokens, q_out_row_stride] bf16
  int64_t q_out_row_stride;
  int32_t rotate_q;
  void* k_cache;
  void* v_cache;
  int64_t cache_slot_stride, num_slots;
  const int64_t* slot_mapping;   // [num_tokens]
  const int32_t* query_lens;     // nullable: skip row r >= query_lens[tok / tokens_per_seq]
  int64_t tokens_per_seq;
  const void* cos;               // [rows, rope_row_stride] bf16
  const void* sin;
  const int64_t* rope_rows;      // nullable: cos/sin row per token (else the token index)
  int64_t rope_row_stride;
  int32_t num_q_heads, num_kv_heads, head_dim;
  int32_t kv_dtype;
  // split-K path (few tokens): fp32 partials [split_count][num_tokens][heads * D]
  float* workspace;
  size_t workspace_bytes;
  int32_t cus;                   // compute units (planning)
  int32_t split_chunk, split_count;
  int32_t vec_stores;            // set by the launcher: rows aligned for 4-element stores
};

size_t qkv_workspace_bytes(int64_t num_tokens, int hidden, int heads, int head_dim, int cus);

hipError_t launch_rope_kv_write(const RopeKVWriteArgs& a, hipStream_t stream);
hipError_t launch_qkv_rope_write(const QKVArgs& a, hipStream_t stream);
hipError_t launch_build_metadata(const MetadataArgs& a, hipStream_t stream);
// MFMA kernels: bf16 or fp16 model (a.dtype), head dim 64 or 128, cache in
// the model dtype or fp8 e4m3fn
hipError_t launch_paged_attention_mfma(const AttnArgs& a, bool has_prefill, bool has_decode, hipStream_t stream);
hipError_t launch_dense_attention_mfma(const AttnArgs& a, int B, int Tq, hipStream_t stream);
hipError_t launch_attention_f32(const AttnArgs& a, bool dense, int B, int max_q, hipStream_t stream);
hipError_t launch_fill_zero_i32(int32_t* p, int64_t n, hipStream_t stream);

}  // namespace gllm

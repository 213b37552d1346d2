// fp32 attention (model dtype float32): paged decode/prefill and the dense-bias
// op.  One wave per (query head, query row, sequence); lanes split the head
// dim, keys are visited in order with an exact online softmax (expf).  This is
// the path for fp32 models (BASELINE config (a)); the bf16 MFMA kernels are the
// performance path.  Compiled with -ffp-contract=off so the q rotation rounds
// each op like the reference (gllm/model/layers/attention.py:105-118).
#include "common.h"
#include "launch.h"

namespace gllm {

template <typename KV> __device__ __forceinline__ float ldkv(const KV* p);
template <> __device__ __forceinline__ float ldkv<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ldkv<__bf16>(const __bf16* p) { return (float)*p; }
// fp8 e4m3fn cache: exact widening (the reference's .to(model dtype) after the gather)
template <> __device__ __forceinline__ float ldkv<fp8e4m3>(const fp8e4m3* p) { return __builtin_amdgcn_cvt_f32_fp8((int)p->bits, 0); }

template <bool DENSE, typename KV>
__global__ void __launch_bounds__(64) attn_f32_kernel(AttnArgs a) {
  const int hq = blockIdx.x, r = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int D = a.head_dim;
  int ctx, qlen, L;
  int64_t qrow;
  if (DENSE) {
    ctx = 0;
    qlen = a.dense_Tq;
    L = a.dense_T;
    qrow = (int64_t)b * a.dense_Tq + r;
  } else {
    if (b >= a.num_seqs) return;
    const SeqInfo si = a.seqs[b];
    ctx = si.ctx_len;
    qlen = si.q_len;
    L = ctx + qlen;
    qrow = si.q_row_start + r;
  }
  if (r >= qlen) return;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int kvh = hq / G;
  const int half = D / 2;
  const float* qp = (const float*)a.q + qrow * a.q_row_stride + (int64_t)hq * D;

  float q[4], acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    acc[i] = 0.f;
    q[i] = 0.f;
    if (d < D) {
      q[i] = qp[d];
      if (!DENSE && a.rope_mode != kRopeNone) {
        const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)(ctx + r) : qrow;
        const float* cp = (const float*)a.rope_cos + crow * a.rope_row_stride;
        const float* sp = (const float*)a.rope_sin + crow * a.rope_row_stride;
        if (d < half) {
          q[i] = __fsub_rn(__fmul_rn(qp[d], cp[d]), __fmul_rn(qp[d + half], sp[d]));
        } else {
          const int j = d - half;
          q[i] = __fadd_rn(__fmul_rn(qp[j], sp[j]), __fmul_rn(qp[d], cp[j]));
        }
      }
    }
  }
  const int nkeys = DENSE ? L : ctx + r + 1;
  const int32_t* bt = DENSE ? nullptr : a.block_table + (int64_t)b * a.block_table_stride;
  float m = kNegInf, l = 0.f;
  for (int p = 0; p < nkeys; ++p) {
    const KV *kp, *vp;
    if (DENSE) {
      kp = (const KV*)a.k + (int64_t)b * a.k_batch_stride + (int64_t)p * a.k_row_stride + (int64_t)kvh * D;
      vp = (const KV*)a.v + (int64_t)b * a.v_batch_stride + (int64_t)p * a.v_row_stride + (int64_t)kvh * D;
    } else {
      uint32_t blk = (uint32_t)bt[p >> a.block_shift];
      if (blk >= (uint64_t)a.num_blocks) blk = 0;
      const int64_t slot = (int64_t)blk * a.block_size + (p & (a.block_size - 1));
      kp = (const KV*)a.k_cache + slot * a.cache_slot_stride + (int64_t)kvh * D;
      vp = (const KV*)a.v_cache + slot * a.cache_slot_stride + (int64_t)kvh * D;
    }
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d < D) part += q[i] * ldkv<KV>(kp + d);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
    float s = part * a.scale;
    if (DENSE) s += ((const float*)a.bias)[(int64_t)b * a.bias_batch_stride + (int64_t)r * a.bias_row_stride + p];
    if (s == kNegInf) continue;
    const float mn = fmaxf(m, s);
    const float alpha = expf(m - mn);
    const float e = expf(s - mn);
    l = l * alpha + e;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d < D) acc[i] = acc[i] * alpha + e * ldkv<KV>(vp + d);
    }
    m = mn;
  }
  float* op = (float*)a.out + qrow * a.out_row_stride + (int64_t)hq * D;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) op[d] = acc[i] / l;  // l == 0 (every key masked) gives NaN, as torch's softmax
  }
}

hipError_t launch_attention_f32(const AttnArgs& a, bool dense, int B, int max_q, hipStream_t st) {
  if (B == 0 || max_q == 0) return hipSuccess;
  dim3 grid(a.num_q_heads, max_q, B), block(64);
  if (dense)
    hipLaunchKernelGGL((attn_f32_kernel<true, float>), grid, block, 0, st, a);
  else if (a.kv_dtype == kF32)
    hipLaunchKernelGGL((attn_f32_kernel<false, float>), grid, block, 0, st, a);
  else if (a.kv_dtype == kFP8)
    hipLaunchKernelGGL((attn_f32_kernel<false, fp8e4m3>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((attn_f32_kernel<false, __bf16>), grid, block, 0, st, a);
  return hipGetLastError();
}

}  // namespace gllm

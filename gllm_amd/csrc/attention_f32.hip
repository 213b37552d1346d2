// Generic attention: paged decode/prefill and the dense-bias op for fp32
// models (benchmark config (a)), for bf16 / fp16 models whose head dim the
// MFMA kernels do not take (not 64 or 128; up to 256), and for a 16-bit model
// over a cache of another dtype (f32, or the other 16-bit type).  One wave
// per (query head, query row, sequence), 64 keys per step, exact online
// softmax (expf) in fp32.  Compiled with -ffp-contract=off so the q rotation
// rounds each op like the reference (gllm/model/layers/attention.py:105-118):
// in fp32, or to the 16-bit model dtype after every op.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace gllm {

template <typename KV> __device__ __forceinline__ float ldkv(const KV* p);
template <> __device__ __forceinline__ float ldkv<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ldkv<__bf16>(const __bf16* p) { return (float)*p; }
template <> __device__ __forceinline__ float ldkv<_Float16>(const _Float16* p) { return (float)*p; }
// fp8 e4m3fn cache: exact widening (the reference's .to(model dtype) after the gather)
template <> __device__ __forceinline__ float ldkv<fp8e4m3>(const fp8e4m3* p) { return __builtin_amdgcn_cvt_f32_fp8((int)p->bits, 0); }

// model dtype: loads widen exactly; each RoPE op rounds to it
template <typename QT> __device__ __forceinline__ float rnd(float x);
template <> __device__ __forceinline__ float rnd<float>(float x) { return x; }
template <> __device__ __forceinline__ float rnd<__bf16>(float x) { return round_bf16(x); }
template <> __device__ __forceinline__ float rnd<_Float16>(float x) { return (float)(_Float16)x; }
template <typename QT> __device__ __forceinline__ void stq(QT* p, float x);
template <> __device__ __forceinline__ void stq<float>(float* p, float x) { *p = x; }
template <> __device__ __forceinline__ void stq<__bf16>(__bf16* p, float x) {
  *reinterpret_cast<uint16_t*>(p) = (uint16_t)pack_bf16x2(x, 0.f);
}
template <> __device__ __forceinline__ void stq<_Float16>(_Float16* p, float x) { *p = (_Float16)x; }

// A cached value as the reference's gather reads it: cast to the model dtype
// (attention.py:169-170, .to(q.dtype)).  Exact when the cache holds the model
// dtype, fp8 e4m3fn (a subset of every model dtype) or feeds an fp32 model;
// rounded to nearest even for an f32 cache (or the other 16-bit type) under
// a 16-bit model.
template <typename KV, typename QT>
__device__ __forceinline__ float kvld(const KV* p) {
  constexpr bool exact = std::is_same<QT, float>::value || std::is_same<KV, QT>::value ||
                         std::is_same<KV, fp8e4m3>::value;
  const float x = ldkv<KV>(p);
  if constexpr (exact) return x;
  else return rnd<QT>(x);
}

// A value of the model dtype stored in the cache dtype, as torch's
// .to(kv_dtype) rounds it (to nearest even; fp8: NaN -> 0x7f|sign).
template <typename KV> __device__ __forceinline__ KV to_kv(float x);
template <> __device__ __forceinline__ float to_kv<float>(float x) { return x; }
template <> __device__ __forceinline__ __bf16 to_kv<__bf16>(float x) {
  return __builtin_bit_cast(__bf16, (uint16_t)pack_bf16x2(x, 0.f));
}
template <> __device__ __forceinline__ _Float16 to_kv<_Float16>(float x) { return (_Float16)x; }
template <> __device__ __forceinline__ fp8e4m3 to_kv<fp8e4m3>(float x) { return fp8e4m3{fp8_byte(x)}; }

// One 4-wave workgroup per (query head, query row, sequence).  Keys go 64 at
// a time, chunk c to wave c % 4: lane j scores key p0 + j against q (q read
// from LDS, so every lane has all of it), one wave max / sum per chunk
// updates the wave's exact online softmax (expf), then the lanes switch to
// the head dims (d = lane + 64 i, i < NI) and accumulate the chunk's
// p-weighted V rows, each key's p and slot read out of its lane.  NI = 1
// (D <= 64, a multiple of 4): the chunk's 64 V rows (one value per lane
// each) and then each lane's whole K row are loaded before any is used, so K
// and V arrive in one memory round trip; NI = 4: 32 keys' V rows per batch
// of loads, after the scores.  The four waves' (max,
// sum, acc) merge through LDS at the end.
// FUSED (a.k_new != null, at most kFusedRows query rows per sequence): the
// new tokens' K/V are written by this launch.  Every workgroup rotates and
// casts the new keys it sees (ctx .. ctx + r) itself into LDS, the value the
// cache round trip gives (stored in KV, read back as QT); the main loop covers
// the cached keys [0, ctx) and wave 0 adds the new ones afterwards.  The
// workgroup of the group's first query head and the sequence's last row
// computes all of the sequence's new tokens and stores them at their slots
// (block table); no workgroup of the launch reads those slots.
constexpr int kFusedRows = 16;
template <bool DENSE, typename KV, typename QT, int NI, bool FUSED>
__global__ void __launch_bounds__(256) attn_f32_kernel(AttnArgs a) {
  constexpr int NWV = 4;                  // waves per workgroup
  constexpr int VB = NI == 1 ? 64 : 32;   // V rows per batch of loads
  __shared__ __attribute__((aligned(16))) float qs[256];
  __shared__ float mrg[NWV][2 + 256];     // per wave: max, sum, acc[D]
  __shared__ float nkv[2][FUSED ? kFusedRows : 1][FUSED ? 64 * NI : 1];   // new keys' K / V (FUSED)
  const int hq = blockIdx.x, r = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int D = a.head_dim;
  int ctx, qlen, L;
  int64_t qrow, row0 = 0;
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
    row0 = si.q_row_start;
  }
  if (r >= qlen) return;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int kvh = hq / G;
  const int half = D / 2;
  const QT* qp = (const QT*)a.q + qrow * a.q_row_stride + (int64_t)hq * D;

  for (int d = tid; d < D; d += 64 * NWV) {
    float qv = (float)qp[d];
    if (!DENSE && a.rope_mode != kRopeNone) {
      const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)(ctx + r) : qrow;
      const QT* cp = (const QT*)a.rope_cos + crow * a.rope_row_stride;
      const QT* sp = (const QT*)a.rope_sin + crow * a.rope_row_stride;
      if (d < half) {
        qv = rnd<QT>(__fsub_rn(rnd<QT>(__fmul_rn((float)qp[d], (float)cp[d])),
                               rnd<QT>(__fmul_rn((float)qp[d + half], (float)sp[d]))));
      } else {
        const int j = d - half;
        qv = rnd<QT>(__fadd_rn(rnd<QT>(__fmul_rn((float)qp[j], (float)sp[j])),
                               rnd<QT>(__fmul_rn((float)qp[d], (float)cp[j]))));
      }
    }
    qs[d] = qv;
  }
  for (int d = D + tid; d < 64 * NI; d += 64 * NWV) qs[d] = 0.f;   // dims past D score 0
  if constexpr (FUSED) {
    // element pairs (token t, dims j and j + D/2); the writer takes every token
    const bool writer = hq % G == 0 && r == qlen - 1;
    const int nt = writer ? qlen : r + 1;
    const int32_t* btr = a.block_table + (int64_t)b * a.block_table_stride;
    for (int e = tid; e < nt * half; e += 64 * NWV) {
      const int t = e / half, j = e - t * half;
      const int64_t row = row0 + t;
      const QT* kn = (const QT*)a.k_new + row * a.k_new_row_stride + (int64_t)kvh * D;
      const QT* vn = (const QT*)a.v_new + row * a.v_new_row_stride + (int64_t)kvh * D;
      float lo = (float)kn[j], hi = (float)kn[j + half];
      if (a.rope_mode != kRopeNone) {
        const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)(ctx + t) : row;
        const float c = (float)((const QT*)a.rope_cos)[crow * a.rope_row_stride + j];
        const float sn = (float)((const QT*)a.rope_sin)[crow * a.rope_row_stride + j];
        const float x1 = lo, x2 = hi;
        lo = rnd<QT>(__fsub_rn(rnd<QT>(__fmul_rn(x1, c)), rnd<QT>(__fmul_rn(x2, sn))));
        hi = rnd<QT>(__fadd_rn(rnd<QT>(__fmul_rn(x1, sn)), rnd<QT>(__fmul_rn(x2, c))));
      }
      const KV k1 = to_kv<KV>(lo), k2 = to_kv<KV>(hi);
      const KV v1 = to_kv<KV>((float)vn[j]), v2 = to_kv<KV>((float)vn[j + half]);
      if (t <= r) {
        nkv[0][t][j] = kvld<KV, QT>(&k1);
        nkv[0][t][j + half] = kvld<KV, QT>(&k2);
        nkv[1][t][j] = kvld<KV, QT>(&v1);
        nkv[1][t][j + half] = kvld<KV, QT>(&v2);
      }
      if (writer) {
        const int p = ctx + t;
        const uint32_t bi = div_bs((uint32_t)p, a.block_magic, a.block_shift);
        const uint32_t blk = (uint32_t)btr[bi];
        if (blk < (uint64_t)a.num_blocks) {   // never address outside the pool
          const int64_t off = ((int64_t)blk * a.block_size + (p - (int64_t)bi * a.block_size)) * a.cache_slot_stride +
                              (int64_t)kvh * D + j;
          KV* kc = (KV*)a.k_cache + off;
          KV* vc = (KV*)a.v_cache + off;
          kc[0] = k1; kc[half] = k2;
          vc[0] = v1; vc[half] = v2;
        }
      }
    }
  }
  __syncthreads();
  const int nkeys = DENSE ? L : (FUSED ? ctx : ctx + r + 1);
  const int32_t* bt = DENSE ? nullptr : a.block_table + (int64_t)b * a.block_table_stride;
  const KV* kbase = DENSE ? (const KV*)a.k + (int64_t)b * a.k_batch_stride + (int64_t)kvh * D
                          : (const KV*)a.k_cache + (int64_t)kvh * D;
  const KV* vbase = DENSE ? (const KV*)a.v + (int64_t)b * a.v_batch_stride + (int64_t)kvh * D
                          : (const KV*)a.v_cache + (int64_t)kvh * D;
  const int64_t kstride = DENSE ? a.k_row_stride : a.cache_slot_stride;
  const int64_t vstride = DENSE ? a.v_row_stride : a.cache_slot_stride;
  const QT* brow = DENSE ? (const QT*)a.bias + (int64_t)b * a.bias_batch_stride + (int64_t)r * a.bias_row_stride
                         : nullptr;
  float m = kNegInf, l = 0.f;
  float acc[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) acc[i] = 0.f;
  for (int p0 = 64 * wave; p0 < nkeys; p0 += 64 * NWV) {
    const int p = p0 + lane;
    const bool valid = p < nkeys;
    const int nk = min(64, nkeys - p0);
    // row of key p in k (dense) or in the paged cache
    int64_t row = 0;
    if (valid) {
      if (DENSE) {
        row = p;
      } else {
        const uint32_t bi = div_bs((uint32_t)p, a.block_magic, a.block_shift);
        uint32_t blk = (uint32_t)bt[bi];
        if (blk >= (uint64_t)a.num_blocks) blk = 0;   // never address outside the pool
        row = (int64_t)blk * a.block_size + (p - (int)bi * a.block_size);
      }
    }
    const int rlo = (int)(uint32_t)row, rhi = (int)((uint64_t)row >> 32);
    // V rows of key j (keys past the chunk re-read its last row, weight 0)
    auto load_v = [&](int j0, float (&vv)[VB][NI]) {
#pragma unroll
      for (int u = 0; u < VB; ++u) {
        const int j = min(j0 + u, nk - 1);
        const int64_t rj = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane(rhi, j) << 32) |
                                     (uint32_t)__builtin_amdgcn_readlane(rlo, j));
        const KV* vp = vbase + rj * vstride;
#pragma unroll
        for (int i = 0; i < NI; ++i) {   // every lane loads (dims past D re-read dim D - 1): no branch per load
          const int d = lane + 64 * i;
          const float v = kvld<KV, QT>(vp + min(d, D - 1));
          vv[u][i] = d < D ? v : 0.f;
        }
      }
    };
    float vpre[NI == 1 ? VB : 1][NI];
    if constexpr (NI == 1) load_v(0, vpre);
    float s = kNegInf;
    if (valid) {
      const KV* kp = kbase + row * kstride;
      float dot = 0.f;
      if constexpr (NI == 1) {
        // D <= 64, a multiple of 4: the whole row's loads are issued before
        // any is used (16 chunks of 4 dims; chunks past D re-read the last
        // one and meet q = 0), then summed chunk by chunk in dim order
        float kv[16][4];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          const int cs = min(4 * c, D - 4);
#pragma unroll
          for (int j = 0; j < 4; ++j) kv[c][j] = kvld<KV, QT>(kp + cs + j);
        }
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          const f32x4 qv = *reinterpret_cast<const f32x4*>(qs + 4 * c);
          dot += qv[0] * kv[c][0] + qv[1] * kv[c][1] + qv[2] * kv[c][2] + qv[3] * kv[c][3];
        }
      } else {
        int d = 0;
#pragma unroll 16
        for (; d + 4 <= D; d += 4) {
          const f32x4 qv = *reinterpret_cast<const f32x4*>(qs + d);
          dot += qv[0] * kvld<KV, QT>(kp + d) + qv[1] * kvld<KV, QT>(kp + d + 1) + qv[2] * kvld<KV, QT>(kp + d + 2) +
                 qv[3] * kvld<KV, QT>(kp + d + 3);
        }
        for (; d < D; ++d) dot += qs[d] * kvld<KV, QT>(kp + d);   // head dims not a multiple of 4
      }
      s = dot * a.scale;
      if (DENSE) s += (float)brow[p];
    }
    float cm = s;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
    if (cm == kNegInf) continue;                       // every key of the chunk masked
    const float mn = fmaxf(m, cm);
    const float alpha = expf(m - mn);                  // m = -inf: 0
    const float e = s == kNegInf ? 0.f : expf(s - mn);
    float es = e;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) es += __shfl_xor(es, off);
    l = l * alpha + es;
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i] *= alpha;
    // p-weighted V rows summed in key order
    auto accumulate = [&](int j0, const float (&vv)[VB][NI]) {
#pragma unroll
      for (int u = 0; u < VB; ++u) {
        const int j = min(j0 + u, nk - 1);
        const float pe = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(e), j));
        const float pj = j0 + u < nk ? pe : 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) acc[i] += pj * vv[u][i];
      }
    };
    if constexpr (NI == 1) {
      accumulate(0, vpre);
    } else {
      for (int j0 = 0; j0 < nk; j0 += VB) {
        float vv[VB][NI];
        load_v(j0, vv);
        accumulate(j0, vv);
      }
    }
    m = mn;
  }
  if constexpr (FUSED) {
    // the new keys ctx .. ctx + r (every one visible to row r), from LDS
    if (wave == 0) {
      const int nk = r + 1;
      float s = kNegInf;
      if (lane < nk) {
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += qs[d] * nkv[0][lane][d];
        s = dot * a.scale;
      }
      float cm = s;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
      const float mn = fmaxf(m, cm);
      const float alpha = expf(m - mn);
      const float e = lane < nk ? expf(s - mn) : 0.f;
      float es = e;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) es += __shfl_xor(es, off);
      l = l * alpha + es;
#pragma unroll
      for (int i = 0; i < NI; ++i) acc[i] *= alpha;
      for (int u = 0; u < nk; ++u) {
        const float pj = __shfl(e, u);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int d = lane + 64 * i;
          if (d < D) acc[i] += pj * nkv[1][u][d];
        }
      }
      m = mn;
    }
  }
  // merge the waves' states (exact LSE merge; a wave without keys has
  // m = -inf and weight 0)
  if (lane == 0) {
    mrg[wave][0] = m;
    mrg[wave][1] = l;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = lane + 64 * i;
    if (d < D) mrg[wave][2 + d] = acc[i];
  }
  __syncthreads();
  if (wave != 0) return;
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < NWV; ++w) M = fmaxf(M, mrg[w][0]);
  float wt[NWV], lt = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    wt[w] = mrg[w][0] == kNegInf ? 0.f : expf(mrg[w][0] - M);
    lt += wt[w] * mrg[w][1];
  }
  QT* op = (QT*)a.out + qrow * a.out_row_stride + (int64_t)hq * D;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = lane + 64 * i;
    if (d < D) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < NWV; ++w) o += wt[w] * mrg[w][2 + d];
      stq<QT>(op + d, o / lt);   // lt == 0 (every key masked) gives NaN, as torch's softmax
    }
  }
}

template <typename QT, int NI, bool FUSED>
static hipError_t launch_f32_kv(const AttnArgs& a, dim3 grid, hipStream_t st) {
  const dim3 block(256);
  switch (a.kv_dtype) {
    case kF32: hipLaunchKernelGGL((attn_f32_kernel<false, float, QT, NI, FUSED>), grid, block, 0, st, a); break;
    case kBF16: hipLaunchKernelGGL((attn_f32_kernel<false, __bf16, QT, NI, FUSED>), grid, block, 0, st, a); break;
    case kF16: hipLaunchKernelGGL((attn_f32_kernel<false, _Float16, QT, NI, FUSED>), grid, block, 0, st, a); break;
    case kFP8: hipLaunchKernelGGL((attn_f32_kernel<false, fp8e4m3, QT, NI, FUSED>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Cache dtype KV under model dtype QT (paged), or QT throughout (dense).
template <typename QT, int NI>
static hipError_t launch_f32_qt(const AttnArgs& a, bool dense, dim3 grid, hipStream_t st) {
  const dim3 block(256);
  if (dense) {
    hipLaunchKernelGGL((attn_f32_kernel<true, QT, QT, NI, false>), grid, block, 0, st, a);
    return hipGetLastError();
  }
  if (a.k_new) return launch_f32_kv<QT, NI, true>(a, grid, st);
  return launch_f32_kv<QT, NI, false>(a, grid, st);
}

template <int NI>
static hipError_t launch_f32_ni(const AttnArgs& a, bool dense, dim3 grid, hipStream_t st) {
  switch (a.dtype) {
    case kF32: return launch_f32_qt<float, NI>(a, dense, grid, st);
    case kBF16: return launch_f32_qt<__bf16, NI>(a, dense, grid, st);
    case kF16: return launch_f32_qt<_Float16, NI>(a, dense, grid, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attention_f32(const AttnArgs& a, bool dense, int B, int max_q, hipStream_t st) {
  if (B == 0 || max_q == 0) return hipSuccess;
  if (a.head_dim <= 0 || a.head_dim > 256) return hipErrorInvalidValue;
  const dim3 grid(a.num_q_heads, max_q, B);
  if (a.head_dim <= 64 && a.head_dim % 4 == 0) return launch_f32_ni<1>(a, dense, grid, st);
  return launch_f32_ni<4>(a, dense, grid, st);
}

}  // namespace gllm

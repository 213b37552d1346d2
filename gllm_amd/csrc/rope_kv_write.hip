// Fused rotate-half RoPE + paged KV-cache write.  Model dtype f32, bf16 or
// f16; cache f32, bf16, f16 or fp8 e4m3fn, in any pairing (each written value
// cast like torch's .to(kv_dtype)).
//
// Replaces gllm/model/layers/attention.py:151-161 (apply_rope on k, the
// index_put_ of k/v through query_slot_mapping) and, optionally, the q half
// of apply_rope (attention.py:76-119).  Every arithmetic step is rounded to
// the model dtype in the same order as the reference's torch ops, so the
// written K rows are bit-identical to the reference's (no FMA contraction:
// this unit is compiled with -ffp-contract=off and uses explicit rounding).
#include "common.h"
#include "launch.h"

namespace gllm {

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 16-byte vector
  __device__ static void load(const void* p, float* v) {
    u32x4 w = ld16(p);
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(w[i]);
  }
  // attention.py:105-118: [x1*c - x2*s, x1*s + x2*c], no contraction
  __device__ static void rope(float& x1, float& x2, float c, float s) {
    const float lo = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
    const float hi = __fadd_rn(__fmul_rn(x1, s), __fmul_rn(x2, c));
    x1 = lo;
    x2 = hi;
  }
};
template <> struct Elem<__bf16> {
  static constexpr int kVec = 8;
  __device__ static void load(const void* p, float* v) { unpack_bf16x8(ld16(p), v); }
  // the same with every op rounded to bf16 (RNE), like torch's bf16 ops
  __device__ static void rope(float& x1, float& x2, float c, float s) { rope_pair_bf16(x1, x2, c, s); }
};
template <> struct Elem<_Float16> {
  static constexpr int kVec = 8;
  __device__ static void load(const void* p, float* v) { unpack8<_Float16>(ld16(p), v); }
  // every op rounded to fp16 (RNE), like torch's fp16 ops
  __device__ static void rope(float& x1, float& x2, float c, float s) { rope_pair<_Float16>(x1, x2, c, s); }
};

// Store `n` values (already representable in T when T is the model dtype)
// as element type S at p.
template <typename S> __device__ void store_vals(void* p, const float* v, int n);
template <> __device__ void store_vals<float>(void* p, const float* v, int n) {
  float* o = reinterpret_cast<float*>(p);
  if (n == 4) {
    u32x4 w;
    for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(v[i]);
    st16(o, w);
  } else {
    for (int i = 0; i < n; ++i) o[i] = v[i];
  }
}
template <> __device__ void store_vals<__bf16>(void* p, const float* v, int n) {
  if (n == 8) {
    u32x4 w;
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    st16(p, w);
  } else {  // n == 4
    u32x2 w;
    for (int i = 0; i < 2; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    st8(p, w);
  }
}

template <> __device__ void store_vals<_Float16>(void* p, const float* v, int n) {
  if (n == 8) {
    st16(p, pack8<_Float16>(v));
  } else {  // n == 4
    st8(p, u32x2{E16<_Float16>::pack2(v[0], v[1]), E16<_Float16>::pack2(v[2], v[3])});
  }
}

// fp8 cache: the model-dtype values are cast like torch's .to(float8_e4m3fn).
template <> __device__ void store_vals<fp8e4m3>(void* p, const float* v, int n) {
  if (n == 8) {
    st8(p, u32x2{pack_fp8x4(v[0], v[1], v[2], v[3]), pack_fp8x4(v[4], v[5], v[6], v[7])});
  } else {  // n == 4
    *reinterpret_cast<uint32_t*>(p) = pack_fp8x4(v[0], v[1], v[2], v[3]);
  }
}

// One wave per token at a time (grid-stride over tokens): the token's slot,
// cos/sin row and padding test are wave-uniform scalar loads, and the lanes
// take the token's items — K vectors of rotate pairs, V vectors, Q vectors of
// rotate pairs — 64 at a time.
template <typename T, typename KV>
__global__ void __launch_bounds__(256) rope_kv_write_kernel(RopeKVWriteArgs a) {
  constexpr int V = Elem<T>::kVec;
  const int D = a.head_dim, half = D / 2;
  const int pv = half / V;          // vectors per half head
  const int dv = D / V;             // vectors per head
  const int k_items = a.k ? a.num_kv_heads * pv : 0;
  const int v_items = a.k ? a.num_kv_heads * dv : 0;
  const int q_items = a.q_out ? a.num_q_heads * pv : 0;
  const int per_tok = k_items + v_items + q_items;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpb = blockDim.x >> 6;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < a.num_tokens; tok += (int64_t)gridDim.x * wpb) {
    // Padded rows of the reference's [B, T_q] layout (r >= query_lens[b])
    // are skipped whole: no K/V write (the reference sends them to dummy slot
    // 0) and no q rotation, so their cos/sin rows are never read (their
    // positions may lie past the table in mixed batches); their q_out rows
    // are left as they are.  K/V of a real row are written unless its slot is
    // outside the pool (never written).
    if (a.query_lens) {
      const int64_t b = tok / a.tokens_per_seq, r = tok - b * a.tokens_per_seq;
      if (r >= a.query_lens[b]) continue;
    }
    bool kv_ok = a.k != nullptr;
    int64_t slot = -1;
    if (kv_ok) {
      slot = a.slot_mapping[tok];
      kv_ok = slot >= 0 && slot < a.num_slots;
    }
    const int u0 = kv_ok ? 0 : k_items + v_items;
    const int64_t crow = a.rope_rows ? a.rope_rows[tok] : tok;
    for (int u = u0 + lane; u < per_tok; u += 64) {
      const char* cosp = reinterpret_cast<const char*>(a.cos) + crow * a.rope_row_stride * sizeof(T);
      const char* sinp = reinterpret_cast<const char*>(a.sin) + crow * a.rope_row_stride * sizeof(T);
      if (u < k_items || u >= k_items + v_items) {
        // rotate one vector of pairs (x[j], x[j + D/2]) of K or Q
        bool is_q = u >= k_items + v_items;
        int uu = is_q ? u - k_items - v_items : u;
        int h = uu / pv, j0 = (uu - h * pv) * V;
        const char* src = reinterpret_cast<const char*>(is_q ? a.q : a.k) +
                          (tok * (is_q ? a.q_row_stride : a.k_row_stride) + (int64_t)h * D) * sizeof(T);
        float x1[V], x2[V], c[V], s[V], lo[V], hi[V];
        Elem<T>::load(src + j0 * sizeof(T), x1);
        Elem<T>::load(src + (j0 + half) * sizeof(T), x2);
        Elem<T>::load(cosp + j0 * sizeof(T), c);
        Elem<T>::load(sinp + j0 * sizeof(T), s);
  #pragma unroll
        for (int i = 0; i < V; ++i) {
          lo[i] = x1[i];
          hi[i] = x2[i];
          Elem<T>::rope(lo[i], hi[i], c[i], s[i]);   // each op in T
        }
        if (is_q) {
          char* dst = reinterpret_cast<char*>(a.q_out) + (tok * a.q_out_row_stride + (int64_t)h * D) * sizeof(T);
          store_vals<T>(dst + j0 * sizeof(T), lo, V);
          store_vals<T>(dst + (j0 + half) * sizeof(T), hi, V);
        } else {
          char* dst = reinterpret_cast<char*>(a.k_cache) + (slot * a.cache_slot_stride + (int64_t)h * D) * sizeof(KV);
          store_vals<KV>(dst + j0 * sizeof(KV), lo, V);
          store_vals<KV>(dst + (j0 + half) * sizeof(KV), hi, V);
        }
      } else {
        int uu = u - k_items;
        int h = uu / dv, j0 = (uu - h * dv) * V;
        const char* src = reinterpret_cast<const char*>(a.v) + (tok * a.v_row_stride + (int64_t)h * D + j0) * sizeof(T);
        float x[V];
        Elem<T>::load(src, x);
        char* dst = reinterpret_cast<char*>(a.v_cache) + (slot * a.cache_slot_stride + (int64_t)h * D + j0) * sizeof(KV);
        store_vals<KV>(dst, x, V);
      }
    }
  }
}

// Model dtype T; the cache's from a.kv_dtype (q-only calls carry no cache).
template <typename T>
static hipError_t launch_rope_kv_t(const RopeKVWriteArgs& a, dim3 grid, hipStream_t stream) {
  const dim3 block(256);
  switch (a.k ? a.kv_dtype : a.dtype) {
    case kF32: hipLaunchKernelGGL((rope_kv_write_kernel<T, float>), grid, block, 0, stream, a); break;
    case kBF16: hipLaunchKernelGGL((rope_kv_write_kernel<T, __bf16>), grid, block, 0, stream, a); break;
    case kF16: hipLaunchKernelGGL((rope_kv_write_kernel<T, _Float16>), grid, block, 0, stream, a); break;
    case kFP8: hipLaunchKernelGGL((rope_kv_write_kernel<T, fp8e4m3>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope_kv_write(const RopeKVWriteArgs& a, hipStream_t stream) {
  const int V = a.dtype == kF32 ? 4 : 8;
  const int64_t per_tok = (a.k ? (int64_t)a.num_kv_heads * (a.head_dim / 2 / V + a.head_dim / V) : 0) +
                          (a.q_out ? (int64_t)a.num_q_heads * (a.head_dim / 2 / V) : 0);
  if (a.num_tokens * per_tok == 0) return hipSuccess;
  int64_t blocks = (a.num_tokens + 3) / 4;    // 4 waves of one token each
  if (blocks > 65536) blocks = 65536;
  const dim3 grid((unsigned)blocks);
  switch (a.dtype) {
    case kF32: return launch_rope_kv_t<float>(a, grid, stream);
    case kBF16: return launch_rope_kv_t<__bf16>(a, grid, stream);
    case kF16: return launch_rope_kv_t<_Float16>(a, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gllm

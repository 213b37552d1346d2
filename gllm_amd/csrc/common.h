// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Lane layouts below were checked on an MI355X with an in-bounds probe:
//   v_mfma_f32_16x16x32_bf16: A[m=l%16][k=8*(l/16)+i], B[k=8*(l/16)+i][n=l%16],
//                             C[m=4*(l/16)+j][n=l%16]            (i<8, j<4)
//   v_mfma_f32_32x32x16_bf16: A[m=l%32][k=8*(l/32)+i], B[k=8*(l/32)+i][n=l%32],
//                             C[m=8*(j/4)+4*(l/32)+j%4][n=l%32]  (i<8, j<16)
//   ds_read_b64_tr_b16 (per 16-lane group, lane s supplies 4 x 16-bit D[s][0..3]):
//                             lane i receives D[4*j + i/4][i%4], j = 0..3
//   permlane16_swap(x, x) / permlane32_swap(x, x): max(r0, r1) is the max of x
//                             over lanes {l, l^16} / {l, l^32}.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gllm {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------- bf16 bits
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Round-to-nearest-even fp32 -> bf16 bits (quiet NaN kept NaN), the rounding
// torch applies when it stores a bf16 result.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even, like torch's bf16 stores.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(pack_bf16x2(f, 0.f) & 0xffffu); }
// Two values rounded the same way with one convert.
__device__ __forceinline__ void round2_bf16(float& a, float& b) {
  const uint32_t w = pack_bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}
// One rotate-half pair, each op rounded to bf16 like the reference's torch ops
// (gllm/model/layers/attention.py:105-118): [x1 c - x2 s, x1 s + x2 c].
__device__ __forceinline__ void rope_pair_bf16(float& x1, float& x2, float c, float s) {
  float a = __fmul_rn(x1, c), b = __fmul_rn(x2, s), e = __fmul_rn(x1, s), f = __fmul_rn(x2, c);
  round2_bf16(a, b);
  round2_bf16(e, f);
  x1 = __fsub_rn(a, b);
  x2 = __fadd_rn(e, f);
  round2_bf16(x1, x2);
}

// 8 fp32 -> one MFMA operand of 8 bf16.
__device__ __forceinline__ bf16x8 to_bf16x8(const float* v) {
  u32x4 w;
  w[0] = pack_bf16x2(v[0], v[1]);
  w[1] = pack_bf16x2(v[2], v[3]);
  w[2] = pack_bf16x2(v[4], v[5]);
  w[3] = pack_bf16x2(v[6], v[7]);
  return __builtin_bit_cast(bf16x8, w);
}

__device__ __forceinline__ void unpack_bf16x8(const u32x4 w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// ---------------------------------------------------------------- fp8 (OCP e4m3fn)
// Storage type of an fp8 KV cache (torch.float8_e4m3fn).  Conversions follow
// torch's cast, checked on gfx950 against torch for all 256 codes and the
// rounding / overflow boundaries: round to nearest even (subnormals too),
// |x| > 464 -> NaN 0x7f|sign, 464 -> 448.  The hardware's f32 -> fp8 agrees
// except that it gives 0xff for every NaN; torch gives 0x7f|sign (fixed up).
struct fp8e4m3 { uint8_t bits; };

__device__ __forceinline__ uint32_t fp8_nan_fix(uint32_t w, float x, int byte) {
  if (x != x) {
    const uint32_t code = 0x7fu | ((__float_as_uint(x) >> 24) & 0x80u);
    w = (w & ~(0xffu << (8 * byte))) | (code << (8 * byte));
  }
  return w;
}

// 4 fp32 values -> 4 fp8 bytes (little-endian order a, b, c, d).
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  if ((a != a) | (b != b) | (c != c) | (d != d)) {
    w = fp8_nan_fix(w, a, 0);
    w = fp8_nan_fix(w, b, 1);
    w = fp8_nan_fix(w, c, 2);
    w = fp8_nan_fix(w, d, 3);
  }
  return w;
}

// One value -> its fp8 byte (torch's cast, NaN -> 0x7f|sign).
__device__ __forceinline__ uint8_t fp8_byte(float x) { return (uint8_t)(pack_fp8x4(x, 0.f, 0.f, 0.f) & 0xffu); }

// 4 fp8 bytes -> 4 fp32 (exact).
__device__ __forceinline__ void unpack_fp8x4(uint32_t w, float* v) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  v[0] = lo[0]; v[1] = lo[1]; v[2] = hi[0]; v[3] = hi[1];
}

// 8 fp8 bytes -> 8 bf16 (exact: every e4m3 value is a bf16 value).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, HI));
}
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
  return u32x4{fp8x2_to_bf16x2<false>(w0), fp8x2_to_bf16x2<true>(w0), fp8x2_to_bf16x2<false>(w1),
               fp8x2_to_bf16x2<true>(w1)};
}

// ---------------------------------------------------------------- 16-bit model types
// The MFMA kernels take a bf16 or an fp16 model (T = __bf16 or _Float16).
// Operands move as raw 32-bit words (two elements each); E16<T> converts,
// rounds (RNE, like torch's stores in T) and multiplies per type.
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

template <typename T> struct E16;
template <> struct E16<__bf16> {
  static constexpr bool kF16 = false;
  __device__ static uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  __device__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static f32x4 mfma16k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c,
                                                     0, 0, 0);
  }
  // 2 fp8 e4m3 values (bytes 2 HI, 2 HI + 1 of w) -> 2 elements (exact)
  template <bool HI> __device__ static uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, HI));
  }
  // c + lo + hi (one v_dot2c against 1.0)
  __device__ static float add2(uint32_t w, float c) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, c, false);
  }
};
template <> struct E16<_Float16> {
  static constexpr bool kF16 = true;
  __device__ static uint32_t pack2(float lo, float hi) {   // v_cvt_pk_f16_f32: RNE, overflow to inf
    f16x2 r;
    r[0] = (_Float16)lo;
    r[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ static float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[0]; }
  __device__ static float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w)[1]; }
  __device__ static f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  __device__ static f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  __device__ static f32x4 mfma16k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c,
                                                 0, 0, 0);
  }
  // every e4m3 value is an fp16 value: exact
  template <bool HI> __device__ static uint32_t fp8x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, HI));
  }
  __device__ static float add2(uint32_t w, float c) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, c, false);
  }
};

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4 w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = E16<T>::lo(w[i]);
    v[2 * i + 1] = E16<T>::hi(w[i]);
  }
}
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* v) {
  return u32x4{E16<T>::pack2(v[0], v[1]), E16<T>::pack2(v[2], v[3]), E16<T>::pack2(v[4], v[5]),
               E16<T>::pack2(v[6], v[7])};
}
// two values rounded to T with one convert
template <typename T>
__device__ __forceinline__ void round2(float& a, float& b) {
  const uint32_t w = E16<T>::pack2(a, b);
  a = E16<T>::lo(w);
  b = E16<T>::hi(w);
}
// Makes rounded fp16 values opaque to the optimizer, which would otherwise
// narrow round(x1 c) - round(x2 s) to half-precision ops, which instruction
// selection then fuses into one FMA under fp-contract=fast (a global backend
// option, so a source pragma does not stop it), dropping the product's own
// rounding.  No instruction is emitted.
__device__ __forceinline__ void opaque4(float& a, float& b, float& c, float& d) {
  asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}

// one rotate-half pair with every op rounded to T (attention.py:105-118)
template <typename T>
__device__ __forceinline__ void rope_pair(float& x1, float& x2, float c, float s) {
  float a = __fmul_rn(x1, c), b = __fmul_rn(x2, s), e = __fmul_rn(x1, s), f = __fmul_rn(x2, c);
  round2<T>(a, b);
  round2<T>(e, f);
  if constexpr (E16<T>::kF16) opaque4(a, b, e, f);   // bf16 has no half-width arithmetic to narrow to
  x1 = __fsub_rn(a, b);
  x2 = __fadd_rn(e, f);
  round2<T>(x1, x2);
}
// 8 fp8 bytes -> 8 elements of T (exact)
template <typename T>
__device__ __forceinline__ u32x4 fp8x8_to(uint32_t w0, uint32_t w1) {
  return u32x4{E16<T>::template fp8x2<false>(w0), E16<T>::template fp8x2<true>(w0),
               E16<T>::template fp8x2<false>(w1), E16<T>::template fp8x2<true>(w1)};
}

// ---------------------------------------------------------------- memory
// Direct global -> LDS copy of 16 bytes per lane: lane l's bytes land at
// lds_base + 16 l (lds_base wave-uniform, in M0).  Written as inline asm so
// the compiler does not wait for every outstanding copy before each LDS read;
// the kernel waits for its own copies with wait_vmcnt before the barrier that
// publishes a stage.  M0 is set inside the asm and listed as clobbered (the
// compiler warns that it reserves M0; in these kernels every M0 write in the
// generated code is this asm's own, checked in the assembly).
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_base) : "memory", "m0");
}
// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Transposed LDS read: see the layout note at the top of this file.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* lds_addr) {
  i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)const_cast<void*>(lds_addr));
  return __builtin_bit_cast(u32x2, r);
}

// ---------------------------------------------------------------- MFMA
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- cross-lane
__device__ __forceinline__ float max_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Division by the KV block size (any size >= 1): floor(p / bs) for
// 0 <= p < 2^31 is umulhi(2p, magic) >> shift with k = ceil(log2 bs),
// magic = ceil(2^(31+k) / bs), shift = k.  Exact: with e = magic bs - 2^(31+k)
// (0 <= e < bs <= 2^k) the quotient is p / bs + p e / (bs 2^(31+k)), and
// p e < 2^(31+k) keeps the error term below 1/bs.  A power of two 2^k gives
// magic = 2^31, i.e. p >> k.
__device__ __forceinline__ uint32_t div_bs(uint32_t p, uint32_t magic, int shift) {
  return __umulhi(p << 1, magic) >> shift;
}

// Sequence / work descriptors shared by host planner and kernels.
struct SeqInfo {
  int32_t q_row_start;   // first query row of the sequence in q / out
  int32_t ctx_len;       // c_i = seq_len - query_len
  int32_t q_len;         // q_i
  int32_t nsplits;       // decode-path splits (0 for prefill-path sequences)
  int32_t partial_base;  // first partial index of (seq, kv head 0, split 0)
  int32_t pad0, pad1, pad2;
};

enum : int32_t { kItemPrefill = 0, kItemDecode = 1 };

// Keys per split of a decode sequence of L keys cut into n equal splits
// (16-key multiples; the last split takes the rest).  The planner picks n so
// that every split is non-empty: n = ceil(L / split_len_of(L, n0)).
__host__ __device__ inline int32_t split_len_of(int64_t L, int32_t n) {
  return (int32_t)(((L + n - 1) / n + 15) / 16 * 16);
}

// One workgroup's work, with its sequence's facts folded in so the kernel's
// prologue needs one dependent load less.
struct WorkItem {
  int32_t kind_b;        // kind | (b << 8); b = prefill: wave-group id, decode: kv-head group
  int32_t seq;
  int32_t a;             // prefill: kv head; decode: split index
  int32_t q_row_start;
  int32_t ctx_len;
  int32_t q_len;
  int32_t nsplits;
  int32_t partial_base;
};

// Key range [k0, k1) of one (sequence, kv-head group) for the page-balanced
// decode launch: the workgroups split the batch's 16-key units evenly, so a
// sequence's keys may be spread over several workgroups.  Its nseg segments
// write partials at pbase + head_in_group * nseg + ord; the workgroup that
// draws the last ticket of counters[ticket] merges them.
struct DecodeSeg {
  int32_t seq;
  int32_t hg;            // kv-head group (heads hg * HW .. hg * HW + HW - 1)
  int32_t k0, k1;
  int32_t q_row_start;
  int32_t ctx_len;
  int32_t q_len;
  int32_t nseg;          // segments of this (sequence, group); 1 = written directly
  int32_t pbase;
  int32_t ord;
  int32_t ticket;        // counter index of this (sequence, group)
  int32_t pad;
};

}  // namespace gllm

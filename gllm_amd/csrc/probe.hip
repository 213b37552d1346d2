// Memory-path probes behind bench.py's box ceilings: what plain access
// patterns reach on this GPU, as context for the attention kernels' roofline
// fractions (which are priced against the published peaks, not these).  Not
// part of the attention path; built into their own libgllm_probe.so.
//
//   gllm_probe_read:    every workgroup streams its contiguous share of a
//                       buffer with 16-byte loads, 8 in flight per lane (a
//                       buffer well above the 256 MB MALL measures HBM).
//   gllm_probe_lds_dma: every workgroup copies 4 KB steps of an L2-sized
//                       window into an LDS ring with global_load_lds_dwordx4,
//                       NS - 1 steps in flight, no compute (the load path the
//                       prefill kernel's K/V ring uses).
//   gllm_probe_mfma:    one wave's cycles per 8 bf16 32x32x16 MFMAs, alone
//                       or with 64 independent FMAs between them.
//   gllm_probe_empty:   a grid of workgroups that do nothing (launch cost).
#include "common.h"

namespace gllm {
namespace {

constexpr int kProbePF = 8;        // 4 KB steps in flight per workgroup (read probe)
constexpr int kProbeStep = 4096;   // bytes per workgroup step: 256 lanes x 16 B

__global__ void __launch_bounds__(256) probe_read_kernel(const char* buf, int64_t per_wg, uint32_t* out) {
  const int tid = threadIdx.x;
  const char* base = buf + (int64_t)blockIdx.x * per_wg + tid * 16;
  const int64_t steps = per_wg / kProbeStep;   // a multiple of kProbePF (checked on the host)
  u32x4 acc = {0u, 0u, 0u, 0u}, r[kProbePF];
#pragma unroll
  for (int j = 0; j < kProbePF; ++j) r[j] = ld16(base + (int64_t)j * kProbeStep);
  for (int64_t s = kProbePF; s < steps; s += kProbePF) {
#pragma unroll
    for (int j = 0; j < kProbePF; ++j) {
      acc ^= r[j];
      r[j] = ld16(base + (s + j) * kProbeStep);
    }
  }
#pragma unroll
  for (int j = 0; j < kProbePF; ++j) acc ^= r[j];
  // keeps the loads live; a plain vector store when it fires
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9e3779b9u) out[blockIdx.x] = 1u;
}

template <int NS>
__global__ void __launch_bounds__(256) probe_lds_dma_kernel(const char* buf, int64_t mask, int iters, uint32_t* out) {
  __shared__ __attribute__((aligned(16))) char lds[NS * kProbeStep];
  const int tid = threadIdx.x, wave = tid >> 6;
  const uint32_t l0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  const int64_t base = (int64_t)blockIdx.x * kProbeStep * 64;
  for (int it = 0; it < iters; ++it) {
    const char* p = buf + ((base + (int64_t)it * kProbeStep + tid * 16) & mask);
    // stage it % NS: its previous copy (it - NS) completed at the last wait
    lds_dma16(p, __builtin_amdgcn_readfirstlane(l0 + (it % NS) * kProbeStep + wave * 1024));
    wait_vmcnt<NS - 1>();
  }
  wait_vmcnt<0>();
  __syncthreads();
  if (tid == 0) out[blockIdx.x] = *reinterpret_cast<const uint32_t*>(lds + 16 * (blockIdx.x & 7));
}

// One wave: `iters` groups of 8 v_mfma_f32_32x32x16_bf16 on one
// accumulator, alone (mode 0) or with 64 independent fp32 FMAs (8 chains)
// placed between them (mode 1); out[0] = shader-clock cycles per group
// (s_memtime), out[1] = 100 MHz ticks of the whole loop (s_memrealtime), so
// cycles / ticks gives the shader clock.  out[2..3] keep the results live.
template <int MODE>
__global__ void __launch_bounds__(64) probe_mfma_kernel(int iters, int64_t* out) {
  const int lane = threadIdx.x;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (lane + i));
    b[i] = (__bf16)(0.002f * (lane - i));
  }
  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  float x[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) x[c] = 1.f + 0.01f * (lane + c);
  const float y = 0.999f, z = 0.001f;
  const int64_t t0 = __builtin_amdgcn_s_memtime();
  const int64_t r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      acc = mfma32(a, b, acc);
      if constexpr (MODE == 1) {
#pragma unroll
        for (int c = 0; c < 8; ++c) x[c] = __builtin_fmaf(x[c], y, z);
      }
    }
  }
  const int64_t t1 = __builtin_amdgcn_s_memtime();
  const int64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += acc[j];
#pragma unroll
  for (int c = 0; c < 8; ++c) s += x[c];
  if (lane == 0) {
    out[0] = (t1 - t0) / iters;
    out[1] = r1 - r0;
    out[2] = (int64_t)s;
    out[3] = iters;
  }
}

// Workgroups that do nothing but take their LDS: the cost of launching and
// retiring a grid of a given shape.
__global__ void probe_empty_kernel(uint32_t* out) {
  extern __shared__ char dyn_lds[];
  if (threadIdx.x == 0 && blockIdx.x == 0x7fffffff) out[0] = (uint32_t)(uintptr_t)dyn_lds;
}

}  // namespace
}  // namespace gllm

using namespace gllm;

// Returns a hipError_t code.  bytes must be a multiple of wgs * 32 KB.
extern "C" int gllm_probe_read(const void* buf, int64_t bytes, int32_t wgs, void* out, void* stream) {
  if (!buf || !out || wgs <= 0 || bytes <= 0) return (int)hipErrorInvalidValue;
  const int64_t unit = (int64_t)kProbeStep * kProbePF;
  if (bytes % ((int64_t)wgs * unit) != 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_read_kernel, dim3(wgs), dim3(256), 0, (hipStream_t)stream, (const char*)buf,
                     bytes / wgs, (uint32_t*)out);
  return (int)hipGetLastError();
}

// window: a power of two >= 4 KB; the buffer holds at least window bytes.
// out holds wgs uint32 values.
extern "C" int gllm_probe_lds_dma(const void* buf, int64_t window, int32_t wgs, int32_t iters, void* out,
                                  void* stream) {
  if (!buf || !out || wgs <= 0 || iters <= 0 || window < kProbeStep || (window & (window - 1)))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_lds_dma_kernel<4>, dim3(wgs), dim3(256), 0, (hipStream_t)stream, (const char*)buf,
                     window - 1, iters, (uint32_t*)out);
  return (int)hipGetLastError();
}

// mode 0: MFMAs alone, 1: with interleaved independent FMAs; out: 4 int64.
extern "C" int gllm_probe_mfma(int32_t mode, int32_t iters, void* out, void* stream) {
  if (!out || iters <= 0 || (mode != 0 && mode != 1)) return (int)hipErrorInvalidValue;
  if (mode == 0)
    hipLaunchKernelGGL(probe_mfma_kernel<0>, dim3(1), dim3(64), 0, (hipStream_t)stream, (int)iters, (int64_t*)out);
  else
    hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(1), dim3(64), 0, (hipStream_t)stream, (int)iters, (int64_t*)out);
  return (int)hipGetLastError();
}

// An empty grid of wgs workgroups of threads threads (<= 1024) with lds bytes
// of LDS each (<= 64 KB).
extern "C" int gllm_probe_empty(int32_t wgs, int32_t threads, int32_t lds, void* out, void* stream) {
  if (!out || wgs <= 0 || threads <= 0 || threads > 1024 || lds < 0 || lds > 65536) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_empty_kernel, dim3(wgs), dim3(threads), (size_t)lds, (hipStream_t)stream, (uint32_t*)out);
  return (int)hipGetLastError();
}

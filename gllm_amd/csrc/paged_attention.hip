// bf16 attention kernels for gfx950: paged decode, paged prefill / chunked
// prefill, the mixed continuous-batch launch, and the dense-bias op.
//
// Replaces, for the engine path, gllm/model/layers/attention.py:163-178 (the
// dense KV gather plus reference_attention); the kernels walk the block table
// instead of materialising a padded window.  Mask: key position p is visible
// to query row r of sequence i iff p <= c_i + r, which is exactly the 0/-inf
// pattern gllm/llm/llm.py:259-274 builds, on every real query row.  GQA: query
// head h reads kv head h / G (gllm/ops/attention/reference_attention.py:19-30).
//
// Decode (one 8-wave workgroup per (sequence, context split, 8 kv heads)):
//   all waves walk the same keys, one kv head each, so every step streams
//   whole pages; S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K loaded from
//   HBM straight into MFMA operand registers (16-byte loads) through a
//   prefetch ring; online softmax in fp32 (log2 domain, lazy rescale);
//   O^T += V^T P^T on v_mfma_f32_16x16x16_bf16 with V transposed through LDS
//   by ds_read_b64_tr_b16; split sequences are merged by a second small launch.
// Prefill (one 8-wave workgroup per (sequence, kv head, 8 row tiles of 32)):
//   K/V tiles of 64 keys staged in LDS, S^T = K Q^T and O^T += V^T P^T on
//   v_mfma_f32_32x32x16_bf16, flash-style running max/sum, causal tile skip.
//   The G query heads of one kv head share every K/V tile.
#include "common.h"
#include "launch.h"

namespace gllm {

// Rotate-half RoPE on 8 pairs, each op rounded to bf16 like the reference's
// torch ops (gllm/model/layers/attention.py:105-118).
__device__ __forceinline__ void rope8_bf16(float* x1, float* x2, const float* c, const float* s) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float a = round_bf16(__fmul_rn(x1[i], c[i]));
    float b = round_bf16(__fmul_rn(x2[i], s[i]));
    float e = round_bf16(__fmul_rn(x1[i], s[i]));
    float f = round_bf16(__fmul_rn(x2[i], c[i]));
    x1[i] = round_bf16(__fsub_rn(a, b));
    x2[i] = round_bf16(__fadd_rn(e, f));
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

__device__ __forceinline__ int64_t paged_slot(const AttnArgs& a, const int32_t* bt, int p) {
  uint32_t blk = (uint32_t)bt[p >> a.block_shift];
  if (blk >= (uint64_t)a.num_blocks) blk = 0;  // never address outside the pool
  return (int64_t)blk * a.block_size + (p & (a.block_size - 1));
}

// ============================================================== decode
constexpr int kWaves = 8;   // waves per workgroup (both paths; one block size)

template <int D, int NW> struct DecodeCfg {
  static constexpr int kPF = D == 64 ? 3 : 2;          // sub-tiles in flight per wave
  static constexpr int kRowBytes = D * 2 + 32;         // V staging row stride (bytes)
  static constexpr int kVBytes = 16 * kRowBytes;       // per-wave V staging: 16 keys
  static constexpr int kMaxBlocks = 512;               // block ids of one split, cached in LDS
  static constexpr int kStage = NW * kVBytes + kMaxBlocks * 4;
  static constexpr int kMerge = NW * 16 * (D + 2) * 4;       // per-wave (acc, m, l), 16 rows
  static constexpr int kLdsBytes = kStage > kMerge ? kStage : kMerge;
};

__device__ __forceinline__ f32x4 mfma16k16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b),
                                                   c, 0, 0, 0);
}

// One (HW x KW)-wave workgroup per (sequence, context split, group of HW kv
// heads).  Wave w serves kv head HW * group + w % HW and takes the split's
// 16-key sub-tiles w / HW, w / HW + KW, ... (KW waves interleave one head).
// Large HW reads long contiguous runs of each page (all the group's kv heads
// of the same slots); large KW gives one sequence more loads in flight, so a
// batch of few sequences needs no split.  K goes from HBM
// straight into MFMA A-operand registers (16-byte loads) through a prefetch
// ring, V is staged through LDS and read transposed.  S^T = K Q^T
// (16x16x32), O^T += V^T P^T (16x16x16); the G query heads (x query rows) of
// the kv head are the 16 MFMA columns.  The KW waves of a head merge through
// LDS; a split sequence writes (max, sum, acc) partials that merge_splits
// combines in a second, tiny launch (no cross-workgroup fences here).
template <int D, int HW, int KW>
__device__ __forceinline__ void decode_wg(const AttnArgs& a, const WorkItem& it, char* lds) {
  constexpr int NW = HW * KW;
  using Cfg = DecodeCfg<D, NW>;
  constexpr int NK = D / 32;   // 32-dim K chunks per key
  constexpr int ND = D / 16;   // 16-dim output blocks
  constexpr int RB = Cfg::kRowBytes;
  constexpr int PF = Cfg::kPF;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, grp = lane >> 4;
  const int hi = wave % HW, ki = wave / HW;
  const int seq = it.seq, split = it.a;
  const int kvh = (it.kind_b >> 8) * HW + hi;
  const bool head_ok = kvh < a.num_kv_heads;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int R = it.q_len * G;
  const int L = it.ctx_len + it.q_len;
  const int kbeg = split * a.split_len;
  const int kend = min(L, kbeg + a.split_len);
  const int nsub = (kend - kbeg + 15) >> 4;
  const bool row_ok = n < R && head_ok;
  const int r = row_ok ? n / G : 0;
  const int g = row_ok ? n - (n / G) * G : 0;
  const int64_t qrow = it.q_row_start + r;
  const int qh = (head_ok ? kvh : 0) * G + g;
  const int vis = it.ctx_len + r;

  // Block ids of this split -> LDS (one HBM round trip, off the per-step path).
  int32_t* lbid = reinterpret_cast<int32_t*>(lds + NW * Cfg::kVBytes);
  const int blk0 = kbeg >> a.block_shift;
  const int nblk = ((kend - 1) >> a.block_shift) - blk0 + 1;
  const int32_t* bt = a.block_table + (int64_t)seq * a.block_table_stride + blk0;
  for (int i = tid; i < nblk; i += 64 * NW) {
    const uint32_t b = (uint32_t)bt[i];
    lbid[i] = b < (uint64_t)a.num_blocks ? (int32_t)b : 0;  // never address outside the pool
  }

  // Q as the B operand of S^T = K Q^T: lane holds Q[row n][32kk + 8grp + i].
  bf16x8 qB[NK];
  {
    const __bf16* qp = (const __bf16*)a.q + qrow * a.q_row_stride + (int64_t)qh * D + 8 * grp;
    float x[NK][8];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) unpack_bf16x8(ld16(qp + 32 * kk), x[kk]);
    if (a.rope_mode != kRopeNone) {
      const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)vis : qrow;
      const __bf16* cp = (const __bf16*)a.rope_cos + crow * a.rope_row_stride + 8 * grp;
      const __bf16* sp = (const __bf16*)a.rope_sin + crow * a.rope_row_stride + 8 * grp;
#pragma unroll
      for (int kk = 0; kk < NK / 2; ++kk) {
        float c[8], s[8];
        unpack_bf16x8(ld16(cp + 32 * kk), c);
        unpack_bf16x8(ld16(sp + 32 * kk), s);
        rope8_bf16(x[kk], x[kk + NK / 2], c, s);
      }
    }
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      if (!row_ok)
        for (int i = 0; i < 8; ++i) x[kk][i] = 0.f;
      qB[kk] = to_bf16x8(x[kk]);
    }
  }
  __syncthreads();

  // byte addressing: slot (< 2^32) x slot bytes (< 2^32) is one 32x32->64 mad
  const uint32_t sbytes = (uint32_t)(a.cache_slot_stride * 2);
  const char* kc = (const char*)a.k_cache + ((int64_t)(head_ok ? kvh : 0) * D + 8 * grp) * 2;
  const char* vc = (const char*)a.v_cache + ((int64_t)(head_ok ? kvh : 0) * D + 8 * grp) * 2;
  const float sl2 = a.scale * kLog2e;
  char* ldsV = lds + wave * Cfg::kVBytes;
  const uint32_t bmask = a.block_size - 1;

  float m = kNegInf, lsum = 0.f;
  f32x4 acc[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // this wave's sub-tiles: j = ki + KW * t, t < ntw
  const int ntw = head_ok && nsub > ki ? (nsub - ki + KW - 1) / KW : 0;
  u32x4 kr[PF + 1][NK], vr[PF + 1][NK];
  auto issue = [&](int t, u32x4 (&kd)[NK], u32x4 (&vd)[NK]) {
    const int key = min(kbeg + 16 * (ki + KW * t) + n, kend - 1);
    const uint32_t slot = (uint32_t)lbid[(key >> a.block_shift) - blk0] * (uint32_t)a.block_size + ((uint32_t)key & bmask);
    const uint64_t off = (uint64_t)slot * sbytes;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      kd[kk] = ld16(kc + off + 64 * kk);
      vd[kk] = ld16(vc + off + 64 * kk);
    }
  };
  auto compute = [&](int t, const u32x4 (&kd)[NK], const u32x4 (&vd)[NK]) {
    // tiles past the last one (ring padding) are fully masked
    const int kb = t < ntw ? kbeg + 16 * (ki + KW * t) : kend;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) s = mfma16(as_bf16x8(kd[kk]), qB[kk], s);
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      *reinterpret_cast<u32x4*>(ldsV + n * RB + (32 * kk + 8 * grp) * 2) = vd[kk];
    // lane holds S[key kb + 4grp + j][row n]
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = s[j] * sl2;
    if (kb + 16 > kend || kb + 15 > it.ctx_len) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = kb + 4 * grp + j;
        if (key >= kend || key > vis) p[j] = kNegInf;
      }
    }
    float tmax = fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3]));
    tmax = max_xor32(max_xor16(tmax));
    // Lazy rescale: the running max only moves when a row's tile max exceeds
    // it by more than 8 (log2 units), so p <= 2^8 and most tiles skip the
    // acc rescale.  Numerator and denominator share m, so the result is exact.
    if (__builtin_amdgcn_ballot_w64(tmax > m + 8.f)) {
      const float mn = tmax > m + 8.f ? tmax : m;
      const float alpha = fast_exp2(m - (mn == kNegInf ? 0.f : mn));
      lsum *= alpha;
#pragma unroll
      for (int d = 0; d < ND; ++d) acc[d] *= alpha;
      m = mn;
    }
    const float mu = m == kNegInf ? 0.f : m;
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = fast_exp2(p[j] - mu);
    lsum += (p[0] + p[1]) + (p[2] + p[3]);
    const u32x2 pb = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
    const char* vrow = ldsV + (4 * grp + (n >> 2)) * RB + 4 * (n & 3) * 2;
#pragma unroll
    for (int d = 0; d < ND; ++d) acc[d] = mfma16k16(lds_read_tr16(vrow + 32 * d), pb, acc[d]);
  };

  // The ring loop has no early exit and issues loads unconditionally (tiles
  // past the end re-read the last tile, a cache hit, and are masked), so the
  // in-flight load order is the same on every path and the PF tiles in
  // flight really overlap the compute of the current one.  sched_barrier
  // keeps the scheduler from reordering the issues.
  if (ntw > 0) {
    const int tlast = ntw - 1;
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      issue(min(u, tlast), kr[u], vr[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int t0 = 0; t0 < ntw; t0 += PF + 1) {
#pragma unroll
      for (int u = 0; u <= PF; ++u) {
        const int t = t0 + u;
        issue(min(t + PF, tlast), kr[(u + PF) % (PF + 1)], vr[(u + PF) % (PF + 1)]);
        __builtin_amdgcn_sched_barrier(0);
        compute(t, kr[u], vr[u]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  float lt = sum_xor32(sum_xor16(lsum));

  if (KW > 1) {
    // merge the KW waves of each head through LDS (reuses the staging area)
    __syncthreads();
    float* macc = reinterpret_cast<float*>(lds);        // [NW waves][16 rows][D]
    float* mml = macc + NW * 16 * D;                     // [NW waves][16 rows][2]
#pragma unroll
    for (int d = 0; d < ND; ++d)
      *reinterpret_cast<f32x4*>(macc + (wave * 16 + n) * D + 16 * d + 4 * grp) = acc[d];
    if (grp == 0) {
      mml[(wave * 16 + n) * 2] = m;
      mml[(wave * 16 + n) * 2 + 1] = lt;
    }
    __syncthreads();
    if (ki != 0) return;
    float M = kNegInf;
#pragma unroll
    for (int k = 0; k < KW; ++k) M = fmaxf(M, mml[((k * HW + hi) * 16 + n) * 2]);
    const float Mu = M == kNegInf ? 0.f : M;
    lt = 0.f;
#pragma unroll
    for (int d = 0; d < ND; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KW; ++k) {
      const int w = k * HW + hi;
      const float wt = fast_exp2(mml[(w * 16 + n) * 2] - Mu);
      lt += wt * mml[(w * 16 + n) * 2 + 1];
#pragma unroll
      for (int d = 0; d < ND; ++d) acc[d] += wt * *reinterpret_cast<const f32x4*>(macc + (w * 16 + n) * D + 16 * d + 4 * grp);
    }
    m = M;
  }
  if (!row_ok) return;
  if (it.nsplits == 1) {
    const float inv = 1.f / lt;
    __bf16* op = (__bf16*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * grp;
#pragma unroll
    for (int d = 0; d < ND; ++d)
      st8(op + 16 * d, u32x2{pack_bf16x2(acc[d][0] * inv, acc[d][1] * inv), pack_bf16x2(acc[d][2] * inv, acc[d][3] * inv)});
    return;
  }
  // split partial: unnormalised acc, running max (log2 units) and sum
  const int64_t pidx = (int64_t)it.partial_base + (int64_t)kvh * it.nsplits + split;
  float* pa = a.partials + (pidx * 16 + n) * D + 4 * grp;
#pragma unroll
  for (int d = 0; d < ND; ++d) *reinterpret_cast<f32x4*>(pa + 16 * d) = acc[d];
  if (grp == 0) {
    a.partial_ml[(pidx * 16 + n) * 2] = m;
    a.partial_ml[(pidx * 16 + n) * 2 + 1] = lt;
  }
}

// Combines the split partials of every (sequence, kv head) whose sequence
// was split: one wave per (sequence, kv head); softmax-weighted (LSE) merge.
template <int D>
__global__ void __launch_bounds__(64) merge_splits_kernel(AttnArgs a) {
  const int seq = blockIdx.x / a.num_kv_heads, kvh = blockIdx.x - seq * a.num_kv_heads;
  const SeqInfo si = a.seqs[seq];
  if (si.nsplits <= 1) return;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int R = si.q_len * G;
  constexpr int CPR = D / 4;
  const int64_t pbase = (int64_t)si.partial_base + (int64_t)kvh * si.nsplits;
  for (int e = threadIdx.x; e < R * CPR; e += 64) {
    const int row = e / CPR, d4 = (e - row * CPR) * 4;
    float M = kNegInf;
    for (int sp = 0; sp < si.nsplits; ++sp) M = fmaxf(M, a.partial_ml[((pbase + sp) * 16 + row) * 2]);
    const float Mu = M == kNegInf ? 0.f : M;
    float Ls = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < si.nsplits; ++sp) {
      const float* ml = a.partial_ml + ((pbase + sp) * 16 + row) * 2;
      const float w = fast_exp2(ml[0] - Mu);
      Ls += w * ml[1];
      o += w * *reinterpret_cast<const f32x4*>(a.partials + ((pbase + sp) * 16 + row) * D + d4);
    }
    const float inv = 1.f / Ls;
    const int rr = row / G, gg = row - rr * G;
    __bf16* op = (__bf16*)a.out + (si.q_row_start + rr) * a.out_row_stride + (int64_t)(kvh * G + gg) * D + d4;
    st8(op, u32x2{pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)});
  }
}

// ============================================================== prefill
template <int D> struct PrefillCfg {
  static constexpr int kBN = 64;                   // keys per tile
  static constexpr int kRow = D * 2;               // bytes per K/V row in LDS (16-byte chunks XOR-swizzled)
  static constexpr int kTile = kBN * kRow;         // bytes per K (or V) tile
  static constexpr int kBidCache = 1024;           // block ids cached per workgroup
  static constexpr int kLdsBytes = 4 * kTile + kBidCache * 4;   // K, V double-buffered + block ids
};

// Logical 16-byte chunk c of LDS row r lives at chunk c ^ (r mod chunks-per-row):
// the 16 rows one MFMA operand read touches land in 16 different bank groups.
template <int D>
__device__ __forceinline__ int swz(int r, int c) { return c ^ (r & (D / 8 - 1)); }

// One 8-wave workgroup: each wave owns 32 query rows of one query head; the
// waves cover (head, row block) pairs of one kv head, so every K/V tile staged
// in LDS serves up to 8 x 32 query rows.  K/V tiles of 64 keys are double
// buffered in LDS (one barrier per tile); the global loads for tile t+2 are
// in flight while tile t is computed.  Softmax: exp argument as one FMA,
// lazy rescale of the running max (exact).
// Paged mode: keys come from the cache through the block table, causal mask.
// Dense mode (DENSE): keys from k/v [B, T, Hkv, D], additive bias [B, T_q, T].
template <int D, bool DENSE>
__device__ __forceinline__ void prefill_wg(const AttnArgs& a, const WorkItem& it, int seq, int kvh, int wgrp, char* lds) {
  using Cfg = PrefillCfg<D>;
  constexpr int NQ = D / 16;               // Q operand chunks (16 dims)
  constexpr int NO = D / 32;               // output blocks (32 dims)
  constexpr int BN = Cfg::kBN;
  constexpr int RW = Cfg::kRow;
  constexpr int CPR = D / 8;               // 16-byte chunks per key row
  constexpr int NT = 64 * kWaves;          // threads per workgroup
  constexpr int CH = BN * CPR / NT;        // chunks per thread per tile
  static_assert(CH >= 1 && BN * CPR % NT == 0, "tile / workgroup mismatch");
  char* const ldsKV = lds;                 // K[buf] at buf * kTile, V[buf] at (2 + buf) * kTile
  int32_t* const lbid = reinterpret_cast<int32_t*>(lds + 4 * Cfg::kTile);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31, h = lane >> 5;

  int ctx, qlen, T;
  int64_t qstart;
  if (DENSE) {
    ctx = 0;
    qlen = a.dense_Tq;
    T = a.dense_T;
    qstart = (int64_t)seq * a.dense_Tq;
  } else {
    ctx = it.ctx_len;
    qlen = it.q_len;
    T = ctx + qlen;
    qstart = it.q_row_start;
  }
  const int G = a.num_q_heads / a.num_kv_heads;
  const int nrb = (qlen + 31) / 32;
  const int combo = wgrp * kWaves + wave;
  const bool wact = combo < G * nrb;
  const int g = wact ? combo % G : 0;
  const int rblk = wact ? combo / G : 0;
  const int r0 = rblk * 32;
  const int last_combo = min(wgrp * kWaves + kWaves - 1, G * nrb - 1);
  const int kend_wg = DENSE ? T : ctx + min(qlen - 1, (last_combo / G) * 32 + 31) + 1;
  const int kend_w = DENSE ? T : ctx + min(qlen - 1, r0 + 31) + 1;
  const int r = r0 + n;
  const bool row_ok = wact && r < qlen;
  const int rr = min(r, qlen - 1);
  const int vis = ctx + rr;
  const int64_t qrow = qstart + rr;
  const int qh = kvh * G + g;

  // block ids of keys [0, kend_wg) -> LDS (first kBidCache blocks; any beyond
  // are read from the table directly)
  const int32_t* bt = DENSE ? nullptr : a.block_table + (int64_t)seq * a.block_table_stride;
  if (!DENSE) {
    const int nblk = ((kend_wg - 1) >> a.block_shift) + 1;
    for (int i = tid; i < min(nblk, Cfg::kBidCache); i += NT) {
      const uint32_t b = (uint32_t)bt[i];
      lbid[i] = b < (uint64_t)a.num_blocks ? (int32_t)b : 0;  // never address outside the pool
    }
  }

  // Q as the B operand of S^T = K Q^T: lane holds Q[row n][16kk + 8h + i].
  bf16x8 qB[NQ];
  {
    const __bf16* qp = (const __bf16*)a.q + qrow * a.q_row_stride + (int64_t)qh * D + 8 * h;
    float x[NQ][8];
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) unpack_bf16x8(ld16(qp + 16 * kk), x[kk]);
    if (!DENSE && a.rope_mode != kRopeNone) {
      const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)vis : qrow;
      const __bf16* cp = (const __bf16*)a.rope_cos + crow * a.rope_row_stride + 8 * h;
      const __bf16* sp = (const __bf16*)a.rope_sin + crow * a.rope_row_stride + 8 * h;
#pragma unroll
      for (int kk = 0; kk < NQ / 2; ++kk) {
        float c[8], s[8];
        unpack_bf16x8(ld16(cp + 16 * kk), c);
        unpack_bf16x8(ld16(sp + 16 * kk), s);
        rope8_bf16(x[kk], x[kk + NQ / 2], c, s);
      }
    }
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) qB[kk] = to_bf16x8(x[kk]);
  }
  if (!DENSE) __syncthreads();  // block ids visible

  const uint32_t sbytes = (uint32_t)(a.cache_slot_stride * 2);
  const uint32_t bmask = a.block_size - 1;
  u32x4 kst[CH], vst[CH];
  auto gload = [&](int ts) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + NT * i;
      const int key = c / CPR, ch = c - key * CPR;
      const int p = min(ts + key, kend_wg - 1);
      const char *kp, *vp;
      if (DENSE) {
        kp = (const char*)a.k + ((int64_t)seq * a.k_batch_stride + (int64_t)p * a.k_row_stride + (int64_t)kvh * D) * 2;
        vp = (const char*)a.v + ((int64_t)seq * a.v_batch_stride + (int64_t)p * a.v_row_stride + (int64_t)kvh * D) * 2;
      } else {
        const int bi = p >> a.block_shift;
        uint32_t blk;
        if (bi < Cfg::kBidCache) {
          blk = (uint32_t)lbid[bi];
        } else {
          blk = (uint32_t)bt[bi];
          if (blk >= (uint64_t)a.num_blocks) blk = 0;
        }
        const uint64_t off = (uint64_t)(blk * (uint32_t)a.block_size + ((uint32_t)p & bmask)) * sbytes +
                             (uint64_t)kvh * D * 2;
        kp = (const char*)a.k_cache + off;
        vp = (const char*)a.v_cache + off;
      }
      kst[i] = ld16(kp + ch * 16);
      vst[i] = ld16(vp + ch * 16);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + NT * i;
      const int key = c / CPR, ch = c - key * CPR;
      const int o = key * RW + (swz<D>(key, ch) << 4);
      *reinterpret_cast<u32x4*>(ldsKV + buf * Cfg::kTile + o) = kst[i];
      *reinterpret_cast<u32x4*>(ldsKV + (2 + buf) * Cfg::kTile + o) = vst[i];
    }
  };

  const float sl2 = a.scale * kLog2e;
  float m = kNegInf, lsum = 0.f;
  f32x16 o[NO];
#pragma unroll
  for (int db = 0; db < NO; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;

  auto compute = [&](const char* ldsK, const char* ldsV, int ts) {
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) s[kb][j] = 0.f;
      const int row = 32 * kb + n;
#pragma unroll
      for (int kk = 0; kk < NQ; ++kk) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(ldsK + row * RW + (swz<D>(row, 2 * kk + h) << 4));
        s[kb] = mfma32(as_bf16x8(ka), qB[kk], s[kb]);
      }
    }
    // lane holds raw scores S[key ts + 32kb + 8(j/4) + 4h + j%4][row n]
    if (DENSE) {
      const __bf16* bp = (const __bf16*)a.bias + (int64_t)seq * a.bias_batch_stride + (int64_t)rr * a.bias_row_stride;
      const float inv_scale = 1.f / a.scale;   // bias is added in natural-log units
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = ts + 32 * kb + 8 * (j >> 2) + 4 * h + (j & 3);
          const float bv = key < T ? (float)bp[key] : kNegInf;
          s[kb][j] = __builtin_fmaf(bv, inv_scale, s[kb][j]);
        }
    } else if (ts + BN - 1 > ctx + r0) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = ts + 32 * kb + 8 * (j >> 2) + 4 * h + (j & 3);
          if (key > vis) s[kb][j] = kNegInf;
        }
    }
    float tmax = kNegInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; j += 2) tmax = __builtin_fmaxf(tmax, __builtin_fmaxf(s[kb][j], s[kb][j + 1]));
    tmax = max_xor32(tmax) * sl2;
    // Lazy rescale: the running max only moves when a row's tile max exceeds
    // it by more than 8 (log2 units), so p <= 2^8; numerator and denominator
    // share m, so the result is exact.
    if (__builtin_amdgcn_ballot_w64(tmax > m + 8.f)) {
      const float mn = tmax > m + 8.f ? tmax : m;
      const float alpha = fast_exp2(m - (mn == kNegInf ? 0.f : mn));
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < NO; ++db) o[db] *= alpha;
      m = mn;
    }
    const float nmu = m == kNegInf ? 0.f : -m;
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[kb][j] = fast_exp2(__builtin_fmaf(s[kb][j], sl2, nmu));
        ps += s[kb][j];
      }
    lsum += ps;
    const int g4 = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int tp = 0; tp < 2; ++tp) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = s[kb][8 * tp + e];
        const bf16x8 pb = to_bf16x8(pv);
        const int row1 = 32 * kb + 16 * tp + 4 * h + (i16 >> 2);
#pragma unroll
        for (int db = 0; db < NO; ++db) {
          const int cb = 64 * db + 32 * (g4 & 1) + 8 * (i16 & 3);  // byte column
          const int c = cb >> 4, within = cb & 15;
          const u32x2 r1 = lds_read_tr16(ldsV + row1 * RW + (swz<D>(row1, c) << 4) + within);
          const u32x2 r2 = lds_read_tr16(ldsV + (row1 + 8) * RW + (swz<D>(row1 + 8, c) << 4) + within);
          const u32x4 av = {r1[0], r1[1], r2[0], r2[1]};
          o[db] = mfma32(as_bf16x8(av), pb, o[db]);
        }
      }
  };

  const int ntiles = (kend_wg + BN - 1) / BN;
  gload(0);
  lstore(0);
  if (ntiles > 1) gload(BN);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1, ts = t * BN;
    if (wact && ts < kend_w) compute(ldsKV + cur * Cfg::kTile, ldsKV + (2 + cur) * Cfg::kTile, ts);
    if (t + 1 < ntiles) {
      lstore(cur ^ 1);                     // tile t+1, loaded during the previous iteration
      if (t + 2 < ntiles) gload(ts + 2 * BN);
    }
    __syncthreads();
  }

  if (row_ok) {
    const float inv = 1.f / sum_xor32(lsum);
    __bf16* op = (__bf16*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * h;
#pragma unroll
    for (int db = 0; db < NO; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        u32x2 w = {pack_bf16x2(o[db][4 * jq] * inv, o[db][4 * jq + 1] * inv),
                   pack_bf16x2(o[db][4 * jq + 2] * inv, o[db][4 * jq + 3] * inv)};
        st8(op + 32 * db + 8 * jq, w);
      }
  }
}

// ============================================================== kernels
template <int D, bool PF, bool DC, int NW> struct MixedLds {
  static constexpr int a = PF ? PrefillCfg<D>::kLdsBytes : 0;
  static constexpr int b = DC ? DecodeCfg<D, NW>::kLdsBytes : 0;
  static constexpr int kBytes = a > b ? a : b;
};

// Work items of both kinds in one launch (mixed continuous batch), or of one
// kind.  Prefill workgroups are 8 waves; decode workgroups are HW x KW waves
// (8 in a mixed launch).
template <int D, bool PF, bool DC, int HW, int KW>
__global__ void __launch_bounds__(64 * HW * KW) paged_attn_bf16_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[MixedLds<D, PF, DC, HW * KW>::kBytes];
  const WorkItem it = a.items[blockIdx.x];
  if (PF && (!DC || (it.kind_b & 0xff) == kItemPrefill)) {
    if constexpr (HW * KW == kWaves) prefill_wg<D, false>(a, it, it.seq, it.a, it.kind_b >> 8, lds);
    return;
  }
  if constexpr (DC) decode_wg<D, HW, KW>(a, it, lds);
}

template <int D>
__global__ void __launch_bounds__(64 * kWaves) dense_attn_bf16_kernel(AttnArgs a, int nwg) {
  __shared__ __attribute__((aligned(16))) char lds[PrefillCfg<D>::kLdsBytes];
  const int w = blockIdx.x % nwg;
  const int rest = blockIdx.x / nwg;
  const int kvh = rest % a.num_kv_heads;
  const int b = rest / a.num_kv_heads;
  const WorkItem none{};
  prefill_wg<D, true>(a, none, b, kvh, w, lds);
}

template <int D, int HW, int KW>
static void launch_paged_hk(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  dim3 grid(a.n_items);
  if (pf && dc) {
    if constexpr (HW * KW == kWaves)
      hipLaunchKernelGGL((paged_attn_bf16_kernel<D, true, true, HW, KW>), grid, dim3(64 * kWaves), 0, st, a);
  } else if (pf) {
    hipLaunchKernelGGL((paged_attn_bf16_kernel<D, true, false, 8, 1>), grid, dim3(64 * kWaves), 0, st, a);
  } else {
    hipLaunchKernelGGL((paged_attn_bf16_kernel<D, false, true, HW, KW>), grid, dim3(64 * HW * KW), 0, st, a);
  }
}

template <int D>
static hipError_t launch_paged_d(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  const int hw = a.heads_per_wg, nw = a.decode_waves;
  if (pf && dc && nw != kWaves) return hipErrorInvalidValue;
  if (nw == 8) {
    switch (hw) {
      case 1: launch_paged_hk<D, 1, 8>(a, pf, dc, st); break;
      case 2: launch_paged_hk<D, 2, 4>(a, pf, dc, st); break;
      case 4: launch_paged_hk<D, 4, 2>(a, pf, dc, st); break;
      case 8: launch_paged_hk<D, 8, 1>(a, pf, dc, st); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !dc || a.n_partials == 0) return e;
  hipLaunchKernelGGL((merge_splits_kernel<D>), dim3(a.num_seqs * a.num_kv_heads), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_paged_attention_bf16(const AttnArgs& a, bool has_prefill, bool has_decode, hipStream_t st) {
  if (a.n_items == 0) return hipSuccess;
  if (a.head_dim == 64) return launch_paged_d<64>(a, has_prefill, has_decode, st);
  if (a.head_dim == 128) return launch_paged_d<128>(a, has_prefill, has_decode, st);
  return hipErrorInvalidValue;
}

hipError_t launch_dense_attention_bf16(const AttnArgs& a, int B, int Tq, hipStream_t st) {
  const int G = a.num_q_heads / a.num_kv_heads;
  const int nwg = (G * ((Tq + 31) / 32) + kWaves - 1) / kWaves;
  const int64_t blocks = (int64_t)B * a.num_kv_heads * nwg;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  dim3 grid((unsigned)blocks), block(64 * kWaves);
  if (a.head_dim == 64)
    hipLaunchKernelGGL((dense_attn_bf16_kernel<64>), grid, block, 0, st, a, nwg);
  else if (a.head_dim == 128)
    hipLaunchKernelGGL((dense_attn_bf16_kernel<128>), grid, block, 0, st, a, nwg);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

__global__ void fill_zero_i32_kernel(int32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

hipError_t launch_fill_zero_i32(int32_t* p, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(fill_zero_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

}  // namespace gllm

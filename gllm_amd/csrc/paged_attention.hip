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
// Decode (one wave per (sequence, kv head, context split)):
//   S^T = K Q^T with v_mfma_f32_16x16x32_bf16, K streamed from HBM straight
//   into MFMA operand registers (16-byte loads); online softmax in fp32 with
//   the log2-domain running max kept per row; O^T += V^T P^T with V transposed
//   through LDS by ds_read_b64_tr_b16; split partials merged by the last wave
//   to finish (atomic ticket), so decode is a single launch.
// Prefill (one 4-wave workgroup per (sequence, kv head, 4 row tiles of 32)):
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
template <int D> struct DecodeCfg {
  static constexpr int kRowBytes = D * 2 + 32;        // V row stride in LDS
  static constexpr int kLdsBytes = 32 * kRowBytes;    // per wave: 32 keys
};

template <int D>
__device__ __forceinline__ void decode_wave(const AttnArgs& a, int seq, int kvh, int split, char* lds) {
  constexpr int NK = D / 32;   // 32-dim K chunks per key
  constexpr int ND = D / 16;   // 16-dim output blocks
  constexpr int RB = DecodeCfg<D>::kRowBytes;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, grp = lane >> 4;
  const SeqInfo si = a.seqs[seq];
  const int G = a.num_q_heads / a.num_kv_heads;
  const int R = si.q_len * G;
  const int L = si.ctx_len + si.q_len;
  const int kbeg = split * a.split_len;
  const int kend = min(L, kbeg + a.split_len);
  const bool row_ok = n < R;
  const int r = row_ok ? n / G : 0;
  const int g = row_ok ? n - (n / G) * G : 0;
  const int64_t qrow = si.q_row_start + r;
  const int qh = kvh * G + g;
  const int vis = si.ctx_len + r;

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

  const int64_t ss = a.cache_slot_stride;
  const __bf16* kc = (const __bf16*)a.k_cache + (int64_t)kvh * D + 8 * grp;
  const __bf16* vc = (const __bf16*)a.v_cache + (int64_t)kvh * D + 8 * grp;
  const int32_t* bt = a.block_table + (int64_t)seq * a.block_table_stride;
  const float sl2 = a.scale * kLog2e;

  float m = kNegInf, lsum = 0.f;
  f32x4 acc[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 kn[2][NK], vn[2][NK];
  auto load_step = [&](int kb) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int p = min(kb + 16 * t + n, kend - 1);
      const int64_t slot = paged_slot(a, bt, p);
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        kn[t][kk] = ld16(kc + slot * ss + 32 * kk);
        vn[t][kk] = ld16(vc + slot * ss + 32 * kk);
      }
    }
  };
  load_step(kbeg);
  for (int kb = kbeg; kb < kend; kb += 32) {
    u32x4 kcur[2][NK], vcur[2][NK];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        kcur[t][kk] = kn[t][kk];
        vcur[t][kk] = vn[t][kk];
      }
    if (kb + 32 < kend) load_step(kb + 32);

    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      s0 = mfma16(as_bf16x8(kcur[0][kk]), qB[kk], s0);
      s1 = mfma16(as_bf16x8(kcur[1][kk]), qB[kk], s1);
    }
    // V rows (key 16t + n, dims 32kk + 8grp) into this wave's LDS tile.
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
        *reinterpret_cast<u32x4*>(lds + (16 * t + n) * RB + (32 * kk + 8 * grp) * 2) = vcur[t][kk];

    // lane holds S[key kb + 16t + 4grp + j][row n]
    float p[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = s0[j] * sl2;
      p[4 + j] = s1[j] * sl2;
    }
    if (kb + 32 > kend || kb + 31 > si.ctx_len) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = kb + 16 * (j >> 2) + 4 * grp + (j & 3);
        if (key >= kend || key > vis) p[j] = kNegInf;
      }
    }
    float tmax = p[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) tmax = fmaxf(tmax, p[j]);
    tmax = max_xor32(max_xor16(tmax));
    const float mn = fmaxf(m, tmax);
    const float mu = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(m - mu);
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = fast_exp2(p[j] - mu);
      ps += p[j];
    }
    lsum = lsum * alpha + ps;
    m = mn;
    const bf16x8 pb = to_bf16x8(p);
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      const char* base = lds + (4 * grp + (n >> 2)) * RB + (16 * d + 4 * (n & 3)) * 2;
      const u32x2 r1 = lds_read_tr16(base);
      const u32x2 r2 = lds_read_tr16(base + 16 * RB);
      const u32x4 av = {r1[0], r1[1], r2[0], r2[1]};
      acc[d] = mfma16(as_bf16x8(av), pb, acc[d] * alpha);
    }
  }
  const float lt = sum_xor32(sum_xor16(lsum));

  if (si.nsplits == 1) {
    if (row_ok) {
      const float inv = 1.f / lt;
      __bf16* op = (__bf16*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * grp;
#pragma unroll
      for (int d = 0; d < ND; ++d) {
        u32x2 w = {pack_bf16x2(acc[d][0] * inv, acc[d][1] * inv), pack_bf16x2(acc[d][2] * inv, acc[d][3] * inv)};
        st8(op + 16 * d, w);
      }
    }
    return;
  }

  // Split partial: unnormalised acc, running max (log2 units) and sum.
  const int pbase = si.partial_base + kvh * si.nsplits;
  if (row_ok) {
    float* pa = a.partials + ((int64_t)(pbase + split) * 16 + n) * D + 4 * grp;
#pragma unroll
    for (int d = 0; d < ND; ++d) *reinterpret_cast<f32x4*>(pa + 16 * d) = acc[d];
    if (grp == 0) {
      float* ml = a.partial_ml + ((int64_t)(pbase + split) * 16 + n) * 2;
      ml[0] = m;
      ml[1] = lt;
    }
  }
  __threadfence();
  int ticket = 0;
  int32_t* ctr = a.counters + (int64_t)seq * a.num_kv_heads + kvh;
  if (lane == 0) ticket = atomicAdd(ctr, 1);
  ticket = __shfl(ticket, 0);
  if (ticket != si.nsplits - 1) return;
  __threadfence();
  if (row_ok) {
    float M = kNegInf;
    for (int s = 0; s < si.nsplits; ++s) M = fmaxf(M, a.partial_ml[((int64_t)(pbase + s) * 16 + n) * 2]);
    float Lsum = 0.f;
    f32x4 o[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < si.nsplits; ++s) {
      const float* ml = a.partial_ml + ((int64_t)(pbase + s) * 16 + n) * 2;
      const float w = fast_exp2(ml[0] - M);
      Lsum += w * ml[1];
      const float* pa = a.partials + ((int64_t)(pbase + s) * 16 + n) * D + 4 * grp;
#pragma unroll
      for (int d = 0; d < ND; ++d) o[d] += w * *reinterpret_cast<const f32x4*>(pa + 16 * d);
    }
    const float inv = 1.f / Lsum;
    __bf16* op = (__bf16*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * grp;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      u32x2 w = {pack_bf16x2(o[d][0] * inv, o[d][1] * inv), pack_bf16x2(o[d][2] * inv, o[d][3] * inv)};
      st8(op + 16 * d, w);
    }
  }
  if (lane == 0) atomicExch(ctr, 0);  // ready for the next launch
}

// ============================================================== prefill
template <int D> struct PrefillCfg {
  static constexpr int kBN = 64;                   // keys per tile
  static constexpr int kKRow = D * 2 + 16;         // K row stride in LDS (bytes)
  static constexpr int kVRow = D * 2 + 32;         // V row stride in LDS (bytes)
  static constexpr int kLdsBytes = kBN * (kKRow + kVRow);
};

// One 4-wave workgroup: each wave owns 32 query rows of one query head.
// Paged mode: keys come from the cache through the block table, causal mask.
// Dense mode (DENSE): keys from k/v [B, T, Hkv, D], additive bias [B, T_q, T].
template <int D, bool DENSE>
__device__ __forceinline__ void prefill_wg(const AttnArgs& a, int seq, int kvh, int wgrp, char* lds) {
  constexpr int NQ = D / 16;   // Q operand chunks (16 dims)
  constexpr int NO = D / 32;   // output blocks (32 dims)
  constexpr int BN = PrefillCfg<D>::kBN;
  constexpr int KR = PrefillCfg<D>::kKRow;
  constexpr int VR = PrefillCfg<D>::kVRow;
  constexpr int CPR = D / 8;               // 16-byte chunks per key row
  constexpr int CH = BN * CPR / 256;       // chunks per thread per tile
  char* ldsK = lds;
  char* ldsV = lds + BN * KR;
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
    const SeqInfo si = a.seqs[seq];
    ctx = si.ctx_len;
    qlen = si.q_len;
    T = ctx + qlen;
    qstart = si.q_row_start;
  }
  const int G = a.num_q_heads / a.num_kv_heads;
  const int nrb = (qlen + 31) / 32;
  const int combo = wgrp * 4 + wave;
  const bool wact = combo < G * nrb;
  const int g = wact ? combo % G : 0;
  const int rblk = wact ? combo / G : 0;
  const int r0 = rblk * 32;
  const int last_combo = min(wgrp * 4 + 3, G * nrb - 1);
  const int kend_wg = DENSE ? T : ctx + min(qlen - 1, (last_combo / G) * 32 + 31) + 1;
  const int kend_w = DENSE ? T : ctx + min(qlen - 1, r0 + 31) + 1;
  const int r = r0 + n;
  const bool row_ok = wact && r < qlen;
  const int rr = min(r, qlen - 1);
  const int vis = ctx + rr;
  const int64_t qrow = qstart + rr;
  const int qh = kvh * G + g;

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

  const int32_t* bt = DENSE ? nullptr : a.block_table + (int64_t)seq * a.block_table_stride;
  u32x4 kreg[CH], vreg[CH];
  auto gload = [&](int ts) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      const int key = c / CPR, part = c - key * CPR;
      const int p = min(ts + key, kend_wg - 1);
      const __bf16 *kp, *vp;
      if (DENSE) {
        kp = (const __bf16*)a.k + (int64_t)seq * a.k_batch_stride + (int64_t)p * a.k_row_stride;
        vp = (const __bf16*)a.v + (int64_t)seq * a.v_batch_stride + (int64_t)p * a.v_row_stride;
      } else {
        const int64_t slot = paged_slot(a, bt, p);
        kp = (const __bf16*)a.k_cache + slot * a.cache_slot_stride;
        vp = (const __bf16*)a.v_cache + slot * a.cache_slot_stride;
      }
      kreg[i] = ld16(kp + (int64_t)kvh * D + 8 * part);
      vreg[i] = ld16(vp + (int64_t)kvh * D + 8 * part);
    }
  };

  const float sl2 = a.scale * kLog2e;
  float m = kNegInf, lsum = 0.f;
  f32x16 o[NO];
#pragma unroll
  for (int db = 0; db < NO; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;

  const int ntiles = (kend_wg + BN - 1) / BN;
  gload(0);
  for (int t = 0; t < ntiles; ++t) {
    const int ts = t * BN;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      const int key = c / CPR, part = c - key * CPR;
      *reinterpret_cast<u32x4*>(ldsK + key * KR + part * 16) = kreg[i];
      *reinterpret_cast<u32x4*>(ldsV + key * VR + part * 16) = vreg[i];
    }
    __syncthreads();
    if (t + 1 < ntiles) gload(ts + BN);
    if (wact && ts < kend_w) {
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int j = 0; j < 16; ++j) s[kb][j] = 0.f;
#pragma unroll
        for (int kk = 0; kk < NQ; ++kk) {
          const u32x4 ka = *reinterpret_cast<const u32x4*>(ldsK + (32 * kb + n) * KR + (16 * kk + 8 * h) * 2);
          s[kb] = mfma32(as_bf16x8(ka), qB[kk], s[kb]);
        }
      }
      // lane holds S[key ts + 32kb + 8(j/4) + 4h + j%4][row n]
      float sv[2][16];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) sv[kb][j] = s[kb][j] * sl2;
      if (DENSE) {
        const __bf16* bp = (const __bf16*)a.bias + (int64_t)seq * a.bias_batch_stride + (int64_t)rr * a.bias_row_stride;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int jq = 0; jq < 4; ++jq) {
            const int key0 = ts + 32 * kb + 8 * jq + 4 * h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int key = key0 + e;
              const float bv = key < T ? (float)bp[key] : kNegInf;
              sv[kb][4 * jq + e] = __builtin_fmaf(bv, kLog2e, sv[kb][4 * jq + e]);
            }
          }
      } else if (ts + BN - 1 > ctx + r0) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = ts + 32 * kb + 8 * (j >> 2) + 4 * h + (j & 3);
            if (key > vis) sv[kb][j] = kNegInf;
          }
      }
      float tmax = sv[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) tmax = fmaxf(tmax, sv[kb][j]);
      tmax = max_xor32(tmax);
      const float mn = fmaxf(m, tmax);
      const float mu = mn == kNegInf ? 0.f : mn;
      const float alpha = fast_exp2(m - mu);
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          sv[kb][j] = fast_exp2(sv[kb][j] - mu);
          ps += sv[kb][j];
        }
      lsum = lsum * alpha + ps;
      m = mn;
#pragma unroll
      for (int db = 0; db < NO; ++db) o[db] *= alpha;
      const int g4 = lane >> 4, i16 = lane & 15;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
          const bf16x8 pb = to_bf16x8(&sv[kb][8 * tp]);
          const int row1 = 32 * kb + 16 * tp + 4 * h + (i16 >> 2);
#pragma unroll
          for (int db = 0; db < NO; ++db) {
            const int col = 32 * db + 16 * (g4 & 1) + 4 * (i16 & 3);
            const u32x2 r1 = lds_read_tr16(ldsV + row1 * VR + col * 2);
            const u32x2 r2 = lds_read_tr16(ldsV + (row1 + 8) * VR + col * 2);
            const u32x4 av = {r1[0], r1[1], r2[0], r2[1]};
            o[db] = mfma32(as_bf16x8(av), pb, o[db]);
          }
        }
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
template <int D, bool PF, bool DC> struct MixedLds {
  static constexpr int a = PF ? PrefillCfg<D>::kLdsBytes : 0;
  static constexpr int b = DC ? 4 * DecodeCfg<D>::kLdsBytes : 0;
  static constexpr int kBytes = a > b ? a : b;
};

template <int D, bool PF, bool DC>
__global__ void __launch_bounds__(256) paged_attn_bf16_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[MixedLds<D, PF, DC>::kBytes];
  const WorkItem it = a.items[blockIdx.x];
  if (PF && (!DC || it.kind == kItemPrefill)) {
    prefill_wg<D, false>(a, it.seq, it.a, it.b, lds);
    return;
  }
  if (DC) {
    const int wave = threadIdx.x >> 6;
    const int kvh = it.b * 4 + wave;
    if (kvh < a.num_kv_heads) decode_wave<D>(a, it.seq, kvh, it.a, lds + wave * DecodeCfg<D>::kLdsBytes);
  }
}

template <int D>
__global__ void __launch_bounds__(256) dense_attn_bf16_kernel(AttnArgs a, int nwg) {
  __shared__ __attribute__((aligned(16))) char lds[PrefillCfg<D>::kLdsBytes];
  const int w = blockIdx.x % nwg;
  const int rest = blockIdx.x / nwg;
  const int kvh = rest % a.num_kv_heads;
  const int b = rest / a.num_kv_heads;
  prefill_wg<D, true>(a, b, kvh, w, lds);
}

template <int D>
static hipError_t launch_paged_d(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  dim3 grid(a.n_items), block(256);
  if (pf && dc)
    hipLaunchKernelGGL((paged_attn_bf16_kernel<D, true, true>), grid, block, 0, st, a);
  else if (pf)
    hipLaunchKernelGGL((paged_attn_bf16_kernel<D, true, false>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((paged_attn_bf16_kernel<D, false, true>), grid, block, 0, st, a);
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
  const int nwg = (G * ((Tq + 31) / 32) + 3) / 4;
  const int64_t blocks = (int64_t)B * a.num_kv_heads * nwg;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  dim3 grid((unsigned)blocks), block(256);
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

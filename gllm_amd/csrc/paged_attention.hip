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
// Decode (8-wave workgroups; a task = one key range of one sequence for HW
//   kv heads): S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K loaded from
//   HBM straight into MFMA operand registers (16-byte loads) through a
//   prefetch ring; online softmax in fp32 (log2 domain, lazy rescale);
//   O^T += V^T P^T on v_mfma_f32_16x16x16_bf16 with V transposed through LDS
//   by ds_read_b64_tr_b16.  Split plans merge split partials in a second
//   small launch; page-balanced plans deal equal key ranges to the
//   workgroups and merge in the same launch (split tickets).
// Prefill (one 8-wave workgroup per (sequence, kv head, 8 row tiles of 32)):
//   K/V tiles of 64 keys staged in LDS, S^T = K Q^T and O^T += V^T P^T on
//   v_mfma_f32_32x32x16_bf16, flash-style running max/sum, causal tile skip.
//   The G query heads of one kv head share every K/V tile.
#include "common.h"
#include "launch.h"

namespace gllm {

// Rotate-half RoPE on 8 pairs, each op rounded to the model dtype T like the
// reference's torch ops (gllm/model/layers/attention.py:105-118).
template <typename T>
__device__ __forceinline__ void rope8(float* x1, float* x2, const float* c, const float* s) {
#pragma unroll
  for (int i = 0; i < 8; ++i) rope_pair<T>(x1[i], x2[i], c[i], s[i]);
}


// ============================================================== decode
constexpr int kWaves = 8;   // waves per workgroup (both paths; one block size)

template <int D, int NW> struct DecodeCfg {
  static constexpr int kPF = 2;                         // sub-tiles in flight per wave (2 beat 3 at D = 64)
  static constexpr int kRowBytes = D * 2 + 32;         // V staging row stride (bytes)
  static constexpr int kVBytes = 16 * kRowBytes;       // per-wave V staging: 16 keys
  static constexpr int kMaxBlocks = 512;               // block ids of one split, cached in LDS
  static constexpr int kStage = NW * kVBytes + kMaxBlocks * 4;
  static constexpr int kMerge = NW * 16 * (D + 2) * 4;       // per-wave (acc, m, l), 16 rows
  static constexpr int kLdsBytes = kStage > kMerge ? kStage : kMerge;
};


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
// Cached K/V come in 16-byte loads per lane: 8 bf16 dims, or 16 fp8 dims
// that are widened (exactly) to bf16 on use and feed two MFMA K-chunks.
// Head dim of element i of MFMA chunk kk in lane group grp:
//   bf16: 32 kk + 8 grp + i
//   fp8:  64 (kk / 2) + 16 grp + 8 (kk % 2) + i
// S = K Q^T sums over dims, so any order serves as long as K and Q agree;
// V is staged to LDS in natural dim order, so the output is too.
template <bool KV8>
__device__ __forceinline__ int chunk_dim(int kk, int grp) {
  return KV8 ? 64 * (kk >> 1) + 16 * grp + 8 * (kk & 1) : 32 * kk + 8 * grp;
}
template <typename T, bool KV8>
__device__ __forceinline__ u32x4 chunk_elems(const u32x4* raw, int kk) {
  if constexpr (KV8) {
    const u32x4 w = raw[kk >> 1];
    return (kk & 1) ? fp8x8_to<T>(w[2], w[3]) : fp8x8_to<T>(w[0], w[1]);
  } else {
    return raw[kk];
  }
}

// One decode task: keys [kbeg, kend) of one sequence for HW kv heads.
struct DecodeTask {
  int seq, hg, kbeg, kend, q_row_start, ctx_len, q_len;
  int nseg;     // tasks of this (sequence, head group); 1: normalise and write the output
  int pbase;    // partial of head i of the group: pbase + i * nseg + ord
  int ord;
  int ticket;   // >= 0: counter whose last ticket merges the partials here; < 0: merge_splits does
};

// New tokens written by the attention launch (a.k_new != null): the task whose
// key range covers key p of a new token writes that token's K (rotated like
// apply_rope, every op rounded to T) and V, cast to the cache dtype, for its
// HW kv heads, at the key's slot.  No other workgroup reads those bytes in
// this launch (each key of each head belongs to one task); the workgroup
// barrier after the prologue orders the stores before this task's own loads
// of the key.  Element-wise stores: at most 16 tokens x HW heads x D.
template <typename T, int D, int HW, bool KV8>
__device__ __forceinline__ void write_new_keys(const AttnArgs& a, const DecodeTask& tk, int tid, int nthreads) {
  const int L = tk.ctx_len + tk.q_len;
  const int p0 = max(tk.ctx_len, tk.kbeg), p1 = min(L, tk.kend);
  if (p0 >= p1) return;
  constexpr int H2 = D / 2;
  const int per_tok = HW * H2;
  const int n = (p1 - p0) * per_tok;
  for (int e = tid; e < n; e += nthreads) {
    const int tok = e / per_tok, rem = e - tok * per_tok;
    const int hh = rem / H2, j = rem - hh * H2;
    const int kvh = tk.hg * HW + hh;
    if (kvh >= a.num_kv_heads) continue;
    const int p = p0 + tok;
    const int64_t row = tk.q_row_start + (p - tk.ctx_len);
    const T* kn = (const T*)a.k_new + row * a.k_new_row_stride + (int64_t)kvh * D;
    const T* vn = (const T*)a.v_new + row * a.v_new_row_stride + (int64_t)kvh * D;
    float x1 = (float)kn[j], x2 = (float)kn[j + H2];
    if (a.rope_mode != kRopeNone) {
      const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)p : row;
      const float c = (float)((const T*)a.rope_cos)[crow * a.rope_row_stride + j];
      const float sn = (float)((const T*)a.rope_sin)[crow * a.rope_row_stride + j];
      rope_pair<T>(x1, x2, c, sn);
    }
    const float v1 = (float)vn[j], v2 = (float)vn[j + H2];
    const uint32_t bi = div_bs((uint32_t)p, a.block_magic, a.block_shift);
    uint32_t blk = (uint32_t)a.block_table[(int64_t)tk.seq * a.block_table_stride + bi];
    if (blk >= (uint64_t)a.num_blocks) continue;   // never address outside the pool
    const int64_t off = ((int64_t)blk * a.block_size + (p - (int64_t)bi * a.block_size)) * a.cache_slot_stride +
                        (int64_t)kvh * D + j;
    if constexpr (KV8) {
      uint8_t* kc = (uint8_t*)a.k_cache + off;
      uint8_t* vc = (uint8_t*)a.v_cache + off;
      kc[0] = fp8_byte(x1); kc[H2] = fp8_byte(x2);
      vc[0] = fp8_byte(v1); vc[H2] = fp8_byte(v2);
    } else {
      T* kc = (T*)a.k_cache + off;
      T* vc = (T*)a.v_cache + off;
      kc[0] = (T)x1; kc[H2] = (T)x2;     // exact: already values of T
      vc[0] = (T)v1; vc[H2] = (T)v2;
    }
  }
}

// Runs one task with every wave of the workgroup; returns with the workgroup
// converged (no early exit), so a workgroup can run several tasks in a row.
template <typename T, int D, int HW, int KW, bool KV8>
__device__ __forceinline__ void decode_task(const AttnArgs& a, const DecodeTask& tk, char* lds, int* ticket_lds) {
  constexpr int NW = HW * KW;
  constexpr int E = KV8 ? 1 : 2;   // bytes per cached element
  using Cfg = DecodeCfg<D, NW>;
  constexpr int NK = D / 32;   // 32-dim K chunks per key
  constexpr int NL = KV8 ? NK / 2 : NK;   // 16-byte loads per key (K and V each)
  constexpr int ND = D / 16;   // 16-dim output blocks
  constexpr int RB = Cfg::kRowBytes;
  // RoPE partners d, d + D/2 in the same lane (chunks kk, kk + NK/2), except
  // for fp8 at D = 64, where a lane's 16 dims lie in one half
  constexpr bool kPairInLane = !KV8 || D >= 128;
  constexpr int NC = kPairInLane ? NK / 2 : NK;   // cos/sin loads
  constexpr int PF = Cfg::kPF;
  // the thread id through an opaque move: nothing derived from it is hoisted
  // out of a caller's loop over tasks (which would hold it in registers
  // across the whole main loop)
  int tid;
  asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, grp = lane >> 4;
  const int hi = wave % HW, ki = wave / HW;
  const int seq = tk.seq;
  const int kvh = tk.hg * HW + hi;
  const bool head_ok = kvh < a.num_kv_heads;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int R = tk.q_len * G;
  const int kbeg = tk.kbeg;
  const int kend = tk.kend;
  const int nsub = (kend - kbeg + 15) >> 4;
  const bool row_ok = n < R && head_ok;
  const int r = row_ok ? n / G : 0;
  const int g = row_ok ? n - (n / G) * G : 0;
  const int64_t qrow = tk.q_row_start + r;
  const int qh = (head_ok ? kvh : 0) * G + g;
  const int vis = tk.ctx_len + r;

  // Prologue: the block ids of this task (-> LDS), the Q rows and their
  // cos/sin rows are loaded together, one HBM round trip before the first
  // K/V loads can be addressed (the block-id load is issued first so its LDS
  // store does not wait for the others).
  static_assert(Cfg::kMaxBlocks <= 64 * NW, "one block id per thread");
  int32_t* lbid = reinterpret_cast<int32_t*>(lds + NW * Cfg::kVBytes);
  const int blk0 = (int)div_bs((uint32_t)kbeg, a.block_magic, a.block_shift);
  const int nblk = (int)div_bs((uint32_t)(kend - 1), a.block_magic, a.block_shift) - blk0 + 1;
  const int32_t* bt = a.block_table + (int64_t)seq * a.block_table_stride + blk0;
  const uint32_t bid = tid < nblk ? (uint32_t)bt[tid] : 0u;
  const T* qp = (const T*)a.q + qrow * a.q_row_stride + (int64_t)qh * D;
  u32x4 qraw[NK], praw[kPairInLane ? 1 : NK], craw[NC], sraw[NC];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) qraw[kk] = ld16(qp + chunk_dim<KV8>(kk, grp));
  const bool rope = a.rope_mode != kRopeNone;
  if (rope) {
    const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)vis : qrow;
    const T* cp = (const T*)a.rope_cos + crow * a.rope_row_stride;
    const T* sp = (const T*)a.rope_sin + crow * a.rope_row_stride;
#pragma unroll
    for (int kk = 0; kk < NC; ++kk) {
      const int d = chunk_dim<KV8>(kk, grp) & (D / 2 - 1);
      craw[kk] = ld16(cp + d);
      sraw[kk] = ld16(sp + d);
    }
    if constexpr (!kPairInLane) {
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) praw[kk] = ld16(qp + (chunk_dim<KV8>(kk, grp) ^ (D / 2)));
    }
  }
  if (tid < nblk) lbid[tid] = bid < (uint64_t)a.num_blocks ? (int32_t)bid : 0;  // never address outside the pool
  if (a.k_new) write_new_keys<T, D, HW, KV8>(a, tk, tid, 64 * NW);

  // Q as the B operand of S^T = K Q^T: lane holds Q[row n][chunk_dim(kk) + i].
  u32x4 qB[NK];
  {
    float x[NK][8];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) unpack8<T>(qraw[kk], x[kk]);
    if (rope) {
      if constexpr (kPairInLane) {
#pragma unroll
        for (int kk = 0; kk < NK / 2; ++kk) {
          float c[8], s[8];
          unpack8<T>(craw[kk], c);
          unpack8<T>(sraw[kk], s);
          rope8<T>(x[kk], x[kk + NK / 2], c, s);
        }
      } else {
        // the same roundings as rope8, one half of the pair per lane
        const bool first = chunk_dim<KV8>(0, grp) < D / 2;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          float c[8], s[8], xp[8];
          unpack8<T>(craw[kk], c);
          unpack8<T>(sraw[kk], s);
          unpack8<T>(praw[kk], xp);
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            float u0 = __fmul_rn(x[kk][i], c[i]), v0 = __fmul_rn(xp[i], s[i]);
            float u1 = __fmul_rn(x[kk][i + 1], c[i + 1]), v1 = __fmul_rn(xp[i + 1], s[i + 1]);
            round2<T>(u0, v0);
            round2<T>(u1, v1);
            if constexpr (E16<T>::kF16) opaque4(u0, v0, u1, v1);
            float r0 = first ? __fsub_rn(u0, v0) : __fadd_rn(u0, v0);
            float r1 = first ? __fsub_rn(u1, v1) : __fadd_rn(u1, v1);
            round2<T>(r0, r1);
            x[kk][i] = r0;
            x[kk][i + 1] = r1;
          }
        }
      }
    }
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      if (!row_ok)
        for (int i = 0; i < 8; ++i) x[kk][i] = 0.f;
      qB[kk] = pack8<T>(x[kk]);
    }
  }
  __syncthreads();

  // byte addressing: slot (< 2^32) x slot bytes (< 2^32) is one 32x32->64 mad
  const uint32_t sbytes = (uint32_t)(a.cache_slot_stride * E);
  const char* kc = (const char*)a.k_cache + (int64_t)(head_ok ? kvh : 0) * D * E + 16 * grp;
  const char* vc = (const char*)a.v_cache + (int64_t)(head_ok ? kvh : 0) * D * E + 16 * grp;
  const float sl2 = a.scale * kLog2e;
  char* ldsV = lds + wave * Cfg::kVBytes;

  float m = kNegInf, lsum = 0.f;
  f32x4 acc[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // this wave's sub-tiles: j = ki + KW * t, t < ntw
  const int ntw = head_ok && nsub > ki ? (nsub - ki + KW - 1) / KW : 0;
  u32x4 kr[PF + 1][NL], vr[PF + 1][NL];
  auto issue = [&](int t, u32x4 (&kd)[NL], u32x4 (&vd)[NL]) {
    // ring padding (t >= ntw): every lane reads the task's last slot, one
    // cache line per load instead of a whole 16-key tile
    const int key = t < ntw ? min(kbeg + 16 * (ki + KW * t) + n, kend - 1) : kend - 1;
    const uint32_t bi = div_bs((uint32_t)key, a.block_magic, a.block_shift);
    const uint32_t slot = (uint32_t)lbid[bi - blk0] * (uint32_t)a.block_size + ((uint32_t)key - bi * (uint32_t)a.block_size);
    const uint64_t off = (uint64_t)slot * sbytes;
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      kd[l] = ld16(kc + off + 64 * l);
      vd[l] = ld16(vc + off + 64 * l);
    }
  };
  auto compute = [&](int t, const u32x4 (&kd)[NL], const u32x4 (&vd)[NL]) {
    // tiles past the last one (ring padding) are fully masked
    const int kb = t < ntw ? kbeg + 16 * (ki + KW * t) : kend;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) s = E16<T>::mfma16(chunk_elems<T, KV8>(kd, kk), qB[kk], s);
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      *reinterpret_cast<u32x4*>(ldsV + n * RB + chunk_dim<KV8>(kk, grp) * 2) = chunk_elems<T, KV8>(vd, kk);
    // lane holds S[key kb + 4grp + j][row n]
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = s[j] * sl2;
    if (kb + 16 > kend || kb + 15 > tk.ctx_len) {
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
    const u32x2 pb = {E16<T>::pack2(p[0], p[1]), E16<T>::pack2(p[2], p[3])};
    lsum = E16<T>::add2(pb[1], E16<T>::add2(pb[0], lsum));   // the rounded p the MFMA sees
    const char* vrow = ldsV + (4 * grp + (n >> 2)) * RB + 4 * (n & 3) * 2;
#pragma unroll
    for (int d = 0; d < ND; ++d) acc[d] = E16<T>::mfma16k16(lds_read_tr16(vrow + 32 * d), pb, acc[d]);
  };

  // The ring issues loads unconditionally (tiles past the end read one
  // cached slot and are masked), so the in-flight load order is the same on
  // every path and the compiler's waits keep PF tiles in flight while the
  // current one is computed (conditional issues would make it wait for all
  // of them); the tail after the last whole group issues nothing.
  // sched_barrier keeps the scheduler from reordering the issues.
  if (ntw > 0) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      issue(u, kr[u], vr[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
    int t0 = 0;
    for (; t0 + PF < ntw; t0 += PF + 1) {   // whole groups: all PF + 1 computes are real tiles
#pragma unroll
      for (int u = 0; u <= PF; ++u) {
        const int t = t0 + u;
        issue(t + PF, kr[(u + PF) % (PF + 1)], vr[(u + PF) % (PF + 1)]);
        __builtin_amdgcn_sched_barrier(0);
        compute(t, kr[u], vr[u]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // last ntw - t0 (<= PF) tiles: already in flight, nothing more to issue
#pragma unroll
    for (int u = 0; u < PF; ++u)
      if (t0 + u < ntw) compute(t0 + u, kr[u], vr[u]);
  }
  float lt = sum_xor32(sum_xor16(lsum));

  bool lead = true;   // this wave holds its head's state for the task
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
    lead = ki == 0;
    if (lead) {
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
        for (int d = 0; d < ND; ++d)
          acc[d] += wt * *reinterpret_cast<const f32x4*>(macc + (w * 16 + n) * D + 16 * d + 4 * grp);
      }
      m = M;
    }
  }
  const bool wr = lead && row_ok;
  if (tk.nseg == 1) {
    if (wr) {
      T* op = (T*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * grp;
      const float inv = 1.f / lt;
#pragma unroll
      for (int d = 0; d < ND; ++d)
        st8(op + 16 * d, u32x2{E16<T>::pack2(acc[d][0] * inv, acc[d][1] * inv), E16<T>::pack2(acc[d][2] * inv, acc[d][3] * inv)});
    }
    return;
  }
  // partial: unnormalised acc, running max (log2 units) and sum
  const int64_t pfirst = (int64_t)tk.pbase + (int64_t)hi * tk.nseg;
  if (wr) {
    float* pa = a.partials + ((pfirst + tk.ord) * 16 + n) * D + 4 * grp;
#pragma unroll
    for (int d = 0; d < ND; ++d) *reinterpret_cast<f32x4*>(pa + 16 * d) = acc[d];
    if (grp == 0) {
      a.partial_ml[((pfirst + tk.ord) * 16 + n) * 2] = m;
      a.partial_ml[((pfirst + tk.ord) * 16 + n) * 2 + 1] = lt;
    }
  }
  if (tk.ticket < 0) return;
  // Ticket: the workgroup that completes a (sequence, group) last merges its
  // partials.  The barrier orders every wave's partial stores before thread
  // 0's agent-scope release (L2 write-back, so workgroups on other XCDs see
  // them); the last ticket holder acquires (L2 invalidate) before reading.
  // Nobody waits on anybody: a workgroup that is not last simply moves on.
  __syncthreads();
  if (tid == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const int t = __hip_atomic_fetch_add(a.counters + tk.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == tk.nseg - 1) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      // every ticket of this launch is drawn: re-arm the counter for the next one
      __hip_atomic_store(a.counters + tk.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *ticket_lds = t;
  }
  __syncthreads();
  const bool last = *ticket_lds == tk.nseg - 1;
  if (!last || !lead || !head_ok) return;
  // LSE merge, latency-bound (it is the launch's tail): the 16 row lanes of
  // each 16-lane group are (row mr, partial slot ps) pairs, R rows x PS
  // slots, and slot ps takes partials ps, ps + PS, ..., CH of them per
  // round trip with all their loads in flight; the slots are then combined
  // through shuffles in slot order.  The sums depend only on the partials,
  // not on which workgroup merges.
  constexpr int CH = 2;
  const int PS = 16 / R;
  const int mr = n % R, ps = n / R;
  const bool mact = ps < PS;
  float Mx = kNegInf, Lx = 0.f;
  f32x4 ox[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d) ox[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto combine = [&](float m2, float l2, const f32x4 (&o2)[ND]) {
    const float nM = fmaxf(Mx, m2);
    if (nM == kNegInf) return;
    const float w1 = fast_exp2(Mx - nM), w2 = fast_exp2(m2 - nM);
    Lx = Lx * w1 + l2 * w2;
#pragma unroll
    for (int d = 0; d < ND; ++d) ox[d] = ox[d] * w1 + o2[d] * w2;
    Mx = nM;
  };
  for (int o0 = 0; o0 < tk.nseg; o0 += PS * CH) {
    float mm[CH], ll[CH];
    f32x4 vv[CH][ND];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int o = o0 + c * PS + ps;
      const bool v = mact && o < tk.nseg;
      const int64_t pi = (pfirst + (v ? o : 0)) * 16 + mr;
      mm[c] = v ? a.partial_ml[pi * 2] : kNegInf;
      ll[c] = v ? a.partial_ml[pi * 2 + 1] : 0.f;
      const float* pa = a.partials + pi * D + 4 * grp;
#pragma unroll
      for (int d = 0; d < ND; ++d) vv[c][d] = v ? *reinterpret_cast<const f32x4*>(pa + 16 * d) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) combine(mm[c], ll[c], vv[c]);
  }
  // slot k's state moves to slot 0 (lanes mr + R k -> mr, same 16-dim group)
  for (int k = 1; k < PS; ++k) {
    const int src = (lane & 48) | min(15, mr + R * k);
    const float m2 = __shfl(Mx, src, 64), l2 = __shfl(Lx, src, 64);
    f32x4 o2[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int j = 0; j < 4; ++j) o2[d][j] = __shfl(ox[d][j], src, 64);
    if (ps == 0) combine(m2, l2, o2);
  }
  if (!row_ok) return;   // ps == 0 lanes: mr == n
  const float inv = 1.f / Lx;
  T* op = (T*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * grp;
#pragma unroll
  for (int d = 0; d < ND; ++d)
    st8(op + 16 * d, u32x2{E16<T>::pack2(ox[d][0] * inv, ox[d][1] * inv), E16<T>::pack2(ox[d][2] * inv, ox[d][3] * inv)});
}

// One decode work item of the split-launch planner (split it.a of the
// sequence's it.nsplits equal key ranges; split partials merged by
// merge_splits_kernel).
template <typename T, int D, int HW, int KW, bool KV8>
__device__ __forceinline__ void decode_wg(const AttnArgs& a, const WorkItem& it, char* lds) {
  DecodeTask tk;
  tk.seq = it.seq;
  tk.hg = it.kind_b >> 8;
  const int L = it.ctx_len + it.q_len;
  const int len = split_len_of(L, it.nsplits);   // equal splits (the planner's split_len bounds them)
  tk.kbeg = it.a * len;
  tk.kend = min(L, tk.kbeg + len);
  tk.q_row_start = it.q_row_start;
  tk.ctx_len = it.ctx_len;
  tk.q_len = it.q_len;
  tk.nseg = it.nsplits;
  tk.pbase = it.partial_base + tk.hg * HW * it.nsplits;
  tk.ord = it.a;
  tk.ticket = -1;
  decode_task<T, D, HW, KW, KV8>(a, tk, lds, nullptr);
}

// Combines the split partials of every (sequence, kv head) whose sequence
// was split: one wave per (sequence, kv head); softmax-weighted (LSE) merge.
template <typename T, int D>
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
    T* op = (T*)a.out + (si.q_row_start + rr) * a.out_row_stride + (int64_t)(kvh * G + gg) * D + d4;
    st8(op, u32x2{E16<T>::pack2(o[0] * inv, o[1] * inv), E16<T>::pack2(o[2] * inv, o[3] * inv)});
  }
}

// ============================================================== prefill
// LDS ring of NS stages: the K tiles of all stages first, then the V tiles
// ([K_0 .. K_{NS-1}][V_0 .. V_{NS-1}]), so that with the stage known at
// compile time every operand read is one per-lane register plus an immediate
// offset (< 64 KB): K reads need no base at all, V reads one base register
// that holds the V region's start.
template <int D, int NS> struct PrefillCfg {
  static constexpr int kBN = 64;                   // keys per tile
  static constexpr int kRow = D * 2;               // bytes per K/V row in LDS (16-byte chunks XOR-swizzled)
  static constexpr int kTile = kBN * kRow;         // bytes per K (or V) tile
  static constexpr int kStages = NS;               // LDS ring: tiles t+1 .. t+NS-1 in flight while t is computed
  static constexpr int kVBase = NS * kTile;        // start of the V tiles
  static constexpr int kBidCache = 1024;           // block ids cached per workgroup
  static constexpr int kLdsBytes = 2 * NS * kTile + kBidCache * 4;
  static_assert((NS - 1) * kTile + (kBN - 16) * kRow < 65536, "stage offsets must fit a DS immediate");
};


// Logical 16-byte chunk c of LDS row r is stored at chunk c ^ pf_swz(r).  The
// pattern keeps the three access shapes of a tile free of bank conflicts:
//   QK operand reads (ds_read_b128): 16 lanes read one logical chunk of 16
//     consecutive rows -> pf_swz is a bijection on r mod 16 (D = 128), or on
//     each parity class of r mod 16 (D = 64, two rows per 256-byte bank line);
//   PV operand reads (ds_read_b64_tr_b16): 32 lanes read chunks 4j..4j+3 of
//     rows 4i..4i+3 -> the upper bits of pf_swz differ across those rows;
//   tile stores: the lanes storing one row write all its chunks.
template <int D>
__device__ __forceinline__ int pf_swz(int r) {
  return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

// One NW-wave workgroup: each wave owns 32 query rows of one query head; the
// waves cover (head, row block) pairs of one kv head, so every K/V tile staged
// in LDS serves up to NW x 32 query rows.  K/V tiles of 64 keys stream from
// HBM straight into an NS-stage LDS ring (global_load_lds, NS/2 tiles ahead,
// one barrier per NS/2 tiles).  A tile is processed as two 32-key halves: S^T = K
// Q^T for both halves is issued first, so the softmax of half 0 runs on the
// VALU while the MFMAs of half 1 execute, and the softmax of half 1 overlaps
// O^T += V^T P^T of half 0.  Softmax: exp argument as one FMA, lazy rescale
// of the running max (exact), branch-free except the rare rescale of O.
// Paged mode: keys through the block table, causal mask on diagonal tiles
// only.  Dense mode (DENSE): keys from k/v [B, T, Hkv, D], additive bias
// [B, T_q, T] on every tile.
template <typename T, int D, bool DENSE, int NW, int NS, bool KV8>
__device__ __forceinline__ void prefill_wg(const AttnArgs& a, const WorkItem& it, int seq, int kvh, int wgrp, char* lds) {
  static_assert(!(DENSE && KV8), "the dense op has no cache");
  using Cfg = PrefillCfg<D, NS>;
  constexpr int NQ = D / 16;               // Q operand chunks (16 dims)
  constexpr int NO = D / 32;               // output blocks (32 dims)
  constexpr int BN = Cfg::kBN;
  constexpr int RW = Cfg::kRow;
  constexpr int CPR = D / 8;               // 16-byte chunks per key row
  constexpr int NT = 64 * NW;              // threads per workgroup
  int32_t* const lbid = reinterpret_cast<int32_t*>(lds + 2 * Cfg::kStages * Cfg::kTile);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31, h = lane >> 5;

  int ctx, qlen, TK;
  int64_t qstart;
  if (DENSE) {
    ctx = 0;
    qlen = a.dense_Tq;
    TK = a.dense_T;
    qstart = (int64_t)seq * a.dense_Tq;
  } else {
    ctx = it.ctx_len;
    qlen = it.q_len;
    TK = ctx + qlen;
    qstart = it.q_row_start;
  }
  const int G = a.num_q_heads / a.num_kv_heads;
  const int nrb = (qlen + 31) / 32;
  const int combo = wgrp * NW + wave;
  const bool wact = combo < G * nrb;
  const int g = wact ? combo % G : 0;
  const int rblk = wact ? combo / G : 0;
  const int r0 = rblk * 32;
  const int last_combo = min(wgrp * NW + NW - 1, G * nrb - 1);
  const int kend_wg = DENSE ? TK : ctx + min(qlen - 1, (last_combo / G) * 32 + 31) + 1;
  const int kend_w = DENSE ? TK : ctx + min(qlen - 1, r0 + 31) + 1;
  const int r = r0 + n;
  const bool row_ok = wact && r < qlen;
  const int rr = min(r, qlen - 1);
  const int vis = ctx + rr;
  const int64_t qrow = qstart + rr;
  const int qh = kvh * G + g;

  // Block ids of keys [0, kend_wg), loaded into registers now and cached in
  // LDS (first kBidCache blocks; any beyond are read from the table
  // directly) after the first tiles' copies are issued.
  const int32_t* bt = DENSE ? nullptr : a.block_table + (int64_t)seq * a.block_table_stride;
  constexpr int KB = (Cfg::kBidCache + NT - 1) / NT;
  const int nbc = DENSE ? 0 : min((int)div_bs((uint32_t)(kend_wg - 1), a.block_magic, a.block_shift) + 1, Cfg::kBidCache);
  uint32_t lb[KB];
#pragma unroll
  for (int k = 0; k < KB; ++k) lb[k] = tid + k * NT < nbc ? (uint32_t)bt[tid + k * NT] : 0u;

  // Q rows (and their cos/sin rows): loads issued now, used after the first
  // K/V copies are on their way.
  u32x4 qraw[NQ], craw[NQ / 2], sraw[NQ / 2];
  const bool q_rope = !DENSE && a.rope_mode != kRopeNone;
  {
    const T* qp = (const T*)a.q + qrow * a.q_row_stride + (int64_t)qh * D + 8 * h;
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) qraw[kk] = ld16(qp + 16 * kk);
    if (q_rope) {
      const int64_t crow = a.rope_mode == kRopeByPosition ? (int64_t)vis : qrow;
      const T* cp = (const T*)a.rope_cos + crow * a.rope_row_stride + 8 * h;
      const T* sp = (const T*)a.rope_sin + crow * a.rope_row_stride + 8 * h;
#pragma unroll
      for (int kk = 0; kk < NQ / 2; ++kk) {
        craw[kk] = ld16(cp + 16 * kk);
        sraw[kk] = ld16(sp + 16 * kk);
      }
    }
  }
  u32x4 qB[NQ];                 // filled once the first tile copies are issued

  // Per-lane byte offsets inside a stage (tile-invariant; the stage and the
  // half / 16-key group go into the instructions' immediate offsets).
  int koff[NQ];                 // K operand: row n, logical chunk 2kk + h
#pragma unroll
  for (int kk = 0; kk < NQ; ++kk) koff[kk] = n * RW + (((2 * kk + h) ^ pf_swz<D>(n)) << 4);
  int voff[2][NO];              // V^T operand: rows 4h + i16/4 (+8), byte column 64db + 32(g4&1) + 8(i16&3)
  {
    const int g4 = lane >> 4, i16 = lane & 15;
    const int clo = 2 * (g4 & 1) + ((i16 & 3) >> 1);
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2) {
      const int row = 4 * h + (i16 >> 2) + 8 * r2;
#pragma unroll
      for (int db = 0; db < NO; ++db) {
        // the V region's start rides in the register (kept opaque so the
        // compiler does not move it into the immediate, where it cannot fit
        // beside the stage offset)
        int v = Cfg::kVBase + row * RW + (((4 * db + clo) ^ pf_swz<D>(row)) << 4) + 8 * (i16 & 1);
        asm volatile("" : "+v"(v));
        voff[r2][db] = v;
      }
    }
  }

  // K/V tile copy: 1 KB segments (RPS key rows each); wave w copies segments
  // w, w + NW, ...; lane l fills physical chunk l % CPR of row l / CPR, i.e.
  // it loads logical chunk (l % CPR) ^ pf_swz(row).
  constexpr int RPS = 1024 / RW;
  constexpr int NSEG = BN / RPS;
  constexpr int CHD = NSEG / NW;          // copies per wave per K (or V) tile
  static_assert(CHD >= 1 && NSEG % NW == 0, "tile / workgroup mismatch");
  constexpr int E = KV8 ? 1 : 2;           // bytes per cached element
  const uint32_t sbytes = (uint32_t)(a.cache_slot_stride * E);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  // Slots of the DMA rows of the tile starting at key ts: block id from the
  // LDS cache (or the table past it) times the block size plus the offset in
  // the block.  Fetched one tile before the copy is issued, so the copy never
  // waits on LDS.
  auto dma_bids = [&](int ts, uint32_t (&slot)[CHD]) {
#pragma unroll
    for (int i = 0; i < CHD; ++i) {
      if (DENSE) {
        slot[i] = 0;
      } else {
        const int p = min(ts + (i * NW + wave) * RPS + lane / CPR, kend_wg - 1);
        const uint32_t bi = div_bs((uint32_t)p, a.block_magic, a.block_shift);
        uint32_t blk;
        if (bi < (uint32_t)Cfg::kBidCache) {
          blk = (uint32_t)lbid[bi];
        } else {
          blk = (uint32_t)bt[bi];
          if (blk >= (uint64_t)a.num_blocks) blk = 0;
        }
        slot[i] = blk * (uint32_t)a.block_size + ((uint32_t)p - bi * (uint32_t)a.block_size);
      }
    }
  };
  // Source of one lane's 8 elements (logical chunk lc of its row) for copy
  // instruction i, K (v = 0) or V (v = 1), of the tile at key ts (paged: the
  // row's slot from dma_bids).
  auto copy_src = [&](int ts, const uint32_t (&slot)[CHD], int i, int v) -> const char* {
    const int sg = i * NW + wave;
    const int row = sg * RPS + lane / CPR;
    const int lc = (lane % CPR) ^ pf_swz<D>(row);
    if (DENSE) {
      const int p = min(ts + row, kend_wg - 1);
      return (v ? (const char*)a.v + ((int64_t)seq * a.v_batch_stride + (int64_t)p * a.v_row_stride + (int64_t)kvh * D) * 2
                : (const char*)a.k + ((int64_t)seq * a.k_batch_stride + (int64_t)p * a.k_row_stride + (int64_t)kvh * D) * 2) +
             lc * 16;
    }
    const uint64_t off = (uint64_t)slot[i] * sbytes + (uint64_t)kvh * D * E;
    return (const char*)(v ? a.v_cache : a.k_cache) + off + lc * 8 * E;
  };
  // One copy instruction into `stage`: bf16 caches go HBM -> LDS directly;
  // fp8 caches are fetched into registers (`fp8_fetch`, a tile ahead) and
  // widened to bf16 when written (`fp8_put`), so LDS always holds bf16.
  auto dma_one = [&](int ts, int stage, const uint32_t (&blk)[CHD], int i, int v) {
    const int sg = i * NW + wave;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds0 + v * Cfg::kVBase + stage * Cfg::kTile + sg * 1024);
    lds_dma16(copy_src(ts, blk, i, v), dst);
  };
  u32x2 f8st[CHD][2];                      // fp8 cache: fetched chunks of the tile being copied
  auto fp8_fetch = [&](int ts, const uint32_t (&blk)[CHD]) {
#pragma unroll
    for (int i = 0; i < CHD; ++i)
#pragma unroll
      for (int v = 0; v < 2; ++v) f8st[i][v] = *reinterpret_cast<const u32x2*>(copy_src(ts, blk, i, v));
  };
  auto fp8_put = [&](int stage, int i, int v) {
    const int sg = i * NW + wave;
    *reinterpret_cast<u32x4*>(lds + v * Cfg::kVBase + stage * Cfg::kTile + sg * 1024 + lane * 16) =
        fp8x8_to<T>(f8st[i][v][0], f8st[i][v][1]);
  };
  auto dma_issue = [&](int ts, int stage, const uint32_t (&blk)[CHD]) {
    if (KV8) fp8_fetch(ts, blk);
#pragma unroll
    for (int i = 0; i < CHD; ++i)
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        if (KV8)
          fp8_put(stage, i, v);
        else
          dma_one(ts, stage, blk, i, v);
      }
  };

  const float sl2 = a.scale * kLog2e;
  float m = kNegInf, lsum = 0.f;
  float sbase = 0.f;             // dense mode: -(the running max) at the tile's start
  f32x16 o[NO];
#pragma unroll
  for (int db = 0; db < NO; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;

  // Softmax of one 32-key half, in pieces that the tile loop interleaves
  // with MFMAs: lane holds raw scores S[key k0 + 8(j/4) + 4h + j%4][row n].
  // Q enters the MFMA as the exact bf16 value (rotated like apply_rope); the
  // raw fp32 dot products are scaled by scale * log2(e) in fp32, so scores in
  // log2 units carry one fp32 rounding, like the reference's q @ k^T / sqrt(D)
  // (rounding q * scale to bf16 instead would move a score s by up to
  // |s| 2^-9, which at large logits reweights the keys visibly).
  //
  // Paged (causal) mode: each row keeps a reference r and p = 2^(s - r), the
  // scale and the reference applied together by one FMA per score.  The
  // first half-tile of the row (keys 0..31; key 0 is visible to every row)
  // sets r = 0 when its max m1 lies in [-T, T] and r = m1 otherwise, so every
  // row holds some p >= 2^-T and later tiny p lose nothing.  After that S
  // accumulates from zero: no S initialisation, no running max.  The only
  // check is one compare of each lane's partial sum against 2^T: a lane over
  // it (some p > 2^T) sends the wave into a rare fix-up that recomputes the
  // half's S from LDS, moves the reference of every row whose max passed T up
  // to that max (O and l rescaled by 2^-max, exactly) and recomputes p.  With
  // T = 64, p <= 2^64 keeps l and O far from fp32 overflow.  An fp16 model
  // takes P in fp16 (largest value 65504): T = 15, and r starts at m1
  // itself, so p <= 2^15 and the keys that carry the row never fall into
  // fp16's subnormal range.  Numerator and denominator share r, so the result
  // is the exact softmax.
  //
  // Dense (arbitrary bias) mode: lazy running max (the max only moves when a
  // row's max exceeds it by more than 8, so p <= 2^8); scale, bias and the
  // tile's starting offset -m enter one FMA per score, so the exponent is
  // s - m directly (a subtract of the max's move otherwise, rare).
  constexpr bool kFast = !DENSE;
  constexpr bool kF16 = E16<T>::kF16;
  constexpr float kT = kF16 ? 15.f : 64.f;
  constexpr float kTwoT = kF16 ? 32768.f : 18446744073709551616.f;   // 2^T
  float rref = 0.f;              // paged mode: the row's reference r (log2 units)
  struct Soft { float alpha, dlt, psum; };
  auto row_max = [&](const f32x16& s) {
    float tmax = kNegInf;
#pragma unroll
    for (int j = 0; j < 16; j += 2)
      tmax = __builtin_elementwise_maximum(tmax, __builtin_elementwise_maximum(s[j], s[j + 1]));
    auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
    return __builtin_elementwise_maximum(__uint_as_float(x[0]), __uint_as_float(x[1]));
  };
  // key k0 + 8(j/4) + 4h + j%4 is hidden iff 8(j/4) + j%4 > vis - k0 - 4h:
  // one per-lane limit against compile-time offsets (nothing to hoist onto the
  // common path)
  auto apply_mask = [&](f32x16& s, int k0) {
    const int lim = vis - k0 - 4 * h;
#pragma unroll
    for (int j = 0; j < 16; ++j) s[j] = 8 * (j >> 2) + (j & 3) > lim ? kNegInf : s[j];
  };
  // paged mode, piece 0: scale and reference (one FMA), the causal mask, and
  // on the row's first half-tile the choice of r
  auto fs_prep = [&](f32x16& s, int k0, bool mask, bool first) {
    const float nr = -rref;
#pragma unroll
    for (int j = 0; j < 16; ++j) s[j] = __builtin_fmaf(s[j], sl2, nr);
    if (mask) apply_mask(s, k0);
    if (first) {
      const float m1 = row_max(s);
      rref = (!kF16 && m1 >= -kT && m1 <= kT) || m1 == kNegInf ? 0.f : m1;
      if (__builtin_amdgcn_ballot_w64(rref != 0.f)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) s[j] -= rref;
      }
    }
  };
  auto sm_max = [&](f32x16& s, int k0, bool mask, Soft& q) {
    if (DENSE) {
      const T* bp = (const T*)a.bias + (int64_t)seq * a.bias_batch_stride + (int64_t)rr * a.bias_row_stride;
#pragma unroll
      for (int j = 0; j < 16; ++j) {   // bias in natural-log units: to log2 units like the scaled scores
        const int key = k0 + 8 * (j >> 2) + 4 * h + (j & 3);
        const float bv = key < TK ? (float)bp[key] : kNegInf;
        s[j] = __builtin_fmaf(s[j], sl2, __builtin_fmaf(bv, kLog2e, sbase));
      }
    } else if (mask) {
      apply_mask(s, k0);
    }
    const float tmax = row_max(s) - sbase;
    const float mn = tmax > m + 8.f ? tmax : m;
    q.alpha = mn > m ? fast_exp2(m - mn) : 1.f;
    m = mn;
    // s holds s_true + sbase; the exponent is s_true - m = s - (sbase + m)
    q.dlt = mn == kNegInf ? 0.f : sbase + mn;
    if (__builtin_amdgcn_ballot_w64(q.dlt != 0.f)) {
#pragma unroll
      for (int j = 0; j < 16; ++j) s[j] -= q.dlt;
    }
  };
  auto sm_exp = [&](f32x16& s, int j0) {
#pragma unroll
    for (int j = j0; j < j0 + 4; ++j) s[j] = fast_exp2(s[j]);
  };
  // row sum of the half's bf16-rounded p (the values the P V MFMA takes)
  auto sm_sum = [&](const u32x4* pb, Soft& q) {
    const u32x4 w0 = pb[0], w1 = pb[1];
    float a0 = E16<T>::add2(w0[0], 0.f), a1 = E16<T>::add2(w1[0], 0.f);
#pragma unroll
    for (int e = 1; e < 4; ++e) {
      a0 = E16<T>::add2(w0[e], a0);
      a1 = E16<T>::add2(w1[e], a1);
    }
    q.psum = a0 + a1;
    if (!kFast) lsum = __builtin_fmaf(lsum, q.alpha, q.psum);
  };
  auto sm_cvt = [&](const f32x16& s, u32x4* pb) {
    float pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = s[e];
    pb[0] = pack8<T>(pv);
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = s[8 + e];
    pb[1] = pack8<T>(pv);
  };
  // Logical softmax piece p (0..7) of a half: max (dense) or prep (paged),
  // 4 x exp, convert, sum.
  auto sm_piece = [&](int p, f32x16& s, int k0, bool mask, Soft& q, u32x4* pb, bool first) {
    if (p == 0) {
      if (kFast) fs_prep(s, k0, mask, first);
      else sm_max(s, k0, mask, q);
    }
    else if (p <= 4) sm_exp(s, 4 * (p - 1));
    else if (p == 5) sm_cvt(s, pb);
    else if (p == 6) sm_sum(pb, q);
  };
  // After a half's pieces.  Dense: the rare O rescale of the lazy max
  // (q.psum >= 0 always; testing it keeps the half's exponentials ahead of
  // the branch, in the region where they overlap the MFMAs).  Paged: the rare
  // fix-up of a half whose p passed 2^T (S recomputed from the stage `st`,
  // half kb), then the half's sum joins the row's.
  auto commit = [&](Soft& q, const char* st, int kb, int k0, bool mask, u32x4* pb) {
    if (!kFast) {
      if (__builtin_amdgcn_ballot_w64(q.alpha != 1.f || q.psum < 0.f)) {
#pragma unroll
        for (int db = 0; db < NO; ++db) o[db] *= q.alpha;
      }
      return;
    }
    if (__builtin_amdgcn_ballot_w64(q.psum > kTwoT)) {
      f32x16 t = {};
#pragma unroll
      for (int kk = 0; kk < NQ; ++kk)
        t = E16<T>::mfma32(*reinterpret_cast<const u32x4*>(st + 32 * kb * RW + koff[kk]), qB[kk], t);
      const float nr = -rref;
#pragma unroll
      for (int j = 0; j < 16; ++j) t[j] = __builtin_fmaf(t[j], sl2, nr);
      if (mask) apply_mask(t, k0);
      const float tmax = row_max(t);
      const float d = tmax > kT ? tmax : 0.f;          // rows whose p passed 2^T move up to their max
      const float alpha = fast_exp2(-d);
#pragma unroll
      for (int db = 0; db < NO; ++db) o[db] *= alpha;
      lsum *= alpha;
      rref += d;
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        float e0 = fast_exp2(t[j] - d), e1 = fast_exp2(t[j + 1] - d);
        round2<T>(e0, e1);                      // the values the P V MFMA takes
        t[j] = e0;
        t[j + 1] = e1;
      }
      // summed in fp32 here (a sum over the packed operands on this rare path
      // costs the common path ~30 VGPRs in the compiler's allocation)
      float ps4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ps4[e] = (t[e] + t[e + 4]) + (t[e + 8] + t[e + 12]);
      q.psum = (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
      sm_cvt(t, pb);
    }
    lsum += q.psum;
  };
  // V^T operand reads of one 16-key group (tp) and output block (db) of half
  // kb; st: the stage's K tile (the V tile sits at the same offset from the V
  // region's start, which voff carries)
  auto vread1 = [&](const char* st, int kb, int tp, int db) -> u32x4 {
    const char* base = st + (32 * kb + 16 * tp) * RW;
    const u32x2 r1 = lds_read_tr16(base + voff[0][db]);
    const u32x2 r2 = lds_read_tr16(base + voff[1][db]);
    return u32x4{r1[0], r1[1], r2[0], r2[1]};
  };

  // st: the tile's stage (its K tile; V at the same offset in the V region).
  // The tile is scheduled by
  // hand (sched_barrier fences keep the source order): (1) K reads of half 0,
  // S^T of half 0 with the K reads of half 1 between its MFMAs, then the
  // MFMAs of S^T half 1 each followed by two V reads of half
  // 0 and one softmax piece of half 0; (2) the MFMAs of O^T += V^T P^T half 0,
  // each followed by V reads and a softmax piece of half 1; (3) P V of half 1.
  // One wave thus keeps the matrix core busy while its own VALU work runs;
  // the two commits (rare wave-uniform branches inside) split the regions.
  // `first`: the row's first tile (key 0).
  auto compute = [&](const char* st, int ts, bool mask, bool dma, int dts, int dstage, const uint32_t (&blk)[CHD],
                     bool first) {
    f32x16 s0, s1;
    u32x4 va0[2][NO], va1[2][NO];
    u32x4 pb0[2], pb1[2];
    Soft q0, q1;
    u32x4 ka[2][NQ];
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) ka[0][kk] = *reinterpret_cast<const u32x4*>(st + koff[kk]);
    s0 = f32x16{};
    s1 = f32x16{};
    if (!kFast) sbase = m == kNegInf ? 0.f : -m;   // both halves start from the max before this tile
    // K of half 1 is read between the MFMAs of half 0: the eight waves' reads
    // after a barrier do not all hit LDS at once, and fewer registers are live
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) {
      s0 = E16<T>::mfma32(ka[0][kk], qB[kk], s0);
      ka[1][kk] = *reinterpret_cast<const u32x4*>(st + 32 * RW + koff[kk]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // region 1: S^T half 1 | V reads half 0 | softmax half 0
    constexpr int V_PER = 2 * NO / NQ;           // V operand reads (pairs) per slot
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) {
      s1 = E16<T>::mfma32(ka[1][kk], qB[kk], s1);
#pragma unroll
      for (int v = 0; v < V_PER; ++v) {
        const int idx = kk * V_PER + v;          // (tp, db) = (idx / NO, idx % NO)
        va0[idx / NO][idx % NO] = vread1(st, 0, idx / NO, idx % NO);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int p = kk * 8 / NQ; p < (kk + 1) * 8 / NQ; ++p) sm_piece(p, s0, ts, mask, q0, pb0, first);
      __builtin_amdgcn_sched_barrier(0);
    }
    commit(q0, st, 0, ts, mask, pb0);
    // region 2: P V half 0 | V reads half 1 | softmax half 1
#pragma unroll
    for (int i = 0; i < 2 * NO; ++i) {
      const int tp = i / NO, db = i % NO;
      o[db] = E16<T>::mfma32(va0[tp][db], pb0[tp], o[db]);
      va1[tp][db] = vread1(st, 1, tp, db);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int p = i * 8 / (2 * NO); p < (i + 1) * 8 / (2 * NO); ++p)
        sm_piece(p, s1, ts + 32, mask, q1, pb1, false);
      __builtin_amdgcn_sched_barrier(0);
    }
    commit(q1, st, 1, ts + 32, mask, pb1);
    // region 3: P V half 1, with the copy of a later tile spread between
    // the MFMAs (a burst of copies right after the barrier stalls the wave)
    static_assert(CHD <= NO, "copy instructions must fit between the P V MFMAs");
    if (dma) {
#pragma unroll
      for (int i = 0; i < 2 * NO; ++i) {
        const int tp = i / NO, db = i % NO;
        o[db] = E16<T>::mfma32(va1[tp][db], pb1[tp], o[db]);
        if (i < 2 * CHD) {
          if (KV8)
            fp8_put(dstage, i / 2, i % 2);     // fetched at the start of the tile
          else
            dma_one(dts, dstage, blk, i / 2, i % 2);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2 * NO; ++i) {
        const int tp = i / NO, db = i % NO;
        o[db] = E16<T>::mfma32(va1[tp][db], pb1[tp], o[db]);
      }
    }
  };

  // Tile t lives in stage t % NS.  Iteration t: wait for this thread's
  // copies of tile t, barrier (tile t visible to all waves; all waves are
  // done with tile t-1), then start the copy of tile t+NS-1 into tile t-1's
  // stage.
  // Tiles are taken TPB = NS / 2 at a time: one barrier per group (tile
  // t0 .. t0+TPB-1 visible to all waves; all waves are done with the previous
  // group).  Tile t lives in stage t % NS; its copy is spread over the P V
  // MFMAs of tile t - TPB, into that tile's stage.
  constexpr int TPB = NS / 2;
  static_assert(NS % 2 == 0 && TPB >= 1, "stage ring must hold two tile groups");
  const int ntiles = (kend_wg + BN - 1) / BN;
  const int full_end = ctx + r0;           // tiles ending at or before key ctx + r0 need no mask
  // The first TPB tiles' copies are addressed with block ids read straight
  // from the table (issued together with the loads above), so they need no
  // trip through LDS and a barrier first; every load so far is waited for
  // here explicitly, so nothing below waits on these copies by accident.
  uint32_t fbid[TPB][CHD], foff[TPB][CHD];
#pragma unroll
  for (int t = 0; t < TPB; ++t)
#pragma unroll
    for (int i = 0; i < CHD; ++i) {
      fbid[t][i] = 0u;
      foff[t][i] = 0u;
      if (!DENSE) {
        const int p = min(t * BN + (i * NW + wave) * RPS + lane / CPR, kend_wg - 1);
        const uint32_t bi = div_bs((uint32_t)p, a.block_magic, a.block_shift);
        fbid[t][i] = (uint32_t)bt[bi];
        foff[t][i] = (uint32_t)p - bi * (uint32_t)a.block_size;
      }
    }
  wait_vmcnt<0>();
#pragma unroll
  for (int t = 0; t < TPB; ++t)
    if (t < ntiles) {
#pragma unroll
      for (int i = 0; i < CHD; ++i) {
        if (fbid[t][i] >= (uint64_t)a.num_blocks) fbid[t][i] = 0u;  // never address outside the pool
        fbid[t][i] = fbid[t][i] * (uint32_t)a.block_size + foff[t][i];   // the row's slot
      }
      dma_issue(t * BN, t, fbid[t]);
    }
  if (!DENSE) {
#pragma unroll
    for (int k = 0; k < KB; ++k)
      if (tid + k * NT < nbc) lbid[tid + k * NT] = lb[k] < (uint64_t)a.num_blocks ? (int32_t)lb[k] : 0;
  }
  uint32_t nbid[CHD];

  // Q as the B operand of S^T = K Q^T: lane holds Q[row n][16kk + 8h + i].
  {
    float x[NQ][8];
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) unpack8<T>(qraw[kk], x[kk]);
    if (q_rope) {
#pragma unroll
      for (int kk = 0; kk < NQ / 2; ++kk) {
        float c[8], sn[8];
        unpack8<T>(craw[kk], c);
        unpack8<T>(sraw[kk], sn);
        rope8<T>(x[kk], x[kk + NQ / 2], c, sn);
      }
    }
#pragma unroll
    for (int kk = 0; kk < NQ; ++kk) qB[kk] = pack8<T>(x[kk]);   // exact: q and its rotation are in T
  }
  if (!DENSE) __syncthreads();  // block ids in LDS visible
  if (TPB < ntiles) dma_bids(TPB * BN, nbid);

  // The loop walks the ring NS tiles at a time so that every stage index is a
  // compile-time constant (operand reads then carry it as an immediate); a
  // barrier opens each group of TPB tiles.
  for (int t0 = 0; t0 < ntiles; t0 += NS) {
#pragma unroll
    for (int gi = 0; gi < NS / TPB; ++gi) {
      const int tg = t0 + gi * TPB;
      if (tg < ntiles) {
        wait_vmcnt<0>();                     // this thread's copies of tiles tg .. tg+TPB-1
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TPB; ++u) {
          const int t = tg + u;
          const int stage = gi * TPB + u;    // == t % NS
          if (t < ntiles) {
            const int ts = t * BN;
            const bool dma = t + TPB < ntiles;
            const int dts = (t + TPB) * BN, dstage = (stage + TPB) % NS;
            if (KV8 && dma && wact && ts < kend_w) fp8_fetch(dts, nbid);   // written in the tile's last region
            if (wact && ts < kend_w)
              compute(lds + stage * Cfg::kTile, ts, DENSE || ts + BN - 1 > full_end, dma, dts, dstage, nbid, t == 0);
            else if (dma)
              dma_issue(dts, dstage, nbid);
            if (t + TPB + 1 < ntiles) dma_bids((t + TPB + 1) * BN, nbid);
          }
        }
      }
    }
  }

  if (row_ok) {
    const float inv = 1.f / sum_xor32(lsum);
    T* op = (T*)a.out + qrow * a.out_row_stride + (int64_t)qh * D + 4 * h;
#pragma unroll
    for (int db = 0; db < NO; ++db)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        u32x2 w = {E16<T>::pack2(o[db][4 * jq] * inv, o[db][4 * jq + 1] * inv),
                   E16<T>::pack2(o[db][4 * jq + 2] * inv, o[db][4 * jq + 3] * inv)};
        st8(op + 32 * db + 8 * jq, w);
      }
  }
}

// ============================================================== kernels
constexpr int kPrefillStages = 4;     // prefill LDS ring: two groups of two 64-key tiles

template <int D, bool PF, bool DC, int NW> struct MixedLds {
  static constexpr int a = PF ? PrefillCfg<D, kPrefillStages>::kLdsBytes : 0;
  static constexpr int b = DC ? DecodeCfg<D, NW>::kLdsBytes : 0;
  static constexpr int kBytes = a > b ? a : b;
};

// Workgroup b of a launch is dispatched to XCD b % 8, and each XCD has its
// own L2.  When a decode workgroup reads less than a 128-byte line of each
// slot (fp8 cache, HW x D < 128 bytes), the neighbouring kv-head group reads
// the rest of the line; unless both run on one XCD, both L2s fetch the whole
// line from HBM.  Grouped, every 64 workgroups are transposed (8 x 8) so
// that XCD x runs items 8x .. 8x+7 of the 64, i.e. the consecutive head
// groups of one sequence (a ragged last group keeps its order).  The
// planner's pairing of item k with item k + CUs on one CU survives: the same
// transposition applies to every full 64.
template <bool GROUP>
__device__ __forceinline__ int xcd_item(int b, int n) {
  if (!GROUP || (b | 63) >= n) return b;
  const int P = b & 63;
  return (b & ~63) + (P & 7) * 8 + (P >> 3);
}

// Work items of both kinds in one launch (mixed continuous batch; 8-wave
// workgroups), or decode items only (HW x KW waves).  T: the model dtype
// (__bf16 or _Float16), also the cache's unless KV8 (fp8 e4m3fn cache).
template <typename T, int D, bool PF, bool DC, int HW, int KW, bool KV8>
__global__ void __launch_bounds__(64 * HW * KW) paged_attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[MixedLds<D, PF, DC, HW * KW>::kBytes];
  const WorkItem it = a.items[xcd_item<!PF && KV8 && HW * D < 128>(blockIdx.x, a.n_items)];
  if (PF && (!DC || (it.kind_b & 0xff) == kItemPrefill)) {
    if constexpr (HW * KW == kWaves)
      prefill_wg<T, D, false, kWaves, kPrefillStages, KV8>(a, it, it.seq, it.a, it.kind_b >> 8, lds);
    return;
  }
  if constexpr (DC) decode_wg<T, D, HW, KW, KV8>(a, it, lds);
}

// Page-balanced decode: workgroup w runs its key segments in order (all
// waves converge between segments; the LDS staging is reused).
template <typename T, int D, int HW, int KW, bool KV8>
__global__ void __launch_bounds__(64 * HW * KW) __attribute__((amdgpu_waves_per_eu(D == 64 ? 4 : 2)))
decode_balanced_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[DecodeCfg<D, HW * KW>::kLdsBytes];
  __shared__ int ticket;
  const int s0 = a.seg_ptr[blockIdx.x], s1 = a.seg_ptr[blockIdx.x + 1];
  for (int s = s0; s < s1; ++s) {
    if (s > s0) __syncthreads();
    const DecodeSeg sg = a.segs[s];
    const DecodeTask tk{sg.seq, sg.hg, sg.k0, sg.k1, sg.q_row_start, sg.ctx_len, sg.q_len,
                        sg.nseg, sg.pbase, sg.ord, sg.ticket};
    decode_task<T, D, HW, KW, KV8>(a, tk, lds, &ticket);
  }
}

// Mixed continuous batch, page-balanced: workgroups [0, n_seg_wgs) run equal
// key shares of the decode sequences (segments, as decode_balanced_kernel);
// each later workgroup runs one prefill item.  One 8-wave workgroup per CU
// (the prefill path's LDS ring and registers).
template <typename T, int D, int HW, bool KV8>
__global__ void __launch_bounds__(64 * kWaves) mixed_balanced_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[MixedLds<D, true, true, kWaves>::kBytes];
  __shared__ int ticket;
  const int b = blockIdx.x;
  if (b >= a.n_seg_wgs) {
    const WorkItem it = a.items[b - a.n_seg_wgs];
    prefill_wg<T, D, false, kWaves, kPrefillStages, KV8>(a, it, it.seq, it.a, it.kind_b >> 8, lds);
    return;
  }
  const int s0 = a.seg_ptr[b], s1 = a.seg_ptr[b + 1];
  for (int s = s0; s < s1; ++s) {
    if (s > s0) __syncthreads();
    const DecodeSeg sg = a.segs[s];
    const DecodeTask tk{sg.seq, sg.hg, sg.k0, sg.k1, sg.q_row_start, sg.ctx_len, sg.q_len,
                        sg.nseg, sg.pbase, sg.ord, sg.ticket};
    decode_task<T, D, HW, kWaves / HW, KV8>(a, tk, lds, &ticket);
  }
}

// Prefill items only: kPrefillOnlyWaves-wave workgroups with a
// kPrefillOnlyStages-stage ring.
template <typename T, int D, bool KV8>
__global__ void __launch_bounds__(64 * kPrefillOnlyWaves) __attribute__((amdgpu_waves_per_eu(2)))
prefill_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[PrefillCfg<D, kPrefillOnlyStages>::kLdsBytes];
  const WorkItem it = a.items[blockIdx.x];
  prefill_wg<T, D, false, kPrefillOnlyWaves, kPrefillOnlyStages, KV8>(a, it, it.seq, it.a, it.kind_b >> 8, lds);
}

template <typename T, int D>
__global__ void __launch_bounds__(64 * kWaves) dense_attn_kernel(AttnArgs a, int nwg) {
  __shared__ __attribute__((aligned(16))) char lds[PrefillCfg<D, kPrefillStages>::kLdsBytes];
  const int w = blockIdx.x % nwg;
  const int rest = blockIdx.x / nwg;
  const int kvh = rest % a.num_kv_heads;
  const int b = rest / a.num_kv_heads;
  const WorkItem none{};
  prefill_wg<T, D, true, kWaves, kPrefillStages, false>(a, none, b, kvh, w, lds);
}

template <typename T, int D, int HW, int KW, bool KV8>
static void launch_paged_hk(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  dim3 grid(a.n_items);
  if (pf && dc) {
    if constexpr (HW * KW == kWaves)
      hipLaunchKernelGGL((paged_attn_kernel<T, D, true, true, HW, KW, KV8>), grid, dim3(64 * kWaves), 0, st, a);
  } else if (pf) {
    hipLaunchKernelGGL((prefill_kernel<T, D, KV8>), grid, dim3(64 * kPrefillOnlyWaves), 0, st, a);
  } else {
    hipLaunchKernelGGL((paged_attn_kernel<T, D, false, true, HW, KW, KV8>), grid, dim3(64 * HW * KW), 0, st, a);
  }
}

template <typename T, int D, bool KV8>
static hipError_t launch_decode_balanced(const AttnArgs& a, hipStream_t st) {
  const dim3 grid(a.n_items);
  switch (a.heads_per_wg) {
    case 1: hipLaunchKernelGGL((decode_balanced_kernel<T, D, 1, 8, KV8>), grid, dim3(512), 0, st, a); break;
    case 2: hipLaunchKernelGGL((decode_balanced_kernel<T, D, 2, 4, KV8>), grid, dim3(512), 0, st, a); break;
    case 4: hipLaunchKernelGGL((decode_balanced_kernel<T, D, 4, 2, KV8>), grid, dim3(512), 0, st, a); break;
    case 8: hipLaunchKernelGGL((decode_balanced_kernel<T, D, 8, 1, KV8>), grid, dim3(512), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int D, bool KV8>
static hipError_t launch_mixed_balanced(const AttnArgs& a, hipStream_t st) {
  const dim3 grid(a.n_items);
  switch (a.heads_per_wg) {
    case 1: hipLaunchKernelGGL((mixed_balanced_kernel<T, D, 1, KV8>), grid, dim3(64 * kWaves), 0, st, a); break;
    case 2: hipLaunchKernelGGL((mixed_balanced_kernel<T, D, 2, KV8>), grid, dim3(64 * kWaves), 0, st, a); break;
    case 4: hipLaunchKernelGGL((mixed_balanced_kernel<T, D, 4, KV8>), grid, dim3(64 * kWaves), 0, st, a); break;
    case 8: hipLaunchKernelGGL((mixed_balanced_kernel<T, D, 8, KV8>), grid, dim3(64 * kWaves), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int D, bool KV8>
static hipError_t launch_paged_d(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  const int hw = a.heads_per_wg, nw = a.decode_waves;
  if (a.n_segs > 0) {
    if (nw != kWaves || (pf && a.prefill_waves != kWaves) || a.n_seg_wgs <= 0 || a.n_seg_wgs > a.n_items)
      return hipErrorInvalidValue;
    if (pf) return dc ? launch_mixed_balanced<T, D, KV8>(a, st) : hipErrorInvalidValue;
    return launch_decode_balanced<T, D, KV8>(a, st);
  }
  if (pf && (a.prefill_waves != (dc ? kWaves : kPrefillOnlyWaves) || (dc && nw != kWaves)))
    return hipErrorInvalidValue;
  if (nw == 8) {
    switch (hw) {
      case 1: launch_paged_hk<T, D, 1, 8, KV8>(a, pf, dc, st); break;
      case 2: launch_paged_hk<T, D, 2, 4, KV8>(a, pf, dc, st); break;
      case 4: launch_paged_hk<T, D, 4, 2, KV8>(a, pf, dc, st); break;
      case 8: launch_paged_hk<T, D, 8, 1, KV8>(a, pf, dc, st); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !dc || a.n_partials == 0) return e;
  hipLaunchKernelGGL((merge_splits_kernel<T, D>), dim3(a.num_seqs * a.num_kv_heads), dim3(64), 0, st, a);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_paged_t(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  const bool kv8 = a.kv_dtype == kFP8;
  if (a.head_dim == 64) return kv8 ? launch_paged_d<T, 64, true>(a, pf, dc, st) : launch_paged_d<T, 64, false>(a, pf, dc, st);
  if (a.head_dim == 128)
    return kv8 ? launch_paged_d<T, 128, true>(a, pf, dc, st) : launch_paged_d<T, 128, false>(a, pf, dc, st);
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t launch_dense_t(const AttnArgs& a, dim3 grid, int nwg, hipStream_t st) {
  const dim3 block(64 * kWaves);
  if (a.head_dim == 64)
    hipLaunchKernelGGL((dense_attn_kernel<T, 64>), grid, block, 0, st, a, nwg);
  else if (a.head_dim == 128)
    hipLaunchKernelGGL((dense_attn_kernel<T, 128>), grid, block, 0, st, a, nwg);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

#ifdef GLLM_PAGED_F16
// fp16 models: this file compiled a second time (paged_attention_f16.hip), so
// the two element types build as separate units in parallel.
hipError_t launch_paged_f16(const AttnArgs& a, bool pf, bool dc, hipStream_t st) {
  return launch_paged_t<_Float16>(a, pf, dc, st);
}
hipError_t launch_dense_f16(const AttnArgs& a, dim3 grid, int nwg, hipStream_t st) {
  return launch_dense_t<_Float16>(a, grid, nwg, st);
}
#else
hipError_t launch_paged_f16(const AttnArgs& a, bool pf, bool dc, hipStream_t st);
hipError_t launch_dense_f16(const AttnArgs& a, dim3 grid, int nwg, hipStream_t st);

hipError_t launch_paged_attention_mfma(const AttnArgs& a, bool has_prefill, bool has_decode, hipStream_t st) {
  if (a.n_items == 0) return hipSuccess;
  // the cache holds the model dtype or fp8 e4m3fn
  if (a.kv_dtype != kFP8 && a.kv_dtype != a.dtype) return hipErrorInvalidValue;
  if (a.dtype == kBF16) return launch_paged_t<__bf16>(a, has_prefill, has_decode, st);
  if (a.dtype == kF16) return launch_paged_f16(a, has_prefill, has_decode, st);
  return hipErrorInvalidValue;
}

hipError_t launch_dense_attention_mfma(const AttnArgs& a, int B, int Tq, hipStream_t st) {
  const int G = a.num_q_heads / a.num_kv_heads;
  const int nwg = (G * ((Tq + 31) / 32) + kWaves - 1) / kWaves;
  const int64_t blocks = (int64_t)B * a.num_kv_heads * nwg;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks);
  if (a.dtype == kBF16) return launch_dense_t<__bf16>(a, grid, nwg, st);
  if (a.dtype == kF16) return launch_dense_f16(a, grid, nwg, st);
  return hipErrorInvalidValue;
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
#endif  // GLLM_PAGED_F16

}  // namespace gllm

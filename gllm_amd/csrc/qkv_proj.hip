// Fused QKV projection + RoPE + paged KV write for gfx950: replaces
// gllm/model/layers/attention.py:139-161 (linear_q / linear_k / linear_v,
// apply_rope, and the K/V stores into the paged cache) with one launch, so
// the projected K/V go from the MFMA accumulators to their cache slots
// without a round trip through HBM.
//
// Semantics (bf16 model): q/k/v = x @ W^T with fp32 accumulation, rounded to
// bf16 as F.linear stores them (gllm/model/layers/linear.py:13-19); q and k
// rotated (rotate-half, every op rounded to bf16 like attention.py:105-118);
// k and v cast to the cache dtype and stored at slot_mapping[token]
// (attention.py:156-161), padded rows skipped; q written to q_out.
//
// Tiling: one 4-wave workgroup per (128 tokens, one head of D outputs); for
// large batches at D = 128, one 8-wave workgroup per (256 tokens, two heads)
// whose waves each take 64 tokens x one head (two row blocks share every W
// operand read); both launched in XCD-grouped order (qkv_groups).  X and W
// K-slices of 32 stream HBM/L2 -> LDS with global_load_lds into a 4-stage
// ring (XOR-swizzled 16-byte chunks: operand reads are bank-conflict free);
// each wave computes 32 tokens x D outputs per row block on
// v_mfma_f32_32x32x16_bf16 (D/32 accumulator blocks).  Output column n of
// block b is head dim 32b + n, so a RoPE pair (d, d + D/2) sits in blocks b
// and b + D/64 of the same lane: the rotation happens in registers and every
// value is stored from its lane (4 dims per store where rows are aligned).
// Batches too small to fill the GPU with such tiles split the hidden
// dimension (qkv_partial_kernel + qkv_finish_kernel, below); up to 32 tokens
// take one launch with the whole hidden dimension per workgroup
// (qkv_small_kernel).
#include <algorithm>

#include "common.h"
#include "launch.h"

namespace gllm {

namespace {

// XCD-grouped order of the large-batch tiles: workgroup b of the launch runs
// on XCD b % kXcds, and each XCD takes super-groups of gt token tiles x gh
// head groups (gt * gh = the workgroups one XCD holds at once), so the
// workgroups of a super-group stream the same X and W K-slices through that
// XCD's L2 together.  gh divides the head-group count where it can, so no
// slot of a super-group idles.
constexpr int kXcds = 8;
struct QKVGroups { int gt, gh, nhg; int64_t nsg; };
__host__ __device__ inline QKVGroups qkv_groups(int64_t tiles, int ngroups, int cus) {
  const int slots = cus / kXcds > 0 ? cus / kXcds : 1;
  int gh = 1;
  for (int c = 8; c > 1; c >>= 1)
    if (c <= slots && ngroups % c == 0) { gh = c; break; }
  QKVGroups g;
  g.gh = gh;
  g.gt = (int)std::max<int64_t>(1, std::min<int64_t>(tiles, slots / gh));
  g.nhg = (ngroups + gh - 1) / gh;
  g.nsg = ((tiles + g.gt - 1) / g.gt) * g.nhg;
  return g;
}

// Lane n ^ 1 / n ^ 2 of the lane's quad (DPP quad permutes: no LDS trip).
__device__ __forceinline__ uint32_t quad_xor1(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xf, 0xf, false);   // quad_perm(1,0,3,2)
}
__device__ __forceinline__ uint32_t quad_xor2(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xf, 0xf, false);   // quad_perm(2,3,0,1)
}

// Physical 16-byte chunk of logical chunk c in 64-byte LDS row r: rows
// r, r+4, r+8, r+12 get the 4 chunk rotations, so 16 consecutive rows
// reading one logical chunk hit 16 distinct bank groups.
__device__ __forceinline__ int qkv_swz(int r) { return (r >> 2) & 3; }

}  // namespace

// s_waitcnt vmcnt(after * IPS) for a run-time `after` in [0, M].
template <int IPS, int M>
__device__ __forceinline__ void wait_stages(int after) {
  if constexpr (M >= 0) {
    if (after >= M) {
      wait_vmcnt<M * IPS>();
      return;
    }
    wait_stages<IPS, M - 1>(after);
  }
}

// TM tokens x HP heads per workgroup; each wave computes 32 RB tokens x one
// head (RB row blocks share every W operand read).  K slices of BK per
// stage of an NS-stage LDS ring.
template <int D, bool KV8, int TM, int RB = 1, int HP = 1, bool GROUPED = false, int BK = 32, int NS = 4>
__global__ void __launch_bounds__(64 * (TM / (32 * RB)) * HP) __attribute__((amdgpu_waves_per_eu(2)))
qkv_rope_write_kernel(QKVArgs a) {
  constexpr int TG = TM / (32 * RB);      // token groups (waves per head)
  constexpr int NT = 64 * TG * HP;        // threads
  constexpr int NB = D / 32;              // accumulator blocks per row block (32 x 32 each)
  constexpr int ROWB = BK * 2;            // LDS row: one K slice of a token / W row
  constexpr int CPR = BK / 8;             // 16-byte chunks per LDS row
  static_assert(CPR == 4 || CPR == 8, "K slice of 32 or 64");
  // physical chunk of logical chunk c in row r: 64-byte rows rotate by
  // qkv_swz, 128-byte rows XOR with r & 7 (8 consecutive rows reading one
  // logical chunk hit 8 distinct 4-bank groups)
  auto swz = [](int r) { return CPR == 4 ? qkv_swz(r) : (r & 7); };
  constexpr int A_BYTES = TM * ROWB;      // X slice
  constexpr int B_BYTES = HP * D * ROWB;  // W slice (HP heads of one kind, consecutive W rows)
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int IA = A_BYTES / (NT * 16);           // copy instructions per thread per stage: X
  constexpr int IB = B_BYTES / (NT * 16);           //                                          W
  constexpr int IPS = IA + IB;
  static_assert(IA >= 1 && IB >= 1 && A_BYTES % (NT * 16) == 0 && B_BYTES % (NT * 16) == 0, "tile / workgroup mismatch");
  __shared__ __attribute__((aligned(16))) char lds[NS * STAGE];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t N = a.num_tokens;
  int head, tile;
  if constexpr (GROUPED) {
    // 1-D grid in XCD-grouped order (qkv_groups)
    const int ngroups = (a.num_q_heads + 2 * a.num_kv_heads) / HP;
    const QKVGroups gr = qkv_groups((N + TM - 1) / TM, ngroups, a.cus);
    const int S = gr.gt * gr.gh;
    const int b = blockIdx.x, xcd = b % kXcds, j = b / kXcds;
    const int sg = xcd + kXcds * (j / S), wi = j % S;
    tile = (sg / gr.nhg) * gr.gt + wi / gr.gh;
    head = (sg % gr.nhg) * gr.gh + wi % gr.gh;
    if ((int64_t)tile * TM >= N || head >= ngroups) return;   // padding of the last super-groups
  } else {
    head = blockIdx.y;
    tile = blockIdx.x;
  }
  head *= HP;                             // first head of the workgroup (all HP of one kind)
  const int kind0 = head < a.num_q_heads ? 0 : (head < a.num_q_heads + a.num_kv_heads ? 1 : 2);   // q, k, v
  const int h0 = kind0 == 0 ? head : (kind0 == 1 ? head - a.num_q_heads : head - a.num_q_heads - a.num_kv_heads);
  const char* w = (const char*)(kind0 == 0 ? a.w_q : (kind0 == 1 ? a.w_k : a.w_v));
  const int64_t wstride = kind0 == 0 ? a.w_q_row_stride : (kind0 == 1 ? a.w_k_row_stride : a.w_v_row_stride);
  w += (int64_t)h0 * D * wstride * 2;
  const int64_t tok0 = (int64_t)tile * TM;
  const int kind = kind0, h = h0 + wave / TG;   // this wave's head
  const int tg = wave % TG;                      // this wave's token group
  const int nk = a.hidden / BK;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  // Copy instruction i of this thread: 16-byte chunk c = i * NT + tid of the
  // stage's X (i < IA) or W part; LDS row c / CPR, physical chunk c % CPR,
  // which holds logical chunk (c % CPR) ^ swz(row).
  auto dma = [&](int ks, int stage) {
    const int64_t k0b = (int64_t)ks * BK * 2;
#pragma unroll
    for (int i = 0; i < IPS; ++i) {
      const bool isA = i < IA;
      const int c = (isA ? i : i - IA) * NT + tid;
      const int row = c / CPR, lc = (c % CPR) ^ swz(row);
      const char* src;
      if (isA) {
        const int64_t t = min(tok0 + row, N - 1);     // rows past the batch re-read the last token
        src = (const char*)a.x + t * a.x_row_stride * 2 + k0b + lc * 16;
      } else {
        src = w + (int64_t)row * wstride * 2 + k0b + lc * 16;
      }
      const uint32_t dst = __builtin_amdgcn_readfirstlane(
          lds0 + stage * STAGE + (isA ? 0 : A_BYTES) + ((isA ? i : i - IA) * NT + wave * 64) * 16);
      lds_dma16(src, dst);
    }
  };

  f32x16 acc[RB][NB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[r][b][j] = 0.f;
  const bool wact = tok0 + tg * 32 * RB < N;  // this wave's tokens hold at least one real one
  const int ar = tg * 32 * RB + (lane & 31);  // X row of the A operand (+ 32 r)
  const int bh = (wave / TG) * D;             // first W row of this wave's head in the tile
  const int hi = lane >> 5;

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) dma(s, s);
  for (int ks = 0; ks < nk; ++ks) {
    // this thread's copies of stage ks are done once at most the copies of the
    // (up to NS - 2) later stages already issued are outstanding
    wait_stages<IPS, NS - 2>(min(NS - 2, nk - 1 - ks));
    __syncthreads();                           // stage ks visible; stage ks - 1 free
    if (ks + NS - 1 < nk) dma(ks + NS - 1, (ks + NS - 1) % NS);
    // Every wave multiplies, also one whose rows are all past the batch (it
    // reads the clamped copies of the last row and stores nothing): a branch
    // here makes the compiler move the accumulators between AGPRs and VGPRs
    // on every k-step.
    {
      const char* As = lds + (ks % NS) * STAGE;
      const char* Bs = As + A_BYTES;
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int lc = 2 * kk + hi;
        bf16x8 av[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const int arr = ar + 32 * r;
          av[r] = __builtin_bit_cast(bf16x8, ld16(As + arr * ROWB + ((lc ^ swz(arr)) << 4)));
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int br = bh + 32 * b + (lane & 31);
          const bf16x8 bv = __builtin_bit_cast(bf16x8, ld16(Bs + br * ROWB + ((lc ^ swz(br)) << 4)));
#pragma unroll
          for (int r = 0; r < RB; ++r) acc[r][b] = mfma32(av[r], bv, acc[r][b]);
        }
      }
    }
  }
  if (!wact) return;

  // Epilogue: lane holds C[token 8(j/4) + 4 hi + j%4][dim 32 b + lane % 32].
  // Every per-token load (slot, cos/sin row, query length) and every cos/sin
  // value is issued before the first store (the stores may alias them, so
  // the compiler would otherwise serialise a round trip per token).
  const int n = lane & 31;
  const bool rope = kind == 1 || (kind == 0 && a.rotate_q);
  constexpr int NH = NB / 2;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
  const int64_t tbase = tok0 + tg * 32 * RB + 32 * r + 4 * hi;
  int64_t dst[16];            // store offset per token (elements), -1: not written
  uint32_t csn[16][NH];       // cos (low 16 bits) and sin (high) of the lane's rotation pairs
  {
    // loads first, each kind in its own loop (the conditions are uniform) and
    // with the token index clamped into the batch, so they are in flight together
    int64_t tc[16], crow[16], slot[16];
    int32_t qlen[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      tc[j] = min(tbase + 8 * (j / 4) + (j % 4), N - 1);
      crow[j] = tc[j];
      slot[j] = 0;
      qlen[j] = 0x7fffffff;
    }
    if (rope && a.rope_rows) {
#pragma unroll
      for (int j = 0; j < 16; ++j) crow[j] = a.rope_rows[tc[j]];
    }
    if (kind != 0) {
#pragma unroll
      for (int j = 0; j < 16; ++j) slot[j] = a.slot_mapping[tc[j]];
    }
    if (a.query_lens) {
#pragma unroll
      for (int j = 0; j < 16; ++j) qlen[j] = a.query_lens[tc[j] / a.tokens_per_seq];
      // padded rows read cos/sin row 0 (their own position may lie past the
      // table in mixed batches) and are not written below
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (tc[j] % a.tokens_per_seq >= qlen[j]) crow[j] = 0;
    }
    if (rope) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint16_t* cp = (const uint16_t*)a.cos + crow[j] * a.rope_row_stride + n;
        const uint16_t* sp = (const uint16_t*)a.sin + crow[j] * a.rope_row_stride + n;
#pragma unroll
        for (int b = 0; b < NH; ++b) csn[j][b] = (uint32_t)cp[32 * b] | ((uint32_t)sp[32 * b] << 16);
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t tok = tbase + 8 * (j / 4) + (j % 4);
      int64_t d = -1;
      // padded rows of the reference's [B, T_q] layout are not written (q
      // included); slots outside the pool are never addressed
      const bool real = !a.query_lens || tok % a.tokens_per_seq < qlen[j];
      if (tok < N && real) {
        if (kind == 0) {
          if (a.q_out) d = tok * a.q_out_row_stride + (int64_t)h * D;
        } else {
          if (slot[j] >= 0 && slot[j] < a.num_slots) d = slot[j] * a.cache_slot_stride + (int64_t)h * D;
        }
      }
      dst[j] = d;
    }
  }
  char* base = (char*)(kind == 0 ? a.q_out : (kind == 1 ? a.k_cache : a.v_cache));
  const bool to_cache = kind != 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float v[NB];
#pragma unroll
    for (int b = 0; b < NB; b += 2) {                              // F.linear's bf16 output
      v[b] = acc[r][b][j];
      v[b + 1] = acc[r][b + 1][j];
      round2_bf16(v[b], v[b + 1]);
    }
    if (rope) {
#pragma unroll
      for (int b = 0; b < NH; ++b)
        rope_pair_bf16(v[b], v[b + NH], bf16_bits_to_f32(csn[j][b] & 0xffffu), bf16_bits_to_f32(csn[j][b] >> 16));
    }
    // Lanes n .. n + 3 hold head dims 32b + n .. + 3 of the same token: the
    // quad gathers them (before the row test: every lane of a quad shares the
    // token) and its first lane stores them with one 4-byte (fp8) or 8-byte
    // (bf16) store.
    uint32_t w[NB][2];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (KV8 && to_cache) {
        const uint32_t x = pack_fp8x4(v[b], 0.f, 0.f, 0.f) & 0xffu;
        const uint32_t y = x | (quad_xor1(x) << 8);
        w[b][0] = y | (quad_xor2(y) << 16);
        w[b][1] = 0u;
      } else {
        const uint32_t x = pack_bf16x2(v[b], 0.f) & 0xffffu;
        const uint32_t y = x | (quad_xor1(x) << 16);
        w[b][0] = y;
        w[b][1] = quad_xor2(y);
      }
    }
    if (dst[j] < 0) continue;
    if (a.vec_stores) {                  // rows 4-element aligned (checked on the host)
      if (n & 3) continue;
      if (KV8 && to_cache) {
        char* cp = base + dst[j];
#pragma unroll
        for (int b = 0; b < NB; ++b) *reinterpret_cast<uint32_t*>(cp + 32 * b + n) = w[b][0];
      } else {
        char* cp = base + dst[j] * 2;
#pragma unroll
        for (int b = 0; b < NB; ++b) st8(cp + (32 * b + n) * 2, u32x2{w[b][0], w[b][1]});
      }
    } else if (KV8 && to_cache) {
      char* cp = base + dst[j];
#pragma unroll
      for (int b = 0; b < NB; ++b)
        *reinterpret_cast<uint8_t*>(cp + 32 * b + n) = (uint8_t)(pack_fp8x4(v[b], 0.f, 0.f, 0.f) & 0xffu);
    } else {
      char* cp = base + dst[j] * 2;
#pragma unroll
      for (int b = 0; b < NB; ++b)
        *reinterpret_cast<uint16_t*>(cp + (32 * b + n) * 2) = (uint16_t)pack_bf16x2(v[b], 0.f);
    }
  }
  }
}

// ------------------------------------------------------------------ split-K
// Batches of few tokens (decode) give the tile kernel too few workgroups to
// stream the weights at full bandwidth.  There the K range is split: each
// workgroup computes fp32 partial sums of 64 tokens x one head over one K
// chunk (plain vector stores into the caller's workspace,
// [chunk][token][head * D + d]); qkv_finish_kernel sums the chunks in fixed
// order (deterministic), rounds like F.linear and does the RoPE and the
// stores exactly as the tile kernel's epilogue.
template <int D, int BK, int NS>
__global__ void __launch_bounds__(256) qkv_partial_kernel(QKVArgs a) {
  constexpr int TM = 64;                  // tokens per workgroup (waves: 2 token blocks x 2 output halves)
  constexpr int NBW = D / 64;             // 32 x 32 blocks per wave (D/2 outputs)
  constexpr int ROWB = BK * 2;
  constexpr int CPR = BK / 8;             // 16-byte chunks per LDS row
  constexpr int A_BYTES = TM * ROWB;
  constexpr int B_BYTES = D * ROWB;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int IA = A_BYTES / (256 * 16);
  constexpr int IB = B_BYTES / (256 * 16);
  constexpr int IPS = IA + IB;
  static_assert(IA >= 1 && IB >= 1 && (CPR == 4 || CPR == 8), "tile / workgroup mismatch");
  // physical chunk of logical chunk c in row r: 64-byte rows as the tile
  // kernel; 128-byte rows XOR with r & 7 (8 consecutive rows, one logical
  // chunk: 8 distinct 4-bank groups)
  auto swz = [](int r) { return CPR == 4 ? qkv_swz(r) : (r & 7); };
  __shared__ __attribute__((aligned(16))) char lds[NS * STAGE];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // 1-D grid over token tiles x (chunk, head) groups, in XCD-grouped order
  // when there are several token tiles: the tiles of a group run on one XCD,
  // so its W slice comes from HBM once and its other reads hit that XCD's L2
  const int heads = a.num_q_heads + 2 * a.num_kv_heads;
  const int ngroups = heads * a.split_count;
  const int64_t N = a.num_tokens;
  int tile, gi;
  if (N <= TM) {
    tile = 0;
    gi = blockIdx.x;
  } else {
    const QKVGroups gr = qkv_groups((N + TM - 1) / TM, ngroups, a.cus);
    const int S = gr.gt * gr.gh;
    const int b = blockIdx.x, xcd = b % kXcds, j = b / kXcds;
    const int sg = xcd + kXcds * (j / S), wi = j % S;
    tile = (sg / gr.nhg) * gr.gt + wi / gr.gh;
    gi = (sg % gr.nhg) * gr.gh + wi % gr.gh;
    if ((int64_t)tile * TM >= N || gi >= ngroups) return;   // padding of the last super-groups
  }
  const int head = gi % heads, chunk = gi / heads;
  const int kind = head < a.num_q_heads ? 0 : (head < a.num_q_heads + a.num_kv_heads ? 1 : 2);
  const int h = kind == 0 ? head : (kind == 1 ? head - a.num_q_heads : head - a.num_q_heads - a.num_kv_heads);
  const char* w = (const char*)(kind == 0 ? a.w_q : (kind == 1 ? a.w_k : a.w_v));
  const int64_t wstride = kind == 0 ? a.w_q_row_stride : (kind == 1 ? a.w_k_row_stride : a.w_v_row_stride);
  w += (int64_t)h * D * wstride * 2;
  const int64_t tok0 = (int64_t)tile * TM;
  const int kc0 = chunk * a.split_chunk;
  const int nk = min(a.split_chunk, a.hidden - kc0) / BK;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  auto dma = [&](int ks, int stage) {
    const int64_t k0b = (int64_t)(kc0 + ks * BK) * 2;
#pragma unroll
    for (int i = 0; i < IPS; ++i) {
      const bool isA = i < IA;
      const int c = (isA ? i : i - IA) * 256 + tid;
      const int row = c / CPR, lc = (c % CPR) ^ swz(row);
      const char* src;
      if (isA) {
        const int64_t t = min(tok0 + row, N - 1);
        src = (const char*)a.x + t * a.x_row_stride * 2 + k0b + lc * 16;
      } else {
        src = w + (int64_t)row * wstride * 2 + k0b + lc * 16;
      }
      const uint32_t dst = __builtin_amdgcn_readfirstlane(
          lds0 + stage * STAGE + (isA ? 0 : A_BYTES) + ((isA ? i : i - IA) * 256 + wave * 64) * 16);
      lds_dma16(src, dst);
    }
  };

  f32x16 acc[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[b][j] = 0.f;
  const int tb = wave & 1, fh = wave >> 1;
  const bool wact = tok0 + tb * 32 < N;
  const int ar = tb * 32 + (lane & 31);
  const int hi = lane >> 5;

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) dma(s, s);
  for (int ks = 0; ks < nk; ++ks) {
    wait_stages<IPS, NS - 2>(min(NS - 2, nk - 1 - ks));   // stage ks in; later stages may still fly
    __syncthreads();
    if (ks + NS - 1 < nk) dma(ks + NS - 1, (ks + NS - 1) % NS);
    {   // every wave multiplies (no branch: accumulators stay in place), inactive ones store nothing
      const char* As = lds + (ks % NS) * STAGE;
      const char* Bs = As + A_BYTES;
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        const int lc = 2 * kk + hi;
        const bf16x8 av = __builtin_bit_cast(bf16x8, ld16(As + ar * ROWB + ((lc ^ swz(ar)) << 4)));
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
          const int br = fh * (D / 2) + 32 * b + (lane & 31);
          const bf16x8 bv = __builtin_bit_cast(bf16x8, ld16(Bs + br * ROWB + ((lc ^ swz(br)) << 4)));
          acc[b] = mfma32(av, bv, acc[b]);
        }
      }
    }
  }
  if (!wact) return;
  const int64_t F = (int64_t)(a.num_q_heads + 2 * a.num_kv_heads) * D;
  float* ws = a.workspace + (int64_t)chunk * N * F + (int64_t)head * D + fh * (D / 2) + (lane & 31);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t tok = tok0 + tb * 32 + 8 * (j / 4) + 4 * hi + (j % 4);
    if (tok >= N) continue;
#pragma unroll
    for (int b = 0; b < NBW; ++b) ws[tok * F + 32 * b] = acc[b][j];
  }
}

// Stores pairs (d + i, d + D/2 + i), i < 4, of one (token, head): q to
// q_out, k / v to their cache slot (slots outside the pool are skipped); 4
// dims per store where rows are 4-element aligned (checked on the host).
template <int D, bool KV8>
__device__ __forceinline__ void store_pairs(const QKVArgs& a, int kind, int h, int64_t tok, int d, const float (&x1)[4],
                                            const float (&x2)[4]) {
  constexpr int PPH = D / 2;
  auto put_bf16 = [&](uint16_t* p, const float (&x)[4]) {
    if (a.vec_stores) {
      st8(p, u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])});
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = (uint16_t)pack_bf16x2(x[i], 0.f);
    }
  };
  if (kind == 0) {
    if (!a.q_out) return;
    uint16_t* op = (uint16_t*)a.q_out + tok * a.q_out_row_stride + (int64_t)h * D + d;
    put_bf16(op, x1);
    put_bf16(op + PPH, x2);
    return;
  }
  const int64_t slot = a.slot_mapping[tok];
  if (slot < 0 || slot >= a.num_slots) return;
  char* cp = (char*)(kind == 1 ? a.k_cache : a.v_cache) + (slot * a.cache_slot_stride + (int64_t)h * D + d) * (KV8 ? 1 : 2);
  if (KV8) {
    const uint32_t w1 = pack_fp8x4(x1[0], x1[1], x1[2], x1[3]), w2 = pack_fp8x4(x2[0], x2[1], x2[2], x2[3]);
    if (a.vec_stores) {
      *reinterpret_cast<uint32_t*>(cp) = w1;
      *reinterpret_cast<uint32_t*>(cp + PPH) = w2;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cp[i] = (char)(w1 >> (8 * i));
        cp[PPH + i] = (char)(w2 >> (8 * i));
      }
    }
  } else {
    put_bf16(reinterpret_cast<uint16_t*>(cp), x1);
    put_bf16(reinterpret_cast<uint16_t*>(cp) + PPH, x2);
  }
}

// One thread per 4 rotation pairs (d .. d+3, d+D/2 .. d+D/2+3) of one
// (token, head): 16-byte partial loads, and 4 values per store (8 bytes bf16,
// 4 bytes fp8).
template <int D, bool KV8>
__global__ void __launch_bounds__(64) qkv_finish_kernel(QKVArgs a) {
  constexpr int PPH = D / 2;              // pairs per head
  constexpr int TPH = PPH / 4;            // threads per head
  constexpr int HPB = 64 / TPH;           // heads per (one-wave) workgroup
  const int heads = a.num_q_heads + 2 * a.num_kv_heads;
  const int64_t tok = blockIdx.x;
  const int head = blockIdx.y * HPB + threadIdx.x / TPH;
  const int d = (threadIdx.x % TPH) * 4;
  if (head >= heads) return;
  const int kind = head < a.num_q_heads ? 0 : (head < a.num_q_heads + a.num_kv_heads ? 1 : 2);
  const int h = kind == 0 ? head : (kind == 1 ? head - a.num_q_heads : head - a.num_q_heads - a.num_kv_heads);
  const int64_t F = (int64_t)heads * D;
  const float* ws = a.workspace + tok * F + (int64_t)head * D + d;
  // every chunk's loads in flight at once (the plan makes at most 16 chunks)
  f32x4 p1[16], p2[16];
#pragma unroll
  for (int c = 0; c < 16; ++c)
    if (c < a.split_count) {
      p1[c] = *reinterpret_cast<const f32x4*>(ws + (int64_t)c * a.num_tokens * F);
      p2[c] = *reinterpret_cast<const f32x4*>(ws + (int64_t)c * a.num_tokens * F + PPH);
    }
  f32x4 s1 = {0.f, 0.f, 0.f, 0.f}, s2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 16; ++c)
    if (c < a.split_count) {                    // chunk order fixed: deterministic sums
      s1 += p1[c];
      s2 += p2[c];
    }
  float x1[4], x2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x1[i] = s1[i];
    x2[i] = s2[i];
    round2_bf16(x1[i], x2[i]);
  }
  // padded rows of the [B, T_q] layout: nothing written, cos/sin not read
  if (a.query_lens && tok % a.tokens_per_seq >= a.query_lens[tok / a.tokens_per_seq]) return;
  if (kind == 1 || (kind == 0 && a.rotate_q)) {
    const int64_t crow = a.rope_rows ? a.rope_rows[tok] : tok;
    const uint16_t* cp = (const uint16_t*)a.cos + crow * a.rope_row_stride + d;
    const uint16_t* sp = (const uint16_t*)a.sin + crow * a.rope_row_stride + d;
#pragma unroll
    for (int i = 0; i < 4; ++i) rope_pair_bf16(x1[i], x2[i], bf16_bits_to_f32(cp[i]), bf16_bits_to_f32(sp[i]));
  }
  store_pairs<D, KV8>(a, kind, h, tok, d, x1, x2);
}

// Few tokens (decode): one 8-wave workgroup per (head, 8 CB rotation pairs)
// -- output columns 8 CB c .. 8 CB (c+1) - 1 and the same plus D/2 of one
// head -- over the whole hidden dimension, for up to 16 TB tokens (blockIdx.y:
// the next 16 TB).  Wave w takes K range [w K/8, (w+1) K/8): all of its weight
// operands are loaded at once (one memory round trip; the weights are the
// bytes that matter, MK bounds the k-steps and so the registers), x operands
// (L2-resident) a k-step ahead, on v_mfma_f32_16x16x32_bf16 (A = x rows,
// B = W^T, 16 columns = 8 pairs per block).  The 8 partial sums meet in LDS
// and are added in wave order (deterministic), rounded like F.linear,
// rotated and stored 4 dims at a time.  No partials in HBM, no second launch.
template <int D, bool KV8, int MK, int CB, int TB>
__global__ void __launch_bounds__(512) qkv_small_kernel(QKVArgs a) {
  constexpr int NWV = 8;
  constexpr int NC = 16 * CB;             // output columns per workgroup
  constexpr int TM = 16 * TB;             // tokens per workgroup
  __shared__ __attribute__((aligned(16))) float red[NWV][TM][NC + 1];   // [wave][token][column]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int GPH = D / NC;             // column groups per head
  const int head = blockIdx.x / GPH, cg = blockIdx.x % GPH;
  const int kind = head < a.num_q_heads ? 0 : (head < a.num_q_heads + a.num_kv_heads ? 1 : 2);
  const int h = kind == 0 ? head : (kind == 1 ? head - a.num_q_heads : head - a.num_q_heads - a.num_kv_heads);
  const char* w = (const char*)(kind == 0 ? a.w_q : (kind == 1 ? a.w_k : a.w_v));
  const int64_t wstride = kind == 0 ? a.w_q_row_stride : (kind == 1 ? a.w_k_row_stride : a.w_v_row_stride);
  const int64_t N = a.num_tokens;
  const int64_t tok0 = (int64_t)blockIdx.y * TM;
  const int ntb = (int)min<int64_t>(TB, (N - tok0 + 15) / 16);   // 16-token blocks present
  const int kq = 8 * (lane >> 4);
  const int ksteps = a.hidden / (NWV * 32);
  const int kw0 = wave * ksteps * 32;
  u32x4 wb[CB][MK];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    // lane's B column: pair lane & 7 of the block, first (lane & 8 == 0) or second half of the head
    const int col = (lane & 8 ? D / 2 : 0) + 8 * (CB * cg + cb) + (lane & 7);
    const char* wrow = w + ((int64_t)h * D + col) * wstride * 2 + (int64_t)(kw0 + kq) * 2;
#pragma unroll
    for (int s = 0; s < MK; ++s)
      if (s < ksteps) wb[cb][s] = ld16(wrow + s * 64);
  }
  f32x4 acc[CB][TB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[cb][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const char* xrow[TB];
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    const int64_t tk = min(tok0 + 16 * t + (lane & 15), N - 1);
    xrow[t] = (const char*)a.x + tk * a.x_row_stride * 2 + (int64_t)(kw0 + kq) * 2;
  }
  // x operands PF k-steps ahead (statically indexed: only PF + 1 steps' registers live)
  constexpr int PF = MK <= 8 ? MK : 2;
  u32x4 xa[MK][TB];
#pragma unroll
  for (int s = 0; s < PF; ++s)
#pragma unroll
    for (int t = 0; t < TB; ++t)
      if (s < ksteps && t < ntb) xa[s][t] = ld16(xrow[t] + s * 64);
#pragma unroll
  for (int s = 0; s < MK; ++s) {
    if (s < ksteps) {
      if (s + PF < MK && s + PF < ksteps) {
#pragma unroll
        for (int t = 0; t < TB; ++t)
          if (t < ntb) xa[s + PF][t] = ld16(xrow[t] + (s + PF) * 64);
      }
#pragma unroll
      for (int t = 0; t < TB; ++t)
        if (t < ntb) {
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
            acc[cb][t] = mfma16(__builtin_bit_cast(bf16x8, xa[s][t]), __builtin_bit_cast(bf16x8, wb[cb][s]),
                                acc[cb][t]);
        }
    }
  }
  // lane holds partial D[token 16t + 4(lane >> 4) + j][column 16cb + (lane & 15)]
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][16 * t + 4 * (lane >> 4) + j][16 * cb + (lane & 15)] = acc[cb][t][j];
  __syncthreads();
  // thread: one token, 4 pairs (pairs 4q .. 4q+3 of column block q / 2)
  if (tid >= TM * 2 * CB) return;
  const int tr = tid / (2 * CB), q = tid % (2 * CB);
  const int64_t tok = tok0 + tr;
  if (tok >= N) return;
  const int c1 = 16 * (q >> 1) + 4 * (q & 1);   // red column of the first half's first pair
  float x1[4], x2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int v = 0; v < NWV; ++v) {       // fixed wave order: deterministic sums
      s1 += red[v][tr][c1 + i];
      s2 += red[v][tr][c1 + 8 + i];
    }
    x1[i] = s1;
    x2[i] = s2;
    round2_bf16(x1[i], x2[i]);            // F.linear's bf16 output
  }
  // padded rows of the [B, T_q] layout: nothing written, cos/sin not read
  if (a.query_lens && tok % a.tokens_per_seq >= a.query_lens[tok / a.tokens_per_seq]) return;
  const int d = 8 * (CB * cg + (q >> 1)) + 4 * (q & 1);   // first head dim of the thread's 4 pairs
  if (kind == 1 || (kind == 0 && a.rotate_q)) {
    const int64_t crow = a.rope_rows ? a.rope_rows[tok] : tok;
    const uint16_t* cp = (const uint16_t*)a.cos + crow * a.rope_row_stride + d;
    const uint16_t* sp = (const uint16_t*)a.sin + crow * a.rope_row_stride + d;
#pragma unroll
    for (int i = 0; i < 4; ++i) rope_pair_bf16(x1[i], x2[i], bf16_bits_to_f32(cp[i]), bf16_bits_to_f32(sp[i]));
  }
  store_pairs<D, KV8>(a, kind, h, tok, d, x1, x2);
}

template <int D, bool KV8, int CB>
static void launch_qkv_small(const QKVArgs& b, int heads, hipStream_t st) {
  constexpr int TB = 2;
  const dim3 grid((unsigned)(heads * (D / (16 * CB))), (unsigned)((b.num_tokens + 16 * TB - 1) / (16 * TB))), block(512);
  const int ks = b.hidden / 256;
  if (ks <= 8) hipLaunchKernelGGL((qkv_small_kernel<D, KV8, 8, CB, TB>), grid, block, 0, st, b);
  else hipLaunchKernelGGL((qkv_small_kernel<D, KV8, 16, CB, TB>), grid, block, 0, st, b);
}

constexpr int64_t kQkvSmallMaxTokens = 32;   // beyond: split-K is faster (x re-read per 16 columns)
// Single-launch path for few tokens: column blocks per wave (1 or 2) such
// that the workgroups (one per 16 CB columns) fit on the CUs at once, or 0
// when the batch takes another path.  Up to 16 k-steps per wave (hidden
// <= 4096): beyond that the weight registers of a workgroup take more than
// one memory round trip and the split-K path is faster.
static int qkv_small_cb(int64_t n, int hidden, int heads, int head_dim, int cus) {
  if (n <= 0 || n > kQkvSmallMaxTokens || hidden % 256 != 0 || hidden > 4096 || (head_dim != 64 && head_dim != 128))
    return 0;
  const int64_t cols = (int64_t)heads * head_dim;
  if (cols / 16 <= cus) return 1;
  if (cols / 32 <= cus) return 2;
  return 0;
}

// Split-K partials: K steps of 64 (each X / W row slice is one whole
// 128-byte line, half the memory requests per byte of 32-wide steps) and a
// 2-stage LDS ring (48 KB at D = 128: three workgroups per CU).  Measured
// against 32-wide steps in a 4-stage ring: 8B layer 64 / 256 / 512 tokens
// 23.5 / 44.9 / 61.0 -> 20.9 / 39.9 / 51.2 us; 3 and 4 stages were slower.
constexpr int kQkvPartialBK = 64, kQkvPartialNS = 2;

// Split-K plan for a batch: chunk length (multiple of 32, >= 256) and count,
// or count 1 when the tile kernel already has enough workgroups.
static void qkv_split_plan(int64_t n, int hidden, int heads, int cus, int* chunk, int* count) {
  *chunk = hidden;
  *count = 1;
  const int64_t tiles = (n + 127) / 128;
  if (n == 0 || tiles * heads >= cus || hidden < 512) return;
  const int64_t wgs64 = ((n + 63) / 64) * heads;
  int64_t want = (2 * (int64_t)cus + wgs64 - 1) / wgs64;           // about two workgroups per CU
  want = std::min<int64_t>(std::min<int64_t>(want, hidden / 256), 16);   // the finish kernel sums <= 16 chunks
  if (want <= 1) return;
  const int g = hidden % kQkvPartialBK == 0 ? kQkvPartialBK : 32;   // chunks in whole k-steps of the partial kernel
  const int c = (int)(((hidden + want - 1) / want + g - 1) / g * g);
  *chunk = c;
  *count = (hidden + c - 1) / c;
}

size_t qkv_workspace_bytes(int64_t n, int hidden, int heads, int head_dim, int cus) {
  if (qkv_small_cb(n, hidden, heads, head_dim, cus)) return 0;
  int chunk, count;
  qkv_split_plan(n, hidden, heads, cus, &chunk, &count);
  return count > 1 ? (size_t)count * n * heads * head_dim * sizeof(float) : 0;
}

// Tile kernels take K slices of 64 in a 2-stage ring when hidden allows:
// whole 128-byte lines per row slice (half the memory requests per byte of
// 32-wide slices).  Measured against 32-wide slices in a 4-stage ring:
// 1B layer 1,024 / 4,096 tokens 41.5 / 109.3 -> 33.4 / 90.6 us, 8B
// 1,024 / 4,096 / 19,679 tokens 90.4 / 274 / 1,247 -> 82.2 / 246 / 1,223 us;
// 3 stages (one workgroup per CU) were slower.
constexpr bool kTileBK64 = true, kTileBig64 = true;
constexpr int kTileNS = 2;

hipError_t launch_qkv_rope_write(const QKVArgs& a, hipStream_t st) {
  if (a.num_tokens == 0) return hipSuccess;
  const int64_t tiles = (a.num_tokens + 127) / 128;
  const int heads = (a.q_out ? a.num_q_heads : 0) + 2 * a.num_kv_heads;
  if (tiles > 0x7fffffff || heads > 65535) return hipErrorInvalidValue;
  // q heads are the first grid rows; without q_out the grid starts at the k heads
  QKVArgs b = a;
  if (!a.q_out) b.num_q_heads = 0;
  // 4 consecutive head dims per store: every row start 8-byte aligned (bf16:
  // element offsets multiple of 4; fp8 cache: 4 bytes)
  const auto al8 = [](const void* p) { return ((uintptr_t)p & 7) == 0; };
  b.vec_stores = al8(a.k_cache) && al8(a.v_cache) && a.cache_slot_stride % 4 == 0 &&
                 (!a.q_out || (al8(a.q_out) && a.q_out_row_stride % 4 == 0));
  const bool kv8 = a.kv_dtype == kFP8;
  // few tokens: one launch, whole K per workgroup
  if (const int cb = qkv_small_cb(a.num_tokens, a.hidden, heads, a.head_dim, a.cus)) {
    if (a.head_dim == 64) {
      if (cb == 1) kv8 ? launch_qkv_small<64, true, 1>(b, heads, st) : launch_qkv_small<64, false, 1>(b, heads, st);
      else kv8 ? launch_qkv_small<64, true, 2>(b, heads, st) : launch_qkv_small<64, false, 2>(b, heads, st);
    } else {
      if (cb == 1) kv8 ? launch_qkv_small<128, true, 1>(b, heads, st) : launch_qkv_small<128, false, 1>(b, heads, st);
      else kv8 ? launch_qkv_small<128, true, 2>(b, heads, st) : launch_qkv_small<128, false, 2>(b, heads, st);
    }
    return hipGetLastError();
  }
  int chunk, count;
  qkv_split_plan(a.num_tokens, a.hidden, heads, a.cus, &chunk, &count);
  if (count > 1 && a.workspace &&
      a.workspace_bytes >= (size_t)count * a.num_tokens * heads * a.head_dim * sizeof(float)) {
    b.split_chunk = chunk;
    b.split_count = count;
    const QKVGroups gr1 = qkv_groups((a.num_tokens + 63) / 64, heads * count, a.cus);
    const int64_t wgs1 = a.num_tokens <= 64 ? (int64_t)heads * count
                                            : (int64_t)kXcds * gr1.gt * gr1.gh * ((gr1.nsg + kXcds - 1) / kXcds);
    if (wgs1 > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g1((unsigned)wgs1), blk(256);
    const int hpb = 64 / (a.head_dim / 8);    // heads per finish workgroup (one wave)
    const dim3 g2((unsigned)a.num_tokens, (unsigned)((heads + hpb - 1) / hpb)), blk2(64);
    const bool bk64 = kQkvPartialBK == 64 && a.hidden % 64 == 0;
    if (a.head_dim == 64) {
      if (bk64) hipLaunchKernelGGL((qkv_partial_kernel<64, 64, kQkvPartialNS>), g1, blk, 0, st, b);
      else hipLaunchKernelGGL((qkv_partial_kernel<64, 32, 4>), g1, blk, 0, st, b);
      if (kv8) hipLaunchKernelGGL((qkv_finish_kernel<64, true>), g2, blk2, 0, st, b);
      else hipLaunchKernelGGL((qkv_finish_kernel<64, false>), g2, blk2, 0, st, b);
    } else if (a.head_dim == 128) {
      if (bk64) hipLaunchKernelGGL((qkv_partial_kernel<128, 64, kQkvPartialNS>), g1, blk, 0, st, b);
      else hipLaunchKernelGGL((qkv_partial_kernel<128, 32, 4>), g1, blk, 0, st, b);
      if (kv8) hipLaunchKernelGGL((qkv_finish_kernel<128, true>), g2, blk2, 0, st, b);
      else hipLaunchKernelGGL((qkv_finish_kernel<128, false>), g2, blk2, 0, st, b);
    } else {
      return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  // 128-token tiles, one head each, in XCD-grouped order (a head's token
  // tiles share its W slice through one XCD's L2)
  const QKVGroups gr = qkv_groups(tiles, heads, a.cus);
  const int64_t wgs = (int64_t)kXcds * gr.gt * gr.gh * ((gr.nsg + kXcds - 1) / kXcds);
  if (wgs > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)wgs), block(256);
  const bool bk64 = kTileBK64 && a.hidden % 64 == 0;
  if (a.head_dim == 64) {
    if (bk64) {
      if (kv8) hipLaunchKernelGGL((qkv_rope_write_kernel<64, true, 128, 1, 1, true, 64, kTileNS>), grid, block, 0, st, b);
      else hipLaunchKernelGGL((qkv_rope_write_kernel<64, false, 128, 1, 1, true, 64, kTileNS>), grid, block, 0, st, b);
    } else {
      if (kv8) hipLaunchKernelGGL((qkv_rope_write_kernel<64, true, 128, 1, 1, true>), grid, block, 0, st, b);
      else hipLaunchKernelGGL((qkv_rope_write_kernel<64, false, 128, 1, 1, true>), grid, block, 0, st, b);
    }
  } else if (a.head_dim == 128) {
    // Large batches: 256 tokens x 2 heads per 8-wave workgroup (each wave 64
    // tokens x one head: two row blocks share every W operand read), in
    // XCD-grouped order; they need heads that pair within q and within k/v.
    const int64_t tiles2 = (a.num_tokens + 255) / 256;
    if (b.num_q_heads % 2 == 0 && a.num_kv_heads % 2 == 0 && tiles2 * (heads / 2) >= 2 * (int64_t)a.cus) {
      const QKVGroups gr2 = qkv_groups(tiles2, heads / 2, a.cus);
      const int64_t wgs2 = (int64_t)kXcds * gr2.gt * gr2.gh * ((gr2.nsg + kXcds - 1) / kXcds);
      if (wgs2 > 0x7fffffff) return hipErrorInvalidValue;
      const dim3 grid2((unsigned)wgs2), block2(512);
      if (bk64 && kTileBig64) {
        if (kv8) hipLaunchKernelGGL((qkv_rope_write_kernel<128, true, 256, 2, 2, true, 64, 2>), grid2, block2, 0, st, b);
        else hipLaunchKernelGGL((qkv_rope_write_kernel<128, false, 256, 2, 2, true, 64, 2>), grid2, block2, 0, st, b);
      } else {
        if (kv8) hipLaunchKernelGGL((qkv_rope_write_kernel<128, true, 256, 2, 2, true>), grid2, block2, 0, st, b);
        else hipLaunchKernelGGL((qkv_rope_write_kernel<128, false, 256, 2, 2, true>), grid2, block2, 0, st, b);
      }
      return hipGetLastError();
    }
    if (bk64) {
      if (kv8) hipLaunchKernelGGL((qkv_rope_write_kernel<128, true, 128, 1, 1, true, 64, kTileNS>), grid, block, 0, st, b);
      else hipLaunchKernelGGL((qkv_rope_write_kernel<128, false, 128, 1, 1, true, 64, kTileNS>), grid, block, 0, st, b);
    } else {
      if (kv8) hipLaunchKernelGGL((qkv_rope_write_kernel<128, true, 128, 1, 1, true>), grid, block, 0, st, b);
      else hipLaunchKernelGGL((qkv_rope_write_kernel<128, false, 128, 1, 1, true>), grid, block, 0, st, b);
    }
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace gllm

// C ABI of libgllm_attn: argument validation, the host work planner and the
// kernel launches.  Declarations and contracts: include/gllm_attn.h.
#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include <rocprofiler-sdk-roctx/roctx.h>

#include "../../include/gllm_attn.h"
#include "launch.h"

using namespace gllm;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return GLLM_ATTN_OK;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(GLLM_ATTN_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// roctx range around each launching entry point (shows in rocprofv3
// --marker-trace and other ROCm tracers; no cost beyond a call when no tool
// is attached).
struct Range {
  explicit Range(const char* name) { roctxRangePushA(name); }
  ~Range() { roctxRangePop(); }
  Range(const Range&) = delete;
  Range& operator=(const Range&) = delete;
};

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int log2i(int64_t x) {
  int s = 0;
  while ((int64_t(1) << s) < x) ++s;
  return s;
}
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Constants of the device division by the block size (div_bs in common.h):
// k = ceil(log2 bs), magic = ceil(2^(31+k) / bs) (< 2^32 for every bs >= 1).
void block_div(int32_t bs, uint32_t* magic, int32_t* shift) {
  const int k = log2i(bs);
  *magic = (uint32_t)(((uint64_t(1) << (31 + k)) + (uint64_t)bs - 1) / (uint64_t)bs);
  *shift = k;
}
constexpr int32_t kMaxBlockSize = 65536;
// query rows per sequence up to which the generic kernel takes the fused KV
// write (each workgroup stages the new keys it reads in LDS)
constexpr int32_t kMaxFusedRows = 16;

// Model dtypes (the reference's model_dtype, model.py:64): f32, bf16, f16;
// cache dtypes (kv_dtype, model.py:75): those and fp8 e4m3fn, any pairing.
bool model_dtype_ok(int32_t d) { return d == GLLM_DTYPE_F32 || d == GLLM_DTYPE_BF16 || d == GLLM_DTYPE_F16; }
bool kv_dtype_ok(int32_t d) { return model_dtype_ok(d) || d == GLLM_DTYPE_FP8_E4M3; }
// 16-bit model dtypes run the MFMA kernels (head dim 64 / 128)
bool mfma_dtype(int32_t d) { return d == GLLM_DTYPE_BF16 || d == GLLM_DTYPE_F16; }

// CUs of the current device (256 when there is none, e.g. a CPU-only host),
// queried once per device: plans and projection calls ask on every engine step.
int device_cus() {
  constexpr int kDevs = 64;
  static std::atomic<int> known[kDevs] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < kDevs) {
    const int c = known[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < kDevs) known[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Pinned staging buffers of plans, reused across plans (an engine builds one
// plan per step): plan_create takes the smallest free buffer that fits and
// plan_destroy hands it back, together with the event of its upload copy; a
// buffer whose copy has not finished yet is only reused once that event has
// completed (checked without blocking).  No hipHostMalloc / hipHostFree on the
// steady-state path; the pool keeps at most kPoolKeep bytes.
struct PinnedPool {
  struct Buf { void* p; size_t n; hipEvent_t done; };
  std::mutex mu;
  std::vector<Buf> free_bufs;   // done == nullptr or completed
  size_t kept = 0;
  static constexpr size_t kPoolKeep = size_t(64) << 20;

  static bool ready(const Buf& b) {
    if (!b.done) return true;
    const hipError_t e = hipEventQuery(b.done);
    if (e == hipErrorNotReady) return false;
    (void)hipGetLastError();
    return true;
  }
  // A pinned buffer of at least n bytes (rounded up to a power of two >= 64 KB).
  void* acquire(size_t n, size_t* cap) {
    {
      std::lock_guard<std::mutex> lk(mu);
      size_t best = free_bufs.size();
      for (size_t i = 0; i < free_bufs.size(); ++i)
        if (free_bufs[i].n >= n && (best == free_bufs.size() || free_bufs[i].n < free_bufs[best].n) &&
            ready(free_bufs[i]))
          best = i;
      if (best < free_bufs.size()) {
        Buf b = free_bufs[best];
        free_bufs.erase(free_bufs.begin() + best);
        kept -= b.n;
        if (b.done) (void)hipEventDestroy(b.done);
        *cap = b.n;
        return b.p;
      }
    }
    size_t c = size_t(64) << 10;
    while (c < n) c <<= 1;
    void* p = nullptr;
    if (hipHostMalloc(&p, c, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    *cap = c;
    return p;
  }
  // Takes ownership of `done` (may be null).
  void release(void* p, size_t n, hipEvent_t done) {
    std::lock_guard<std::mutex> lk(mu);
    if (kept + n > kPoolKeep) {
      if (done) {
        (void)hipEventSynchronize(done);   // the copy must finish before the free
        (void)hipEventDestroy(done);
      }
      (void)hipHostFree(p);
      return;
    }
    free_bufs.push_back(Buf{p, n, done});
    kept += n;
  }
};
PinnedPool& pinned_pool() {
  static PinnedPool* pool = new PinnedPool();   // never destroyed: buffers live until the process ends
  return *pool;
}

}  // namespace

struct gllm_attn_plan {
  int32_t num_seqs = 0, Hq = 0, Hkv = 0, D = 0, bs = 0, dtype = 0;
  int32_t split_len = 0, max_q = 0;
  int32_t n_decode_seqs = 0, n_prefill_seqs = 0, heads_per_wg = 8, decode_waves = 8, prefill_waves = 8;
  bool mfma = false;      // bf16 head dim 64 / 128: the MFMA kernels; otherwise the generic kernel
  int64_t total_rows = 0;
  int64_t n_partials = 0;
  std::vector<SeqInfo> seqs;
  std::vector<WorkItem> items;
  // page-balanced decode: workgroup w runs segs[seg_ptr[w] .. seg_ptr[w + 1])
  std::vector<DecodeSeg> segs;
  std::vector<int32_t> seg_ptr;
  // staging copy of [items | seqs] in pinned host memory (from the pool), device offsets
  void* pinned = nullptr;
  size_t pinned_cap = 0;
  bool pinned_is_host_malloc = false;  // hipHostMalloc unavailable (no device): plain malloc
  size_t off_items = 0, off_seqs = 0, off_segs = 0, off_segptr = 0, off_ctr = 0, off_ml = 0, off_part = 0, ws_bytes = 0;
  char* ws = nullptr;
  hipEvent_t upload_done = nullptr;
};

namespace {

// Resident 8-wave decode workgroups per CU (register-bound: 2 at D = 64,
// 1 at D = 128).
#ifndef GLLM_DECODE_WG_PER_CU
#define GLLM_DECODE_WG_PER_CU(D) ((D) == 64 ? 2 : 1)
#endif

// Page-balanced decode plan (decode-only batches): the batch's keys, in
// 16-key units per (sequence, kv-head group), are dealt out as equal
// contiguous ranges to one workgroup per resident slot, so every
// CU streams the same number of bytes whatever the spread of sequence
// lengths.  A workgroup's range becomes one segment per (sequence, group) it
// touches (cut further so a segment caches at most 511 block ids).  A
// (sequence, group) with several segments writes partials; the workgroup
// drawing its last ticket merges them in the same launch.  HW: the largest
// of 8, 4, 2, 1 that divides Hkv, so the 8 waves read all HW heads of a slot
// (HW x D x 2 contiguous bytes) together.
// Units (16 keys x one kv-head group) and workgroups of a page-balanced plan.
struct BalancedShape {
  int hw, hgroups;
  int64_t units, wgs;
};
// Decode-path sequences (q_len x G <= 16 query rows) only: in a mixed batch
// the others are prefill items.
BalancedShape balanced_shape(const gllm_attn_plan* p, int cus, int heads_req) {
  BalancedShape b{};
  b.hw = heads_req;
  if (!b.hw) {
    b.hw = 8;
    while (b.hw > 1 && p->Hkv % b.hw) b.hw /= 2;
  }
  b.hgroups = (p->Hkv + b.hw - 1) / b.hw;
  const int G = p->Hq / p->Hkv;
  for (const SeqInfo& si : p->seqs)
    if (si.q_len * G <= 16) b.units += (int64_t)b.hgroups * ((si.ctx_len + si.q_len + 15) / 16);
  b.wgs = std::max<int64_t>(1, std::min<int64_t>(b.units, (int64_t)cus * GLLM_DECODE_WG_PER_CU(p->D)));
  return b;
}

// Page-balanced plans pay a partial write, an L2 write-back (agent-scope
// release) and a ticket per segment, and the merges of the last segments
// sit on the launch's tail: measured on MI355X this wins when a workgroup
// streams enough keys and loses to the split planner below that.  D=64:
// from ~2048 keys (128 units) per workgroup.  D=128 (Hkv 8, one workgroup per
// CU): the split planner is 3-3.5% faster at 128-137 units per workgroup, the
// two are within 1% from 248 to 514, and page-balanced is 0.6-5% faster at
// 740-770; the cut sits between the measured points.
int64_t balanced_min_units_per_wg(int D) { return D == 128 ? 192 : 128; }

// wgs > 0: that many workgroups (a mixed launch's decode share), else one
// per resident decode slot.
void plan_balanced_decode(gllm_attn_plan* p, int cus, int heads_req, int64_t wgs) {
  const BalancedShape shape = balanced_shape(p, cus, heads_req);
  const int hw = shape.hw, hgroups = shape.hgroups;
  const int64_t bs = p->bs;
  const int G = p->Hq / p->Hkv;
  // a segment's keys start on a 16-key unit, so a block size that is not a
  // power of two <= 16 can add one partial block at the front: stay <= 511
  const int64_t ucap = std::max<int64_t>(1, (is_pow2(bs) && bs <= 16 ? 512 * bs : 510 * bs) / 16);
  const int64_t U = shape.units;
  const int64_t W = wgs > 0 ? std::max<int64_t>(1, std::min(wgs, U)) : shape.wgs;
  p->heads_per_wg = hw;
  p->decode_waves = 8;
  p->split_len = 0;
  p->n_decode_seqs = 0;
  p->segs.clear();
  p->seg_ptr.assign((size_t)W + 1, 0);
  std::vector<int32_t> seg_wg;
  int64_t u0 = 0, j = 0;
  for (int i = 0; i < p->num_seqs; ++i) {
    SeqInfo& si = p->seqs[i];
    if (si.q_len * G > 16) continue;   // a prefill item of the mixed launch
    ++p->n_decode_seqs;
    si.nsplits = 1;
    const int L = si.ctx_len + si.q_len;
    const int64_t nu = (L + 15) / 16;
    for (int hg = 0; hg < hgroups; ++hg) {
      const size_t first = p->segs.size();
      for (int64_t u = 0; u < nu;) {
        while (U * (j + 1) / W <= u0 + u) ++j;        // workgroup owning unit u0 + u
        const int64_t take = std::min(std::min(nu - u, U * (j + 1) / W - (u0 + u)), ucap);
        DecodeSeg sg{};
        sg.seq = i; sg.hg = hg;
        sg.k0 = (int32_t)(16 * u);
        sg.k1 = (int32_t)std::min<int64_t>(L, 16 * (u + take));
        sg.q_row_start = si.q_row_start; sg.ctx_len = si.ctx_len; sg.q_len = si.q_len;
        sg.ticket = i * hgroups + hg;
        p->segs.push_back(sg);
        seg_wg.push_back((int32_t)j);
        u += take;
      }
      u0 += nu;
      const int nseg = (int)(p->segs.size() - first);
      const int32_t pbase = (int32_t)p->n_partials;
      if (nseg > 1) p->n_partials += (int64_t)hw * nseg;
      for (int k = 0; k < nseg; ++k) {
        DecodeSeg& sg = p->segs[first + k];
        sg.nseg = nseg; sg.ord = k; sg.pbase = nseg > 1 ? pbase : 0;
      }
    }
  }
  for (int32_t w : seg_wg) ++p->seg_ptr[(size_t)w + 1];
  for (int64_t w = 0; w < W; ++w) p->seg_ptr[(size_t)w + 1] += p->seg_ptr[(size_t)w];
}

// A prefill work item: 8 waves over the (query head, 32-row block) pairs
// c = w*8 .. w*8+7 of one kv head (row block c / G, head c % G), with its
// last visible key + 1 and its (query row, visible key) pairs.
struct PrefillPiece {
  WorkItem it;
  int64_t kend;
  int64_t pairs;
};
void prefill_pieces(const SeqInfo& s, int i, int G, int Hkv, std::vector<PrefillPiece>& out, int pw = 8) {
  const int nrb = (s.q_len + 31) / 32;
  const int nwg = (G * nrb + pw - 1) / pw;
  for (int h = 0; h < Hkv; ++h)
    for (int w = 0; w < nwg; ++w) {
      const int c0 = w * pw, c1 = std::min(w * pw + pw - 1, G * nrb - 1);
      const int64_t kend = s.ctx_len + std::min(s.q_len - 1, (c1 / G) * 32 + 31) + 1;
      int64_t pairs = 0;
      for (int c = c0; c <= c1; ++c) {
        const int64_t r0 = (int64_t)(c / G) * 32, r1 = std::min<int64_t>(s.q_len, r0 + 32);
        pairs += (r1 - r0) * (s.ctx_len + 1) + (r0 + r1 - 1) * (r1 - r0) / 2;   // row r sees ctx + r + 1 keys
      }
      out.push_back({WorkItem{kItemPrefill | (w << 8), i, h, s.q_row_start, s.ctx_len, s.q_len, 0, 0}, kend, pairs});
    }
}

// Mixed launch, page-balanced: workgroups [0, kd) stream equal key shares of
// the decode sequences while the other CUs run the prefill items one after
// another.  kd balances the two with a cost model fitted to per-workgroup
// timestamps of config (d) and decode-only launches on MI355X (one 8-wave
// workgroup per CU): k decode workgroups together stream 5.7 (1 - e^(-k / 57))
// TB/s of a bf16 cache (measured 3.7, 5.3, 5.6 TB/s at k = 64, 128, 256); a
// prefill item computes 4 D flops per (row, key) pair at ~4.2 TFLOP/s per CU
// at D = 128 (3.0 assumed at D = 64), and the prefill CUs end up to half the
// longest item apart.  kd is a multiple of 8 (the same on every XCD) and
// leaves CUs on every XCD for prefill.
int64_t mixed_decode_wgs(const gllm_attn_plan* p, int cus, int heads_req, const std::vector<PrefillPiece>& pcs) {
  const BalancedShape sh = balanced_shape(p, cus, heads_req);
  if (sh.units == 0) return 1;
  const double dec_bytes = (double)sh.units * 16 * sh.hw * p->D * 2 * 2;
  const double rate = p->D == 128 ? 4.2e12 : 3.0e12;
  double pf_total = 0, pf_max = 0;
  for (const PrefillPiece& pc : pcs) {
    const double t = 4.0 * p->D * (double)pc.pairs / rate;
    pf_total += t;
    pf_max = std::max(pf_max, t);
  }
  const int step = cus >= 16 && cus % 8 == 0 ? 8 : 1;
  int64_t best = 0;
  double best_t = 0;
  for (int64_t kd = step; kd <= cus - step; kd += step) {
    const double td = dec_bytes / (5.7e12 * (1.0 - std::exp(-(double)kd / 57.0)));
    const double tp = pf_total / (double)(cus - kd) + 0.5 * pf_max;
    const double t = std::max(td, tp);
    if (best == 0 || t < best_t) {
      best = kd;
      best_t = t;
    }
  }
  return std::min<int64_t>(std::max<int64_t>(best, 1), sh.units);
}

// Prefill items of a mixed page-balanced launch; they follow its kd decode
// workgroups, so with kd a multiple of 8 item j runs on XCD j % 8.  The
// items of one (sequence, kv head) read the same K/V tiles: they go to one
// XCD, next to each other, so they run together and read each tile from that
// XCD's L2 instead of HBM.  Bundles, largest first, go to the XCD with the
// least prefill work so far; each XCD runs its bundles in that order, a
// bundle's items largest first.
void plan_mixed_prefill(gllm_attn_plan* p, const std::vector<PrefillPiece>& pcs) {
  constexpr int NX = 8;
  struct Bundle { int64_t work; std::vector<const PrefillPiece*> items; };
  std::vector<Bundle> bundles;
  for (size_t i = 0; i < pcs.size();) {   // pieces come grouped by (sequence, kv head)
    Bundle bu{0, {}};
    size_t j = i;
    for (; j < pcs.size() && pcs[j].it.seq == pcs[i].it.seq && pcs[j].it.a == pcs[i].it.a; ++j) {
      bu.work += pcs[j].pairs;
      bu.items.push_back(&pcs[j]);
    }
    std::stable_sort(bu.items.begin(), bu.items.end(),
                     [](const PrefillPiece* x, const PrefillPiece* y) { return x->pairs > y->pairs; });
    bundles.push_back(std::move(bu));
    i = j;
  }
  std::stable_sort(bundles.begin(), bundles.end(), [](const Bundle& x, const Bundle& y) { return x.work > y.work; });
  std::vector<std::vector<const PrefillPiece*>> q(NX);
  std::vector<int64_t> load(NX, 0);
  for (const Bundle& bu : bundles) {
    int x = 0;
    for (int y = 1; y < NX; ++y)
      if (load[y] < load[x]) x = y;
    q[x].insert(q[x].end(), bu.items.begin(), bu.items.end());
    load[x] += bu.work;
  }
  p->items.clear();
  p->items.reserve(pcs.size());
  for (size_t k = 0; p->items.size() < pcs.size(); ++k)
    for (int x = 0; x < NX; ++x)
      if (k < q[x].size()) p->items.push_back(q[x][k]->it);
  p->prefill_waves = 8;
}

}  // namespace

extern "C" {

const char* gllm_attn_last_error(void) { return g_last_error.c_str(); }
int gllm_attn_version(void) { return 1; }

int gllm_build_metadata(const int32_t* block_table, int64_t block_table_stride, int64_t block_table_width,
                        const int32_t* seq_lens, const int32_t* query_lens, int32_t num_seqs,
                        int64_t q_seq_stride, int32_t block_size, int64_t* slot_mapping, int64_t* positions,
                        int32_t* cu_seqlens, int64_t num_rows, void* stream) {
  Range range("gllm_build_metadata");
  if (num_seqs < 0 || num_rows < 0) return fail(GLLM_ATTN_EINVAL, "num_seqs / num_rows < 0");
  if (num_seqs == 0) return ok();
  if (!block_table || !seq_lens || !query_lens) return fail(GLLM_ATTN_EINVAL, "null block_table or lengths");
  if (!slot_mapping && !positions && !cu_seqlens) return fail(GLLM_ATTN_EINVAL, "nothing to do: no output given");
  if (block_size <= 0 || block_size > kMaxBlockSize)
    return fail(GLLM_ATTN_EINVAL, "block_size %d must be in [1, %d]", block_size, kMaxBlockSize);
  if (block_table_width <= 0 || block_table_stride < block_table_width)
    return fail(GLLM_ATTN_EINVAL, "block_table width %lld / stride %lld invalid", (long long)block_table_width,
                (long long)block_table_stride);
  if (q_seq_stride < 0) return fail(GLLM_ATTN_EINVAL, "q_seq_stride < 0");
  if (q_seq_stride > 0 && num_rows < (int64_t)num_seqs * q_seq_stride)
    return fail(GLLM_ATTN_EINVAL, "num_rows %lld < num_seqs * q_seq_stride", (long long)num_rows);
  if (cu_seqlens && q_seq_stride > 0) return fail(GLLM_ATTN_EINVAL, "cu_seqlens is for the packed layout");
  MetadataArgs a{};
  a.block_table = block_table; a.block_table_stride = block_table_stride; a.bt_width = block_table_width;
  a.seq_lens = seq_lens; a.query_lens = query_lens; a.num_seqs = num_seqs; a.q_seq_stride = q_seq_stride;
  a.block_size = block_size;
  block_div(block_size, &a.block_magic, &a.block_shift);
  a.slot_mapping = slot_mapping; a.positions = positions; a.cu_seqlens = cu_seqlens; a.num_rows = num_rows;
  return hip_check(launch_build_metadata(a, (hipStream_t)stream), "build_metadata launch");
}

int gllm_rope_kv_write(const void* q, void* q_out, const void* k, const void* v, void* k_cache,
                       void* v_cache, const int64_t* slot_mapping, const int32_t* query_lens,
                       int64_t tokens_per_seq, const void* cos, const void* sin,
                       const int64_t* rope_rows, int64_t rope_row_stride, int64_t num_tokens,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                       int64_t q_out_row_stride, int64_t cache_slot_stride, int64_t num_slots,
                       int32_t dtype, int32_t kv_dtype, void* stream) {
  Range range("gllm_rope_kv_write");
  if (num_tokens < 0) return fail(GLLM_ATTN_EINVAL, "num_tokens < 0");
  const bool kv = k || v;
  if (!cos || !sin) return fail(GLLM_ATTN_EINVAL, "null cos/sin");
  if (kv && (!k || !v || !k_cache || !v_cache || !slot_mapping))
    return fail(GLLM_ATTN_EINVAL, "k, v, k_cache, v_cache and slot_mapping go together");
  if (!kv && !q_out) return fail(GLLM_ATTN_EINVAL, "nothing to do: neither k/v nor q_out given");
  if (q_out && !q) return fail(GLLM_ATTN_EINVAL, "q_out given without q");
  if (num_kv_heads <= 0 || num_q_heads <= 0) return fail(GLLM_ATTN_EINVAL, "head counts must be > 0");
  if (!model_dtype_ok(dtype)) return fail(GLLM_ATTN_EUNSUPPORTED, "model dtype %d (f32, bf16 or f16)", dtype);
  if (kv && !kv_dtype_ok(kv_dtype)) return fail(GLLM_ATTN_EUNSUPPORTED, "kv_dtype %d (f32, bf16, f16 or fp8 e4m3fn)", kv_dtype);
  const int vec = dtype == GLLM_DTYPE_F32 ? 4 : 8;
  if (head_dim <= 0 || head_dim % (2 * vec) != 0)
    return fail(GLLM_ATTN_EUNSUPPORTED, "head_dim %d must be a positive multiple of %d", head_dim, 2 * vec);
  if (kv && (k_row_stride < (int64_t)num_kv_heads * head_dim || v_row_stride < (int64_t)num_kv_heads * head_dim))
    return fail(GLLM_ATTN_EINVAL, "k/v row stride smaller than num_kv_heads * head_dim");
  if (q_out && (q_row_stride < (int64_t)num_q_heads * head_dim || q_out_row_stride < (int64_t)num_q_heads * head_dim))
    return fail(GLLM_ATTN_EINVAL, "q row stride smaller than num_q_heads * head_dim");
  if (kv && cache_slot_stride < (int64_t)num_kv_heads * head_dim) return fail(GLLM_ATTN_EINVAL, "cache_slot_stride too small");
  if (rope_row_stride < head_dim / 2) return fail(GLLM_ATTN_EINVAL, "rope_row_stride < head_dim / 2");
  if (query_lens && tokens_per_seq <= 0) return fail(GLLM_ATTN_EINVAL, "tokens_per_seq must be > 0 with query_lens");
  if (kv && num_slots <= 0) return fail(GLLM_ATTN_EINVAL, "num_slots must be > 0");
  RopeKVWriteArgs a{};
  a.q = q; a.q_out = q_out; a.k = k; a.v = v; a.k_cache = k_cache; a.v_cache = v_cache;
  a.slot_mapping = slot_mapping; a.query_lens = query_lens; a.tokens_per_seq = tokens_per_seq;
  a.cos = cos; a.sin = sin; a.rope_rows = rope_rows; a.rope_row_stride = rope_row_stride;
  a.num_tokens = num_tokens; a.num_q_heads = num_q_heads; a.num_kv_heads = num_kv_heads; a.head_dim = head_dim;
  a.q_row_stride = q_row_stride; a.k_row_stride = k_row_stride; a.v_row_stride = v_row_stride;
  a.q_out_row_stride = q_out_row_stride; a.cache_slot_stride = cache_slot_stride; a.num_slots = num_slots;
  a.dtype = dtype; a.kv_dtype = kv_dtype;
  return hip_check(launch_rope_kv_write(a, (hipStream_t)stream), "rope_kv_write launch");
}

int gllm_qkv_rope_kv_write(const void* x, int64_t x_row_stride, int64_t num_tokens, int32_t hidden,
                           const void* w_q, int64_t w_q_row_stride, const void* w_k, int64_t w_k_row_stride,
                           const void* w_v, int64_t w_v_row_stride, void* q_out, int64_t q_out_row_stride,
                           int32_t rotate_q, void* k_cache, void* v_cache, int64_t cache_slot_stride,
                           int64_t num_slots, const int64_t* slot_mapping, const int32_t* query_lens,
                           int64_t tokens_per_seq, const void* cos, const void* sin, const int64_t* rope_rows,
                           int64_t rope_row_stride, int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t dtype, int32_t kv_dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
  Range range("gllm_qkv_rope_kv_write");
  if (num_tokens < 0) return fail(GLLM_ATTN_EINVAL, "num_tokens < 0");
  if (dtype != GLLM_DTYPE_BF16) return fail(GLLM_ATTN_EUNSUPPORTED, "fused QKV projection needs a bf16 model (dtype %d)", dtype);
  if (kv_dtype != GLLM_DTYPE_BF16 && kv_dtype != GLLM_DTYPE_FP8_E4M3)
    return fail(GLLM_ATTN_EUNSUPPORTED, "kv_dtype %d (bf16 or fp8 e4m3fn)", kv_dtype);
  if (head_dim != 64 && head_dim != 128) return fail(GLLM_ATTN_EUNSUPPORTED, "head_dim %d (64 or 128)", head_dim);
  if (num_q_heads <= 0 || num_kv_heads <= 0) return fail(GLLM_ATTN_EINVAL, "head counts must be > 0");
  if (hidden <= 0 || hidden % 32) return fail(GLLM_ATTN_EUNSUPPORTED, "hidden %d must be a positive multiple of 32", hidden);
  if (!x || !w_k || !w_v || !k_cache || !v_cache || !slot_mapping || !cos || !sin)
    return fail(GLLM_ATTN_EINVAL, "null pointer argument");
  if (q_out && !w_q) return fail(GLLM_ATTN_EINVAL, "q_out given without w_q");
  auto aligned16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!aligned16(x) || !aligned16(w_k) || !aligned16(w_v) || (q_out && !aligned16(w_q)))
    return fail(GLLM_ATTN_EINVAL, "x and the weights must be 16-byte aligned");
  if (x_row_stride < hidden || x_row_stride % 8 || w_k_row_stride < hidden || w_k_row_stride % 8 ||
      w_v_row_stride < hidden || w_v_row_stride % 8 || (q_out && (w_q_row_stride < hidden || w_q_row_stride % 8)))
    return fail(GLLM_ATTN_EINVAL, "row strides must be >= hidden and multiples of 8 elements");
  if (q_out && q_out_row_stride < (int64_t)num_q_heads * head_dim)
    return fail(GLLM_ATTN_EINVAL, "q_out row stride < num_q_heads * head_dim");
  if (cache_slot_stride < (int64_t)num_kv_heads * head_dim) return fail(GLLM_ATTN_EINVAL, "cache_slot_stride too small");
  if (num_slots <= 0) return fail(GLLM_ATTN_EINVAL, "num_slots must be > 0");
  if (rope_row_stride < head_dim / 2) return fail(GLLM_ATTN_EINVAL, "rope_row_stride < head_dim / 2");
  if (query_lens && tokens_per_seq <= 0) return fail(GLLM_ATTN_EINVAL, "tokens_per_seq must be > 0 with query_lens");
  QKVArgs a{};
  a.x = x; a.x_row_stride = x_row_stride; a.num_tokens = num_tokens; a.hidden = hidden;
  a.w_q = w_q; a.w_k = w_k; a.w_v = w_v;
  a.w_q_row_stride = w_q_row_stride; a.w_k_row_stride = w_k_row_stride; a.w_v_row_stride = w_v_row_stride;
  a.q_out = q_out; a.q_out_row_stride = q_out_row_stride; a.rotate_q = rotate_q ? 1 : 0;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slot_stride = cache_slot_stride; a.num_slots = num_slots;
  a.slot_mapping = slot_mapping; a.query_lens = query_lens; a.tokens_per_seq = tokens_per_seq;
  a.cos = cos; a.sin = sin; a.rope_rows = rope_rows; a.rope_row_stride = rope_row_stride;
  a.num_q_heads = num_q_heads; a.num_kv_heads = num_kv_heads; a.head_dim = head_dim; a.kv_dtype = kv_dtype;
  if (workspace && ((uintptr_t)workspace & 15)) return fail(GLLM_ATTN_EINVAL, "workspace must be 16-byte aligned");
  a.workspace = (float*)workspace; a.workspace_bytes = workspace ? workspace_bytes : 0;
  a.cus = device_cus();
  return hip_check(launch_qkv_rope_write(a, (hipStream_t)stream), "qkv projection launch");
}

}  // extern "C"

// ---------------------------------------------------------------- no-alloc QKV
// Scratch of gllm_qkv_rope_kv_write_noalloc: the split-K partial sums live in
// this file-scope device array (one copy per GPU, held until the process
// ends).  Host code never passes the array's name to a kernel: it is only a
// host-side stand-in.  Its device address comes from hipGetSymbolAddress, once
// per device with that device current, and that address is what the kernels
// get.  Every call on a GPU shares the GPU's array, so calls that overlap on
// one GPU race; each call fully rewrites the partials it reads (the partial
// kernel stores every element before the finish kernel sums them), so no
// clearing is needed.
namespace {
constexpr size_t kQkvScratchBytes = size_t(24) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) char g_qkv_scratch[kQkvScratchBytes];
void* g_qkv_scratch_ptr[kMaxDevices] = {};
std::mutex g_qkv_scratch_mu;

int qkv_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_check(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(GLLM_ATTN_EUNSUPPORTED, "device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_qkv_scratch_mu);
  if (!g_qkv_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_qkv_scratch));
    if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(qkv scratch)");
    g_qkv_scratch_ptr[dev] = p;
  }
  *out = g_qkv_scratch_ptr[dev];
  return ok();
}
}  // namespace

extern "C" {

int gllm_qkv_rope_kv_write_noalloc(const void* x, int64_t x_row_stride, int64_t num_tokens, int32_t hidden,
                                   const void* w_q, int64_t w_q_row_stride, const void* w_k, int64_t w_k_row_stride,
                                   const void* w_v, int64_t w_v_row_stride, void* q_out, int64_t q_out_row_stride,
                                   int32_t rotate_q, void* k_cache, void* v_cache, int64_t cache_slot_stride,
                                   int64_t num_slots, const int64_t* slot_mapping, const int32_t* query_lens,
                                   int64_t tokens_per_seq, const void* cos, const void* sin, const int64_t* rope_rows,
                                   int64_t rope_row_stride, int32_t num_q_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t dtype, int32_t kv_dtype, void* stream) {
  Range range("gllm_qkv_rope_kv_write_noalloc");
  if (num_tokens < 0 || hidden <= 0 || num_kv_heads <= 0 || num_q_heads <= 0)
    return gllm_qkv_rope_kv_write(x, x_row_stride, num_tokens, hidden, w_q, w_q_row_stride, w_k, w_k_row_stride,
                                  w_v, w_v_row_stride, q_out, q_out_row_stride, rotate_q, k_cache, v_cache,
                                  cache_slot_stride, num_slots, slot_mapping, query_lens, tokens_per_seq, cos, sin,
                                  rope_rows, rope_row_stride, num_q_heads, num_kv_heads, head_dim, dtype, kv_dtype,
                                  nullptr, 0, stream);   // the argument checks and their messages
  const size_t need = gllm_qkv_workspace_bytes(num_tokens, hidden, num_q_heads, num_kv_heads, head_dim, q_out != nullptr);
  if (need > kQkvScratchBytes)
    return fail(GLLM_ATTN_EUNSUPPORTED,
                "this batch's split-K partials need %zu bytes, more than the %zu-byte static scratch of the "
                "no-alloc entry point; call gllm_qkv_rope_kv_write with a workspace", need, kQkvScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = qkv_scratch(&ws)) return rc;
  }
  return gllm_qkv_rope_kv_write(x, x_row_stride, num_tokens, hidden, w_q, w_q_row_stride, w_k, w_k_row_stride,
                                w_v, w_v_row_stride, q_out, q_out_row_stride, rotate_q, k_cache, v_cache,
                                cache_slot_stride, num_slots, slot_mapping, query_lens, tokens_per_seq, cos, sin,
                                rope_rows, rope_row_stride, num_q_heads, num_kv_heads, head_dim, dtype, kv_dtype,
                                ws, need, stream);
}

size_t gllm_qkv_workspace_bytes(int64_t num_tokens, int32_t hidden, int32_t num_q_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t with_q) {
  if (num_tokens <= 0 || hidden <= 0 || num_kv_heads <= 0 || num_q_heads < 0) return 0;
  return qkv_workspace_bytes(num_tokens, hidden, (with_q ? num_q_heads : 0) + 2 * num_kv_heads, head_dim,
                             device_cus());
}

int gllm_attn_plan_create(gllm_attn_plan** out, const int32_t* query_lens, const int32_t* seq_lens,
                          int32_t num_seqs, int64_t q_seq_stride, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t dtype,
                          int32_t split_tokens, int32_t decode_heads_per_wg) {
  if (!out) return fail(GLLM_ATTN_EINVAL, "plan out-pointer is null");
  *out = nullptr;
  if (num_seqs < 0 || (num_seqs > 0 && (!query_lens || !seq_lens)))
    return fail(GLLM_ATTN_EINVAL, "bad sequence arrays");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(GLLM_ATTN_EINVAL, "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)",
                num_q_heads, num_kv_heads);
  if (block_size <= 0 || block_size > kMaxBlockSize)
    return fail(GLLM_ATTN_EINVAL, "block_size %d must be in [1, %d]", block_size, kMaxBlockSize);
  if (!model_dtype_ok(dtype)) return fail(GLLM_ATTN_EUNSUPPORTED, "model dtype %d (f32, bf16 or f16)", dtype);
  if (head_dim <= 0 || head_dim > 256 || head_dim % 2)
    return fail(GLLM_ATTN_EUNSUPPORTED, "head_dim %d (even, at most 256)", head_dim);
  const bool mfma = mfma_dtype(dtype) && (head_dim == 64 || head_dim == 128);
  if (split_tokens != GLLM_SPLIT_BALANCED && (split_tokens < 0 || split_tokens % 32))
    return fail(GLLM_ATTN_EINVAL, "split_tokens must be a multiple of 32 or GLLM_SPLIT_BALANCED");
  if (decode_heads_per_wg != 0 && decode_heads_per_wg != 1 && decode_heads_per_wg != 2 &&
      decode_heads_per_wg != 4 && decode_heads_per_wg != 8)
    return fail(GLLM_ATTN_EINVAL, "decode_heads_per_wg must be 0 (auto), 1, 2, 4 or 8");
  if (q_seq_stride < 0) return fail(GLLM_ATTN_EINVAL, "q_seq_stride < 0");
  const int G = num_q_heads / num_kv_heads;

  gllm_attn_plan* p = new (std::nothrow) gllm_attn_plan();
  if (!p) return fail(GLLM_ATTN_EINVAL, "out of host memory");
  p->num_seqs = num_seqs; p->Hq = num_q_heads; p->Hkv = num_kv_heads; p->D = head_dim;
  p->bs = block_size; p->dtype = dtype; p->mfma = mfma;
  p->seqs.resize(num_seqs);
  int64_t row = 0, decode_tokens = 0;
  for (int i = 0; i < num_seqs; ++i) {
    const int32_t ql = query_lens[i], sl = seq_lens[i];
    if (ql < 1 || sl < ql) {
      delete p;
      return fail(GLLM_ATTN_EINVAL, "sequence %d: query_len %d / seq_len %d invalid", i, ql, sl);
    }
    if (q_seq_stride > 0 && ql > q_seq_stride) {
      delete p;
      return fail(GLLM_ATTN_EINVAL, "sequence %d: query_len %d exceeds q_seq_stride %lld", i, ql, (long long)q_seq_stride);
    }
    SeqInfo& s = p->seqs[i];
    s = SeqInfo{};
    s.q_row_start = (int32_t)(q_seq_stride > 0 ? (int64_t)i * q_seq_stride : row);
    s.ctx_len = sl - ql;
    s.q_len = ql;
    row += ql;
    p->max_q = std::max(p->max_q, ql);
    if (mfma && ql * G <= 16) decode_tokens += sl;
  }
  p->total_rows = q_seq_stride > 0 ? (int64_t)num_seqs * q_seq_stride : row;
  if (p->total_rows > INT32_MAX) {
    delete p;
    return fail(GLLM_ATTN_EINVAL, "too many query rows");
  }

  if (mfma) {
    const int cus = device_cus();
    int64_t n_pf = 0;
    for (int i = 0; i < num_seqs; ++i)
      if ((int64_t)query_lens[i] * G > 16) ++n_pf;
    bool balanced = false;
    std::vector<PrefillPiece> pcs;   // prefill items of a mixed page-balanced launch
    int64_t mixed_wgs = 0;
    if (n_pf > 0) {
      // Mixed batch, page-balanced decode share plus prefill items: on
      // request only (config (d): 482-487 µs against 455-464 for the item plan
      // below; 291 vs 299 µs with 128 decodes and 4 prefills).
      if (n_pf < num_seqs && split_tokens == GLLM_SPLIT_BALANCED) {
        for (int i = 0; i < num_seqs; ++i)
          if (p->seqs[i].q_len * G > 16) prefill_pieces(p->seqs[i], i, G, num_kv_heads, pcs);
        mixed_wgs = mixed_decode_wgs(p, cus, decode_heads_per_wg, pcs);
        balanced = true;
      }
    } else if (split_tokens == GLLM_SPLIT_BALANCED) {
      balanced = num_seqs > 0;
    } else if (split_tokens == 0 && num_seqs > 0) {
      const BalancedShape bsh = balanced_shape(p, cus, decode_heads_per_wg);
      balanced = bsh.units >= balanced_min_units_per_wg(p->D) * bsh.wgs;
    }
    if (balanced) {
      plan_balanced_decode(p, cus, decode_heads_per_wg, mixed_wgs);
      if (n_pf > 0) {
        p->n_prefill_seqs = (int32_t)n_pf;
        plan_mixed_prefill(p, pcs);
        if (p->items.size() + p->seg_ptr.size() > (size_t)INT32_MAX) {
          delete p;
          return fail(GLLM_ATTN_EINVAL, "too many work items");
        }
      }
    } else {
    // Decode: one 8-wave workgroup per (sequence, split, HW kv heads); the
    // other 8 / HW waves interleave each head's keys.  Rule (fitted to MI355X
    // measurements of the benchmark batches): the first HW of 2, 1, 4, 8
    // whose unsplit units give every CU its resident workgroups (2 at D=64,
    // 1 at D=128) wins; HW=2 reads 256-byte runs of each slot and still
    // spreads one sequence over several CUs.  If none fills the GPU, HW=2 and
    // sequences are split into equal key ranges.  A split caches at most 511
    // block ids.
    int64_t cap = (int64_t)511 * block_size / 32 * 32;
    cap = std::max<int64_t>(32, std::min<int64_t>(cap, 8192));
    int64_t ndec = 0;
    for (int i = 0; i < num_seqs; ++i)
      if (query_lens[i] * G <= 16) ++ndec;
    const int64_t target = (int64_t)cus * (head_dim == 64 ? 2 : 1);
    int best_hw = 0;
    const int hw_pref[4] = {2, 1, 4, 8};
    for (int hw : hw_pref) {
      if (decode_heads_per_wg && hw != decode_heads_per_wg) continue;
      if (ndec * ((num_kv_heads + hw - 1) / hw) >= target) {
        best_hw = hw;
        break;
      }
    }
    const bool fills = best_hw != 0;
    if (!fills) best_hw = decode_heads_per_wg ? decode_heads_per_wg : 2;
    while (best_hw > 1 && best_hw / 2 >= num_kv_heads) best_hw /= 2;  // no idle head slots
    const int best_nw = 8;
    int64_t best_S = split_tokens < 0 ? 0 : split_tokens;
    if (best_S == 0) {
      if (fills) {
        best_S = cap;
      } else {
        // about half as many items as resident slots, at least 256 keys each:
        // a split's partial write and merge cost more than the parallelism
        // of smaller ones buys (measured: 2 x 8000-key 8B sequences 48.8 ->
        // 38.7 us, config (a)'s 16-layer bf16 decode step 229 -> 194 us)
        const int64_t hg = (num_kv_heads + best_hw - 1) / best_hw;
        best_S = (2 * decode_tokens * hg + target - 1) / std::max<int64_t>(target, 1);
        best_S = std::max<int64_t>((best_S + 31) / 32 * 32, 256);
      }
    }
    best_S = std::min(best_S, cap);
    p->heads_per_wg = best_hw;
    p->decode_waves = best_nw;
    // Prefill: 8-wave workgroups, one per CU (4-stage K/V ring in LDS).
    // prefill-only launches: kPrefillOnlyWaves-wave workgroups (prefill_kernel);
    // a mixed launch's prefill items run in its 8-wave workgroups
    const int pw = ndec == 0 ? kPrefillOnlyWaves : 8;
    p->prefill_waves = pw;
    const int hgroups = (num_kv_heads + best_hw - 1) / best_hw;
    const int64_t S = best_S;
    p->split_len = (int32_t)S;
    struct Keyed { int64_t work; WorkItem it; };
    std::vector<Keyed> pf, dc;
    for (int i = 0; i < num_seqs; ++i) {
      SeqInfo& s = p->seqs[i];
      const int L = s.ctx_len + s.q_len;
      if (s.q_len * G <= 16) {
        ++p->n_decode_seqs;
        // equal splits of 16-key multiples (a remainder split after full
        // S-key ones was the slowest item): len = ceil16(ceil(L / n)) for
        // the final n, which the kernel recomputes from (L, nsplits) alone
        s.nsplits = (int32_t)((L + S - 1) / S);
        int64_t len = split_len_of(L, s.nsplits);
        s.nsplits = (int32_t)((L + len - 1) / len);
        len = split_len_of(L, s.nsplits);
        s.partial_base = (int32_t)p->n_partials;
        if (s.nsplits > 1) p->n_partials += (int64_t)num_kv_heads * s.nsplits;
        for (int sp = 0; sp < s.nsplits; ++sp)
          for (int hg = 0; hg < hgroups; ++hg) {
            const int64_t keys = std::min<int64_t>(L, (int64_t)(sp + 1) * len) - (int64_t)sp * len;
            dc.push_back({keys, WorkItem{kItemDecode | (hg << 8), i, sp, s.q_row_start, s.ctx_len, s.q_len,
                                         s.nsplits, s.partial_base}});
          }
      } else {
        ++p->n_prefill_seqs;
        pcs.clear();
        prefill_pieces(s, i, G, num_kv_heads, pcs, pw);
        for (const PrefillPiece& pc : pcs) pf.push_back({pc.kend, pc.it});
      }
    }
    // Longest work first so the tail is made of short items.
    std::stable_sort(pf.begin(), pf.end(), [](const Keyed& x, const Keyed& y) { return x.work > y.work; });
    std::stable_sort(dc.begin(), dc.end(), [](const Keyed& x, const Keyed& y) { return x.work > y.work; });
    // Workgroups are dispatched slot-major: while every slot is free, item k
    // and item k + cus land on the same CU, and the older (first) one wins
    // the CU's memory pipeline.
    std::vector<Keyed> all;
    all.reserve(pf.size() + dc.size());
    const size_t ncu = (size_t)cus;
    if (pf.empty() && head_dim == 64 && dc.size() > ncu && dc.size() <= 2 * ncu) {
      // Decode items that all fit at once, two per CU: CU k pairs the k-th
      // longest with the k-th shortest item (equal work per CU) and gets the
      // short one first, so it finishes quickly and the long one then has the
      // CU's full bandwidth (long-first starves the short item until the long
      // one is done, then leaves it alone on the CU).  CUs without a pair take
      // the middle items.  Config (b): 37.5 µs, against 44.1 in the snake
      // order of the other decode-only plans.
      const size_t n = dc.size(), m = n - ncu;   // m paired CUs
      all.resize(n);
      for (size_t k = 0; k < m; ++k) {
        all[k] = dc[n - 1 - k];                  // first slot: short
        all[ncu + k] = dc[k];                    // second slot: long
      }
      for (size_t k = m; k < ncu; ++k) all[k] = dc[k];   // middle items, alone on their CU
    } else {
      // Mixed batch: the prefill items (MFMA-bound, longest first) are spread
      // evenly through the first half of the decode items (HBM-bound, longest
      // first): prefill item i goes before decode item i * ndc / (2 npf).
      // Some CUs compute while the others keep HBM busy (a mixed launch holds
      // one workgroup per CU), every prefill item has started by the middle
      // of the launch, and the short decode items fill the tail.  Measured on
      // config (d), mean of 8 runs each: 460 µs, against 469 with the prefill
      // items spread through all the decode items, 464 / 463 with them in the
      // first 40% / 30%, 485 with all of them first and 512 with them last.
      // Decode-only item plans: snake order, the direction alternating every
      // cus / 8 items, so long and short work interleave as slots free up
      // (decode_8b on one box: 390.5 µs against 397.5 with the direction
      // alternating every cus items, 402 / 413 every 1.5 / 2 cus, 390.7
      // every cus / 4, 406 in plain longest-first order).
      size_t di = 0;
      for (size_t i = 0; i < pf.size(); ++i) {
        const size_t upto = i * dc.size() / (2 * pf.size());
        while (di < upto) all.push_back(dc[di++]);
        all.push_back(pf[i]);
      }
      while (di < dc.size()) all.push_back(dc[di++]);
      if (pf.empty()) {
        const size_t per = std::max<size_t>(8, ncu / 8);
        for (size_t c0 = per, chunk = 1; c0 < all.size(); c0 += per, ++chunk)
          if (chunk & 1) std::reverse(all.begin() + c0, all.begin() + std::min(all.size(), c0 + per));
      }
    }
    p->items.reserve(all.size());
    for (auto& k : all) p->items.push_back(k.it);
    if (p->items.size() > (size_t)INT32_MAX) {
      delete p;
      return fail(GLLM_ATTN_EINVAL, "too many work items");
    }
    }
  }
  if (p->n_partials > (int64_t)INT32_MAX / 16) {
    delete p;
    return fail(GLLM_ATTN_EINVAL, "too many split partials");
  }

  // Workspace layout: items | seqs | segments | segment ranges | tickets |
  // partial (m, l) | partial acc.
  size_t o = 0;
  p->off_items = o; o = align256(o + p->items.size() * sizeof(WorkItem));
  p->off_seqs = o; o = align256(o + p->seqs.size() * sizeof(SeqInfo));
  p->off_segs = o; o = align256(o + p->segs.size() * sizeof(DecodeSeg));
  p->off_segptr = o; o = align256(o + p->seg_ptr.size() * sizeof(int32_t));
  p->off_ctr = o; o = align256(o + (size_t)num_seqs * num_kv_heads * sizeof(int32_t));
  p->off_ml = o; o = align256(o + (size_t)p->n_partials * 16 * 2 * sizeof(float));
  p->off_part = o; o = align256(o + (size_t)p->n_partials * 16 * head_dim * sizeof(float));
  p->ws_bytes = std::max<size_t>(o, 256);
  const size_t stage = p->off_ctr;
  if (stage > 0) {
    p->pinned = pinned_pool().acquire(stage, &p->pinned_cap);
    if (!p->pinned) {
      p->pinned = std::malloc(stage);
      p->pinned_is_host_malloc = true;
      if (!p->pinned) {
        delete p;
        return fail(GLLM_ATTN_EINVAL, "out of host memory for %zu staging bytes", stage);
      }
    }
    std::memset(p->pinned, 0, stage);
    if (!p->items.empty()) std::memcpy((char*)p->pinned + p->off_items, p->items.data(), p->items.size() * sizeof(WorkItem));
    if (!p->seqs.empty()) std::memcpy((char*)p->pinned + p->off_seqs, p->seqs.data(), p->seqs.size() * sizeof(SeqInfo));
    if (!p->segs.empty()) std::memcpy((char*)p->pinned + p->off_segs, p->segs.data(), p->segs.size() * sizeof(DecodeSeg));
    if (!p->seg_ptr.empty())
      std::memcpy((char*)p->pinned + p->off_segptr, p->seg_ptr.data(), p->seg_ptr.size() * sizeof(int32_t));
  }
  *out = p;
  return ok();
}

size_t gllm_attn_plan_workspace_bytes(const gllm_attn_plan* p) { return p ? p->ws_bytes : 0; }

int gllm_attn_plan_info(const gllm_attn_plan* p, int64_t* info, int32_t n) {
  if (!p || !info) return fail(GLLM_ATTN_EINVAL, "null plan or info");
  const int64_t n_wg = (int64_t)p->items.size() + (p->segs.empty() ? 0 : (int64_t)p->seg_ptr.size() - 1);
  const int64_t v[10] = {n_wg, p->split_len, p->n_decode_seqs, p->n_prefill_seqs, p->n_partials,
                         p->total_rows, p->heads_per_wg, p->decode_waves, p->prefill_waves,
                         (int64_t)p->segs.size()};
  for (int i = 0; i < n && i < 10; ++i) info[i] = v[i];
  return ok();
}

int gllm_attn_plan_upload(gllm_attn_plan* p, void* workspace, size_t bytes, void* stream) {
  Range range("gllm_attn_plan_upload");
  if (!p) return fail(GLLM_ATTN_EINVAL, "null plan");
  if (!workspace || bytes < p->ws_bytes)
    return fail(GLLM_ATTN_EINVAL, "workspace of %zu bytes is smaller than the %zu the plan needs", bytes, p->ws_bytes);
  if (((uintptr_t)workspace & 255) != 0) return fail(GLLM_ATTN_EINVAL, "workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  p->ws = (char*)workspace;
  if (p->off_ctr > 0) {
    hipError_t e = hipMemcpyAsync(p->ws, p->pinned, p->off_ctr, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_check(e, "plan upload copy");
  }
  hipError_t e = launch_fill_zero_i32((int32_t*)(p->ws + p->off_ctr), (int64_t)p->num_seqs * p->Hkv, st);
  if (e != hipSuccess) return hip_check(e, "ticket clear");
  if (!p->upload_done) {
    e = hipEventCreateWithFlags(&p->upload_done, hipEventDisableTiming);
    if (e != hipSuccess) return hip_check(e, "hipEventCreate");
  }
  return hip_check(hipEventRecord(p->upload_done, st), "hipEventRecord");
}

int gllm_attn_plan_destroy(gllm_attn_plan* p) {
  if (!p) return ok();
  if (p->pinned && !p->pinned_is_host_malloc) {
    // back to the pool with the upload's event: reused once the copy is done
    pinned_pool().release(p->pinned, p->pinned_cap, p->upload_done);
  } else {
    if (p->upload_done) {
      (void)hipEventSynchronize(p->upload_done);  // the staging copy must finish before the free
      (void)hipEventDestroy(p->upload_done);
    }
    if (p->pinned) std::free(p->pinned);
  }
  delete p;
  return ok();
}

static int fill_common(AttnArgs& a, int32_t Hq, int32_t Hkv, int32_t D, float scale, int32_t dtype, int32_t kv_dtype) {
  a.num_q_heads = Hq; a.num_kv_heads = Hkv; a.head_dim = D;
  a.scale = scale; a.dtype = dtype; a.kv_dtype = kv_dtype;
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(GLLM_ATTN_EINVAL, "scale must be finite and > 0");
  return ok();
}

// gllm_paged_attention and, with k_new / v_new, gllm_paged_attention_write_kv.
static int paged_attention_impl(const gllm_attn_plan* p, const void* q, int64_t q_row_stride, void* out,
                                int64_t out_row_stride, const void* k_cache, const void* v_cache,
                                int64_t cache_slot_stride, int64_t num_blocks, const int32_t* block_table,
                                int64_t block_table_stride, const void* k_new, int64_t k_new_row_stride,
                                const void* v_new, int64_t v_new_row_stride, const void* rope_cos,
                                const void* rope_sin, int64_t rope_row_stride, int32_t rope_mode, float scale,
                                int32_t dtype, int32_t kv_dtype, void* stream) {
  if (!p) return fail(GLLM_ATTN_EINVAL, "null plan");
  if (!p->ws) return fail(GLLM_ATTN_EINVAL, "plan was not uploaded (gllm_attn_plan_upload)");
  if (dtype != p->dtype) return fail(GLLM_ATTN_EINVAL, "dtype %d differs from the plan's %d", dtype, p->dtype);
  if (!q || !out || !k_cache || !v_cache || !block_table) return fail(GLLM_ATTN_EINVAL, "null pointer argument");
  const int64_t hd = (int64_t)p->Hq * p->D;
  if (q_row_stride < hd || out_row_stride < hd) return fail(GLLM_ATTN_EINVAL, "q/out row stride < num_q_heads * head_dim");
  if (cache_slot_stride < (int64_t)p->Hkv * p->D) return fail(GLLM_ATTN_EINVAL, "cache_slot_stride too small");
  if (num_blocks <= 0) return fail(GLLM_ATTN_EINVAL, "num_blocks must be > 0");
  if ((uint64_t)num_blocks * (uint64_t)p->bs >= (1ull << 32))
    return fail(GLLM_ATTN_EUNSUPPORTED, "pool of %lld blocks x %d slots exceeds 2^32 slots", (long long)num_blocks, p->bs);
  if (block_table_stride <= 0) return fail(GLLM_ATTN_EINVAL, "block_table_stride must be > 0");
  if (rope_mode != GLLM_ROPE_NONE && rope_mode != GLLM_ROPE_BY_POSITION && rope_mode != GLLM_ROPE_BY_ROW)
    return fail(GLLM_ATTN_EINVAL, "rope_mode %d", rope_mode);
  if (rope_mode != GLLM_ROPE_NONE && (!rope_cos || !rope_sin || rope_row_stride < p->D / 2))
    return fail(GLLM_ATTN_EINVAL, "rope tables missing or row stride < head_dim / 2");
  if (!kv_dtype_ok(kv_dtype)) return fail(GLLM_ATTN_EUNSUPPORTED, "kv_dtype %d (f32, bf16, f16 or fp8 e4m3fn)", kv_dtype);
  AttnArgs a{};
  if (int rc = fill_common(a, p->Hq, p->Hkv, p->D, scale, dtype, kv_dtype)) return rc;
  a.q = q; a.q_row_stride = q_row_stride; a.out = out; a.out_row_stride = out_row_stride;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_slot_stride = cache_slot_stride; a.num_blocks = num_blocks;
  a.block_table = block_table; a.block_table_stride = block_table_stride;
  a.block_size = p->bs;
  block_div(p->bs, &a.block_magic, &a.block_shift);
  a.rope_cos = rope_cos; a.rope_sin = rope_sin; a.rope_row_stride = rope_row_stride; a.rope_mode = rope_mode;
  a.seqs = (const SeqInfo*)(p->ws + p->off_seqs);
  a.items = (const WorkItem*)(p->ws + p->off_items);
  a.n_items = (int32_t)p->items.size();
  if (!p->segs.empty()) {
    a.segs = (const DecodeSeg*)(p->ws + p->off_segs);
    a.seg_ptr = (const int32_t*)(p->ws + p->off_segptr);
    a.n_segs = (int32_t)p->segs.size();
    a.n_seg_wgs = (int32_t)p->seg_ptr.size() - 1;
    a.n_items = a.n_seg_wgs + (int32_t)p->items.size();   // decode workgroups, then any prefill items
  }
  a.num_seqs = p->num_seqs;
  a.counters = (int32_t*)(p->ws + p->off_ctr);
  a.partial_ml = (float*)(p->ws + p->off_ml);
  a.partials = (float*)(p->ws + p->off_part);
  a.split_len = p->split_len;
  a.n_partials = p->n_partials;
  a.heads_per_wg = p->heads_per_wg;
  a.decode_waves = p->decode_waves;
  a.prefill_waves = p->prefill_waves;
  // the MFMA kernels read a cache in the model dtype or fp8; a 16-bit model
  // over an f32 (or the other 16-bit) cache takes the generic kernel, which
  // rounds each cached value to the model dtype as the reference's gather does
  const bool use_mfma = p->mfma && (kv_dtype == dtype || kv_dtype == GLLM_DTYPE_FP8_E4M3);
  if (k_new || v_new) {
    if (!k_new || !v_new) return fail(GLLM_ATTN_EINVAL, "k_new and v_new go together");
    const int64_t kvd = (int64_t)p->Hkv * p->D;
    if (k_new_row_stride < kvd || v_new_row_stride < kvd)
      return fail(GLLM_ATTN_EINVAL, "k_new / v_new row stride < num_kv_heads * head_dim");
    // every sequence on the decode path: its new keys are read only by the
    // task that writes them (prefill items read other items' new keys)
    if (use_mfma ? p->n_prefill_seqs > 0 : p->max_q > kMaxFusedRows)
      return fail(GLLM_ATTN_EINVAL, "the fused KV write needs a decode-path plan (query_len x G <= 16 on the MFMA "
                                    "kernels, query_len <= %d on the generic one)", kMaxFusedRows);
    a.k_new = k_new; a.v_new = v_new;
    a.k_new_row_stride = k_new_row_stride; a.v_new_row_stride = v_new_row_stride;
  }
  hipStream_t st = (hipStream_t)stream;
  if (use_mfma)
    return hip_check(launch_paged_attention_mfma(a, p->n_prefill_seqs > 0, p->n_decode_seqs > 0, st),
                     "paged attention launch");
  return hip_check(launch_attention_f32(a, false, p->num_seqs, p->max_q, st), "generic attention launch");
}

int gllm_paged_attention(const gllm_attn_plan* p, const void* q, int64_t q_row_stride, void* out,
                         int64_t out_row_stride, const void* k_cache, const void* v_cache,
                         int64_t cache_slot_stride, int64_t num_blocks, const int32_t* block_table,
                         int64_t block_table_stride, const void* rope_cos, const void* rope_sin,
                         int64_t rope_row_stride, int32_t rope_mode, float scale, int32_t dtype,
                         int32_t kv_dtype, void* stream) {
  Range range("gllm_paged_attention");
  return paged_attention_impl(p, q, q_row_stride, out, out_row_stride, k_cache, v_cache, cache_slot_stride,
                              num_blocks, block_table, block_table_stride, nullptr, 0, nullptr, 0, rope_cos,
                              rope_sin, rope_row_stride, rope_mode, scale, dtype, kv_dtype, stream);
}

int gllm_paged_attention_write_kv(const gllm_attn_plan* p, const void* q, int64_t q_row_stride, void* out,
                                  int64_t out_row_stride, void* k_cache, void* v_cache,
                                  int64_t cache_slot_stride, int64_t num_blocks, const int32_t* block_table,
                                  int64_t block_table_stride, const void* k_new, int64_t k_new_row_stride,
                                  const void* v_new, int64_t v_new_row_stride, const void* rope_cos,
                                  const void* rope_sin, int64_t rope_row_stride, int32_t rope_mode, float scale,
                                  int32_t dtype, int32_t kv_dtype, void* stream) {
  Range range("gllm_paged_attention_write_kv");
  if (!k_new || !v_new) return fail(GLLM_ATTN_EINVAL, "null k_new / v_new");
  return paged_attention_impl(p, q, q_row_stride, out, out_row_stride, k_cache, v_cache, cache_slot_stride,
                              num_blocks, block_table, block_table_stride, k_new, k_new_row_stride, v_new,
                              v_new_row_stride, rope_cos, rope_sin, rope_row_stride, rope_mode, scale, dtype,
                              kv_dtype, stream);
}

int gllm_attention_dense(const void* q, int64_t q_row_stride, const void* k, int64_t k_batch_stride,
                         int64_t k_row_stride, const void* v, int64_t v_batch_stride, int64_t v_row_stride,
                         const void* bias, int64_t bias_batch_stride, int64_t bias_row_stride, void* out,
                         int64_t out_row_stride, int32_t batch, int32_t q_len, int32_t kv_len,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                         int32_t dtype, void* stream) {
  Range range("gllm_attention_dense");
  if (!q || !k || !v || !bias || !out) return fail(GLLM_ATTN_EINVAL, "null pointer argument");
  if (batch < 0 || q_len < 0 || kv_len < 0) return fail(GLLM_ATTN_EINVAL, "negative size");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads)
    return fail(GLLM_ATTN_EINVAL, "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads, num_kv_heads);
  const int64_t hd = (int64_t)num_q_heads * head_dim;
  if (q_row_stride < hd || out_row_stride < hd) return fail(GLLM_ATTN_EINVAL, "q/out row stride too small");
  if (k_row_stride < (int64_t)num_kv_heads * head_dim || v_row_stride < (int64_t)num_kv_heads * head_dim)
    return fail(GLLM_ATTN_EINVAL, "k/v row stride too small");
  if (bias_row_stride < kv_len) return fail(GLLM_ATTN_EINVAL, "bias row stride < kv_len");
  if (!model_dtype_ok(dtype)) return fail(GLLM_ATTN_EUNSUPPORTED, "model dtype %d (f32, bf16 or f16)", dtype);
  if (head_dim <= 0 || head_dim > 256 || head_dim % 2)
    return fail(GLLM_ATTN_EUNSUPPORTED, "head_dim %d (even, at most 256)", head_dim);
  if (kv_len == 0 && batch * q_len > 0) return fail(GLLM_ATTN_EINVAL, "kv_len == 0 (softmax over no keys)");
  AttnArgs a{};
  if (int rc = fill_common(a, num_q_heads, num_kv_heads, head_dim, scale, dtype, dtype)) return rc;
  a.q = q; a.q_row_stride = q_row_stride; a.out = out; a.out_row_stride = out_row_stride;
  a.k = k; a.v = v; a.k_batch_stride = k_batch_stride; a.k_row_stride = k_row_stride;
  a.v_batch_stride = v_batch_stride; a.v_row_stride = v_row_stride;
  a.bias = bias; a.bias_batch_stride = bias_batch_stride; a.bias_row_stride = bias_row_stride;
  a.dense_T = kv_len; a.dense_Tq = q_len;
  hipStream_t st = (hipStream_t)stream;
  if (mfma_dtype(dtype) && (head_dim == 64 || head_dim == 128))
    return hip_check(launch_dense_attention_mfma(a, batch, q_len, st), "dense attention launch");
  return hip_check(launch_attention_f32(a, true, batch, q_len, st), "generic dense attention launch");
}

}  // extern "C"

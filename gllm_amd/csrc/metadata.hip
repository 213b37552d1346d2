// Device-side batch metadata: the per-row slot and position tensors that
// gllm/llm/llm.py:245-281 builds on the host with a per-row Python loop (and
// a dense O(B*T_q*T) bias that the paged kernels do not need).
//
// For query row r of sequence i (c_i = seq_len_i - query_len_i, L_i = seq_len_i):
//   position = c_i + r                                   if r < q_i (llm.py:281)
//              L_i - 1 (the last real position)           otherwise (padded rows)
//   slot     = block_table[i][(c_i + r) / bs] * bs + (c_i + r) % bs   if r < q_i
//              0 (the reserved dummy slot)                             otherwise
// which is what llm.py:245-247, 259-268 and 277 produce for the query
// columns of the left-padded slot mapping.  llm.py:281 gives padded rows
// c_i + r as well; in a mixed batch that can pass the RoPE table's last row
// (model.py:195 then indexes out of range), so padded rows are clamped to the
// sequence's last position: every position stays below max(seq_len), and
// real rows are unchanged.  Packed layout: sequence i's rows
// start at cu_seqlens[i] = q_0 + ... + q_{i-1}.
#include "common.h"
#include "launch.h"

namespace gllm {

// One workgroup per sequence: the row start is a reduction over the
// preceding query lengths (B is at most a few thousand), then the rows are
// written with a grid-stride loop.  Reads stay inside the caller's tables:
// block-table columns at or beyond `bt_width` and inconsistent lengths give
// slot 0.
__global__ void __launch_bounds__(256) build_metadata_kernel(MetadataArgs a) {
  __shared__ int64_t part[256 / 64];
  const int i = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t q = a.query_lens[i];
  const int32_t L = a.seq_lens[i];
  const int64_t c = (int64_t)L - q;
  int64_t start;
  int64_t nrows;
  if (a.q_seq_stride > 0) {
    start = (int64_t)i * a.q_seq_stride;
    nrows = a.q_seq_stride;
  } else {
    int64_t acc = 0;
    for (int j = tid; j < i; j += 256) acc += a.query_lens[j];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((tid & 63) == 0) part[tid >> 6] = acc;
    __syncthreads();
    start = part[0] + part[1] + part[2] + part[3];
    nrows = q;
    if (a.cu_seqlens && tid == 0) {
      a.cu_seqlens[i] = (int32_t)start;
      if (i == a.num_seqs - 1) a.cu_seqlens[i + 1] = (int32_t)(start + q);
    }
  }
  const int32_t* bt = a.block_table + (int64_t)i * a.block_table_stride;
  const bool ok = q >= 0 && c >= 0;
  for (int64_t r = tid; r < nrows; r += 256) {
    const int64_t row = start + r;
    if (row >= a.num_rows) break;
    // padded rows: the last real position (0 for an empty sequence)
    const int64_t pos = r < q ? c + r : (L > 0 ? (int64_t)L - 1 : 0);
    int64_t slot = 0;
    if (ok && r < q) {
      const int64_t bi = div_bs((uint32_t)pos, a.block_magic, a.block_shift);
      if (bi < a.bt_width) slot = (int64_t)bt[bi] * a.block_size + (pos - bi * a.block_size);
    }
    if (a.slot_mapping) a.slot_mapping[row] = slot;
    if (a.positions) a.positions[row] = pos;
  }
}

hipError_t launch_build_metadata(const MetadataArgs& a, hipStream_t st) {
  if (a.num_seqs == 0) return hipSuccess;
  hipLaunchKernelGGL(build_metadata_kernel, dim3((unsigned)a.num_seqs), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace gllm

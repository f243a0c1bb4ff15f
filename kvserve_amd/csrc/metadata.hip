// Device-side attention metadata: block tables resident in HBM, one packed upload per step.
//
// The reference rebuilds every step's metadata on the host (src/kvserve/model_runner.py:165-197,
// and the graph runner's buffer refresh, src/kvserve/cuda_graph.py:111-134): Python lists of
// every sequence's whole block table, 0- (or scratch-) padded, and one torch.tensor upload per
// field, O(B x W) host work per step. Here the tables live in a device pool (one row per
// sequence, kept across steps) and the host sends, in one int32 buffer,
//   seqs    [B][4]  row in the pool, first position of this step (start), query length q,
//                   number of table entries n_blocks (len(seq.block_table))
//   updates [U][3]  (row, column, block id): table entries appended since the last step
//   tokens  [T]     input token ids (when input_ids is requested)
// Two kernels then write the reference's tensors: the updates land in the pool, and workgroup b
// writes sequence b's row of block_tables (pool entries, padded to bt_width with bt_pad), its
// seq_len = start + q, query_len and query_start_loc, and, for its tokens, position start + i,
// slot pool[row][pos / BS] * BS + pos % BS (kv_cache.py:155-157) and the token id. P padding
// sequences follow the B real ones like the graph runner's pad rows: one token each, slot
// pad_slot, position 0, token 0, seq_len 1, a row of bt_pad.
//
// Nothing read from the packed buffer can move a write out of bounds: updates outside the pool
// are skipped, a position past a sequence's table gets slot -1 (which the cache-write kernels
// skip) and token indices are bounded by num_tokens.
#include <hip/hip_runtime.h>

#include "kvh_internal.h"

namespace kvh {
namespace {

constexpr int kMetaThreads = 256;

__global__ __launch_bounds__(kMetaThreads) void table_update_kernel(const int32_t* __restrict__ upd, int32_t n,
                                                                    int64_t* __restrict__ pool, int64_t rows,
                                                                    int64_t row_stride, int32_t width) {
  const int64_t step = (int64_t)gridDim.x * kMetaThreads;
  for (int64_t i = (int64_t)blockIdx.x * kMetaThreads + threadIdx.x; i < n; i += step) {
    const int32_t r = upd[3 * i], c = upd[3 * i + 1], blk = upd[3 * i + 2];
    if (r >= 0 && r < rows && c >= 0 && c < width) pool[r * row_stride + c] = blk;
  }
}

__global__ __launch_bounds__(kMetaThreads) void expand_metadata_kernel(MetaParams m) {
  __shared__ int s_prefix;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid == 0) s_prefix = 0;
  __syncthreads();
  // query_start_loc[b]: the real sequences' query lengths before b, then one token per pad row
  const int nreal = min(b, m.B);
  int part = 0;
  for (int i = tid; i < nreal; i += kMetaThreads) part += max(0, m.seqs[4 * i + 2]);
  if (part) atomicAdd(&s_prefix, part);
  __syncthreads();
  const int64_t prefix = (int64_t)s_prefix + (b - nreal);

  const bool pad = b >= m.B;
  int32_t row = 0, start = 0, q = 1, nblk = 0;
  if (!pad) {
    row = m.seqs[4 * b];
    start = m.seqs[4 * b + 1];
    q = max(0, m.seqs[4 * b + 2]);
    nblk = m.seqs[4 * b + 3];
  }
  const bool row_ok = !pad && row >= 0 && row < m.pool_rows && nblk >= 0 && nblk <= m.pool_width;
  const int nb = row_ok ? nblk : 0;
  const int64_t* prow = m.pool + (row_ok ? (int64_t)row * m.pool_rs : 0);
  if (tid == 0) {
    m.seq_lens[b] = pad ? 1 : (int64_t)start + q;
    if (m.query_lens) m.query_lens[b] = q;
    m.qsl[b] = prefix;
    if (b == m.B + m.P - 1) m.qsl[b + 1] = prefix + q;
  }
  if (m.bt) {
    int64_t* brow = m.bt + (int64_t)b * m.bt_rs;
    for (int c = tid; c < m.bt_width; c += kMetaThreads) brow[c] = c < nb ? prow[c] : m.bt_pad;
  }
  const int64_t tok_end = pad ? m.T + m.P : m.T;
  for (int i = tid; i < q; i += kMetaThreads) {
    const int64_t t = prefix + i;
    if (t >= tok_end) break;
    int64_t pos = 0, slot = m.pad_slot;
    if (!pad) {
      pos = (int64_t)start + i;
      const int64_t bi = pos / m.BS;
      slot = (pos >= 0 && bi < nb) ? prow[bi] * m.BS + pos % m.BS : -1;
    }
    m.slots[t] = slot;
    if (m.positions) m.positions[t] = pos;
    if (m.input_ids) m.input_ids[t] = pad ? 0 : (int64_t)m.tokens[t];
  }
}

}  // namespace

int launch_prepare_metadata(const MetaParams& m, const int32_t* updates, int32_t num_updates, hipStream_t s) {
  if (num_updates > 0) {
    int grid = (num_updates + kMetaThreads - 1) / kMetaThreads;
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(table_update_kernel, dim3(grid), dim3(kMetaThreads), 0, s, updates, num_updates, m.pool,
                       (int64_t)m.pool_rows, m.pool_rs, m.pool_width);
    if (hipError_t e = hipGetLastError()) return (int)e;
  }
  hipLaunchKernelGGL(expand_metadata_kernel, dim3(m.B + m.P), dim3(kMetaThreads), 0, s, m);
  return (int)hipGetLastError();
}

}  // namespace kvh

// On-device builders of the per-step attention metadata.
//
// Reference: ModelRunner.prepare_step, nanokvllm/engine/model_runner.py:160-219
// (per-token Python loop: positions = range(start, end), slot =
// block_table[pos // B] * B + pos % B, cu_seqlens_q/k prefix sums of the new
// tokens and of end = start + new, context_lens = end, logits_indices = last
// row of each sequence), prepare_block_tables (:154-158, rows right-padded with
// -1) and the decode builder of prepare_decode (:265-285, RoPE position =
// rope_pos, which runs ahead of the KV position once a sequence was
// compressed).
//
// MI355X design: the host sends one packed int32 buffer (per-sequence start,
// new-token count, RoPE offset, and the block tables) and two kernels expand
// it: a one-workgroup scan for the per-sequence arrays, then a (sequence,
// chunk) grid for the per-token arrays and the padded block-table rows. Block
// tables come either as a flat list with offsets, or -- the steady state of a
// serving loop -- as rows of a device-resident table store that the host keeps
// current with (row, col, id) updates for the blocks that changed since the
// last step (a decode step appends a block per sequence only every block_size
// tokens). Host work is O(sequences + changed blocks) instead of O(tokens).
#include "nkv_common.h"

namespace nkv {

constexpr int kScanThreads = 1024;
constexpr int kFillThreads = 256;
constexpr int kFillMaxChunks = 1024;

// One workgroup: exclusive prefix sums of new and of end = start + new; with a
// table store, first the store updates (row, col, id) that the fill kernel
// (next launch on the stream) will read.
__global__ __launch_bounds__(kScanThreads) void step_metadata_scan_kernel(
    const int32_t* __restrict__ starts, const int32_t* __restrict__ num_new, int32_t n,
    int32_t* __restrict__ cu_q, int32_t* __restrict__ cu_k, int32_t* __restrict__ context_lens,
    int64_t* __restrict__ logits_indices, int32_t* __restrict__ max_seqlens,
    int32_t* __restrict__ store, int64_t store_row_stride, int32_t store_rows,
    const int32_t* __restrict__ updates, int32_t n_updates) {
  __shared__ int32_t sq[kScanThreads], sk[kScanThreads], mq[kScanThreads], mk[kScanThreads];
  const int tid = threadIdx.x;
  for (int u = tid; u < n_updates; u += kScanThreads) {
    const int row = updates[3 * u], col = updates[3 * u + 1];
    if (row >= 0 && row < store_rows && col >= 0 && col < store_row_stride)
      store[(int64_t)row * store_row_stride + col] = updates[3 * u + 2];
  }
  const int per = (n + kScanThreads - 1) / kScanThreads;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
  int lq = 0, lk = 0, xq = 0, xk = 0;
  for (int i = i0; i < i1; ++i) {
    const int nw = max(num_new[i], 0);
    const int e = max(starts[i], 0) + nw;
    lq += nw;
    lk += e;
    xq = max(xq, nw);
    xk = max(xk, e);
  }
  sq[tid] = lq;
  sk[tid] = lk;
  mq[tid] = xq;
  mk[tid] = xk;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 1024 partial sums (and max reductions)
  for (int o = 1; o < kScanThreads; o <<= 1) {
    const int aq = tid >= o ? sq[tid - o] : 0;
    const int ak = tid >= o ? sk[tid - o] : 0;
    const int bq = tid >= o ? mq[tid - o] : 0;
    const int bk = tid >= o ? mk[tid - o] : 0;
    __syncthreads();
    sq[tid] += aq;
    sk[tid] += ak;
    mq[tid] = max(mq[tid], bq);
    mk[tid] = max(mk[tid], bk);
    __syncthreads();
  }
  int cq = sq[tid] - lq, ck = sk[tid] - lk;  // exclusive offsets of this thread's range
  if (tid == 0) {
    cu_q[0] = 0;
    cu_k[0] = 0;
    if (max_seqlens) {
      max_seqlens[0] = mq[kScanThreads - 1];
      max_seqlens[1] = mk[kScanThreads - 1];
    }
  }
  for (int i = i0; i < i1; ++i) {
    const int nw = max(num_new[i], 0);
    const int e = max(starts[i], 0) + nw;
    cq += nw;
    ck += e;
    cu_q[i + 1] = cq;
    cu_k[i + 1] = ck;
    if (context_lens) context_lens[i] = e;
    if (logits_indices) logits_indices[i] = (int64_t)cq - 1;
  }
}

// Grid (sequence, chunk): the sequence's tokens in strides of chunks*256, and
// (chunk 0) its block-table row padded with -1.
// Tables: flat list (bt_flat + bt_offsets) or store rows (store + rows/counts).
__global__ __launch_bounds__(kFillThreads) void step_metadata_fill_kernel(
    const int32_t* __restrict__ starts, const int32_t* __restrict__ num_new,
    const int32_t* __restrict__ pos_offsets, const int32_t* __restrict__ bt_flat,
    const int32_t* __restrict__ bt_offsets, const int32_t* __restrict__ store,
    int64_t store_row_stride, int32_t store_rows, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ cu_q, int32_t block_size,
    int64_t total_tokens, int64_t* __restrict__ positions, int32_t* __restrict__ slot_mapping,
    int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t bt_width) {
  const int s = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t* table;
  int nb;
  if (store) {
    const int row = rows[s];
    const bool ok = row >= 0 && row < store_rows;
    table = store + (ok ? (int64_t)row * store_row_stride : 0);
    nb = ok ? (int)min((int64_t)max(counts[s], 0), store_row_stride) : 0;
  } else {
    table = bt_flat + bt_offsets[s];
    nb = max(bt_offsets[s + 1] - bt_offsets[s], 0);
  }
  if (block_tables && blockIdx.y == 0) {
    for (int c = tid; c < bt_width; c += kFillThreads)
      block_tables[(int64_t)s * bt_row_stride + c] = c < nb ? table[c] : -1;
  }
  const int nw = max(num_new[s], 0);
  const int start = max(starts[s], 0);
  const int off = pos_offsets ? pos_offsets[s] : 0;
  const int64_t q0 = cu_q[s];
  const int n_tok = (int)min((int64_t)nw, max(total_tokens - q0, (int64_t)0));  // stay in bounds
  for (int i = blockIdx.y * kFillThreads + tid; i < n_tok; i += gridDim.y * kFillThreads) {
    const int kv = start + i;
    const int blk = kv / block_size;
    const int id = blk < nb ? table[blk] : -1;
    positions[q0 + i] = (int64_t)kv + off;
    slot_mapping[q0 + i] = id >= 0 ? id * block_size + (kv - blk * block_size) : -1;
  }
}

}  // namespace nkv

extern "C" int nkv_build_step_metadata(const int32_t* packed, int32_t n_seqs, int32_t block_size,
                                       int32_t max_new_tokens, int64_t total_tokens,
                                       int32_t flags, int32_t* table_store,
                                       int64_t store_row_stride, int32_t store_rows,
                                       int32_t n_updates, int32_t* cu_seqlens_q,
                                       int32_t* cu_seqlens_k, int32_t* context_lens,
                                       int64_t* positions, int32_t* slot_mapping,
                                       int64_t* logits_indices, int32_t* max_seqlens,
                                       int32_t* block_tables, int64_t bt_row_stride,
                                       int32_t bt_width, void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n_seqs >= 0 && block_size > 0 && max_new_tokens >= 0 && bt_width >= 0 &&
                  total_tokens >= 0 && n_updates >= 0 && (flags & ~1) == 0,
              NKV_EINVAL, "build_step_metadata: bad sizes or flags");
  NKV_REQUIRE(!table_store || (store_rows >= 0 && store_row_stride > 0), NKV_EINVAL,
              "build_step_metadata: bad table store shape");
  NKV_REQUIRE(table_store || n_updates == 0, NKV_EINVAL,
              "build_step_metadata: updates need a table store");
  if (n_seqs == 0 && n_updates == 0) return NKV_OK;
  NKV_REQUIRE(packed && cu_seqlens_q && cu_seqlens_k && positions && slot_mapping, NKV_EINVAL,
              "build_step_metadata: null pointer");
  NKV_REQUIRE(!block_tables || bt_row_stride >= bt_width, NKV_EINVAL,
              "build_step_metadata: bt_row_stride < bt_width");
  const int64_t n = n_seqs;
  const int32_t* starts = packed;
  const int32_t* num_new = packed + n;
  const int32_t* offs = (flags & 1) ? packed + 2 * n : nullptr;
  const int32_t* rest = packed + ((flags & 1) ? 3 : 2) * n;
  const int32_t* bt_offsets = table_store ? nullptr : rest;
  const int32_t* bt_flat = table_store ? nullptr : rest + n + 1;
  const int32_t* rows = table_store ? rest : nullptr;
  const int32_t* counts = table_store ? rest + n : nullptr;
  const int32_t* updates = table_store ? rest + 2 * n : nullptr;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(step_metadata_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, starts,
                     num_new, n_seqs, cu_seqlens_q, cu_seqlens_k, context_lens, logits_indices,
                     max_seqlens, table_store, store_row_stride, store_rows, updates, n_updates);
  int rc = check_launch("nkv_build_step_metadata (scan)");
  if (rc != NKV_OK || n_seqs == 0) return rc;
  const int chunks = std::max(1, std::min(kFillMaxChunks,
                                          (max_new_tokens + kFillThreads - 1) / kFillThreads));
  hipLaunchKernelGGL(step_metadata_fill_kernel, dim3((unsigned)n_seqs, (unsigned)chunks),
                     dim3(kFillThreads), 0, s, starts, num_new, offs, bt_flat, bt_offsets,
                     table_store, store_row_stride, store_rows, rows, counts, cu_seqlens_q,
                     block_size, total_tokens, positions, slot_mapping, block_tables,
                     bt_row_stride, bt_width);
  return check_launch("nkv_build_step_metadata (fill)");
}

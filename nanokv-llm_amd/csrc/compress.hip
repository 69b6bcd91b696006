// Window-based periodic KV compression step (SnapKV scoring, wave-level top-k
// selection, in-place compaction, last-layer bookkeeping).
//
// Reference: MyCompressCompact + helpers, nanokvllm/layers/compress_utils.py:
// 9-290, and SnapKV, nanokvllm/layers/CompressMethod.py:4-57.
//
// MI355X design. The step is HBM-bound (read the K window, move the kept K/V
// rows) and tiny in flops, so it is organised around bytes and launches:
//  * score: one workgroup per (selected sequence, KV head, 256-key chunk of
//    the window). K is read IN PLACE from the paged cache (the reference
//    first gathers K and V of the window into new tensors) straight into the
//    MFMA B layout; q K^T runs on v_mfma_f32_16x16x32_bf16 exactly as in
//    paged decode. Scaled scores (log2 domain) go to a small fp32 workspace.
//  * importance: one workgroup per kept set (sequence, or sequence x KV
//    head): per-head softmax statistics by wavefront reductions, then
//    importance[t] = sum_h softmax_h[t] over the set's query heads.
//  * top-k: one wavefront per kept set selects the num_keep largest
//    importances with a 32-step bitwise radix select on order-preserving
//    integer keys held in registers (ballot-free counts via shuffles), ties
//    broken by lower index, and writes the kept positions in ascending order
//    with a wave prefix sum -- no sort.
//  * compact: one workgroup per (sequence, KV head, K|V, 128-byte half of the
//    head row). Every source row of the unit is loaded into registers before
//    any destination row is written (s_waitcnt 0 + barrier), which gives the
//    reference's two-phase index_select().clone() / index_copy_ semantics
//    without a staging buffer, at one read + one write per moved byte.
//  * finalize (last layer): events, freed blocks, block-table and slot rewrite;
//    its own one-wave-per-sequence launch, or, on the fused path, done inside
//    the step's launch by the last (sequence, KV head) workgroup of each
//    sequence to arrive (self-resetting arrival counters, no fences).
#include "nkv_common.h"

namespace nkv {

constexpr int kCD = 128;      // head_dim of the fused kernels
// head_dim of the general path (score and compaction kernels): 64, 128 or 256
constexpr bool compress_dim_ok(int D) { return D == 64 || D == 128 || D == 256; }
constexpr int kChunk = 256;   // keys per scoring workgroup
constexpr int kMaxWindowBlocks = 64;
constexpr int kMaxRows = 1024;  // rows per read-then-write round of a compaction unit

// ------------------------------------------------------------------ score
// scores[j][h][t] for t < Lw (window tokens); t == 0 and t >= n_cand are -inf
// (sink mask; the query-window tokens are not scored: n_cand = Lw - query window).
// G query rows per KV head, any number (16 per MFMA pass): a query window of w
// tokens per head is G = heads x w rows, consecutive per head (q row stride = the
// row of one sequence).
// F8: K is fp8 (OCP E4M3FN) codes, widened to bf16 (exact) on load; the K scale is
// folded into scale_log2 by the caller. D: head_dim (64, 128 or 256).
template <bool F8, int D, bool H16 = false>
__global__ __launch_bounds__(256) void compress_score_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride, const void* __restrict__ k,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t max_blocks,
    const int32_t* __restrict__ base_context_lens, const int32_t* __restrict__ seq_idx,
    int32_t Hk, int32_t G, int32_t block_size, int32_t window_blocks, int64_t n_blocks,
    float scale_log2, int32_t n_cand, float* __restrict__ scores) {
  static_assert(compress_dim_ok(D), "head_dim 64, 128 or 256");
  static_assert(!(F8 && H16), "fp8 caches are scored with bf16 queries");
  constexpr int kEl = F8 ? 1 : 2;
  constexpr int kLpr = D * kEl / 16;  // lanes per K row (16-byte loads)
  constexpr int kRpl = 64 / kLpr;     // K rows per load
  constexpr int kNld = 16 / kRpl;     // loads per 16-key group
  constexpr int kKs = D / 32;         // k-steps of the product
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int Lw = window_blocks * block_size;
  const int n_chunks = (Lw + kChunk - 1) / kChunk;  // the last one masked past Lw (contiguous K)
  const int c = blockIdx.x % n_chunks;
  const int kvh = (blockIdx.x / n_chunks) % Hk;
  const int j = blockIdx.x / (n_chunks * Hk);
  const int Hq = Hk * G;
  const int t0 = c * kChunk;

  int64_t base;            // element offset of key t0 (this KV head)
  int64_t tok_stride;      // elements between consecutive keys
  int64_t qrow;
  bool valid = true;
  if (block_tables) {
    const int seq = seq_idx[j];
    const int len = seq >= 0 ? base_context_lens[seq] : 0;  // seq -1: padding entry
    const int full = len / block_size;
    const int wblk = full - window_blocks + t0 / block_size;
    int64_t pb = -1;
    if (full >= window_blocks && full <= max_blocks)
      pb = block_tables[(int64_t)seq * bt_row_stride + wblk];
    NKV_DBG(seq >= 0 && full >= window_blocks && full <= max_blocks && (pb < 0 || pb >= n_blocks),
            NKV_DEBUG_BLOCK);
    valid = pb >= 0 && pb < n_blocks;
    base = ((pb * block_size + t0 % block_size) * Hk + kvh) * (int64_t)D;
    tok_stride = (int64_t)Hk * D;
    qrow = seq;
  } else {  // contiguous K [m, Hk, Lw, D]
    base = (((int64_t)j * Hk + kvh) * Lw + t0) * D;
    tok_stride = D;
    qrow = j;
  }
  float* srow = scores + ((int64_t)j * Hq + (int64_t)kvh * G) * Lw + t0;
  if (!valid) {
    for (int i = threadIdx.x; i < G * kChunk; i += blockDim.x)
      if (t0 + i % kChunk < Lw) srow[(int64_t)(i / kChunk) * Lw + i % kChunk] = -INFINITY;
    return;
  }
  // K rows are read whole (one head row per kLpr lanes: at head_dim 128, 256 bytes per
  // 16 lanes for bf16, 128 bytes per 8 lanes for fp8), staged row-major in LDS as bf16
  // and re-read in the MFMA operand layout (lane l: key l%16, dims 8*(l/16) + 32ks).
  constexpr int kSR = D + 8;
  __shared__ __attribute__((aligned(16))) bf16_t stage_all[4][16 * kSR];
  bf16_t* stage = stage_all[wave];
  u32x4_t kraw[4][kNld];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int r = 0; r < kNld; ++r) {
      const int key = wave * 64 + g * 16 + kRpl * r + lane / kLpr;
      kraw[g][r] = u32x4_t{0u, 0u, 0u, 0u};
      if (t0 + key < Lw) {  // keys past the window (a contiguous tail chunk) read as 0
        if constexpr (F8) {
          kraw[g][r] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint8_t*>(k) + base +
                                                        key * tok_stride + (lane % kLpr) * 16);
        } else {
          kraw[g][r] = *reinterpret_cast<const u32x4_t*>(static_cast<const bf16_t*>(k) + base +
                                                        key * tok_stride + (lane % kLpr) * 8);
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads issued before the first MFMA
  u32x4_t qreg[kKs];
  auto load_q = [&](int h0) {  // query rows h0 .. h0+15 of the KV head as the MFMA A operand
    const int hr = h0 + (lane & 15);
    const int hc = hr < G ? hr : 0;  // MFMA rows >= G are computed and discarded
    const bf16_t* qp = q + qrow * q_row_stride + (int64_t)(kvh * G + hc) * D + (lane >> 4) * 8;
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) qreg[ks] = *reinterpret_cast<const u32x4_t*>(qp + ks * 32);
  };
  load_q(0);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if constexpr (F8) {
#pragma unroll
      for (int r = 0; r < kNld; ++r) {
        u32x4_t lo, hi;
        fp8x16_to_bf16(kraw[g][r], lo, hi);
        bf16_t* d = &stage[(kRpl * r + lane / kLpr) * kSR + (lane % kLpr) * 16];
        *reinterpret_cast<u32x4_t*>(d) = lo;
        *reinterpret_cast<u32x4_t*>(d + 8) = hi;
      }
    } else {
#pragma unroll
      for (int r = 0; r < kNld; ++r)
        *reinterpret_cast<u32x4_t*>(&stage[(kRpl * r + lane / kLpr) * kSR + (lane % kLpr) * 8]) =
            kraw[g][r];
    }
    const int tw = wave * 64 + g * 16 + (lane & 15);
    const int t = t0 + tw;
    for (int h0 = 0; h0 < G; h0 += 16) {  // uniform; one pass for G <= 16
      if (h0 > 0 || g > 0) {
        if (G > 16) load_q(h0);
      }
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kKs; ++ks) {
        const u32x4_t kb = *reinterpret_cast<const u32x4_t*>(
            &stage[(lane & 15) * kSR + (lane >> 4) * 8 + ks * 32]);
        acc = mfma_16x16x32<H16>(qreg[ks], kb, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = h0 + (lane >> 4) * 4 + r;
        if (h < G && t < Lw)
          srow[(int64_t)h * Lw + tw] = (t == 0 || t >= n_cand) ? -INFINITY : acc[r] * scale_log2;
      }
    }
  }
}

// -------------------------------------------------------------- importance
// importance[r][t] (t < n_cand) for kept set r = j*n_sets + s, heads of the set
// are [s*hps, (s+1)*hps) with hps = Hq / n_sets (query rows: heads x query window).
__global__ __launch_bounds__(256) void compress_importance_kernel(
    const float* __restrict__ scores, int32_t Hq, int32_t n_sets, int32_t Lw, int32_t n_cand,
    float* __restrict__ importance) {
  extern __shared__ float stats[];  // [hps][2]: max, 1/sum
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = blockIdx.x;
  const int j = r / n_sets, s = r % n_sets;
  const int hps = Hq / n_sets;
  const float* sbase = scores + ((int64_t)j * Hq + (int64_t)s * hps) * Lw;
  for (int h = wave; h < hps; h += 4) {
    const float* sr = sbase + (int64_t)h * Lw;
    float mx = -INFINITY;
    for (int t = lane; t < Lw; t += 64) mx = fmaxf(mx, sr[t]);
    mx = wave_max(mx);
    float sum = 0.f;
    if (mx != -INFINITY)
      for (int t = lane; t < Lw; t += 64) sum += fast_exp2(sr[t] - mx);
    sum = wave_sum(sum);
    if (lane == 0) {
      stats[2 * h] = mx;
      stats[2 * h + 1] = sum > 0.f ? 1.f / sum : 0.f;
    }
  }
  __syncthreads();
  float* irow = importance + (int64_t)r * n_cand;
  for (int t = threadIdx.x; t < n_cand; t += blockDim.x) {
    float acc = 0.f;
    for (int h = 0; h < hps; ++h) {
      const float mx = stats[2 * h];
      const float sv = sbase[(int64_t)h * Lw + t];
      if (mx != -INFINITY && sv != -INFINITY) acc += fast_exp2(sv - mx) * stats[2 * h + 1];
    }
    irow[t] = acc;
  }
}

// ------------------------------------------------------------------- top-k
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int wave_excl_scan_i(int v) {
  const int lane = threadIdx.x & 63;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x - v;
}

// One wavefront per row; lane l holds candidates [l*ITEMS, (l+1)*ITEMS).
template <int ITEMS>
__global__ __launch_bounds__(64) void compress_topk_kernel(
    const float* __restrict__ importance, int32_t n_cand, int32_t num_keep, int32_t n_tail,
    int32_t* __restrict__ keep_idx) {
  const int lane = threadIdx.x;
  const int r = blockIdx.x;
  const float* irow = importance + (int64_t)r * n_cand;
  uint32_t key[ITEMS];
#pragma unroll
  for (int e = 0; e < ITEMS; ++e) {
    const int i = lane * ITEMS + e;
    key[e] = (i < n_cand) ? order_key(irow[i]) : 0u;  // padding sorts last
  }
  // k-th largest key by bitwise radix select
  uint32_t T = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < ITEMS; ++e) cnt += key[e] >= cand;
    if (wave_sum_i(cnt) >= num_keep) T = cand;
  }
  int gt = 0, eq = 0;
#pragma unroll
  for (int e = 0; e < ITEMS; ++e) {
    gt += key[e] > T;
    eq += key[e] == T;
  }
  const int need = num_keep - wave_sum_i(gt);  // ties at T taken lowest index first
  int eq_rank = wave_excl_scan_i(eq);
  uint64_t selmask = 0;
#pragma unroll
  for (int e = 0; e < ITEMS; ++e) {
    const int i = lane * ITEMS + e;
    bool sel = key[e] > T;
    if (key[e] == T) {
      sel = eq_rank < need;
      ++eq_rank;
    }
    if (i >= n_cand) sel = false;
    selmask |= (uint64_t)sel << e;
  }
  int pos = wave_excl_scan_i(__builtin_popcountll(selmask));
  int32_t* out = keep_idx + (int64_t)r * (num_keep + 1 + n_tail);
#pragma unroll
  for (int e = 0; e < ITEMS; ++e)
    if (selmask & (1ull << e)) out[1 + pos++] = lane * ITEMS + e;
  if (lane == 0) out[0] = 0;
  for (int i = lane; i < n_tail; i += 64) out[num_keep + 1 + i] = n_cand + i;  // query window
}

// ------------------------------------------------------------- fused step
// One 1024-thread workgroup per (selected sequence, KV head) holds that KV
// head's whole window: wave w scores window keys [64w, 64w + 64) for the G
// query heads of the KV head (K read in place, q K^T on MFMA), so per-head
// softmax statistics are two workgroup reductions and the head sum of the
// group is lane-local plus one permlane step.
//  * agg "group" (compress_group_kernel): the workgroup owns its kept set:
//    score -> select -> (step) compact this KV head's K and V rows. One launch.
//  * agg "all": compress_partial_kernel writes each group's importance; then
//    compress_sum_kernel, per (sequence, KV head), adds the Hk partials in
//    KV-head order (every KV head's workgroup derives the same kept set),
//    selects and compacts. The kernel boundary makes the partials visible
//    across XCDs; a device-scope fence inside a kernel would write back the
//    whole L2.
// Selection: the num_keep-th largest order key is bracketed by 256-bucket histograms of
// the candidates' keys (one candidate per thread, LDS atomics), 8 key bits per level,
// until its bucket holds at most 64 keys, which are ranked exactly; ties to the lower
// index; ascending output by a workgroup prefix count -- no sort. Compaction: every source row of the
// (sequence, KV head) unit, K and V, is loaded into registers before any
// destination is written (the reference's two-phase index_select().clone() /
// index_copy_), one 256-byte row per 16 lanes.
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelKeysPerWave = 64;
constexpr int kSelMaxWindow = kSelWaves * kSelKeysPerWave;  // 1024
constexpr int kStepRounds = 12;                             // 64 rows per round
constexpr int kStepMaxRows = 64 * kStepRounds;              // rows per read-then-write round
// kept + tail rows (< W*B + B <= 2 * 1024), rounded up to whole rounds
constexpr int kStepTable = (2 * kSelMaxWindow + kStepMaxRows - 1) / kStepMaxRows * kStepMaxRows;

constexpr int kStageRow = kCD + 8;  // LDS row stride (elements) of a staged 16-key group

struct SelectLds {
  // per wave: one 16-key group of K rows, row-major (bf16), re-read as MFMA operands
  __attribute__((aligned(16))) bf16_t kstage[kSelWaves][16 * kStageRow];
  float red[kSelWaves][16];
  __attribute__((aligned(16))) float imp[kSelMaxWindow];
  int wcnt[kSelWaves];
  uint32_t wmax[kSelWaves];
  uint32_t wmin[kSelWaves];
  int sel_bucket, sel_above, sel_nb;  // selection: boundary bucket, keys above it, its size
  int32_t keep[kSelMaxWindow];
  int32_t win_pb[kMaxWindowBlocks + 1];
  int32_t sel_hist[256];             // selection: bucket counts
  uint32_t sel_key[kSelMaxWindow];   // selection: keys and indices of the last bucket
  int32_t sel_idx[kSelMaxWindow];
  int32_t src[kStepTable];
  int32_t dst[kStepTable];
};

__device__ __forceinline__ float row16_max(float v) {  // over the 16 lanes of a row
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Exclusive prefix count of `flag` over the workgroup (thread order) + total.
__device__ __forceinline__ int block_excl_count(bool flag, int* wcnt, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t b = __builtin_amdgcn_ballot_w64(flag);
  const int before = __builtin_popcountll(b & ((1ull << lane) - 1ull));
  if (lane == 0) wcnt[wave] = __builtin_popcountll(b);
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const int c = wcnt[w];
    base += w < wave ? c : 0;
    tot += c;
  }
  __syncthreads();  // wcnt is reused by the next call
  total = tot;
  return base + before;
}

// Workgroup barrier ordering LDS only: waits for this wave's LDS operations, not for its
// global loads (a __syncthreads() waits for every outstanding load), so loads issued
// before it stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Selects the num_keep largest of L.imp[0, n_cand) (ties: the lower index) and writes
// [0, ascending kept indices, n_cand] to L.keep and (if out) to out. One candidate per
// thread. The candidates' order-preserving keys are counted into 256 buckets spanning
// [min key, max key] (LDS atomics); one wave finds the bucket holding the num_keep-th
// largest; keys in higher buckets are kept, lower ones dropped, and the bucket is split
// again into 256 (8 more key bits) until it holds at most 64 keys; those are ranked
// exactly by (key, index) against each other (all of them when the keys are equal). Two
// levels for these scores (the masked sink key, importance 0, widens the first level's
// span).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}

__device__ __forceinline__ void block_select(SelectLds& L, int n_cand, int num_keep,
                                             int32_t* __restrict__ out) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool real = tid < n_cand;
  const uint32_t key = real ? order_key(L.imp[tid]) : 0u;
  int* hist = L.sel_hist;
  uint32_t* bkey = L.sel_key;  // members of the last bucket
  int* bidx = L.sel_idx;
  // ---- key range of the candidates
  uint32_t kmax = wave_max_u32(real ? key : 0u);
  uint32_t kmin = wave_min_u32(real ? key : 0xffffffffu);
  if (lane == 0) {
    L.wmax[wave] = kmax;
    L.wmin[wave] = kmin;
  }
  if (tid < 256) hist[tid] = 0;
  if (tid == 0) L.sel_nb = 0;
  lds_barrier();
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    kmax = max(kmax, L.wmax[w]);
    kmin = min(kmin, L.wmin[w]);
  }
  // ---- levels: bucket = (key - lo) >> sh in 0..255 among the keys still undecided
  uint32_t lo = kmin;
  const uint32_t span = kmax - kmin;
  int sh = span == 0 ? 0 : max(0, 32 - __builtin_clz(span) - 8);
  int need = num_keep;  // keys still to take from the undecided ones
  bool active = real, sel = false;
  for (;;) {  // uniform: every thread reads the same bucket and counts
    const int b = active ? (int)((key - lo) >> sh) : -1;
    if (active) atomicAdd(&hist[b], 1);
    lds_barrier();
    if (wave == 0) {  // lane l: buckets 255-4l .. 252-4l, scanned from the top
      int h[4], sum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[i] = hist[255 - 4 * lane - i];
        hist[255 - 4 * lane - i] = 0;  // ready for the next level (ordered by the barrier)
        sum += h[i];
      }
      int incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      int before = incl - sum;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (before < need && before + h[i] >= need) {  // exactly one (bucket, lane)
          L.sel_bucket = 255 - 4 * lane - i;
          L.sel_above = before;
          L.sel_nb = h[i];
        }
        before += h[i];
      }
    }
    lds_barrier();
    const int bb = L.sel_bucket;
    if (active) {
      sel = b > bb;
      active = b == bb;
    }
    need -= L.sel_above;
    if (L.sel_nb <= 64 || sh == 0) break;
    lo += (uint32_t)bb << sh;
    sh = max(sh - 8, 0);
  }
  // ---- the last bucket's members, ranked by (larger key, then lower index)
  if (tid == 0) L.sel_nb = 0;
  lds_barrier();
  if (active) {
    const int slot = atomicAdd(&L.sel_nb, 1);
    bkey[slot] = key;
    bidx[slot] = tid;
  }
  lds_barrier();
  if (active) {
    const int nb = L.sel_nb;
    int rk = 0;
    for (int i = 0; i < nb; ++i) {
      const uint32_t k2 = bkey[i];
      rk += k2 > key || (k2 == key && bidx[i] < tid);
    }
    sel = rk < need;
  }
  // ---- kept positions: exclusive count of the kept keys before each (index order)
  const uint64_t bs = __builtin_amdgcn_ballot_w64(sel);
  if (lane == 0) L.wcnt[wave] = __builtin_popcountll(bs);
  lds_barrier();
  int pos = __builtin_popcountll(bs & ((1ull << lane) - 1ull));
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) pos += w < wave ? L.wcnt[w] : 0;
  if (sel) {
    L.keep[1 + pos] = tid;
    if (out) out[1 + pos] = tid;
  }
  if (tid == 0) {
    L.keep[0] = 0;
    L.keep[num_keep + 1] = n_cand;
    if (out) {
      out[0] = 0;
      out[num_keep + 1] = n_cand;
    }
  }
  lds_barrier();
}

// Window of (sequence j, KV head kvh): the importance of each key summed over
// the G query heads of the group, for this thread's keys t0 + 16g + col
// (valid in lanes of row group 0). Uses L.red.
// F8: the cache holds fp8 (OCP E4M3FN) codes, 128-byte head rows read by 8 lanes (8 rows
// per load) and widened to bf16 when staged; the K scale is folded into scale_log2.
template <bool F8, bool H16>
__device__ __forceinline__ void group_importance(
    SelectLds& L, const bf16_t* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ k, const int32_t* __restrict__ block_tables,
    int64_t bt_row_stride, int32_t max_blocks, const int32_t* __restrict__ base_context_lens,
    const int32_t* __restrict__ seq_idx, int j, int kvh, int Hk, int G, int block_size,
    int window_blocks, int64_t n_blocks, float scale_log2, float gi[4]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hg = lane >> 4;   // MFMA row group: heads 4hg .. 4hg+3
  const int col = lane & 15;  // key within a 16-key group
  const int Lw = window_blocks * block_size;
  const int t0 = wave * kSelKeysPerWave;
  // ---- locate this wave's 64 keys (one cache block holds them all)
  int64_t base = 0, tok_stride, qrow;
  bool valid = t0 < Lw;
  if (block_tables) {
    const int seq = seq_idx[j];
    // the table row's first 128 entries (two per lane) are loaded with the length, so the
    // wave's block id needs no round trip after it
    const int32_t* bt_row = block_tables + (int64_t)(seq >= 0 ? seq : 0) * bt_row_stride;
    const int32_t e0 = (seq >= 0 && lane < max_blocks) ? bt_row[lane] : -1;
    const int32_t e1 = (seq >= 0 && lane + 64 < max_blocks) ? bt_row[lane + 64] : -1;
    const int len = seq >= 0 ? base_context_lens[seq] : 0;  // seq -1: padding entry
    const int full = len / block_size;
    int64_t pb = -1;
    if (valid && full >= window_blocks && full <= max_blocks) {
      const int e = full - window_blocks + t0 / block_size;  // wave-uniform entry
      pb = e < 64    ? __builtin_amdgcn_readlane(e0, e)
           : e < 128 ? __builtin_amdgcn_readlane(e1, e - 64)
                     : bt_row[e];
    }
    NKV_DBG(valid && seq >= 0 && full >= window_blocks && full <= max_blocks &&
                (pb < 0 || pb >= n_blocks),
            NKV_DEBUG_BLOCK);
    valid = valid && pb >= 0 && pb < n_blocks;
    base = ((pb * block_size + t0 % block_size) * Hk + kvh) * (int64_t)kCD;
    tok_stride = (int64_t)Hk * kCD;
    qrow = seq;
  } else {  // contiguous K [m, Hk, Lw, D]
    base = (((int64_t)j * Hk + kvh) * Lw + t0) * kCD;
    tok_stride = kCD;
    qrow = j;
  }
  f32x4_t acc[4] = {};
  if (valid) {  // wave-uniform
    // K rows are read whole: load r of group g brings keys 16g + 4r .. +3, one 256-byte
    // head row per 16 lanes (lane l: key 16g + 4r + l/16, dims 8*(l%16)), so every load
    // instruction is 4 row-sized requests; each group is staged row-major in LDS and
    // re-read in the MFMA operand layout (lane l: key l%16, dims 8*(l/16) + 32ks).
    constexpr int kLd = F8 ? 2 : 4;  // loads per 16-key group
    u32x4_t kreg[4][kLd];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int r = 0; r < kLd; ++r) {
        if constexpr (F8) {
          const uint8_t* kp = static_cast<const uint8_t*>(k) + base +
                              (g * 16 + 8 * r + (lane >> 3)) * tok_stride + (lane & 7) * 16;
          kreg[g][r] = *reinterpret_cast<const u32x4_t*>(kp);
        } else {
          const bf16_t* kp = static_cast<const bf16_t*>(k) + base +
                             (g * 16 + 4 * r + hg) * tok_stride + col * 8;
          kreg[g][r] = *reinterpret_cast<const u32x4_t*>(kp);
        }
      }
    }
    u32x4_t qreg[4];
    const int hc = col < G ? col : 0;  // MFMA rows >= G are computed and discarded
    const bf16_t* qp = q + qrow * q_row_stride + (int64_t)(kvh * G + hc) * kCD + hg * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qreg[ks] = *reinterpret_cast<const u32x4_t*>(qp + ks * 32);
    bf16_t* stage = L.kstage[wave];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if constexpr (F8) {
#pragma unroll
        for (int r = 0; r < kLd; ++r) {
          u32x4_t lo, hi;
          fp8x16_to_bf16(kreg[g][r], lo, hi);
          bf16_t* d = &stage[(8 * r + (lane >> 3)) * kStageRow + (lane & 7) * 16];
          *reinterpret_cast<u32x4_t*>(d) = lo;
          *reinterpret_cast<u32x4_t*>(d + 8) = hi;
        }
      } else {
#pragma unroll
        for (int r = 0; r < kLd; ++r)
          *reinterpret_cast<u32x4_t*>(&stage[(4 * r + hg) * kStageRow + col * 8]) = kreg[g][r];
      }
      f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4_t kb =
            *reinterpret_cast<const u32x4_t*>(&stage[col * kStageRow + hg * 8 + ks * 32]);
        a = mfma_16x16x32<H16>(qreg[ks], kb, a);
      }
      acc[g] = a;
    }
  }
  // log2-domain scores; -inf for the sink (t = 0), the unscored last token,
  // invalid keys and the discarded MFMA rows (heads >= G)
  float sv[4][4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int t = t0 + g * 16 + col;
    const bool key_ok = valid && t > 0 && t < Lw - 1;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sv[g][r] = (key_ok && 4 * hg + r < G) ? acc[g][r] * scale_log2 : -INFINITY;
  }
  // ---- per-head softmax statistics over the window (heads 4hg + r)
  float hm[4], hinv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = row16_max(fmaxf(fmaxf(sv[0][r], sv[1][r]), fmaxf(sv[2][r], sv[3][r])));
    if (col == 0) L.red[wave][4 * hg + r] = v;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) v = fmaxf(v, L.red[w][4 * hg + r]);
    hm[r] = v;
  }
  __syncthreads();
  float p[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float ssum = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      p[g][r] = (sv[g][r] == -INFINITY) ? 0.f : fast_exp2(sv[g][r] - hm[r]);
      ssum += p[g][r];
    }
    ssum = row16_sum(ssum);
    if (col == 0) L.red[wave][4 * hg + r] = ssum;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) v += L.red[w][4 * hg + r];
    hinv[r] = v > 0.f ? 1.f / v : 0.f;
  }
  // ---- the group's importance per key (heads summed in order)
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float v = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) v += p[g][r] * hinv[r];
    gi[g] = col_sum4(v);  // + the other row groups' heads
  }
}

// Slot of logical window position pos (0 .. W*B + B - 2: the window blocks, then the
// tail block) from the unit's block ids, or -1.
__device__ __forceinline__ int64_t window_slot(const int32_t* win_pb, int pos, int B) {
  const int32_t pb = win_pb[pos / B];
  return pb >= 0 ? (int64_t)pb * B + pos % B : -1;
}

// Row i of a compaction unit (i < keep_tokens + tail): source and destination slots, or -1
// for both when either is missing. Kept row i moves from window position keep[i] to
// position i; tail row u = i - keep_tokens moves from offset u of the tail block (logical
// position W*B + u) to logical position keep_tokens + u. Every row moves to a position
// no later than its source, and sources ascend with i (keep[] ascends and ends below W*B),
// so rows can be moved in ascending rounds, each round's reads before its writes: a write
// never lands on a source of a later round.
// The reference places tail row u at physical slot slot(keep_tokens - 1) + 1 + u
// (compress_utils.py:210-231); that is the same slot whenever it stays in the block of
// position keep_tokens - 1, and the block past it (another sequence's) otherwise.
__device__ __forceinline__ void unit_row(const int32_t* win_pb, const int32_t* keep, int i,
                                         int keep_tokens, int nrows, int Lw, int B,
                                         int64_t& src, int64_t& dst) {
  src = dst = -1;
  if (i < keep_tokens) {
    const int pos = keep[i];
    if (pos >= 0 && pos < Lw) src = window_slot(win_pb, pos, B);
    dst = window_slot(win_pb, i, B);
  } else if (i < nrows) {
    src = window_slot(win_pb, Lw + (i - keep_tokens), B);
    dst = window_slot(win_pb, i, B);
  }
  if (src < 0 || dst < 0) src = dst = -1;
}

// Block id of the unit for thread t <= window_blocks (window block t, then the tail block;
// -1 if missing) into pb_out, as a load whose value is first used by the caller; returns
// false (nothing to do) when the sequence is not compressible or its table is too short.
__device__ __forceinline__ bool unit_block_load(const int32_t* __restrict__ bt, int len, int B,
                                                int window_blocks, int max_blocks,
                                                int32_t& pb_out) {
  const int full = len / B;
  const int tail = len - full * B;
  pb_out = -1;
  if (full < window_blocks || full > max_blocks || (tail > 0 && full >= max_blocks))
    return false;
  if ((int)threadIdx.x < window_blocks) pb_out = bt[full - window_blocks + threadIdx.x];
  else if ((int)threadIdx.x == window_blocks && tail > 0) pb_out = bt[full];
  return true;
}

// unit_block_load's id into win_pb (threads t <= window_blocks).
__device__ __forceinline__ void unit_block_store(int32_t* win_pb, int32_t pb, int len, int B,
                                                 int window_blocks, int64_t n_blocks) {
  if ((int)threadIdx.x <= window_blocks) {
    NKV_DBG(((int)threadIdx.x < window_blocks || len % B > 0) && (pb < 0 || pb >= n_blocks),
            NKV_DEBUG_BLOCK);
    win_pb[threadIdx.x] = (pb >= 0 && pb < n_blocks) ? pb : -1;
  }
}

// Both: the block ids of the unit (window blocks, then the tail block or -1) into win_pb.
__device__ __forceinline__ bool unit_blocks(int32_t* win_pb, const int32_t* __restrict__ bt,
                                            int len, int B, int window_blocks, int max_blocks,
                                            int64_t n_blocks) {
  int32_t pb;
  if (!unit_block_load(bt, len, B, window_blocks, max_blocks, pb)) return false;
  unit_block_store(win_pb, pb, len, B, window_blocks, n_blocks);
  return true;
}

// In-place compaction of KV head kvh of sequence seq_idx[j], K and V, with the
// kept window positions in L.keep and the unit's block ids in L.win_pb (unit_blocks,
// visible); kvh 0 also sets the new context length. F8:
// 1-byte rows (a 128-byte head row per 8 lanes, 128 rows per round). Rows go in
// rounds of kStepMaxRows (one for the reference's shapes), all source rows of a
// round in registers before any destination is written.
template <bool F8>
__device__ __forceinline__ void compact_unit(
    SelectLds& L, void* __restrict__ k_cache, void* __restrict__ v_cache,
    const int32_t* __restrict__ base_context_lens, int32_t* __restrict__ context_lens,
    const int32_t* __restrict__ seq_idx, int j, int kvh, int keep_tokens, int Hk, int B,
    int window_blocks) {
  const int tid = threadIdx.x;
  const int seq = seq_idx[j];
  const int len = base_context_lens[seq];
  const int Lw = window_blocks * B;
  const int nrows = keep_tokens + len % B;
  constexpr int kEl = F8 ? 1 : 2;
  constexpr int kLanes = 8 * kEl;                  // 16-byte lanes per head row
  constexpr int kRpr = kSelThreads / kLanes;       // rows per round: 64 (bf16), 128 (fp8)
  constexpr int kRounds = kStepMaxRows / kRpr;     // 12 (bf16), 6 (fp8)
  char* kc = static_cast<char*>(k_cache);
  char* vc = static_cast<char*>(v_cache);
  const int64_t row = (int64_t)Hk * kCD * kEl;    // bytes
  const int64_t col = (int64_t)kvh * kCD * kEl + (tid % kLanes) * 16;
  const int rsub = tid / kLanes;  // row within a round
  // source and destination slot of every row (-1: not moved; rows past nrows too)
  const int n_tab = (nrows + kStepMaxRows - 1) / kStepMaxRows * kStepMaxRows;
  for (int i = tid; i < n_tab; i += kSelThreads) {
    int64_t sv, d;
    unit_row(L.win_pb, L.keep, i, keep_tokens, nrows, Lw, B, sv, d);
    L.src[i] = (int32_t)sv;
    L.dst[i] = (int32_t)d;
  }
  __syncthreads();
  for (int base = 0; base < nrows; base += kStepMaxRows) {  // uniform
    // all source rows (K and V) as unconditional 16-byte loads (rows that are
    // not moved re-read slot 0, always valid), then the writes
    u32x4_t kr[kRounds], vr[kRounds];
#pragma unroll
    for (int rr = 0; rr < kRounds; ++rr) {
      const int64_t sv = max(L.src[base + rr * kRpr + rsub], 0);
      kr[rr] = *reinterpret_cast<const u32x4_t*>(kc + sv * row + col);
      vr[rr] = *reinterpret_cast<const u32x4_t*>(vc + sv * row + col);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);  // all reads of the round land before any write
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < kRounds; ++rr) {
      const int64_t d = L.dst[base + rr * kRpr + rsub];
      if (d >= 0) {
        *reinterpret_cast<u32x4_t*>(kc + d * row + col) = kr[rr];
        *reinterpret_cast<u32x4_t*>(vc + d * row + col) = vr[rr];
      }
    }
  }
  if (kvh == 0 && tid == 0) context_lens[seq] = len - Lw + keep_tokens;
}

// ---------------------------------------------------------------- finalize
// Bookkeeping of one selected sequence, by one wave: the events row, the next token's
// slot and the table row's tail. fin_load reads what it needs (the row's entries from
// keep_blocks on, the first 128 two per lane, and the entry of the next token's block);
// fin_store writes, reading further entries of rows longer than that itself. A caller
// can issue fin_load early and fin_store after every other reader of the row is done.
struct FinRow {
  int32_t seq, len, new_len, keep_blocks, skip;  // uniform over the wave
  int32_t id0, id1;  // entries keep_blocks + lane and keep_blocks + 64 + lane (-1 past the row)
  int32_t pb;        // entry of the block holding position new_len (-1: none)
};

// Arguments of the bookkeeping when a compression step launch carries it.
struct FinArgs {
  int32_t* block_tables;  // the tables the step reads, writable; null: no bookkeeping
  int32_t* slot_mapping;  // optional
  int32_t* events;        // [m, 4 + max_blocks]
  int32_t rewrite_tables;
};

__device__ __forceinline__ FinRow fin_load(const int32_t* __restrict__ bt_row, int seq, int len,
                                           int max_blocks, int keep_tokens, int B,
                                           int window_blocks, int lane) {
  FinRow f;
  f.seq = seq;
  f.len = len;
  const int full = len / B, tail = len - (len / B) * B;
  // the compaction's skip rule: not compressible -> left unchanged; seq -1 (padding) too
  f.skip = seq < 0 || full < window_blocks || full > max_blocks ||
           (tail > 0 && full >= max_blocks);
  f.new_len = len - window_blocks * B + keep_tokens;
  f.keep_blocks = (f.new_len + B - 1) / B;
  f.id0 = f.id1 = f.pb = -1;
  if (!f.skip) {
    const int i0 = f.keep_blocks + lane;
    if (i0 < max_blocks) f.id0 = bt_row[i0];
    if (i0 + 64 < max_blocks) f.id1 = bt_row[i0 + 64];
    const int blk = f.new_len / B;  // kept (blk < keep_blocks) whenever the slot exists
    if (f.new_len % B != 0 && blk < max_blocks) f.pb = bt_row[blk];
  }
  return f;
}

// events row: [seq, new_len, keep_blocks, n_freed, freed ids..., -1...]; a sequence left
// unchanged reads [seq, len, ceil(len/B), -1, -1...] and a padding entry [-1, 0, 0, 0, -1...]
__device__ __forceinline__ void fin_store(const FinRow& f, int32_t* __restrict__ bt_row,
                                          int32_t* __restrict__ ev, int max_blocks, int B,
                                          int rewrite_tables, int32_t* __restrict__ slot_mapping,
                                          int lane) {
  if (f.skip) {
    if (lane == 0) {
      ev[0] = f.seq; ev[1] = f.len; ev[2] = (f.len + B - 1) / B; ev[3] = f.seq >= 0 ? -1 : 0;
    }
    for (int i = lane; i < max_blocks; i += 64) ev[4 + i] = -1;
    return;
  }
  // freed ids (entries >= 0 past the kept blocks, in table order) packed by ballot
  // prefix counts
  int n = 0;  // uniform
  auto pack = [&](int32_t id) {
    const uint64_t valid = __builtin_amdgcn_ballot_w64(id >= 0);
    if (id >= 0) ev[4 + n + __builtin_popcountll(valid & ((1ull << lane) - 1ull))] = id;
    n += __builtin_popcountll(valid);
  };
  pack(f.id0);
  pack(f.id1);
  for (int i0 = f.keep_blocks + 128; i0 < max_blocks; i0 += 64) {
    const int i = i0 + lane;
    pack(i < max_blocks ? bt_row[i] : -1);
  }
  for (int i = n + lane; i < max_blocks; i += 64) ev[4 + i] = -1;
  if (lane == 0) {
    ev[0] = f.seq; ev[1] = f.new_len; ev[2] = f.keep_blocks; ev[3] = n;
    if (slot_mapping) slot_mapping[f.seq] = f.pb < 0 ? -1 : f.pb * B + f.new_len % B;
  }
  if (rewrite_tables)  // after every read of the row (the loads above, in program order)
    for (int i = f.keep_blocks + lane; i < max_blocks; i += 64) bt_row[i] = -1;
}

// One wave per selected sequence.
__global__ __launch_bounds__(64) void compress_finalize_kernel(
    int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t max_blocks,
    const int32_t* __restrict__ base_context_lens, const int32_t* __restrict__ seq_idx,
    int32_t m, int32_t keep_tokens, int32_t block_size, int32_t window_blocks,
    int32_t rewrite_tables, int32_t* __restrict__ slot_mapping, int32_t* __restrict__ events) {
  const int j = blockIdx.x;
  const int lane = threadIdx.x;
  const int seq = seq_idx[j];
  const int len = seq >= 0 ? base_context_lens[seq] : 0;  // seq -1: padding entry
  int32_t* bt = block_tables + (int64_t)(seq >= 0 ? seq : 0) * bt_row_stride;
  const FinRow f = fin_load(bt, seq, len, max_blocks, keep_tokens, block_size, window_blocks,
                            lane);
  fin_store(f, bt, events + (int64_t)j * (4 + max_blocks), max_blocks, block_size,
            rewrite_tables, slot_mapping, lane);
}

// Arrivals of the units of each selected sequence in a step launch that carries the
// bookkeeping (FinArgs): the unit that arrives last does it, after every unit of the
// sequence has read the table row. atomicInc wraps each counter back to 0 at its last
// arrival, so the counters are zero between launches; launches that overlap on one GPU
// share them and must not.
constexpr int kFinMaxSeqs = 16384;
static __device__ uint32_t fin_arrivals[kFinMaxSeqs];

// Called by one thread once every table read of its unit has returned (the reads were
// consumed before a workgroup barrier that precedes the call); true for the last arrival
// of the n_units units of sequence j. The result is needed only at the end of the unit,
// so the round trip overlaps the unit's work.
__device__ __forceinline__ uint32_t fin_arrive(int j, int n_units) {
  return atomicInc(&fin_arrivals[j], (uint32_t)(n_units - 1));
}

// The bookkeeping of a padding entry (seq -1), by wave 0 of its first unit.
__device__ __forceinline__ void fin_padding(const FinArgs& fin, int j, int max_blocks, int B) {
  if (threadIdx.x < 64) {
    const FinRow f = fin_load(nullptr, -1, 0, max_blocks, 0, B, 1, threadIdx.x);
    fin_store(f, nullptr, fin.events + (int64_t)j * (4 + max_blocks), max_blocks, B, 0, nullptr,
              threadIdx.x);
  }
}

// agg "group": score -> select -> (if k_cache_w) compact. Grid m * Hk.
template <bool F8, bool H16 = false>
__global__ __launch_bounds__(kSelThreads) void compress_group_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride, const void* __restrict__ k,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t max_blocks,
    const int32_t* __restrict__ base_context_lens, const int32_t* __restrict__ seq_idx,
    int32_t Hk, int32_t G, int32_t block_size, int32_t window_blocks, int64_t n_blocks, float scale_log2,
    int32_t num_keep, float* __restrict__ importance_out, int32_t* __restrict__ keep_idx,
    void* __restrict__ k_cache_w, void* __restrict__ v_cache_w,
    int32_t* __restrict__ context_lens, FinArgs fin) {
  __shared__ SelectLds L;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int j = blockIdx.x / Hk;
  // workgroups go to the XCDs round-robin: rotating the head by the sequence gives each
  // XCD's L2 every head's 256-byte column of the token rows instead of always the same one
  const int kvh = (blockIdx.x + j) % Hk;
  if (block_tables && seq_idx[j] < 0) {  // padding entry (uniform): nothing else written
    if (fin.block_tables && blockIdx.x % Hk == 0) fin_padding(fin, j, max_blocks, block_size);
    return;
  }
  const int Lw = window_blocks * block_size;
  const int n_cand = Lw - 1;
  float gi[4];
  group_importance<F8, H16>(L, q, q_row_stride, k, block_tables, bt_row_stride, max_blocks,
                       base_context_lens, seq_idx, j, kvh, Hk, G, block_size, window_blocks,
                       n_blocks, scale_log2, gi);
  // compaction: the unit's block ids, loaded now (the selection hides the round trip, and
  // the scoring's chain to its K loads stays short); not compressible or inconsistent with
  // the table width: left untouched
  bool compact = false;
  int32_t wpb = -1;
  const int seq = block_tables ? seq_idx[j] : 0;  // no seq_idx for contiguous K
  const int len = k_cache_w ? base_context_lens[seq] : 0;
  if (k_cache_w)
    compact = unit_block_load(block_tables + (int64_t)seq * bt_row_stride, len, block_size,
                              window_blocks, max_blocks, wpb);
  const int t0 = (tid >> 6) * kSelKeysPerWave;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int t = t0 + g * 16 + (lane & 15);
    if ((lane >> 4) == 0 && t < Lw) L.imp[t] = gi[g];
  }
  __syncthreads();
  float* irow = importance_out + ((int64_t)j * Hk + kvh) * n_cand;
  for (int t = tid; t < n_cand; t += kSelThreads) irow[t] = L.imp[t];
  block_select(L, n_cand, num_keep, keep_idx + ((int64_t)j * Hk + kvh) * (num_keep + 2));
  if (compact) {  // uniform
    unit_block_store(L.win_pb, wpb, len, block_size, window_blocks, n_blocks);
    __syncthreads();
  }
  uint32_t fin_old = 0;  // every table read of the unit has returned (the barriers before)
  FinRow fr{};
  if (fin.block_tables && tid < 64) {
    if (tid == 0) fin_old = fin_arrive(j, Hk);
    // read by every unit, used by the last to arrive: the compaction hides the round trip
    fr = fin_load(fin.block_tables + (int64_t)seq * bt_row_stride, seq, len, max_blocks,
                  num_keep + 2, block_size, window_blocks, lane);
  }
  if (compact)
    compact_unit<F8>(L, k_cache_w, v_cache_w, base_context_lens, context_lens, seq_idx, j, kvh,
                     num_keep + 2, Hk, block_size, window_blocks);
  if (fin.block_tables && tid < 64 &&
      (uint32_t)__builtin_amdgcn_readfirstlane(fin_old) == (uint32_t)(Hk - 1))
    fin_store(fr, fin.block_tables + (int64_t)fr.seq * bt_row_stride,
              fin.events + (int64_t)j * (4 + max_blocks), max_blocks, block_size,
              fin.rewrite_tables, fin.slot_mapping, lane);
}

// agg "all", first kernel: each group's importance -> partial[j][kvh][Lw]. Grid m * Hk.
template <bool F8, bool H16 = false>
__global__ __launch_bounds__(kSelThreads) void compress_partial_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride, const void* __restrict__ k,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t max_blocks,
    const int32_t* __restrict__ base_context_lens, const int32_t* __restrict__ seq_idx,
    int32_t Hk, int32_t G, int32_t block_size, int32_t window_blocks, int64_t n_blocks, float scale_log2,
    float* __restrict__ partial) {
  __shared__ SelectLds L;
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x / Hk;
  const int kvh = (blockIdx.x + j) % Hk;  // rotated as in compress_group_kernel
  if (block_tables && seq_idx[j] < 0) return;  // padding entry (uniform): nothing written
  const int Lw = window_blocks * block_size;
  float gi[4];
  group_importance<F8, H16>(L, q, q_row_stride, k, block_tables, bt_row_stride, max_blocks,
                       base_context_lens, seq_idx, j, kvh, Hk, G, block_size, window_blocks,
                       n_blocks, scale_log2, gi);
  float* prow = partial + ((int64_t)j * Hk + kvh) * Lw;
  const int t0 = (threadIdx.x >> 6) * kSelKeysPerWave;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int t = t0 + g * 16 + (lane & 15);
    if ((lane >> 4) == 0 && t < Lw) prow[t] = gi[g];
  }
}

// agg "all", second kernel: importance[j] = sum over KV heads (in order) of the
// partials, the selection, and (if k_cache_w) the compaction of KV head kvh.
// Grid m (selection only) or m * Hk (step: every KV head derives the same set).
template <bool F8>
__global__ __launch_bounds__(kSelThreads) void compress_sum_kernel(
    const float* __restrict__ partial, int32_t Hk, int32_t n_units_per_seq, int32_t block_size,
    int32_t window_blocks, int32_t num_keep, float* __restrict__ importance_out,
    int32_t* __restrict__ keep_idx, void* __restrict__ k_cache_w,
    void* __restrict__ v_cache_w, const int32_t* __restrict__ block_tables,
    int64_t bt_row_stride, int32_t max_blocks, const int32_t* __restrict__ base_context_lens,
    int32_t* __restrict__ context_lens, const int32_t* __restrict__ seq_idx, int64_t n_blocks,
    FinArgs fin) {
  __shared__ SelectLds L;
  const int tid = threadIdx.x;
  const int j = blockIdx.x / n_units_per_seq;
  const int kvh = (blockIdx.x + j) % n_units_per_seq;  // rotated as in compress_group_kernel
  if (block_tables && seq_idx[j] < 0) {  // padding entry (uniform): nothing else written
    if (fin.block_tables && blockIdx.x % n_units_per_seq == 0)
      fin_padding(fin, j, max_blocks, block_size);
    return;
  }
  const int Lw = window_blocks * block_size;
  const int n_cand = Lw - 1;
  bool compact = false;  // as in compress_group_kernel
  int32_t wpb = -1;
  const int seq = block_tables ? seq_idx[j] : 0;
  const int len = k_cache_w ? base_context_lens[seq] : 0;
  if (k_cache_w)
    compact = unit_block_load(block_tables + (int64_t)seq * bt_row_stride, len, block_size,
                              window_blocks, max_blocks, wpb);
  const float* pj = partial + (int64_t)j * Hk * Lw;
  const bool writer = kvh == 0;
  float* irow = importance_out + (int64_t)j * n_cand;
  for (int t = tid; t < Lw; t += kSelThreads) {
    float v = 0.f;
    for (int h0 = 0; h0 < Hk; h0 += 16) {  // 16 loads in flight, added in KV-head order
      float part[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) part[i] = pj[(int64_t)min(h0 + i, Hk - 1) * Lw + t];
#pragma unroll
      for (int i = 0; i < 16; ++i) v += h0 + i < Hk ? part[i] : 0.f;
    }
    L.imp[t] = v;
    if (writer && t < n_cand) irow[t] = v;
  }
  if (compact) unit_block_store(L.win_pb, wpb, len, block_size, window_blocks, n_blocks);
  __syncthreads();
  uint32_t fin_old = 0;  // the unit's table reads (wave 0's) preceded the barrier
  FinRow fr{};
  if (fin.block_tables && tid < 64) {
    if (tid == 0) fin_old = fin_arrive(j, n_units_per_seq);
    fr = fin_load(fin.block_tables + (int64_t)seq * bt_row_stride, seq, len, max_blocks,
                  num_keep + 2, block_size, window_blocks, tid);  // as in the group kernel
  }
  block_select(L, n_cand, num_keep, writer ? keep_idx + (int64_t)j * (num_keep + 2) : nullptr);
  if (compact)
    compact_unit<F8>(L, k_cache_w, v_cache_w, base_context_lens, context_lens, seq_idx, j, kvh,
                     num_keep + 2, Hk, block_size, window_blocks);
  if (fin.block_tables && tid < 64 &&
      (uint32_t)__builtin_amdgcn_readfirstlane(fin_old) == (uint32_t)(n_units_per_seq - 1))
    fin_store(fr, fin.block_tables + (int64_t)fr.seq * bt_row_stride,
              fin.events + (int64_t)j * (4 + max_blocks), max_blocks, block_size,
              fin.rewrite_tables, fin.slot_mapping, tid);
}

// ----------------------------------------------------------------- compact
// Unit = (selected j, KV head, K|V, 64-dim part of the head row: two at head_dim 128).
// Rows i < keep_tokens move from window position keep_idx[i] to window position i; rows
// keep_tokens + u (u < tail) move from the tail block offset u to window position
// keep + u (unit_row). Rows go in rounds of ROUNDS * rows-per-round, each round's reads
// before its writes. F8: 1-byte (fp8) cache rows: a 64-dim part is 64 bytes, moved by 4
// lanes, so a round covers 64 rows instead of 32.
template <int ROUNDS, bool F8>
__global__ __launch_bounds__(256) void compress_compact_kernel(
    void* __restrict__ k_cache, void* __restrict__ v_cache,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t max_blocks,
    const int32_t* __restrict__ base_context_lens, int32_t* __restrict__ context_lens,
    const int32_t* __restrict__ seq_idx, const int32_t* __restrict__ keep_idx, int32_t n_sets,
    int32_t keep_tokens, int32_t Hk, int32_t head_dim, int32_t block_size,
    int32_t window_blocks, int64_t n_blocks) {
  const int parts = head_dim / 64;  // 64-dim parts per head row
  const int half = blockIdx.x % parts;
  const int is_v = (blockIdx.x / parts) & 1;
  const int kvh = (blockIdx.x / (2 * parts)) % Hk;
  const int j = (blockIdx.x / (2 * parts)) / Hk;
  const int seq = seq_idx[j];
  const int len = seq >= 0 ? base_context_lens[seq] : 0;  // seq -1: padding entry
  const int B = block_size;
  __shared__ int32_t win_pb[kMaxWindowBlocks + 1];
  __shared__ int32_t src_lds[kMaxRows];
  __shared__ int32_t dst_lds[kMaxRows];
  // not compressible, or inconsistent with the table width: leave untouched
  if (!unit_blocks(win_pb, block_tables + (int64_t)seq * bt_row_stride, len, B, window_blocks,
                   max_blocks, n_blocks))
    return;
  __syncthreads();
  const int32_t* kidx = keep_idx + ((int64_t)j * n_sets + (n_sets > 1 ? kvh : 0)) * keep_tokens;
  const int Lw = window_blocks * B;
  const int nrows = keep_tokens + len % B;
  constexpr int kEl = F8 ? 1 : 2;
  constexpr int kLanesPerRow = 4 * kEl;             // 16-byte lanes per 64-dim part
  constexpr int kRowsPerRound = 256 / kLanesPerRow;  // 32 (bf16) or 64 (fp8)
  constexpr int kBatch = ROUNDS * kRowsPerRound;    // rows per read-then-write round
  static_assert(kBatch <= kMaxRows, "compaction table too small");
  char* cache = static_cast<char*>(is_v ? v_cache : k_cache);
  const int64_t row = (int64_t)Hk * head_dim * kEl;  // bytes
  const int64_t col =
      ((int64_t)kvh * head_dim + half * 64) * kEl + (threadIdx.x % kLanesPerRow) * 16;
  const int rsub = threadIdx.x / kLanesPerRow;  // row within a round
  for (int base = 0; base < nrows; base += kBatch) {  // uniform
    // source and destination slot of every row of the round (-1 = row not moved)
    for (int i = threadIdx.x; i < kBatch; i += blockDim.x) {
      int64_t sv, d;
      unit_row(win_pb, kidx, base + i, keep_tokens, nrows, Lw, B, sv, d);
      src_lds[i] = (int32_t)sv;
      dst_lds[i] = (int32_t)d;
    }
    __syncthreads();
    // every source row of the round, as unconditional 128-bit loads (rows that are not
    // moved re-read slot 0, always valid)
    u32x4_t reg[ROUNDS];
#pragma unroll
    for (int rr = 0; rr < ROUNDS; ++rr) {
      const int32_t sv = max(src_lds[rr * kRowsPerRound + rsub], 0);
      reg[rr] = *reinterpret_cast<const u32x4_t*>(cache + (int64_t)sv * row + col);
    }
    __builtin_amdgcn_sched_barrier(0);
    // all reads of the round land before any write (two-phase semantics)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < ROUNDS; ++rr) {
      const int32_t d = dst_lds[rr * kRowsPerRound + rsub];
      if (d >= 0) *reinterpret_cast<u32x4_t*>(cache + (int64_t)d * row + col) = reg[rr];
    }
    if (base + kBatch < nrows) __syncthreads();  // the tables are rebuilt
  }

  if (blockIdx.x % (2 * parts * Hk) == 0 && threadIdx.x == 0)
    context_lens[seq] = len - Lw + keep_tokens;
}

// ----------------------------------------------------------------- schedule
// The compression block of ModelRunner.prepare_decode (model_runner.py:300-332)
// on the device, so a compression step needs no host data: the decode-step
// counter advances; on every period-th step sequence i is eligible iff
// len % B != B - 1, tail_uncompressed >= W*B and len / B >= W; the first topk
// eligible in batch order (policy 0, the reference) or the topk longest
// (policy 1, ties to the lower index) go to seq_idx, the rest is -1; each
// sequence's eligibility key is its length, or -1; base_context_lens receives a
// copy of context_lens.
constexpr int kSchedMaxBatch = 16384;  // eligibility keys staged in LDS (64 KiB)
constexpr int kSchedSlots = 16;                      // sequences per lane, one-wave kernel
constexpr int kSchedRegBatch = 64 * kSchedSlots;     // batches up to this: one wave

__device__ __forceinline__ int sched_count(uint64_t m) { return __builtin_popcountll(m); }
// Lanes below this one with their bit set in m.
__device__ __forceinline__ int sched_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Batches up to kSchedRegBatch: one wave, no workgroup barriers. Lane l holds sequences
// l + 64 s (s < kSlots: 8 up to batch 512, 16 above) in registers, all their loads issued
// together; every count is
// a ballot over the wave. Policy 1 finds the take-th largest eligible length T bit by bit
// (the largest T with at least `take` keys >= T), takes the keys above T and the
// lowest-indexed ones equal to it, and ranks them (longest first, ties to the lower index)
// with lane reads of the candidates when there are at most 64, through LDS otherwise.
template <int kSlots>  // sequences per lane: batch <= 64 * kSlots
__global__ __launch_bounds__(64) void compress_schedule_wave_kernel(
    const int32_t* __restrict__ context_lens, const int32_t* __restrict__ tail_uncompressed,
    int32_t batch, int32_t block_size, int32_t window_blocks, int32_t topk, int32_t period,
    int32_t policy, int32_t* __restrict__ step_counter, int32_t* __restrict__ seq_idx,
    int32_t* __restrict__ n_selected, int32_t* __restrict__ base_context_lens) {
  __shared__ int32_t cand[64 * kSlots];   // policy 1: the selected sequences, index order
  __shared__ int32_t candk[64 * kSlots];  // and their lengths
  const int lane = threadIdx.x;
  int c = 0;
  if (lane == 0) c = step_counter[0];
  int len[kSlots], tail[kSlots];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    const int i = s * 64 + lane;
    len[s] = i < batch ? context_lens[i] : 0;
    tail[s] = i < batch ? tail_uncompressed[i] : 0;
  }
  c = __builtin_amdgcn_readfirstlane(c) + 1;
  if (lane == 0) step_counter[0] = c;
  const bool fire = c % period == 0;  // period > 0 (checked by the caller)
  const int B = block_size;
  const int min_tail = window_blocks * B;
  int key[kSlots];
  int n_elig = 0, mx = 0;
  const bool pow2 = (B & (B - 1)) == 0;  // uniform: shifts instead of divisions
  const int b_log2 = __builtin_ctz((unsigned)B);
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    const int i = s * 64 + lane;
    if (base_context_lens && i < batch) base_context_lens[i] = len[s];
    const int nb = pow2 ? len[s] >> b_log2 : len[s] / B;  // negative: never eligible
    const int rem = len[s] - nb * B;
    const bool ok = i < batch && fire && rem != B - 1 && tail[s] >= min_tail &&
                    nb >= window_blocks;
    key[s] = ok ? len[s] : -1;
    n_elig += sched_count(__builtin_amdgcn_ballot_w64(ok));
    mx = max(mx, key[s]);
  }
  const int take = min(n_elig, topk);
  if (lane == 0) n_selected[0] = take;
  for (int r = take + lane; r < topk; r += 64) seq_idx[r] = -1;  // unused slots
  if (take == 0) return;  // uniform
  if (policy == 0) {  // first `take` eligible in batch order
    int rank = 0;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      const uint64_t m = __builtin_amdgcn_ballot_w64(key[s] >= 0);
      const int pos = rank + sched_below(m);
      if (key[s] >= 0 && pos < take) seq_idx[pos] = s * 64 + lane;
      rank += sched_count(m);
    }
    return;
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) mx = max(mx, __shfl_xor(mx, o, 64));
  mx = __builtin_amdgcn_readfirstlane(mx);
  // T: the largest value with at least `take` eligible keys >= T
  int T = 0;
  for (int bit = 31 - __builtin_clz((uint32_t)mx | 1u); bit >= 0; --bit) {  // uniform
    const int t = T | (1 << bit);
    int cnt = 0;  // uniform: ballots and scalar bit counts, no cross-lane data movement
#pragma unroll
    for (int s = 0; s < kSlots; ++s) cnt += sched_count(__builtin_amdgcn_ballot_w64(key[s] >= t));
    if (cnt >= take) T = t;
  }
  // the keys above T, then the lowest-indexed ones equal to T, in index order
  int n_gt = 0;
#pragma unroll
  for (int s = 0; s < kSlots; ++s) n_gt += sched_count(__builtin_amdgcn_ballot_w64(key[s] > T));
  int ties = take - n_gt;  // > 0
  int pos = 0;
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    const int k = key[s];
    const uint64_t meq = __builtin_amdgcn_ballot_w64(k == T);
    const bool sel = k > T || (k == T && sched_below(meq) < ties);
    const uint64_t msel = __builtin_amdgcn_ballot_w64(sel);
    const int p = pos + sched_below(msel);
    if (sel) {
      cand[p] = s * 64 + lane;
      candk[p] = k;
    }
    pos += sched_count(msel);
    ties -= min(sched_count(meq), ties);
  }
  __syncthreads();
  if (take <= 64) {
    const int my_cand = lane < take ? cand[lane] : -1;  // candidate `lane`
    const int my_key = lane < take ? candk[lane] : -1;
    int rank = 0;
    for (int t = 0; t < take; ++t) {  // uniform
      const int j = __builtin_amdgcn_readlane(my_cand, t);
      const int lj = __builtin_amdgcn_readlane(my_key, t);
      rank += lj > my_key || (lj == my_key && j < my_cand);
    }
    if (lane < take) seq_idx[rank] = my_cand;
    return;
  }
  // longest first, ties to the lower index
  for (int r = lane; r < take; r += 64) {
    const int i = cand[r];
    const int li = candk[r];
    int rank = 0;
    for (int t = 0; t < take; ++t) {
      const int j = cand[t];
      const int lj = candk[t];
      rank += lj > li || (lj == li && j < i);
    }
    seq_idx[rank] = i;
  }
}

constexpr int kSchedThreads = 1024;

// Exclusive prefix sum of v over the workgroup in thread order; *total gets the sum.
// Wave scans with shuffles, then the 16 wave totals through LDS (two barriers).
__device__ __forceinline__ int sched_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < kSchedThreads / 64; ++k) {
    const int t = wsum[k];
    off += k < w ? t : 0;
    tot += t;
  }
  *total = tot;
  __syncthreads();  // wsum is reused by the next scan
  return off + incl - v;
}

// Batches above kSchedRegBatch: one 1024-thread workgroup, each thread owning a contiguous
// range of sequences. Policy 1 finds the topk-th largest length with a 4-bit radix select,
// takes the sequences above it and the lowest-indexed ones equal to it, and ranks only those
// (written longest first).
__global__ __launch_bounds__(kSchedThreads) void compress_schedule_kernel(
    const int32_t* __restrict__ context_lens, const int32_t* __restrict__ tail_uncompressed,
    int32_t batch, int32_t block_size, int32_t window_blocks, int32_t topk, int32_t period,
    int32_t policy, int32_t* __restrict__ step_counter, int32_t* __restrict__ seq_idx,
    int32_t* __restrict__ n_selected, int32_t* __restrict__ base_context_lens) {
  __shared__ int32_t key[kSchedMaxBatch];   // length if eligible, else -1
  __shared__ int32_t cand[kSchedMaxBatch];  // policy 1: the selected sequences, index order
  __shared__ int32_t wsum[kSchedThreads / 64];
  __shared__ int32_t hist[16];
  __shared__ uint32_t sh_prefix;
  __shared__ int32_t sh_need;
  __shared__ int32_t sh_max;  // longest eligible length
  __shared__ int32_t fire;
  const int tid = threadIdx.x;
  if (tid == 0) {
    const int c = step_counter[0] + 1;
    step_counter[0] = c;
    fire = period > 0 && c % period == 0;
    sh_max = 0;
  }
  for (int r = tid; r < topk; r += kSchedThreads) seq_idx[r] = -1;
  __syncthreads();
  const int B = block_size;
  for (int i = tid; i < batch; i += kSchedThreads) {
    const int len = context_lens[i];
    if (base_context_lens) base_context_lens[i] = len;
    const bool ok = fire && len % B != B - 1 &&
                    tail_uncompressed[i] >= window_blocks * B && len / B >= window_blocks;
    key[i] = ok ? len : -1;
    if (ok && policy == 1) atomicMax(&sh_max, len);
  }
  __syncthreads();
  const int per = (batch + kSchedThreads - 1) / kSchedThreads;
  const int i0 = min(batch, tid * per), i1 = min(batch, i0 + per);
  int cnt = 0;
  for (int i = i0; i < i1; ++i) cnt += key[i] >= 0;
  int n_elig;
  const int before = sched_scan(cnt, wsum, &n_elig);
  const int take = min(n_elig, topk);
  if (tid == 0) n_selected[0] = take;
  if (policy == 0) {  // first topk in batch order
    int rank = before;
    for (int i = i0; i < i1 && rank < topk; ++i)
      if (key[i] >= 0) seq_idx[rank++] = i;
    return;
  }
  if (take == 0) return;  // uniform
  // topk longest. T = the take-th largest eligible length, 4 bits a pass from the highest
  // nibble any eligible length uses; need = how many sequences of length T are taken (the
  // lowest indices).
  uint32_t prefix = 0;
  int need = take;
  const int top_bit = 31 - __builtin_clz((uint32_t)sh_max | 1u);
  for (int shift = top_bit & ~3; shift >= 0; shift -= 4) {
    if (tid < 16) hist[tid] = 0;
    __syncthreads();
    const uint32_t hi = shift >= 28 ? 0u : ~((1u << (shift + 4)) - 1u);  // digits already fixed
    for (int i = tid; i < batch; i += kSchedThreads) {
      const int k = key[i];
      if (k >= 0 && ((uint32_t)k & hi) == prefix) atomicAdd(&hist[((uint32_t)k >> shift) & 15u], 1);
    }
    __syncthreads();
    if (tid < 64) {  // the digit whose bucket holds the need-th largest: suffix sums over 16 lanes
      const int h = tid < 16 ? hist[tid] : 0;
      int incl = h;  // sum of hist[tid .. 15]
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int y = __shfl_down(incl, o, 64);
        if (tid + o < 16) incl += y;
      }
      const int above = incl - h;
      if (tid < 16 && above < need && incl >= need) {
        sh_prefix = prefix | ((uint32_t)tid << shift);
        sh_need = need - above;
      }
    }
    __syncthreads();
    prefix = sh_prefix;
    need = sh_need;
  }
  const int T = (int)prefix;
  int ties = 0;
  for (int i = i0; i < i1; ++i) ties += key[i] == T;
  int tie_total;
  const int tie_before = sched_scan(ties, wsum, &tie_total);
  int nsel = 0;
  {
    int tr = tie_before;
    for (int i = i0; i < i1; ++i) {
      const int k = key[i];
      nsel += k > T || (k == T && tr < need);
      tr += k == T;
    }
  }
  int sel_total;
  int pos = sched_scan(nsel, wsum, &sel_total);  // sel_total == take
  {
    int tr = tie_before;
    for (int i = i0; i < i1; ++i) {
      const int k = key[i];
      if (k > T || (k == T && tr < need)) cand[pos++] = i;
      tr += k == T;
    }
  }
  __syncthreads();
  // longest first, ties to the lower index
  for (int r = tid; r < take; r += kSchedThreads) {
    const int i = cand[r];
    const int li = key[i];
    int rank = 0;
    for (int t = 0; t < take; ++t) {
      const int j = cand[t];
      const int lj = key[j];
      rank += lj > li || (lj == li && j < i);
    }
    seq_idx[rank] = i;
  }
}

}  // namespace nkv

// ============================================================= C ABI
using namespace nkv;

namespace nkv {
// The score kernel's head_dim instance (64, 128 or 256; checked by the caller).
template <bool F8, bool H16 = false>
static void launch_score(int32_t head_dim, unsigned grid, hipStream_t s, const bf16_t* q,
                         int64_t q_row_stride, const void* k, const int32_t* block_tables,
                         int64_t bt_row_stride, int32_t max_blocks,
                         const int32_t* base_context_lens, const int32_t* seq_idx, int32_t Hk,
                         int32_t G, int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                         float scale_log2, int32_t n_cand, float* scores) {
#define NKV_SCORE_LAUNCH(D)                                                                    \
  hipLaunchKernelGGL((compress_score_kernel<F8, D, H16>), dim3(grid), dim3(256), 0, s, q,        \
                     q_row_stride, k, block_tables, bt_row_stride, max_blocks,                   \
                     base_context_lens, seq_idx, Hk, G, block_size, window_blocks, n_blocks,     \
                     scale_log2, n_cand, scores)
  if (head_dim == 64) NKV_SCORE_LAUNCH(64);
  else if (head_dim == 128) NKV_SCORE_LAUNCH(128);
  else NKV_SCORE_LAUNCH(256);
#undef NKV_SCORE_LAUNCH
}
}  // namespace nkv

extern "C" size_t nkv_compress_workspace_bytes(int32_t m, int32_t n_q_heads,
                                               int32_t window_blocks, int32_t block_size) {
  if (m <= 0 || n_q_heads <= 0 || window_blocks <= 0 || block_size <= 0) return 0;
  return (size_t)m * n_q_heads * window_blocks * block_size * sizeof(float);
}

namespace nkv {
template <bool H16>
static int compress_score_impl(const void* q, int64_t q_row_stride, const void* k_cache,
                               const int32_t* block_tables, int64_t bt_row_stride,
                               int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                               const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                               int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t window_blocks, int64_t n_blocks, float scale,
                               int32_t agg_mode, float* importance_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  NKV_REQUIRE(m >= 0 && n_q_heads > 0 && n_kv_heads > 0 && window_blocks > 0 && block_size > 0,
              NKV_EINVAL, "compress_score: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(compress_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "compress_score: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "compress_score: Hq %% Hk != 0");
  const int g = n_q_heads / n_kv_heads;  // any group: query rows in passes of 16
  NKV_REQUIRE(!block_tables || block_size % kChunk == 0, NKV_EUNSUPPORTED,
              "compress_score: block_size must be a multiple of 256");
  NKV_REQUIRE(agg_mode == NKV_AGG_ALL || agg_mode == NKV_AGG_GROUP, NKV_EINVAL,
              "compress_score: bad agg_mode %d", agg_mode);
  NKV_REQUIRE(q && k_cache && importance_out, NKV_EINVAL, "compress_score: null pointer");
  NKV_REQUIRE(!block_tables || (seq_idx && base_context_lens && max_blocks_per_seq > 0 &&
                                 bt_row_stride >= max_blocks_per_seq),
              NKV_EINVAL, "compress_score: paged mode needs seq_idx, base_context_lens and a "
              "block table width");
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && q_row_stride % 8 == 0, NKV_EINVAL,
              "compress_score: q/k must be 16-byte aligned");
  const size_t need = nkv_compress_workspace_bytes(m, n_q_heads, window_blocks, block_size);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "compress_score: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  const int Lw = window_blocks * block_size;
  NKV_REQUIRE(Lw >= 2, NKV_EINVAL, "compress_score: window too short");
  float* scores = (float*)workspace;
  hipStream_t s = as_stream(stream);
  const unsigned grid = (unsigned)(m * n_kv_heads * ((Lw + kChunk - 1) / kChunk));
  const float sl2 = scale * kLog2e;
  launch_score<false, H16>(head_dim, grid, s, (const bf16_t*)q, q_row_stride, k_cache,
                           block_tables, bt_row_stride, max_blocks_per_seq, base_context_lens,
                           seq_idx, n_kv_heads, g, block_size, window_blocks, n_blocks, sl2,
                           Lw - 1, scores);
  int rc = check_launch("nkv_compress_score");
  if (rc) return rc;
  const int n_sets = agg_mode == NKV_AGG_ALL ? 1 : n_kv_heads;
  const int hps = n_q_heads / n_sets;
  hipLaunchKernelGGL(compress_importance_kernel, dim3((unsigned)(m * n_sets)), dim3(256),
                     (size_t)hps * 2 * sizeof(float), s, scores, n_q_heads, n_sets, Lw, Lw - 1,
                     importance_out);
  return check_launch("nkv_compress_score(importance)");
}
}  // namespace nkv

extern "C" int nkv_compress_score(const void* q, int64_t q_row_stride, const void* k_cache,
                                  const int32_t* block_tables, int64_t bt_row_stride,
                                  int32_t max_blocks_per_seq,
                                  const int32_t* base_context_lens, const int32_t* seq_idx,
                                  int32_t m, int32_t n_q_heads, int32_t n_kv_heads,
                                  int32_t head_dim, int32_t block_size, int32_t window_blocks,
                                  int64_t n_blocks, float scale, int32_t agg_mode,
                                  float* importance_out, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  clear_error();
  return compress_score_impl<false>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                                    max_blocks_per_seq, base_context_lens, seq_idx, m, n_q_heads,
                                    n_kv_heads, head_dim, block_size, window_blocks, n_blocks,
                                    scale, agg_mode, importance_out, workspace, workspace_bytes,
                                    stream);
}

extern "C" int nkv_compress_topk(const float* importance, int32_t n_rows, int32_t n_cand,
                                 int32_t num_keep, int32_t* keep_idx, void* stream) {
  clear_error();
  NKV_REQUIRE(n_rows >= 0 && n_cand > 0 && n_cand <= 4096, NKV_EINVAL,
              "compress_topk: need 0 < n_cand <= 4096 (got %d)", n_cand);
  NKV_REQUIRE(num_keep > 0 && num_keep < n_cand, NKV_EINVAL,
              "compress_topk: need 0 < num_keep < n_cand (got %d, %d)", num_keep, n_cand);
  if (n_rows == 0) return NKV_OK;
  NKV_REQUIRE(importance && keep_idx, NKV_EINVAL, "compress_topk: null pointer");
  hipStream_t s = as_stream(stream);
  if (n_cand <= 64 * 16) {
    hipLaunchKernelGGL(compress_topk_kernel<16>, dim3((unsigned)n_rows), dim3(64), 0, s,
                       importance, n_cand, num_keep, 1, keep_idx);
  } else {
    hipLaunchKernelGGL(compress_topk_kernel<64>, dim3((unsigned)n_rows), dim3(64), 0, s,
                       importance, n_cand, num_keep, 1, keep_idx);
  }
  return check_launch("nkv_compress_topk");
}

extern "C" size_t nkv_compress_select_workspace_bytes(int32_t m, int32_t n_q_heads,
                                                      int32_t n_kv_heads, int32_t window_blocks,
                                                      int32_t block_size) {
  if (m <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || window_blocks <= 0 || block_size <= 0)
    return 0;
  const size_t lw = (size_t)window_blocks * block_size;
  const size_t partials = (size_t)m * n_kv_heads * lw * sizeof(float);
  const size_t scores = (size_t)m * n_q_heads * lw * sizeof(float);  // general path
  return partials > scores ? partials : scores;
}

namespace nkv {
// Launches the fused selection (and, with k_cache_w, the compaction) when the
// shape allows it; returns 1 if the caller must take the general path.
template <bool F8, bool H16 = false>
static int launch_fused(const void* q, int64_t q_row_stride, const void* k_cache,
                        const int32_t* block_tables, int64_t bt_row_stride,
                        int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                        const int32_t* seq_idx, int32_t m, int32_t n_q_heads, int32_t n_kv_heads,
                        int32_t head_dim, int32_t block_size, int32_t window_blocks,
                        int64_t n_blocks, float scale, int32_t agg_mode, int32_t num_keep,
                        float* importance_out, int32_t* keep_idx, void* workspace,
                        void* k_cache_w, void* v_cache_w, int32_t* context_lens,
                        hipStream_t s, const FinArgs& fin = FinArgs{}) {
  const int g = n_q_heads / n_kv_heads;
  const int Lw = window_blocks * block_size;
  const bool step = k_cache_w != nullptr;
  const bool ok = Lw <= kSelMaxWindow && block_size % kSelKeysPerWave == 0 && g <= 16 &&
                  head_dim == kCD && window_blocks <= kMaxWindowBlocks;
  if (!ok) return 1;
  const float sl2 = scale * kLog2e;
  const unsigned units = (unsigned)(m * n_kv_heads);
  float* partial = (float*)workspace;
  if (agg_mode == NKV_AGG_GROUP) {
    hipLaunchKernelGGL((compress_group_kernel<F8, H16>), dim3(units), dim3(kSelThreads), 0, s,
                       (const bf16_t*)q, q_row_stride, k_cache, block_tables, bt_row_stride,
                       max_blocks_per_seq, base_context_lens, seq_idx, n_kv_heads, g,
                       block_size, window_blocks, n_blocks, sl2, num_keep, importance_out,
                       keep_idx, k_cache_w, v_cache_w, context_lens, fin);
    return check_launch("compress (group)") ? -1 : 0;
  }
  hipLaunchKernelGGL((compress_partial_kernel<F8, H16>), dim3(units), dim3(kSelThreads), 0, s,
                     (const bf16_t*)q, q_row_stride, k_cache, block_tables, bt_row_stride,
                     max_blocks_per_seq, base_context_lens, seq_idx, n_kv_heads, g, block_size,
                     window_blocks, n_blocks, sl2, partial);
  if (check_launch("compress (partial)")) return -1;
  const int per_seq = step ? n_kv_heads : 1;
  hipLaunchKernelGGL((compress_sum_kernel<F8>), dim3((unsigned)(m * per_seq)), dim3(kSelThreads),
                     0, s, (const float*)partial, n_kv_heads, per_seq, block_size,
                     window_blocks, num_keep, importance_out, keep_idx, k_cache_w, v_cache_w,
                     block_tables, bt_row_stride, max_blocks_per_seq, base_context_lens,
                     context_lens, seq_idx, n_blocks, fin);
  return check_launch("compress (sum)") ? -1 : 0;
}
}  // namespace nkv

namespace nkv {
template <bool H16>
static int compress_select_impl(const void* q, int64_t q_row_stride, const void* k_cache,
                                const int32_t* block_tables, int64_t bt_row_stride,
                                int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                                const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                                int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t window_blocks, int64_t n_blocks, float scale,
                                int32_t agg_mode, int32_t num_keep, float* importance_out,
                                int32_t* keep_idx, void* workspace, size_t workspace_bytes,
                                void* stream) {
  NKV_REQUIRE(m >= 0 && n_q_heads > 0 && n_kv_heads > 0 && window_blocks > 0 && block_size > 0,
              NKV_EINVAL, "compress_select: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "compress_select: Hq %% Hk != 0");
  NKV_REQUIRE(agg_mode == NKV_AGG_ALL || agg_mode == NKV_AGG_GROUP, NKV_EINVAL,
              "compress_select: bad agg_mode %d", agg_mode);
  const int Lw = window_blocks * block_size;
  NKV_REQUIRE(num_keep > 0 && num_keep < Lw - 1, NKV_EINVAL,
              "compress_select: need 0 < num_keep < window tokens - 1 (got %d)", num_keep);
  NKV_REQUIRE(keep_idx && importance_out, NKV_EINVAL, "compress_select: null output");
  NKV_REQUIRE(q && k_cache, NKV_EINVAL, "compress_select: null pointer");
  NKV_REQUIRE(!block_tables || (seq_idx && base_context_lens && max_blocks_per_seq > 0 &&
                                 bt_row_stride >= max_blocks_per_seq),
              NKV_EINVAL, "compress_select: paged mode needs seq_idx, base_context_lens and a "
              "block table width");
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && q_row_stride % 8 == 0, NKV_EINVAL,
              "compress_select: q/k must be 16-byte aligned");
  const size_t need = nkv_compress_select_workspace_bytes(m, n_q_heads, n_kv_heads,
                                                          window_blocks, block_size);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "compress_select: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  hipStream_t s = as_stream(stream);
  const int rc = launch_fused<false, H16>(q, q_row_stride, k_cache, block_tables,
                                          bt_row_stride, max_blocks_per_seq, base_context_lens,
                                          seq_idx, m, n_q_heads, n_kv_heads, head_dim,
                                          block_size, window_blocks, n_blocks, scale, agg_mode,
                                          num_keep, importance_out, keep_idx, workspace, nullptr,
                                          nullptr, nullptr, s);
  if (rc <= 0) return rc < 0 ? NKV_ELAUNCH : NKV_OK;
  // general path: score + importance kernels, then the one-wave top-k
  const int n_sets = agg_mode == NKV_AGG_ALL ? 1 : n_kv_heads;
  int e = compress_score_impl<H16>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                                   max_blocks_per_seq, base_context_lens, seq_idx, m, n_q_heads,
                                   n_kv_heads, head_dim, block_size, window_blocks, n_blocks,
                                   scale, agg_mode, importance_out, workspace, workspace_bytes,
                                   stream);
  if (e) return e;
  return nkv_compress_topk(importance_out, m * n_sets, Lw - 1, num_keep, keep_idx, stream);
}
}  // namespace nkv

extern "C" int nkv_compress_select(const void* q, int64_t q_row_stride, const void* k_cache,
                                   const int32_t* block_tables, int64_t bt_row_stride,
                                   int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                                   const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                                   int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                   int32_t window_blocks, int64_t n_blocks, float scale,
                                   int32_t agg_mode, int32_t num_keep, float* importance_out,
                                   int32_t* keep_idx, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  clear_error();
  return compress_select_impl<false>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                                     max_blocks_per_seq, base_context_lens, seq_idx, m,
                                     n_q_heads, n_kv_heads, head_dim, block_size, window_blocks,
                                     n_blocks, scale, agg_mode, num_keep, importance_out,
                                     keep_idx, workspace, workspace_bytes, stream);
}

extern "C" int nkv_compress_select_f16(const void* q, int64_t q_row_stride, const void* k_cache,
                                       const int32_t* block_tables, int64_t bt_row_stride,
                                       int32_t max_blocks_per_seq,
                                       const int32_t* base_context_lens, const int32_t* seq_idx,
                                       int32_t m, int32_t n_q_heads, int32_t n_kv_heads,
                                       int32_t head_dim, int32_t block_size,
                                       int32_t window_blocks, int64_t n_blocks, float scale,
                                       int32_t agg_mode, int32_t num_keep,
                                       float* importance_out, int32_t* keep_idx,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return compress_select_impl<true>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                                    max_blocks_per_seq, base_context_lens, seq_idx, m,
                                    n_q_heads, n_kv_heads, head_dim, block_size, window_blocks,
                                    n_blocks, scale, agg_mode, num_keep, importance_out,
                                    keep_idx, workspace, workspace_bytes, stream);
}

extern "C" int nkv_compress_compact(void* k_cache, void* v_cache, const int32_t* block_tables,
                                    int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                    const int32_t* base_context_lens,
                                    int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                                    const int32_t* keep_idx, int32_t n_sets,
                                    int32_t keep_tokens, int32_t n_kv_heads, int32_t head_dim,
                                    int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                                    void* stream) {
  clear_error();
  NKV_REQUIRE(m >= 0 && n_kv_heads > 0 && block_size > 0 && window_blocks > 0, NKV_EINVAL,
              "compress_compact: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(compress_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "compress_compact: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(n_sets == 1 || n_sets == n_kv_heads, NKV_EINVAL,
              "compress_compact: n_sets must be 1 or n_kv_heads");
  NKV_REQUIRE(keep_tokens > 0 && keep_tokens <= window_blocks * block_size, NKV_EINVAL,
              "compress_compact: need 0 < keep_tokens <= window tokens");
  const int max_rows = keep_tokens + block_size - 1;
  NKV_REQUIRE(k_cache && v_cache && block_tables && base_context_lens && context_lens &&
                  seq_idx && keep_idx,
              NKV_EINVAL, "compress_compact: null pointer");
  NKV_REQUIRE(aligned16(k_cache) && aligned16(v_cache), NKV_EINVAL,
              "compress_compact: caches must be 16-byte aligned");
  NKV_REQUIRE(max_blocks_per_seq > 0 && bt_row_stride >= max_blocks_per_seq, NKV_EINVAL,
              "compress_compact: bad block table width/stride");
  NKV_REQUIRE(window_blocks <= kMaxWindowBlocks, NKV_EUNSUPPORTED,
              "compress_compact: window_blocks > %d", kMaxWindowBlocks);
  NKV_REQUIRE(n_blocks * block_size < (1ll << 31), NKV_EUNSUPPORTED,
              "compress_compact: pool of %lld slots exceeds 2^31", (long long)(n_blocks * block_size));
  hipStream_t s = as_stream(stream);
  const unsigned grid = (unsigned)(m * n_kv_heads * 2 * (head_dim / 64));
#define NKV_COMPACT_LAUNCH(R)                                                                  \
  hipLaunchKernelGGL((compress_compact_kernel<R, false>), dim3(grid), dim3(256), 0, s, k_cache, \
                     v_cache, block_tables, bt_row_stride, max_blocks_per_seq,                  \
                     base_context_lens,                                                         \
                     context_lens, seq_idx, keep_idx, n_sets, keep_tokens, n_kv_heads,          \
                     head_dim, block_size, window_blocks, n_blocks)
  if (max_rows <= 256) NKV_COMPACT_LAUNCH(8);
  else if (max_rows <= 512) NKV_COMPACT_LAUNCH(16);
  else if (max_rows <= 768) NKV_COMPACT_LAUNCH(24);
  else NKV_COMPACT_LAUNCH(32);  // more rows: rounds of 1024
#undef NKV_COMPACT_LAUNCH
  return check_launch("nkv_compress_compact");
}

namespace nkv {
static int launch_finalize(const FinArgs& fin, int64_t bt_row_stride, int32_t max_blocks_per_seq,
                           const int32_t* base_context_lens, const int32_t* seq_idx, int32_t m,
                           int32_t keep_tokens, int32_t block_size, int32_t window_blocks,
                           hipStream_t s) {
  hipLaunchKernelGGL(compress_finalize_kernel, dim3((unsigned)m), dim3(64), 0, s,
                     fin.block_tables, bt_row_stride, max_blocks_per_seq, base_context_lens,
                     seq_idx, m, keep_tokens, block_size, window_blocks, fin.rewrite_tables,
                     fin.slot_mapping, fin.events);
  return check_launch("nkv_compress_finalize");
}
}  // namespace nkv

extern "C" int nkv_compress_finalize(int32_t* block_tables, int64_t bt_row_stride,
                                     int32_t max_blocks_per_seq,
                                     const int32_t* base_context_lens, const int32_t* seq_idx,
                                     int32_t m, int32_t keep_tokens, int32_t block_size,
                                     int32_t window_blocks, int32_t rewrite_tables,
                                     int32_t* slot_mapping, int32_t* events, void* stream) {
  clear_error();
  NKV_REQUIRE(m >= 0 && block_size > 0 && window_blocks > 0 && max_blocks_per_seq > 0,
              NKV_EINVAL, "compress_finalize: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(block_tables && base_context_lens && seq_idx && events, NKV_EINVAL,
              "compress_finalize: null pointer");
  NKV_REQUIRE(bt_row_stride >= max_blocks_per_seq, NKV_EINVAL,
              "compress_finalize: bt_row_stride < max_blocks_per_seq");
  return launch_finalize(FinArgs{block_tables, slot_mapping, events, rewrite_tables},
                         bt_row_stride, max_blocks_per_seq, base_context_lens, seq_idx, m,
                         keep_tokens, block_size, window_blocks, as_stream(stream));
}

namespace nkv {
template <bool H16>
static int compress_step_impl(const void* q, int64_t q_row_stride, void* k_cache,
                              void* v_cache, const int32_t* block_tables,
                              int64_t bt_row_stride, int32_t max_blocks_per_seq,
                              const int32_t* base_context_lens, int32_t* context_lens,
                              const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                              int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                              int32_t window_blocks, int64_t n_blocks, float scale,
                              int32_t agg_mode, int32_t keep_tokens, float* importance_out,
                              int32_t* keep_idx, void* workspace, size_t workspace_bytes,
                              void* stream, const FinArgs& fin = FinArgs{}) {
  NKV_REQUIRE(m >= 0 && n_q_heads > 0 && n_kv_heads > 0 && window_blocks > 0 && block_size > 0,
              NKV_EINVAL, "compress_step: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(block_tables && v_cache && context_lens && seq_idx && base_context_lens,
              NKV_EINVAL, "compress_step: null pointer");
  NKV_REQUIRE(aligned16(v_cache), NKV_EINVAL, "compress_step: caches must be 16-byte aligned");
  NKV_REQUIRE(n_blocks * block_size < (1ll << 31), NKV_EUNSUPPORTED,
              "compress_step: cache of %lld slots exceeds int32 slot ids",
              (long long)(n_blocks * block_size));
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "compress_step: Hq %% Hk != 0");
  NKV_REQUIRE(agg_mode == NKV_AGG_ALL || agg_mode == NKV_AGG_GROUP, NKV_EINVAL,
              "compress_step: bad agg_mode %d", agg_mode);
  const int n_sets = agg_mode == NKV_AGG_ALL ? 1 : n_kv_heads;
  const int num_keep = keep_tokens - 2;
  NKV_REQUIRE(keep_tokens > 2 && num_keep < window_blocks * block_size - 1, NKV_EINVAL,
              "compress_step: need 2 < keep_tokens <= window tokens");
  NKV_REQUIRE(q && k_cache && keep_idx && importance_out && aligned16(q) && aligned16(k_cache) &&
                  q_row_stride % 8 == 0 && max_blocks_per_seq > 0 &&
                  bt_row_stride >= max_blocks_per_seq,
              NKV_EINVAL, "compress_step: bad q/k/tables");
  const size_t need = nkv_compress_select_workspace_bytes(m, n_q_heads, n_kv_heads,
                                                          window_blocks, block_size);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "compress_step: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  hipStream_t s = as_stream(stream);
  // the bookkeeping rides in the fused launch (m within the arrival counters), else it
  // follows as its own launch
  const FinArgs fused_fin = m <= kFinMaxSeqs ? fin : FinArgs{};
  int rc = launch_fused<false, H16>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                                    max_blocks_per_seq, base_context_lens, seq_idx, m,
                                    n_q_heads, n_kv_heads, head_dim, block_size, window_blocks,
                                    n_blocks, scale, agg_mode, num_keep, importance_out,
                                    keep_idx, workspace, k_cache, v_cache, context_lens, s,
                                    fused_fin);
  if (rc < 0) return NKV_ELAUNCH;
  if (rc == 1) {
    // general path: selection, then the compaction kernel (2-byte rows move as bytes)
    rc = compress_select_impl<H16>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                                   max_blocks_per_seq, base_context_lens, seq_idx, m, n_q_heads,
                                   n_kv_heads, head_dim, block_size, window_blocks, n_blocks,
                                   scale, agg_mode, num_keep, importance_out, keep_idx,
                                   workspace, workspace_bytes, stream);
    if (rc) return rc;
    rc = nkv_compress_compact(k_cache, v_cache, block_tables, bt_row_stride,
                              max_blocks_per_seq, base_context_lens, context_lens, seq_idx, m,
                              keep_idx, n_sets, keep_tokens, n_kv_heads, head_dim, block_size,
                              window_blocks, n_blocks, stream);
    if (rc) return rc;
  } else if (fused_fin.block_tables) {
    return NKV_OK;
  }
  if (!fin.block_tables) return NKV_OK;
  return launch_finalize(fin, bt_row_stride, max_blocks_per_seq, base_context_lens, seq_idx, m,
                         keep_tokens, block_size, window_blocks, s);
}
}  // namespace nkv

extern "C" int nkv_compress_step(const void* q, int64_t q_row_stride, void* k_cache,
                                 void* v_cache, const int32_t* block_tables,
                                 int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                 const int32_t* base_context_lens, int32_t* context_lens,
                                 const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                                 int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                 int32_t window_blocks, int64_t n_blocks, float scale,
                                 int32_t agg_mode, int32_t keep_tokens, float* importance_out,
                                 int32_t* keep_idx, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  nkv::clear_error();
  return nkv::compress_step_impl<false>(q, q_row_stride, k_cache, v_cache, block_tables,
                                        bt_row_stride, max_blocks_per_seq, base_context_lens,
                                        context_lens, seq_idx, m, n_q_heads, n_kv_heads,
                                        head_dim, block_size, window_blocks, n_blocks, scale,
                                        agg_mode, keep_tokens, importance_out, keep_idx,
                                        workspace, workspace_bytes, stream);
}

extern "C" int nkv_compress_step_f16(const void* q, int64_t q_row_stride, void* k_cache,
                                     void* v_cache, const int32_t* block_tables,
                                     int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                     const int32_t* base_context_lens, int32_t* context_lens,
                                     const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                                     int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                     int32_t window_blocks, int64_t n_blocks, float scale,
                                     int32_t agg_mode, int32_t keep_tokens,
                                     float* importance_out, int32_t* keep_idx, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  nkv::clear_error();
  return nkv::compress_step_impl<true>(q, q_row_stride, k_cache, v_cache, block_tables,
                                       bt_row_stride, max_blocks_per_seq, base_context_lens,
                                       context_lens, seq_idx, m, n_q_heads, n_kv_heads,
                                       head_dim, block_size, window_blocks, n_blocks, scale,
                                       agg_mode, keep_tokens, importance_out, keep_idx,
                                       workspace, workspace_bytes, stream);
}

extern "C" int nkv_compress_step_finalize(
    const void* q, int64_t q_row_stride, void* k_cache, void* v_cache, int32_t* block_tables,
    int64_t bt_row_stride, int32_t max_blocks_per_seq, const int32_t* base_context_lens,
    int32_t* context_lens, const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
    int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t window_blocks,
    int64_t n_blocks, float scale, int32_t agg_mode, int32_t keep_tokens, float* importance_out,
    int32_t* keep_idx, void* workspace, size_t workspace_bytes, int32_t rewrite_tables,
    int32_t* slot_mapping, int32_t* events, void* stream) {
  nkv::clear_error();
  NKV_REQUIRE(events, NKV_EINVAL, "compress_step_finalize: null events");
  return nkv::compress_step_impl<false>(
      q, q_row_stride, k_cache, v_cache, block_tables, bt_row_stride, max_blocks_per_seq,
      base_context_lens, context_lens, seq_idx, m, n_q_heads, n_kv_heads, head_dim, block_size,
      window_blocks, n_blocks, scale, agg_mode, keep_tokens, importance_out, keep_idx, workspace,
      workspace_bytes, stream, nkv::FinArgs{block_tables, slot_mapping, events, rewrite_tables});
}

extern "C" int nkv_compress_step_finalize_f16(
    const void* q, int64_t q_row_stride, void* k_cache, void* v_cache, int32_t* block_tables,
    int64_t bt_row_stride, int32_t max_blocks_per_seq, const int32_t* base_context_lens,
    int32_t* context_lens, const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
    int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t window_blocks,
    int64_t n_blocks, float scale, int32_t agg_mode, int32_t keep_tokens, float* importance_out,
    int32_t* keep_idx, void* workspace, size_t workspace_bytes, int32_t rewrite_tables,
    int32_t* slot_mapping, int32_t* events, void* stream) {
  nkv::clear_error();
  NKV_REQUIRE(events, NKV_EINVAL, "compress_step_finalize: null events");
  return nkv::compress_step_impl<true>(
      q, q_row_stride, k_cache, v_cache, block_tables, bt_row_stride, max_blocks_per_seq,
      base_context_lens, context_lens, seq_idx, m, n_q_heads, n_kv_heads, head_dim, block_size,
      window_blocks, n_blocks, scale, agg_mode, keep_tokens, importance_out, keep_idx, workspace,
      workspace_bytes, stream, nkv::FinArgs{block_tables, slot_mapping, events, rewrite_tables});
}

extern "C" int nkv_compress_schedule(const int32_t* context_lens,
                                     const int32_t* tail_uncompressed, int32_t batch,
                                     int32_t block_size, int32_t window_blocks, int32_t topk,
                                     int32_t period, int32_t policy, int32_t* step_counter,
                                     int32_t* seq_idx, int32_t* n_selected,
                                     int32_t* base_context_lens, void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(batch >= 0 && block_size > 0 && window_blocks > 0 && topk > 0 && period > 0 &&
                  (policy == 0 || policy == 1),
              NKV_EINVAL, "compress_schedule: bad arguments");
  NKV_REQUIRE(batch <= kSchedMaxBatch, NKV_EUNSUPPORTED, "compress_schedule: batch above %d",
              kSchedMaxBatch);
  NKV_REQUIRE(context_lens && tail_uncompressed && step_counter && seq_idx && n_selected,
              NKV_EINVAL, "compress_schedule: null pointer");
  if (batch <= kSchedRegBatch / 2)  // half the slots: half the compares of every count
    hipLaunchKernelGGL(compress_schedule_wave_kernel<kSchedSlots / 2>, dim3(1), dim3(64), 0,
                       as_stream(stream), context_lens, tail_uncompressed, batch, block_size,
                       window_blocks, topk, period, policy, step_counter, seq_idx, n_selected,
                       base_context_lens);
  else if (batch <= kSchedRegBatch)
    hipLaunchKernelGGL(compress_schedule_wave_kernel<kSchedSlots>, dim3(1), dim3(64), 0,
                       as_stream(stream), context_lens, tail_uncompressed, batch, block_size,
                       window_blocks, topk, period, policy, step_counter, seq_idx, n_selected,
                       base_context_lens);
  else
    hipLaunchKernelGGL(compress_schedule_kernel, dim3(1), dim3(kSchedThreads), 0,
                       as_stream(stream), context_lens, tail_uncompressed, batch, block_size,
                       window_blocks, topk, period, policy, step_counter, seq_idx, n_selected,
                       base_context_lens);
  return check_launch("nkv_compress_schedule");
}

// Compression step over fp8 (OCP E4M3FN) caches: K codes are widened to bf16 for
// scoring (k_scale folded into the score scale), then importance, top-k, and the
// compaction of the 1-byte rows. Windows of up to 1024 tokens take the fused kernels
// (as nkv_compress_step), longer ones the four-kernel general path; same results.
namespace nkv {
static int compress_step_fp8_impl(const void* q, int64_t q_row_stride, void* k_cache,
                                  void* v_cache, const int32_t* block_tables,
                                  int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                  const int32_t* base_context_lens, int32_t* context_lens,
                                  const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                                  int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                  int32_t window_blocks, int64_t n_blocks, float scale,
                                  float k_scale, int32_t agg_mode, int32_t keep_tokens,
                                  float* importance_out, int32_t* keep_idx, void* workspace,
                                  size_t workspace_bytes, void* stream,
                                  const FinArgs& fin = FinArgs{}) {
  NKV_REQUIRE(m >= 0 && n_q_heads > 0 && n_kv_heads > 0 && window_blocks > 0 &&
                  block_size > 0 && k_scale > 0.f,
              NKV_EINVAL, "compress_step_fp8: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(compress_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "compress_step_fp8: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "compress_step_fp8: Hq %% Hk != 0");
  const int g = n_q_heads / n_kv_heads;  // any group: above 16 the general path
  NKV_REQUIRE(block_size % kChunk == 0, NKV_EUNSUPPORTED,
              "compress_step_fp8: block_size must be a multiple of 256");
  NKV_REQUIRE(agg_mode == NKV_AGG_ALL || agg_mode == NKV_AGG_GROUP, NKV_EINVAL,
              "compress_step_fp8: bad agg_mode %d", agg_mode);
  NKV_REQUIRE(q && k_cache && v_cache && block_tables && base_context_lens && context_lens &&
                  seq_idx && importance_out && keep_idx,
              NKV_EINVAL, "compress_step_fp8: null pointer");
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && q_row_stride % 8 == 0,
              NKV_EINVAL, "compress_step_fp8: q/k/v must be 16-byte aligned");
  NKV_REQUIRE(max_blocks_per_seq > 0 && bt_row_stride >= max_blocks_per_seq, NKV_EINVAL,
              "compress_step_fp8: bad block table width/stride");
  NKV_REQUIRE(window_blocks <= kMaxWindowBlocks, NKV_EUNSUPPORTED,
              "compress_step_fp8: window_blocks > %d", kMaxWindowBlocks);
  NKV_REQUIRE(n_blocks * block_size < (1ll << 31), NKV_EUNSUPPORTED,
              "compress_step_fp8: pool exceeds 2^31 slots");
  const int Lw = window_blocks * block_size;
  const int num_keep = keep_tokens - 2;
  NKV_REQUIRE(num_keep > 0 && num_keep < Lw - 1 && Lw - 1 <= 4096, NKV_EINVAL,
              "compress_step_fp8: need 0 < keep_tokens - 2 < W*B - 1 <= 4096");
  const int max_rows = keep_tokens + block_size - 1;
  const size_t need = nkv_compress_workspace_bytes(m, n_q_heads, window_blocks, block_size);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "compress_step_fp8: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  hipStream_t s = as_stream(stream);
  const FinArgs fused_fin = m <= kFinMaxSeqs ? fin : FinArgs{};  // as compress_step_impl
  int rc = launch_fused<true>(q, q_row_stride, k_cache, block_tables, bt_row_stride,
                              max_blocks_per_seq, base_context_lens, seq_idx, m, n_q_heads,
                              n_kv_heads, head_dim, block_size, window_blocks, n_blocks,
                              scale * k_scale, agg_mode, num_keep, importance_out, keep_idx,
                              workspace, k_cache, v_cache, context_lens, s, fused_fin);
  if (rc < 0) return NKV_ELAUNCH;
  if (rc == 0) {
    if (fused_fin.block_tables || !fin.block_tables) return NKV_OK;
    return launch_finalize(fin, bt_row_stride, max_blocks_per_seq, base_context_lens, seq_idx,
                           m, keep_tokens, block_size, window_blocks, s);
  }
  // general path: score, importance, top-k, compaction
  float* scores = (float*)workspace;
  const unsigned sgrid = (unsigned)(m * n_kv_heads * (Lw / kChunk));
  const float sl2 = scale * k_scale * kLog2e;
  launch_score<true>(head_dim, sgrid, s, (const bf16_t*)q, q_row_stride, k_cache, block_tables,
                     bt_row_stride, max_blocks_per_seq, base_context_lens, seq_idx, n_kv_heads,
                     g, block_size, window_blocks, n_blocks, sl2, Lw - 1, scores);
  rc = check_launch("nkv_compress_step_fp8 (score)");
  if (rc) return rc;
  const int n_sets = agg_mode == NKV_AGG_ALL ? 1 : n_kv_heads;
  const int hps = n_q_heads / n_sets;
  hipLaunchKernelGGL(compress_importance_kernel, dim3((unsigned)(m * n_sets)), dim3(256),
                     (size_t)hps * 2 * sizeof(float), s, scores, n_q_heads, n_sets, Lw, Lw - 1,
                     importance_out);
  rc = check_launch("nkv_compress_step_fp8 (importance)");
  if (rc) return rc;
  rc = nkv_compress_topk(importance_out, m * n_sets, Lw - 1, num_keep, keep_idx, stream);
  if (rc) return rc;
  const unsigned cgrid = (unsigned)(m * n_kv_heads * 2 * (head_dim / 64));
#define NKV_COMPACT8_LAUNCH(R)                                                                 \
  hipLaunchKernelGGL((compress_compact_kernel<R, true>), dim3(cgrid), dim3(256), 0, s, k_cache, \
                     v_cache, block_tables, bt_row_stride, max_blocks_per_seq,                  \
                     base_context_lens, context_lens, seq_idx, keep_idx, n_sets, keep_tokens,   \
                     n_kv_heads, head_dim, block_size, window_blocks, n_blocks)
  if (max_rows <= 256) NKV_COMPACT8_LAUNCH(4);
  else if (max_rows <= 512) NKV_COMPACT8_LAUNCH(8);
  else if (max_rows <= 768) NKV_COMPACT8_LAUNCH(12);
  else NKV_COMPACT8_LAUNCH(16);
#undef NKV_COMPACT8_LAUNCH
  rc = check_launch("nkv_compress_step_fp8 (compact)");
  if (rc || !fin.block_tables) return rc;
  return launch_finalize(fin, bt_row_stride, max_blocks_per_seq, base_context_lens, seq_idx, m,
                         keep_tokens, block_size, window_blocks, s);
}
}  // namespace nkv

extern "C" int nkv_compress_step_fp8(const void* q, int64_t q_row_stride, void* k_cache,
                                     void* v_cache, const int32_t* block_tables,
                                     int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                     const int32_t* base_context_lens, int32_t* context_lens,
                                     const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
                                     int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                     int32_t window_blocks, int64_t n_blocks, float scale,
                                     float k_scale, int32_t agg_mode, int32_t keep_tokens,
                                     float* importance_out, int32_t* keep_idx, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  nkv::clear_error();
  return nkv::compress_step_fp8_impl(q, q_row_stride, k_cache, v_cache, block_tables,
                                     bt_row_stride, max_blocks_per_seq, base_context_lens,
                                     context_lens, seq_idx, m, n_q_heads, n_kv_heads, head_dim,
                                     block_size, window_blocks, n_blocks, scale, k_scale,
                                     agg_mode, keep_tokens, importance_out, keep_idx, workspace,
                                     workspace_bytes, stream);
}

extern "C" int nkv_compress_step_finalize_fp8(
    const void* q, int64_t q_row_stride, void* k_cache, void* v_cache, int32_t* block_tables,
    int64_t bt_row_stride, int32_t max_blocks_per_seq, const int32_t* base_context_lens,
    int32_t* context_lens, const int32_t* seq_idx, int32_t m, int32_t n_q_heads,
    int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t window_blocks,
    int64_t n_blocks, float scale, float k_scale, int32_t agg_mode, int32_t keep_tokens,
    float* importance_out, int32_t* keep_idx, void* workspace, size_t workspace_bytes,
    int32_t rewrite_tables, int32_t* slot_mapping, int32_t* events, void* stream) {
  nkv::clear_error();
  NKV_REQUIRE(events, NKV_EINVAL, "compress_step_finalize_fp8: null events");
  return nkv::compress_step_fp8_impl(
      q, q_row_stride, k_cache, v_cache, block_tables, bt_row_stride, max_blocks_per_seq,
      base_context_lens, context_lens, seq_idx, m, n_q_heads, n_kv_heads, head_dim, block_size,
      window_blocks, n_blocks, scale, k_scale, agg_mode, keep_tokens, importance_out, keep_idx,
      workspace, workspace_bytes, stream,
      nkv::FinArgs{block_tables, slot_mapping, events, rewrite_tables});
}

// SnapKV as called directly (the plug-in API): Q [m, Hq, window, D], contiguous K
// [m, Hk, L, D]. A query window of w tokens is scored as G*w query rows per KV head (rows
// of one head consecutive, which is Q's layout); the w window keys are not scored and are
// always kept. window 1 with L <= 1024, L % 64 == 0 takes the fused selection.
extern "C" size_t nkv_snapkv_workspace_bytes(int32_t m, int32_t n_q_heads, int32_t n_kv_heads,
                                             int32_t seq_len, int32_t window) {
  if (m <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || seq_len <= 0 || window <= 0) return 0;
  const size_t scores = (size_t)m * n_q_heads * window * seq_len * sizeof(float);
  const size_t fused = nkv_compress_select_workspace_bytes(m, n_q_heads, n_kv_heads, 1, seq_len);
  return scores > fused ? scores : fused;
}

namespace nkv {
template <bool H16>
static int snapkv_select_impl(const void* q, const void* k, int32_t m, int32_t n_q_heads,
                              int32_t n_kv_heads, int32_t head_dim, int32_t seq_len,
                              int32_t window, float scale, int32_t agg_mode, int32_t num_keep,
                              float* importance_out, int32_t* keep_idx, void* workspace,
                              size_t workspace_bytes, void* stream) {
  NKV_REQUIRE(m >= 0 && n_q_heads > 0 && n_kv_heads > 0 && seq_len > 0 && window > 0,
              NKV_EINVAL, "snapkv_select: bad sizes");
  if (m == 0) return NKV_OK;
  NKV_REQUIRE(compress_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "snapkv_select: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "snapkv_select: Hq %% Hk != 0");
  NKV_REQUIRE(agg_mode == NKV_AGG_ALL || agg_mode == NKV_AGG_GROUP, NKV_EINVAL,
              "snapkv_select: bad agg_mode %d", agg_mode);
  const int n_cand = seq_len - window;
  NKV_REQUIRE(n_cand > 0 && num_keep > 0 && num_keep < n_cand, NKV_EINVAL,
              "snapkv_select: need 0 < num_keep < seq_len - window (%d, %d, %d)", num_keep,
              seq_len, window);
  NKV_REQUIRE(q && k && importance_out && keep_idx, NKV_EINVAL, "snapkv_select: null pointer");
  NKV_REQUIRE(aligned16(q) && aligned16(k), NKV_EINVAL,
              "snapkv_select: q/k must be 16-byte aligned");
  const size_t need = nkv_snapkv_workspace_bytes(m, n_q_heads, n_kv_heads, seq_len, window);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "snapkv_select: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  if (window == 1)  // the periodic step's own shape: fused when it fits
    return compress_select_impl<H16>(q, (int64_t)n_q_heads * head_dim, k, nullptr, 0, 0,
                                     nullptr, nullptr, m, n_q_heads, n_kv_heads, head_dim,
                                     seq_len, 1, 0, scale, agg_mode, num_keep, importance_out,
                                     keep_idx, workspace, workspace_bytes, stream);
  NKV_REQUIRE(n_cand <= 4096, NKV_EUNSUPPORTED, "snapkv_select: more than 4096 candidates");
  const int g = n_q_heads / n_kv_heads;
  const int rows = g * window;  // query rows per KV head
  float* scores = (float*)workspace;
  hipStream_t s = as_stream(stream);
  const unsigned grid = (unsigned)(m * n_kv_heads * ((seq_len + kChunk - 1) / kChunk));
  launch_score<false, H16>(head_dim, grid, s, (const bf16_t*)q,
                           (int64_t)n_q_heads * window * head_dim, k, nullptr, 0, 0, nullptr,
                           nullptr, n_kv_heads, rows, seq_len, 1, 0, scale * kLog2e, n_cand,
                           scores);
  int rc = check_launch("nkv_snapkv_select (score)");
  if (rc) return rc;
  const int n_sets = agg_mode == NKV_AGG_ALL ? 1 : n_kv_heads;
  const int hps = n_q_heads * window / n_sets;
  hipLaunchKernelGGL(compress_importance_kernel, dim3((unsigned)(m * n_sets)), dim3(256),
                     (size_t)hps * 2 * sizeof(float), s, scores, n_q_heads * window, n_sets,
                     seq_len, n_cand, importance_out);
  rc = check_launch("nkv_snapkv_select (importance)");
  if (rc) return rc;
  if (n_cand <= 64 * 16) {
    hipLaunchKernelGGL(compress_topk_kernel<16>, dim3((unsigned)(m * n_sets)), dim3(64), 0, s,
                       importance_out, n_cand, num_keep, window, keep_idx);
  } else {
    hipLaunchKernelGGL(compress_topk_kernel<64>, dim3((unsigned)(m * n_sets)), dim3(64), 0, s,
                       importance_out, n_cand, num_keep, window, keep_idx);
  }
  return check_launch("nkv_snapkv_select (top-k)");
}
}  // namespace nkv

extern "C" int nkv_snapkv_select(const void* q, const void* k, int32_t m, int32_t n_q_heads,
                                 int32_t n_kv_heads, int32_t head_dim, int32_t seq_len,
                                 int32_t window, float scale, int32_t agg_mode, int32_t num_keep,
                                 float* importance_out, int32_t* keep_idx, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  clear_error();
  return snapkv_select_impl<false>(q, k, m, n_q_heads, n_kv_heads, head_dim, seq_len, window,
                                   scale, agg_mode, num_keep, importance_out, keep_idx,
                                   workspace, workspace_bytes, stream);
}

extern "C" int nkv_snapkv_select_f16(const void* q, const void* k, int32_t m, int32_t n_q_heads,
                                     int32_t n_kv_heads, int32_t head_dim, int32_t seq_len,
                                     int32_t window, float scale, int32_t agg_mode,
                                     int32_t num_keep, float* importance_out, int32_t* keep_idx,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return snapkv_select_impl<true>(q, k, m, n_q_heads, n_kv_heads, head_dim, seq_len, window,
                                  scale, agg_mode, num_keep, importance_out, keep_idx,
                                  workspace, workspace_bytes, stream);
}

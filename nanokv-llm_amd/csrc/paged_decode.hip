// Paged decode attention (one new query token per sequence, GQA) over the
// [num_blocks, block_size, Hk, D] bf16 cache.
//
// Reference: flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
// cache_seqlens=context_lens, block_table=block_tables, softmax_scale,
// causal=True) at nanokvllm/layers/attention.py:104-107.
//
// MI355X design (HBM-bound: every K/V byte is read exactly once):
//  * Balanced split-K ("stream-K"): the K/V stream of the batch is cut into
//    16-token chunks ordered (sequence, KV head group, chunk). Persistent
//    one-wave workgroups, as many as are resident at once, each take an equal
//    contiguous range of C chunks, so every wave moves the same number of
//    bytes whatever the context-length mix. A range crosses at most a few
//    (sequence, head group) segments; each segment it touches yields one
//    partial (m, l, O) per query head.
//    A head group is one KV head, or two (HP = 2; four for fp8 rows, HP = 4)
//    whose parts of every token row are read as one contiguous piece.
//  * Within a segment the wave streams chunks through a register ring holding
//    16 KiB of K and V (one chunk of 512-byte rows, two of 256-byte rows): the
//    chunk one ring ahead is issued as soon as the current chunk's rows are
//    staged in LDS, before its products are computed. Loads are
//    non-temporal raw buffer loads whose per-chunk descriptor covers only the
//    chunk's valid rows: keys past the context,
//    padding chunks and invalid block-table entries read as zero without
//    touching memory. Each consumed chunk is staged row-major in LDS.
//  * Both contractions run on the matrix cores:
//      S^T = K q^T   v_mfma_f32_16x16x32_bf16, A = 16 keys (read back from
//                    LDS, one key row per lane), B = the g query heads of the
//                    KV head; lane l ends up with head l%16, keys 4(l/16)..+3.
//      O^T += V^T P^T v_mfma_f32_16x16x16_bf16 per 16-dim block; the B
//                    operand is exactly the lane's 4 softmax weights (bf16),
//                    the A operand V^T comes from LDS with ds_read_b64_tr_b16.
//    Every lane holds state for one head (its column): the online softmax
//    needs no cross-lane traffic except one xor-max over the 4 key groups.
//  * A combine kernel merges the few partials of each (sequence, query head).
// Scores are kept in the log2 domain (scale * log2 e folded in) so the
// exponentials are single v_exp_f32 instructions.
//
// Workspace (caller-owned, sized by what the grid can write, not by the batch
// times the table width): one descriptor per (sequence, KV head) -- first
// partial row, partial count, row stride -- then the partial rows. Within a
// head group, wave wi's partial of sequence b is row wi + b: a segment's
// partials come from consecutive waves, and the next segment's first wave is
// at least its last one, so wi + b never collides and stays below
// waves + batch. A row holds O (D floats), m, l and two pad floats.
//
// head_dim D is 64, 128 or 256 (a template parameter of both kernels).
#include "nkv_common.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace nkv {

constexpr int kChunk = 16;               // tokens per pipeline stage
constexpr int kMinChunks = 4;            // minimum chunks per wave range
constexpr int kMaxSlots = 128;           // partials per (sequence, query head) at most
constexpr int kWinBlocks = 64;           // block ids held per window (one per lane)
constexpr int kBufferFlags = 0x00020000; // raw buffer resource word 3 (dword data)
constexpr int kStreamPolicy = 2;         // cache policy "nt": K/V are read exactly once
constexpr int kWavesPerCU = 8;           // resident split waves per CU (2 per SIMD)
// floats per partial row: O, m, l, 2 pad (528 B at D = 128)
constexpr int part_row(int D) { return D + 4; }
constexpr bool decode_dim_ok(int D) { return D == 64 || D == 128 || D == 256; }
constexpr int kMaxCols = 16;             // MFMA columns: query heads per wave at most
constexpr int kMaxGroup = 256;           // GQA group at most (above 16: column groups)
// Column groups per KV head: its G query heads over ceil(G / 16) waves when G > 16.
constexpr int decode_ncg(int G) { return G > kMaxCols ? (G + kMaxCols - 1) / kMaxCols : 1; }

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4v_t __attribute__((ext_vector_type(4)));

// Partial slots per (sequence, query head): a segment of n chunks is touched by at most
// ceil(n / C) + 1 waves, and the kernel takes C >= decode_min_chunks, which is at least
// kMinChunks and at least max_chunks / (slots - 1), so no segment has more than kMaxSlots
// partials (the combine holds up to 128, two per lane).
static inline int64_t decode_slots(int32_t max_blocks, int32_t block_size) {
  const int64_t max_chunks = ((int64_t)max_blocks * block_size + kChunk - 1) / kChunk;
  const int64_t s = (max_chunks + kMinChunks - 1) / kMinChunks + 1;
  return s < kMaxSlots ? s : kMaxSlots;
}
// The smallest range a wave takes: kMinChunks, or longer when the table width allows
// segments that would otherwise need more than `slots` partials.
static inline int32_t decode_min_chunks(int32_t max_blocks, int32_t block_size) {
  const int64_t max_chunks = ((int64_t)max_blocks * block_size + kChunk - 1) / kChunk;
  const int64_t slots = decode_slots(max_blocks, block_size);
  const int64_t c = (max_chunks + slots - 2) / (slots - 1);
  return (int32_t)(c > kMinChunks ? c : kMinChunks);
}

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(v, o, 64);
    if (lane >= o) v += y;
  }
  return v;
}

// Cursor over sequences in batches of 64 (one per lane): in the chunk stream
// of one KV head, sequence s owns chunks [g_s, g_s + nc_s).
struct SeqCursor {
  int cb;    // first sequence of the loaded batch (uniform)
  int base;  // stream index of sequence cb's first chunk (uniform)
  int tot;   // chunks of the batch (uniform)
  int ctx;   // lane: context length of sequence cb + lane
  int nc;    // lane: chunks of that sequence
  int incl;  // lane: inclusive prefix of nc over the batch
};

__device__ __forceinline__ void seq_load(SeqCursor& c, const int32_t* __restrict__ ctx_lens,
                                         int batch, int max_tokens) {
  const int s = c.cb + (int)threadIdx.x;
  c.ctx = s < batch ? ctx_lens[s] : 0;
  NKV_DBG(c.ctx < 0 || c.ctx > max_tokens, NKV_DEBUG_LENGTH);
  c.nc = c.ctx > 0 ? (min(c.ctx, max_tokens) + kChunk - 1) / kChunk : 0;
  c.incl = wave_incl_scan(c.nc);
  c.tot = __builtin_amdgcn_readlane(c.incl, 63);
}

// Element offset of head dim `dim` (a multiple of 4) in a staged LDS row. bf16 rows are
// dense. fp8 rows are staged as 8-dim pieces with the even pieces first (piece 2c at slot
// c, piece 2c+1 at slot D/16 + c): a lane widens 16 codes into pieces 2c and 2c+1, and
// each of its two 16-byte writes then lands beside its neighbours' (the 32-byte stride of
// a dense row would leave half the banks idle and pair the others up).
template <bool F8, int D>
__device__ __forceinline__ int stage_off(int dim) {
  if constexpr (F8) {
    const int piece = dim >> 3;
    return ((piece >> 1) + (D / 16) * (piece & 1)) * 8 + (dim & 7);
  } else {
    return dim;
  }
}

// F8: the caches hold fp8 (OCP E4M3FN) codes; a chunk's rows are half as many
// bytes and are widened to bf16 (exact) when staged in LDS; the K scale is
// folded into scale_log2 and the V scale multiplies the partial O.
// HP: KV heads per wave. With HP = 2 a wave reads both heads' halves of every
// token row as one contiguous piece (512 B bf16, 256 B fp8) instead of one
// head's 256 B: on this part a stream of 256-byte pieces at 2 KiB stride runs
// unevenly (pieces at odd 256-byte offsets come back later), and the waves of
// the slow heads set the kernel's length. The HP*G query heads fill MFMA columns
// 0..HP*G-1; each head's scores use its own K, the softmax weights of a column
// are zero for the other heads, so all heads' PV products add into one O^T.
// fp8 rows (1 KiB at Hk = 8) take HP = 4 for 512-byte pieces, with K and V
// staged through one LDS buffer so two waves per SIMD still fit.
// G (query heads per KV head) is any value with HP*G <= 16: the columns past
// HP*G are computed and dropped. D: head_dim (64, 128 or 256); a wave's piece of
// a token row (HP*D elements) is 128 to 512 bytes.
template <bool F8, int HP, int D, bool H16 = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
void paged_decode_split_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride,
    const void* __restrict__ k_cache, const void* __restrict__ v_cache,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride,
    const int32_t* __restrict__ context_lens, int32_t batch, int32_t Hk, int32_t G,
    int32_t NCG, int32_t block_size, int32_t max_blocks, int64_t n_blocks, int32_t min_chunks,
    float scale_log2, float v_scale, float* __restrict__ part, i32x4v_t* __restrict__ desc) {
  static_assert(decode_dim_ok(D), "head_dim 64, 128 or 256");
  static_assert(!(F8 && H16), "fp8 caches are read with bf16 queries");
  constexpr int kEl = F8 ? 1 : 2;              // bytes per cache element
  constexpr int kSeg = HP * D * kEl;           // bytes a wave reads of each token row
  static_assert(kSeg >= 64 && kSeg <= 512, "a wave's piece of a row is 64..512 bytes");
  constexpr int kKs = D / 32;                  // k-steps of S^T (32 dims each)
  constexpr int kDb = D / 16;                  // 16-dim blocks of O^T
  constexpr int kVRow = D + 16;                // LDS row stride of a staged chunk (elements)
  constexpr int kPartRow = part_row(D);
  constexpr int kLpr = kSeg / 16;              // lanes per row (16-byte loads)
  constexpr int kRpl = 64 / kLpr;              // rows per load instruction
  constexpr int kLoads = kChunk / kRpl;        // loads per lane per K (or V) chunk
  // ring depth: 16 KiB of K and V in flight per wave (one chunk of 512-byte pieces, two of
  // 256-byte ones ...); a chunk's slot is refilled as soon as its rows are staged in LDS
  constexpr int kRing = kLoads >= 8 ? 1 : kLoads >= 4 ? 2 : 4;
  constexpr int kLph = kLpr / HP;              // lanes per head within a row
  // K and V of a chunk share one staging buffer (V is written after the K reads of S^T)
  // where two would take 20 KiB or more (four heads at D <= 128, two at D = 256), which
  // keeps two waves per SIMD within the LDS
  constexpr bool kShared = 2 * HP * kChunk * kVRow * 2 >= 20480;
  __shared__ __attribute__((aligned(16))) bf16_t lbuf[kShared ? 1 : 2][HP][kChunk * kVRow];
  auto& kbuf = lbuf[0];
  auto& vbuf = lbuf[kShared ? 0 : 1];

  const int lane = threadIdx.x;
  const int g4 = lane >> 4;   // key group: keys 4*g4 .. 4*g4+3 of a chunk
  const int col = lane & 15;  // MFMA column: query head (S^T, O^T) / key row (K)
  // Column groups: the G > 16 query heads of a KV head are split over NCG = ceil(G / 16)
  // waves of 16 MFMA columns (the last one fewer; HP = 1 then); NCG = 1 otherwise.
  const int row_b = Hk * D * kEl;  // bytes of one cache row (token)
  const int max_tokens = max_blocks * block_size;

  // ---- this wave's KV heads and chunk range. Every head group has the same
  // chunk stream (sequence-major); waves p, p+NP, p+2NP, ... split it into
  // equal ranges, so the NP waves i*NP .. i*NP+NP-1 read the Hk heads of the
  // same cache blocks at the same time.
  const int NP = Hk * NCG / HP;
  const int grp = blockIdx.x % NP;
  const int kvh0 = (grp / NCG) * HP;
  const int cg = grp - (grp / NCG) * NCG;  // column group
  // MFMA columns that are query heads (= partial rows per wave and sequence)
  const int HPG = NCG > 1 ? min(kMaxCols, G - cg * kMaxCols) : HP * G;
  const int qh0 = kvh0 * G + cg * kMaxCols;  // query head of column 0
  const int wi = blockIdx.x / NP;
  const int Wh = gridDim.x / NP;
  if (wi >= Wh) return;
  // partial rows of this head group: (wave + sequence) x HPG columns, after the groups of
  // the query heads before qh0 (so the groups' regions add up to (waves + batch) x Hq rows)
  float* gpart = part + (int64_t)(Wh + batch) * qh0 * kPartRow;
  SeqCursor cur;
  int T = 0;
  for (cur.cb = 0; cur.cb < batch; cur.cb += 64) {
    seq_load(cur, context_lens, batch, max_tokens);
    T += cur.tot;
  }
  // equal ranges over the resident waves, at least min_chunks (which keeps every
  // segment within its partial slots)
  const int C = max((T + Wh - 1) / Wh, min_chunks);
  const int k_begin = wi * C;
  if (k_begin >= T) return;
  const int k_end = min(T, k_begin + C);
  cur.cb = 0;
  cur.base = 0;
  seq_load(cur, context_lens, batch, max_tokens);

  // per-lane load offset: lane l reads 16 bytes of row l / kLpr (+ kRpl per
  // load), byte 16 * (l % kLpr) of the wave's piece of the row; it stages them
  // in head sh's LDS rows at dim sd (fp8 codes widen to 16 bf16 there). K is
  // re-read from LDS in the MFMA A layout.
  const int roff = (lane / kLpr) * row_b + (lane % kLpr) * 16;
  const int rstep = kRpl * row_b;  // bytes between a lane's consecutive loads
  const int sh = (lane % kLpr) / kLph;
  const int sd = (lane % kLph) * (16 / kEl);
  const int tr_row = 4 * g4 + (col >> 2);  // ds_read_b64_tr_b16 source row / column
  const int tr_col = (col & 3) * 4;
  const int hsel = col / G;                // head (of the HP) of this lane's column

  for (int k = k_begin; k < k_end;) {
    // ---- locate the sequence holding stream chunk k (wave-uniform)
    while (k >= cur.base + cur.tot) {
      cur.base += cur.tot;
      cur.cb += 64;
      seq_load(cur, context_lens, batch, max_tokens);
    }
    const int ln = __builtin_amdgcn_readfirstlane(__builtin_ctzll(__ballot(cur.base + cur.incl > k)));
    const int b = cur.cb + ln;
    const int ctx = __builtin_amdgcn_readlane(cur.ctx, ln);
    const int nc = __builtin_amdgcn_readlane(cur.nc, ln);
    const int g0 = cur.base + __builtin_amdgcn_readlane(cur.incl, ln) - nc;
    const int c_lo = k - g0;
    const int n_seg = min(nc - c_lo, k_end - k);
    const int w_first = g0 / C;  // first wave of the segment

    // q^T as the MFMA B operand: lane l -> query head kvh0*G + l%16 (columns
    // >= HP*G re-read the first head and are discarded), dims 8*(l/16) + 32*ks
    u32x4_t qreg[kKs];
    {
      const int hc = col < HPG ? col : 0;
      const u32x4_t* qp = reinterpret_cast<const u32x4_t*>(
          q + (int64_t)b * q_row_stride + (int64_t)(qh0 + hc) * D + g4 * 8);
#pragma unroll
      for (int ks = 0; ks < kKs; ++ks) qreg[ks] = qp[ks * 4];
    }
    const char* kbase = static_cast<const char*>(k_cache) + (int64_t)kvh0 * D * kEl;
    const char* vbase = static_cast<const char*>(v_cache) + (int64_t)kvh0 * D * kEl;
    const int32_t* bt_row = block_tables + (int64_t)b * bt_row_stride;

    f32x4_t acc[kDb];  // O^T: lane l -> column l%16, dims 16*db + 4*(l/16) .. +3
#pragma unroll
    for (int db = 0; db < kDb; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    // windows of at most kWinBlocks cache blocks (block ids one per lane)
    const int win_cap = (kWinBlocks - 1) * (block_size / kChunk);
    for (int wc = 0; wc < n_seg; wc += win_cap) {
      const int wlo = c_lo + wc;                 // first chunk of the window
      const int wn = min(n_seg - wc, win_cap);   // chunks in the window
      const int blk0 = wlo * kChunk / block_size;
      int blk_id = -1;
      {
        const int bi = blk0 + lane;
        if (bi < max_blocks && bi * block_size < (wlo + wn) * kChunk) {
          const int id = bt_row[bi];
          NKV_DBG(id < 0 || id >= n_blocks, NKV_DEBUG_BLOCK);  // every block here is needed
          blk_id = (id >= 0 && id < n_blocks) ? id : -1;
        }
      }

      u32x4_t kreg[kRing][kLoads];
      u32x4_t vreg[kRing][kLoads];
      int nv[kRing];  // valid keys of the chunk in each ring slot (0: masked)
      auto issue = [&](int j, int s) {
        const int t0 = (wlo + j) * kChunk;
        const int pb = __builtin_amdgcn_readlane(blk_id, min(t0 / block_size - blk0, 63));
        const int n = (j < wn && pb >= 0) ? min(max(ctx - t0, 0), kChunk) : 0;
        nv[s] = n;
        const int64_t r0 = (int64_t)(pb < 0 ? 0 : pb) * block_size + t0 % block_size;
        const uint32_t bytes = (uint32_t)(n * row_b);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(kbase + r0 * row_b), (short)0, bytes, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(vbase + r0 * row_b), (short)0, bytes, kBufferFlags);
#pragma unroll
        for (int r = 0; r < kLoads; ++r)
          kreg[s][r] = __builtin_bit_cast(
              u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, roff + r * rstep, 0,
                                                             kStreamPolicy));
#pragma unroll
        for (int r = 0; r < kLoads; ++r)
          vreg[s][r] = __builtin_bit_cast(
              u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, roff + r * rstep, 0,
                                                             kStreamPolicy));
      };

      auto consume = [&](int s, auto refill, int nxt) {
        constexpr bool kRefill = decltype(refill)::value;
        const int nv_cur = nv[s];  // the refill below overwrites the slot's count
        // stage the chunk's K and V rows (row-major per head, bf16) in LDS
#pragma unroll
        for (int r = 0; r < kLoads; ++r) {
          const int row = (kRpl * r + lane / kLpr) * kVRow;
          const int e = row + stage_off<F8, D>(sd);
          if constexpr (F8) {
            const int e2 = row + stage_off<F8, D>(sd + 8);
            u32x4_t lo, hi;
            fp8x16_to_bf16(kreg[s][r], lo, hi);
            *reinterpret_cast<u32x4_t*>(&kbuf[sh][e]) = lo;
            *reinterpret_cast<u32x4_t*>(&kbuf[sh][e2]) = hi;
            if constexpr (!kShared) {
              fp8x16_to_bf16(vreg[s][r], lo, hi);
              *reinterpret_cast<u32x4_t*>(&vbuf[sh][e]) = lo;
              *reinterpret_cast<u32x4_t*>(&vbuf[sh][e2]) = hi;
            }
          } else {
            *reinterpret_cast<u32x4_t*>(&kbuf[sh][e]) = kreg[s][r];
            if constexpr (!kShared) *reinterpret_cast<u32x4_t*>(&vbuf[sh][e]) = vreg[s][r];
          }
        }
        if constexpr (kRefill && !kShared) {
          __builtin_amdgcn_sched_barrier(0);
          issue(nxt, s);  // the slot's registers are staged: refill now
          __builtin_amdgcn_sched_barrier(0);
        }
        // S^T for 16 keys x 16 columns per head; A operand: lane l -> key l%16,
        // dims 8*(l/16) + 32*ks
        f32x4_t st[HP];
#pragma unroll
        for (int hh = 0; hh < HP; ++hh) {
          f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < kKs; ++ks) {
            const u32x4_t ka =
                *reinterpret_cast<const u32x4_t*>(
                    &kbuf[hh][col * kVRow + stage_off<F8, D>(g4 * 8 + ks * 32)]);
            a = mfma_16x16x32<H16>(ka, qreg[ks], a);
          }
          st[hh] = a;
        }
        // online softmax for column `col` over keys 4*g4 .. +3 of the chunk
        float sv[4];
        float cmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = st[0][r];
#pragma unroll
          for (int hh = 1; hh < HP; ++hh) x = hsel == hh ? st[hh][r] : x;
          sv[r] = (4 * g4 + r < nv_cur) ? x * scale_log2 : -INFINITY;
          cmax = fmaxf(cmax, sv[r]);
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m_run - m_new);
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = (sv[r] == -INFINITY) ? 0.f : fast_exp2(sv[r] - m_new);
        l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        m_run = m_new;
        if (alpha != 1.f) {
#pragma unroll
          for (int db = 0; db < kDb; ++db) acc[db] *= alpha;
        }
        const uint2 pw = {cvt_pk16<H16>(p[0], p[1]), cvt_pk16<H16>(p[2], p[3])};
        if constexpr (kShared) {  // V over the K rows: the S^T reads above come first
#pragma unroll
          for (int r = 0; r < kLoads; ++r) {
            const int row = (kRpl * r + lane / kLpr) * kVRow;
            if constexpr (F8) {
              u32x4_t lo, hi;
              fp8x16_to_bf16(vreg[s][r], lo, hi);
              *reinterpret_cast<u32x4_t*>(&vbuf[sh][row + stage_off<F8, D>(sd)]) = lo;
              *reinterpret_cast<u32x4_t*>(&vbuf[sh][row + stage_off<F8, D>(sd + 8)]) = hi;
            } else {
              *reinterpret_cast<u32x4_t*>(&vbuf[sh][row + sd]) = vreg[s][r];
            }
          }
          if constexpr (kRefill) {
            __builtin_amdgcn_sched_barrier(0);
            issue(nxt, s);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        // P^T per head: a column's weights only in its own head's product
        i16x4_t pbh[HP];
#pragma unroll
        for (int hh = 0; hh < HP; ++hh)
          pbh[hh] = __builtin_bit_cast(i16x4_t, (HP == 1 || hsel == hh) ? pw : uint2{0u, 0u});
        // O^T[dims][cols] += V^T[dims][keys] P^T[keys][cols], 16 dims per MFMA
#pragma unroll
        for (int db = 0; db < kDb; ++db) {
#pragma unroll
          for (int hh = 0; hh < HP; ++hh) {
            const i16x4_t va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_i16x4_t*)&vbuf[hh][tr_row * kVRow + stage_off<F8, D>(db * 16 + tr_col)]);
            acc[db] = mfma_16x16x16<H16>(va, pbh[hh], acc[db]);
          }
        }
      };

      // Ring schedule over the window padded to a multiple of kRing: every
      // group but the last refills each slot once its rows are staged
      // (branch-free, so the wait counts stay exact); the last group drains.
      const int n_groups = (wn + kRing - 1) / kRing;
#pragma unroll
      for (int s = 0; s < kRing; ++s) issue(s, s);
      for (int gi = 0; gi + 1 < n_groups; ++gi) {
#pragma unroll
        for (int s = 0; s < kRing; ++s)
          consume(s, std::integral_constant<bool, true>{}, (gi + 1) * kRing + s);
      }
#pragma unroll
      for (int s = 0; s < kRing; ++s) consume(s, std::integral_constant<bool, false>{}, 0);
    }

    // ---- segment epilogue: l over the four key groups, then the partial
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if constexpr (F8) {
#pragma unroll
      for (int db = 0; db < kDb; ++db) acc[db] *= v_scale;
    }
    // partial row (wi + b) * HPG + col of the group; the wave that ends the segment
    // writes each of its KV heads' descriptor {first row, count, row stride}
    const int prow0 = (wi + b) * HPG;
    if (col < HPG) {
      float* pr = gpart + (int64_t)(prow0 + col) * kPartRow;
#pragma unroll
      for (int db = 0; db < kDb; ++db)
        *reinterpret_cast<f32x4_t*>(&pr[db * 16 + g4 * 4]) = acc[db];
      if (g4 == 0) *reinterpret_cast<float2*>(&pr[D]) = float2{m_run, l_run};
    }
    if (c_lo + n_seg == nc && lane < HP) {
      const int64_t first = (int64_t)(Wh + batch) * qh0 + (int64_t)(w_first + b) * HPG +
                            lane * G;
      desc[((int64_t)b * Hk + kvh0 + lane) * NCG + cg] =
          i32x4v_t{(int32_t)first, wi - w_first + 1, HPG, 0};
    }
    k += n_seg;
  }
}

// N consecutive floats of a partial row (N = D / 64 output dims per lane).
template <int N>
__device__ __forceinline__ void load_dims(const float* p, float (&v)[N]) {
  if constexpr (N == 1) {
    v[0] = *p;
  } else if constexpr (N == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x;
    v[1] = t.y;
  } else {
    static_assert(N == 4, "1, 2 or 4 dims per lane");
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
    v[3] = t.w;
  }
}
// N output dims of one lane as bf16 or fp16 (2, 4 or 8 bytes).
template <bool H16>
__device__ __forceinline__ uint32_t out_pk(float lo, float hi) {
  if constexpr (H16) return cvt_pk16<true>(lo, hi);
  else return pack_bf16x2(lo, hi);
}
template <int N, bool H16>
__device__ __forceinline__ void store_dims(bf16_t* op, const float (&o)[N], float scale) {
  if constexpr (N == 1) {
    *reinterpret_cast<uint16_t*>(op) = (uint16_t)(out_pk<H16>(o[0] * scale, 0.f) & 0xffffu);
  } else if constexpr (N == 2) {
    *reinterpret_cast<uint32_t*>(op) = out_pk<H16>(o[0] * scale, o[1] * scale);
  } else {
    *reinterpret_cast<uint2*>(op) =
        uint2{out_pk<H16>(o[0] * scale, o[1] * scale), out_pk<H16>(o[2] * scale, o[3] * scale)};
  }
}

// Merge the partials of one (sequence, query head): O = sum_s 2^(m_s-M) O_s /
// sum_s 2^(m_s-M) l_s. One wave per pair; lane l owns output dims N*l .. N*l+N-1.
template <int D, bool H16 = false>
__global__ __launch_bounds__(64) void paged_decode_combine_kernel(
    const int32_t* __restrict__ context_lens, int32_t Hq, int32_t Hk, int32_t NCG,
    const float* __restrict__ part, const i32x4v_t* __restrict__ desc,
    bf16_t* __restrict__ out, int64_t out_row_stride) {
  static_assert(decode_dim_ok(D), "head_dim 64, 128 or 256");
  constexpr int N = D / 64;
  constexpr int kPartRow = part_row(D);
  const int b = blockIdx.x / Hq;
  const int h = blockIdx.x % Hq;
  const int lane = threadIdx.x;
  const int G = Hq / Hk;
  // The context length and the KV head's descriptor first (one round trip), then every
  // (m, l) pair and the first eight partial rows at once (the second).
  static_assert(kMaxSlots <= 128, "two partials per lane");
  const int ctx = context_lens[b];
  const int hq = h % G;                         // query head within the KV head's group
  const int cg = NCG > 1 ? hq / kMaxCols : 0;    // its column group (0 unless G > 16)
  const i32x4v_t d = desc[((int64_t)b * Hk + h / G) * NCG + cg];
  bf16_t* op = out + (int64_t)b * out_row_stride + (int64_t)h * D + N * lane;
  float o[N];
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = 0.f;
  // the descriptor is written by this call for every sequence with ctx > 0
  const int ns = ctx > 0 ? min(d.y, kMaxSlots) : 0;
  if (ns == 0) {
    store_dims<N, H16>(op, o, 0.f);
    return;
  }
  const int64_t stride = (int64_t)d.z * kPartRow;  // floats between a head's partials
  const float* pbase = part + ((int64_t)d.x + hq - cg * kMaxCols) * kPartRow;
  const float* po = pbase + N * lane;
  float2 ml0 = {-INFINITY, 0.f}, ml1 = {-INFINITY, 0.f};
  if (lane < ns) ml0 = *reinterpret_cast<const float2*>(pbase + lane * stride + D);
  if (lane + 64 < ns) ml1 = *reinterpret_cast<const float2*>(pbase + (lane + 64) * stride + D);
  float v0[16][N];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    if (u < ns) {
      load_dims<N>(po + u * stride, v0[u]);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) v0[u][i] = 0.f;
    }
  }
  // lane l holds partials l and l + 64 (ns <= kMaxSlots = 128): the global max and
  // the weights w_s = 2^(m_s - M) with two wave reductions, then each lane
  // accumulates its output dims over the partials in order (the first sixteen came
  // with the (m, l) pairs; the rest in batches of eight loads in flight)
  const float M = wave_max(fmaxf(ml0.x, ml1.x));
  const float w0 = (ml0.x == -INFINITY) ? 0.f : fast_exp2(ml0.x - M);
  const float w1 = (ml1.x == -INFINITY) ? 0.f : fast_exp2(ml1.x - M);
  const float L = wave_sum(w0 * ml0.y + w1 * ml1.y);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const float w = __shfl(w0, u, 64);
    if (u < ns) {  // uniform
#pragma unroll
      for (int i = 0; i < N; ++i) o[i] = fmaf(w, v0[u][i], o[i]);
    }
  }
  for (int s = 16; s < ns; s += 8) {  // uniform
    float v[8][N];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s + u < ns) load_dims<N>(po + (s + u) * stride, v[u]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float w = __shfl(s + u < 64 ? w0 : w1, (s + u) & 63, 64);  // uniform select
      if (s + u < ns) {
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = fmaf(w, v[u][i], o[i]);
      }
    }
  }
  store_dims<N, H16>(op, o, L > 0.f ? 1.f / L : 0.f);
}

static int decode_check(const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* block_tables, const int32_t* context_lens, int32_t batch,
                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t block_size, int32_t max_blocks_per_seq, int64_t q_row_stride,
                        int64_t bt_row_stride) {
  NKV_REQUIRE(batch >= 0 && n_kv_heads > 0 && n_q_heads > 0, NKV_EINVAL,
              "paged_decode: bad sizes (batch=%d, Hq=%d, Hk=%d)", batch, n_q_heads, n_kv_heads);
  NKV_REQUIRE(decode_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "paged_decode: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL,
              "paged_decode: n_q_heads %% n_kv_heads != 0 (%d, %d)", n_q_heads, n_kv_heads);
  const int g = n_q_heads / n_kv_heads;
  NKV_REQUIRE(g <= kMaxGroup, NKV_EUNSUPPORTED, "paged_decode: GQA group %d above %d", g,
              kMaxGroup);
  NKV_REQUIRE(block_size > 0 && block_size % kChunk == 0, NKV_EUNSUPPORTED,
              "paged_decode: block_size must be a multiple of 16 (got %d)", block_size);
  NKV_REQUIRE(max_blocks_per_seq > 0 && bt_row_stride >= max_blocks_per_seq, NKV_EINVAL,
              "paged_decode: bad block table width/stride (%d, %lld)", max_blocks_per_seq,
              (long long)bt_row_stride);
  NKV_REQUIRE((int64_t)max_blocks_per_seq * block_size < (1ll << 30), NKV_EUNSUPPORTED,
              "paged_decode: max_blocks_per_seq * block_size too large");
  NKV_REQUIRE((int64_t)block_size * n_kv_heads * head_dim * 2 < (1ll << 31), NKV_EUNSUPPORTED,
              "paged_decode: cache block too large for 32-bit buffer offsets");
  NKV_REQUIRE(q_row_stride >= (int64_t)n_q_heads * head_dim && q_row_stride % 8 == 0,
              NKV_EINVAL, "paged_decode: q row stride must be >= Hq*D and a multiple of 8");
  NKV_REQUIRE(q && k_cache && v_cache && block_tables && context_lens, NKV_EINVAL,
              "paged_decode: null pointer");
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache), NKV_EINVAL,
              "paged_decode: q/k_cache/v_cache must be 16-byte aligned");
  return NKV_OK;
}

// Compute units of the current device (cached per device; 256 when it cannot be queried).
static int device_cus() {
  // threads that race here compute and store the same value
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Persistent grid: as many one-wave workgroups as are resident at once, at most
// kWavesPerCU per CU (the workspace bound assumes no more).
template <bool F8, int HP, int D>
static int decode_grid() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(paged_decode_split_kernel<F8, HP, D>), 64,
            0) != hipSuccess ||
        per_cu <= 0)
      per_cu = kWavesPerCU;
    n = device_cus() * std::min(per_cu, kWavesPerCU);
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// KV heads per wave at most for head_dim D: a 512-byte piece of every token row
// (bf16: 4 / 2 / 1 at D = 64 / 128 / 256; fp8: 4 / 4 / 2).
template <bool F8>
static constexpr int decode_max_hp(int D) {
  const int hp = 512 / (D * (F8 ? 1 : 2));
  return hp > 4 ? 4 : hp;
}

// The resident grid of instance (F8, hp, D) -- hp and D from the plan.
template <bool F8>
static int decode_grid_of(int hp, int D) {
  if (D == 64) {
    return hp == 4 ? decode_grid<F8, 4, 64>() : hp == 2 ? decode_grid<F8, 2, 64>()
                                                        : decode_grid<F8, 1, 64>();
  }
  if (D == 128) {
    if constexpr (F8) {
      if (hp == 4) return decode_grid<true, 4, 128>();
    }
    return hp == 2 ? decode_grid<F8, 2, 128>() : decode_grid<F8, 1, 128>();
  }
  if constexpr (F8) {
    if (hp == 2) return decode_grid<true, 2, 256>();
  }
  return decode_grid<F8, 1, 256>();
}

// The launch a decode call makes: KV heads per wave, the grid and the smallest range.
struct DecodePlan {
  int hp;          // KV heads per wave (1, 2 or 4)
  int ncg;         // column groups per KV head (1 unless G > 16; then hp = 1)
  unsigned grid;   // one-wave workgroups
  int32_t min_chunks;
};

static int64_t decode_useful_waves(int32_t batch, int32_t max_blocks, int32_t block_size) {
  const int64_t max_chunks = ((int64_t)max_blocks * block_size + kChunk - 1) / kChunk;
  const int32_t min_chunks = decode_min_chunks(max_blocks, block_size);
  return std::max<int64_t>(1, (batch * max_chunks + min_chunks - 1) / min_chunks);
}

template <bool F8>
static DecodePlan decode_plan(int32_t batch, int32_t Hq, int32_t Hk, int32_t max_blocks,
                              int32_t block_size, int32_t D) {
  const int g = Hq / Hk;
  const int64_t max_chunks = ((int64_t)max_blocks * block_size + kChunk - 1) / kChunk;
  // Several KV heads per wave (up to a 512-byte piece of every token row) when the heads
  // group evenly, the hp*G query heads fit the 16 MFMA columns and there is enough work
  // for every wave (upper bound from the table width: >= 32 chunks per head group per
  // resident wave of the two-head instance); otherwise one.
  const int64_t work = (int64_t)batch * max_chunks * Hk;
  int hp = 1;
  if (decode_max_hp<F8>(D) >= 2 && Hk % 2 == 0 && 2 * g <= kMaxCols &&
      work >= 32 * (int64_t)decode_grid_of<F8>(2, D)) {
    hp = 2;
    if (decode_max_hp<F8>(D) >= 4 && Hk % 4 == 0 && 4 * g <= kMaxCols) hp = 4;
  }
  DecodePlan p;
  p.hp = hp;
  p.ncg = decode_ncg(g);
  p.min_chunks = decode_min_chunks(max_blocks, block_size);
  // Resident waves per head group, but no more than the table width lets receive a range
  // of min_chunks (small batches launch only the waves that can get work).
  const int resident = decode_grid_of<F8>(hp, D);
  const int np = Hk * p.ncg / p.hp;
  const int64_t per =
      std::min<int64_t>(std::max(1, resident / np), decode_useful_waves(batch, max_blocks,
                                                                        block_size));
  p.grid = (unsigned)(per * np);
  return p;
}

// Bytes of the descriptors (one per sequence, KV head and column group; 16-byte aligned)
// and of the partial rows a plan writes: each head group (waves + batch) x its columns,
// i.e. (grid / head groups + batch) x Hq rows in all (grid * hp*g + batch * Hq for G <= 16;
// at most grid * 16 + batch * Hq).
static size_t decode_desc_bytes(int32_t batch, int32_t n_groups) {
  return (size_t)batch * n_groups * sizeof(i32x4v_t);
}
static size_t decode_part_bytes(int64_t waves, int32_t batch, int32_t Hq, int32_t D) {
  return (size_t)((waves + batch) * (int64_t)Hq) * part_row(D) * sizeof(float);
}
// Waves per head group of a plan.
static int64_t decode_waves(const DecodePlan& p, int32_t Hk) {
  return (int64_t)p.grid / (Hk * p.ncg / p.hp);
}

}  // namespace nkv

extern "C" size_t nkv_paged_decode_workspace_bytes(int32_t batch, int32_t n_q_heads,
                                                   int32_t head_dim, int32_t max_blocks_per_seq,
                                                   int32_t block_size) {
  using namespace nkv;
  if (batch <= 0 || n_q_heads <= 0 || max_blocks_per_seq <= 0 || block_size <= 0 ||
      !decode_dim_ok(head_dim))
    return 0;
  // Whatever the plan: waves per head group x Hq <= grid x min(16, Hq) (a group's columns
  // are at most 16 and the groups' columns add up to Hq), grid <= CUs * kWavesPerCU and
  // grid <= useful * (head groups); the descriptors (per KV head and column group) at most
  // batch * Hq.
  const int64_t resident = (int64_t)device_cus() * kWavesPerCU;
  const int64_t cols = std::min<int64_t>(
      resident * std::min(kMaxCols, n_q_heads),
      decode_useful_waves(batch, max_blocks_per_seq, block_size) * n_q_heads);
  return decode_desc_bytes(batch, n_q_heads) + decode_part_bytes(0, batch, n_q_heads, head_dim) +
         (size_t)cols * part_row(head_dim) * sizeof(float);
}

namespace nkv {
template <bool F8, bool H16 = false>
static int decode_split(const void* q, int64_t q_row_stride, const void* k_cache,
                        const void* v_cache, const int32_t* block_tables, int64_t bt_row_stride,
                        const int32_t* context_lens, int32_t batch, int32_t n_q_heads,
                        int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                        int32_t max_blocks_per_seq, int64_t n_blocks, float scale, float k_scale,
                        float v_scale, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = decode_check(q, k_cache, v_cache, block_tables, context_lens, batch, n_q_heads,
                        n_kv_heads, head_dim, block_size, max_blocks_per_seq, q_row_stride,
                        bt_row_stride);
  if (rc) return rc;
  if (batch == 0) return NKV_OK;
  NKV_REQUIRE(k_scale > 0.f && v_scale > 0.f, NKV_EINVAL, "paged_decode: scales must be > 0");
  const int64_t max_chunks = ((int64_t)max_blocks_per_seq * block_size + kChunk - 1) / kChunk;
  NKV_REQUIRE(max_chunks * batch * n_kv_heads < (1ll << 31), NKV_EUNSUPPORTED,
              "paged_decode: too many chunks in one call");
  const int g = n_q_heads / n_kv_heads;
  const DecodePlan p = decode_plan<F8>(batch, n_q_heads, n_kv_heads, max_blocks_per_seq,
                                       block_size, head_dim);
  const size_t desc_b = decode_desc_bytes(batch, n_kv_heads * p.ncg);
  const int64_t waves = decode_waves(p, n_kv_heads);
  const size_t need = desc_b + decode_part_bytes(waves, batch, n_q_heads, head_dim);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "paged_decode: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  NKV_REQUIRE((waves + batch) * n_q_heads < (1ll << 31), NKV_EUNSUPPORTED,
              "paged_decode: too many partial rows");
  i32x4v_t* desc = static_cast<i32x4v_t*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + desc_b);
  const float scale_log2 = scale * k_scale * kLog2e;
  hipStream_t s = as_stream(stream);
#define NKV_DECODE_LAUNCH(HP, D)                                                               \
  hipLaunchKernelGGL((paged_decode_split_kernel<F8, HP, D, H16>), dim3(p.grid), dim3(64), 0, s, \
                     (const bf16_t*)q, q_row_stride, k_cache, v_cache, block_tables,           \
                     bt_row_stride, context_lens, batch, n_kv_heads, g, p.ncg, block_size,     \
                     max_blocks_per_seq, n_blocks, p.min_chunks, scale_log2, v_scale, part,    \
                     desc)
  if (head_dim == 64) {
    if (p.hp == 4) NKV_DECODE_LAUNCH(4, 64);
    else if (p.hp == 2) NKV_DECODE_LAUNCH(2, 64);
    else NKV_DECODE_LAUNCH(1, 64);
  } else if (head_dim == 128) {
    if (p.hp == 4) {
      if constexpr (F8) NKV_DECODE_LAUNCH(4, 128);
    } else if (p.hp == 2) {
      NKV_DECODE_LAUNCH(2, 128);
    } else {
      NKV_DECODE_LAUNCH(1, 128);
    }
  } else {
    if (p.hp == 2) {
      if constexpr (F8) NKV_DECODE_LAUNCH(2, 256);
    } else {
      NKV_DECODE_LAUNCH(1, 256);
    }
  }
#undef NKV_DECODE_LAUNCH
  return check_launch("nkv_paged_decode_split");
}

// The combine of a split launched with the same arguments: the partial rows start after
// the descriptors, whatever the plan.
template <bool H16 = false>
static int decode_combine(const int32_t* context_lens, int32_t batch, int32_t n_q_heads,
                          int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                          int32_t max_blocks_per_seq, void* out, int64_t out_row_stride,
                          const void* workspace, size_t workspace_bytes, void* stream) {
  NKV_REQUIRE(decode_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "paged_decode: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(batch >= 0 && n_q_heads > 0 && n_kv_heads > 0 && n_q_heads % n_kv_heads == 0 &&
                  n_q_heads / n_kv_heads <= kMaxGroup && block_size > 0 &&
                  max_blocks_per_seq > 0,
              NKV_EINVAL, "paged_decode_combine: bad sizes");
  const int ncg = decode_ncg(n_q_heads / n_kv_heads);
  if (batch == 0) return NKV_OK;
  NKV_REQUIRE(out && context_lens, NKV_EINVAL, "paged_decode_combine: null pointer");
  // each lane stores D/64 consecutive bf16 (2, 4 or 8 bytes)
  const int al = head_dim / 64;  // elements per lane store
  NKV_REQUIRE(out_row_stride >= (int64_t)n_q_heads * head_dim && out_row_stride % al == 0 &&
                  (reinterpret_cast<uintptr_t>(out) & (2 * al - 1)) == 0,
              NKV_EINVAL,
              "paged_decode_combine: out must be %d-byte aligned with a row stride >= Hq*D "
              "that is a multiple of %d", 2 * al, al);
  const size_t desc_b = decode_desc_bytes(batch, n_kv_heads * ncg);
  NKV_REQUIRE(workspace && workspace_bytes > desc_b, NKV_EWORKSPACE,
              "paged_decode_combine: workspace of %zu bytes holds no partials",
              workspace_bytes);
  const i32x4v_t* desc = static_cast<const i32x4v_t*>(workspace);
  const float* part = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + desc_b);
  const dim3 grid((unsigned)(batch * n_q_heads));
#define NKV_COMBINE_LAUNCH(D)                                                                  \
  hipLaunchKernelGGL((paged_decode_combine_kernel<D, H16>), grid, dim3(64), 0,                 \
                     as_stream(stream), context_lens, n_q_heads, n_kv_heads, ncg, part, desc,  \
                     (bf16_t*)out, out_row_stride)
  if (head_dim == 64) NKV_COMBINE_LAUNCH(64);
  else if (head_dim == 128) NKV_COMBINE_LAUNCH(128);
  else NKV_COMBINE_LAUNCH(256);
#undef NKV_COMBINE_LAUNCH
  return check_launch("nkv_paged_decode_combine");
}
}  // namespace nkv

extern "C" int nkv_paged_decode_split(const void* q, int64_t q_row_stride, const void* k_cache,
                                      const void* v_cache, const int32_t* block_tables,
                                      int64_t bt_row_stride, const int32_t* context_lens,
                                      int32_t batch, int32_t n_q_heads, int32_t n_kv_heads,
                                      int32_t head_dim, int32_t block_size,
                                      int32_t max_blocks_per_seq, int64_t n_blocks, float scale,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  nkv::clear_error();
  return nkv::decode_split<false>(q, q_row_stride, k_cache, v_cache, block_tables,
                                  bt_row_stride, context_lens, batch, n_q_heads, n_kv_heads,
                                  head_dim, block_size, max_blocks_per_seq, n_blocks, scale, 1.f,
                                  1.f, workspace, workspace_bytes, stream);
}

extern "C" int nkv_paged_decode_combine(const int32_t* context_lens, int32_t batch,
                                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                        int32_t block_size, int32_t max_blocks_per_seq,
                                        void* out, int64_t out_row_stride, const void* workspace,
                                        size_t workspace_bytes, void* stream) {
  nkv::clear_error();
  return nkv::decode_combine(context_lens, batch, n_q_heads, n_kv_heads, head_dim, block_size,
                             max_blocks_per_seq, out, out_row_stride, workspace, workspace_bytes,
                             stream);
}

extern "C" int nkv_paged_decode(const void* q, int64_t q_row_stride, const void* k_cache,
                                const void* v_cache, const int32_t* block_tables,
                                int64_t bt_row_stride, const int32_t* context_lens, int32_t batch,
                                int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                int32_t block_size, int32_t max_blocks_per_seq, int64_t n_blocks,
                                float scale, void* out, int64_t out_row_stride, void* workspace,
                                size_t workspace_bytes, void* stream) {
  int rc = nkv_paged_decode_split(q, q_row_stride, k_cache, v_cache, block_tables, bt_row_stride,
                                  context_lens, batch, n_q_heads, n_kv_heads, head_dim,
                                  block_size, max_blocks_per_seq, n_blocks, scale, workspace,
                                  workspace_bytes, stream);
  if (rc) return rc;
  return nkv_paged_decode_combine(context_lens, batch, n_q_heads, n_kv_heads, head_dim,
                                  block_size, max_blocks_per_seq, out, out_row_stride, workspace,
                                  workspace_bytes, stream);
}

extern "C" int nkv_paged_decode_f16(const void* q, int64_t q_row_stride, const void* k_cache,
                                    const void* v_cache, const int32_t* block_tables,
                                    int64_t bt_row_stride, const int32_t* context_lens,
                                    int32_t batch, int32_t n_q_heads, int32_t n_kv_heads,
                                    int32_t head_dim, int32_t block_size,
                                    int32_t max_blocks_per_seq, int64_t n_blocks, float scale,
                                    void* out, int64_t out_row_stride, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  nkv::clear_error();
  int rc = nkv::decode_split<false, true>(q, q_row_stride, k_cache, v_cache, block_tables,
                                          bt_row_stride, context_lens, batch, n_q_heads,
                                          n_kv_heads, head_dim, block_size, max_blocks_per_seq,
                                          n_blocks, scale, 1.f, 1.f, workspace, workspace_bytes,
                                          stream);
  if (rc) return rc;
  return nkv::decode_combine<true>(context_lens, batch, n_q_heads, n_kv_heads, head_dim,
                                   block_size, max_blocks_per_seq, out, out_row_stride,
                                   workspace, workspace_bytes, stream);
}

extern "C" int nkv_paged_decode_fp8(const void* q, int64_t q_row_stride, const void* k_cache,
                                    const void* v_cache, const int32_t* block_tables,
                                    int64_t bt_row_stride, const int32_t* context_lens,
                                    int32_t batch, int32_t n_q_heads, int32_t n_kv_heads,
                                    int32_t head_dim, int32_t block_size,
                                    int32_t max_blocks_per_seq, int64_t n_blocks, float scale,
                                    float k_scale, float v_scale, void* out,
                                    int64_t out_row_stride, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  nkv::clear_error();
  int rc = nkv::decode_split<true>(q, q_row_stride, k_cache, v_cache, block_tables,
                                   bt_row_stride, context_lens, batch, n_q_heads, n_kv_heads,
                                   head_dim, block_size, max_blocks_per_seq, n_blocks, scale,
                                   k_scale, v_scale, workspace, workspace_bytes, stream);
  if (rc) return rc;
  return nkv_paged_decode_combine(context_lens, batch, n_q_heads, n_kv_heads, head_dim,
                                  block_size, max_blocks_per_seq, out, out_row_stride, workspace,
                                  workspace_bytes, stream);
}

// ------------------------------------------------------------------ no-allocation variant
// The decode workspace in a fixed device array: for callers that cannot allocate (code
// under graph capture, tight serving loops). Each device holds its own copy of the array
// for the life of the process. Host code never passes the array's name to a kernel (on
// the host it is only a stand-in): its device address comes from hipGetSymbolAddress,
// taken once per device on the first call there, with that device current.
namespace nkv {
constexpr size_t kScratchBytes = NKV_DECODE_NOALLOC_MAX_BYTES;  // batch*Hq up to ~94k heads
}  // namespace nkv

static __device__ __align__(256) unsigned char scratch[nkv::kScratchBytes];

namespace nkv {
// Device address of `scratch` on the current device, or nullptr (error text set).
static void* scratch_ptr() {
  static std::atomic<void*> ptrs[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("paged_decode_noalloc: no current device");
    return nullptr;
  }
  void* p = ptrs[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    // threads that race here obtain the same address
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("paged_decode_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    ptrs[dev].store(p, std::memory_order_release);
  }
  return p;
}
}  // namespace nkv

extern "C" int nkv_paged_decode_noalloc(const void* q, int64_t q_row_stride, const void* k_cache,
                                        const void* v_cache, const int32_t* block_tables,
                                        int64_t bt_row_stride, const int32_t* context_lens,
                                        int32_t batch, int32_t n_q_heads, int32_t n_kv_heads,
                                        int32_t head_dim, int32_t block_size,
                                        int32_t max_blocks_per_seq, int64_t n_blocks,
                                        float scale, void* out, int64_t out_row_stride,
                                        void* stream) {
  using namespace nkv;
  clear_error();
  int rc = decode_check(q, k_cache, v_cache, block_tables, context_lens, batch, n_q_heads,
                        n_kv_heads, head_dim, block_size, max_blocks_per_seq, q_row_stride,
                        bt_row_stride);
  if (rc) return rc;
  if (batch == 0) return NKV_OK;
  // the bytes this call's plan needs, against the array's fixed size
  const DecodePlan p = decode_plan<false>(batch, n_q_heads, n_kv_heads, max_blocks_per_seq,
                                          block_size, head_dim);
  const size_t need = decode_desc_bytes(batch, n_kv_heads * p.ncg) +
                      decode_part_bytes(decode_waves(p, n_kv_heads), batch, n_q_heads,
                                        head_dim);
  NKV_REQUIRE(need <= kScratchBytes, NKV_EUNSUPPORTED,
              "paged_decode_noalloc: batch %d x %d query heads needs %zu bytes of partials, "
              "above the fixed %zu-byte array; use nkv_paged_decode with a workspace",
              batch, n_q_heads, need, kScratchBytes);
  void* ws = scratch_ptr();
  if (ws == nullptr) return NKV_ELAUNCH;
  rc = decode_split<false>(q, q_row_stride, k_cache, v_cache, block_tables, bt_row_stride,
                           context_lens, batch, n_q_heads, n_kv_heads, head_dim, block_size,
                           max_blocks_per_seq, n_blocks, scale, 1.f, 1.f, ws, kScratchBytes,
                           stream);
  if (rc) return rc;
  return decode_combine(context_lens, batch, n_q_heads, n_kv_heads, head_dim, block_size,
                        max_blocks_per_seq, out, out_row_stride, ws, kScratchBytes, stream);
}

// Varlen causal prefill over the paged K/V cache (bf16 MFMA, fp32 softmax).
//
// Reference: flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
// max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True, block_table) at
// nanokvllm/layers/attention.py:96-102 (bottom-right causal alignment: query
// j of a sequence with Lq queries and Lk keys sees keys 0 .. Lk-Lq+j).
//
// MI355X design (MFMA-bound):
//  * Workgroup = (sequence, tile of floor(R/g) queries, KV head) x 4 waves.
//    The tile's R "rows" are its queries for all g query heads of the KV
//    head, query-major (row r = query r/g, head r%g; rows past the tile's
//    queries x g are computed and dropped), so one K/V tile in LDS serves g
//    heads (GQA sharing). Wave w owns three 16-row groups at head_dim 128
//    (R = 192), two at 64 and in the fp8 instance (R = 128), one at 256
//    (R = 64, and the 128 KiB ring leaves one workgroup per CU). head_dim D
//    is 64, 128 or 256 (a template parameter).
//  * Keys advance in 64-key steps. Each step's K and V tiles (2 x 16 KiB at
//    D = 128) go from HBM straight into LDS with gfx950's 16-byte buffer-load-to-LDS
//    (no staging registers, no LDS write instructions) through a ring of
//    kStages tiles, issued kStages-1 steps ahead; one barrier per step.
//    LDS rows are dense (2D bytes) with the 16-byte chunks of row r XOR-permuted
//    by chunk_swz(r), which keeps both the K row reads and the V transpose reads
//    free of bank conflicts; the permutation is applied on the global side
//    (each lane fetches the chunk that belongs at its fixed LDS slot).
//  * S^T = K Q^T  (v_mfma_f32_16x16x32_bf16: A = 16 keys from LDS, B = the
//    wave's Q^T held in registers for the whole sequence) puts, in lane l,
//    row l%16 and keys 4(l/16)..+3 of each 16-key quarter. Two quarters make
//    the B operand of  O^T += V^T P^T  (16x16x32 over 32 keys) once their
//    weights are packed to bf16; V^T (A operand) comes from LDS with two
//    ds_read_b64_tr_b16 per 16-dim block and 32-key chunk. Each lane owns one row: the
//    online softmax needs one max over the 4 key groups per step.
//  * Causal: a tile stops at its last visible key; masks are applied per
//    element only where needed. Tiles are dispatched largest-first and the
//    KV head is the fastest grid index, so with 8 KV heads each head's tiles
//    share one XCD's L2.
//  * F8 (paged fp8 pool): K/V tiles come as 1-byte E4M3FN codes through
//    registers instead of straight into LDS: the next step's codes are loaded
//    while this step computes, then widened to bf16 (exact) and written to the
//    same swizzled LDS rows, so the MFMA part is the bf16 kernel's. The K scale
//    is folded into the softmax scale, the V scale into the final 1/l.
#include "nkv_common.h"

#include <algorithm>
#include <type_traits>

namespace nkv {

constexpr int kStep = 64;                 // keys per step
constexpr int kStages = 2;                // LDS ring depth (steps)
constexpr int kBufferFlags = 0x00020000;  // raw buffer descriptor word 3 for gfx950
constexpr bool prefill_dim_ok(int D) { return D == 64 || D == 128 || D == 256; }
// 16-row groups per wave: three at head_dim 128 (each K and V^T read from LDS serves three
// MFMAs; bit-identical to two, at par to 2% faster), two at 64 and in the fp8 instance (whose
// staging registers leave no room for a third), one at 256 (its O^T and Q^T registers
// would not fit two waves per SIMD otherwise)
constexpr int prefill_row_groups(int D, bool F8) {
  return D == 256 ? 1 : (D == 128 && !F8 ? 3 : 2);
}
// rows (query, head pairs) of a workgroup's tile: 4 waves
constexpr int prefill_tile_rows(int D, bool F8) { return 64 * prefill_row_groups(D, F8); }
// largest GQA group, the same for every instance of a head_dim: each tile holds at least
// one query for all g heads of its KV head
constexpr int prefill_max_group(int D) { return D == 256 ? 64 : 128; }
// XOR applied to the 16-byte chunk index of LDS row r (even: chunk pairs stay together).
// Keeps the K row reads and the V transpose reads free of bank conflicts: 2*(r & 7) for
// 256- and 512-byte rows, 2*((r >> 1) & 3) for 128-byte rows (two rows per bank line).
template <int D>
__device__ __forceinline__ int chunk_swz(int r) {
  if constexpr (D == 64) return 2 * ((r >> 1) & 3);
  else return 2 * (r & 7);
}
constexpr float kLazy = 8.f;              // log2 headroom before the running max is raised

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4_t;
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

// Output pair: bf16 with the round-to-nearest-even of pack_bf16x2, or fp16.
template <bool H16>
__device__ __forceinline__ uint32_t out_pack(float a, float b) {
  if constexpr (H16) return cvt_pk16<true>(a, b);
  else return pack_bf16x2(a, b);
}
// Raw buffer descriptor over [base, base + bytes): loads past `bytes` return 0.
__device__ __forceinline__ i32x4_t buffer_desc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return i32x4_t{__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a),
                 __builtin_amdgcn_readfirstlane((int32_t)((a >> 32) & 0xffffu)),
                 __builtin_amdgcn_readfirstlane((int32_t)bytes), kBufferFlags};
}
// 16 bytes per lane from desc+voff into LDS at lds_addr + 16 * lane. Written as
// asm so that the compiler does not add a wait for it before every barrier;
// the ring's own s_waitcnt (vmcnt) orders it.
__device__ __forceinline__ void load_to_lds(i32x4_t desc, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(desc)
               : "memory");
}

template <bool F8, int D, bool H16, bool PAGED>
__global__ __launch_bounds__(256, D == 256 ? 1 : 2) void prefill_varlen_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride, const void* __restrict__ k_cache,
    const void* __restrict__ v_cache, int64_t k_row_stride, int64_t v_row_stride,
    const int32_t* __restrict__ cu_seqlens_q, const int32_t* __restrict__ cu_seqlens_k,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t Hk, int32_t G,
    int32_t block_size, int32_t max_blocks, int32_t n_limit, int32_t n_tiles, float scale_log2,
    float v_scale, bf16_t* __restrict__ out, int64_t out_row_stride) {
  static_assert(prefill_dim_ok(D), "head_dim 64, 128 or 256");
  static_assert(!(F8 && H16), "fp8 caches are read with bf16 queries");
  constexpr int kEl = F8 ? 1 : 2;          // bytes per cache element
  constexpr int kRB = D * 2;               // bytes of a staged (bf16) K or V row
  constexpr int kNC = D / 8;               // 16-byte chunks per staged row
  constexpr int kRG = prefill_row_groups(D, F8);
  constexpr int kTileB = kStep * kRB;      // bytes of one K or V tile
  constexpr int kStageB = 2 * kTileB;      // K tile then V tile
  constexpr int kKs = D / 32;              // k-steps of S^T
  constexpr int kDb = D / 16;              // 16-dim blocks of O^T
  constexpr int kRpl = 1024 / kRB;         // rows per 1 KiB load into LDS
  constexpr int kNl = 16 / kRpl;           // such loads per wave per tile
  constexpr int kLpr8 = D / 16;            // F8: lanes per row (16 codes each)
  constexpr int kRpl8 = 64 / kLpr8;        // F8: rows per load
  constexpr int kNl8 = 16 / kRpl8;         // F8: loads per wave per tile
  const int QT = prefill_tile_rows(D, F8) / G;  // queries per tile
  __shared__ __attribute__((aligned(1024))) char ring[kStages * kStageB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4;
  const int col = lane & 15;

  const int kvh = blockIdx.x % Hk;
  const int rest = blockIdx.x / Hk;
  const int tile = n_tiles - 1 - rest % n_tiles;  // largest tiles first
  const int seq = rest / n_tiles;
  const int q0 = cu_seqlens_q[seq];
  const int Lq = cu_seqlens_q[seq + 1] - q0;
  const int kb0 = cu_seqlens_k[seq];
  const int Lk = cu_seqlens_k[seq + 1] - kb0;
  const int j0 = tile * QT;
  NKV_DBG(tid == 0 && tile == 0 && (Lq < 0 || Lk < 0 || Lq > Lk), NKV_DEBUG_LENGTH);
  if (j0 >= Lq) return;  // uniform
  const int diag = Lk - Lq;  // query j sees keys <= diag + j
  const int last_key = min(Lk - 1, diag + j0 + QT - 1);
  const int n_steps = last_key >= 0 ? last_key / kStep + 1 : 0;

  // ---- K/V tile loads. Wave w fills rows 16w .. 16w+15 of a tile with 1 KiB
  // loads (kRpl rows each: 4 at head_dim 128); lane i of load h lands at row
  // 16w + kRpl*h + i/kNC, slot i%kNC, and fetches the row's chunk
  // (i%kNC) ^ chunk_swz(row). A wave's 16
  // keys are consecutive rows (one cache block, B % 16 == 0, or the contiguous
  // K/V), so each wave's share of a step is one uniform base row and a byte
  // window covering only its valid keys: keys past Lk and keys of invalid
  // blocks read as 0. vol[] are the K offsets; V rows may have another stride
  // (contiguous mode), and their offsets differ by r * (row_bv - row_b).
  const uint32_t row_b = (uint32_t)k_row_stride * kEl;
  const uint32_t row_bv = (uint32_t)v_row_stride * kEl;
  const int lrow = lane / kNC;
  const int slot = lane % kNC;
  uint32_t vol[kNl];
#pragma unroll
  for (int h = 0; h < kNl; ++h) {
    const int r = kRpl * h + lrow;  // row within the wave's 16 (16w + r within the tile)
    vol[h] = (uint32_t)r * row_b + (uint32_t)kvh * (D * 2) +
             (uint32_t)(slot ^ chunk_swz<D>(r)) * 16u;
  }
  const uint32_t ring_base =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)ring +
      (uint32_t)wave * (16u * kRB);
  // F8: load f of the wave's K (or V) codes brings rows kRpl8*f + lane/kLpr8, bytes
  // 16*(lane%kLpr8) of the head's D-byte piece, i.e. logical bf16 chunks 2c, 2c+1
  // (c = lane%kLpr8) of that LDS row
  const int f8_row0 = lane / kLpr8;
  const int f8_c = lane % kLpr8;
  u32x4_t kq[kNl8], vq[kNl8];  // F8: the next step's codes

  // Block ids: lane i holds entry bt_base + i of the sequence's table row, read
  // by the uniform v_readlane of the wave's block (reloaded every 64 blocks).
  const int32_t* bt = PAGED ? block_tables + (int64_t)seq * bt_row_stride : nullptr;
  int bt_base = 0;
  int bt_lane = -1;
  auto load_window = [&]() {
    const int e = bt_base + lane;
    const int id = e < max_blocks ? bt[e] : -1;
    NKV_DBG((int64_t)e * block_size < Lk && (e >= max_blocks || id < 0 || id >= n_limit),
            e >= max_blocks ? NKV_DEBUG_LENGTH : NKV_DEBUG_BLOCK);
    bt_lane = (id >= 0 && id < n_limit) ? id : -1;
  };
  // cursor of this wave's rows in the step loaded next: first key c_t0,
  // block c_blk, offset c_off in it
  int c_t0 = 16 * wave, c_blk = 0, c_off = 0;
  if constexpr (PAGED) {
    c_blk = c_t0 / block_size;
    c_off = c_t0 - c_blk * block_size;
    bt_base = c_blk & ~63;
    load_window();
  }
  // Scalar selects only (no branches), so that the compiler can spread it between the
  // MFMAs that follow its call.
  auto issue = [&](int stage) {
    int nv = min(16, Lk - c_t0);
    int64_t row0;
    if constexpr (PAGED) {
      const int pb = __builtin_amdgcn_readlane(bt_lane, c_blk - bt_base);
      nv = pb < 0 ? 0 : nv;
      row0 = (int64_t)pb * block_size + c_off;
    } else {
      const int r0 = kb0 + c_t0;
      NKV_DBG(nv > 0 && (r0 < 0 || r0 > n_limit - nv), NKV_DEBUG_BLOCK);
      nv = (r0 < 0 || r0 > n_limit - nv) ? 0 : nv;  // outside the K/V rows
      row0 = r0;
    }
    nv = max(nv, 0);
    row0 = nv > 0 ? row0 : 0;
    const char* kp = static_cast<const char*>(k_cache) + row0 * k_row_stride * kEl;
    const char* vp = static_cast<const char*>(v_cache) + row0 * v_row_stride * kEl;
    if constexpr (F8) {  // into registers; widened into the stage by commit()
      (void)stage;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          (void*)kp, (short)0, (uint32_t)nv * row_b, kBufferFlags);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          (void*)vp, (short)0, (uint32_t)nv * row_bv, kBufferFlags);
#pragma unroll
      for (int f = 0; f < kNl8; ++f) {
        const uint32_t r = (uint32_t)(kRpl8 * f + f8_row0);
        const uint32_t col = (uint32_t)kvh * D + (uint32_t)f8_c * 16u;
        kq[f] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, r * row_b + col, 0, 0));
        vq[f] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, r * row_bv + col, 0, 0));
      }
    } else {
      const i32x4_t dk = buffer_desc(kp, (uint32_t)nv * row_b);
      const i32x4_t dv = buffer_desc(vp, (uint32_t)nv * row_bv);
      const uint32_t at = ring_base + (uint32_t)stage * kStageB;
#pragma unroll
      for (int h = 0; h < kNl; ++h) load_to_lds(dk, at + 1024u * h, vol[h]);
#pragma unroll
      for (int h = 0; h < kNl; ++h)
        load_to_lds(dv, at + kTileB + 1024u * h,
                    vol[h] + (uint32_t)(kRpl * h + lrow) * (row_bv - row_b));
    }
    c_t0 += kStep;
    if constexpr (PAGED) {  // blocks crossed: at most 4 (c_off < block_size, a multiple of 16)
      const int v = c_off + kStep;
      const int n = (v >= block_size) + (v >= 2 * block_size) + (v >= 3 * block_size) +
                    (v >= 4 * block_size);
      c_off = v - n * block_size;
      c_blk = __builtin_amdgcn_readfirstlane(c_blk + n);
    }
  };
  auto refill_window = [&]() {  // uniform; once per 64 blocks
    if constexpr (PAGED) {
      if (c_blk - bt_base >= 64) {
        bt_base = c_blk & ~63;
        load_window();
      }
    }
  };
  // F8: the codes of the last issue() (after their loads land) widened into LDS stage
  // `stage`, rows 16w .. 16w+15 of the K and V tiles, in the bf16 path's swizzled layout
  // Lanes in the second half of a row write their pair's second chunk first (their codes'
  // halves swapped before widening), so each 16-byte write instruction covers distinct
  // bank groups of a row instead of pairing them up.
  const bool f8_swap = f8_c >= kLpr8 / 2;
  auto commit = [&](int stage) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    char* at = ring + stage * kStageB + wave * (16 * kRB);
#pragma unroll
    for (int f = 0; f < kNl8; ++f) {
      const int r = kRpl8 * f + f8_row0;  // row within the wave's 16 (16w + r within the tile)
      const int off = r * kRB + ((2 * f8_c) ^ chunk_swz<D>(r)) * 16;  // chunks 2c, 2c+1: adjacent
      const int o1 = off + (f8_swap ? 16 : 0), o2 = off + (f8_swap ? 0 : 16);
      u32x4_t lo, hi;
      u32x4_t c = kq[f];
      if (f8_swap) c = u32x4_t{c[2], c[3], c[0], c[1]};
      fp8x16_to_bf16(c, lo, hi);
      *reinterpret_cast<u32x4_t*>(at + o1) = lo;
      *reinterpret_cast<u32x4_t*>(at + o2) = hi;
      c = vq[f];
      if (f8_swap) c = u32x4_t{c[2], c[3], c[0], c[1]};
      fp8x16_to_bf16(c, lo, hi);
      *reinterpret_cast<u32x4_t*>(at + kTileB + o1) = lo;
      *reinterpret_cast<u32x4_t*>(at + kTileB + o2) = hi;
    }
  };

  // ---- prologue: the first kStages-1 steps in flight, then Q
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st) {
    issue(st);
    refill_window();
  }

  // ---- this wave's row groups: head and query of this lane's row (query-major;
  // rows past QT*G take query Lq: attended like the others, never stored)
  int head[kRG], jrow[kRG];
#pragma unroll
  for (int rr = 0; rr < kRG; ++rr) {
    const int r = (wave * kRG + rr) * 16 + col;
    const bool real = r < QT * G;
    head[rr] = real ? r % G : 0;
    jrow[rr] = real ? j0 + r / G : Lq;
  }
  // Q^T as the MFMA B operand: lane l -> row l%16, dims 8*(l/16) + 32*ks
  u32x4_t qreg[kRG][kKs];
#pragma unroll
  for (int rr = 0; rr < kRG; ++rr) {
    const int jc = jrow[rr] < Lq ? jrow[rr] : j0;  // rows past the sequence: discarded
    const u32x4_t* qp = reinterpret_cast<const u32x4_t*>(
        q + (int64_t)(q0 + jc) * q_row_stride + (int64_t)(kvh * G + head[rr]) * D + g4 * 8);
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) qreg[rr][ks] = qp[ks * 4];
  }

  // LDS read offsets (bytes from a tile's start). K A operand, 16-key half hh,
  // dims 32ks + 8*g4: row 16hh + col, logical chunk g4 + 4ks.
  uint32_t ko[kKs];
#pragma unroll
  for (int ks = 0; ks < kKs; ++ks)
    ko[ks] = (uint32_t)col * kRB + (uint32_t)((g4 + 4 * ks) ^ chunk_swz<D>(col)) * 16u;
  // V^T via ds_read_b64_tr_b16: lane 16g + 4r + c reads row 4g + r (and +16),
  // dims 16db + 4c .. +3 = logical chunk 2db + c/2, half c%2.
  const int vrow = 4 * g4 + (col >> 2);
  const int vc = col & 3;
  uint32_t vo[kDb];
#pragma unroll
  for (int db = 0; db < kDb; ++db)
    vo[db] = (uint32_t)vrow * kRB + (uint32_t)(db ^ (chunk_swz<D>(vrow) >> 1)) * 32u +
             (uint32_t)vc * 8u;

  f32x4_t acc[kRG][kDb];  // O^T: lane l -> row l%16, dims 16*db + 4*(l/16) .. +3
#pragma unroll
  for (int rr = 0; rr < kRG; ++rr)
#pragma unroll
    for (int db = 0; db < kDb; ++db) acc[rr][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[kRG], l_run[kRG];
  float mb_run[kRG];  // m_run, or 0 while the row has no visible key
#pragma unroll
  for (int rr = 0; rr < kRG; ++rr) {
    m_run[rr] = -INFINITY;
    l_run[rr] = 0.f;
    mb_run[rr] = 0.f;
  }

  // Q is in registers before the loop: the empty asm uses pin the loads'
  // completion here, so no wait for them (which would also wait for the ring's
  // loads) lands inside the loop.
#pragma unroll
  for (int rr = 0; rr < kRG; ++rr)
#pragma unroll
    for (int ks = 0; ks < kKs; ++ks) asm volatile("" ::"v"(qreg[rr][ks]));
  // first step's tile landed (each wave waits for its own loads; the barrier
  // publishes all of them)
  if constexpr (F8) {
    commit(0);
  } else {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 * (kStages - 2)) : "memory");
  }
  __syncthreads();

  const char* lds = (const char*)(__attribute__((address_space(3))) char*)ring;
  auto step = [&](auto stage_c, int s) {
    constexpr int ST = decltype(stage_c)::value;
    if constexpr (F8) issue((ST + kStages - 1) % kStages);  // step s + kStages - 1
    const char* kt = lds + ST * kStageB;
    const char* vt = kt + kTileB;

    // S^T for the four 16-key quarters and the wave's row groups
    f32x4_t st[kRG][4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      u32x4_t ka[kKs];
#pragma unroll
      for (int ks = 0; ks < kKs; ++ks)
        ka[ks] = *reinterpret_cast<const u32x4_t*>(kt + h * (16 * kRB) + ko[ks]);
      // step s + kStages - 1 into the other stage, after the third quarter's K reads: its
      // scalar work spreads over the QK MFMAs around it (measured against quarters 0, 1 and
      // 3, the PV chunks and the step's start: 2-4% faster than the start)
      if constexpr (!F8) {
        if (h == 2) issue((ST + kStages - 1) % kStages);
      }
#pragma unroll
      for (int rr = 0; rr < kRG; ++rr) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < kKs; ++ks)
          a = mfma_16x16x32<H16>(ka[ks], qreg[rr][ks], a);
        st[rr][h] = a;
      }
    }
    // online softmax (log2 domain, running max m_run kept scaled). The max is
    // only raised when a row's maximum grows by more than kLazy (log2 units):
    // weights then stay <= 2^kLazy, exact after the final 1/l. Both row groups'
    // maxima first (one rescale branch), then per 32-key chunk the weights,
    // packed as the P^T B operand (8 bf16 per lane), and that chunk's PV
    // MFMAs: chunk 1's exp work overlaps chunk 0's MFMAs. The row sum is taken
    // over the same bf16 weights that multiply V.
    const bool edge = (s * kStep + kStep - 1 > diag + j0) || (s * kStep + kStep > Lk);  // uniform
    float sv[kRG][16];
#pragma unroll
    for (int rr = 0; rr < kRG; ++rr)
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[rr][4 * h + r] = st[rr][h][r];
    if (edge) {
#pragma unroll
      for (int rr = 0; rr < kRG; ++rr) {
        const int lim = min(diag + jrow[rr], Lk - 1);  // last visible key of this row
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (s * kStep + 16 * h + 4 * g4 + r > lim) sv[rr][4 * h + r] = -INFINITY;
      }
    }
    // Each lane first tests its own 16 scores of a row group against the headroom; only
    // when some lane's exceed it does the wave take the row maxima across the 4 lane groups
    // (two permlane swaps) and rescale. The decisions are those of testing the row maxima
    // every step, which rarely rise past the headroom after the first steps.
    float lmax[kRG];
    bool lraise = false;
#pragma unroll
    for (int rr = 0; rr < kRG; ++rr) {
      const float* v = sv[rr];
      lmax[rr] = fmax3(fmax3(fmax3(v[0], v[1], v[2]), fmax3(v[3], v[4], v[5]),
                             fmax3(v[6], v[7], v[8])),
                       fmax3(v[9], v[10], v[11]),
                       fmax3(fmax3(v[12], v[13], v[14]), v[15], -INFINITY));
      lraise = lraise || (lmax[rr] * scale_log2 > m_run[rr] + kLazy);
    }
    if (__builtin_amdgcn_ballot_w64(lraise) != 0) {
#pragma unroll
      for (int rr = 0; rr < kRG; ++rr) {
        const float cm = col_max4(lmax[rr]) * scale_log2;
        const bool raise = cm > m_run[rr] + kLazy;  // false while the row has no visible key
        const float alpha = raise ? fast_exp2(m_run[rr] - cm) : 1.f;  // exp2(-inf) = 0
        m_run[rr] = raise ? cm : m_run[rr];
        mb_run[rr] = m_run[rr] == -INFINITY ? 0.f : m_run[rr];
        l_run[rr] *= alpha;
#pragma unroll
        for (int db = 0; db < kDb; ++db) acc[rr][db] *= alpha;
      }
    }
    const float* mb = mb_run;
    // O^T[dims][rows] += V^T[dims][keys] P^T[keys][rows] per 32-key chunk c:
    // k-slot j of lane group g is key 32c+4g+j (j<4), or 32c+16+4g+(j-4)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      u32x4_t pb[kRG];
#pragma unroll
      for (int rr = 0; rr < kRG; ++rr) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          p[e] = fast_exp2(fmaf(sv[rr][8 * c + e], scale_log2, -mb[rr]));  // -inf -> 0
        pb[rr] = u32x4_t{cvt_pk16<H16>(p[0], p[1]), cvt_pk16<H16>(p[2], p[3]),
                         cvt_pk16<H16>(p[4], p[5]), cvt_pk16<H16>(p[6], p[7])};
        float l = l_run[rr];
#pragma unroll
        for (int e = 0; e < 4; ++e) l = sum2_16<H16>(pb[rr][e], l);
        l_run[rr] = l;
      }
#pragma unroll
      for (int db = 0; db < kDb; ++db) {
        const char* vc = vt + c * (32 * kRB) + vo[db];
        const i16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)vc);
        const i16x4_t v1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vc + 16 * kRB));
        const u32x4_t va = {__builtin_bit_cast(uint2, v0).x, __builtin_bit_cast(uint2, v0).y,
                            __builtin_bit_cast(uint2, v1).x, __builtin_bit_cast(uint2, v1).y};
#pragma unroll
        for (int rr = 0; rr < kRG; ++rr)
          acc[rr][db] = mfma_16x16x32<H16>(va, pb[rr], acc[rr][db]);
      }
    }
    // next step's tile landed (own loads), then publish and free this stage
    if constexpr (F8) {
      if (s + 1 < n_steps) commit((ST + 1) % kStages);  // uniform
    } else {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 * (kStages - 2)) : "memory");
    }
    __syncthreads();
    refill_window();
  };
  static_assert(kStages == 2, "the step loop below is unrolled for 2 stages");
  for (int s = 0;;) {
    if (s >= n_steps) break;
    step(std::integral_constant<int, 0>{}, s++);
    if (s >= n_steps) break;
    step(std::integral_constant<int, 1>{}, s++);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the workgroup

  // ---- epilogue: normalise and store this lane's 4 dims of each 16-dim block
#pragma unroll
  for (int rr = 0; rr < kRG; ++rr) {
    const float l = col_sum4(l_run[rr]);
    if (jrow[rr] >= Lq) continue;
    const float inv = l > 0.f ? (F8 ? v_scale : 1.f) / l : 0.f;
    bf16_t* op = out + (int64_t)(q0 + jrow[rr]) * out_row_stride +
                 (int64_t)(kvh * G + head[rr]) * D + g4 * 4;
#pragma unroll
    for (int db = 0; db < kDb; ++db) {
      const uint2 w = {out_pack<H16>(acc[rr][db][0] * inv, acc[rr][db][1] * inv),
                       out_pack<H16>(acc[rr][db][2] * inv, acc[rr][db][3] * inv)};
      *reinterpret_cast<uint2*>(op + db * 16) = w;
    }
  }
}

}  // namespace nkv

namespace nkv {
template <bool F8, bool H16 = false>
static int prefill_launch(const void* q, int64_t q_row_stride, const void* k_cache,
                          const void* v_cache, int64_t k_row_stride, int64_t v_row_stride,
                          const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                          const int32_t* block_tables, int64_t bt_row_stride,
                          int32_t max_blocks_per_seq, int32_t n_seqs, int32_t max_seqlen_q,
                          int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                          int32_t block_size, int64_t n_rows, float scale, float k_scale,
                          float v_scale, void* out, int64_t out_row_stride, void* stream) {
  constexpr int kEl = F8 ? 1 : 2;
  const char* what = F8 ? "prefill_varlen_fp8" : H16 ? "prefill_varlen_f16" : "prefill_varlen";
  NKV_REQUIRE(n_seqs >= 0 && max_seqlen_q >= 0 && n_q_heads > 0 && n_kv_heads > 0, NKV_EINVAL,
              "%s: bad sizes", what);
  if (n_seqs == 0 || max_seqlen_q == 0) return NKV_OK;
  NKV_REQUIRE(prefill_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "%s: head_dim must be 64, 128 or 256 (got %d)", what, head_dim);
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "%s: Hq %% Hk != 0", what);
  const int g = n_q_heads / n_kv_heads;
  // a tile holds at least one query for all g heads of its KV head
  NKV_REQUIRE(g <= prefill_max_group(head_dim), NKV_EUNSUPPORTED, "%s: GQA group %d above %d",
              what, g, prefill_max_group(head_dim));
  NKV_REQUIRE(q && k_cache && v_cache && cu_seqlens_q && cu_seqlens_k && out, NKV_EINVAL,
              "%s: null pointer", what);
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
              NKV_EINVAL, "%s: q/k/v/out must be 16-byte aligned", what);
  NKV_REQUIRE(q_row_stride >= (int64_t)n_q_heads * head_dim && q_row_stride % 8 == 0 &&
                  out_row_stride >= (int64_t)n_q_heads * head_dim && out_row_stride % 8 == 0 &&
                  k_row_stride >= (int64_t)n_kv_heads * head_dim &&
                  k_row_stride % (16 / kEl) == 0 &&
                  v_row_stride >= (int64_t)n_kv_heads * head_dim &&
                  v_row_stride % (16 / kEl) == 0,
              NKV_EINVAL, "%s: row strides must cover the heads, in 16-byte multiples", what);
  NKV_REQUIRE(n_rows > 0, NKV_EINVAL, "%s: empty K/V", what);
  NKV_REQUIRE(k_row_stride * kEl * kStep < (1ll << 31) && v_row_stride * kEl * kStep < (1ll << 31),
              NKV_EUNSUPPORTED, "%s: K/V row stride too large", what);
  NKV_REQUIRE(!block_tables || k_row_stride == v_row_stride, NKV_EINVAL,
              "%s: paged K and V caches share one row stride", what);
  NKV_REQUIRE(!F8 || block_tables, NKV_EINVAL, "%s: fp8 K/V are read from a paged pool", what);
  NKV_REQUIRE(k_scale > 0.f && v_scale > 0.f, NKV_EINVAL, "%s: scales must be > 0", what);
  int max_blocks = 0;
  if (block_tables) {
    NKV_REQUIRE(block_size > 0 && block_size % 16 == 0, NKV_EUNSUPPORTED,
                "%s: block_size must be a positive multiple of 16", what);
    NKV_REQUIRE(max_blocks_per_seq > 0 && bt_row_stride >= max_blocks_per_seq,
                NKV_EINVAL, "%s: paged mode needs block_size, max_blocks_per_seq "
                "and bt_row_stride >= max_blocks_per_seq", what);
    max_blocks = max_blocks_per_seq;
  }
  // paged: valid block ids are [0, n_rows / block_size); contiguous: valid rows
  const int32_t n_limit = (int32_t)std::min<int64_t>(block_tables ? n_rows / block_size : n_rows,
                                                     INT32_MAX);
  const int qt = prefill_tile_rows(head_dim, F8) / g;
  const int n_tiles = (max_seqlen_q + qt - 1) / qt;
  const int64_t grid = (int64_t)n_seqs * n_tiles * n_kv_heads;
  NKV_REQUIRE(grid < (1ll << 31), NKV_EUNSUPPORTED, "%s: grid too large", what);
  const float sl2 = scale * k_scale * kLog2e;
#define NKV_PREFILL_LAUNCH_P(D, P)                                                             \
  hipLaunchKernelGGL((prefill_varlen_kernel<F8, D, H16, P>), dim3((unsigned)grid), dim3(256), 0, \
                     as_stream(stream), (const bf16_t*)q, q_row_stride, k_cache, v_cache,        \
                     k_row_stride, v_row_stride, cu_seqlens_q, cu_seqlens_k, block_tables,       \
                     bt_row_stride, n_kv_heads, g, block_size, max_blocks, n_limit, n_tiles, sl2, \
                     v_scale, (bf16_t*)out, out_row_stride)
#define NKV_PREFILL_LAUNCH(D)                                                                  \
  do {                                                                                         \
    if (block_tables) NKV_PREFILL_LAUNCH_P(D, true);                                           \
    else if constexpr (!F8) NKV_PREFILL_LAUNCH_P(D, false);                                    \
  } while (0)
  if (head_dim == 64) NKV_PREFILL_LAUNCH(64);
  else if (head_dim == 128) NKV_PREFILL_LAUNCH(128);
  else NKV_PREFILL_LAUNCH(256);
#undef NKV_PREFILL_LAUNCH
#undef NKV_PREFILL_LAUNCH_P
  return check_launch(F8 ? "nkv_prefill_varlen_fp8"
                         : H16 ? "nkv_prefill_varlen_f16" : "nkv_prefill_varlen");
}
}  // namespace nkv

extern "C" int nkv_prefill_varlen(const void* q, int64_t q_row_stride, const void* k_cache,
                                  const void* v_cache, int64_t k_row_stride,
                                  int64_t v_row_stride, const int32_t* cu_seqlens_q,
                                  const int32_t* cu_seqlens_k, const int32_t* block_tables,
                                  int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                  int32_t n_seqs, int32_t max_seqlen_q, int32_t n_q_heads,
                                  int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                  int64_t n_rows, float scale, void* out, int64_t out_row_stride,
                                  void* stream) {
  nkv::clear_error();
  return nkv::prefill_launch<false>(q, q_row_stride, k_cache, v_cache, k_row_stride,
                                    v_row_stride, cu_seqlens_q, cu_seqlens_k, block_tables,
                                    bt_row_stride, max_blocks_per_seq, n_seqs, max_seqlen_q,
                                    n_q_heads, n_kv_heads, head_dim, block_size, n_rows, scale,
                                    1.f, 1.f, out, out_row_stride, stream);
}

extern "C" int nkv_prefill_varlen_f16(const void* q, int64_t q_row_stride, const void* k_cache,
                                      const void* v_cache, int64_t k_row_stride,
                                      int64_t v_row_stride, const int32_t* cu_seqlens_q,
                                      const int32_t* cu_seqlens_k, const int32_t* block_tables,
                                      int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                      int32_t n_seqs, int32_t max_seqlen_q, int32_t n_q_heads,
                                      int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                      int64_t n_rows, float scale, void* out,
                                      int64_t out_row_stride, void* stream) {
  nkv::clear_error();
  return nkv::prefill_launch<false, true>(q, q_row_stride, k_cache, v_cache, k_row_stride,
                                          v_row_stride, cu_seqlens_q, cu_seqlens_k, block_tables,
                                          bt_row_stride, max_blocks_per_seq, n_seqs,
                                          max_seqlen_q, n_q_heads, n_kv_heads, head_dim,
                                          block_size, n_rows, scale, 1.f, 1.f, out,
                                          out_row_stride, stream);
}

extern "C" int nkv_prefill_varlen_fp8(const void* q, int64_t q_row_stride, const void* k_cache,
                                      const void* v_cache, const int32_t* cu_seqlens_q,
                                      const int32_t* cu_seqlens_k, const int32_t* block_tables,
                                      int64_t bt_row_stride, int32_t max_blocks_per_seq,
                                      int32_t n_seqs, int32_t max_seqlen_q, int32_t n_q_heads,
                                      int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                      int64_t n_blocks, float scale, float k_scale,
                                      float v_scale, void* out, int64_t out_row_stride,
                                      void* stream) {
  nkv::clear_error();
  const int64_t row = (int64_t)n_kv_heads * head_dim;  // codes (bytes) per cache row
  return nkv::prefill_launch<true>(q, q_row_stride, k_cache, v_cache, row, row, cu_seqlens_q,
                                   cu_seqlens_k, block_tables, bt_row_stride, max_blocks_per_seq,
                                   n_seqs, max_seqlen_q, n_q_heads, n_kv_heads, head_dim,
                                   block_size, n_blocks * block_size, scale, k_scale, v_scale,
                                   out, out_row_stride, stream);
}

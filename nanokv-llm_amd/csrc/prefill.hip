// Varlen causal prefill over the paged K/V cache (bf16 MFMA, fp32 softmax).
//
// Reference: flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
// max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True, block_table) at
// nanokvllm/layers/attention.py:96-102 (bottom-right causal alignment: query
// j of a sequence with Lq queries and Lk keys sees keys 0 .. Lk-Lq+j).
//
// MI355X design (MFMA-bound):
//  * Workgroup = (sequence, tile of 128/g queries, KV head) x 4 waves. The
//    tile's 128 "rows" are its queries for all g query heads of the KV head,
//    so one K/V tile in LDS serves g heads (GQA sharing). Wave w owns two
//    16-row groups (32 rows).
//  * Keys advance in 32-key steps; each step's K and V (2 x 8 KiB) are
//    loaded by the whole workgroup with 16-byte loads into registers,
//    written to a double-buffered LDS tile, one barrier per step.
//  * S^T = K Q^T  (v_mfma_f32_16x16x32_bf16: A = 16 keys from LDS, B = the
//    wave's Q^T held in registers for the whole sequence) puts, in lane l,
//    row l%16 and keys 4(l/16)..+3 of each 16-key half. That is exactly the
//    B operand of  O^T += V^T P^T  (16x16x32 over the 32 keys) once the two
//    halves' weights are packed to bf16; V^T (A operand) comes from LDS with
//    two ds_read_b64_tr_b16 per 16-dim block. Each lane owns one row: the
//    online softmax needs one xor-max over the 4 key groups per step.
//  * Causal: a tile stops at its last visible key; masks are applied per
//    element only where needed. Tiles are dispatched largest-first and the
//    KV head is the fastest grid index, so with 8 KV heads each head's tiles
//    share one XCD's L2.
#include "nkv_common.h"

#include <algorithm>

namespace nkv {

constexpr int kPD = 128;                // head_dim
constexpr int kStep = 32;               // keys per step
constexpr int kBufferFlags = 0x00020000;  // raw buffer descriptor word 3 for gfx950
constexpr int kRowE = kPD + 16;         // LDS row stride (elements; 288 B)
constexpr int kRowsPerWave = 32;        // two 16-row groups
constexpr int kWGRows = 4 * kRowsPerWave;
constexpr float kLazy = 8.f;             // log2 headroom before the running max is raised

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const bf16x2v_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

template <int G>
__global__ __launch_bounds__(256, 2) void prefill_varlen_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, int64_t kv_row_stride,
    const int32_t* __restrict__ cu_seqlens_q, const int32_t* __restrict__ cu_seqlens_k,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t Hk,
    int32_t block_size, int32_t max_blocks, int32_t n_limit, int32_t n_tiles, float scale_log2,
    bf16_t* __restrict__ out, int64_t out_row_stride) {
  constexpr int QT = kWGRows / G;  // queries per tile
  constexpr int GPH = QT / 16;     // 16-row groups per head
  __shared__ __attribute__((aligned(16))) bf16_t kbuf[2][kStep * kRowE];
  __shared__ __attribute__((aligned(16))) bf16_t vbuf[2][kStep * kRowE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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
  if (j0 >= Lq) return;  // uniform
  const int diag = Lk - Lq;  // query j sees keys <= diag + j
  const int last_key = min(Lk - 1, diag + j0 + QT - 1);
  const int n_steps = last_key >= 0 ? last_key / kStep + 1 : 0;

  // ---- this wave's two row groups: head and first query of each
  int head[2], jrow[2];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int rg = wave * 2 + rr;
    head[rr] = rg / GPH;
    jrow[rr] = j0 + (rg % GPH) * 16 + col;  // this lane's query (row)
  }
  // Q^T as the MFMA B operand: lane l -> row l%16, dims 8*(l/16) + 32*ks
  u32x4_t qreg[2][4];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int jc = jrow[rr] < Lq ? jrow[rr] : j0;  // rows past the sequence: discarded
    const u32x4_t* qp = reinterpret_cast<const u32x4_t*>(
        q + (int64_t)(q0 + jc) * q_row_stride + (int64_t)(kvh * G + head[rr]) * kPD + g4 * 8);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qreg[rr][ks] = qp[ks * 4];
  }

  // ---- K/V tile loader: thread t moves 16 B of keys t/16 and t/16 + 16 with raw
  // buffer loads. A step's 32 keys are consecutive rows (one cache block, or the
  // contiguous K/V), so each step is one uniform base row and a byte window that
  // covers only its valid keys: keys past Lk and keys of invalid blocks read as 0.
  const int lk = tid >> 4;         // key 0..15 within a half
  const int lch = (tid & 15) * 8;  // dims offset (elements)
  const uint32_t row_b = (uint32_t)kv_row_stride * 2u;
  const uint32_t voff = (uint32_t)lk * row_b + (uint32_t)(kvh * kPD + lch) * 2u;
  const uint32_t voff16 = voff + 16u * row_b;
  // Block ids: lane i holds entry bt_base + i of the sequence's table row, read
  // by the uniform v_readlane of the step's block (reloaded every 64 blocks).
  const int32_t* bt = block_tables ? block_tables + (int64_t)seq * bt_row_stride : nullptr;
  int bt_base = 0;
  int bt_lane = -1;
  auto load_window = [&]() {
    const int e = bt_base + lane;
    const int id = e < max_blocks ? bt[e] : -1;
    bt_lane = (id >= 0 && id < n_limit) ? id : -1;
  };
  if (bt) load_window();
  // cursor: the step loaded next (first key c_t0, block c_blk, offset c_off in it)
  int c_t0 = 0, c_blk = 0, c_off = 0;
  u32x4_t stg[4];  // K(lk), K(lk+16), V(lk), V(lk+16)
  auto load_step = [&]() {
    int nv = min(kStep, Lk - c_t0);
    int64_t row0;
    if (bt) {
      if (c_blk - bt_base >= 64) {  // uniform, once per 64 blocks
        bt_base += 64;
        load_window();
      }
      const int pb = __builtin_amdgcn_readlane(bt_lane, c_blk - bt_base);
      if (pb < 0) nv = 0;
      row0 = (int64_t)pb * block_size + c_off;
    } else {
      row0 = (int64_t)kb0 + c_t0;
      if (kb0 + c_t0 < 0 || kb0 + c_t0 > n_limit - nv) nv = 0;  // outside the K/V rows
    }
    if (nv <= 0) {
      nv = 0;
      row0 = 0;
    }
    const uint32_t bytes = (uint32_t)nv * row_b;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(k_cache + row0 * kv_row_stride), (short)0, bytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(v_cache + row0 * kv_row_stride), (short)0, bytes, kBufferFlags);
    stg[0] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, voff, 0, 0));
    stg[1] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, voff16, 0, 0));
    stg[2] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, voff, 0, 0));
    stg[3] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, voff16, 0, 0));
    c_t0 += kStep;
    c_off += kStep;
    if (bt && c_off >= block_size) {  // block_size is a multiple of kStep
      c_off = 0;
      c_blk = __builtin_amdgcn_readfirstlane(c_blk + 1);
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<u32x4_t*>(&kbuf[buf][(lk + 16 * h) * kRowE + lch]) = stg[h];
      *reinterpret_cast<u32x4_t*>(&vbuf[buf][(lk + 16 * h) * kRowE + lch]) = stg[2 + h];
    }
  };

  f32x4_t acc[2][8];  // O^T: lane l -> row l%16, dims 16*db + 4*(l/16) .. +3
#pragma unroll
  for (int rr = 0; rr < 2; ++rr)
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[rr][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};
  const int tr_row = 4 * g4 + (col >> 2);  // ds_read_b64_tr_b16 source row / column
  const int tr_col = (col & 3) * 4;

  if (n_steps > 0) {
    load_step();
    store_step(0);
  }
  // Q and the first tile are in registers/LDS: an explicit full wait here lets the
  // loop's next-tile loads stay in flight across the whole step.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < n_steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < n_steps) load_step();
    const bf16_t* kt = kbuf[buf];
    const bf16_t* vt = vbuf[buf];

    // S^T for both 16-key halves and both row groups
    f32x4_t st[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4_t ka[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        ka[ks] = *reinterpret_cast<const u32x4_t*>(&kt[(16 * h + col) * kRowE + g4 * 8 + ks * 32]);
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_v(ka[ks]), as_bf16x8_v(qreg[rr][ks]),
                                                       a, 0, 0, 0);
        st[rr][h] = a;
      }
    }
    // online softmax per row group (log2 domain, running max m_run kept scaled).
    // The max is only raised when a row's maximum grows by more than kLazy
    // (log2 units): weights then stay <= 2^kLazy, exact after the final 1/l.
    // P^T is packed as the MFMA B operand (8 bf16 per lane).
    const bool edge = (s * kStep + kStep - 1 > diag + j0) || (s * kStep + kStep > Lk);  // uniform
    u32x4_t pb[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      float sv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[4 * h + r] = st[rr][h][r];
      if (edge) {
        const int lim = min(diag + jrow[rr], Lk - 1);  // last visible key of this row
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (s * kStep + 16 * h + 4 * g4 + r > lim) sv[4 * h + r] = -INFINITY;
      }
      float cmax = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
      const float cm = col_max4(cmax) * scale_log2;
      const bool raise = cm > m_run[rr] + kLazy;  // false while the row has no visible key
      if (__builtin_amdgcn_ballot_w64(raise) != 0) {
        const float alpha = raise ? fast_exp2(m_run[rr] - cm) : 1.f;  // exp2(-inf) = 0
        m_run[rr] = raise ? cm : m_run[rr];
        l_run[rr] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[rr][db] *= alpha;
      }
      const float mb = m_run[rr] == -INFINITY ? 0.f : m_run[rr];
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = fast_exp2(fmaf(sv[e], scale_log2, -mb));  // -inf -> 0
      l_run[rr] += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      pb[rr] = u32x4_t{pack2(p[0], p[1]), pack2(p[2], p[3]), pack2(p[4], p[5]), pack2(p[6], p[7])};
    }
    // O^T[dims][rows] += V^T[dims][keys] P^T[keys][rows]: k-slot j of lane group
    // g is key 4g+j (j<4) of the first half, key 16+4g+(j-4) of the second
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const i16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4_t*)&vt[tr_row * kRowE + db * 16 + tr_col]);
      const i16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4_t*)&vt[(16 + tr_row) * kRowE + db * 16 + tr_col]);
      const u32x4_t va = {__builtin_bit_cast(uint2, v0).x, __builtin_bit_cast(uint2, v0).y,
                          __builtin_bit_cast(uint2, v1).x, __builtin_bit_cast(uint2, v1).y};
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
        acc[rr][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8_v(va), as_bf16x8_v(pb[rr]),
                                                               acc[rr][db], 0, 0, 0);
    }
    if (s + 1 < n_steps) store_step(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: normalise and store this lane's 4 dims of each 16-dim block
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const float l = col_sum4(l_run[rr]);
    if (jrow[rr] >= Lq) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    bf16_t* op = out + (int64_t)(q0 + jrow[rr]) * out_row_stride +
                 (int64_t)(kvh * G + head[rr]) * kPD + g4 * 4;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint2 w = {pack_bf16x2(acc[rr][db][0] * inv, acc[rr][db][1] * inv),
                       pack_bf16x2(acc[rr][db][2] * inv, acc[rr][db][3] * inv)};
      *reinterpret_cast<uint2*>(op + db * 16) = w;
    }
  }
}

}  // namespace nkv

extern "C" int nkv_prefill_varlen(const void* q, int64_t q_row_stride, const void* k_cache,
                                  const void* v_cache, int64_t kv_row_stride,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  const int32_t* block_tables, int64_t bt_row_stride,
                                  int32_t max_blocks_per_seq, int32_t n_seqs, int32_t max_seqlen_q, int32_t n_q_heads,
                                  int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                  int64_t n_rows, float scale, void* out, int64_t out_row_stride,
                                  void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n_seqs >= 0 && max_seqlen_q >= 0 && n_q_heads > 0 && n_kv_heads > 0, NKV_EINVAL,
              "prefill_varlen: bad sizes");
  if (n_seqs == 0 || max_seqlen_q == 0) return NKV_OK;
  NKV_REQUIRE(head_dim == kPD, NKV_EUNSUPPORTED, "prefill_varlen: head_dim must be 128");
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL, "prefill_varlen: Hq %% Hk != 0");
  const int g = n_q_heads / n_kv_heads;
  NKV_REQUIRE(g == 1 || g == 2 || g == 4 || g == 8, NKV_EUNSUPPORTED,
              "prefill_varlen: GQA group %d not in {1,2,4,8}", g);
  NKV_REQUIRE(q && k_cache && v_cache && cu_seqlens_q && cu_seqlens_k && out, NKV_EINVAL,
              "prefill_varlen: null pointer");
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
              NKV_EINVAL, "prefill_varlen: q/k/v/out must be 16-byte aligned");
  NKV_REQUIRE(q_row_stride >= (int64_t)n_q_heads * kPD && q_row_stride % 8 == 0 &&
                  out_row_stride >= (int64_t)n_q_heads * kPD && out_row_stride % 8 == 0 &&
                  kv_row_stride >= (int64_t)n_kv_heads * kPD && kv_row_stride % 8 == 0,
              NKV_EINVAL, "prefill_varlen: row strides must cover the heads, multiples of 8");
  NKV_REQUIRE(n_rows > 0, NKV_EINVAL, "prefill_varlen: empty K/V");
  NKV_REQUIRE(kv_row_stride * 2 * kStep < (1ll << 31), NKV_EUNSUPPORTED,
              "prefill_varlen: K/V row stride too large");
  int max_blocks = 0;
  if (block_tables) {
    NKV_REQUIRE(block_size > 0 && block_size % kStep == 0, NKV_EUNSUPPORTED,
                "prefill_varlen: block_size must be a positive multiple of %d", kStep);
    NKV_REQUIRE(max_blocks_per_seq > 0 && bt_row_stride >= max_blocks_per_seq,
                NKV_EINVAL, "prefill_varlen: paged mode needs block_size, max_blocks_per_seq "
                "and bt_row_stride >= max_blocks_per_seq");
    max_blocks = max_blocks_per_seq;
  }
  // paged: valid block ids are [0, n_rows / block_size); contiguous: valid rows
  const int32_t n_limit = (int32_t)std::min<int64_t>(block_tables ? n_rows / block_size : n_rows,
                                                     INT32_MAX);
  const int qt = kWGRows / g;
  const int n_tiles = (max_seqlen_q + qt - 1) / qt;
  const int64_t grid = (int64_t)n_seqs * n_tiles * n_kv_heads;
  NKV_REQUIRE(grid < (1ll << 31), NKV_EUNSUPPORTED, "prefill_varlen: grid too large");
  const float sl2 = scale * kLog2e;
  hipStream_t s = as_stream(stream);
#define NKV_PREFILL_LAUNCH(G)                                                                   \
  hipLaunchKernelGGL(prefill_varlen_kernel<G>, dim3((unsigned)grid), dim3(256), 0, s,            \
                     (const bf16_t*)q, q_row_stride, (const bf16_t*)k_cache,                     \
                     (const bf16_t*)v_cache, kv_row_stride, cu_seqlens_q, cu_seqlens_k,          \
                     block_tables, bt_row_stride, n_kv_heads, block_size, max_blocks, n_limit,   \
                     n_tiles, sl2, (bf16_t*)out, out_row_stride)
  switch (g) {
    case 1: NKV_PREFILL_LAUNCH(1); break;
    case 2: NKV_PREFILL_LAUNCH(2); break;
    case 4: NKV_PREFILL_LAUNCH(4); break;
    default: NKV_PREFILL_LAUNCH(8); break;
  }
#undef NKV_PREFILL_LAUNCH
  return check_launch("nkv_prefill_varlen");
}

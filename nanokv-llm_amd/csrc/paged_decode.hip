// Paged decode attention (one new query token per sequence, GQA) over the
// [num_blocks, block_size, Hk, D] bf16 cache.
//
// Reference: flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
// cache_seqlens=context_lens, block_table=block_tables, softmax_scale,
// causal=True) at nanokvllm/layers/attention.py:104-107.
//
// MI355X design (HBM-bound: every K/V byte is read exactly once):
//  * Split-K work unit = (sequence b, KV head, 256-token split). One
//    workgroup of 4 wave64s per unit; wave w owns tokens [64w, 64w+64).
//    A unit streams 64 KiB of K + 64 KiB of V (256 rows x 256 B, rows 2 KiB
//    apart in the cache), issued up front as 16+16 128-bit loads per lane so
//    each wave keeps 16 KiB in flight.
//  * QK^T runs on the matrix cores: v_mfma_f32_16x16x32_bf16 with the g query
//    heads of the KV head as rows (rows >= g are zero) and 16 keys as columns;
//    the B operand is loaded straight from HBM in the MFMA lane layout
//    (lane l: key l%16, dims 8*(l/16)..+8 of each 32-dim step).
//  * Softmax max/sum are wavefront shuffle reductions over the split's 256
//    scores staged in LDS; probabilities go back to LDS for the PV product.
//  * PV is VALU FMA on fp32 (V rows are token-major, the wrong orientation
//    for the MFMA B operand); lanes reduce with shuffles, waves through LDS.
//  * Partial (m, l, O) per split go to the workspace; a combine kernel merges
//    the splits of each (sequence, query head) and writes bf16.
// Scores are kept in the log2 domain (scale * log2 e folded in) so the
// exponentials are single v_exp_f32 instructions.
#include "nkv_common.h"

namespace nkv {

constexpr int kD = 128;       // head_dim
constexpr int kSplit = 256;   // tokens per split-K work unit
constexpr int kWaves = 4;     // wave64s per workgroup
constexpr int kTokPerWave = kSplit / kWaves;

static inline int64_t decode_max_splits(int32_t max_blocks, int32_t block_size) {
  return ((int64_t)max_blocks * block_size + kSplit - 1) / kSplit;
}

template <int G>
__global__ __launch_bounds__(256) void paged_decode_split_kernel(
    const bf16_t* __restrict__ q, int64_t q_row_stride,
    const bf16_t* __restrict__ k_cache, const bf16_t* __restrict__ v_cache,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride,
    const int32_t* __restrict__ context_lens, int32_t batch, int32_t Hk,
    int32_t block_size, int32_t max_blocks, int32_t max_splits, int64_t n_blocks,
    float scale_log2, float* __restrict__ part_o, float* __restrict__ part_ml) {
  __shared__ float s_lds[G][kSplit];            // scores (log2 domain)
  __shared__ float p_lds[kSplit][G];            // probabilities, token-major
  __shared__ float o_lds[kWaves][G][kD];        // per-wave PV partials
  __shared__ float ml_lds[G][2];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kvh = blockIdx.x % Hk;
  const int rest = blockIdx.x / Hk;
  const int b = rest % batch;
  const int split = rest / batch;
  const int ctx = context_lens[b];
  const int t0 = split * kSplit;
  if (t0 >= ctx) return;  // uniform over the workgroup

  const int Hq = Hk * G;
  const int64_t row = (int64_t)Hk * kD;
  const int blk = t0 / block_size;
  const int off0 = t0 - blk * block_size;
  const int64_t pb = (blk < max_blocks) ? (int64_t)block_tables[(int64_t)b * bt_row_stride + blk] : -1;
  const int64_t obase = ((int64_t)b * Hq + (int64_t)kvh * G) * max_splits + split;
  if (pb < 0 || pb >= n_blocks) {  // invalid table entry: empty split
    for (int i = threadIdx.x; i < G * kD; i += blockDim.x) {
      const int h = i / kD, d = i % kD;
      part_o[(obase + (int64_t)h * max_splits) * kD + d] = 0.f;
      if (d == 0) {
        part_ml[(obase + (int64_t)h * max_splits) * 2 + 0] = -INFINITY;
        part_ml[(obase + (int64_t)h * max_splits) * 2 + 1] = 0.f;
      }
    }
    return;
  }
  const int n_valid = min(ctx - t0, kSplit);
  const int64_t row0 = pb * block_size + off0;  // cache row of the split's first token

  // ---- issue all K and V loads of this wave (16 + 16 x 16 B per lane)
  uint4 kreg[4][4];  // [16-key group][32-dim step]
  uint4 vreg[16];
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tw = wave * kTokPerWave + j * 16 + (lane & 15);
    const bf16_t* kp = k_cache + (row0 + tw) * row + (int64_t)kvh * kD + (lane >> 4) * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kreg[j][ks] = (tw < n_valid) ? *reinterpret_cast<const uint4*>(kp + ks * 32) : zero4;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tw = wave * kTokPerWave + (lane >> 4) + 4 * i;
    const bf16_t* vp = v_cache + (row0 + tw) * row + (int64_t)kvh * kD + (lane & 15) * 8;
    vreg[i] = (tw < n_valid) ? *reinterpret_cast<const uint4*>(vp) : zero4;
  }

  // ---- q in the MFMA A layout: lane l -> head row l%16, dims 8*(l/16) of each step
  uint4 qreg[4];
  {
    const int hr = lane & 15;
    const bf16_t* qp = q + (int64_t)b * q_row_stride + (int64_t)(kvh * G + hr) * kD + (lane >> 4) * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qreg[ks] = (hr < G) ? *reinterpret_cast<const uint4*>(qp + ks * 32) : zero4;
  }

  // ---- S = q K^T on MFMA; lane l holds rows 4*(l/16)+r, key column l%16
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qreg[ks]), as_bf16x8(kreg[j][ks]),
                                                     acc, 0, 0, 0);
    const int tw = wave * kTokPerWave + j * 16 + (lane & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = (lane >> 4) * 4 + r;
      if (h < G) s_lds[h][tw] = (tw < n_valid) ? acc[r] * scale_log2 : -INFINITY;
    }
  }
  __syncthreads();

  // ---- softmax statistics per head (one wave per head)
  for (int h = wave; h < G; h += kWaves) {
    float sv[4];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sv[k] = s_lds[h][lane + 64 * k];
      mx = fmaxf(mx, sv[k]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float p = (mx == -INFINITY) ? 0.f : fast_exp2(sv[k] - mx);
      p_lds[lane + 64 * k][h] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      ml_lds[h][0] = mx;
      ml_lds[h][1] = sum;
    }
  }
  __syncthreads();

  // ---- O = P V on VALU: lane l owns dims 8*(l%16)..+8 of keys (l/16)+4i
  float acc_o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc_o[h][d] = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int tw = wave * kTokPerWave + (lane >> 4) + 4 * i;
    float p[G];
#pragma unroll
    for (int h = 0; h < G; ++h) p[h] = p_lds[tw][h];
    const uint32_t w[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v0 = bf16_lo(w[e]), v1 = bf16_hi(w[e]);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        acc_o[h][2 * e] = fmaf(p[h], v0, acc_o[h][2 * e]);
        acc_o[h][2 * e + 1] = fmaf(p[h], v1, acc_o[h][2 * e + 1]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float v = acc_o[h][d];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc_o[h][d] = v;
    }
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int d = 0; d < 8; ++d) o_lds[wave][h][lane * 8 + d] = acc_o[h][d];
  }
  __syncthreads();

  for (int i = threadIdx.x; i < G * kD; i += blockDim.x) {
    const int h = i / kD, d = i % kD;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) o += o_lds[w][h][d];
    part_o[(obase + (int64_t)h * max_splits) * kD + d] = o;
    if (d == 0) {
      part_ml[(obase + (int64_t)h * max_splits) * 2 + 0] = ml_lds[h][0];
      part_ml[(obase + (int64_t)h * max_splits) * 2 + 1] = ml_lds[h][1];
    }
  }
}

// Merge the splits of one (sequence, query head): O = sum_s 2^(m_s-M) O_s /
// sum_s 2^(m_s-M) l_s. One workgroup of kD lanes (one dim each) per pair.
__global__ __launch_bounds__(kD) void paged_decode_combine_kernel(
    const int32_t* __restrict__ context_lens, int32_t Hq, int32_t max_splits,
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    bf16_t* __restrict__ out, int64_t out_row_stride) {
  const int b = blockIdx.x / Hq;
  const int h = blockIdx.x % Hq;
  const int d = threadIdx.x;
  const int ctx = context_lens[b];
  const int ns = ctx > 0 ? min((ctx + kSplit - 1) / kSplit, max_splits) : 0;
  const int64_t base = ((int64_t)b * Hq + h) * max_splits;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, part_ml[(base + s) * 2]);
  float L = 0.f, acc = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < ns; ++s) {
      const float ms = part_ml[(base + s) * 2];
      const float w = (ms == -INFINITY) ? 0.f : fast_exp2(ms - M);
      L = fmaf(w, part_ml[(base + s) * 2 + 1], L);
      acc = fmaf(w, part_o[(base + s) * kD + d], acc);
    }
  }
  const float o = (L > 0.f) ? acc / L : 0.f;
  out[(int64_t)b * out_row_stride + (int64_t)h * kD + d] = (bf16_t)f32_to_bf16_bits(o);
}

static int decode_check(const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* block_tables, const int32_t* context_lens, int32_t batch,
                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t block_size, int32_t max_blocks_per_seq, int64_t q_row_stride,
                        int64_t bt_row_stride) {
  NKV_REQUIRE(batch >= 0 && n_kv_heads > 0 && n_q_heads > 0, NKV_EINVAL,
              "paged_decode: bad sizes (batch=%d, Hq=%d, Hk=%d)", batch, n_q_heads, n_kv_heads);
  NKV_REQUIRE(head_dim == kD, NKV_EUNSUPPORTED, "paged_decode: head_dim must be 128 (got %d)",
              head_dim);
  NKV_REQUIRE(n_q_heads % n_kv_heads == 0, NKV_EINVAL,
              "paged_decode: n_q_heads %% n_kv_heads != 0 (%d, %d)", n_q_heads, n_kv_heads);
  const int g = n_q_heads / n_kv_heads;
  NKV_REQUIRE(g == 1 || g == 2 || g == 4 || g == 8 || g == 16, NKV_EUNSUPPORTED,
              "paged_decode: GQA group %d not in {1,2,4,8,16}", g);
  NKV_REQUIRE(block_size > 0 && block_size % kSplit == 0, NKV_EUNSUPPORTED,
              "paged_decode: block_size must be a multiple of 256 (got %d)", block_size);
  NKV_REQUIRE(max_blocks_per_seq > 0 && bt_row_stride >= max_blocks_per_seq, NKV_EINVAL,
              "paged_decode: bad block table width/stride (%d, %lld)", max_blocks_per_seq,
              (long long)bt_row_stride);
  NKV_REQUIRE(q_row_stride >= (int64_t)n_q_heads * kD && q_row_stride % 8 == 0, NKV_EINVAL,
              "paged_decode: q row stride must be >= Hq*D and a multiple of 8");
  NKV_REQUIRE(q && k_cache && v_cache && block_tables && context_lens, NKV_EINVAL,
              "paged_decode: null pointer");
  NKV_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache), NKV_EINVAL,
              "paged_decode: q/k_cache/v_cache must be 16-byte aligned");
  return NKV_OK;
}

}  // namespace nkv

extern "C" size_t nkv_paged_decode_workspace_bytes(int32_t batch, int32_t n_q_heads,
                                                   int32_t head_dim, int32_t max_blocks_per_seq,
                                                   int32_t block_size) {
  if (batch <= 0 || n_q_heads <= 0 || max_blocks_per_seq <= 0 || block_size <= 0) return 0;
  const int64_t ms = nkv::decode_max_splits(max_blocks_per_seq, block_size);
  return (size_t)batch * n_q_heads * ms * (head_dim + 2) * sizeof(float);
}

extern "C" int nkv_paged_decode_split(const void* q, int64_t q_row_stride, const void* k_cache,
                                      const void* v_cache, const int32_t* block_tables,
                                      int64_t bt_row_stride, const int32_t* context_lens,
                                      int32_t batch, int32_t n_q_heads, int32_t n_kv_heads,
                                      int32_t head_dim, int32_t block_size,
                                      int32_t max_blocks_per_seq, int64_t n_blocks, float scale,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  using namespace nkv;
  clear_error();
  int rc = decode_check(q, k_cache, v_cache, block_tables, context_lens, batch, n_q_heads,
                        n_kv_heads, head_dim, block_size, max_blocks_per_seq, q_row_stride,
                        bt_row_stride);
  if (rc) return rc;
  if (batch == 0) return NKV_OK;
  const size_t need = nkv_paged_decode_workspace_bytes(batch, n_q_heads, head_dim,
                                                       max_blocks_per_seq, block_size);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "paged_decode: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  const int64_t ms = decode_max_splits(max_blocks_per_seq, block_size);
  const int64_t grid = ms * batch * n_kv_heads;
  NKV_REQUIRE(grid < (1ll << 31), NKV_EUNSUPPORTED, "paged_decode: grid too large");
  float* part_o = (float*)workspace;
  float* part_ml = part_o + (int64_t)batch * n_q_heads * ms * kD;
  const float scale_log2 = scale * kLog2e;
  const int g = n_q_heads / n_kv_heads;
  hipStream_t s = as_stream(stream);
#define NKV_DECODE_LAUNCH(G)                                                                   \
  hipLaunchKernelGGL(paged_decode_split_kernel<G>, dim3((unsigned)grid), dim3(256), 0, s,      \
                     (const bf16_t*)q, q_row_stride, (const bf16_t*)k_cache,                    \
                     (const bf16_t*)v_cache, block_tables, bt_row_stride, context_lens, batch, \
                     n_kv_heads, block_size, max_blocks_per_seq, (int32_t)ms, n_blocks,        \
                     scale_log2, part_o, part_ml)
  switch (g) {
    case 1: NKV_DECODE_LAUNCH(1); break;
    case 2: NKV_DECODE_LAUNCH(2); break;
    case 4: NKV_DECODE_LAUNCH(4); break;
    case 8: NKV_DECODE_LAUNCH(8); break;
    default: NKV_DECODE_LAUNCH(16); break;
  }
#undef NKV_DECODE_LAUNCH
  return check_launch("nkv_paged_decode_split");
}

extern "C" int nkv_paged_decode_combine(const int32_t* context_lens, int32_t batch,
                                        int32_t n_q_heads, int32_t head_dim, int32_t block_size,
                                        int32_t max_blocks_per_seq, void* out,
                                        int64_t out_row_stride, const void* workspace,
                                        size_t workspace_bytes, void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(head_dim == kD, NKV_EUNSUPPORTED, "paged_decode: head_dim must be 128");
  NKV_REQUIRE(batch >= 0 && n_q_heads > 0 && block_size > 0 && max_blocks_per_seq > 0,
              NKV_EINVAL, "paged_decode_combine: bad sizes");
  if (batch == 0) return NKV_OK;
  NKV_REQUIRE(out && context_lens, NKV_EINVAL, "paged_decode_combine: null pointer");
  NKV_REQUIRE(out_row_stride >= (int64_t)n_q_heads * kD, NKV_EINVAL,
              "paged_decode_combine: out row stride must be >= Hq*D");
  const size_t need = nkv_paged_decode_workspace_bytes(batch, n_q_heads, head_dim,
                                                       max_blocks_per_seq, block_size);
  NKV_REQUIRE(workspace && workspace_bytes >= need, NKV_EWORKSPACE,
              "paged_decode: workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  const int64_t ms = decode_max_splits(max_blocks_per_seq, block_size);
  const float* part_o = (const float*)workspace;
  const float* part_ml = part_o + (int64_t)batch * n_q_heads * ms * kD;
  hipLaunchKernelGGL(paged_decode_combine_kernel, dim3((unsigned)(batch * n_q_heads)), dim3(kD),
                     0, as_stream(stream), context_lens, n_q_heads, (int32_t)ms, part_o, part_ml,
                     (bf16_t*)out, out_row_stride);
  return check_launch("nkv_paged_decode_combine");
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
  return nkv_paged_decode_combine(context_lens, batch, n_q_heads, head_dim, block_size,
                                  max_blocks_per_seq, out, out_row_stride, workspace,
                                  workspace_bytes, stream);
}

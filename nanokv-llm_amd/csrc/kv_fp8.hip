// fp8 (OCP E4M3FN) K/V: conversion and the fp8 store_kvcache.
//
// Reference: the K/V pool of ModelRunner.allocate_kv_cache
// (nanokvllm/engine/model_runner.py:133-152) holds the model dtype; an fp8
// pool halves its bytes (twice the cached tokens in the same HBM, half the
// bytes per decoded token). Values are stored as E4M3FN(clamp(x / scale))
// with one scale per K or V cache (per layer), and read back as code * scale.
// The store replaces store_kvcache (nanokvllm/layers/attention.py:10-40) for
// an fp8 pool: same slot rules (-1 and out-of-range slots skipped).
//
// HBM-bound copies: a thread converts 16 elements (32 bytes of bf16 in,
// 16 bytes of fp8 out) with full-width loads and stores. Prefill over an fp8
// pool gathers each sequence's rows into contiguous bf16 rows first (prefill
// is MFMA-bound: the extra bytes cost a few percent of its time) and runs the
// contiguous prefill on them.
#include "nkv_common.h"

namespace nkv {

constexpr int kF8Threads = 256;
constexpr int kF8MaxGrid = 8192;

__global__ __launch_bounds__(kF8Threads) void fp8_quantize_kernel(
    const bf16_t* __restrict__ src, int64_t n16, float inv_scale, uint8_t* __restrict__ dst) {
  for (int64_t i = (int64_t)blockIdx.x * kF8Threads + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * kF8Threads) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(src + 16 * i);
    const u32x4_t b = *reinterpret_cast<const u32x4_t*>(src + 16 * i + 8);
    u32x4_t o;
    o[0] = f32x4_to_fp8x4(bf16_lo(a[0]) * inv_scale, bf16_hi(a[0]) * inv_scale,
                          bf16_lo(a[1]) * inv_scale, bf16_hi(a[1]) * inv_scale);
    o[1] = f32x4_to_fp8x4(bf16_lo(a[2]) * inv_scale, bf16_hi(a[2]) * inv_scale,
                          bf16_lo(a[3]) * inv_scale, bf16_hi(a[3]) * inv_scale);
    o[2] = f32x4_to_fp8x4(bf16_lo(b[0]) * inv_scale, bf16_hi(b[0]) * inv_scale,
                          bf16_lo(b[1]) * inv_scale, bf16_hi(b[1]) * inv_scale);
    o[3] = f32x4_to_fp8x4(bf16_lo(b[2]) * inv_scale, bf16_hi(b[2]) * inv_scale,
                          bf16_lo(b[3]) * inv_scale, bf16_hi(b[3]) * inv_scale);
    *reinterpret_cast<u32x4_t*>(dst + 16 * i) = o;
  }
}

__global__ __launch_bounds__(kF8Threads) void fp8_dequantize_kernel(
    const uint8_t* __restrict__ src, int64_t n16, float scale, bf16_t* __restrict__ dst) {
  for (int64_t i = (int64_t)blockIdx.x * kF8Threads + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * kF8Threads) {
    u32x4_t lo, hi;
    fp8x16_to_bf16(*reinterpret_cast<const u32x4_t*>(src + 16 * i), lo, hi);
    if (scale != 1.f) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        lo[w] = pack_bf16x2(bf16_lo(lo[w]) * scale, bf16_hi(lo[w]) * scale);
        hi[w] = pack_bf16x2(bf16_lo(hi[w]) * scale, bf16_hi(hi[w]) * scale);
      }
    }
    *reinterpret_cast<u32x4_t*>(dst + 16 * i) = lo;
    *reinterpret_cast<u32x4_t*>(dst + 16 * i + 8) = hi;
  }
}

// (token, K|V, 16-element chunk) units; chunks of a row are consecutive.
__global__ __launch_bounds__(kF8Threads) void store_kvcache_fp8_kernel(
    const bf16_t* __restrict__ key, int64_t key_row_stride, const bf16_t* __restrict__ value,
    int64_t value_row_stride, uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens, int32_t chunks_per_row,
    int64_t n_slots, float inv_k_scale, float inv_v_scale) {
  const int64_t n_units = n_tokens * 2 * chunks_per_row;
  for (int64_t u = (int64_t)blockIdx.x * kF8Threads + threadIdx.x; u < n_units;
       u += (int64_t)gridDim.x * kF8Threads) {
    const int64_t t = u / (2 * chunks_per_row);
    const int r = (int)(u - t * 2 * chunks_per_row);
    const bool is_v = r >= chunks_per_row;
    const int c = is_v ? r - chunks_per_row : r;
    const int64_t slot = slot_mapping[t];
    if (slot < 0 || slot >= n_slots) continue;
    const bf16_t* src = (is_v ? value + t * value_row_stride : key + t * key_row_stride) + 16 * c;
    const float s = is_v ? inv_v_scale : inv_k_scale;
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(src);
    const u32x4_t b = *reinterpret_cast<const u32x4_t*>(src + 8);
    u32x4_t o;
    o[0] = f32x4_to_fp8x4(bf16_lo(a[0]) * s, bf16_hi(a[0]) * s, bf16_lo(a[1]) * s,
                          bf16_hi(a[1]) * s);
    o[1] = f32x4_to_fp8x4(bf16_lo(a[2]) * s, bf16_hi(a[2]) * s, bf16_lo(a[3]) * s,
                          bf16_hi(a[3]) * s);
    o[2] = f32x4_to_fp8x4(bf16_lo(b[0]) * s, bf16_hi(b[0]) * s, bf16_lo(b[1]) * s,
                          bf16_hi(b[1]) * s);
    o[3] = f32x4_to_fp8x4(bf16_lo(b[2]) * s, bf16_hi(b[2]) * s, bf16_lo(b[3]) * s,
                          bf16_hi(b[3]) * s);
    uint8_t* dst = (is_v ? v_cache : k_cache) + slot * (int64_t)chunks_per_row * 16 + 16 * c;
    *reinterpret_cast<u32x4_t*>(dst) = o;
  }
}

// Gather + widen: row t of sequence s (cu_seqlens_k[s] + t, t < Lk_s) of the contiguous bf16
// output <- cache row block_tables[s, t / B] * B + t % B, as code * scale; rows whose table
// entry is missing or outside [0, n_blocks) are zero. Grid (sequence, row chunk).
__global__ __launch_bounds__(kF8Threads) void fp8_gather_rows_kernel(
    const uint8_t* __restrict__ k_cache, const uint8_t* __restrict__ v_cache,
    const int32_t* __restrict__ block_tables, int64_t bt_row_stride, int32_t max_blocks,
    const int32_t* __restrict__ cu_seqlens_k, int32_t block_size, int64_t n_blocks,
    int32_t chunks_per_row, float k_scale, float v_scale, bf16_t* __restrict__ k_out,
    bf16_t* __restrict__ v_out) {
  const int s = blockIdx.x;
  const int k0 = cu_seqlens_k[s];
  const int Lk = cu_seqlens_k[s + 1] - k0;
  const int64_t units = (int64_t)max(Lk, 0) * 2 * chunks_per_row;
  const int32_t* bt = block_tables + (int64_t)s * bt_row_stride;
  for (int64_t u = (int64_t)blockIdx.y * kF8Threads + threadIdx.x; u < units;
       u += (int64_t)gridDim.y * kF8Threads) {
    const int t = (int)(u / (2 * chunks_per_row));
    const int r = (int)(u - (int64_t)t * 2 * chunks_per_row);
    const bool is_v = r >= chunks_per_row;
    const int c = is_v ? r - chunks_per_row : r;
    const int blk = t / block_size;
    const int id = blk < max_blocks ? bt[blk] : -1;
    u32x4_t lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
    if (id >= 0 && id < n_blocks) {
      const int64_t slot = (int64_t)id * block_size + (t - blk * block_size);
      const uint8_t* src = (is_v ? v_cache : k_cache) + (slot * chunks_per_row + c) * 16;
      fp8x16_to_bf16(*reinterpret_cast<const u32x4_t*>(src), lo, hi);
      const float sc = is_v ? v_scale : k_scale;
      if (sc != 1.f) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          lo[w] = pack_bf16x2(bf16_lo(lo[w]) * sc, bf16_hi(lo[w]) * sc);
          hi[w] = pack_bf16x2(bf16_lo(hi[w]) * sc, bf16_hi(hi[w]) * sc);
        }
      }
    }
    bf16_t* dst = (is_v ? v_out : k_out) + ((int64_t)(k0 + t) * chunks_per_row + c) * 16;
    *reinterpret_cast<u32x4_t*>(dst) = lo;
    *reinterpret_cast<u32x4_t*>(dst + 8) = hi;
  }
}

static unsigned f8_grid(int64_t units) {
  const int64_t b = (units + kF8Threads - 1) / kF8Threads;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, kF8MaxGrid));
}

}  // namespace nkv

extern "C" int nkv_fp8_quantize(const void* src, int64_t n, float scale, void* dst,
                                void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n >= 0 && n % 16 == 0 && scale > 0.f, NKV_EINVAL,
              "fp8_quantize: n must be a multiple of 16 and scale > 0");
  if (n == 0) return NKV_OK;
  NKV_REQUIRE(src && dst && aligned16(src) && aligned16(dst), NKV_EINVAL,
              "fp8_quantize: null or misaligned pointer");
  hipLaunchKernelGGL(fp8_quantize_kernel, dim3(f8_grid(n / 16)), dim3(kF8Threads), 0,
                     as_stream(stream), (const bf16_t*)src, n / 16, 1.f / scale, (uint8_t*)dst);
  return check_launch("nkv_fp8_quantize");
}

extern "C" int nkv_fp8_dequantize(const void* src, int64_t n, float scale, void* dst,
                                  void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n >= 0 && n % 16 == 0 && scale > 0.f, NKV_EINVAL,
              "fp8_dequantize: n must be a multiple of 16 and scale > 0");
  if (n == 0) return NKV_OK;
  NKV_REQUIRE(src && dst && aligned16(src) && aligned16(dst), NKV_EINVAL,
              "fp8_dequantize: null or misaligned pointer");
  hipLaunchKernelGGL(fp8_dequantize_kernel, dim3(f8_grid(n / 16)), dim3(kF8Threads), 0,
                     as_stream(stream), (const uint8_t*)src, n / 16, scale, (bf16_t*)dst);
  return check_launch("nkv_fp8_dequantize");
}

extern "C" int nkv_store_kvcache_fp8(const void* key, int64_t key_row_stride, const void* value,
                                     int64_t value_row_stride, void* k_cache, void* v_cache,
                                     const int32_t* slot_mapping, int64_t n_tokens,
                                     int32_t n_kv_heads, int32_t head_dim, int64_t n_slots,
                                     float k_scale, float v_scale, void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n_tokens >= 0 && n_kv_heads > 0 && head_dim > 0 && n_slots >= 0 &&
                  k_scale > 0.f && v_scale > 0.f,
              NKV_EINVAL, "store_kvcache_fp8: bad sizes or scales");
  if (n_tokens == 0) return NKV_OK;
  const int64_t row = (int64_t)n_kv_heads * head_dim;
  NKV_REQUIRE(row % 16 == 0 && key_row_stride >= row && value_row_stride >= row &&
                  key_row_stride % 8 == 0 && value_row_stride % 8 == 0,
              NKV_EINVAL, "store_kvcache_fp8: rows must be multiples of 16 elements, strides "
              "multiples of 8 covering the row");
  NKV_REQUIRE(key && value && k_cache && v_cache && slot_mapping && aligned16(key) &&
                  aligned16(value) && aligned16(k_cache) && aligned16(v_cache),
              NKV_EINVAL, "store_kvcache_fp8: null or misaligned pointer");
  const int cpr = (int)(row / 16);
  hipLaunchKernelGGL(store_kvcache_fp8_kernel, dim3(f8_grid(n_tokens * 2 * cpr)),
                     dim3(kF8Threads), 0, as_stream(stream), (const bf16_t*)key, key_row_stride,
                     (const bf16_t*)value, value_row_stride, (uint8_t*)k_cache, (uint8_t*)v_cache,
                     slot_mapping, n_tokens, cpr, n_slots, 1.f / k_scale, 1.f / v_scale);
  return check_launch("nkv_store_kvcache_fp8");
}

extern "C" int nkv_fp8_gather_rows(const void* k_cache, const void* v_cache,
                                   const int32_t* block_tables, int64_t bt_row_stride,
                                   int32_t max_blocks_per_seq, const int32_t* cu_seqlens_k,
                                   int32_t n_seqs, int32_t max_seqlen_k, int32_t n_kv_heads,
                                   int32_t head_dim, int32_t block_size, int64_t n_blocks,
                                   float k_scale, float v_scale, void* k_out, void* v_out,
                                   void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n_seqs >= 0 && max_seqlen_k >= 0 && n_kv_heads > 0 && head_dim > 0 &&
                  block_size > 0 && n_blocks >= 0 && max_blocks_per_seq > 0 &&
                  bt_row_stride >= max_blocks_per_seq && k_scale > 0.f && v_scale > 0.f,
              NKV_EINVAL, "fp8_gather_rows: bad sizes or scales");
  if (n_seqs == 0 || max_seqlen_k == 0) return NKV_OK;
  const int64_t row = (int64_t)n_kv_heads * head_dim;
  NKV_REQUIRE(row % 16 == 0, NKV_EINVAL, "fp8_gather_rows: Hk*D must be a multiple of 16");
  NKV_REQUIRE(k_cache && v_cache && block_tables && cu_seqlens_k && k_out && v_out &&
                  aligned16(k_cache) && aligned16(v_cache) && aligned16(k_out) &&
                  aligned16(v_out),
              NKV_EINVAL, "fp8_gather_rows: null or misaligned pointer");
  const int cpr = (int)(row / 16);
  const int64_t units = (int64_t)max_seqlen_k * 2 * cpr;
  const unsigned gy = (unsigned)std::max<int64_t>(
      1, std::min<int64_t>((units + kF8Threads - 1) / kF8Threads, 1024));
  hipLaunchKernelGGL(fp8_gather_rows_kernel, dim3((unsigned)n_seqs, gy), dim3(kF8Threads), 0,
                     as_stream(stream), (const uint8_t*)k_cache, (const uint8_t*)v_cache,
                     block_tables, bt_row_stride, max_blocks_per_seq, cu_seqlens_k, block_size,
                     n_blocks, cpr, k_scale, v_scale, (bf16_t*)k_out, (bf16_t*)v_out);
  return check_launch("nkv_fp8_gather_rows");
}

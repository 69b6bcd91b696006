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
// 16 bytes of fp8 out) with full-width loads and stores. Decode, prefill and
// the compression step read fp8 pools themselves (paged_decode.hip,
// prefill.hip, compress.hip).
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
    NKV_DBG(slot < -1 || slot >= n_slots, NKV_DEBUG_SLOT);
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

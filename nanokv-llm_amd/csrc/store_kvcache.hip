// store_kvcache: scatter the step's new K/V rows into the paged cache.
//
// Reference: nanokvllm/layers/attention.py:10-40 (one Triton program per
// token copying Hk*D contiguous elements to row slot_mapping[i]).
//
// MI355X design: the copy is pure HBM traffic (read 2*Hk*D*2 bytes, write the
// same per token). The (token, K|V, 16-byte chunk) space is flattened; each
// thread issues kUnroll independent 16-byte loads (plus the slot of each) before
// any store, lanes of a wave cover consecutive chunks of one row so every
// wave-wide load/store is a coalesced 1 KiB access, and a bounded grid strides
// over the rest (prefill-sized token counts keep ~128 KiB in flight per CU).
#include "nkv_common.h"

namespace nkv {

constexpr int kStoreThreads = 256;
constexpr int kUnroll = 4;

template <typename Chunk>
__global__ __launch_bounds__(kStoreThreads) void store_kvcache_kernel(
    const char* __restrict__ key, int64_t key_stride_b,
    const char* __restrict__ value, int64_t value_stride_b,
    char* __restrict__ k_cache, char* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens,
    int32_t chunks_per_row, int64_t n_slots) {
  const int64_t row_bytes = (int64_t)chunks_per_row * sizeof(Chunk);
  const int64_t per_token = 2 * (int64_t)chunks_per_row;
  const int64_t n_items = n_tokens * per_token;
  const int64_t span = (int64_t)kStoreThreads * kUnroll;
  for (int64_t base = (int64_t)blockIdx.x * span; base < n_items;
       base += (int64_t)gridDim.x * span) {
    Chunk val[kUnroll];
    int64_t dst[kUnroll];  // byte offset of the destination chunk, -1 = skip
    bool is_v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kStoreThreads + threadIdx.x;
      const bool ok = i < n_items;
      const int64_t ic = ok ? i : 0;
      const int64_t tok = ic / per_token;
      const int64_t r = ic - tok * per_token;
      is_v[u] = r >= chunks_per_row;
      const int64_t c = is_v[u] ? r - chunks_per_row : r;
      const char* src = is_v[u] ? value + tok * value_stride_b : key + tok * key_stride_b;
      val[u] = reinterpret_cast<const Chunk*>(src)[c];
      const int64_t slot = slot_mapping[tok];
      // -1 = padding; slots outside the cache are skipped
      NKV_DBG(ok && (slot < -1 || slot >= n_slots), NKV_DEBUG_SLOT);
      dst[u] = (ok && slot >= 0 && slot < n_slots) ? slot * row_bytes + c * (int64_t)sizeof(Chunk)
                                                  : -1;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (dst[u] >= 0) {
        char* cache = is_v[u] ? v_cache : k_cache;
        *reinterpret_cast<Chunk*>(cache + dst[u]) = val[u];
      }
    }
  }
}

}  // namespace nkv

extern "C" int nkv_store_kvcache(const void* key, int64_t key_row_stride,
                                 const void* value, int64_t value_row_stride,
                                 void* k_cache, void* v_cache,
                                 const int32_t* slot_mapping, int64_t n_tokens,
                                 int32_t n_kv_heads, int32_t head_dim, int64_t n_slots,
                                 void* stream) {
  using namespace nkv;
  clear_error();
  NKV_REQUIRE(n_tokens >= 0 && n_kv_heads > 0 && head_dim > 0 && n_slots >= 0, NKV_EINVAL,
              "nkv_store_kvcache: bad sizes (n_tokens=%lld, n_kv_heads=%d, head_dim=%d)",
              (long long)n_tokens, n_kv_heads, head_dim);
  if (n_tokens == 0) return NKV_OK;
  NKV_REQUIRE(key && value && k_cache && v_cache && slot_mapping, NKV_EINVAL,
              "nkv_store_kvcache: null pointer");
  const int64_t row_elems = (int64_t)n_kv_heads * head_dim;
  NKV_REQUIRE(key_row_stride >= row_elems && value_row_stride >= row_elems, NKV_EINVAL,
              "nkv_store_kvcache: row stride smaller than n_kv_heads*head_dim");
  const int64_t row_bytes = row_elems * 2;
  const bool vec = (row_bytes % 16 == 0) && ((key_row_stride * 2) % 16 == 0) &&
                   ((value_row_stride * 2) % 16 == 0) && aligned16(key) && aligned16(value) &&
                   aligned16(k_cache) && aligned16(v_cache);
  const int32_t cpr = (int32_t)(vec ? row_bytes / 16 : row_bytes / 2);
  const int64_t n_items = n_tokens * 2 * cpr;
  const int64_t spans = (n_items + kStoreThreads * kUnroll - 1) / (kStoreThreads * kUnroll);
  const unsigned grid = (unsigned)(spans < 4096 ? spans : 4096);
  hipStream_t s = as_stream(stream);
  if (vec) {
    hipLaunchKernelGGL(store_kvcache_kernel<uint4>, dim3(grid), dim3(kStoreThreads), 0, s,
                       (const char*)key, key_row_stride * 2, (const char*)value,
                       value_row_stride * 2, (char*)k_cache, (char*)v_cache, slot_mapping,
                       n_tokens, cpr, n_slots);
  } else {
    hipLaunchKernelGGL(store_kvcache_kernel<uint16_t>, dim3(grid), dim3(kStoreThreads), 0, s,
                       (const char*)key, key_row_stride * 2, (const char*)value,
                       value_row_stride * 2, (char*)k_cache, (char*)v_cache, slot_mapping,
                       n_tokens, cpr, n_slots);
  }
  return check_launch("nkv_store_kvcache");
}

// store_kvcache: scatter the step's new K/V rows into the paged cache.
//
// Reference: nanokvllm/layers/attention.py:10-40 (one Triton program per
// token copying Hk*D contiguous elements to row slot_mapping[i]).
//
// MI355X design: the copy is pure HBM traffic (read 2*Hk*D*2 bytes, write the
// same per token). Each lane moves one 16-byte chunk, lanes of a wave cover
// consecutive chunks of one row so every wave-wide load/store is a fully
// coalesced 1 KiB access; the K and V rows of a token are handled by the same
// workgroup (256 lanes = 2 rows of 2 KiB at Qwen3 geometry). A grid-stride
// loop keeps the grid bounded for prefill-sized token counts.
#include "nkv_common.h"

namespace nkv {

template <typename Chunk>
__global__ __launch_bounds__(256) void store_kvcache_kernel(
    const char* __restrict__ key, int64_t key_stride_b,
    const char* __restrict__ value, int64_t value_stride_b,
    char* __restrict__ k_cache, char* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens,
    int32_t chunks_per_row, int64_t n_slots) {
  const int64_t row_bytes = (int64_t)chunks_per_row * sizeof(Chunk);
  const int32_t per_token = 2 * chunks_per_row;
  for (int64_t tok = blockIdx.x; tok < n_tokens; tok += gridDim.x) {
    const int64_t slot = slot_mapping[tok];
    if (slot < 0 || slot >= n_slots) continue;  // -1 = padding; others invalid
    const Chunk* ksrc = reinterpret_cast<const Chunk*>(key + tok * key_stride_b);
    const Chunk* vsrc = reinterpret_cast<const Chunk*>(value + tok * value_stride_b);
    Chunk* kdst = reinterpret_cast<Chunk*>(k_cache + slot * row_bytes);
    Chunk* vdst = reinterpret_cast<Chunk*>(v_cache + slot * row_bytes);
    for (int32_t r = threadIdx.x; r < per_token; r += blockDim.x) {
      if (r < chunks_per_row) {
        kdst[r] = ksrc[r];
      } else {
        vdst[r - chunks_per_row] = vsrc[r - chunks_per_row];
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
  const unsigned grid = (unsigned)(n_tokens < 65536 ? n_tokens : 65536);
  hipStream_t s = as_stream(stream);
  if (vec) {
    hipLaunchKernelGGL(store_kvcache_kernel<uint4>, dim3(grid), dim3(256), 0, s,
                       (const char*)key, key_row_stride * 2, (const char*)value,
                       value_row_stride * 2, (char*)k_cache, (char*)v_cache, slot_mapping,
                       n_tokens, cpr, n_slots);
  } else {
    hipLaunchKernelGGL(store_kvcache_kernel<uint16_t>, dim3(grid), dim3(256), 0, s,
                       (const char*)key, key_row_stride * 2, (const char*)value,
                       value_row_stride * 2, (char*)k_cache, (char*)v_cache, slot_mapping,
                       n_tokens, cpr, n_slots);
  }
  return check_launch("nkv_store_kvcache");
}

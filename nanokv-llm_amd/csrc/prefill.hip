// Varlen causal prefill over the paged K/V cache (bf16 MFMA).
//
// Reference: flash_attn_varlen_func(..., causal=True, block_table) at
// nanokvllm/layers/attention.py:96-102.
#include "nkv_common.h"

extern "C" int nkv_prefill_varlen(const void* q, int64_t q_row_stride, const void* k_cache,
                                  const void* v_cache, int64_t kv_row_stride,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  const int32_t* block_tables, int64_t bt_row_stride,
                                  int32_t n_seqs, int32_t max_seqlen_q, int32_t n_q_heads,
                                  int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                                  int64_t n_rows, float scale, void* out, int64_t out_row_stride,
                                  void* stream) {
  nkv::clear_error();
  nkv::set_error("nkv_prefill_varlen: not implemented yet");
  return NKV_EUNSUPPORTED;
}

/*
 * nkv.h -- C ABI of libnkv_amd.so, the MI355X (gfx950) attention hot path of
 * nano-kvllm: paged K/V store, paged decode attention, varlen causal prefill
 * over the paged cache, and the window-based periodic KV-compression step;
 * beside it the steps either side of the path: the fused q/k RMSNorm + RoPE
 * + K/V store, and the per-step metadata builders.
 *
 * Conventions (every entry point):
 *   - All tensor pointers are DEVICE pointers. Element types are fixed per
 *     argument: bf16 for q/k/v/cache/out, int32 for metadata (int64 for
 *     token positions), fp32 for scores and the rotary cos/sin table.
 *   - Strides are in ELEMENTS of the pointed-to type.
 *   - `stream` is a hipStream_t (NULL = the null stream). Every call is
 *     asynchronous on that stream, performs no host<->device synchronisation
 *     and allocates no memory; callers pass workspaces explicitly.
 *   - Return value: NKV_OK (0) or a negative NKV_E* code; nkv_last_error()
 *     then holds a human-readable message (thread-local).
 *   - K/V cache layout is the reference's [num_blocks, block_size, Hk, D]
 *     with the token row contiguous (stride(1) == Hk*D), i.e. slot s of the
 *     flattened cache holds Hk*D elements starting at s*Hk*D.
 *     (nanokvllm/engine/model_runner.py:145, nanokvllm/layers/attention.py:38)
 */
#ifndef NKV_H
#define NKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NKV_OK 0
#define NKV_EINVAL (-1)  /* bad argument: shape, stride, alignment, null pointer */
#define NKV_ELAUNCH (-2) /* HIP launch / runtime error */
#define NKV_EWORKSPACE (-3) /* workspace missing or too small */
#define NKV_EUNSUPPORTED (-4) /* valid but unsupported configuration */

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* nkv_last_error(void);

/* Library version string. */
const char* nkv_version(void);

/*
 * Input checks of the debug build. The kernels run asynchronously and cannot
 * return an error, so inputs the reference would stop on (its asserts, e.g.
 * nanokvllm/layers/attention.py:36-39 and layers/compress_utils.py:39-41) or
 * would read or write out of bounds with are skipped or clamped silently: a
 * slot past the pool, a block-table entry outside the pool where a sequence
 * needs a block, a context longer than its table row. libnkv_amd_debug.so
 * (the same sources built with NKV_DEBUG) also records each such input as one
 * of the bits below, in a word per device. nkv_debug_flags waits for the
 * current device (hipDeviceSynchronize: the one call of this ABI that
 * synchronises), stores the bits recorded there since the last clearing call
 * in *flags and clears them if `clear` is non-zero. The release library sets
 * *flags = 0 and returns NKV_EUNSUPPORTED. No counterpart in the reference.
 */
#define NKV_DEBUG_SLOT 1u     /* store: slot_mapping entry < -1 or >= n_slots (row skipped) */
#define NKV_DEBUG_BLOCK 2u    /* a needed block-table entry (or contiguous K/V row) outside
                                 the cache: its rows read as zeros */
#define NKV_DEBUG_LENGTH 4u   /* a context longer than its table row covers, a negative
                                 length, or a prefill sequence with Lq > Lk (clamped) */
#define NKV_DEBUG_POSITION 8u /* q/k norm + RoPE: position outside [0, max_position)
                                 (clamped) */
int nkv_debug_flags(uint32_t* flags, int clear);

/*
 * store_kvcache: for every token i < n_tokens with slot_mapping[i] != -1,
 * copy key[i] and value[i] (n_kv_heads*head_dim contiguous elements each)
 * into row slot_mapping[i] of k_cache / v_cache. Rows with slot -1 are
 * skipped; slots outside [0, n_slots) are skipped as well (the reference
 * would write out of bounds there).
 * key/value rows may be strided views (e.g. the v part of a fused qkv
 * projection): element (i, h, d) lives at ptr[i*row_stride + h*head_dim + d].
 * Elements are 2-byte (bf16 or fp16, the model's dtype): the rows are copied
 * as they are.
 * Replaces: store_kvcache / store_kvcache_kernel,
 *           nanokvllm/layers/attention.py:10-40
 */
int nkv_store_kvcache(const void* key, int64_t key_row_stride,
                      const void* value, int64_t value_row_stride,
                      void* k_cache, void* v_cache,
                      const int32_t* slot_mapping, int64_t n_tokens,
                      int32_t n_kv_heads, int32_t head_dim, int64_t n_slots,
                      void* stream);

/*
 * fp8 K/V (OCP E4M3FN: bias 7, largest finite 448, round to nearest even).
 * An fp8 pool stores code = E4M3FN(clamp(x * (1/scale), -448, 448)) (NaN kept)
 * with one scale per K or V cache, and reads code * scale.
 *   nkv_fp8_quantize:   dst[i] = code of src[i] (bf16 in, 1 byte out)
 *   nkv_fp8_dequantize: dst[i] = bf16(value(src[i]) * scale)
 *   nkv_store_kvcache_fp8: store_kvcache into fp8 caches (same slot rules as
 *     nkv_store_kvcache; rows of n_kv_heads*head_dim codes).
 * n and rows are multiples of 16 elements, pointers 16-byte aligned.
 * Replaces: the store of an fp8 pool (store_kvcache, nanokvllm/layers/attention.py:10-40;
 *           pool of ModelRunner.allocate_kv_cache, nanokvllm/engine/model_runner.py:133-152).
 */
int nkv_fp8_quantize(const void* src, int64_t n, float scale, void* dst, void* stream);
int nkv_fp8_dequantize(const void* src, int64_t n, float scale, void* dst, void* stream);
int nkv_store_kvcache_fp8(const void* key, int64_t key_row_stride, const void* value,
                          int64_t value_row_stride, void* k_cache, void* v_cache,
                          const int32_t* slot_mapping, int64_t n_tokens, int32_t n_kv_heads,
                          int32_t head_dim, int64_t n_slots, float k_scale, float v_scale,
                          void* stream);

/*
 * Fused q/k RMSNorm + rotary embedding + K/V store, the step between the qkv
 * projection and attention. q, k, v are row-strided bf16 views: element
 * (i, h, d) of q at q[i*q_row_stride + h*head_dim + d], likewise k and v
 * (normally the three parts of one fused qkv row). For every token i and q or
 * k head (head_dim D = 64, 128 or 256; Qwen3: 128):
 *   x   = head row (fp32);
 *   if norm weights are given (both, or neither = no norm):
 *     x = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)   (w = q or k weight)
 *   x1, x2 = x[:D/2], x[D/2:];  c, s = cos_sin_cache[p][:D/2], [p][D/2:]
 *   y   = bf16([x1*c - x2*s | x2*c + x1*s])            (p = positions[i])
 * q heads -> q_out[i*q_out_row_stride + h*D ...]; k heads -> k_out
 * ([n_tokens, n_kv_heads, D] contiguous, optional) and, with a cache, the
 * k_cache row slot_mapping[i]; v heads are copied unchanged to the v_cache
 * row. Slots -1 or outside [0, n_slots) are skipped; positions outside
 * [0, max_position) are clamped (the reference would raise an index error).
 * positions is int64 and cos_sin_cache fp32 [max_position, D] as the
 * reference builds them. k_cache, v_cache, v and slot_mapping are all given
 * or all NULL; at least one of k_out and k_cache is given. Pointers are
 * 16-byte aligned and row strides multiples of 8 elements.
 * Replaces: q_norm/k_norm + rotary_emb in Qwen3Attention.forward
 *           (nanokvllm/models/qwen3.py:109-113), RMSNorm.rms_forward
 *           (nanokvllm/layers/layernorm.py:16-26), apply_rotary_emb /
 *           RotaryEmbedding.forward (nanokvllm/layers/rotary_embedding.py:7-49)
 *           and the store_kvcache call at the top of Attention.forward
 *           (nanokvllm/layers/attention.py:71-73).
 */
int nkv_qk_norm_rope_store(const void* q, int64_t q_row_stride, const void* k,
                           int64_t k_row_stride, const void* v, int64_t v_row_stride,
                           const int64_t* positions, const void* q_norm_weight,
                           const void* k_norm_weight, float eps,
                           const float* cos_sin_cache, int64_t max_position,
                           void* q_out, int64_t q_out_row_stride, void* k_out,
                           void* k_cache, void* v_cache, const int32_t* slot_mapping,
                           int64_t n_slots, int64_t n_tokens, int32_t n_q_heads,
                           int32_t n_kv_heads, int32_t head_dim, void* stream);

/* fp16 model dtype: nkv_qk_norm_rope_store with q, k, v, the norm weights, q_out,
 * k_out and the caches in fp16 and every rounding to fp16 (the reference's
 * .to(orig_dtype) for an fp16 checkpoint). Replaces: the same calls
 * (qwen3.py:109-113, layernorm.py:16-26, rotary_embedding.py:7-49,
 * attention.py:71-73) when torch_dtype is float16 (model_runner.py:27). */
int nkv_qk_norm_rope_store_f16(const void* q, int64_t q_row_stride, const void* k,
                               int64_t k_row_stride, const void* v, int64_t v_row_stride,
                               const int64_t* positions, const void* q_norm_weight,
                               const void* k_norm_weight, float eps,
                               const float* cos_sin_cache, int64_t max_position,
                               void* q_out, int64_t q_out_row_stride, void* k_out,
                               void* k_cache, void* v_cache, const int32_t* slot_mapping,
                               int64_t n_slots, int64_t n_tokens, int32_t n_q_heads,
                               int32_t n_kv_heads, int32_t head_dim, void* stream);

/*
 * Paged decode attention (one query token per sequence, GQA, causal with the
 * new token already stored): for b < batch, query head h,
 *   out[b,h] = sum_{t<ctx_b} softmax_t(scale * q[b,h].K[b,t,h/g]) V[b,t,h/g]
 * with K[b,t] = k_cache row (block_tables[b, t/block_size]*block_size
 * + t%block_size). Sequences with context_lens[b] <= 0 produce zeros.
 * Balanced split-K over 16-token chunks, then a combine pass; workspace
 * must hold nkv_paged_decode_workspace_bytes(...), which is sized by what the
 * split grid can write on the current device (descriptors per sequence and
 * KV head, then partial rows: batch*Hq plus at most 8 resident waves per CU
 * x 16 query heads, (head_dim + 4) * 4 bytes each; ~35 MB at batch 500, Hq 64,
 * head_dim 128, 64-block tables), not by batch x table width. Calls on one
 * stream may share one workspace (the layers of a model, one after another).
 * q[b,h,d] at q[b*q_row_stride + h*head_dim + d]; out likewise with
 * out_row_stride. head_dim 64, 128 or 256 (out then 2-, 4- or 8-byte aligned
 * with a row stride that is a multiple of head_dim/64); any GQA group
 * n_q_heads/n_kv_heads up to 256 (above 16 the group's query heads are split
 * over ceil(g/16) waves, each reading the KV head's rows: K/V are then read
 * ceil(g/16) times); block_size a multiple of 16. Block-table
 * entries outside [0, n_blocks) contribute nothing.
 * Replaces: flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 *           cache_seqlens=context_lens, block_table=block_tables,
 *           softmax_scale=scale, causal=True),
 *           nanokvllm/layers/attention.py:104-107
 */
size_t nkv_paged_decode_workspace_bytes(int32_t batch, int32_t n_q_heads,
                                        int32_t head_dim, int32_t max_blocks_per_seq,
                                        int32_t block_size);

int nkv_paged_decode(const void* q, int64_t q_row_stride,
                     const void* k_cache, const void* v_cache,
                     const int32_t* block_tables, int64_t bt_row_stride,
                     const int32_t* context_lens, int32_t batch,
                     int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                     int32_t block_size, int32_t max_blocks_per_seq,
                     int64_t n_blocks, float scale,
                     void* out, int64_t out_row_stride,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Paged decode that allocates nothing and takes no workspace: the same arguments
 * (without workspace/workspace_bytes), kernels and result as nkv_paged_decode,
 * with the partials in a fixed device array of NKV_DECODE_NOALLOC_MAX_BYTES that
 * the library holds on every GPU it runs on until the process ends. A call whose
 * partials would exceed it (nkv_paged_decode_workspace_bytes is an upper bound;
 * about batch * n_q_heads <= 94k at 256 CUs) returns NKV_EUNSUPPORTED before
 * launching anything. Nothing in the array needs to start at zero. Every call on a
 * GPU uses that GPU's one array: calls that overlap on one GPU (different streams
 * without ordering between them) race and give wrong results.
 * No counterpart in the reference: for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
#define NKV_DECODE_NOALLOC_MAX_BYTES (64u << 20)
int nkv_paged_decode_noalloc(const void* q, int64_t q_row_stride,
                             const void* k_cache, const void* v_cache,
                             const int32_t* block_tables, int64_t bt_row_stride,
                             const int32_t* context_lens, int32_t batch,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                             int32_t block_size, int32_t max_blocks_per_seq,
                             int64_t n_blocks, float scale,
                             void* out, int64_t out_row_stride, void* stream);

/* Paged decode over fp8 (OCP E4M3FN) caches: same arguments and result as
 * nkv_paged_decode with K = code * k_scale and V = code * v_scale (codes of
 * nkv_store_kvcache_fp8); half the cache bytes per decoded token. Same
 * workspace size. Replaces: the same flash_attn_with_kvcache call
 * (attention.py:104-107) over an fp8 pool. */
int nkv_paged_decode_fp8(const void* q, int64_t q_row_stride,
                         const void* k_cache, const void* v_cache,
                         const int32_t* block_tables, int64_t bt_row_stride,
                         const int32_t* context_lens, int32_t batch,
                         int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t block_size, int32_t max_blocks_per_seq,
                         int64_t n_blocks, float scale, float k_scale, float v_scale,
                         void* out, int64_t out_row_stride,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Paged decode for an fp16 model: nkv_paged_decode with q, the caches and out in
 * fp16 (fp16 MFMA, fp32 softmax and accumulation). Same workspace size.
 * Replaces: the same flash_attn_with_kvcache call (attention.py:104-107) with
 * the fp16 pool the reference allocates for a float16 checkpoint
 * (model_runner.py:27, 142-145). */
int nkv_paged_decode_f16(const void* q, int64_t q_row_stride,
                         const void* k_cache, const void* v_cache,
                         const int32_t* block_tables, int64_t bt_row_stride,
                         const int32_t* context_lens, int32_t batch,
                         int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t block_size, int32_t max_blocks_per_seq,
                         int64_t n_blocks, float scale,
                         void* out, int64_t out_row_stride,
                         void* workspace, size_t workspace_bytes, void* stream);

/* The two stages nkv_paged_decode launches, exported so a caller can time or
 * schedule them separately. Same arguments as nkv_paged_decode.
 * Replaces: the same flash_attn_with_kvcache call (attention.py:104-107). */
int nkv_paged_decode_split(const void* q, int64_t q_row_stride,
                           const void* k_cache, const void* v_cache,
                           const int32_t* block_tables, int64_t bt_row_stride,
                           const int32_t* context_lens, int32_t batch,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           int32_t block_size, int32_t max_blocks_per_seq,
                           int64_t n_blocks, float scale,
                           void* workspace, size_t workspace_bytes, void* stream);
int nkv_paged_decode_combine(const int32_t* context_lens, int32_t batch,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                             int32_t block_size, int32_t max_blocks_per_seq,
                             void* out, int64_t out_row_stride,
                             const void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * Varlen causal prefill over K/V rows (flash-attn bottom-right causal):
 * sequence i has Lq = cu_seqlens_q[i+1]-cu_seqlens_q[i] query rows and
 * Lk = cu_seqlens_k[i+1]-cu_seqlens_k[i] keys; query j attends keys
 * 0 .. Lk-Lq+j. If block_tables != NULL, key t of sequence i is k_cache row
 * block_tables[i, t/block_size]*block_size + t%block_size (paged); otherwise
 * it is row cu_seqlens_k[i]+t of k_cache/v_cache (contiguous [sum Lk, Hk, D]
 * with row strides k_row_stride / v_row_stride, e.g. a roped K next to V as a
 * view of the qkv projection; paged caches share one stride). Table entries at or beyond
 * max_blocks_per_seq, negative, or past n_rows read as zero keys/values.
 * q/out are [sum Lq, Hq, D] with row strides. head_dim 64, 128 or 256; any
 * GQA group Hq/Hk up to 128 (64 at head_dim 256: a tile holds 128 (64) query x
 * head rows). Rows with no visible key (Lk < Lq) are zero.
 * Replaces: flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
 *           max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True,
 *           block_table), nanokvllm/layers/attention.py:96-102
 */
int nkv_prefill_varlen(const void* q, int64_t q_row_stride,
                       const void* k_cache, const void* v_cache, int64_t k_row_stride,
                       int64_t v_row_stride,
                       const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                       const int32_t* block_tables, int64_t bt_row_stride,
                       int32_t max_blocks_per_seq, int32_t n_seqs, int32_t max_seqlen_q,
                       int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                       int32_t block_size, int64_t n_rows, float scale,
                       void* out, int64_t out_row_stride, void* stream);

/* Varlen causal prefill over a paged fp8 (OCP E4M3FN) pool: the paged mode of
 * nkv_prefill_varlen with K = code * k_scale and V = code * v_scale (codes of
 * nkv_store_kvcache_fp8), cache rows of n_kv_heads*head_dim bytes and n_blocks
 * blocks. The kernel widens the codes to bf16 (exact) as it stages them; no
 * intermediate buffer. Replaces: the flash_attn_varlen_func(..., block_table)
 * call (nanokvllm/layers/attention.py:96-102) over an fp8 pool. */
int nkv_prefill_varlen_fp8(const void* q, int64_t q_row_stride,
                           const void* k_cache, const void* v_cache,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                           const int32_t* block_tables, int64_t bt_row_stride,
                           int32_t max_blocks_per_seq, int32_t n_seqs, int32_t max_seqlen_q,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           int32_t block_size, int64_t n_blocks, float scale, float k_scale,
                           float v_scale, void* out, int64_t out_row_stride, void* stream);

/* Varlen causal prefill for an fp16 model: nkv_prefill_varlen with q, K/V (paged
 * or contiguous) and out in fp16. Replaces: the flash_attn_varlen_func call
 * (attention.py:96-102) for a float16 checkpoint (model_runner.py:27). */
int nkv_prefill_varlen_f16(const void* q, int64_t q_row_stride,
                           const void* k_cache, const void* v_cache, int64_t k_row_stride,
                           int64_t v_row_stride,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                           const int32_t* block_tables, int64_t bt_row_stride,
                           int32_t max_blocks_per_seq, int32_t n_seqs, int32_t max_seqlen_q,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           int32_t block_size, int64_t n_rows, float scale,
                           void* out, int64_t out_row_stride, void* stream);

/* Aggregation of key importance over query heads (compression scoring). */
#define NKV_AGG_ALL 0   /* sum over all Hq heads -> one kept set per sequence
                           (nanokvllm/layers/CompressMethod.py:41-42) */
#define NKV_AGG_GROUP 1 /* sum over the g query heads of each KV head -> one
                           kept set per (sequence, KV head) */

/*
 * Compression scoring (SnapKV with window = 1): for selected sequence j
 * (batch row seq_idx[j]) the window is its last `window_blocks` FULL blocks,
 * located from base_context_lens[seq_idx[j]] and block_tables. Keys
 * t < W*B-1 of the window are scored with the sequence's current query:
 *   imp[j, s, t] = sum_{h in set s} softmax_t(scale * q[h].K[t, h/g])
 * with key 0 masked to -inf (attention sink) before the softmax.
 * importance_out: fp32 [m, n_sets, W*B-1], n_sets = 1 (ALL) or n_kv_heads
 * (GROUP). workspace: nkv_compress_workspace_bytes(...). head_dim 64, 128 or
 * 256 (every compression entry point; the fused one-launch kernels of
 * nkv_compress_select / nkv_compress_step serve head_dim 128 with windows of
 * up to 1024 tokens, other shapes take the score / importance / top-k /
 * compaction kernels, same results).
 * If block_tables == NULL the keys come from a contiguous K tensor
 * [m, Hk, L, D] (k_cache points at it, L = window_blocks*block_size), as in
 * SnapKV(Q, K, V, ...) called directly; seq_idx and base_context_lens are
 * then ignored.
 * Replaces: get_tail_window_and_tail_slots + gather_kv_by_slots + the scoring
 *           half of SnapKV, nanokvllm/layers/compress_utils.py:9-97,155-173,
 *           nanokvllm/layers/CompressMethod.py:4-42
 */
size_t nkv_compress_workspace_bytes(int32_t m, int32_t n_q_heads,
                                    int32_t window_blocks, int32_t block_size);

int nkv_compress_score(const void* q, int64_t q_row_stride,
                       const void* k_cache, const int32_t* block_tables,
                       int64_t bt_row_stride, int32_t max_blocks_per_seq,
                       const int32_t* base_context_lens,
                       const int32_t* seq_idx, int32_t m,
                       int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                       int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                       float scale, int32_t agg_mode, float* importance_out,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Top-k selection on importance [m*n_sets, n_cand] (fp32): keep the num_keep
 * largest (ties -> lower index first), sorted ascending, and emit
 *   keep_idx[r] = [0, kept..., n_cand]  (1 + num_keep + 1 int32 entries)
 * i.e. the reference's [bos, sorted top-k, last window token].
 * Requires num_keep < n_cand <= 4096.
 * Replaces: the topk/sort/cat tail of SnapKV, CompressMethod.py:44-57
 */
int nkv_compress_topk(const float* importance, int32_t n_rows, int32_t n_cand,
                      int32_t num_keep, int32_t* keep_idx, void* stream);

/*
 * Fused selection: score + importance + top-k in one launch (agg "group") or
 * two (agg "all": per-KV-head partial importance, then their sum and the
 * top-k) when W*B <= 1024 and B % 64 == 0 (the reference's W = 4, B = 256
 * qualifies); otherwise nkv_compress_score + nkv_compress_topk run on the
 * same workspace. Any GQA group Hq/Hk (the fused kernels take up to 16; larger
 * groups score in passes of 16 query rows). Outputs are those of the two
 * calls:
 *   importance_out fp32 [m, n_sets, W*B-1],
 *   keep_idx int32 [m, n_sets, num_keep+2] = [0, ascending kept..., W*B-1].
 * Workspace: caller-owned, >= nkv_compress_select_workspace_bytes bytes.
 * Replaces: the scoring and selection of MyCompressCompact, i.e. SnapKV
 *           (nanokvllm/layers/CompressMethod.py:4-57) as called from
 *           nanokvllm/layers/compress_utils.py:133-183
 */
size_t nkv_compress_select_workspace_bytes(int32_t m, int32_t n_q_heads, int32_t n_kv_heads,
                                           int32_t window_blocks, int32_t block_size);

int nkv_compress_select(const void* q, int64_t q_row_stride,
                        const void* k_cache, const int32_t* block_tables,
                        int64_t bt_row_stride, int32_t max_blocks_per_seq,
                        const int32_t* base_context_lens,
                        const int32_t* seq_idx, int32_t m,
                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                        float scale, int32_t agg_mode, int32_t num_keep,
                        float* importance_out, int32_t* keep_idx,
                        void* workspace, size_t workspace_bytes, void* stream);
/* nkv_compress_select with fp16 q and K (an fp16 pool). Replaces: the same
 * scoring and selection for a float16 checkpoint. */
int nkv_compress_select_f16(const void* q, int64_t q_row_stride,
                            const void* k_cache, const int32_t* block_tables,
                            int64_t bt_row_stride, int32_t max_blocks_per_seq,
                            const int32_t* base_context_lens,
                            const int32_t* seq_idx, int32_t m,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                            int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                            float scale, int32_t agg_mode, int32_t num_keep,
                            float* importance_out, int32_t* keep_idx,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * SnapKV as the compression plug-in calls it (contiguous tensors): Q [m, Hq,
 * window, D], K [m, Hk, seq_len, D] (bf16, both contiguous). With w = window and
 * n_cand = seq_len - w, the importance of key t < n_cand is
 *   imp[j, s, t] = sum_{h in set s} sum_{i < w} softmax_t(scale * Q[j,h,i].K[j,h/g,t])
 * with key 0 masked (attention sink) and the w query-window keys not scored;
 * importance_out fp32 [m, n_sets, n_cand] (n_sets 1 for ALL, Hk for GROUP),
 * keep_idx int32 [m, n_sets, num_keep + 1 + w] =
 *   [0, ascending top-num_keep (ties -> lower index), n_cand, ..., seq_len - 1].
 * window 1 is nkv_compress_select on the contiguous K; any seq_len (keys are
 * scored in 256-key chunks, the last one masked) with n_cand <= 4096.
 * Workspace: nkv_snapkv_workspace_bytes(...).
 * Replaces: SnapKV(Q, K, V, num_keep, window), nanokvllm/layers/CompressMethod.py:4-57
 *           (the policy API of CHANGE_LOG.md:197-208).
 */
size_t nkv_snapkv_workspace_bytes(int32_t m, int32_t n_q_heads, int32_t n_kv_heads,
                                  int32_t seq_len, int32_t window);
int nkv_snapkv_select(const void* q, const void* k, int32_t m, int32_t n_q_heads,
                      int32_t n_kv_heads, int32_t head_dim, int32_t seq_len, int32_t window,
                      float scale, int32_t agg_mode, int32_t num_keep, float* importance_out,
                      int32_t* keep_idx, void* workspace, size_t workspace_bytes,
                      void* stream);
/* nkv_snapkv_select with fp16 Q and K. Replaces: SnapKV (CompressMethod.py:4-57)
 * on fp16 tensors. */
int nkv_snapkv_select_f16(const void* q, const void* k, int32_t m, int32_t n_q_heads,
                          int32_t n_kv_heads, int32_t head_dim, int32_t seq_len,
                          int32_t window, float scale, int32_t agg_mode, int32_t num_keep,
                          float* importance_out, int32_t* keep_idx, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * One layer's compression step: nkv_compress_select (num_keep = keep_tokens-2)
 * followed by nkv_compress_compact, fused when the selection is (one launch
 * for agg "group": each (sequence, KV head) workgroup scores, selects and
 * compacts its KV head; two for agg "all": per-KV-head partial importance,
 * then sum + select + compact). Same outputs and cache/context_lens effects
 * as the two calls. Workspace as nkv_compress_select.
 * Replaces: MyCompressCompact's per-layer work (scoring, selection,
 *           compaction, context_lens), nanokvllm/layers/compress_utils.py:100-263
 */
int nkv_compress_step(const void* q, int64_t q_row_stride, void* k_cache, void* v_cache,
                      const int32_t* block_tables, int64_t bt_row_stride,
                      int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                      int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                      int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                      int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                      float scale, int32_t agg_mode, int32_t keep_tokens,
                      float* importance_out, int32_t* keep_idx,
                      void* workspace, size_t workspace_bytes, void* stream);
/* nkv_compress_step with fp16 q and caches (the compaction moves 2-byte rows
 * either way). Replaces: MyCompressCompact's per-layer work
 * (compress_utils.py:100-263) for a float16 checkpoint. */
int nkv_compress_step_f16(const void* q, int64_t q_row_stride, void* k_cache, void* v_cache,
                          const int32_t* block_tables, int64_t bt_row_stride,
                          int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                          int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                          int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                          float scale, int32_t agg_mode, int32_t keep_tokens,
                          float* importance_out, int32_t* keep_idx,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * The last layer's compression step: nkv_compress_step followed by
 * nkv_compress_finalize (same arguments, same effects), in the step's launch
 * when it is fused (m <= 16384): the bookkeeping of each selected sequence is
 * done by the last of its (sequence, KV head) workgroups to arrive, after all
 * of them have read its block-table row, so it needs no launch of its own.
 * Arrival counters are device-global and zero between calls; calls that
 * overlap on one GPU (concurrent streams) must not. block_tables is written
 * (rewrite_tables) as by nkv_compress_finalize.
 * Replaces: MyCompressCompact on the last layer (layer_id + 1 == num_layers):
 *           the per-layer work and the event construction,
 *           nanokvllm/layers/compress_utils.py:100-290, with the table/slot
 *           effect of Scheduler.postprocess + BlockManager.truncate_blocks
 *           (nanokvllm/engine/scheduler.py:104-125,
 *            nanokvllm/engine/block_manager.py:117-138)
 */
int nkv_compress_step_finalize(const void* q, int64_t q_row_stride, void* k_cache,
                               void* v_cache, int32_t* block_tables, int64_t bt_row_stride,
                               int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                               int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                               int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                               int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                               float scale, int32_t agg_mode, int32_t keep_tokens,
                               float* importance_out, int32_t* keep_idx, void* workspace,
                               size_t workspace_bytes, int32_t rewrite_tables,
                               int32_t* slot_mapping, int32_t* events, void* stream);
/* nkv_compress_step_finalize with fp16 q and caches. Replaces: as
 * nkv_compress_step_finalize, for a float16 checkpoint. */
int nkv_compress_step_finalize_f16(const void* q, int64_t q_row_stride, void* k_cache,
                                   void* v_cache, int32_t* block_tables, int64_t bt_row_stride,
                                   int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                                   int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                                   int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                   int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                                   float scale, int32_t agg_mode, int32_t keep_tokens,
                                   float* importance_out, int32_t* keep_idx, void* workspace,
                                   size_t workspace_bytes, int32_t rewrite_tables,
                                   int32_t* slot_mapping, int32_t* events, void* stream);

/*
 * In-place compaction of the window of each selected sequence, K and V:
 * kept window token keep_idx[j,s,i] moves to window position i
 * (i < keep_tokens); tail token u (tail = len % B tokens, block
 * block_tables[seq, len/B]) moves to window position keep_tokens + u (the
 * window blocks, then the tail block). That is the reference's slot
 * slot(keep_tokens-1)+1+u whenever that slot stays in its block (always for
 * the default keep 2*B+1); past it the reference writes into an unrelated
 * block (compress_utils.py:210-231). Rows move in ascending rounds, each
 * round's reads before its writes, and no row moves to a later position, so
 * overlapping sources and destinations behave like the reference's
 * two-phase index_select().clone() / index_copy_, for any keep_tokens <= W*B.
 * Then context_lens[seq_idx[j]] = len - W*B + keep_tokens.
 * keep_idx: int32 [m, n_sets, keep_tokens] with n_sets 1 (shared by all KV
 * heads) or n_kv_heads, ascending per row.
 * Replaces: MyCompressCompact's compaction and context_lens update,
 *           nanokvllm/layers/compress_utils.py:186-263
 */
int nkv_compress_compact(void* k_cache, void* v_cache,
                         const int32_t* block_tables, int64_t bt_row_stride,
                         int32_t max_blocks_per_seq,
                         const int32_t* base_context_lens, int32_t* context_lens,
                         const int32_t* seq_idx, int32_t m,
                         const int32_t* keep_idx, int32_t n_sets, int32_t keep_tokens,
                         int32_t n_kv_heads, int32_t head_dim, int32_t block_size,
                         int32_t window_blocks, int64_t n_blocks, void* stream);

/*
 * Last-layer bookkeeping of a compression step, after the compaction of every
 * layer: for selected sequence j (new_len = len - W*B + keep_tokens,
 * keep_blocks = ceil(new_len / B)) write
 *   events[j, :] = [seq_idx[j], new_len, keep_blocks, n_freed, freed ids...,
 *                   -1 padding]   (int32, row length 4 + max_blocks_per_seq)
 * where the freed ids are block_tables[seq, keep_blocks:] entries >= 0. A
 * selected sequence the step left unchanged (fewer than window_blocks full
 * blocks, or a table too short: the reference asserts there) reads
 * [seq, len, ceil(len/B), -1, -1...] (n_freed = -1: skipped) and its table
 * and slot are not rewritten. Then, for the others,
 * if rewrite_tables != 0, set those block_tables entries to -1 and, if
 * slot_mapping != NULL, set slot_mapping[seq] to the slot of token position
 * new_len (-1 if that position starts a new block).
 * Replaces: the event construction of MyCompressCompact
 *           (compress_utils.py:266-288) and the table/slot effect of
 *           Scheduler.postprocess + BlockManager.truncate_blocks
 *           (nanokvllm/engine/scheduler.py:104-125,
 *            nanokvllm/engine/block_manager.py:117-138)
 */
int nkv_compress_finalize(int32_t* block_tables, int64_t bt_row_stride,
                          int32_t max_blocks_per_seq,
                          const int32_t* base_context_lens, const int32_t* seq_idx,
                          int32_t m, int32_t keep_tokens, int32_t block_size,
                          int32_t window_blocks, int32_t rewrite_tables,
                          int32_t* slot_mapping, int32_t* events, void* stream);

/*
 * Device-side compression scheduling (graph-capturable): advances
 * *step_counter by one; when the new value is a multiple of period, sequence
 * i < batch is eligible iff context_lens[i] % block_size != block_size - 1,
 * tail_uncompressed[i] >= window_blocks*block_size and
 * context_lens[i] / block_size >= window_blocks; seq_idx[0:topk] receives the
 * first topk eligible indices in batch order (policy 0) or the topk longest
 * (policy 1, ties to the lower index), padded with -1; *n_selected the count;
 * base_context_lens (optional) a copy of context_lens; batch <= 16384. Every compression
 * entry point accepts such a -1 padded seq_idx (padding rows are skipped;
 * their importance / keep_idx rows are left unwritten, their event rows read
 * [-1, 0, 0, 0, -1...]), so a step can always be launched with m = topk.
 * Replaces: the compression block of ModelRunner.prepare_decode
 *           (nanokvllm/engine/model_runner.py:300-332).
 */
int nkv_compress_schedule(const int32_t* context_lens, const int32_t* tail_uncompressed,
                          int32_t batch, int32_t block_size, int32_t window_blocks,
                          int32_t topk, int32_t period, int32_t policy, int32_t* step_counter,
                          int32_t* seq_idx, int32_t* n_selected, int32_t* base_context_lens,
                          void* stream);

/* The compression step over fp8 (OCP E4M3FN) caches (nkv_store_kvcache_fp8 codes):
 * same arguments and effects as nkv_compress_step with K = code * k_scale;
 * scoring widens K to bf16, compaction moves the 1-byte rows. Needs the
 * workspace of nkv_compress_workspace_bytes (or more); block_size a multiple
 * of 256. -1 padded seq_idx accepted.
 * Replaces: MyCompressCompact (compress_utils.py:100-290) over an fp8 pool. */
int nkv_compress_step_fp8(const void* q, int64_t q_row_stride, void* k_cache, void* v_cache,
                          const int32_t* block_tables, int64_t bt_row_stride,
                          int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                          int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                          int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                          float scale, float k_scale, int32_t agg_mode, int32_t keep_tokens,
                          float* importance_out, int32_t* keep_idx, void* workspace,
                          size_t workspace_bytes, void* stream);
/* nkv_compress_step_fp8 followed by nkv_compress_finalize, fused as in
 * nkv_compress_step_finalize (same counters, same rule for overlapping calls).
 * Replaces: MyCompressCompact on the last layer (compress_utils.py:100-290)
 * over an fp8 pool, with the table/slot effect of Scheduler.postprocess +
 * BlockManager.truncate_blocks (scheduler.py:104-125, block_manager.py:117-138). */
int nkv_compress_step_finalize_fp8(const void* q, int64_t q_row_stride, void* k_cache,
                                   void* v_cache, int32_t* block_tables, int64_t bt_row_stride,
                                   int32_t max_blocks_per_seq, const int32_t* base_context_lens,
                                   int32_t* context_lens, const int32_t* seq_idx, int32_t m,
                                   int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                   int32_t block_size, int32_t window_blocks, int64_t n_blocks,
                                   float scale, float k_scale, int32_t agg_mode,
                                   int32_t keep_tokens, float* importance_out, int32_t* keep_idx,
                                   void* workspace, size_t workspace_bytes,
                                   int32_t rewrite_tables, int32_t* slot_mapping,
                                   int32_t* events, void* stream);

/*
 * Per-step attention metadata built on the device from one packed int32
 * buffer (device memory, n = n_seqs):
 *   packed = [starts[n] | num_new[n] | pos_offsets[n] (if flags & NKV_META_POS_OFFSETS)
 *             | tables]
 *   tables, without a table store: [bt_offsets[n+1] | bt_flat[bt_offsets[n]]]
 *     (sequence s's table is bt_flat[bt_offsets[s] .. bt_offsets[s+1]),
 *     offsets nondecreasing from 0);
 *   tables, with table_store [store_rows, store_row_stride] (device, kept by
 *     the caller across steps): [rows[n] | counts[n] | updates[3*n_updates]]
 *     -- first every update (row, col, id) is written to the store, then
 *     sequence s's table is the first counts[s] entries of store row rows[s].
 * Sequence s schedules num_new[s] tokens at KV positions starts[s] ..
 * starts[s]+num_new[s]-1. Outputs:
 *   cu_seqlens_q[n+1] = prefix sums of num_new; cu_seqlens_k[n+1] = prefix
 *   sums of end = starts + num_new; context_lens[n] = end (optional);
 *   logits_indices[n] = cu_seqlens_q[s+1] - 1 (int64, optional);
 *   max_seqlens[2] = {max num_new, max end} (optional);
 *   for token i of s at row r = cu_seqlens_q[s] + i (r < total_tokens):
 *     positions[r] = starts[s] + i + pos_offsets[s] (int64; offset 0 if absent)
 *     slot_mapping[r] = table[kv / block_size] * block_size + kv % block_size
 *                       (kv = starts[s] + i; -1 if the table is too short or
 *                       the entry is negative);
 *   block_tables[s, 0:bt_width] = the table right-padded with -1 (optional).
 * total_tokens = sum(num_new) sizes positions/slot_mapping; max_new_tokens
 * sizes the launch only (any value gives the same result). Negative counts
 * or starts are treated as 0; updates and rows outside the store are ignored.
 * Replaces: ModelRunner.prepare_step's per-token loop and prepare_block_tables
 *           (nanokvllm/engine/model_runner.py:154-219) and the decode builder
 *           of prepare_decode (model_runner.py:265-285: RoPE position =
 *           rope_pos, i.e. pos_offsets = rope_pos - (len - 1)).
 */
#define NKV_META_POS_OFFSETS 1
int nkv_build_step_metadata(const int32_t* packed, int32_t n_seqs, int32_t block_size,
                            int32_t max_new_tokens, int64_t total_tokens, int32_t flags,
                            int32_t* table_store, int64_t store_row_stride, int32_t store_rows,
                            int32_t n_updates, int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                            int32_t* context_lens, int64_t* positions, int32_t* slot_mapping,
                            int64_t* logits_indices, int32_t* max_seqlens,
                            int32_t* block_tables, int64_t bt_row_stride, int32_t bt_width,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NKV_H */

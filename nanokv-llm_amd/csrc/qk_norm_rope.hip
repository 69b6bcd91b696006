// Fused q/k RMSNorm + rotary embedding + K/V store: the step just before the
// attention path.
//
// Reference: Qwen3Attention.forward, nanokvllm/models/qwen3.py:104-114 (qkv
// split, q_norm/k_norm when the projection has no bias, rotary_emb, then
// Attention.forward's store_kvcache); RMSNorm.rms_forward,
// nanokvllm/layers/layernorm.py:16-26 (fp32 variance, x * rsqrt(var + eps)
// rounded to bf16, then * weight rounded to bf16); apply_rotary_emb and
// RotaryEmbedding.forward, nanokvllm/layers/rotary_embedding.py:7-49 (halves
// x1 | x2 in fp32, y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin, rounded to
// bf16; cos_sin_cache[pos] = [cos | sin] of pos * inv_freq, fp32).
//
// MI355X design: one pass over the qkv projection output instead of the
// reference's five (norm q, norm k, rope q, rope k, store k and v). q, k, v
// are row-strided views (normally the three parts of one qkv row). HBM-bound:
// per token it reads the (Hq + 2 Hk) head rows, one cos|sin row (512 bytes at
// head_dim 128) and writes q, the K and V cache rows and optionally a contiguous K.
// A group of D/16 lanes owns one (token, head) unit; lane i holds elements
// [8i, 8i+8) and [D/2+8i, D/2+8i+8) of the head (D = head_dim: 64, 128 or 256),
// so both halves of a rotary pair sit in the same lane (no exchange), the RMS
// reduction is a log2(D/16)-step butterfly and every access is 16 bytes.
// Consecutive units are consecutive head rows, so a wave reads 2 KiB contiguous.
#include "nkv_common.h"

namespace nkv {

constexpr int kRopeThreads = 256;
constexpr bool rope_dim_ok(int D) { return D == 64 || D == 128 || D == 256; }
// units per block: one per group of D/16 lanes
constexpr int rope_units_per_block(int D) { return kRopeThreads / (D / 16); }

// One 16-bit element (low bits of b16) -> fp32, and fp32 rounded to the element type and
// back (round to nearest even): bf16, or fp16 with H16.
template <bool H16>
__device__ __forceinline__ float el(uint32_t b16) {
  if constexpr (H16) return (float)__builtin_bit_cast(_Float16, (uint16_t)b16);
  else return __uint_as_float(b16 << 16);
}
template <bool H16>
__device__ __forceinline__ float round_el(float f) {
  if constexpr (H16) return (float)(_Float16)f;
  else return el<false>(f32_to_bf16_bits(f));
}
template <bool H16>
__device__ __forceinline__ uint32_t pack_el(float lo, float hi) {
  if constexpr (H16) return cvt_pk16<true>(lo, hi);
  else return pack_bf16x2(lo, hi);
}

struct RopeArgs {
  const bf16_t* q_in;
  int64_t q_row_stride;
  const bf16_t* k_in;
  int64_t k_row_stride;
  const bf16_t* v_in;
  int64_t v_row_stride;
  const int64_t* positions;
  const bf16_t* q_weight;
  const bf16_t* k_weight;
  float eps;
  const float* cos_sin;
  int64_t max_position;
  bf16_t* q_out;
  int64_t q_out_row_stride;
  bf16_t* k_cache;
  bf16_t* v_cache;
  const int32_t* slot_mapping;
  int64_t n_slots;
  bf16_t* k_out;
  uint32_t n_units;
  uint32_t units_per_token;
  int32_t Hq;
  int32_t Hk;
};

// Units per token: Hq q heads, Hk k heads, then (when storing) Hk v heads. A
// group of D/16 lanes owns one unit; lane i holds elements [8i, 8i+8) and
// [D/2+8i, D/2+8i+8) of the head (16-byte accesses). The head row, the position
// and the slot are loaded together; the cos|sin row (which needs the position)
// is the only dependent load. One unit per group measured fastest at every size
// (more units per group serialise their dependent loads). Loads and stores are
// non-temporal: every byte is touched once (4-5% faster than cached stores).
template <int D, bool H16 = false>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_store_kernel(const RopeArgs a) {
  // Every product is rounded on its own, as the reference's separate torch ops are:
  // no a*b - c*d -> fma contraction.
#pragma clang fp contract(off)
  static_assert(rope_dim_ok(D), "head_dim 64, 128 or 256");
  constexpr int kL = D / 16;   // lanes per unit
  constexpr int kH = D / 2;    // offset of the rotary partners
  const uint32_t u = blockIdx.x * rope_units_per_block(D) + threadIdx.x / kL;
  if (u >= a.n_units) return;
  const int l8 = threadIdx.x % kL;
  const uint32_t t = u / a.units_per_token;
  const int h = (int)(u - t * a.units_per_token);
  const bool is_q = h < a.Hq;
  const bool is_k = !is_q && h < a.Hq + a.Hk;
  const int kvh = is_q ? 0 : (is_k ? h - a.Hq : h - a.Hq - a.Hk);
  const bf16_t* src = is_q ? a.q_in + (int64_t)t * a.q_row_stride + (int64_t)h * D
                      : is_k ? a.k_in + (int64_t)t * a.k_row_stride + (int64_t)kvh * D
                             : a.v_in + (int64_t)t * a.v_row_stride + (int64_t)kvh * D;
  u32x4_t vlo = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src + 8 * l8));
  u32x4_t vhi = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src + kH + 8 * l8));
  const int64_t sl = (!is_q && a.k_cache) ? (int64_t)a.slot_mapping[t] : -1;
  if (is_q || is_k) {  // uniform over the unit's 8 lanes
    int64_t pos = a.positions[t];
    NKV_DBG(pos < 0 || pos >= a.max_position, NKV_DEBUG_POSITION);
    pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);
    const float* cs = a.cos_sin + pos * D + 8 * l8;
    const f32x4_t c0 = *reinterpret_cast<const f32x4_t*>(cs);
    const f32x4_t c1 = *reinterpret_cast<const f32x4_t*>(cs + 4);
    const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(cs + kH);
    const f32x4_t s1 = *reinterpret_cast<const f32x4_t*>(cs + kH + 4);
    float x[16];  // x[0..7] first half, x[8..15] the rotary partners
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = el<H16>(vlo[e] & 0xffffu);
      x[2 * e + 1] = el<H16>(vlo[e] >> 16);
      x[8 + 2 * e] = el<H16>(vhi[e] & 0xffffu);
      x[9 + 2 * e] = el<H16>(vhi[e] >> 16);
    }
    if (a.q_weight) {
      const bf16_t* w = is_q ? a.q_weight : a.k_weight;
      const u32x4_t wlo = *reinterpret_cast<const u32x4_t*>(w + 8 * l8);
      const u32x4_t whi = *reinterpret_cast<const u32x4_t*>(w + kH + 8 * l8);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) ss += x[e] * x[e];
#pragma unroll
      for (int o = 1; o < kL; o <<= 1) ss += __shfl_xor(ss, o, 64);
      const float r = rsqrtf(ss * (1.0f / D) + a.eps);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = round_el<H16>(round_el<H16>(x[2 * e] * r) * el<H16>(wlo[e] & 0xffffu));
        x[2 * e + 1] = round_el<H16>(round_el<H16>(x[2 * e + 1] * r) * el<H16>(wlo[e] >> 16));
        x[8 + 2 * e] = round_el<H16>(round_el<H16>(x[8 + 2 * e] * r) * el<H16>(whi[e] & 0xffffu));
        x[9 + 2 * e] = round_el<H16>(round_el<H16>(x[9 + 2 * e] * r) * el<H16>(whi[e] >> 16));
      }
    }
    const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    float y[16];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x1 = x[e], x2 = x[8 + e];
      y[e] = x1 * cv[e] - x2 * sv[e];
      y[8 + e] = x2 * cv[e] + x1 * sv[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vlo[e] = pack_el<H16>(y[2 * e], y[2 * e + 1]);
      vhi[e] = pack_el<H16>(y[8 + 2 * e], y[9 + 2 * e]);
    }
  }
  if (is_q) {
    bf16_t* dst = a.q_out + (int64_t)t * a.q_out_row_stride + (int64_t)h * D;
    __builtin_nontemporal_store(vlo, reinterpret_cast<u32x4_t*>(dst + 8 * l8));
    __builtin_nontemporal_store(vhi, reinterpret_cast<u32x4_t*>(dst + kH + 8 * l8));
    return;
  }
  NKV_DBG(sl < -1 || sl >= a.n_slots, NKV_DEBUG_SLOT);
  if (sl >= 0 && sl < a.n_slots) {  // -1 (padding) or out of range: skipped
    bf16_t* dst = (is_k ? a.k_cache : a.v_cache) + (sl * a.Hk + kvh) * (int64_t)D;
    __builtin_nontemporal_store(vlo, reinterpret_cast<u32x4_t*>(dst + 8 * l8));
    __builtin_nontemporal_store(vhi, reinterpret_cast<u32x4_t*>(dst + kH + 8 * l8));
  }
  if (is_k && a.k_out) {
    bf16_t* dst = a.k_out + ((int64_t)t * a.Hk + kvh) * D;
    __builtin_nontemporal_store(vlo, reinterpret_cast<u32x4_t*>(dst + 8 * l8));
    __builtin_nontemporal_store(vhi, reinterpret_cast<u32x4_t*>(dst + kH + 8 * l8));
  }
}

}  // namespace nkv

namespace nkv {
template <bool H16>
static int qk_norm_rope_store_impl(const void* q, int64_t q_row_stride, const void* k,
                                   int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                   const int64_t* positions, const void* q_norm_weight,
                                   const void* k_norm_weight, float eps,
                                   const float* cos_sin_cache, int64_t max_position,
                                   void* q_out, int64_t q_out_row_stride, void* k_out,
                                   void* k_cache, void* v_cache, const int32_t* slot_mapping,
                                   int64_t n_slots, int64_t n_tokens, int32_t n_q_heads,
                                   int32_t n_kv_heads, int32_t head_dim, void* stream) {
  NKV_REQUIRE(n_tokens >= 0 && n_q_heads > 0 && n_kv_heads > 0 && n_slots >= 0, NKV_EINVAL,
              "qk_norm_rope_store: bad sizes");
  if (n_tokens == 0) return NKV_OK;
  NKV_REQUIRE(rope_dim_ok(head_dim), NKV_EUNSUPPORTED,
              "qk_norm_rope_store: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  NKV_REQUIRE(q && k && positions && cos_sin_cache && q_out && max_position > 0, NKV_EINVAL,
              "qk_norm_rope_store: null pointer or empty rotary cache");
  NKV_REQUIRE(!q_norm_weight == !k_norm_weight, NKV_EINVAL,
              "qk_norm_rope_store: give both norm weights or neither");
  NKV_REQUIRE(!k_cache == !v_cache && (!k_cache || (slot_mapping && v)), NKV_EINVAL,
              "qk_norm_rope_store: k_cache, v_cache, v and slot_mapping go together");
  NKV_REQUIRE(k_cache || k_out, NKV_EINVAL,
              "qk_norm_rope_store: nowhere to put K (no cache and no k_out)");
  const int64_t per_tok = (int64_t)n_q_heads + n_kv_heads + (k_cache ? n_kv_heads : 0);
  const int64_t qw = (int64_t)n_q_heads * head_dim, kw = (int64_t)n_kv_heads * head_dim;
  NKV_REQUIRE(q_row_stride >= qw && q_out_row_stride >= qw && k_row_stride >= kw &&
                  (!k_cache || v_row_stride >= kw) &&
                  ((q_row_stride | q_out_row_stride | k_row_stride | v_row_stride) % 8) == 0,
              NKV_EINVAL, "qk_norm_rope_store: row strides must cover the heads, multiples of 8");
  NKV_REQUIRE(n_tokens * per_tok < (int64_t)1 << 31, NKV_EINVAL,
              "qk_norm_rope_store: tokens x heads must stay below 2^31");
  NKV_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_out) &&
                  aligned16(cos_sin_cache) && aligned16(k_out) && aligned16(k_cache) &&
                  aligned16(v_cache) && aligned16(q_norm_weight) && aligned16(k_norm_weight),
              NKV_EINVAL, "qk_norm_rope_store: pointers must be 16-byte aligned");
  const uint32_t n_units = (uint32_t)(n_tokens * per_tok);
  const uint32_t upb = (uint32_t)rope_units_per_block(head_dim);
  const unsigned grid = (unsigned)((n_units + upb - 1) / upb);
  RopeArgs a;
  a.q_in = (const bf16_t*)q;
  a.q_row_stride = q_row_stride;
  a.k_in = (const bf16_t*)k;
  a.k_row_stride = k_row_stride;
  a.v_in = (const bf16_t*)v;
  a.v_row_stride = v_row_stride;
  a.positions = positions;
  a.q_weight = (const bf16_t*)q_norm_weight;
  a.k_weight = (const bf16_t*)k_norm_weight;
  a.eps = eps;
  a.cos_sin = cos_sin_cache;
  a.max_position = max_position;
  a.q_out = (bf16_t*)q_out;
  a.q_out_row_stride = q_out_row_stride;
  a.k_cache = (bf16_t*)k_cache;
  a.v_cache = (bf16_t*)v_cache;
  a.slot_mapping = slot_mapping;
  a.n_slots = k_cache ? n_slots : 0;
  a.k_out = (bf16_t*)k_out;
  a.n_units = n_units;
  a.units_per_token = (uint32_t)per_tok;
  a.Hq = n_q_heads;
  a.Hk = n_kv_heads;
  if (head_dim == 64)
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<64, H16>), dim3(grid), dim3(kRopeThreads), 0,
                       as_stream(stream), a);
  else if (head_dim == 128)
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<128, H16>), dim3(grid), dim3(kRopeThreads), 0,
                       as_stream(stream), a);
  else
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<256, H16>), dim3(grid), dim3(kRopeThreads), 0,
                       as_stream(stream), a);
  return check_launch(H16 ? "nkv_qk_norm_rope_store_f16" : "nkv_qk_norm_rope_store");
}
}  // namespace nkv

extern "C" int nkv_qk_norm_rope_store(const void* q, int64_t q_row_stride, const void* k,
                                      int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                      const int64_t* positions, const void* q_norm_weight,
                                      const void* k_norm_weight, float eps,
                                      const float* cos_sin_cache, int64_t max_position,
                                      void* q_out, int64_t q_out_row_stride, void* k_out,
                                      void* k_cache, void* v_cache, const int32_t* slot_mapping,
                                      int64_t n_slots, int64_t n_tokens, int32_t n_q_heads,
                                      int32_t n_kv_heads, int32_t head_dim, void* stream) {
  nkv::clear_error();
  return nkv::qk_norm_rope_store_impl<false>(
      q, q_row_stride, k, k_row_stride, v, v_row_stride, positions, q_norm_weight,
      k_norm_weight, eps, cos_sin_cache, max_position, q_out, q_out_row_stride, k_out, k_cache,
      v_cache, slot_mapping, n_slots, n_tokens, n_q_heads, n_kv_heads, head_dim, stream);
}

extern "C" int nkv_qk_norm_rope_store_f16(const void* q, int64_t q_row_stride, const void* k,
                                          int64_t k_row_stride, const void* v,
                                          int64_t v_row_stride, const int64_t* positions,
                                          const void* q_norm_weight, const void* k_norm_weight,
                                          float eps, const float* cos_sin_cache,
                                          int64_t max_position, void* q_out,
                                          int64_t q_out_row_stride, void* k_out, void* k_cache,
                                          void* v_cache, const int32_t* slot_mapping,
                                          int64_t n_slots, int64_t n_tokens, int32_t n_q_heads,
                                          int32_t n_kv_heads, int32_t head_dim, void* stream) {
  nkv::clear_error();
  return nkv::qk_norm_rope_store_impl<true>(
      q, q_row_stride, k, k_row_stride, v, v_row_stride, positions, q_norm_weight,
      k_norm_weight, eps, cos_sin_cache, max_position, q_out, q_out_row_stride, k_out, k_cache,
      v_cache, slot_mapping, n_slots, n_tokens, n_q_heads, n_kv_heads, head_dim, stream);
}

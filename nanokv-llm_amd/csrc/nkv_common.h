// Shared device/host helpers for the gfx950 kernels of libnkv_amd.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/nkv.h"

namespace nkv {

// ---------------------------------------------------------------- errors
// Thread-local last-error text; every entry point returns NKV_OK or a code.
void set_error(const char* fmt, ...);
void clear_error();

#define NKV_REQUIRE(cond, code, ...)       \
  do {                                     \
    if (!(cond)) {                         \
      ::nkv::set_error(__VA_ARGS__);       \
      return (code);                       \
    }                                      \
  } while (0)

// Checks the launch just issued on the current thread.
int check_launch(const char* what);

// Input checks of the debug build (-DNKV_DEBUG, libnkv_amd_debug.so): NKV_DBG(cond, bit)
// ORs an NKV_DEBUG_* bit into this source file's device word when cond holds, and each
// source file registers a reader of its word with nkv_debug_flags. Without NKV_DEBUG the
// checks compile to nothing.
bool debug_register(int (*take)(uint32_t* bits, int clear));

// ---------------------------------------------------------------- types
typedef uint16_t bf16_t;  // raw bf16 bits in memory
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));  // 16-byte payload

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, v);
}
__device__ __forceinline__ bf16x8_t as_bf16x8_v(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// ---------------------------------------------------------------- 16-bit element types
// q, K, V and outputs are bf16 or fp16 (the model's dtype); a kernel instance takes one of
// them as the template flag H16 (true: fp16) and the helpers below pick the matching
// conversion or MFMA. The bits travel as raw uint16 either way.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// 16-bit value in the low / high half of a word -> fp32 (exact)
template <bool H16>
__device__ __forceinline__ float e16_lo(uint32_t w) {
  if constexpr (H16) return (float)__builtin_bit_cast(f16x2_t, w)[0];
  else return bf16_lo(w);
}
template <bool H16>
__device__ __forceinline__ float e16_hi(uint32_t w) {
  if constexpr (H16) return (float)__builtin_bit_cast(f16x2_t, w)[1];
  else return bf16_hi(w);
}

// fp32 pair -> packed pair (lo in bits 0-15), round to nearest even: the hardware
// conversions (v_cvt_f16_f32; for bf16 the packed bf16 conversion)
template <bool H16>
__device__ __forceinline__ uint32_t cvt_pk16(float lo, float hi) {
  if constexpr (H16) {
    const f16x2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// v_mfma_f32_16x16x32_{bf16,f16}: 8 elements of A and B per lane (raw bits)
template <bool H16>
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (H16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                   __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                    __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// v_mfma_f32_16x16x16_{bf16,f16}: 4 elements of A and B per lane (raw bits)
template <bool H16>
__device__ __forceinline__ f32x4_t mfma_16x16x16(s16x4_t a, s16x4_t b, f32x4_t c) {
  if constexpr (H16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                  __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// acc + lo + hi of a packed pair (v_dot2_f32_{bf16,f16} against (1, 1))
template <bool H16>
__device__ __forceinline__ float sum2_16(uint32_t pair, float acc) {
  if constexpr (H16) {
    const f16x2_t ones = {(_Float16)1.f, (_Float16)1.f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), ones, acc, false);
  } else {
    const bf16x2_t ones = {(__bf16)1.f, (__bf16)1.f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), ones, acc, false);
  }
}

// 64-lane wavefront reductions (butterfly over the whole wave).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// max(a, b, c) as one v_maximum3_f32 (no operand canonicalisation; NaN-propagating)
__device__ __forceinline__ float fmax3(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Max over the four 16-lane rows of a wave for each column (lane % 16), without
// LDS: v_permlane16_swap pairs rows 0/1 and 2/3, v_permlane32_swap pairs the
// two halves; each swap leaves both values of a pair in (r[0], r[1]).
__device__ __forceinline__ float col_max4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_sum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------- fp8 KV (OCP E4M3FN)
// gfx950's v_cvt_pk_f32_fp8 / v_cvt_pk_fp8_f32 convert between fp32 and the OCP
// E4M3FN format (bias 7, largest finite 448, NaN = S.1111.111), round to
// nearest even. An E4M3FN value has at most 4 significant bits and an
// exponent in [-9, 8], so it is exact in bf16, and v_cvt_scalef32_pk_bf16_fp8
// (scale 1) produces it directly.
constexpr float kFp8Max = 448.f;

// 16 codes (one 16-byte word) -> 16 bf16 (two 16-byte words), exact.
__device__ __forceinline__ void fp8x16_to_bf16(u32x4_t in, u32x4_t& lo, u32x4_t& hi) {
  // v_cvt_scalef32_pk_bf16_fp8 with scale 1: two codes to a packed bf16 pair, exact
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const bf16x2v a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(in[w], 1.0f, false);  // bytes 0, 1
    const bf16x2v b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(in[w], 1.0f, true);   // bytes 2, 3
    const uint32_t p0 = __builtin_bit_cast(uint32_t, a);
    const uint32_t p1 = __builtin_bit_cast(uint32_t, b);
    if (w < 2) {
      lo[2 * w] = p0;
      lo[2 * w + 1] = p1;
    } else {
      hi[2 * (w - 2)] = p0;
      hi[2 * (w - 2) + 1] = p1;
    }
  }
}

// x -> E4M3FN after clamping to +-448 (NaN stays NaN), round to nearest even.
__device__ __forceinline__ float fp8_clamp(float x) {
  return __builtin_isnan(x) ? x : fminf(fmaxf(x, -kFp8Max), kFp8Max);
}
__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float x0, float x1, float x2, float x3) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(x0), fp8_clamp(x1), 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(x2), fp8_clamp(x3), r, true);
  return (uint32_t)r;
}

}  // namespace nkv

#ifdef NKV_DEBUG
namespace nkv {
// This source file's debug word (one per device) and its reader.
static __device__ unsigned int g_debug_bits;
static int debug_take(uint32_t* bits, int clear) {
  unsigned int v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_debug_bits), sizeof(v), 0,
                          hipMemcpyDeviceToHost) != hipSuccess)
    return NKV_ELAUNCH;
  if (clear && v) {
    const unsigned int zero = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_debug_bits), &zero, sizeof(zero), 0,
                          hipMemcpyHostToDevice) != hipSuccess)
      return NKV_ELAUNCH;
  }
  *bits |= v;
  return NKV_OK;
}
[[maybe_unused]] static const bool g_debug_registered = debug_register(&debug_take);
}  // namespace nkv
#define NKV_DBG(cond, bit)                                                   \
  do {                                                                       \
    if (cond) atomicOr(&::nkv::g_debug_bits, (unsigned int)(bit));           \
  } while (0)
#else
#define NKV_DBG(cond, bit) \
  do {                     \
  } while (0)
#endif

// hq_device.hpp — gfx950 device helpers: MFMA fragments and in-register dequantisation.
//
// Fragment convention for v_mfma_f32_16x16x32_{f16,bf16} (wave64): lane l holds
// 8 consecutive-k elements of row (A) or column (B) l % 16, k-slice l / 16; the
// 16x16 fp32 result has column l % 16 and rows 4 * (l / 16) + v, v = 0..3.
// Fragments travel as u4 (four 32-bit words = eight 16-bit elements).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hq_layout.hpp"
#include "hq_qgemm.h"

namespace hq {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ f4 mfma16x16x32(u4 a, u4 b, f4 c) {
  if constexpr (DT == HQ_DTYPE_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b),
                                                  c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, a), __builtin_bit_cast(b8, b),
                                                   c, 0, 0, 0);
  }
}

__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 bits_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// int4 word (tile nibble order) -> exact fp16 (q - 8) fragment.
// (q | 0x6400) is the fp16 1024 + q; (16q | 0x6400) is 1024 + 16q. Subtracting 1032, or
// scaling by 1/16 and subtracting 72, leaves q - 8 exactly.
__device__ __forceinline__ u4 dq_int4_f16(uint32_t w) {
  const h2 c1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 c72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t hi = w >> 8;
  h2 v0 = bits_h2((w & 0x000F000Fu) | 0x64006400u) + c1032;
  h2 v1 = __builtin_elementwise_fma(bits_h2((w & 0x00F000F0u) | 0x64006400u), s16, c72);
  h2 v2 = bits_h2((hi & 0x000F000Fu) | 0x64006400u) + c1032;
  h2 v3 = __builtin_elementwise_fma(bits_h2((hi & 0x00F000F0u) | 0x64006400u), s16, c72);
  return u4{h2_bits(v0), h2_bits(v1), h2_bits(v2), h2_bits(v3)};
}

// int4 word -> bf16 fragment of (16 + q) / 16 = 0x3F80 | q << 3 (exact). gfx950 has no
// packed bf16 add, so the offset is removed after the MFMA: the caller accumulates
// -1.5 * sum(x) over the same k range and the group sum is 16 * (acc + corr).
__device__ __forceinline__ u4 dq_int4_bf16_biased(uint32_t w) {
  return u4{((w << 3) & 0x00780078u) | 0x3F803F80u, ((w >> 1) & 0x00780078u) | 0x3F803F80u,
            ((w >> 5) & 0x00780078u) | 0x3F803F80u, ((w >> 9) & 0x00780078u) | 0x3F803F80u};
}

// Ternary word -> fragment of chunk CW (0 or 1): elements 2t in fp16 and in bf16
// (the 2-bit field is the sign bit and the top exponent bit of +-2.0).
template <int CW>
__device__ __forceinline__ u4 dq_tern2(uint32_t w) {
  return u4{(w << (8 * CW + 0)) & 0xC000C000u, (w << (8 * CW + 2)) & 0xC000C000u,
            (w << (8 * CW + 4)) & 0xC000C000u, (w << (8 * CW + 6)) & 0xC000C000u};
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__device__ __forceinline__ uint16_t f32_to_out(float v) {
  if constexpr (DT == HQ_DTYPE_F16) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  } else {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
  }
}

}  // namespace hq

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

// Raw buffer resource (gfx9 family descriptor word 3 = 0x00020000). Loads past
// num_records return zero without touching memory, which lets every load in a
// pipelined loop be unconditional (no branches, so s_waitcnt stays exact).
constexpr int kBufferFlags = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;  // a voffset past any descriptor used here
// Cache policy of the decode weight stream: non-temporal (each byte is read once).
constexpr int kStreamAux = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferFlags);
}

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ... lds): lane i
// writes lds + 16 * i; lds must be wave-uniform. Kept out of kernel templates: clang's host
// pass rejects this builtin and would otherwise silently drop the kernel's host stub.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
// The range check covers voff; keep soff (wave-uniform) in range.
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt <= n only (n < 64).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00; }

__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 bits_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// Registers the compiler cannot see through. gfx9 VOP3 instructions take no literal
// constants and read at most one SGPR, so (w & mask) | magic only becomes a single
// v_and_or_b32 when the mask sits in an SGPR and the magic in a VGPR.
__device__ __forceinline__ uint32_t opaque_sgpr(uint32_t v) {
  uint32_t r;
  asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
  return r;
}
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
  return r;
}

// Constants of the int4 dequantisation, materialised once per kernel.
struct DqConst {
  uint32_t lo, hi, magic;  // nibble masks (SGPR) and exponent magic (VGPR)
};
__device__ __forceinline__ DqConst dq_const_f16() {
  return {opaque_sgpr(0x000F000Fu), opaque_sgpr(0x00F000F0u), opaque_vgpr(0x64006400u)};
}
__device__ __forceinline__ DqConst dq_const_bf16() {
  return {opaque_sgpr(0x00780078u), 0u, opaque_vgpr(0x3F803F80u)};
}

// int4 word (tile nibble order) -> exact fp16 (q - 8) fragment.
// (q | 0x6400) is the fp16 1024 + q; (16q | 0x6400) is 1024 + 16q. Subtracting 1032, or
// scaling by 1/16 and subtracting 72, leaves q - 8 exactly.
__device__ __forceinline__ u4 dq_int4_f16(uint32_t w, const DqConst& k) {
  const h2 c1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 c72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t hi = w >> 8;
  h2 v0 = bits_h2((w & k.lo) | k.magic) + c1032;
  h2 v1 = __builtin_elementwise_fma(bits_h2((w & k.hi) | k.magic), s16, c72);
  h2 v2 = bits_h2((hi & k.lo) | k.magic) + c1032;
  h2 v3 = __builtin_elementwise_fma(bits_h2((hi & k.hi) | k.magic), s16, c72);
  return u4{h2_bits(v0), h2_bits(v1), h2_bits(v2), h2_bits(v3)};
}

// int4 word -> bf16 fragment of (16 + q) / 16 = 0x3F80 | q << 3 (exact). gfx950 has no
// packed bf16 add, so the offset is removed after the MFMA: the caller accumulates
// -1.5 * sum(x) over the same k range and the group sum is 16 * (acc + corr).
__device__ __forceinline__ u4 dq_int4_bf16_biased(uint32_t w, const DqConst& k) {
  return u4{((w << 3) & k.lo) | k.magic, ((w >> 1) & k.lo) | k.magic, ((w >> 5) & k.lo) | k.magic,
            ((w >> 9) & k.lo) | k.magic};
}

// Biased int4 dequantisation (decode path): each nibble q is OR-ed into the mantissa of a
// power of two chosen so that its unit in the last place is 1, giving the exact value
// magic + q with one v_and_or_b32 per 32-bit word of the fragment:
//   fp16: nibble at bits 0..3 -> 1024 + q (0x6400), bits 4..7 -> 64 + q (0x5400);
//   bf16: nibble at bits 0..3 -> 128 + q (0x4300), bits 3..6 -> 16 + q (0x4180).
// The bias magic + 8 is removed after the MFMA: the caller seeds each tile's accumulator
// with MFMA(x, kInt4Corr*), i.e. -sum_k x_k (magic_k + 8) over the same chunk, so the
// result is sum_k x_k (q_k - 8) with exact products and fp32 accumulation.
struct DqBiasConst {
  uint32_t m_lo, m_hi;  // nibble masks (SGPR)
  uint32_t v_lo, v_hi;  // magics (VGPR)
};
__device__ __forceinline__ DqBiasConst dq_bias_const_f16() {
  return {opaque_sgpr(0x000F000Fu), opaque_sgpr(0x00F000F0u), opaque_vgpr(0x64006400u), opaque_vgpr(0x54005400u)};
}
__device__ __forceinline__ DqBiasConst dq_bias_const_bf16() {
  return {opaque_sgpr(0x000F000Fu), opaque_sgpr(0x00780078u), opaque_vgpr(0x43004300u), opaque_vgpr(0x41804180u)};
}
// Correction fragments (every chunk alike): -(1024 + 8), -(64 + 8) in fp16; -(128 + 8),
// -(16 + 8) in bf16, matching the magic of each fragment word.
constexpr uint32_t kInt4CorrF16Lo = 0xE408E408u, kInt4CorrF16Hi = 0xD480D480u;
constexpr uint32_t kInt4CorrBf16Lo = 0xC308C308u, kInt4CorrBf16Hi = 0xC1C0C1C0u;

template <int DT>
__device__ __forceinline__ u4 int4_corr_fragment() {
  if constexpr (DT == HQ_DTYPE_F16) return u4{kInt4CorrF16Lo, kInt4CorrF16Hi, kInt4CorrF16Lo, kInt4CorrF16Hi};
  else return u4{kInt4CorrBf16Lo, kInt4CorrBf16Hi, kInt4CorrBf16Lo, kInt4CorrBf16Hi};
}

// int4 word (tile nibble order: elements (0,1) at nibbles (0,4), (2,3) at (1,5), (4,5) at
// (2,6), (6,7) at (3,7)) -> biased fragment.
template <int DT>
__device__ __forceinline__ u4 dq_int4_biased(uint32_t w, const DqBiasConst& k) {
  if constexpr (DT == HQ_DTYPE_F16) {
    const uint32_t h = w >> 8;
    return u4{(w & k.m_lo) | k.v_lo, (w & k.m_hi) | k.v_hi, (h & k.m_lo) | k.v_lo, (h & k.m_hi) | k.v_hi};
  } else {
    return u4{(w & k.m_lo) | k.v_lo, ((w >> 1) & k.m_hi) | k.v_hi, ((w >> 8) & k.m_lo) | k.v_lo,
              ((w >> 9) & k.m_hi) | k.v_hi};
  }
}

// Ternary word -> fragment of chunk CW (0 or 1): elements 2t in fp16 and in bf16
// (the 2-bit field is the sign bit and the top exponent bit of +-2.0).
template <int CW>
__device__ __forceinline__ u4 dq_tern2(uint32_t w) {
  return u4{(w << (8 * CW + 0)) & 0xC000C000u, (w << (8 * CW + 2)) & 0xC000C000u,
            (w << (8 * CW + 4)) & 0xC000C000u, (w << (8 * CW + 6)) & 0xC000C000u};
}

// 64-bit left shift of a register pair by S in one instruction. Written as asm because the
// compiler splits a 64-bit shift whose high word is only partly used into two 32-bit ones.
template <int S>
__device__ __forceinline__ uint64_t shl64(uint64_t v) {
  if constexpr (S == 0) {
    return v;
  } else {
    uint64_t x;
    asm("v_lshlrev_b64 %0, %1, %2" : "=v"(x) : "I"(S), "v"(v));
    return x;
  }
}

// A lane's two ternary words (w0: chunks 0, 1; w1: chunks 2, 3) -> fragments H and 2 + H
// (H = 0 or 1), the same values as dq_tern2. One 64-bit shift serves both words: the bits
// w0 shifts into the high word land below bit 14 and the mask drops them (12 instead of 16
// VALU per two fragments; ternary decode 4-5% faster on MI355X).
template <int H>
__device__ __forceinline__ void dq_tern2_pair(uint64_t v, u4& f0, u4& f1) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint64_t x;
    if (e == 0) x = shl64<8 * H>(v);
    else if (e == 1) x = shl64<8 * H + 2>(v);
    else if (e == 2) x = shl64<8 * H + 4>(v);
    else x = shl64<8 * H + 6>(v);
    f0[e] = (uint32_t)x & 0xC000C000u;
    f1[e] = (uint32_t)(x >> 32) & 0xC000C000u;
  }
}

__device__ __forceinline__ uint64_t tern2_words(uint32_t w0, uint32_t w1) {
  return ((uint64_t)w1 << 32) | w0;
}

// All four fragments of a lane's two ternary words.
__device__ __forceinline__ void dq_tern2_all(uint32_t w0, uint32_t w1, u4 (&f)[4]) {
  const uint64_t v = tern2_words(w0, w1);
  dq_tern2_pair<0>(v, f[0], f[2]);
  dq_tern2_pair<1>(v, f[1], f[3]);
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

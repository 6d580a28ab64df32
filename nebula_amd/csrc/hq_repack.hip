// hq_repack.hip — device repack of linear int4 / ternary weights into the gfx950 tile
// layout (hq_layout.hpp). One thread per packed output word; the host variants in
// hq_api.cpp (hq_repack_int4, hq_repack_ternary2, hq_convert_tq1_0) produce the same words.
#include <hip/hip_runtime.h>

#include "hq_internal.hpp"
#include "hq_layout.hpp"

namespace hq {
namespace {

__global__ void __launch_bounds__(256) repack_int4_kernel(const uint32_t* __restrict__ src,
                                                          uint32_t* __restrict__ dst, uint32_t N,
                                                          uint32_t nkb, size_t total) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint32_t w = (uint32_t)(idx & 3u);
  const uint32_t lane = (uint32_t)((idx >> 2) & 63u);
  const size_t blk = idx >> 8;
  const uint32_t kb = (uint32_t)(blk % nkb);
  const uint32_t ct = (uint32_t)(blk / nkb);
  const uint32_t n = ct * 16u + (lane & 15u);
  const uint32_t lin = n < N ? src[(size_t)int4_linear_kw(kb, lane, w) * N + n] : 0x88888888u;
  dst[idx] = int4_linear_to_tile(lin);
}

__global__ void __launch_bounds__(256) repack_tern_kernel(const uint32_t* __restrict__ src,
                                                          uint32_t* __restrict__ dst, uint32_t N,
                                                          uint32_t nkb, size_t total,
                                                          uint32_t* __restrict__ bad_flag) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint32_t w = (uint32_t)(idx & 1u);
  const uint32_t lane = (uint32_t)((idx >> 1) & 63u);
  const size_t blk = idx >> 7;
  const uint32_t kb = (uint32_t)(blk % nkb);
  const uint32_t ct = (uint32_t)(blk / nkb);
  const uint32_t n = ct * 16u + (lane & 15u);
  const uint32_t g4 = lane >> 4;
  bool bad = false;
  uint32_t out = 0;
  if (n < N) {
    const size_t kw0 = (size_t)8u * kb + 4u * w + (g4 >> 1);
    out = tern_pack_word(src[kw0 * N + n], src[(kw0 + 2u) * N + n], g4 & 1u, &bad);
  }
  dst[idx] = out;
  if (bad && bad_flag) *bad_flag = 1u;
}

// GGUF TQ1_0 blocks straight into the ternary tile layout: one thread per (column n, block b),
// consecutive threads on consecutive columns (so the tile-layout stores of a column tile are
// contiguous). A thread reads its 56-byte block with seven 8-byte loads, expands the 52 trit
// bytes through a 256-entry table (byte -> the (sign, nonzero) fields of its five digits, 10
// bits) into the block's 256 fields in element order, then writes the 16 packed words of
// column n in k-blocks 2b and 2b + 1, and the block's d as the scale of group b. Columns
// past N up to the next multiple of 16 write zero words (padding decodes to zero).
__global__ void __launch_bounds__(256) repack_tq1_0_kernel(const uint8_t* __restrict__ blocks,
                                                           uint32_t* __restrict__ dst,
                                                           uint16_t* __restrict__ scales, uint32_t N,
                                                           uint32_t N16, uint32_t nb, size_t total) {
  __shared__ uint32_t tab[256];
  {
    uint32_t v = threadIdx.x, f = 0;
#pragma unroll
    for (uint32_t d = 0; d < 5; ++d) {
      f |= tern_c_to_field(v % 3u) << (2u * d);
      v /= 3u;
    }
    tab[threadIdx.x] = f;
  }
  __syncthreads();
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint32_t n = (uint32_t)(idx % N16);
  const uint32_t b = (uint32_t)(idx / N16);
  // F: the fields of elements 0..255, element i at bits 2 (i % 16) of F[i / 16].
  uint32_t F[16];
#pragma unroll
  for (int w = 0; w < 16; ++w) F[w] = 0u;
  if (n < N) {
    const uint64_t* p = reinterpret_cast<const uint64_t*>(blocks + ((size_t)n * nb + b) * kTq1Bytes);
    uint64_t q[7];
#pragma unroll
    for (int i = 0; i < 7; ++i) q[i] = p[i];
    auto byte_at = [&](uint32_t o) { return (uint32_t)(q[o / 8u] >> (8u * (o % 8u))) & 0xFFu; };
    scales[(size_t)b * N + n] = (uint16_t)(q[0] & 0xFFFFu);
#pragma unroll
    for (uint32_t j = 0; j < 52; ++j) {
      // Trit byte j holds elements 5 j .. 5 j + 4 (j < 50) or 250 + 3 (j - 50) .. + 2.
      const uint32_t t = tab[byte_at(2u + j)] & (j < 50u ? 0x3FFu : 0x3Fu);
      const uint32_t bit = j < 50u ? 10u * j : 500u + 6u * (j - 50u);
      F[bit / 32u] |= t << (bit % 32u);
      if (bit % 32u > 22u && bit / 32u < 15u) F[bit / 32u + 1u] |= t >> (32u - bit % 32u);
    }
  }
  const uint32_t ct = n / 16u, nkb = 2u * nb;
#pragma unroll
  for (uint32_t h = 0; h < 2; ++h)      // k-block 2 b + h
#pragma unroll
    for (uint32_t g4 = 0; g4 < 4; ++g4)
#pragma unroll
      for (uint32_t w = 0; w < 2; ++w) {
        uint32_t out = 0;
#pragma unroll
        for (uint32_t cw = 0; cw < 2; ++cw) {
          const uint32_t i0 = 128u * h + 32u * (2u * w + cw) + 8u * g4;  // first of 8 elements
          const uint32_t run = F[i0 / 16u] >> (2u * (i0 % 16u));
#pragma unroll
          for (uint32_t e = 0; e < 8; ++e) out |= ((run >> (2u * e)) & 3u) << tern_field_bit(cw, e);
        }
        const uint32_t lane = 16u * g4 + (n % 16u);
        dst[(((size_t)ct * nkb + 2u * b + h) * 64u + lane) * 2u + w] = out;
      }
}

}  // namespace

hipError_t launch_repack_tq1_0(const uint8_t* blocks, uint32_t* dst, uint16_t* scales, uint32_t K, uint32_t N,
                               hipStream_t stream) {
  const uint32_t nb = K / kTq1K, N16 = col_tiles(N) * 16u;
  const size_t total = (size_t)N16 * nb;
  const size_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(repack_tq1_0_kernel, dim3((uint32_t)grid), dim3(256), 0, stream, blocks, dst, scales, N, N16,
                     nb, total);
  return hipGetLastError();
}

hipError_t launch_repack_int4(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N,
                              hipStream_t stream) {
  const uint32_t nkb = K / kBlockK;
  const size_t total = (size_t)col_tiles(N) * nkb * 64u * 4u;
  const size_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(repack_int4_kernel, dim3((uint32_t)grid), dim3(256), 0, stream, src, dst, N, nkb, total);
  return hipGetLastError();
}

hipError_t launch_repack_ternary2(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N,
                                  uint32_t* bad_flag, hipStream_t stream) {
  const uint32_t nkb = K / kBlockK;
  const size_t total = (size_t)col_tiles(N) * nkb * 64u * 2u;
  const size_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(repack_tern_kernel, dim3((uint32_t)grid), dim3(256), 0, stream, src, dst, N, nkb, total,
                     bad_flag);
  return hipGetLastError();
}

}  // namespace hq

// hq_repack.hip — device repack of linear int4 / ternary weights into the gfx950 tile
// layout (hq_layout.hpp). One thread per packed output word; the host variants in
// hq_host.cpp produce the same words.
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

}  // namespace

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

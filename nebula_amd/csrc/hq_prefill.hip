// hq_prefill.hip — qGEMM for M > 16.
// First version: runs the decode kernel over 16-row slices of X (correct for any M;
// the MFMA tile kernel replaces it).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hq_internal.hpp"

namespace hq {

hipError_t launch_prefill(int fmt, int dtype, GemmDesc d, hipStream_t stream) {
  for (uint32_t m0 = 0; m0 < d.M; m0 += 16) {
    GemmDesc e = d;
    e.M = std::min<uint32_t>(16, d.M - m0);
    e.X = reinterpret_cast<const char*>(d.X) + (size_t)m0 * (size_t)d.ldx * 2u;
    for (uint32_t i = 0; i < d.nseg; ++i)
      e.seg[i].Y = reinterpret_cast<char*>(d.seg[i].Y) + (size_t)m0 * (size_t)d.seg[i].ldy * 2u;
    hipError_t err = launch_decode(fmt, dtype, e, stream);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace hq

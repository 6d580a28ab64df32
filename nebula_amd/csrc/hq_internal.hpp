// hq_internal.hpp — descriptors shared by the C-ABI layer and the kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hq_qgemm.h"

namespace hq {

// One projection inside a (possibly fused) launch. blk_begin is the first workgroup
// (grid x index) that works on this segment; the launcher fills it.
struct SegDesc {
  const uint32_t* Wp;
  const uint16_t* S;
  void* Y;
  int64_t ldy;
  uint32_t N;
  uint32_t ntiles;     // ceil(N / 16)
  uint32_t blk_begin;  // first slab of this segment (decode) / first grid x index (prefill)
  uint32_t blk_count;  // slabs of this segment (decode) / grid x extent (prefill)
  uint32_t slab_w;     // decode: tiles per slab (the first slab_r slabs hold one more)
  uint32_t slab_r;
};

struct GemmDesc {
  const void* X;
  int64_t ldx;
  uint32_t M, K;
  uint32_t nkb;  // K / 128
  uint32_t gkb;  // group / 128
  uint32_t nseg;
  uint32_t pad;
  SegDesc seg[HQ_MAX_SEGMENTS];
};

// Decode tiling: T column tiles per wavefront, WK wavefronts splitting K inside a
// workgroup (LDS reduction), SK workgroups splitting K across the grid (workspace fixup).
struct DecodeConfig {
  int T;
  int WK;
  int SK;      // workgroups (stream-K grid size)
  bool contig; // wavefronts take contiguous k runs of a piece (else interleaved)
  uint32_t G = 0;  // target slab count (0: ceil(tiles / T)); slabs then hold <= T tiles
};
DecodeConfig choose_decode(int fmt, const GemmDesc& d);
// Workspace bytes a decode launch with this config needs (0 when SK == 1). The first
// 256 bytes-aligned part holds one uint32 counter per column group; these must be zero
// before the first launch and are left zero by every launch.
size_t decode_workspace_bytes(const GemmDesc& d, const DecodeConfig& c);

// Decode (M <= 16): HBM-streaming MFMA kernel. Validated descriptor in, status out.
hipError_t launch_decode(int fmt, int dtype, GemmDesc d, const DecodeConfig& c, void* ws, hipStream_t stream);
// Prefill (M > 16): MFMA tile kernel.
hipError_t launch_prefill(int fmt, int dtype, GemmDesc d, hipStream_t stream);

hipError_t launch_repack_int4(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N,
                              hipStream_t stream);
hipError_t launch_repack_ternary2(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N,
                                  uint32_t* bad_flag, hipStream_t stream);

}  // namespace hq

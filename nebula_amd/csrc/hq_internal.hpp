// hq_internal.hpp — descriptors shared by the C-ABI layer and the kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hq_qgemm.h"

// Sets the calling thread's hq_last_error message (cleared for HQ_OK) and returns s.
hq_status hq_set_error(hq_status s, const char* fmt, ...);

namespace hq {

// One projection inside a (possibly fused) launch. blk_begin is the first workgroup
// (grid x index) that works on this segment; the launcher fills it.
struct SegDesc {
  const uint32_t* Wp;
  const uint16_t* S;
  const float* B;      // fp32 per-group bias [K/group][lds] (int4, general kernels only) or null
  void* Y;
  int64_t ldy;
  uint32_t N;
  uint32_t lds;        // scale row stride in elements (N unless the segment is a column range)
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
  uint32_t gkb;  // group / 128 (fast kernels: group % 128 == 0)
  uint32_t nseg;
  // General kernels (a bias, or a group that is not a multiple of 128): one scale (and bias)
  // per 32-wide k chunk, scale row (4 kb + c) / g32 of chunk c of k-block kb.
  uint32_t gen;       // 1: run the general kernels
  uint32_t g32;       // group / 32
  uint32_t g32_m;     // plan_div_magic(g32)
  uint32_t has_bias;  // some segment has a bias (the others read it as 0 and add nothing)
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
  int U = 0;       // register ring depth in k-blocks (0: the default for T)
};
DecodeConfig choose_decode(int fmt, const GemmDesc& d);
// Workspace bytes a decode launch with this config needs (0 when SK == 1). The first
// 256 bytes-aligned part holds one uint32 counter per column group; these must be zero
// before the first launch and are left zero by every launch.
size_t decode_workspace_bytes(const GemmDesc& d, const DecodeConfig& c);

// Decode (M <= 16): HBM-streaming MFMA kernel. Validated descriptor in, status out.
hipError_t launch_decode(int fmt, int dtype, GemmDesc d, const DecodeConfig& c, void* ws, hipStream_t stream);

// X-resident decode (M <= 16, activation rows of all K in LDS): one workgroup per slab of T
// column tiles, WK wavefronts splitting its k-blocks, a register ring of U steps.
struct XrConfig {
  int T;
  int U;
  int WK;
  int S;         // pieces per slab along K (workspace fix-up when > 1)
  uint32_t lds;  // dynamic LDS bytes per workgroup
  bool ok;       // the rows fit in LDS and the kernel takes the call
  uint32_t G = 0;  // slabs over all segments; 0: ceil(tiles / T) per segment (else up to T tiles each)
  int SG = 1;      // slab groups of WK wavefronts per workgroup sharing one copy of the rows (S = 1)
};
// LDS one X-resident workgroup may use (the whole 160 KiB of a gfx950 CU).
constexpr uint32_t kXrLdsMax = 160u * 1024u;
// ws_cap: the largest workspace the plan may use (no plan with pieces above it).
XrConfig choose_decode_xr(int fmt, const GemmDesc& d, size_t ws_cap = SIZE_MAX);
size_t decode_xr_workspace_bytes(const GemmDesc& d, const XrConfig& c);
hipError_t launch_decode_xr(int fmt, int dtype, GemmDesc d, const XrConfig& c, void* ws, hipStream_t stream);

// The int8 path (hq_int8.hip): T column tiles per slab, U steps in flight, WK wavefronts, S K
// pieces per slab; lds: dynamic LDS bytes per workgroup.
struct W8Config {
  int T;
  int U;
  int WK;
  int S;
  uint32_t lds;
  bool ok;
  bool qx = false;  // the GEMM quantises its own activation rows (one launch)
};
W8Config choose_w8a8(uint32_t M, uint32_t K, uint32_t N);
size_t w8a8_workspace_bytes(uint32_t M, uint32_t K, uint32_t N, const W8Config& c);
hipError_t launch_w8a8(const float* X, uint32_t ldx, const int8_t* Wp, const float* scales, float* Y, uint32_t ldy,
                       uint32_t M, uint32_t K, uint32_t N, const W8Config& c, void* ws, hipStream_t stream);

// Lockstep decode (M <= 80): KG k-groups of GW wavefronts per workgroup own a slab of up
// to GW * T column tiles and walk one piece of its k-blocks together (S pieces per slab),
// each k-group sharing its activation k-block (MT tiles of 16 rows) through LDS.
struct LsConfig {
  int T;  // tiles per wavefront (1, 2 or 4)
  int U;   // steps in flight per wavefront (register ring depth)
  int S;   // pieces (workgroups) per slab along K
  int KG;  // k-groups per workgroup (1, 2 or 4)
  int GW;  // wavefronts per k-group (2 or 4)
  int SW;  // tiles per slab, at most GW * T (wavefront i takes tiles T i .. min(T i + T, SW) - 1)
  int MT;  // 16-row tiles of activations (1 .. kLsMaxRowTiles): rows M <= 16 MT
  int P = 0;  // balanced grid (several row tiles, more slabs than CUs): P workgroups, each an
              // equal run of (slab, k-block) units; 0 = the S-piece grid
};
// The lockstep kernel takes up to this many 16-row tiles (M <= 80: a split-fuse step of 16
// decode tokens and a 64-token prefill chunk fits one call).
constexpr uint32_t kLsMaxRowTiles = 5;
struct LsPlan {
  uint32_t sw;      // tiles per slab
  uint32_t S;       // pieces per slab
  uint32_t kq, kr;  // piece p covers k-blocks [p * kq + min(p, kr), ...) of kq (+1 if p < kr)
  uint32_t gmul;    // plan_gmul(gkb)
  uint32_t* cnt;    // [G] arrival counters, zero between launches (S > 1)
  float* part;      // [G][S][GW * T * MT tiles][64 lanes] f4 partial tiles (S > 1)
  uint32_t* fault;  // host-visible word set to 1 when a k-group barrier gives up (may be null)
  uint32_t spin;    // polls before a k-group barrier gives up
  // Balanced grid (LsConfig::P > 0, more slabs than workgroups): workgroup b takes units
  // (g nkb + kb, slab-major) [begin(b), begin(b + 1)), begin(b) = b bL + min(b, brem): its
  // first and last slab may be partial (at most two contributors each, bL >= nkb); part then
  // holds [P][2][GW * T * MT tiles][64 lanes] f4 (slot 0: first slab, 1: last slab).
  uint32_t bL, brem;
  uint32_t nkb_m;   // plan_div_magic(nkb)
};
// Polls of the lockstep k-group barrier before it gives up (each poll sleeps ~64 cycles):
// far beyond any correct launch, whose k-groups stay within one step of each other.
constexpr uint32_t kLsSpinLimit = 1u << 22;
// ws_cap: the largest workspace the plan may use (fewer pieces per slab below it).
LsConfig choose_decode_ls(int fmt, const GemmDesc& d, size_t ws_cap = SIZE_MAX);
size_t decode_ls_workspace_bytes(const GemmDesc& d, const LsConfig& c);
hipError_t launch_decode_ls(int fmt, int dtype, GemmDesc d, const LsConfig& c, void* ws, uint32_t* fault,
                            uint32_t spin, hipStream_t stream);

// One prefill launch: (16 * RT * WM)-row x 256-column tiles over the columns of d; psk
// stream-K workgroups share the last tiles - dp tiles along K, dp workgroups own one tile
// each.
struct PrefillLaunch {
  int RT;
  int WM;
  int KS;  // 2: each tile's k-blocks split between two halves of one workgroup (whole tiles)
  int TW;  // column tiles per wavefront: 4 (256-column tiles) or 2 (128-column whole tiles)
  GemmDesc d;
  uint32_t tiles;
  uint32_t dp;
  uint32_t psk;
};
// A prefill call: one launch, or two over disjoint column ranges (the second with
// half-height tiles).
struct PrefillConfig {
  int n;
  PrefillLaunch l[2];
};
// ws_cap: the largest workspace the plan may use (fewer stream-K workgroups, or none, below it).
// dtype: the activation type (the tile width depends on it; the workspace does not).
PrefillConfig choose_prefill(int fmt, const GemmDesc& d, size_t ws_cap = SIZE_MAX, int dtype = HQ_DTYPE_F16);
// Workspace bytes of a prefill call (0 without stream-K): the counter area, then two fp32
// partial tiles per stream-K workgroup.
size_t prefill_workspace_bytes(const GemmDesc& d, const PrefillConfig& c);
// Prefill (M > 16): MFMA tile kernel.
// fault / spin: the fault word and the poll bound of the K halves' barrier (KS = 2 launches).
hipError_t launch_prefill(int fmt, int dtype, const PrefillConfig& c, void* ws, uint32_t* fault, uint32_t spin,
                          hipStream_t stream);

// Whether this build has the general kernels (a bias, groups that are multiples of 32 but
// not of 128); without them such calls fail with HQ_ERR_UNSUPPORTED.
constexpr bool kGeneralKernels = true;

// Counter area at the start of every workspace, the same for all shapes and both kernels
// so that one workspace can serve calls of different shapes (the counters stay zero
// between calls; the partial area after them does not).
constexpr uint32_t kMaxCounters = 16384;
constexpr size_t kCounterBytes = kMaxCounters * 4u;

// Compute units of the current device (256 if it cannot be queried).
int cu_count();

hipError_t launch_repack_int4(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N,
                              hipStream_t stream);
hipError_t launch_repack_ternary2(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N,
                                  uint32_t* bad_flag, hipStream_t stream);
hipError_t launch_repack_tq1_0(const uint8_t* blocks, uint32_t* dst, uint16_t* scales, uint32_t K, uint32_t N,
                               hipStream_t stream);

}  // namespace hq

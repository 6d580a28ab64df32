// hq_decode.hip — memory-bound qGEMM for M <= 16 (decode), gfx950.
//
// Replaces kernel_marlin_gemm_int4_templated / _dynamic
// (hydrogen/src/model/marlin_gemm.cu:130-237, 242-322). The reference gives each
// thread one output column and does 32 x M scalar FMAs per 16-byte weight load,
// then merges 16 fixed K-splits with fp32 atomics into a pre-zeroed Y. Two kernels here,
// both dequantising weights in registers straight into MFMA B fragments multiplied
// against the activation rows (M padded to 16) with v_mfma_f32_16x16x32_{f16,bf16}; int4 uses
// the biased form (magic + q, one v_and_or_b32 per fragment word) and removes the bias with
// one extra MFMA per chunk whose result seeds every tile's accumulator; the group scale
// multiplies the fp32 k-block sum once per (column, k-block).
//   * hq_decode_xr_kernel, the default for M <= 16: one workgroup per (slab of T column
//     tiles, piece of K), or per group of two to four whole slabs; the activation rows are copied
//     into LDS once, then the wavefronts stream the slab's weights through a barrier-free
//     register ring and meet once, at the end, in LDS (pieces of a slab: a last-arriver
//     fix-up in piece order);
//   * hq_decode_kernel, the per-wavefront kernel, at up to four rows when the X-resident
//     kernel has no plan (rows too long even in eight pieces, or pieces beyond a workspace
//     cap) and when tests force it: the work is cut into units of
//     (slab of T column tiles) x (128-deep k-block) and every workgroup streams an equal
//     contiguous range of units (hq_plan.hpp); inside a workgroup the WK wavefronts take the
//     units of each slab in turn, each with U k-blocks of weights, scales and activations in
//     flight in a register ring, and meet once to sum their per-slab results through LDS;
//     slabs cut by a range boundary are completed by a last-arriver fix-up in workgroup order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>

#include "hq_device.hpp"
#include "hq_internal.hpp"
#include "hq_plan.hpp"

namespace hq {
namespace {

template <int FMT>
struct WTraits;
template <>
struct WTraits<HQ_FORMAT_INT4> {
  using V = u4;
  static constexpr uint32_t wpl = 4;
};
template <>
struct WTraits<HQ_FORMAT_TERNARY2> {
  using V = u2;
  static constexpr uint32_t wpl = 2;
};

// Largest workgroup (in wavefronts) per slab width: the register rings of T >= 2 leave
// room for two wavefronts per SIMD, those of T = 1 for four.
constexpr int max_wk(int T) { return T >= 2 ? 8 : 16; }

struct Piece {
  uint32_t g, ka, kz;  // slab and its k-block range [ka, kz) inside this workgroup
};

template <int FMT, int DT, int T, int U, bool FUSED>
__global__ void __launch_bounds__(64 * max_wk(T)) hq_decode_kernel(const GemmDesc d, const DecodePlan pl) {
  using W = typename WTraits<FMT>::V;
  constexpr uint32_t WPL = WTraits<FMT>::wpl;
  constexpr uint32_t kLaneBytes = WPL * 4u;
  constexpr uint32_t kBlockBytes = 64u * kLaneBytes;  // one tile x one k-block
  constexpr uint32_t kCols = 16u * T;                 // output columns of a slab
  constexpr bool kInt4 = FMT == HQ_FORMAT_INT4;
  extern __shared__ float red[];  // [np_max][WK][M * kCols]
  __shared__ uint32_t sh_last[2];

  const uint32_t lane = threadIdx.x & 63u;
  // Wave index through readfirstlane so all unit bookkeeping stays scalar.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t WK = pl.WK;
  const uint32_t c16 = lane & 15u;
  const uint32_t g4 = lane >> 4;
  const uint32_t nkb = d.nkb;
  const uint32_t b = blockIdx.x;
  const uint32_t M = d.M;
  const uint32_t SL = M * kCols;  // floats of one piece's partial tile

  const uint32_t u0 = plan_begin(pl.L, pl.rem, b);
  const uint32_t u1 = plan_begin(pl.L, pl.rem, b + 1);
  const uint32_t gfirst = plan_div(u0, nkb, pl.nkb_m), glast = plan_div(u1 - 1u, nkb, pl.nkb_m);
  const uint32_t np = glast - gfirst + 1u;
  auto piece = [&](uint32_t i) {
    Piece p;
    p.g = plan_piece_slab(gfirst, glast, i);
    p.ka = p.g == gfirst ? u0 - p.g * nkb : 0u;
    p.kz = p.g == glast ? u1 - p.g * nkb : nkb;
    return p;
  };
  // k-blocks [s, e) step st of wavefront w inside piece p: interleaved (w, w + WK, ...) or
  // one contiguous run per wavefront.
  const uint32_t kstep = pl.contig ? 1u : WK;
  auto span_begin = [&](const Piece& p, uint32_t w) {
    return pl.contig ? p.ka + (w * (p.kz - p.ka)) / WK : p.ka + w;
  };
  auto span_end = [&](const Piece& p, uint32_t w) {
    return pl.contig ? p.ka + ((w + 1u) * (p.kz - p.ka)) / WK : p.kz;
  };

  // Fixed per-lane offsets. Tile t of a slab lies t * nkb blocks after tile 0, so the
  // slab descriptor (sized to its valid tiles) turns missing tiles into zero reads.
  uint32_t wvo[T];
#pragma unroll
  for (int t = 0; t < T; ++t) wvo[t] = lane * kLaneBytes + (uint32_t)t * nkb * kBlockBytes;
  // A operand: row c16 of X, k-slice g4 of each chunk; rows >= M read as zero.
  const uint32_t xbytes = M * (uint32_t)d.ldx * 2u;
  const uint32_t xo = c16 * (uint32_t)d.ldx * 2u + g4 * 16u;

  // Load-side iterator: piece lp, k-block lkb of this wavefront, with the buffer
  // extents of the piece's slab (zero once the wavefront's units are exhausted, which
  // turns the remaining ring loads into zero reads without memory traffic).
  uint32_t lp = 0, lkb = 0, lkz = 0;
  const uint32_t* lw_base = d.seg[0].Wp;
  const uint16_t* ls_base = d.seg[0].S;
  uint32_t lw_num = 0, ls_num = 0, lsrow = 0;
  // Scales: load j of a unit gives lane l column 64 j + l % (16 T) of the slab (one load
  // per four tiles); the flush gathers tile t's scale for column c16 from lane
  // 16 (t % 4) + c16 of load t / 4.
  constexpr int kSL = (T + 3) / 4;
  uint32_t svo[kSL];
#pragma unroll
  for (int j = 0; j < kSL; ++j) svo[j] = 0;

  // Segment of slab g; a plain loop so the segment table is read on demand, not held. A
  // one-segment call (FUSED = false) reads its fields at fixed offsets, without a chain of
  // dependent argument loads.
  auto seg_of = [&](uint32_t g) -> uint32_t {
    if constexpr (!FUSED) return 0u;
    uint32_t s = 0;
    for (uint32_t i = 1; i < d.nseg; ++i)
      if (g >= d.seg[i].blk_begin) s = i;
    return __builtin_amdgcn_readfirstlane(s);
  };
  // Column tiles [ct0, ct0 + nv) of slab g: a segment's slabs split its tiles as evenly
  // as integers allow (the first slab_r slabs hold slab_w + 1 tiles, the rest slab_w).
  auto slab_tiles = [&](const SegDesc& sg, uint32_t g, uint32_t& ct0, uint32_t& nv) {
    const uint32_t l = g - sg.blk_begin;
    ct0 = l * sg.slab_w + min(l, sg.slab_r);
    nv = sg.slab_w + (l < sg.slab_r ? 1u : 0u);
  };
  auto open_piece = [&](uint32_t i) {  // set the load extents for piece i (< np)
    const Piece p = piece(i);
    const uint32_t s = seg_of(p.g);
    uint32_t ct0, nv;
    slab_tiles(d.seg[s], p.g, ct0, nv);
    const uint32_t N = d.seg[s].N, lds = d.seg[s].lds;
    lw_base = d.seg[s].Wp + (size_t)ct0 * nkb * 64u * WPL;
    lw_num = __builtin_amdgcn_readfirstlane(nv * nkb * kBlockBytes);
    ls_base = d.seg[s].S;
    ls_num = __builtin_amdgcn_readfirstlane(((nkb / d.gkb - 1u) * lds + N) * 2u);
    lsrow = __builtin_amdgcn_readfirstlane(lds * 2u);
#pragma unroll
    for (int j = 0; j < kSL; ++j) svo[j] = min(ct0 * 16u + 64u * j + lane % kCols, N - 1u) * 2u;
    lkb = span_begin(p, wave);
    lkz = span_end(p, wave);
  };
  // Move to the next piece in which this wavefront has units (or past the last one).
  auto next_load_piece = [&]() {
    while (lp < np) {
      open_piece(lp);
      if (lkb < lkz) return;
      ++lp;
    }
    lw_num = 0;
    ls_num = 0;
    lkb = 0;
  };
  auto advance_load = [&]() {
    if (lp >= np) return;
    lkb += kstep;
    if (lkb >= lkz) {
      ++lp;
      next_load_piece();
    }
  };

  // Register ring: slot u holds one unit's weights, scales and activations, issued
  // together. vmcnt retires loads in issue order, so anything fetched later than the
  // weights it is used with would drain the whole ring; one issue point per unit keeps
  // U - 1 units in flight. Loads past the wavefront's units read zero.
  W wr[U][T];
  uint32_t sr[U][kSL];
  u4 ar[U][4];
  auto load = [&](int slot) {
    const __amdgpu_buffer_rsrc_t lw = make_rsrc(lw_base, lw_num);
    const __amdgpu_buffer_rsrc_t ls = make_rsrc(ls_base, ls_num);
    // Past the wavefront's units every extent is zero: the ring's trailing loads return
    // zeros without a memory access, so the final wait does not hang on cache round trips.
    const __amdgpu_buffer_rsrc_t lx = make_rsrc(d.X, lw_num ? xbytes : 0u);
    const uint32_t kbo = __builtin_amdgcn_readfirstlane(lkb * kBlockBytes);
    const uint32_t so = __builtin_amdgcn_readfirstlane(plan_group_of_kb(lkb, pl.gmul) * lsrow);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if constexpr (WPL == 4) wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b128(lw, wvo[t], kbo, kStreamAux);
      else wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b64(lw, wvo[t], kbo, kStreamAux);
    }
#pragma unroll
    for (int j = 0; j < kSL; ++j) sr[slot][j] = __builtin_amdgcn_raw_buffer_load_b16(ls, svo[j], so, 0);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      ar[slot][c] = __builtin_amdgcn_raw_buffer_load_b128(lx, xo + c * 64u, __builtin_amdgcn_readfirstlane(lkb * 256u), 0);
  };

  // Compute-side iterator over the same sequence.
  uint32_t cp = 0, ckb = 0, ckz = 0;
  auto next_compute_piece = [&]() {
    while (cp < np) {
      const Piece p = piece(cp);
      ckb = span_begin(p, wave);
      ckz = span_end(p, wave);
      if (ckb < ckz) return;
      ++cp;
    }
  };

  f4 acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

  // Park the current piece's sums (rows < M only) in this wavefront's LDS slot.
  auto park = [&](uint32_t p) {
    float* dst = red + (p * WK + wave) * SL;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t row = 4u * g4 + v;
        if (row < M) dst[row * kCols + t * 16u + c16] = acc[t][v];
        acc[t][v] = 0.0f;
      }
  };

  const DqBiasConst dqb = DT == HQ_DTYPE_F16 ? dq_bias_const_f16() : dq_bias_const_bf16();
  const u4 corr_b = int4_corr_fragment<DT>();

  auto compute = [&](int u) {
    // Scale of tile t for this lane's column, gathered first so the LDS-crossbar
    // latency overlaps the MFMAs.
    uint32_t sbits[T];
#pragma unroll
    for (int t = 0; t < T; ++t)
      sbits[t] = T == 1 ? sr[u][0]
                        : (uint32_t)__builtin_amdgcn_ds_bpermute((int)((16u * (t % 4) + c16) * 4u), (int)sr[u][t / 4]);
    f4 seed = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kInt4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) seed = mfma16x16x32<DT>(ar[u][c], corr_b, seed);
    }
    // Chunk-outer order: the T accumulation chains are independent and interleave.
    f4 g[T];
#pragma unroll
    for (int t = 0; t < T; ++t) g[t] = seed;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        u4 bf;
        if constexpr (kInt4) {
          bf = dq_int4_biased<DT>(wr[u][t][c], dqb);
        } else {
          const uint32_t word = wr[u][t][c >> 1];
          bf = (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);
        }
        g[t] = mfma16x16x32<DT>(ar[u][c], bf, g[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float sc = f16_to_f32((uint16_t)sbits[t]);
      if constexpr (!kInt4) {
        // A non-finite block scale drops the block (native_decoder.cu:174); fields hold 2t.
        sc = __builtin_isfinite(sc) ? 0.5f * sc : 0.0f;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(g[t][v], sc, acc[t][v]);
    }
  };

  // Prologue: position both iterators and fill the ring in slot order (no reordering
  // across the barriers: the loop header's wait count assumes slot 0 is the oldest load).
  next_load_piece();
  next_compute_piece();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    load(u);
    advance_load();
    __builtin_amdgcn_sched_barrier(0);
  }

  while (cp < np) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (cp < np) {  // uniform; no loads inside, so waitcnt stays exact across it
        compute(u);
        ckb += kstep;
        if (ckb >= ckz) {
          park(cp);
          ++cp;
          next_compute_piece();
        }
      }
      load(u);
      advance_load();
    }
  }

  // Epilogue. Each piece's tile is summed over the wavefronts that worked on it, in
  // wavefront order, four consecutive columns per thread (16-byte LDS reads).
  __syncthreads();
  const uint32_t nthr = WK * 64u;
  const uint32_t SL4 = SL / 4u;  // SL is a multiple of 16
  // The workspace partials as a buffer, accessed 16 bytes at a time with the sc1 cache
  // policy: agent-coherent (visible across XCDs once the store has completed).
  constexpr int kCoherent = 16;
  const __amdgpu_buffer_rsrc_t partr = make_rsrc(pl.part, pl.part ? pl.P * 2u * SL * 4u : 0u);
  // Stores four consecutive outputs of a slab tile; only the slab's own columns
  // (local column < ncols) that exist (< N) are written.
  auto store4 = [&](const SegDesc& sg, uint32_t col0, uint32_t ncols, uint32_t o4, f4 v) {
    const uint32_t o = 4u * o4, row = o / kCols, lc = o % kCols, n = col0 + lc;
    if (lc >= ncols) return;  // ncols is a multiple of 16, so lc + 3 < ncols too
    uint16_t* y = reinterpret_cast<uint16_t*>(sg.Y) + (size_t)row * sg.ldy + n;
    if (n + 3u < sg.N && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
      const u2 packed = {(uint32_t)f32_to_out<DT>(v[0]) | ((uint32_t)f32_to_out<DT>(v[1]) << 16),
                         (uint32_t)f32_to_out<DT>(v[2]) | ((uint32_t)f32_to_out<DT>(v[3]) << 16)};
      *reinterpret_cast<u2*>(y) = packed;
    } else {
#pragma unroll
      for (uint32_t e = 0; e < 4u; ++e)
        if (n + e < sg.N) y[e] = f32_to_out<DT>(v[e]);
    }
  };
  bool partial_any = false;
  for (uint32_t i = 0; i < np; ++i) {
    const Piece p = piece(i);
    const SegDesc& sg = d.seg[seg_of(p.g)];
    uint32_t ct0, nv;
    slab_tiles(sg, p.g, ct0, nv);
    const uint32_t col0 = ct0 * 16u, ncols = nv * 16u;
    const bool full = p.ka == 0u && p.kz == nkb;
    partial_any |= !full;
    uint32_t wmask = 0;  // wavefronts with units in this piece
    for (uint32_t w = 0; w < WK; ++w)
      if (span_begin(p, w) < span_end(p, w)) wmask |= 1u << w;
    for (uint32_t o4 = threadIdx.x; o4 < SL4; o4 += nthr) {
      f4 v = f4{0.f, 0.f, 0.f, 0.f};
      for (uint32_t w = 0; w < WK; ++w)
        if ((wmask >> w) & 1u) v += *reinterpret_cast<const f4*>(red + (i * WK + w) * SL + 4u * o4);
      if (full) store4(sg, col0, ncols, o4, v);
      else __builtin_amdgcn_raw_buffer_store_b128(v, partr, (((b * 2u + i) * SL) + 4u * o4) * 4u, 0, kCoherent);
    }
  }
  if (!partial_any) return;  // uniform: depends only on the range

  // Fix-up of partial pieces (pieces 0 and 1 only): publish, count arrivals, and let the
  // last contributor of each slab sum all contributors' partials in workgroup order.
  // Waiting for the coherent partial stores to complete before the barrier orders them
  // before the arrival count without an L2 write-back; the last contributor reads them
  // with coherent loads after seeing the count.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  if (threadIdx.x < 2u) {
    const uint32_t i = threadIdx.x;
    uint32_t last = 0;
    if (i < np) {
      const Piece p = piece(i);
      if (!(p.ka == 0u && p.kz == nkb)) {
        const uint32_t bf = plan_wg_of_unit(pl.L, pl.rem, p.g * nkb);
        const uint32_t bl = plan_wg_of_unit(pl.L, pl.rem, (p.g + 1u) * nkb - 1u);
        const uint32_t old = __hip_atomic_fetch_add(pl.cnt + p.g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == bl - bf) {
          last = 1u;
          __hip_atomic_store(pl.cnt + p.g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    sh_last[i] = last;
  }
  __syncthreads();
  const uint32_t last0 = sh_last[0], last1 = sh_last[1];
  if (!(last0 | last1)) return;
  constexpr uint32_t kMaxIt = (16u * kCols / 4u + 63u) / 64u;  // float4 per thread, WK >= 1
  for (uint32_t i = 0; i < 2u; ++i) {
    if (!(i == 0 ? last0 : last1)) continue;
    const Piece p = piece(i);
    const SegDesc& sg = d.seg[seg_of(p.g)];
    uint32_t ct0, nv;
    slab_tiles(sg, p.g, ct0, nv);
    const uint32_t col0 = ct0 * 16u, ncols = nv * 16u;
    const uint32_t bf = plan_wg_of_unit(pl.L, pl.rem, p.g * nkb);
    const uint32_t bl = plan_wg_of_unit(pl.L, pl.rem, (p.g + 1u) * nkb - 1u);
    f4 v[kMaxIt];
#pragma unroll
    for (uint32_t j = 0; j < kMaxIt; ++j) v[j] = f4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t c = bf; c <= bl; ++c) {  // contributors in workgroup order
      const uint32_t cslot = plan_div(plan_begin(pl.L, pl.rem, c), nkb, pl.nkb_m) == p.g ? 0u : 1u;
      const uint32_t base = (c * 2u + cslot) * SL * 4u;
#pragma unroll
      for (uint32_t j = 0; j < kMaxIt; ++j) {
        const uint32_t o4 = threadIdx.x + j * nthr;
        if (o4 < SL4) v[j] += __builtin_amdgcn_raw_buffer_load_b128(partr, base + 16u * o4, 0, kCoherent);
      }
    }
#pragma unroll
    for (uint32_t j = 0; j < kMaxIt; ++j) {
      const uint32_t o4 = threadIdx.x + j * nthr;
      if (o4 < SL4) store4(sg, col0, ncols, o4, v[j]);
    }
  }
}

// ---------------------------------------------------------------------------------------
// X-resident decode kernel: one workgroup per (slab of T column tiles, piece of its
// k-blocks), its WK wavefronts splitting the piece's k-blocks (k-block w, w + WK, ... for
// wavefront w). The activation rows of the piece (M <= 16) are copied into LDS once, by
// LDS-DMA, before the weight stream starts; afterwards every wavefront streams its weights through a register ring of U
// steps (T tiles x one k-block each) with no barrier and no activation load in the ring,
// and reads its A fragments from LDS. Measured on MI355X, a barrier-free register ring
// streams at the rate of a plain copy, while activation loads from L2 inside the ring (one
// wavefront fetching them per k-block) or a workgroup barrier per k-block cost 15-25% of
// the stream. The partial sums of the wavefronts meet once, in LDS, summed in wavefront
// order (deterministic), after the activation rows are no longer needed. With S > 1 pieces
// per slab each workgroup stores its partial tile to the workspace and the last of the
// slab's workgroups to arrive (per-slab counter) sums the S partials in piece order.
// Slab groups (GRP, whole slabs only): a workgroup of SG groups of WK wavefronts, group h
// streaming slab blockIdx.x + h * gridDim.x over the one copy of the rows, so that a CU that
// would hold two workgroups copies the rows once and starts both streams at once.
//
// LDS layout of the activation rows of a piece of nkbp k-blocks from kb0: 16-byte units,
// unit (r * nkbp + kb - kb0) * 16 + (j ^ r) holds elements 8 j .. 8 j + 7 of k-block kb of
// row r (j = 0..15). A fragment read of
// chunk c (lane: row c16, slice g4, piece j = 4 c + g4) touches 16 distinct units mod 16
// in every group of 16 lanes, i.e. every bank once. Lanes of rows >= M read row M - 1:
// an MFMA output row depends only on its own A row, and rows >= M are never stored.
struct XrPlan {
  uint32_t wk;       // wavefronts per slab (per slab group)
  uint32_t S;        // pieces per slab (grid y)
  uint32_t kq, kr;   // piece p covers k-blocks [p * kq + min(p, kr), ...), kq + (p < kr) of them
  uint32_t m_lo;     // plan_div_magic(16 * kq)
  uint32_t m_hi;     // plan_div_magic(16 * (kq + 1))
  uint32_t gmul;     // plan_gmul(gkb)
  uint32_t* cnt;     // [G] arrival counters, zero between launches (S > 1)
  float* part;       // [G][S][M * 16 * T] partial tiles (S > 1)
  uint32_t sg;       // slab groups per workgroup (S = 1): group h of workgroup b takes slab b + h * gridDim.x
  uint32_t nslabs;   // slabs over all segments
};

constexpr int xr_max_wk(int T) { return T >= 8 ? 8 : 16; }

// GRP: slab groups (pl.sg of them per workgroup); without it one slab per workgroup.
template <int FMT, int DT, int T, int U, bool FUSED, bool GRP = false>
__global__ void __launch_bounds__(64 * xr_max_wk(T)) hq_decode_xr_kernel(const GemmDesc d, const XrPlan pl) {
  using W = typename WTraits<FMT>::V;
  constexpr uint32_t WPL = WTraits<FMT>::wpl;
  constexpr uint32_t kLaneBytes = WPL * 4u;
  constexpr uint32_t kBlockBytes = 64u * kLaneBytes;  // one tile x one k-block
  constexpr uint32_t kCols = 16u * T;
  constexpr bool kInt4 = FMT == HQ_FORMAT_INT4;
  constexpr int kSL = (T + 3) / 4;  // scale loads per step (one per four tiles)
  extern __shared__ __attribute__((aligned(16))) char xs[];

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t c16 = lane & 15u;
  const uint32_t g4 = lane >> 4;
  const uint32_t p = blockIdx.y;  // piece
  // Every scalar the prologue needs, read from the kernel arguments in one batch: the empty
  // asm uses them all, so the loads issue together and are waited for once (left to itself
  // the compiler waited for the plan fields, then the shape, then the activation pointer:
  // three round trips before the first copy, 0.2-0.3 us on 5120 x 5120).
  const uint32_t WK = pl.wk, SG = GRP ? pl.sg : 1u, nkb = d.nkb, M = d.M, gkb = d.gkb, ldx = (uint32_t)d.ldx;
  const uint32_t kq = pl.kq, kr = pl.kr, m_lo = pl.m_lo, m_hi = pl.m_hi, gmul = pl.gmul;
  const void* const Xp = d.X;
  asm volatile("" ::"s"(WK), "s"(SG), "s"(nkb), "s"(M), "s"(gkb), "s"(ldx), "s"(kq), "s"(kr), "s"(m_lo),
               "s"(m_hi), "s"(gmul), "s"(Xp));
  const uint32_t kb0 = p * kq + min(p, kr);
  const uint32_t nkbp = kq + (p < kr ? 1u : 0u);
  // Slab groups: the workgroup's SG * WK wavefronts are SG groups of WK, group h streaming
  // slab blockIdx.x + h * gridDim.x over the one copy of the activation rows (wi: the
  // wavefront within its group). A group past the last slab loads and stores nothing.
  uint32_t h = 0;
  if constexpr (GRP)
    while (h + 1u < SG && wave >= (h + 1u) * WK) ++h;
  const uint32_t wi = wave - h * WK;
  const uint32_t graw = blockIdx.x + h * gridDim.x;
  const bool gl = !GRP || graw < pl.nslabs;
  const uint32_t g = gl ? graw : pl.nslabs - 1u;  // slab

  uint32_t s = 0;
  if constexpr (FUSED) {
    for (uint32_t i = 1; i < d.nseg; ++i)
      if (g >= d.seg[i].blk_begin) s = i;
    s = __builtin_amdgcn_readfirstlane(s);
  }
  const SegDesc& sg = d.seg[s];
  const uint32_t lsl = g - sg.blk_begin;
  const uint32_t ct0 = lsl * sg.slab_w + min(lsl, sg.slab_r);
  const uint32_t nv = sg.slab_w + (lsl < sg.slab_r ? 1u : 0u);
  const uint32_t N = sg.N;

  // 1. Activation rows -> LDS: 64 units per LDS-DMA instruction, instruction q by
  //    wavefront q mod (WK * SG); lane i of instruction q fetches the element piece of unit
  //    64 q + i.
  {
    const uint32_t ldx2 = ldx * 2u;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(Xp, M * ldx2);
    const uint32_t nkb16 = nkbp * 16u;
    const uint32_t m16 = p < kr ? m_hi : m_lo;
    const uint32_t nq = (M * nkb16 + 63u) / 64u;
    for (uint32_t q = wave; q < nq; q += WK * SG) {
      const uint32_t u = q * 64u + lane;
      const uint32_t r = plan_div(u, nkb16, m16);
      const uint32_t rem = u - r * nkb16;
      const uint32_t voff =
          r < M ? r * ldx2 + (kb0 + (rem >> 4)) * 256u + (((rem & 15u) ^ (r & 15u)) * 16u) : kOutOfRange;
      buffer_to_lds16(xr, xs + q * 1024u, voff);
    }
  }
  // The ring's first loads must be issued after the copies (vmcnt retires in order).
  __builtin_amdgcn_sched_barrier(0);

  // 2. Weight ring: step j of this wavefront is k-block kb = kb0 + wi + j * WK, T tiles.
  const uint32_t nj = gl && wi < nkbp ? (nkbp - wi + WK - 1u) / WK : 0u;
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(sg.Wp + (size_t)ct0 * nkb * 64u * WPL, __builtin_amdgcn_readfirstlane(nv * nkb * kBlockBytes));
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(sg.S, __builtin_amdgcn_readfirstlane(((nkb / gkb - 1u) * sg.lds + N) * 2u));
  const uint32_t lsrow = sg.lds * 2u;
  uint32_t wvo[T];
#pragma unroll
  for (int t = 0; t < T; ++t) wvo[t] = lane * kLaneBytes + (uint32_t)t * nkb * kBlockBytes;
  uint32_t svo[kSL];
#pragma unroll
  for (int jj = 0; jj < kSL; ++jj) svo[jj] = min(ct0 * 16u + 64u * jj + lane % kCols, N - 1u) * 2u;

  W wr[U][T];
  uint32_t sr[U][kSL];
  auto load = [&](int slot, uint32_t j) {
    const bool live = j < nj;
    const uint32_t kb = kb0 + wi + j * WK;
    const uint32_t kbo = __builtin_amdgcn_readfirstlane(live ? kb * kBlockBytes : 0u);
    const uint32_t so = __builtin_amdgcn_readfirstlane(live ? plan_group_of_kb(kb, gmul) * lsrow : 0u);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if constexpr (WPL == 4) wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b128(wrs, live ? wvo[t] : kOutOfRange, kbo, kStreamAux);
      else wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b64(wrs, live ? wvo[t] : kOutOfRange, kbo, kStreamAux);
    }
#pragma unroll
    for (int jj = 0; jj < kSL; ++jj) sr[slot][jj] = __builtin_amdgcn_raw_buffer_load_b16(srs, live ? svo[jj] : kOutOfRange, so, 0);
  };
#pragma unroll
  for (int u = 0; u < U; ++u) load(u, (uint32_t)u);
  __builtin_amdgcn_sched_barrier(0);

  // Wait for this wavefront's activation copies only: the ring's U * (T + kSL) loads were
  // issued after them and stay in flight. Then publish the rows to the workgroup.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(U * (T + kSL)));
  __syncthreads();

  // A fragment addresses: a[c] = xa[c] + (kb - kb0) * 256.
  uint32_t xa[4];
  const uint32_t xrow = min(c16, M - 1u);
#pragma unroll
  for (int c = 0; c < 4; ++c) xa[c] = (xrow * nkbp * 16u + (((4u * c + g4) ^ xrow))) * 16u;

  const DqBiasConst dqb = DT == HQ_DTYPE_F16 ? dq_bias_const_f16() : dq_bias_const_bf16();
  const u4 corr_b = int4_corr_fragment<DT>();
  f4 acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int u, uint32_t j) {
    const uint32_t kbl = wi + j * WK;  // k-block within the piece
    u4 a[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) a[c] = *reinterpret_cast<const u4*>(xs + xa[c] + kbl * 256u);
    // Ternary: a non-finite group scale drops the group, checked once per loaded scale
    // (before it is handed to the lanes of its tiles) and replaced by +0.
    uint32_t sl[kSL];
#pragma unroll
    for (int jj = 0; jj < kSL; ++jj)
      sl[jj] = kInt4 || (sr[u][jj] & 0x7C00u) != 0x7C00u ? sr[u][jj] : 0u;
    uint32_t sbits[T];
#pragma unroll
    for (int t = 0; t < T; ++t)
      sbits[t] = T == 1 ? sl[0] : (uint32_t)__builtin_amdgcn_ds_bpermute((int)((16u * (t % 4) + c16) * 4u), (int)sl[t / 4]);
    f4 seed = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kInt4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) seed = mfma16x16x32<DT>(a[c], corr_b, seed);
    }
    f4 gs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) gs[t] = seed;
    if constexpr (kInt4) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) gs[t] = mfma16x16x32<DT>(a[c], dq_int4_biased<DT>(wr[u][t][c], dqb), gs[t]);
    } else {
      // Ternary: chunks 0 and 2, then 1 and 3, each pair from one set of 64-bit shifts.
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u4 f0[T], f1[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (h == 0) dq_tern2_pair<0>(tern2_words(wr[u][t][0], wr[u][t][1]), f0[t], f1[t]);
          else dq_tern2_pair<1>(tern2_words(wr[u][t][0], wr[u][t][1]), f0[t], f1[t]);
        }
#pragma unroll
        for (int t = 0; t < T; ++t) gs[t] = mfma16x16x32<DT>(a[h], f0[t], gs[t]);
#pragma unroll
        for (int t = 0; t < T; ++t) gs[t] = mfma16x16x32<DT>(a[2 + h], f1[t], gs[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      // Ternary fields hold 2t: the sums are halved once after the loop (exact).
      const float sc = f16_to_f32((uint16_t)sbits[t]);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(gs[t][v], sc, acc[t][v]);
    }
  };

  for (uint32_t j = 0; j < nj; j += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j + u < nj) compute(u, j + u);  // uniform; no loads inside, so waitcnt stays exact across it
      load(u, j + u + U);
    }
  }
  // Loads past this wavefront's k-blocks read nothing; retire them before the registers
  // and the LDS are reused.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if constexpr (!kInt4) {
    // Halving commutes with fp32 rounding (no overflow or underflow at these magnitudes), so
    // this equals scaling every term by s / 2.
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] *= 0.5f;
  }

  // 3. Reduction: park each wavefront's sums (rows < M) over the activation rows, then
  //    sum them in wavefront order, four consecutive columns per thread.
  __syncthreads();
  const uint32_t SL = M * kCols;
  float* red = reinterpret_cast<float*>(xs);
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t row = 4u * g4 + v;
      if (row < M) red[wave * SL + row * kCols + t * 16u + c16] = acc[t][v];
    }
  __syncthreads();
  const uint32_t col0 = ct0 * 16u, ncols = nv * 16u;
  const uint32_t nthr = WK * 64u;
  const uint32_t tg = threadIdx.x - h * nthr;  // thread within the slab group
  red += h * WK * SL;                          // the group's parked sums
  // Workspace partials, accessed 16 bytes at a time with the sc1 cache policy: agent-coherent
  // (visible across XCDs once the store has completed).
  constexpr int kCoherent = 16;
  const uint32_t S = pl.S;
  const __amdgpu_buffer_rsrc_t partr = make_rsrc(pl.part, S > 1u ? gridDim.x * S * SL * 4u : 0u);
  if (S > 1u) {
    for (uint32_t o4 = tg; o4 < SL / 4u; o4 += nthr) {
      f4 v = f4{0.f, 0.f, 0.f, 0.f};
      for (uint32_t w = 0; w < WK; ++w) v += *reinterpret_cast<const f4*>(red + w * SL + 4u * o4);
      __builtin_amdgcn_raw_buffer_store_b128(v, partr, ((g * S + p) * SL + 4u * o4) * 4u, 0, kCoherent);
    }
    // The stores have completed before the barrier, so they are ordered before the arrival
    // count; the last arriver reads them with coherent loads after seeing the count. The
    // flag word reuses the (no longer read) reduction area.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    uint32_t* flag = reinterpret_cast<uint32_t*>(xs);
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(pl.cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t last = old == S - 1u ? 1u : 0u;
      if (last) __hip_atomic_store(pl.cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = last;
    }
    __syncthreads();
    if (*flag == 0u) return;
  }
  if (!gl) return;
  for (uint32_t o4 = tg; o4 < SL / 4u; o4 += nthr) {
    f4 v = f4{0.f, 0.f, 0.f, 0.f};
    if (S > 1u) {
      for (uint32_t q = 0; q < S; ++q)  // pieces in order
        v += __builtin_amdgcn_raw_buffer_load_b128(partr, ((g * S + q) * SL + 4u * o4) * 4u, 0, kCoherent);
    } else {
      for (uint32_t w = 0; w < WK; ++w) v += *reinterpret_cast<const f4*>(red + w * SL + 4u * o4);
    }
    const uint32_t o = 4u * o4, row = o / kCols, lc = o % kCols, n = col0 + lc;
    if (lc >= ncols) continue;
    uint16_t* y = reinterpret_cast<uint16_t*>(sg.Y) + (size_t)row * sg.ldy + n;
    if (n + 3u < N && (reinterpret_cast<uintptr_t>(y) & 7u) == 0) {
      const u2 packed = {(uint32_t)f32_to_out<DT>(v[0]) | ((uint32_t)f32_to_out<DT>(v[1]) << 16),
                         (uint32_t)f32_to_out<DT>(v[2]) | ((uint32_t)f32_to_out<DT>(v[3]) << 16)};
      *reinterpret_cast<u2*>(y) = packed;
    } else {
#pragma unroll
      for (uint32_t e = 0; e < 4u; ++e)
        if (n + e < N) y[e] = f32_to_out<DT>(v[e]);
    }
  }
}

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

}  // namespace

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  static std::mutex mu;
  static int cached[64] = {0};
  std::lock_guard<std::mutex> lock(mu);
  if (dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace {

// Slabs per segment for slab width T and a target total Gt (0: the fewest, ceil(nt / T)):
// each segment gets at least ceil(nt / T) slabs and about its share of Gt. Sets
// blk_begin / blk_count and returns the total.
uint32_t assign_slabs(GemmDesc& d, int T, uint32_t Gt) {
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) tiles += d.seg[i].ntiles;
  uint32_t g = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    const uint32_t nt = d.seg[i].ntiles;
    uint32_t ns = (nt + T - 1) / T;
    if (Gt) ns = std::max<uint32_t>(ns, (uint32_t)(((uint64_t)Gt * nt + tiles - 1) / tiles));
    ns = std::min(ns, nt);
    d.seg[i].blk_begin = g;
    d.seg[i].blk_count = ns;
    d.seg[i].slab_w = nt / ns;
    d.seg[i].slab_r = nt % ns;
    g += ns;
  }
  return g;
}
uint32_t total_slabs(const GemmDesc& d, int T, uint32_t Gt = 0) {
  GemmDesc c = d;
  return assign_slabs(c, T, Gt);
}

// Dynamic LDS budget of one workgroup (160 KiB per CU, less the kernel's static LDS).
constexpr size_t kLdsLimit = 160u * 1024u - 1024u;

size_t lds_bytes(const GemmDesc& d, const DecodeConfig& c, uint32_t np_max) {
  return (size_t)np_max * c.WK * d.M * 16u * c.T * sizeof(float);
}

template <int FMT, int DT, int T, int U>
hipError_t launch_t(GemmDesc d, const DecodeConfig& c, void* ws, hipStream_t stream) {
  DecodePlan pl{};
  const uint32_t blk = assign_slabs(d, T, c.G);
  pl.G = blk;
  pl.utot = blk * d.nkb;
  pl.P = (uint32_t)c.SK;
  pl.WK = (uint32_t)c.WK;
  pl.L = pl.utot / pl.P;
  pl.rem = pl.utot % pl.P;
  pl.nkb_m = plan_div_magic(d.nkb);
  pl.wk_m = plan_div_magic(pl.WK);
  pl.np_max = plan_np_max(pl.utot, pl.P, d.nkb);
  pl.gmul = plan_gmul(d.gkb);
  pl.contig = (uint32_t)c.contig;
  if (plan_has_partial(pl.G, pl.P)) {
    if (!ws) return hipErrorInvalidValue;
    pl.cnt = static_cast<uint32_t*>(ws);
    pl.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  }
  const size_t lds = lds_bytes(d, c, pl.np_max);
  if (lds > kLdsLimit) return hipErrorInvalidConfiguration;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_decode_kernel<FMT, DT, T, U, false>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsLimit) != hipSuccess
          ? hipErrorInvalidConfiguration
          : hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_decode_kernel<FMT, DT, T, U, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsLimit);
  if (attr != hipSuccess) return attr;
  if (d.nseg > 1)
    hipLaunchKernelGGL((hq_decode_kernel<FMT, DT, T, U, true>), dim3(pl.P), dim3(64 * c.WK), lds, stream, d, pl);
  else
    hipLaunchKernelGGL((hq_decode_kernel<FMT, DT, T, U, false>), dim3(pl.P), dim3(64 * c.WK), lds, stream, d, pl);
  return hipGetLastError();
}

template <int FMT, int DT>
hipError_t launch_fd(const GemmDesc& d, const DecodeConfig& c, void* ws, hipStream_t stream) {
  switch (c.T) {
    // Ring depth U (k-blocks in flight per wavefront): measured best 2 for T = 8 and 3
    // for T = 4 and 2 (deeper rings were slower); c.U overrides.
    case 8: return c.U == 3 ? launch_t<FMT, DT, 8, 3>(d, c, ws, stream) : launch_t<FMT, DT, 8, 2>(d, c, ws, stream);
    case 4:
      return c.U == 2   ? launch_t<FMT, DT, 4, 2>(d, c, ws, stream)
             : c.U == 4 ? launch_t<FMT, DT, 4, 4>(d, c, ws, stream)
                        : launch_t<FMT, DT, 4, 3>(d, c, ws, stream);
    case 2:
      return c.U == 2   ? launch_t<FMT, DT, 2, 2>(d, c, ws, stream)
             : c.U == 4 ? launch_t<FMT, DT, 2, 4>(d, c, ws, stream)
                        : launch_t<FMT, DT, 2, 3>(d, c, ws, stream);
    default: return launch_t<FMT, DT, 1, 4>(d, c, ws, stream);
  }
}

}  // namespace

// Tiling choice (measured on MI355X over the 27B-class decode shapes). The memory
// pipeline wants every CU streaming the same number of bytes with few wavefronts per CU,
// and whole slabs per workgroup (a cut slab costs a fix-up round trip at the end):
//   1. the widest uniform slab (8, 4 or 2 tiles) whose slab count keeps the last round of
//      workgroups >= 80% full (g / (CUs * ceil(g / CUs)) >= 0.8), one slab per workgroup;
//   2. otherwise balanced variable-width slabs: the tiles split over k * CUs workgroups (k
//      the smallest count giving <= 8 tiles each) when the widest holds at most 20% more
//      than the mean, one slab per workgroup (slab width 2, 4 or 8);
//   3. otherwise, for large weights (>= 24 MiB), 4-tile slabs each cut into
//      floor(CUs / slabs) k-ranges (stream-K fix-up);
//   4. otherwise (small weights, latency-bound) the widest slab giving >= 150 slabs
//      (else 2-tile, else 1-tile slabs), uncut, with two wavefronts per workgroup for
//      M > 8.
// Four wavefronts per workgroup otherwise. HQ_DECODE_T / _WK / _P / _CONTIG / _G override.
DecodeConfig choose_decode(int fmt, const GemmDesc& d) {
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) tiles += d.seg[i].ntiles;
  const uint32_t cus = (uint32_t)cu_count();
  const double bytes = (double)tiles * 16.0 * d.K * (fmt == HQ_FORMAT_INT4 ? 0.5 : 0.25);
  const bool large = bytes >= 24.0 * 1024 * 1024;
  int T = 0, WK = 4;
  long P = 0;
  uint32_t G = 0;
  for (int t : {8, 4, 2}) {
    const uint32_t g = total_slabs(d, t);
    const uint32_t rounds = (g + cus - 1) / cus;
    if (g * 5 >= rounds * cus * 4) {
      T = t;
      P = g;
      break;
    }
  }
  if (T == 0 && tiles >= cus) {
    const uint32_t k = (tiles + 8u * cus - 1u) / (8u * cus);
    const uint32_t g = k * cus;
    const uint32_t wmax = (tiles + g - 1u) / g;
    if ((double)wmax * g <= 1.2 * tiles && wmax >= 2) {
      T = wmax <= 2 ? 2 : (wmax <= 4 ? 4 : 8);
      G = g;
      P = total_slabs(d, T, G);
    }
  }
  if (T == 0 && large) {
    T = 4;
    const uint32_t g = total_slabs(d, 4);
    P = (long)g * std::max<uint32_t>(1, cus / std::max<uint32_t>(1, g));
  }
  if (T == 0) {
    T = tiles >= 16 ? 2 : 1;
    for (int t : {8, 4}) {
      if (total_slabs(d, t) >= 150) {
        T = t;
        break;
      }
    }
    P = total_slabs(d, T);
    if (d.M > 8) WK = 2;
  }
  bool contig = true;
  const int eT = env_int("HQ_DECODE_T", 0);
  if (eT == 1 || eT == 2 || eT == 4 || eT == 8) {
    T = eT;
    G = 0;
    P = total_slabs(d, T);
  }
  const int eG = env_int("HQ_DECODE_G", 0);
  if (eG >= 1) {
    G = (uint32_t)eG;
    P = total_slabs(d, T, G);
  }
  const int eWK = env_int("HQ_DECODE_WK", 0);
  if (eWK >= 1) WK = eWK;
  WK = std::min(WK, max_wk(T));
  const int eP = env_int("HQ_DECODE_P", 0);
  if (eP >= 1) P = eP;
  const char* ec = std::getenv("HQ_DECODE_CONTIG");
  if (ec && *ec) contig = std::atoi(ec) != 0;
  const int eU = env_int("HQ_DECODE_U", 0);  // tuning override: ring depth (T = 8: 2 or 3; T = 4: 3 or 4)
  uint32_t slabs = total_slabs(d, T, G);
  // More slabs than counters: use a grid that never cuts a slab.
  if (slabs > kMaxCounters) {
    G = 0;
    slabs = total_slabs(d, T);
    P = slabs;
  }
  const uint32_t utot = slabs * d.nkb;
  P = std::max(1L, std::min<long>(P, utot));
  DecodeConfig c{T, WK, (int)P, contig, G, eU};
  // Grow the grid (fewer slabs per workgroup) until the per-piece LDS slots fit; with one
  // unit per workgroup a piece needs M * 16 * T floats per wavefront, which always fits.
  while ((uint32_t)c.SK < utot && lds_bytes(d, c, plan_np_max(utot, (uint32_t)c.SK, d.nkb)) > kLdsLimit)
    c.SK = (int)std::min<long>(utot, (long)c.SK * 4 / 3 + 1);
  return c;
}

size_t decode_workspace_bytes(const GemmDesc& d, const DecodeConfig& c) {
  const uint32_t G = total_slabs(d, c.T, c.G);
  if (!plan_has_partial(G, (uint32_t)c.SK)) return 0;
  return kCounterBytes + (size_t)c.SK * 2u * d.M * 16u * c.T * sizeof(float);
}

hipError_t launch_decode(int fmt, int dtype, GemmDesc d, const DecodeConfig& c, void* ws, hipStream_t stream) {
  if (fmt == HQ_FORMAT_INT4) {
    return dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_F16>(d, c, ws, stream)
                                 : launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_BF16>(d, c, ws, stream);
  }
  return dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16>(d, c, ws, stream)
                               : launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_BF16>(d, c, ws, stream);
}

}  // namespace hq

namespace hq {
namespace {

// Padded activation area (whole LDS-DMA instructions) of an X-resident workgroup whose
// piece has the most k-blocks (ceil(nkb / S)).
uint32_t xr_x_bytes(const GemmDesc& d, int S) {
  const uint32_t nkbp = (d.nkb + (uint32_t)S - 1u) / (uint32_t)S;
  return (d.M * nkbp * 16u + 63u) / 64u * 1024u;
}

uint32_t xr_lds_bytes(const GemmDesc& d, int T, int WK, int S, int SG = 1) {
  const uint32_t x = xr_x_bytes(d, S);
  const uint32_t red = (uint32_t)(WK * SG) * d.M * 16u * (uint32_t)T * 4u;
  return std::max(x, red);
}

template <int FMT, int DT, int T, int U, bool GRP = false>
hipError_t xr_launch_t(GemmDesc d, const XrConfig& c, void* ws, hipStream_t stream) {
  if (c.WK < 1 || c.SG < 1 || c.WK * c.SG > xr_max_wk(T) || d.M > 16u || c.S < 1 || (uint32_t)c.S > d.nkb ||
      (c.SG > 1 && (c.S > 1 || !GRP)))
    return hipErrorInvalidValue;
  const uint32_t G = assign_slabs(d, T, c.G);
  const uint32_t GW = (G + (uint32_t)c.SG - 1u) / (uint32_t)c.SG;  // workgroups along x
  XrPlan pl{};
  pl.S = (uint32_t)c.S;
  pl.kq = d.nkb / pl.S;
  pl.kr = d.nkb % pl.S;
  pl.m_lo = plan_div_magic(16u * pl.kq);
  pl.m_hi = plan_div_magic(16u * (pl.kq + 1u));
  pl.gmul = plan_gmul(d.gkb);
  pl.wk = (uint32_t)c.WK;
  pl.sg = (uint32_t)c.SG;
  pl.nslabs = G;
  if (pl.S > 1) {
    if (!ws || G > kMaxCounters) return hipErrorInvalidValue;
    pl.cnt = static_cast<uint32_t*>(ws);
    pl.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  }
  // Byte offsets into X, a slab's weights, Y and the partials are 32-bit buffer or LDS offsets.
  bool fits = G >= 1 && G <= 65535 && (uint64_t)d.M * (uint64_t)d.ldx * 2u < (1ull << 31) && c.lds <= kXrLdsMax &&
              c.lds >= xr_lds_bytes(d, T, c.WK, c.S, c.SG) && (uint64_t)G * pl.S * d.M * 64u * T < (1ull << 31);
  for (uint32_t i = 0; i < d.nseg; ++i)
    fits = fits && (uint64_t)(d.seg[i].slab_w + 1u) * d.nkb * 64u * WTraits<FMT>::wpl * 4u < (1ull << 31);
  if (!fits) return hipErrorInvalidValue;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_decode_xr_kernel<FMT, DT, T, U, false, GRP>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kXrLdsMax) != hipSuccess
          ? hipErrorInvalidConfiguration
          : hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_decode_xr_kernel<FMT, DT, T, U, true, GRP>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kXrLdsMax);
  if (attr != hipSuccess) return attr;
  const dim3 grid(GW, pl.S);
  if (d.nseg > 1)
    hipLaunchKernelGGL((hq_decode_xr_kernel<FMT, DT, T, U, true, GRP>), grid, dim3(64 * c.WK * c.SG), c.lds, stream, d,
                       pl);
  else
    hipLaunchKernelGGL((hq_decode_xr_kernel<FMT, DT, T, U, false, GRP>), grid, dim3(64 * c.WK * c.SG), c.lds, stream,
                       d, pl);
  return hipGetLastError();
}

template <int FMT, int DT>
hipError_t xr_launch_fd(const GemmDesc& d, const XrConfig& c, void* ws, hipStream_t stream) {
  switch (c.T * 10 + c.U) {
    case 82: return xr_launch_t<FMT, DT, 8, 2>(d, c, ws, stream);
    case 42:
      if (c.SG > 1) return xr_launch_t<FMT, DT, 4, 2, true>(d, c, ws, stream);
      return xr_launch_t<FMT, DT, 4, 2>(d, c, ws, stream);
    case 23: return xr_launch_t<FMT, DT, 2, 3>(d, c, ws, stream);
    case 24: return xr_launch_t<FMT, DT, 2, 4>(d, c, ws, stream);
    case 14: return xr_launch_t<FMT, DT, 1, 4>(d, c, ws, stream);
    case 16: return xr_launch_t<FMT, DT, 1, 6>(d, c, ws, stream);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace

// Wavefronts per SIMD the register use of hq_decode_xr_kernel<fmt, T, U> allows (runtime
// occupancy query, cached per device; 4 when there is no device to ask).
static int xr_waves_per_simd(int fmt, int T, int U) {
  const void* f = nullptr;
  const int key = T * 10 + U;
  if (fmt == HQ_FORMAT_INT4) {
    switch (key) {
      case 82: f = reinterpret_cast<const void*>(&hq_decode_xr_kernel<HQ_FORMAT_INT4, HQ_DTYPE_F16, 8, 2, false>); break;
      case 42: f = reinterpret_cast<const void*>(&hq_decode_xr_kernel<HQ_FORMAT_INT4, HQ_DTYPE_F16, 4, 2, false>); break;
      case 23: f = reinterpret_cast<const void*>(&hq_decode_xr_kernel<HQ_FORMAT_INT4, HQ_DTYPE_F16, 2, 3, false>); break;
      default: return 4;
    }
  } else {
    switch (key) {
      case 82: f = reinterpret_cast<const void*>(&hq_decode_xr_kernel<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16, 8, 2, false>); break;
      case 42: f = reinterpret_cast<const void*>(&hq_decode_xr_kernel<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16, 4, 2, false>); break;
      case 23: f = reinterpret_cast<const void*>(&hq_decode_xr_kernel<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16, 2, 3, false>); break;
      default: return 4;
    }
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 4;
  static std::mutex mu;
  static int cached[64][2][9][5] = {};
  std::lock_guard<std::mutex> lock(mu);
  int& c = cached[dev][fmt == HQ_FORMAT_INT4 ? 0 : 1][T][U];
  if (c == 0) {
    int n = 0;  // workgroups of four wavefronts (one per SIMD) per CU, no LDS
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 256, 0) != hipSuccess || n <= 0) n = 4;
    c = std::min(n, 8);
  }
  return c;
}

// Tiling of the X-resident kernel. A workgroup places ceil(WK / 4) wavefronts on each SIMD,
// so it fits on a CU as often as the register use and the LDS both allow. The planner takes
// whole slabs (S = 1: the activation rows of all of K in LDS) and the narrowest slabs
// (T = 2, 4 or 8 tiles; 1 when that gives at most one workgroup per CU and fills at least half
// of them) whose grid fits on the CUs in one round; only when whole slabs of up to
// four rows leave more than half of the CUs idle does it cut K into pieces (S > 1) to fill
// them. When the rows of all of K do not fit in LDS (long K), up to eight rows take the K
// pieces that fill the most CUs in one round; above eight rows those calls stay with the
// lockstep kernel (27648 x 5120, M = 16: six pieces of 8-tile slabs 19.6 us against 17.8; each
// workgroup copies 147 KiB of rows before streaming). Eight wavefronts per workgroup (four with 8-tile slabs), two steps in flight (three
// with 2-tile slabs). Measured on MI355X against the per-wavefront and lockstep kernels
// (graph-timed, weights rotated past the 256 MiB cache): 5120 x 5120 at M = 1..16 5.7-7.1 us
// against 7.5-8.4, 27648 x 5120 at M = 1, 2 15.0-15.8 against 16.8-17.3, ternary 5120 x 27648
// at M = 1 12.3 against 14.1. With wide weights (more tiles than two per CU) and more than
// eight rows the lockstep kernel, which streams each activation k-block through LDS instead of
// copying all of K per workgroup up front, is as fast or faster when the only one-round
// X-resident grid has 8-tile slabs of four wavefronts (5120 x 27648, M = 12 and 16: 17.0-18.5
// us against 17.7-18.8), so the planner leaves those calls to it; one round of 4-tile slabs
// of eight wavefronts wins at any row count (M = 9..16: ternary 5120 x 14336 11.7-12.4 ->
// 8.8-9.1 us, int4 bf16 14.4-14.8 -> 10.2-10.9, 5120 x 10240 and 16384 7-15% faster), and at
// five to eight rows the 4-tile slabs still fit two workgroups per CU and win (M = 5, 8:
// 15.5-16.3 against 16.6-17.7 us; ternary bf16 M = 8: 13.5 against 15.0).
// HQ_XR_T / _WK / _U / _S / _G (slab count) / _SG (slab groups per workgroup) override (tuning and tests).
XrConfig choose_decode_xr(int fmt, const GemmDesc& d, size_t ws_cap) {
  XrConfig c{2, 3, 8, 1, 0, false};
  if (d.M > 16u || d.gen) return c;
  const uint32_t cus = (uint32_t)cu_count();
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) tiles += d.seg[i].ntiles;
  const int eT = env_int("HQ_XR_T", 0), eWK = env_int("HQ_XR_WK", 0), eU = env_int("HQ_XR_U", 0);
  const int eS = env_int("HQ_XR_S", 0), eG = env_int("HQ_XR_G", 0), eSG = env_int("HQ_XR_SG", 0);
  const bool forced = eT || eWK || eU || eS || eG || eSG;
  bool found = false, one_round = false;
  // Few tiles (at most half as many as CUs): one-tile slabs of eight wavefronts, whole or in
  // as many K pieces as keep each wavefront near eight steps (ceil(nkb / 64)), more where the
  // rows need them to fit in LDS, within one workgroup per CU. Measured on MI355X (best of three
  // alternated runs, M = 1..16, int4 and ternary): N = 256..2048 at K = 4096..8192 20-30%
  // faster than 2-tile slabs in two pieces at M <= 4 and 10-20% at M = 8..16 (5120 x 1024
  // M = 1 5.82 -> 4.34 us, 8192 x 1024 M = 8 7.41 -> 6.00), whole slabs ahead of pieces there;
  // K = 27648, N = 512 / 1024: four pieces 7.2 / 8.2 us at M = 1 against 10.0 / 10.2 whole and
  // 10.2 / 10.7 before; K = 14336 M = 16 and K = 8192, N = 2048 M = 16 11-14% ahead of the
  // lockstep kernel.
  if (!forced && 2u * tiles <= cus) {
    const uint32_t s0 = std::min(8u, std::max(1u, (d.nkb + 63u) / 64u));
    for (uint32_t s = s0; s <= 8u && s <= d.nkb && !found; ++s) {
      if (xr_x_bytes(d, (int)s) > kXrLdsMax) continue;
      const uint32_t lds = xr_lds_bytes(d, 1, 8, (int)s);
      const XrConfig cand{1, 4, 8, (int)s, lds, false};
      if (lds > kXrLdsMax || total_slabs(d, 1) * s > cus ||
          (s > 1u && (total_slabs(d, 1) > kMaxCounters || decode_xr_workspace_bytes(d, cand) > ws_cap)))
        break;
      c = cand;
      found = one_round = true;
    }
  }
  // Rows of all of K that do not fit in LDS (long K) at up to eight rows: K pieces, the
  // one-round grid (at most one workgroup per CU) that keeps the most CUs busy, the fewest
  // pieces among equals. Measured on MI355X (alternated runs), 27648 x 5120: M = 4 16.3 us with
  // 4-tile slabs in three pieces (240 workgroups) against 16.8 in two (160); M = 8 17.1 against
  // 17.2 for the lockstep kernel. Ternary weights over a long K (192 k-blocks or more) take the
  // pieces also where the rows fit but 2-tile slabs would leave CUs idle: 27648 x 5120 at M = 1,
  // 2 12.6-12.8 us in three pieces against 13.9-14.2 for 160 whole slabs, 24576 x 5120 at M =
  // 1..3 8-11% faster (int4 2-3% slower; 17408 x 5120 within 2%, shorter K 4-27% slower).
  const bool tern_long = fmt == HQ_FORMAT_TERNARY2 && d.nkb >= 192u && tiles > cus && total_slabs(d, 2) < cus;
  if (!found && !forced && (xr_x_bytes(d, 1) > kXrLdsMax || tern_long) && d.M <= 8u) {
    uint32_t best = 0;
    for (int s = 2; s <= 8; ++s) {
      if ((uint32_t)s > d.nkb || xr_x_bytes(d, s) > kXrLdsMax) continue;
      for (int t : {2, 4, 8}) {
        const int wk = t == 8 ? 4 : 8, u = t == 2 ? 3 : 2;
        const uint32_t lds = xr_lds_bytes(d, t, wk, s);
        const uint32_t wgs = total_slabs(d, t) * (uint32_t)s;
        if (lds > kXrLdsMax || wgs > cus || wgs <= best || total_slabs(d, t) > kMaxCounters) continue;
        const XrConfig cand{t, u, wk, s, lds, false};
        if (decode_xr_workspace_bytes(d, cand) > ws_cap) continue;
        best = wgs;
        c = cand;
      }
    }
    found = one_round = best > 0;
  }
  for (int s = 1; s <= 8 && !found; ++s) {
    if ((uint32_t)s > d.nkb || xr_x_bytes(d, s) > kXrLdsMax || (s > 1 && d.M > 4u)) continue;
    for (int t : {1, 2, 4, 8}) {
      // One-tile slabs only when they give every CU at most one (4096 x 4096, M = 16: 256
      // workgroups, 5.96 against 6.55-6.69 us with 2-tile slabs; with more tiles than CUs,
      // 2-tile slabs measured faster: 5120 x 5120, M = 4: 6.08 against 7.14); fewer tiles than
      // half the CUs took one-tile slabs above.
      if (t == 1 && (tiles > cus || 2u * tiles <= cus || s > 1)) continue;
      // 2-tile slabs two to a CU lose to 4-tile slabs one to a CU (eight wavefronts each).
      // Measured on MI355X (best of three alternated runs, M = 1..8): int4 4096 x 11008 /
      // 12288 / 14336 and 5120 x 13824 5-13% faster (4096 x 11008 M = 1 8.36 -> 7.26 us),
      // ternary 2-12%.
      if (t == 2 && !forced && total_slabs(d, 2) > cus && total_slabs(d, 4) <= cus &&
          xr_lds_bytes(d, 4, 8, s) <= kXrLdsMax && xr_waves_per_simd(fmt, 4, 2) >= 2)
        continue;
      const int wk = t == 8 ? 4 : 8, u = t == 1 ? 4 : t == 2 ? 3 : 2;
      const uint32_t lds = xr_lds_bytes(d, t, wk, s);
      if (lds > kXrLdsMax) continue;
      const uint32_t by_regs = (uint32_t)(xr_waves_per_simd(fmt, t, u) / ((wk + 3) / 4));
      const uint32_t per_cu = std::min(by_regs, kXrLdsMax / lds);
      const uint32_t wgs = total_slabs(d, t) * (uint32_t)s;
      // 4-tile slabs up to one and a half rounds beat 8-tile slabs of four wavefronts in one
      // round. Measured on MI355X (M = 1..8): ternary 5120 x 34816 20.0 -> 16.0 us at M = 1,
      // int4 4096 x 40960 22.8 -> 17.4 us; at 1.7 rounds (5120 x 55296) 8-tile slabs stay
      // ahead from M = 4.
      const bool t4_spill = t == 4 && 2u * wgs <= 3u * cus * per_cu;
      if (per_cu < 1 || (wgs > cus * per_cu && !t4_spill)) continue;
      // Whole slabs leaving more than half of the CUs idle: try a split first.
      if (s == 1 && wgs * 2u < cus && total_slabs(d, t) * 2u <= cus * per_cu && d.nkb >= 2 && d.M <= 4u) break;
      // 4-tile slabs past one round at one or two rows: 2-tile slabs of four wavefronts, when
      // their grid fits in one round. Measured on MI355X: ternary 5120 x 34816 (the decoder's
      // fused gate||up) 15.5-15.7 -> 14.3-14.9 us, 4096 x 40960 13.6-14.1 -> 12.3-12.6; int4
      // 2-8% faster; at four rows, or with 4-tile slabs in one round, no gain.
      if (t == 4 && wgs > cus * per_cu && d.M <= 2u) {
        const uint32_t lds2 = xr_lds_bytes(d, 2, 4, s);
        const uint32_t per2 = std::min((uint32_t)xr_waves_per_simd(fmt, 2, 3), kXrLdsMax / lds2);
        if (lds2 <= kXrLdsMax && total_slabs(d, 2) * (uint32_t)s <= cus * per2) {
          c = XrConfig{2, 3, 4, s, lds2, false};
          found = true;
          one_round = true;
          break;
        }
      }
      c = XrConfig{t, u, wk, s, lds, false};
      found = true;
      one_round = wgs <= cus * per_cu;
      break;
    }
  }
  // Whole 4-tile slabs at up to eight rows, more of them than CUs: four wavefronts (one per
  // SIMD, each streaming twice the k-blocks) instead of eight, when that grid still fits on the
  // CUs in one round. Measured on MI355X (alternated runs): 5120 x 27648 int4 M = 1..8
  // 14.7-16.3 -> 14.2-15.7 us, ternary bf16 11.5-12.6 -> 11.4-11.9; ternary 5120 x 34816 M = 4
  // 16.2 -> 14.9. Past one round it loses (5120 x 34816 at M = 8, 544 slabs on 512 slots: 17.2
  // -> 18.7), and so it does with one slab per CU (4096 x 14336, 224 slabs: 8.26 -> 8.49 us).
  if (!forced && found && c.T == 4 && c.WK == 8 && c.S == 1 && d.M <= 8u && total_slabs(d, 4) > cus) {
    const uint32_t lds4 = xr_lds_bytes(d, 4, 4, 1);
    const uint32_t per4 = std::min((uint32_t)xr_waves_per_simd(fmt, 4, 2), kXrLdsMax / lds4);
    if (lds4 <= kXrLdsMax && per4 >= 1u && total_slabs(d, 4) <= cus * per4) {
      c.WK = 4;
      c.lds = lds4;
    }
  }
  // Groups of whole 4-tile slabs per workgroup (SG groups of four wavefronts over one copy of
  // the rows, SG = the slabs per CU, 2 to 4) when the slabs number more than the CUs: a CU
  // then holds one workgroup instead of SG, each of which would copy the rows, the later
  // copies queued behind the first's weight loads (timestamps: a second workgroup's stream
  // starting up to 2 us later), and the grid fits in one round where single slabs would not.
  // Measured on MI355X (alternated runs, best of two or three). Pairs: 5120 x 27648 int4 M =
  // 1..8 14.4-15.8 -> 14.2-14.9 us, M = 12 and 16 17.0-17.7 -> 15.4-15.9 (against the lockstep
  // kernel), ternary bf16 at M = 16 13.4-13.7 -> 12.4-12.5; 272-352 slabs (N = 17408..22528,
  // K = 4096..8192): int4 M = 1..8 4-25% faster (8192 x 20480 M = 8 24.3 -> 18.3 us), int4 and
  // ternary M = 9..16 14-28% faster than the lockstep kernel. Triples (544-640 slabs, 5120 x
  // 34816 / 40960, 4096 x 40960): int4 M = 4..16 8-27% faster (5120 x 34816 M = 12 25.2 ->
  // 18.4), ternary M = 8..16 13-28%, M = 4 3-4%. Quads (864-896 slabs, 5120 x 55296, 4096 x
  // 57344): 4-15% at M = 1..16, int4 and ternary (ternary M = 1 16.8 -> 15.9 us). Ternary in
  // pairs at up to eight rows, whose steps are bound by their VALU work, keeps all CUs busy
  // instead (5120 x 27648 M = 1: 11.7 -> 12.3 us in pairs; 272-352 slabs within 3%), and in
  // triples below four rows (M = 1: 11.8 -> 12.6 us); so do one or two rows where 2-tile slabs
  // of four wavefronts fit in one round (above; int4 triples no faster there).
  if (!forced && xr_x_bytes(d, 1) <= kXrLdsMax && !(found && (c.T < 4 || c.S > 1))) {
    const uint32_t sl4 = total_slabs(d, 4);
    const uint32_t sg = (sl4 + cus - 1u) / cus;
    const bool rows_ok = fmt == HQ_FORMAT_INT4 || sg >= 4u || (sg == 3u ? d.M >= 4u : d.M > 8u);
    const uint32_t ldsg = xr_lds_bytes(d, 4, 4, 1, (int)sg);
    if (sl4 > cus && sg <= 4u && rows_ok && ldsg <= kXrLdsMax && (uint32_t)xr_waves_per_simd(fmt, 4, 2) >= sg) {
      c = XrConfig{4, 2, 4, 1, ldsg, false};
      c.SG = (int)sg;
      found = one_round = true;
    }
  }
  // Wide weights at more than eight rows: the lockstep kernel unless one round of slabs of at
  // most four tiles (eight wavefronts) fits.
  const bool wide_rows = tiles > 2u * cus && d.M > 8u && (c.T > 4 || !one_round) && c.SG == 1;
  if (!forced && (!found || wide_rows)) return c;
  if (eT == 1 || eT == 2 || eT == 4 || eT == 8) c.T = eT;
  if (eWK >= 1) c.WK = eWK;
  if (eU >= 2) c.U = eU;
  if (eS >= 1) c.S = eS;
  if (eG >= 1) c.G = (uint32_t)eG;
  if (eSG >= 1) c.SG = eSG;
  // Snap to an instantiated (T, U).
  if (c.T == 8) c.U = 2;
  if (c.T == 4) c.U = 2;
  if (c.T == 2) c.U = std::min(std::max(c.U, 3), 4);
  if (c.T == 1) c.U = c.U >= 6 ? 6 : 4;
  c.WK = std::max(1, std::min(c.WK, xr_max_wk(c.T)));
  c.SG = std::max(1, std::min(c.SG, xr_max_wk(c.T) / c.WK));
  if (c.S > 1 || c.T != 4) c.SG = 1;  // slab groups: whole 4-tile slabs only
  c.S = std::max(1, std::min<int>(c.S, (int)d.nkb));
  if (c.G && total_slabs(d, c.T, c.G) > 65535u) return c;
  if (c.S > 1 && (total_slabs(d, c.T, c.G) > kMaxCounters || decode_xr_workspace_bytes(d, c) > ws_cap)) return c;
  c.lds = xr_lds_bytes(d, c.T, c.WK, c.S, c.SG);
  c.ok = c.lds <= kXrLdsMax;
  return c;
}

size_t decode_xr_workspace_bytes(const GemmDesc& d, const XrConfig& c) {
  if (c.S <= 1) return 0;
  return kCounterBytes + (size_t)total_slabs(d, c.T, c.G) * (size_t)c.S * d.M * 16u * (size_t)c.T * 4u;
}

hipError_t launch_decode_xr(int fmt, int dtype, GemmDesc d, const XrConfig& c, void* ws, hipStream_t stream) {
  if (fmt == HQ_FORMAT_INT4) {
    return dtype == HQ_DTYPE_F16 ? xr_launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_F16>(d, c, ws, stream)
                                 : xr_launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_BF16>(d, c, ws, stream);
  }
  return dtype == HQ_DTYPE_F16 ? xr_launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16>(d, c, ws, stream)
                               : xr_launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_BF16>(d, c, ws, stream);
}

}  // namespace hq

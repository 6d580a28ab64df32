// hq_decode.hip — memory-bound qGEMM for M <= 16 (decode), gfx950.
//
// Replaces kernel_marlin_gemm_int4_templated / _dynamic
// (hydrogen/src/model/marlin_gemm.cu:130-237, 242-322). The reference gives each
// thread one output column and does 32 x M scalar FMAs per 16-byte weight load,
// then merges 16 fixed K-splits with fp32 atomics into a pre-zeroed Y. Here:
//   * the work is cut into units of (slab of T column tiles) x (128-deep k-block) and
//     every workgroup streams an equal contiguous range of units (hq_plan.hpp), so all
//     CUs finish together whatever N and K are; slabs cut by a range boundary are
//     completed by a last-arriver fix-up through the workspace, in workgroup order;
//   * inside a workgroup the WK wavefronts take the units of each slab in turn
//     (unit j -> wavefront j mod WK), each with U k-blocks of weights, scales and
//     activations in flight in a register ring, and meet only once, at the end, to sum
//     their per-slab results through LDS in wavefront order;
//   * weights are dequantised in registers straight into MFMA B fragments and
//     multiplied against the activation rows (M padded to 16) with
//     v_mfma_f32_16x16x32_{f16,bf16}. int4 uses the biased form (magic + q, one
//     v_and_or_b32 per fragment word) and removes the bias with one extra MFMA per
//     chunk whose result seeds every tile's accumulator;
//   * the group scale multiplies the fp32 k-block sum once per (column, k-block).
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
  // A operand: row c16 of X, k-slice g4 of each chunk; rows >= M read as zero (activation
  // and scale loads past the wavefront's units re-read cached data and are discarded).
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(d.X, M * (uint32_t)d.ldx * 2u);
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
    const __amdgpu_buffer_rsrc_t lx = xr;
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

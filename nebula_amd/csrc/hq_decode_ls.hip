// hq_decode_ls.hip — memory-bound qGEMM for M <= 80 (decode and split-fuse steps), gfx950:
// lockstep slabs.
//
// Replaces kernel_marlin_gemm_int4_templated / _dynamic
// (hydrogen/src/model/marlin_gemm.cu:130-237, 242-322): the reference gives each thread
// one output column and does 32 x M scalar FMAs per 16-byte weight load, then merges 16
// fixed K-splits with fp32 atomics into a pre-zeroed Y.
//
// Here a workgroup owns a slab of up to 4 * T column tiles (16 columns each) and a
// contiguous range of 128-deep k-blocks ("piece"); a slab's k-blocks are split over S
// workgroups (S = 1 for wide weights). With more slabs than CUs (several row tiles, or int4
// weights of up to 1.25 slabs per CU at one row tile), a balanced grid gives every workgroup
// an equal run of (slab, k-block) units instead: whole slabs in the middle, its first and last
// slab shared with a neighbour (fix-up as below). The activation rows come in MT tiles of 16 rows
// (M <= 16 MT): every dequantised weight fragment feeds all MT row tiles. The workgroup has KG k-groups of four wavefronts; wavefront i
// of every k-group streams tiles T i .. T i + T - 1 of the slab, and at step q k-group kg
// takes k-block q * KG + kg of the piece, so the KG k-groups split K inside the CU and
// meet once, at the end, in LDS. The four wavefronts of a k-group walk its k-blocks in
// lockstep, each streaming its T tiles (1 KiB per tile and k-block, int4) from HBM into
// a register ring U steps deep. The activation k-block (M rows x 256 B) is fetched once
// per k-group (each wavefront loads four rows, full 128-byte lines) and shared through
// LDS, so activation traffic is 1/(4 T) of a per-wavefront fetch; its 16-byte pieces are
// XOR-swizzled by row so the MFMA A-fragment reads (ds_read_b128) are bank-conflict free.
// Each step's loads are issued before the barrier that publishes the step's activations,
// so the HBM stream never waits on the barrier.
//
// Hot-loop memory operations are inline asm: the compiler would otherwise re-order the
// loads against the explicit wait counts and drain the ring at every barrier. Each use is
// preceded by an explicit s_waitcnt tied to the registers it covers, so no instruction
// reads a register whose load is in flight.
//
// Weights are dequantised in registers straight into v_mfma_f32_16x16x32 B fragments:
// int4 in the biased form magic + q (one v_and_or_b32 per fragment word), with the bias
// removed by a correction MFMA that seeds every tile's k-block sum; the fp16 group scale
// multiplies the fp32 k-block sum (int4 with several fp16 row tiles: exact q - 8 instead of
// the correction; at five row tiles the scale is folded into the fragment). Pieces of a
// split slab are summed in piece order by the last workgroup to finish (arrival counter),
// so results are deterministic.
//
// General kernels (GEN): one scale per 32-wide k chunk (groups that are multiples of 32, not
// of 128) and an optional fp32 per-group bias, the reference's w = q * s + b
// (marlin_gemm.cu:195-196). With e = 8 s + b (the weight of code 8) the chunk's contribution
// is s * sum x (q - 8) + e * sum x: the first term is the fast kernels' (per chunk), the
// second a row sum of the chunk (one MFMA against a fragment of ones) times e. Without a bias
// e is 0, and so is e for a bias of exactly -8 s: such calls give the same bits.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <utility>

#include "hq_device.hpp"
#include "hq_internal.hpp"
#include "hq_plan.hpp"

namespace hq {
namespace {

// ---- inline-asm memory operations of the hot loop (see the header comment) ----
__device__ __forceinline__ u4 ls_load_b128_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  u4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen nt" : "=v"(v) : "v"(voff), "s"(r), "s"(soff));
  return v;
}
__device__ __forceinline__ u2 ls_load_b64_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  u2 v;
  asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen nt" : "=v"(v) : "v"(voff), "s"(r), "s"(soff));
  return v;
}
__device__ __forceinline__ uint32_t ls_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  uint32_t v;
  asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff));
  return v;
}
__device__ __forceinline__ uint32_t ls_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff));
  return v;
}
__device__ __forceinline__ u4 ls_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  u4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(r), "s"(soff));
  return v;
}
// 16 bytes to LDS at addr + OFF (the instruction's 16-bit offset field): one address register
// serves several writes.
template <uint32_t OFF>
__device__ __forceinline__ void ls_lds_write_b128_at(uint32_t addr, const u4& v) {
  static_assert(OFF < 65536u, "ds offset field");
  asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(addr), "v"(v), "i"(OFF) : "memory");
}
// Ring slot v[0 .. XL) of activation loads to addr + 1024 x.
template <int... X>
__device__ __forceinline__ void ls_lds_write_rows(uint32_t addr, const u4* v, std::integer_sequence<int, X...>) {
  (ls_lds_write_b128_at<1024u * X>(addr, v[X]), ...);
}
__device__ __forceinline__ u4 ls_lds_read_b128(uint32_t addr) {
  u4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ void ls_lds_add_u32(uint32_t addr, uint32_t v) {
  asm volatile("ds_add_u32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t ls_lds_read_u32_sync(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t ls_bpermute(uint32_t byte_lane, uint32_t v) {
  uint32_t r;
  asm volatile("ds_bpermute_b32 %0, %1, %2" : "=v"(r) : "v"(byte_lane), "v"(v));
  return r;
}

// Biased fp16 int4 fragment (words 1024 + q, 64 + q, 1024 + q, 64 + q) -> exact q - 8.
__device__ __forceinline__ u4 unbias_f16(const u4& f) {
  const h2 c1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 c72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  return u4{h2_bits(bits_h2(f[0]) + c1032), h2_bits(bits_h2(f[1]) + c72), h2_bits(bits_h2(f[2]) + c1032),
            h2_bits(bits_h2(f[3]) + c72)};
}

template <int FMT>
struct LsW;
template <>
struct LsW<HQ_FORMAT_INT4> {
  using V = u4;
  static constexpr uint32_t kLaneBytes = 16;
};
template <>
struct LsW<HQ_FORMAT_TERNARY2> {
  using V = u2;
  static constexpr uint32_t kLaneBytes = 8;
};

constexpr uint32_t kStageBytes = 4096;  // one activation k-block: 16 rows x 256 B
constexpr uint32_t kMaxPieces = 8;      // largest K split of a slab (pieces summed by the last one)

// Waits, and ties registers to them: an empty asm that "rewrites" a register after the
// wait keeps every instruction that reads it below the wait.
template <int N>
__device__ __forceinline__ void ls_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N));
}
__device__ __forceinline__ void ls_wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)"); }
__device__ __forceinline__ void ls_tie(u4& a) { asm volatile("" : "+v"(a)); }
__device__ __forceinline__ void ls_tie(u2& a) { asm volatile("" : "+v"(a)); }
__device__ __forceinline__ void ls_tie(uint32_t& a) { asm volatile("" : "+v"(a)); }

template <int FMT, int DT, int KG, int GW, int T, int U, int MT, bool FUSED, bool GEN, bool BAL = false>
__global__ void __launch_bounds__(64 * KG * GW, KG == 1 && MT > 1 ? 2 : 1)
    hq_decode_ls_kernel(const GemmDesc d, const LsPlan pl) {
  static_assert(!BAL || (KG > 1 && !GEN), "the balanced grid is for the fast kernels with two k-groups");
  static_assert(KG == 1 || KG == 2 || KG == 4, "one, two or four k-groups");
  static_assert(GW == 2 || GW == 4, "k-groups of two or four wavefronts");
  static_assert(T >= 1 && T <= 4, "the scale load covers at most four tiles");
  static_assert(MT >= 1 && MT <= 5 && (4 * MT) % GW == 0, "one to five 16-row tiles, whole loads per wavefront");
  using WV = typename LsW<FMT>::V;
  constexpr uint32_t kLaneBytes = LsW<FMT>::kLaneBytes;
  constexpr uint32_t kBlockBytes = 64u * kLaneBytes;  // one tile x one k-block
  constexpr bool kInt4 = FMT == HQ_FORMAT_INT4;
  // Several row tiles with fp16 activations: int4 fragments are dequantised exactly to q - 8
  // (four v_pk_add_f16 per fragment) instead of carrying the bias into a correction MFMA,
  // which would be a third of the MFMAs of a row tile. Measured on MI355X (5120 x 27648 and
  // 27648 x 5120, M = 24..80): 5-11% faster. One row tile keeps the biased form (fewer VALU
  // instructions in the memory-bound case); bf16 has no packed add on gfx950.
  constexpr bool kUnbiased = kInt4 && DT == HQ_DTYPE_F16 && MT > 1;
  // Five row tiles of int4 with fp16 activations: the group scale is folded into the
  // dequantised fragment (one v_pk_mul_f16 per fragment word; (q - 8) s rounds to fp16, as in
  // the prefill kernel), so the MFMAs accumulate straight into the result across k-blocks and
  // the per-k-block sums (40 VGPRs) that would not fit beside the fragments are not needed.
  // Measured on MI355X (5120 x 27648, M = 80): 36.2 -> 35.0 us. With fewer row tiles, or
  // ternary weights, scaling each k-block's sums in fp32 measured as fast or faster (one
  // v_pk_mul_f16 per fragment word against MT x T x 4 FMAs per k-block).
  constexpr bool kFold = !GEN && DT == HQ_DTYPE_F16 && kInt4 && MT == 5;
  // Several row tiles: every A fragment of a k-block is read before the first wait, and the
  // weight fragments are dequantised while those reads are in flight (a wait per row tile
  // left the LDS latency exposed MT times per step). Measured on MI355X: ternary 5120 x 34816
  // at M = 80 61.4 -> 52.9 us, 5120 x 14336 31.6 -> 28.6 us. Not for int4 bf16 at five row
  // tiles, whose correction chains would not fit in 256 VGPRs beside the fragments.
  constexpr bool kAllA = !GEN && MT > 1 && (kFold || !kInt4 || MT <= 4) && !(BAL && (MT == 5 || (kInt4 && DT == HQ_DTYPE_BF16 && MT == 4)));
  // Ternary fragments from 64-bit shifts of the word pair (dq_tern2_pair) up to three row
  // tiles, and at four outside the balanced grid; beyond, the register pairs the shifts need
  // made the kernel spill.
  constexpr bool kPairTern = !kInt4 && (MT <= 3 || (MT == 4 && !BAL));
  // The register ring holds U steps in flight plus the one being consumed. Activations
  // are staged through two LDS stages: a stage is written just before the barrier of its
  // step and rewritten two steps later, after every wavefront has passed the next barrier
  // (and so finished reading it). A stage holds one k-block per k-group.
  constexpr int R = U + 1;
  constexpr int NS = 2;
  constexpr int XL = 4 * MT / GW;   // activation loads (four rows each) per wavefront and step
  // Loads per wavefront and step: activation rows, T tiles, scales (GEN: T scale and T bias loads).
  constexpr int PER = XL + T + (GEN ? 2 * T : 1);
  constexpr uint32_t kXStage = MT * kStageBytes;  // one k-group's activation k-block: 16 MT rows
  constexpr uint32_t kStep = KG * kXStage;
  static_assert((KG - 1) * GW * T * MT * 1024 <= NS * kStep, "the k-group reduction reuses the activation stages");
  __shared__ __attribute__((aligned(16))) char xs[NS * kStep];
  __shared__ uint32_t sh_last;
  __shared__ uint32_t sh_tail[2];  // balanced grid: last contributor of the first / last slab
  __shared__ uint32_t kg_arrived[KG];  // per k-group arrival count (k-group barrier)

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wi = wave % GW, kg = wave / GW;  // wavefront within its k-group, k-group
  const uint32_t c16 = lane & 15u, g4 = lane >> 4;
  const uint32_t nkb = d.nkb;
  const uint32_t M = d.M;
  const uint32_t piece = BAL ? 0u : blockIdx.x;  // grid (S, G); balanced grid (P)
  // Pieces of this workgroup. S-piece grid: one, slab blockIdx.y, k-blocks of piece blockIdx.x.
  // Balanced grid: the slabs gfirst .. glast of the units [u0, u1), in order; the first and the
  // last may be partial (workspace slots 0 and 1), summed by the last contributor to arrive.
  uint32_t u0 = 0, u1 = 0, gfirst = 0, glast = 0, npieces = 1;
  if constexpr (BAL) {
    u0 = plan_begin(pl.bL, pl.brem, blockIdx.x);
    u1 = plan_begin(pl.bL, pl.brem, blockIdx.x + 1u);
    gfirst = plan_div(u0, nkb, pl.nkb_m);
    glast = plan_div(u1 - 1u, nkb, pl.nkb_m);
    npieces = glast - gfirst + 1u;
  }
  uint32_t arrivals = 0;  // k-group barrier count, across pieces
  for (uint32_t pi = 0; pi < npieces; ++pi) {
  const uint32_t g = BAL ? gfirst + pi : blockIdx.y;

  // Segment of slab g, and its fields, read once (a reference into the kernel arguments
  // would be re-read from memory inside the loop). A one-segment call (FUSED = false) reads
  // all its arguments in one round of scalar loads (0.25 us per launch, measured); a fused
  // call looks its segment up first.
  const uint32_t* sWp = d.seg[0].Wp;
  const uint16_t* sS = d.seg[0].S;
  const float* sB = d.seg[0].B;
  void* sY = d.seg[0].Y;
  uint32_t sN = d.seg[0].N, sLds = d.seg[0].lds, sNt = d.seg[0].ntiles;
  uint32_t sLdy = (uint32_t)d.seg[0].ldy, sBegin = d.seg[0].blk_begin;
  if constexpr (FUSED) {
    uint32_t si = 0;
    for (uint32_t i = 1; i < d.nseg; ++i)
      if (g >= d.seg[i].blk_begin) si = i;
    si = __builtin_amdgcn_readfirstlane(si);
    sWp = d.seg[si].Wp;
    sS = d.seg[si].S;
    sB = d.seg[si].B;
    sY = d.seg[si].Y;
    sN = d.seg[si].N;
    sLds = d.seg[si].lds;
    sNt = d.seg[si].ntiles;
    sLdy = (uint32_t)d.seg[si].ldy;
    sBegin = d.seg[si].blk_begin;
  }
  // First tile of this wavefront, and how many of its T tiles it owns (the slab may be
  // narrower than GW * T tiles, and the segment's last slab narrower still).
  const uint32_t ctw = (g - sBegin) * pl.sw + wi * T;
  const uint32_t own = wi * T < pl.sw ? min((uint32_t)T, pl.sw - wi * T) : 0u;
  const uint32_t ntw = ctw < sNt ? min(own, sNt - ctw) : 0u;
  const uint32_t srow2 = sLds * 2u;  // bytes per scale row
  // k-blocks [ka, kz) of this piece; at step q k-group kg takes k-block ka + q * KG + kg.
  const uint32_t ka = !BAL ? piece * pl.kq + min(piece, pl.kr) : (pi == 0u ? u0 - gfirst * nkb : 0u);
  const uint32_t kz = !BAL ? ka + pl.kq + (piece < pl.kr ? 1u : 0u) : (g == glast ? u1 - glast * nkb : nkb);

  // Weights: tile t of this wavefront at t * nkb blocks; missing tiles read zero.
  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(reinterpret_cast<const char*>(sWp) + (size_t)min(ctw, sNt) * nkb * kBlockBytes,
                ntw * nkb * kBlockBytes);
  uint32_t wvo[T];
#pragma unroll
  for (int t = 0; t < T; ++t) wvo[t] = lane * kLaneBytes + (uint32_t)t * nkb * kBlockBytes;
  // Scales: lane l loads column 16 (ctw + l / 16) + l % 16 (clamped to N - 1). GEN: scale load
  // t (and bias load t) gives lane l tile t's column 16 (ctw + t) + l % 16 in chunk l / 16.
  const uint32_t srows = GEN ? 4u * nkb / d.g32 : nkb / d.gkb;  // scale (and bias) rows
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(sS, ((srows - 1u) * sLds + sN) * 2u);
  const uint32_t svo = min((ctw + min(g4, (uint32_t)T - 1u)) * 16u + c16, sN - 1u) * 2u;
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(sB, GEN && sB ? ((srows - 1u) * sLds + sN) * 4u : 0u);
  uint32_t gvo[GEN ? T : 1];
#pragma unroll
  for (int t = 0; t < (GEN ? T : 1); ++t) gvo[t] = min((ctw + t) * 16u + c16, sN - 1u);
  // Activations: load x of this wavefront covers rows 4 (XL wi + x) + lane / 16 of its
  // k-group's k-block; lane l holds the 16-byte piece (l % 16) ^ row of its row's 256
  // bytes (rows >= M read zero) and writes it to LDS at row * 256 + 16 * (l % 16) of the
  // k-group's stage slot.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(d.X, M * (uint32_t)d.ldx * 2u);
  const uint32_t xs0 = (uint32_t)(uintptr_t)xs + kg * kXStage;
  uint32_t xvo[XL];
#pragma unroll
  for (int x = 0; x < XL; ++x) {
    const uint32_t xrow = 4u * (XL * wi + x) + g4;
    xvo[x] = xrow < M ? xrow * (uint32_t)d.ldx * 2u + ((c16 ^ (xrow & 15u)) * 16u) : kOutOfRange;
  }
  // LDS address of load x: xwo + x * 1024 (the write's offset field carries x * 1024).
  const uint32_t xwo = xs0 + XL * wi * 1024u + lane * 16u;
  // A fragment of row tile r, chunk c: row 16 r + c16, 16-byte piece 4c + g4, at
  // r * 4096 + c16 * 256 + 16 * (piece ^ c16).
  uint32_t xro[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xro[c] = xs0 + c16 * 256u + 16u * ((4u * c + g4) ^ c16);

  WV wring[R][T];
  uint32_t sring[R][GEN ? T : 1];
  uint32_t bring[R][GEN ? T : 1];
  u4 xring[R][XL];
  // Loads of ring slot `slot` for step q (past the piece: zero reads).
  auto issue = [&](int slot, uint32_t q) {
    const uint32_t kb = ka + q * KG + kg;
    const bool live = kb < kz;
    const uint32_t kbu = __builtin_amdgcn_readfirstlane(live ? kb : 0u);
#pragma unroll
    for (int x = 0; x < XL; ++x) xring[slot][x] = ls_load_b128(xr, live ? xvo[x] : kOutOfRange, kbu * 256u);
    const uint32_t kbo = kbu * kBlockBytes;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if constexpr (kInt4) wring[slot][t] = ls_load_b128_nt(wr, live ? wvo[t] : kOutOfRange, kbo);
      else wring[slot][t] = ls_load_b64_nt(wr, live ? wvo[t] : kOutOfRange, kbo);
    }
    if constexpr (GEN) {
      // Chunk g4 of k-block kb: scale row (4 kb + g4) / g32, per lane.
      const uint32_t row = plan_div(4u * kbu + g4, d.g32, d.g32_m);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        sring[slot][t] = ls_load_u16(srs, live ? row * srow2 + gvo[t] * 2u : kOutOfRange, 0u);
        bring[slot][t] = ls_load_b32(brs, live ? row * (srow2 * 2u) + gvo[t] * 4u : kOutOfRange, 0u);
      }
    } else {
      sring[slot][0] = ls_load_u16(srs, live ? svo : kOutOfRange,
                                   __builtin_amdgcn_readfirstlane(plan_group_of_kb(kbu, pl.gmul) * srow2));
    }
  };

  f4 acc[MT][T];
#pragma unroll
  for (int r = 0; r < MT; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[r][t] = f4{0.f, 0.f, 0.f, 0.f};
  const DqBiasConst dqb = DT == HQ_DTYPE_F16 ? dq_bias_const_f16() : dq_bias_const_bf16();
  const u4 corr_b = int4_corr_fragment<DT>();
  const uint32_t one2 = DT == HQ_DTYPE_F16 ? 0x3C003C00u : 0x3F803F80u;  // 1.0 in both halves
  const u4 ones = u4{one2, one2, one2, one2};
  const bool has_bias = GEN && sB != nullptr;

  // Several row tiles (kAllA): the k-block's A fragments, read at once.
  auto compute_all = [&](int slot, uint32_t stage) {
    if constexpr (kAllA) {
      const uint32_t so = stage * kStep;
      u4 xa[MT][4];
#pragma unroll
      for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) xa[r][c] = ls_lds_read_b128(xro[c] + so + (uint32_t)r * kStageBytes);
      uint32_t sbt[T];
#pragma unroll
      for (int t = 0; t < T; ++t) sbt[t] = T == 1 ? sring[slot][0] : ls_bpermute((16u * t + c16) * 4u, sring[slot][0]);
      // Dequantisation (VALU) while the LDS reads are in flight.
      u4 bq[4][T];
      if constexpr (kInt4) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int t = 0; t < T; ++t) {
            bq[c][t] = dq_int4_biased<DT>(wring[slot][t][c], dqb);
            if constexpr (kUnbiased) bq[c][t] = unbias_f16(bq[c][t]);
          }
      } else if constexpr (kPairTern) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint64_t v = tern2_words(wring[slot][t][0], wring[slot][t][1]);
          dq_tern2_pair<0>(v, bq[0][t], bq[2][t]);
          dq_tern2_pair<1>(v, bq[1][t], bq[3][t]);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const uint32_t word = wring[slot][t][c >> 1];
            bq[c][t] = (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);
          }
      }
      ls_wait_lgkmcnt0();
#pragma unroll
      for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) ls_tie(xa[r][c]);
#pragma unroll
      for (int t = 0; t < T; ++t) ls_tie(sbt[t]);
      if constexpr (kFold) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint32_t s = sbt[t] & 0xFFFFu;
          const h2 s2 = bits_h2(s | (s << 16));
#pragma unroll
          for (int c = 0; c < 4; ++c)
            bq[c][t] = u4{h2_bits(bits_h2(bq[c][t][0]) * s2), h2_bits(bits_h2(bq[c][t][1]) * s2),
                          h2_bits(bits_h2(bq[c][t][2]) * s2), h2_bits(bits_h2(bq[c][t][3]) * s2)};
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < MT; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = mfma16x16x32<DT>(xa[r][c], bq[c][t], acc[r][t]);
      } else {
        float scf[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          scf[t] = f16_to_f32((uint16_t)sbt[t]);
          if constexpr (!kInt4) scf[t] = __builtin_isfinite(scf[t]) ? 0.5f * scf[t] : 0.0f;  // fields hold 2t
        }
        f4 corr[MT], gs[MT][T];
#pragma unroll
        for (int r = 0; r < MT; ++r) {
          corr[r] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < T; ++t) gs[r][t] = f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < MT; ++r) {
            if constexpr (kInt4 && !kUnbiased) corr[r] = mfma16x16x32<DT>(xa[r][c], corr_b, corr[r]);
#pragma unroll
            for (int t = 0; t < T; ++t) gs[r][t] = mfma16x16x32<DT>(xa[r][c], bq[c][t], gs[r][t]);
          }
#pragma unroll
        for (int r = 0; r < MT; ++r)
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[r][t][v] =
                  __builtin_fmaf(kInt4 && !kUnbiased ? gs[r][t][v] + corr[r][v] : gs[r][t][v], scf[t], acc[r][t][v]);
      }
    }
  };
  auto compute = [&](int slot, uint32_t stage) {
    const uint32_t so = stage * kStep;
    uint32_t sb[T];
    uint32_t gsb[GEN ? T : 1][4], gbb[GEN ? T : 1][4];  // GEN: scale / bias bits of (tile, chunk)
    if constexpr (GEN) {
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          gsb[t][c] = ls_bpermute((16u * c + c16) * 4u, sring[slot][t]);
          gbb[t][c] = ls_bpermute((16u * c + c16) * 4u, bring[slot][t]);
        }
    } else {
#pragma unroll
      for (int t = 0; t < T; ++t) sb[t] = T == 1 ? sring[slot][0] : ls_bpermute((16u * t + c16) * 4u, sring[slot][0]);
    }
    // The weight fragments of the k-block, dequantised once and used by every row tile.
    u4 bf[4][T];
    if constexpr (kInt4) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) {
          bf[c][t] = dq_int4_biased<DT>(wring[slot][t][c], dqb);
          if constexpr (kUnbiased) bf[c][t] = unbias_f16(bf[c][t]);
        }
    } else if constexpr (kPairTern) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint64_t v = tern2_words(wring[slot][t][0], wring[slot][t][1]);
        dq_tern2_pair<0>(v, bf[0][t], bf[2][t]);
        dq_tern2_pair<1>(v, bf[1][t], bf[3][t]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint32_t word = wring[slot][t][c >> 1];
          bf[c][t] = (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);
        }
    }
    float sc[T];
    float gs_[GEN ? T : 1][4], ge_[GEN ? T : 1][4];  // GEN: scale and e = 8 s + b of (tile, chunk)
    if constexpr (GEN) {
      // The scale and bias bits become floats before the row tiles: the permuted bits then die
      // (at five row tiles of bf16 they kept the kernel two registers past 256).
      ls_wait_lgkmcnt0();
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          ls_tie(gsb[t][c]);
          ls_tie(gbb[t][c]);
          float sv = f16_to_f32((uint16_t)gsb[t][c]);
          if constexpr (!kInt4) sv = __builtin_isfinite(sv) ? 0.5f * sv : 0.0f;  // fields hold 2t
          gs_[t][c] = sv;
          ge_[t][c] = has_bias ? __builtin_fmaf(8.0f, sv, __builtin_bit_cast(float, gbb[t][c])) : 0.0f;
        }
    }
#pragma unroll
    for (int r = 0; r < MT; ++r) {
      u4 xf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) xf[c] = ls_lds_read_b128(xro[c] + so + (uint32_t)r * kStageBytes);
      ls_wait_lgkmcnt0();
#pragma unroll
      for (int c = 0; c < 4; ++c) ls_tie(xf[c]);
      if constexpr (GEN) {
        // Per chunk: the tiles' sums x (q - 8) (or x 2t), scaled, and the row sum times e.
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          f4 cc = f4{0.f, 0.f, 0.f, 0.f};
          if constexpr (kInt4 && !kUnbiased) cc = mfma16x16x32<DT>(xf[c], corr_b, cc);
          const f4 rs = mfma16x16x32<DT>(xf[c], ones, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const f4 g = mfma16x16x32<DT>(xf[c], bf[c][t], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[r][t][v] = __builtin_fmaf(kInt4 && !kUnbiased ? g[v] + cc[v] : g[v], gs_[t][c], acc[r][t][v]);
              acc[r][t][v] = __builtin_fmaf(rs[v], ge_[t][c], acc[r][t][v]);
            }
          }
        }
        continue;
      }
      if (r == 0) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          ls_tie(sb[t]);
          sc[t] = f16_to_f32((uint16_t)sb[t]);
          if constexpr (!kInt4) sc[t] = __builtin_isfinite(sc[t]) ? 0.5f * sc[t] : 0.0f;  // fields hold 2t; non-finite drops
        }
      }
      // Independent accumulation chains: one per tile and (int4) one for the bias
      // correction -sum x (magic + 8), added after the chunk loop.
      f4 corr = f4{0.f, 0.f, 0.f, 0.f}, gs[T];
#pragma unroll
      for (int t = 0; t < T; ++t) gs[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if constexpr (kInt4 && !kUnbiased) corr = mfma16x16x32<DT>(xf[c], corr_b, corr);
#pragma unroll
        for (int t = 0; t < T; ++t) gs[t] = mfma16x16x32<DT>(xf[c], bf[c][t], gs[t]);
      }
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          acc[r][t][v] = __builtin_fmaf(kInt4 && !kUnbiased ? gs[t][v] + corr[v] : gs[t][v], sc[t], acc[r][t][v]);
    }
  };

  // Prologue: steps 0 .. U - 1 into slots 0 .. U - 1.
#pragma unroll
  for (int u = 0; u < U; ++u) issue(u, u);
  const uint32_t nsteps = (kz - ka + KG - 1) / KG;
  // The k-groups synchronise separately, so the wavefronts sharing a SIMD (one per
  // k-group) drift apart and hide each other's waits. A k-group barrier is an LDS
  // arrival count: each wavefront adds one after writing its activation rows (LDS
  // executes a wavefront's operations in order) and waits until all four have arrived.
  // The wait is bounded: every wavefront executes the same steps, so the bound is never
  // reached by a correct launch, and a wrong one cannot hang the GPU. A wavefront that gives
  // up sets the host-visible fault word (the host reports it as HQ_ERR_DEVICE) and carries
  // on, so every wavefront still reaches the end of the kernel.
  const uint32_t arr = (uint32_t)(uintptr_t)&kg_arrived[kg];
  const uint32_t arr_next = (uint32_t)(uintptr_t)&kg_arrived[(kg + 1u) % KG];
  if constexpr (KG > 1) {
    if (pi == 0u) {  // uniform
      if (threadIdx.x < (uint32_t)KG) kg_arrived[threadIdx.x] = 0;
      __syncthreads();
    }
  }
  auto kgroup_barrier = [&]() {
    if constexpr (KG == 1) {
      ls_wait_lgkmcnt0();
      __builtin_amdgcn_s_barrier();
    } else {
      arrivals += GW;
      if (lane == 0) ls_lds_add_u32(arr, 1u);
      bool met = false;
      for (uint32_t spin = 0; spin < pl.spin; ++spin) {
        if (__builtin_amdgcn_readfirstlane(ls_lds_read_u32_sync(arr)) >= arrivals) {
          met = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!met && lane == 0 && pl.fault)
        __hip_atomic_store(pl.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      // The SIMD arbiter favours older wavefronts, which would let k-group 0 run ahead
      // and leave k-group 1 streaming alone at the end: a k-group behind the one after
      // it (cyclically) raises its issue priority until it catches up.
      const uint32_t other = __builtin_amdgcn_readfirstlane(ls_lds_read_u32_sync(arr_next));
      if (other > arrivals) __builtin_amdgcn_s_setprio(2);
      else __builtin_amdgcn_s_setprio(0);
    }
  };
  uint32_t st = 0;  // LDS stage of step q
  for (uint32_t i = 0; i < nsteps; i += R) {
#pragma unroll
    for (int s = 0; s < R; ++s) {
      if (i + s < nsteps) {  // uniform; every step issues the same loads
        ls_wait_vmcnt<(U - 1) * PER>();  // this wavefront's loads of step i + s have landed
#pragma unroll
        for (int t = 0; t < T; ++t) ls_tie(wring[s][t]);
    #pragma unroll
        for (int t = 0; t < (GEN ? T : 1); ++t) {
          ls_tie(sring[s][t]);
          if constexpr (GEN) ls_tie(bring[s][t]);
        }
#pragma unroll
        for (int x = 0; x < XL; ++x) ls_tie(xring[s][x]);
        issue((s + U) % R, i + s + U);
        ls_lds_write_rows(xwo + st * kStep, xring[s], std::make_integer_sequence<int, XL>{});
        kgroup_barrier();  // every wavefront's activation rows of step i + s are in LDS
        if constexpr (kAllA) compute_all(s, st);
        else compute(s, st);
        st ^= 1u;
      }
    }
  }
  // The ring's trailing loads (past the piece) are still in flight and their results are
  // never used: tie every ring register to the final wait, or the compiler would reuse
  // those registers for the epilogue while the loads can still overwrite them.
  ls_wait_vmcnt<0>();
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int t = 0; t < T; ++t) ls_tie(wring[r][t]);
#pragma unroll
    for (int t = 0; t < (GEN ? T : 1); ++t) {
      ls_tie(sring[r][t]);
      if constexpr (GEN) ls_tie(bring[r][t]);
    }
#pragma unroll
    for (int x = 0; x < XL; ++x) ls_tie(xring[r][x]);
  }

  // k-groups 1.. hand their sums to k-group 0 through LDS, which adds them in k-group
  // order. Every wavefront stays to the end so that all of them meet every barrier.
  const bool lead = kg == 0;
  if constexpr (KG > 1) {
    __syncthreads();  // every wavefront is done reading the activation stages
    float* red = reinterpret_cast<float*>(xs);
    if (!lead) {
#pragma unroll
      for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t)
          *reinterpret_cast<f4*>(red + ((((kg - 1u) * GW + wi) * T + t) * MT + r) * 256u + lane * 4u) = acc[r][t];
    }
    __syncthreads();
    if (lead) {
#pragma unroll
      for (uint32_t k = 1; k < (uint32_t)KG; ++k)
#pragma unroll
        for (int r = 0; r < MT; ++r)
#pragma unroll
          for (int t = 0; t < T; ++t)
            acc[r][t] += *reinterpret_cast<const f4*>(red + ((((k - 1u) * GW + wi) * T + t) * MT + r) * 256u + lane * 4u);
    }
  }

  // Output: lane holds rows 16 r + 4 g4 + v of column 16 (ctw + t) + c16.
  const __amdgpu_buffer_rsrc_t yr = make_rsrc(sY, M * sLdy * 2u);
  auto store_out = [&](int r, const f4* v) {  // row tile r
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t col = (ctw + t) * 16u + c16;
      const bool mine = (uint32_t)t < ntw && col < sN;  // tiles past ntw belong to the next slab
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t row = 16u * r + 4u * g4 + e;
        const uint32_t o = row < M && mine ? (row * sLdy + col) * 2u : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_out<DT>(v[t][e]), yr, o, 0, 0);
      }
    }
  };
  constexpr uint32_t kTilesWg = GW * T * MT;  // 16 x 16 fp32 tiles per workgroup
  if constexpr (BAL) {
    // Whole slab: store. Partial (first or last slab of the range): publish the partial
    // tile to slot 0 (first) or 1 (last) with agent-coherent stores; the arrival count
    // follows after the last piece.
    if (ka == 0u && kz == nkb) {
      if (lead) {
#pragma unroll
        for (int r = 0; r < MT; ++r) store_out(r, acc[r]);
      }
    } else if (lead) {
      const uint32_t slot = pi == 0u ? 0u : 1u;
      const __amdgpu_buffer_rsrc_t bpart = make_rsrc(pl.part, gridDim.x * 2u * kTilesWg * 1024u);
#pragma unroll
      for (int r = 0; r < MT; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint32_t o = 16u * r + 4u * g4 < M
                                 ? (((blockIdx.x * 2u + slot) * kTilesWg + (wi * T + t) * MT + r) * 64u + lane) * 16u
                                 : kOutOfRange;
          __builtin_amdgcn_raw_buffer_store_b128(acc[r][t], bpart, o, 0, 16);
        }
    }
    __syncthreads();  // this piece's LDS stages and reduction area are free for the next piece
    continue;
  }
  if (pl.S == 1) {
    if (lead) {
#pragma unroll
      for (int r = 0; r < MT; ++r) store_out(r, acc[r]);
    }
    return;
  }

  // Split slab: publish this piece (agent-coherent 16-byte stores, only lanes holding
  // rows < M), count arrivals, and let the last piece to arrive sum all pieces in piece
  // order. Waiting for the stores before the barrier orders them before the count.
  constexpr int kCoherent = 16;
  const uint32_t pieces = pl.S;
  const __amdgpu_buffer_rsrc_t partr = make_rsrc(pl.part, gridDim.y * pieces * kTilesWg * 1024u);
  auto part_off = [&](uint32_t p, int r, int t) {
    return 16u * r + 4u * g4 < M ? (((g * pieces + p) * kTilesWg + (wi * T + t) * MT + r) * 64u + lane) * 16u
                                 : kOutOfRange;
  };
  if (lead) {
#pragma unroll
    for (int r = 0; r < MT; ++r)
#pragma unroll
      for (int t = 0; t < T; ++t)
        __builtin_amdgcn_raw_buffer_store_b128(acc[r][t], partr, part_off(piece, r, t), 0, kCoherent);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(pl.cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = old == pieces - 1u;
    if (last) __hip_atomic_store(pl.cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh_last = last;
  }
  __syncthreads();
  if (!sh_last || !lead) return;
  // Every piece's partial of a row tile is loaded at once (a loop that waited for each
  // piece before loading the next cost one memory round trip per piece), then summed in
  // piece order.
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    f4 part[kMaxPieces][T];
#pragma unroll
    for (uint32_t p = 0; p < kMaxPieces; ++p)
#pragma unroll
      for (int t = 0; t < T; ++t)
        part[p][t] = p < pieces && p != piece
                         ? __builtin_amdgcn_raw_buffer_load_b128(partr, part_off(p, r, t), 0, kCoherent)
                         : acc[r][t];
    f4 sum[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      sum[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t p = 0; p < kMaxPieces; ++p)
        if (p < pieces) sum[t] += part[p][t];
    }
    store_out(r, sum);
  }
  }  // pieces

  if constexpr (BAL) {
    // Partial first / last slabs: count this workgroup's arrival at each; the last of a slab's
    // (at most two) contributors sums their partials in workgroup order and stores the slab.
    const uint32_t pfirst = u0 != gfirst * nkb || (glast == gfirst && u1 != (gfirst + 1u) * nkb) ? 1u : 0u;
    const uint32_t plast = glast != gfirst && u1 != (glast + 1u) * nkb ? 1u : 0u;
    if (!(pfirst | plast)) return;  // uniform
    constexpr uint32_t kTiles = GW * T * MT;
    const __amdgpu_buffer_rsrc_t bpart = make_rsrc(pl.part, gridDim.x * 2u * kTiles * 1024u);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the partial stores have completed
    __syncthreads();
    if (threadIdx.x < 2u) {
      const uint32_t i = threadIdx.x;
      uint32_t last = 0;
      if (i == 0u ? pfirst : plast) {
        const uint32_t gs = i == 0u ? gfirst : glast;
        const uint32_t bf = plan_wg_of_unit(pl.bL, pl.brem, gs * nkb);
        const uint32_t bl = plan_wg_of_unit(pl.bL, pl.brem, (gs + 1u) * nkb - 1u);
        const uint32_t old = __hip_atomic_fetch_add(pl.cnt + gs, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == bl - bf) {
          last = 1u;
          __hip_atomic_store(pl.cnt + gs, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      sh_tail[i] = last;
    }
    __syncthreads();
    const uint32_t last0 = sh_tail[0], last1 = sh_tail[1];
    if (!(last0 | last1) || kg != 0u) return;
    for (uint32_t i = 0; i < 2u; ++i) {
      if (!(i == 0u ? last0 : last1)) continue;  // uniform
      const uint32_t gs = i == 0u ? gfirst : glast;
      const uint32_t bf = plan_wg_of_unit(pl.bL, pl.brem, gs * nkb);
      const uint32_t bl = plan_wg_of_unit(pl.bL, pl.brem, (gs + 1u) * nkb - 1u);
      // The slab's segment, output and columns (as at the top of its piece).
      uint32_t si = 0;
      if constexpr (FUSED) {
        for (uint32_t k = 1; k < d.nseg; ++k)
          if (gs >= d.seg[k].blk_begin) si = k;
        si = __builtin_amdgcn_readfirstlane(si);
      }
      const SegDesc& sg = d.seg[si];
      const uint32_t ldyo = (uint32_t)sg.ldy, No = sg.N;
      const uint32_t ctwo = (gs - sg.blk_begin) * pl.sw + wi * T;
      const uint32_t owno = wi * T < pl.sw ? min((uint32_t)T, pl.sw - wi * T) : 0u;
      const uint32_t ntwo = ctwo < sg.ntiles ? min(owno, sg.ntiles - ctwo) : 0u;
      const __amdgpu_buffer_rsrc_t yro = make_rsrc(sg.Y, M * ldyo * 2u);
      // Contributors bf .. bl (at most two): slot 0 when gs is the contributor's first slab.
      const uint32_t s0 = plan_div(plan_begin(pl.bL, pl.brem, bf), nkb, pl.nkb_m) == gs ? 0u : 1u;
      const uint32_t s1 = plan_div(plan_begin(pl.bL, pl.brem, bl), nkb, pl.nkb_m) == gs ? 0u : 1u;
#pragma unroll
      for (int r = 0; r < MT; ++r) {
        if (16u * r + 4u * g4 >= M) continue;
        f4 p0[T], p1[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint32_t tile = (wi * T + t) * MT + r;
          p0[t] = __builtin_amdgcn_raw_buffer_load_b128(
              bpart, (((bf * 2u + s0) * kTiles + tile) * 64u + lane) * 16u, 0, 16);
          p1[t] = bl != bf ? __builtin_amdgcn_raw_buffer_load_b128(
                                 bpart, (((bl * 2u + s1) * kTiles + tile) * 64u + lane) * 16u, 0, 16)
                           : f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const f4 v = p0[t] + p1[t];
          const uint32_t col = (ctwo + t) * 16u + c16;
          const bool mine = (uint32_t)t < ntwo && col < No;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t row = 16u * r + 4u * g4 + e;
            const uint32_t o = row < M && mine ? (row * ldyo + col) * 2u : kOutOfRange;
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_out<DT>(v[e]), yro, o, 0, 0);
          }
        }
      }
    }
  }
}

int ls_env(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

uint32_t ls_assign_slabs(GemmDesc& d, uint32_t sw) {
  uint32_t g = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    const uint32_t ns = (d.seg[i].ntiles + sw - 1) / sw;
    d.seg[i].blk_begin = g;
    d.seg[i].blk_count = ns;
    g += ns;
  }
  return g;
}

template <int FMT, int DT, int KG, int GW, int T, int U, int MT, bool GEN = false>
hipError_t ls_launch_t(GemmDesc d, const LsConfig& c, void* ws, uint32_t* fault, uint32_t spin, hipStream_t stream) {
  const bool fused = d.nseg > 1;
  if (d.M > 16u * MT) return hipErrorInvalidValue;
  LsPlan pl{};
  pl.fault = fault;
  pl.spin = spin;
  if (c.SW < 1 || c.SW > GW * T) return hipErrorInvalidValue;
  pl.sw = (uint32_t)c.SW;
  const uint32_t G = ls_assign_slabs(d, pl.sw);
  pl.S = (uint32_t)c.S;
  pl.kq = d.nkb / pl.S;
  pl.kr = d.nkb % pl.S;
  pl.gmul = plan_gmul(d.gkb);
  if (pl.S > 1) {
    if (!ws) return hipErrorInvalidValue;
    pl.cnt = static_cast<uint32_t*>(ws);
    pl.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  }
  if (c.P > 0) {  // balanced grid
    if constexpr (GEN || KG == 1 || (MT == 1 && !(KG == 2 && GW == 4 && T == 2 && U == 2))) {
      return hipErrorInvalidConfiguration;
    } else {
      const uint32_t P = (uint32_t)c.P;
      const uint64_t utot = (uint64_t)G * d.nkb;
      if (P >= G || !ws || G > kMaxCounters || utot >= (1ull << 31) || utot / P < d.nkb) return hipErrorInvalidValue;
      pl.S = 1;
      pl.bL = (uint32_t)(utot / P);
      pl.brem = (uint32_t)(utot % P);
      pl.nkb_m = plan_div_magic(d.nkb);
      pl.cnt = static_cast<uint32_t*>(ws);
      pl.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
      bool fitsb = (uint64_t)d.M * (uint64_t)d.ldx * 2u < (1ull << 31) && (uint64_t)P * 2u * GW * T * MT * 1024u < (1ull << 31);
      for (uint32_t i = 0; i < d.nseg; ++i) fitsb = fitsb && (uint64_t)d.M * (uint64_t)d.seg[i].ldy * 2u < (1ull << 31);
      if (!fitsb) return hipErrorInvalidValue;
      if (fused)
        hipLaunchKernelGGL((hq_decode_ls_kernel<FMT, DT, KG, GW, T, U, MT, true, false, true>), dim3(P, 1),
                           dim3(64 * KG * GW), 0, stream, d, pl);
      else
        hipLaunchKernelGGL((hq_decode_ls_kernel<FMT, DT, KG, GW, T, U, MT, false, false, true>), dim3(P, 1),
                           dim3(64 * KG * GW), 0, stream, d, pl);
      return hipGetLastError();
    }
  }
  // Byte offsets into X, Y and the partials are 32-bit buffer offsets.
  const uint64_t xbytes = (uint64_t)d.M * (uint64_t)d.ldx * 2u;
  bool fits = G >= 1 && G <= 65535 && xbytes < (1ull << 31) && (uint64_t)G * pl.S * GW * T * MT * 1024u < (1ull << 31);
  for (uint32_t i = 0; i < d.nseg; ++i) fits = fits && (uint64_t)d.M * (uint64_t)d.seg[i].ldy * 2u < (1ull << 31);
  if (!fits) return hipErrorInvalidValue;
  if constexpr (GEN) {  // the general kernels always look their segment up
    hipLaunchKernelGGL((hq_decode_ls_kernel<FMT, DT, KG, GW, T, U, MT, true, true>), dim3(pl.S, G), dim3(64 * KG * GW),
                       0, stream, d, pl);
  } else if (fused) {
    hipLaunchKernelGGL((hq_decode_ls_kernel<FMT, DT, KG, GW, T, U, MT, true, false>), dim3(pl.S, G),
                       dim3(64 * KG * GW), 0, stream, d, pl);
  } else {
    hipLaunchKernelGGL((hq_decode_ls_kernel<FMT, DT, KG, GW, T, U, MT, false, false>), dim3(pl.S, G),
                       dim3(64 * KG * GW), 0, stream, d, pl);
  }
  return hipGetLastError();
}

template <int FMT, int DT>
hipError_t ls_launch_fd(const GemmDesc& d, const LsConfig& c, void* ws, uint32_t* fault, uint32_t spin,
                        hipStream_t stream) {
  if (d.gen) {  // general kernels: two k-groups of four wavefronts, two tiles each, two steps in flight
    if (c.GW * 1000 + c.KG * 100 + c.T * 10 + c.U != 4222) return hipErrorInvalidConfiguration;
    switch (c.MT) {
      case 1: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 1, true>(d, c, ws, fault, spin, stream);
      case 2: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 2, true>(d, c, ws, fault, spin, stream);
      case 3: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 3, true>(d, c, ws, fault, spin, stream);
      case 4: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 4, true>(d, c, ws, fault, spin, stream);
      case 5: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 5, true>(d, c, ws, fault, spin, stream);
      default: return hipErrorInvalidConfiguration;
    }
  }
  if (c.MT > 1 && c.KG == 1) {  // one k-group, two workgroups per CU
    if (c.GW * 1000 + c.KG * 100 + c.T * 10 + c.U != 4122) return hipErrorInvalidConfiguration;
    switch (c.MT) {
      case 2: return ls_launch_t<FMT, DT, 1, 4, 2, 2, 2>(d, c, ws, fault, spin, stream);
      case 3: return ls_launch_t<FMT, DT, 1, 4, 2, 2, 3>(d, c, ws, fault, spin, stream);
      case 4: return ls_launch_t<FMT, DT, 1, 4, 2, 2, 4>(d, c, ws, fault, spin, stream);
      case 5: return ls_launch_t<FMT, DT, 1, 4, 2, 2, 5>(d, c, ws, fault, spin, stream);
      default: return hipErrorInvalidConfiguration;
    }
  }
  if (c.MT > 1) {  // several row tiles: two k-groups of four wavefronts, two tiles each, two steps in flight
    if (c.GW * 1000 + c.KG * 100 + c.T * 10 + c.U != 4222) return hipErrorInvalidConfiguration;
    switch (c.MT) {
      case 2: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 2>(d, c, ws, fault, spin, stream);
      case 3: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 3>(d, c, ws, fault, spin, stream);
      case 4: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 4>(d, c, ws, fault, spin, stream);
      case 5: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 5>(d, c, ws, fault, spin, stream);
      default: return hipErrorInvalidConfiguration;
    }
  }
  switch (c.GW * 1000 + c.KG * 100 + c.T * 10 + c.U) {
    case 4124: return ls_launch_t<FMT, DT, 1, 4, 2, 4, 1>(d, c, ws, fault, spin, stream);
    case 4214: return ls_launch_t<FMT, DT, 2, 4, 1, 4, 1>(d, c, ws, fault, spin, stream);
    case 4222: return ls_launch_t<FMT, DT, 2, 4, 2, 2, 1>(d, c, ws, fault, spin, stream);
    case 4223: return ls_launch_t<FMT, DT, 2, 4, 2, 3, 1>(d, c, ws, fault, spin, stream);
    case 4242: return ls_launch_t<FMT, DT, 2, 4, 4, 2, 1>(d, c, ws, fault, spin, stream);
    case 4413: return ls_launch_t<FMT, DT, 4, 4, 1, 3, 1>(d, c, ws, fault, spin, stream);
    case 4422: return ls_launch_t<FMT, DT, 4, 4, 2, 2, 1>(d, c, ws, fault, spin, stream);
    case 4423: return ls_launch_t<FMT, DT, 4, 4, 2, 3, 1>(d, c, ws, fault, spin, stream);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace

// Lockstep tiling: KG k-groups of four wavefronts, T tiles per wavefront (slabs of up to
// 4 T tiles), ring depth U, and S pieces per slab chosen so that the grid covers the CUs.
// HQ_DECODE_LS_KG / _T / _U / _S / _SW override (tuning and tests).
LsConfig choose_decode_ls(int fmt, const GemmDesc& d, size_t ws_cap) {
  const uint32_t cus = (uint32_t)cu_count();
  // Measured on MI355X (27B-class shapes, M = 4..16): two k-groups of four wavefronts,
  // two tiles per wavefront, two steps in flight; a K split only when the slabs alone
  // leave more than a quarter of the CUs idle.
  LsConfig c{2, 2, 1, 2, 4, 0, (int)std::min<uint32_t>(kLsMaxRowTiles, (d.M + 15u) / 16u)};
  const int eKG = ls_env("HQ_DECODE_LS_KG", 0);
  if (eKG == 1 || eKG == 2 || eKG == 4) c.KG = eKG;
  const int eT = ls_env("HQ_DECODE_LS_T", 0);
  if (eT == 1 || eT == 2 || eT == 4) c.T = eT;
  const int eU = ls_env("HQ_DECODE_LS_U", 0);
  if (eU >= 2 && eU <= 4) c.U = eU;
  // Snap to an instantiated (KG, T, U); several row tiles have two configurations (one or
  // two k-groups of four wavefronts, two tiles each, two steps in flight).
  if (c.KG == 1) { c.T = 2; c.U = 4; }
  if (c.KG == 2 && c.T == 1) c.U = 4;
  if (c.KG == 2 && c.T == 2) c.U = std::min(c.U, 3);
  if (c.KG == 2 && c.T == 4) c.U = 2;
  if (c.KG == 4) { c.T = std::min(c.T, 2); c.U = c.T == 1 ? 3 : std::min(c.U, 3); }
  if (c.MT > 1) { c.KG = eKG == 1 ? 1 : 2; c.T = 2; c.U = 2; }
  GemmDesc x = d;
  c.SW = c.GW * c.T;
  const uint32_t G = ls_assign_slabs(x, (uint32_t)c.SW);
  if (G < cus * 3 / 4) c.S = (int)std::max<uint32_t>(1, std::min<uint32_t>(d.nkb, (cus * 15 / 16 + G - 1) / G));
  // Several row tiles: as many pieces as keep the grid within one workgroup per CU, when that
  // still covers three quarters of the CUs, so that the two k-groups of a workgroup share its
  // CU (the rule above can give more workgroups than CUs, which then run one k-group each).
  // Measured on MI355X (ternary 5120 x 14336, 112 slabs): M = 48 19.9 -> 18.0 us, M = 80
  // 28.1 -> 24.8 us with two pieces instead of three.
  if (c.MT > 1 && G < cus && (cus / G) * G >= cus * 3 / 4)
    c.S = (int)std::max<uint32_t>(1, std::min<uint32_t>(d.nkb, cus / G));
  // Ternary tiles are half the bytes of int4 ones, so a step of the same shape has half the
  // bytes in flight: when the grid is one round and each k-group still gets at least five
  // steps, four k-groups (16 wavefronts) keep more of them in flight. Measured on MI355X:
  // 5120 x 27648 20% faster, 17408 x 5120 13% faster; shorter pieces (5120 x 14336 cut in
  // three) or two rounds (5120 x 34816) are slower so.
  // Int4 weights take four k-groups (two steps in flight) when each still gets eight or more
  // steps. Measured on MI355X (alternated runs): 27648 x 5120 (nine steps per k-group) M = 9 /
  // 12 / 16 18.6 / 18.4 / 17.8 -> 17.8 / 17.8 / 17.7 us (bf16 M = 16 20.3 -> 18.6); 17408 x 5120
  // (six steps) no gain.
  if (c.MT == 1 && eKG == 0 && eT == 0 && eU == 0 && c.T == 2 && c.KG == 2 && (uint64_t)G * (uint32_t)c.S <= cus) {
    const uint32_t steps4 = (d.nkb / (uint32_t)c.S + 3u) / 4u;
    if (fmt == HQ_FORMAT_TERNARY2 && steps4 >= 5u) {
      c.KG = 4;
      c.U = steps4 >= 8u ? 3 : 2;
    } else if (fmt == HQ_FORMAT_INT4 && steps4 >= 8u) {
      c.KG = 4;
      c.U = 2;
    }
  }
  // Several row tiles: one workgroup per CU (two k-groups of four wavefronts near 256 VGPRs
  // each), so a grid of more slabs than CUs would run a second, nearly empty round. One k-group
  // per workgroup lets two workgroups share a CU and the whole grid run at once. Measured on
  // MI355X (ternary 5120 x 34816, 272 slabs): M = 48 47 -> 41.5 us, M = 80 63 -> 60 us; with
  // slabs for every CU already (216-240) one k-group is 5-20% slower.
  if (c.MT > 1 && eKG == 0 && (uint64_t)G * (uint32_t)c.S > cus && (uint64_t)G * (uint32_t)c.S <= 2ull * cus) c.KG = 1;
  // More slabs than CUs: a balanced grid, one workgroup of two k-groups
  // per CU, each an equal run of (slab, k-block) units (its first and last slab possibly
  // shared with a neighbour through the workspace), where one k-group per workgroup would
  // leave a few CUs with two (up to 1.25 slabs per CU) or where two k-groups would run more
  // than two rounds. Measured on MI355X (M = 32 / 80, alternated): int4 5120 x 34816 (272
  // slabs) 36.5 -> 29.8 / 54.7 -> 50.5 us, 4096 x 40960 (320) 28.5 -> 26.8 / 45.9 -> 44.5,
  // ternary 5120 x 69632 (544) 55.8 -> 47.2 / 92.2 -> 84.3; at 432 slabs (int4 5120 x 55296)
  // two workgroups per CU on most CUs stay 13-17% ahead. One row tile (M <= 16): int4 up to
  // 1.25 slabs per CU (int4 5120 x 34816, M = 9..16: 25.3-27.2 -> 23.8-25.5 us; 4096 x 40960
  // 25.0-25.5 -> 21.7-22.1); ternary weights and 432 slabs measured slower, 544 even.
  // HQ_DECODE_LS_BAL = 0 / 1: off / on.
  const int ebal = ls_env("HQ_DECODE_LS_BAL", -1);
  const bool one_tile = c.MT == 1 && c.GW == 4 && c.T == 2;
  const bool bal_fit = c.MT > 1 ? (4u * G <= 5u * cus || G > 2u * cus) : (fmt == HQ_FORMAT_INT4 && 4u * G <= 5u * cus);
  if ((c.MT > 1 || one_tile) && !d.gen && G > cus && G <= kMaxCounters && (ebal == 1 || (ebal != 0 && bal_fit))) {
    c.P = (int)cus;
    c.KG = 2;
    c.S = 1;
    if (c.MT == 1) c.U = 2;
  }
  // Narrower slabs that would cover every CU measured slower (5120 x 27648, M = 1..16:
  // 247 slabs of 7 tiles 2-15% behind 216 of 8), so slabs stay GW * T tiles wide.
  // The general kernels exist in one configuration: two k-groups of four wavefronts, two
  // tiles each, two steps in flight (8-tile slabs).
  if (d.gen) {
    c.KG = 2;
    c.GW = 4;
    c.T = 2;
    c.U = 2;
  }
  const int eSW = ls_env("HQ_DECODE_LS_SW", 0);
  if (eSW >= 1 && eSW <= c.GW * c.T) c.SW = eSW;
  const int eS = ls_env("HQ_DECODE_LS_S", 0);
  if (eS >= 1) c.S = eS;
  c.S = std::max(1, std::min<int>({c.S, (int)d.nkb, (int)kMaxPieces}));
  if (c.S > 1 && ls_assign_slabs(x, (uint32_t)c.SW) > kMaxCounters) c.S = 1;
  while (c.S > 1 && decode_ls_workspace_bytes(d, c) > ws_cap) --c.S;  // fewer pieces under a cap
  if (c.P > 0 && decode_ls_workspace_bytes(d, c) > ws_cap) {  // the S-piece grid under a cap
    c.P = 0;
    if (eKG == 0) c.KG = 1;
  }
  return c;
}

size_t decode_ls_workspace_bytes(const GemmDesc& d, const LsConfig& c) {
  if (c.P > 0) return kCounterBytes + (size_t)c.P * 2u * c.GW * c.T * c.MT * 1024u;
  if (c.S <= 1) return 0;
  GemmDesc x = d;
  const uint32_t G = ls_assign_slabs(x, (uint32_t)c.SW);
  return kCounterBytes + (size_t)G * c.S * c.GW * c.T * c.MT * 1024u;
}

hipError_t launch_decode_ls(int fmt, int dtype, GemmDesc d, const LsConfig& c, void* ws, uint32_t* fault,
                            uint32_t spin, hipStream_t stream) {
  if (fmt == HQ_FORMAT_INT4) {
    return dtype == HQ_DTYPE_F16 ? ls_launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_F16>(d, c, ws, fault, spin, stream)
                                 : ls_launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_BF16>(d, c, ws, fault, spin, stream);
  }
  return dtype == HQ_DTYPE_F16 ? ls_launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16>(d, c, ws, fault, spin, stream)
                               : ls_launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_BF16>(d, c, ws, fault, spin, stream);
}

}  // namespace hq

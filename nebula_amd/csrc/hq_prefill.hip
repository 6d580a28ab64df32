// hq_prefill.hip — compute-bound qGEMM for M > 16 (prefill, split-fuse batches), gfx950.
//
// The reference has no prefill GEMM (hydrogen's decoder feeds prompt tokens one at a
// time, native_decoder.cu:1297); this is the MFMA path the target operator asks for.
//
// Workgroup tile: (16 * RT * WM) rows x 256 columns, K stepped one 128-deep k-block at a
// time. 4 * WM wavefronts: WM along M, 4 along N; each owns 16 * RT rows and 64 columns
// (4 column tiles, 16 * RT * 4 fp32 accumulators). A weight fragment is dequantised with
// its group scale folded in by the WM wavefronts sharing its columns and reused by RT
// MFMAs each; WM = 2 gives two waves per SIMD so one's dequantisation hides under the
// other's MFMAs. Activation tiles are staged in LDS, double-buffered, with the
// gfx950 buffer->LDS path (buffer_load_dwordx4 ... lds), in a layout whose 16-byte units
// are XOR-swizzled by row so the ds_read_b128 fragment reads are bank-conflict free.
// Weights go straight from HBM into registers in the tile layout (hq_layout.hpp), which
// already is the v_mfma_f32_16x16x32 fragment order; they are the MFMA's A operand and the
// activations its B operand, so each result is the transposed 16 x 16 tile and a lane holds
// four consecutive output columns of one row (8-byte output stores). Accumulation is fp32.
// Workgroups are renumbered so that each XCD owns a contiguous band of row blocks and
// keeps its activation rows resident in its own L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "hq_device.hpp"
#include "hq_internal.hpp"
#include "hq_plan.hpp"

namespace hq {
namespace {

constexpr int kTilesPerWave = 4;  // 64 columns per wavefront, 256 per workgroup
// fp16 128-row tiles order each k-block's instructions explicitly (see step()): the LDS
// read of A fragment i + kReadAhead issues before the MFMAs of fragment i, and the next
// chunk's dequantisation is spread between the MFMAs, kValuPerFrag VALU instructions after
// each fragment's four (the first chunk's, kValuFirst of them, come first). Measured on
// MI355X against the compiler's own order (which waits on each LDS read right after it):
// 3-7% faster at M = 512..4096, N = 27648.
constexpr int kReadAhead = 3;
constexpr int kValuFirst = 32;
constexpr int kValuPerFrag = 7;

// Dequantised B fragment with the group scale applied. s2 holds the fp16 scale twice.
// GEN (int4): `add` is the weight of code 8, e = 8 s + b, as fp16 bits (fp16 activations) or
// the bias b as fp32 bits (bf16 activations), so that the fragment is q * s + b.
template <int FMT, int DT, bool GEN = false>
__device__ __forceinline__ u4 dq_scaled(const u4& w, int c, uint32_t s_f16, const DqConst& k, uint32_t add = 0) {
  if constexpr (DT == HQ_DTYPE_F16) {
    const h2 s2 = bits_h2(s_f16 | (s_f16 << 16));
    u4 q;
    if constexpr (FMT == HQ_FORMAT_INT4) {
      q = dq_int4_f16(w[c], k);  // exact q - 8
    } else {
      const uint32_t word = w[c >> 1];
      q = (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);  // exact 2t; the epilogue halves
    }
    if constexpr (GEN && FMT == HQ_FORMAT_INT4) {
      const h2 e2 = bits_h2(add | (add << 16));
      return u4{h2_bits(__builtin_elementwise_fma(bits_h2(q[0]), s2, e2)),
                h2_bits(__builtin_elementwise_fma(bits_h2(q[1]), s2, e2)),
                h2_bits(__builtin_elementwise_fma(bits_h2(q[2]), s2, e2)),
                h2_bits(__builtin_elementwise_fma(bits_h2(q[3]), s2, e2))};
    }
    return u4{h2_bits(bits_h2(q[0]) * s2), h2_bits(bits_h2(q[1]) * s2), h2_bits(bits_h2(q[2]) * s2),
              h2_bits(bits_h2(q[3]) * s2)};
  } else {
    // No packed bf16 arithmetic on gfx950: form w * s in fp32, round pairs with v_cvt_pk_bf16_f32.
    const float s = f16_to_f32((uint16_t)s_f16);
    float v[8];
    if constexpr (FMT == HQ_FORMAT_INT4) {
      const uint32_t x = w[c];
      const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
      // byte b of lo holds element {0,4,1,5}[b], of hi element {2,6,3,7}[b] (nibble order of hq_layout.hpp)
      const float ms = GEN ? __builtin_bit_cast(float, add) : -8.0f * s;
      v[0] = __builtin_fmaf((float)((lo >> 0) & 0xFFu), s, ms);
      v[4] = __builtin_fmaf((float)((lo >> 8) & 0xFFu), s, ms);
      v[1] = __builtin_fmaf((float)((lo >> 16) & 0xFFu), s, ms);
      v[5] = __builtin_fmaf((float)((lo >> 24) & 0xFFu), s, ms);
      v[2] = __builtin_fmaf((float)((hi >> 0) & 0xFFu), s, ms);
      v[6] = __builtin_fmaf((float)((hi >> 8) & 0xFFu), s, ms);
      v[3] = __builtin_fmaf((float)((hi >> 16) & 0xFFu), s, ms);
      v[7] = __builtin_fmaf((float)((hi >> 24) & 0xFFu), s, ms);
    } else {
      const uint32_t word = w[c >> 1];
      const u4 q = (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);  // bf16 bits of 2t
      const float hs = 0.5f * s;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __builtin_bit_cast(float, q[i] << 16) * hs;
        v[2 * i + 1] = __builtin_bit_cast(float, q[i] & 0xFFFF0000u) * hs;
      }
    }
    u4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
      const bf2 p = {(__bf16)v[2 * i], (__bf16)v[2 * i + 1]};
      r[i] = __builtin_bit_cast(uint32_t, p);
    }
    return r;
  }
}

// Output tile `tile`, numbered row-band major over all segments' 256-column blocks
// (tile = mt * nb + cb, cb counting segment 0's blocks, then segment 1's, ...; a
// segment's first block is its blk_begin): its segment, first row and this wavefront's
// first column tile. Consecutive tiles share their activation rows across segments.
template <uint32_t BM, int TW = kTilesPerWave>
__device__ __forceinline__ void tile_geom(const GemmDesc& d, uint32_t nb, uint32_t tile, uint32_t wn, uint32_t& s,
                                          uint32_t& m0, uint32_t& ct0) {
  const uint32_t mt = tile / nb;
  const uint32_t cb = tile - mt * nb;
  s = 0;
#pragma unroll
  for (uint32_t i = 1; i < HQ_MAX_SEGMENTS; ++i)
    if (i < d.nseg && cb >= d.seg[i].blk_begin) s = i;
  m0 = mt * BM;
  ct0 = (cb - d.seg[s].blk_begin) * (4u * TW) + wn * TW;
}

// SKP = false: workgroup b computes whole tile b (grid dp). SKP = true: workgroup b
// computes stream-K range b (grid psk). Two kernels, so that the stream-K fix-up's
// registers never weigh on the whole-tile pipeline.
// One-row-wave 128-row tiles are held to 256 VGPRs so that two workgroups share a CU (their
// barriers are independent, so one's dequantisation overlaps the other's MFMAs).
// GEN: the general kernels (one scale per 32-wide k chunk, optional int4 bias), 64-row tiles.
// KS = 2 (whole 128-row tiles only): the workgroup's eight wavefronts are two halves of four,
// each computing the tile over half of its k-blocks through its own LDS stages; the halves'
// sums meet in LDS at the end (half 0 + half 1). A grid of one tile per CU then still keeps
// two wavefronts on every SIMD, as two workgroups per CU do.
template <int FMT, int DT, int RT, int WM, bool SKP, bool GEN = false, int KS = 1, int TW = 4>
__global__ void __launch_bounds__(256 * WM * KS, WM == 1 && RT == 8 && KS == 1 ? 2 : 1)
    hq_prefill_kernel(const GemmDesc d, const PrefillPlan pp) {
  static_assert(KS == 1 || (KS == 2 && !SKP && !GEN && WM == 1), "the K split is for whole fast tiles");
  static_assert(TW == 4 || (TW == 2 && KS == 1 && !SKP && !GEN && WM == 1 && RT == 8),
                "128-column tiles are whole 128-row fast tiles");
  // Column tiles per wavefront: 4 (256-column workgroup tiles) or 2 (128 columns).
  constexpr int kTilesPerWave = TW;
  constexpr uint32_t BM = 16u * RT * WM;
  constexpr uint32_t kStageBytes = BM * 256u;        // BM rows x 128 fp16
  constexpr uint32_t kPartBytes = BM * 256u * 4u;    // one fp32 partial tile
  constexpr uint32_t kWavePart = RT * kTilesPerWave * 1024u;  // one wavefront's share of it
  // The explicit order holds more values live; the fp16 128-row kernels make room for it with
  // a weight ring of two k-blocks (one ahead: a k-block's MFMAs outlast a load's latency).
  // 128-column tiles keep the compiler's order (the explicit one, scaled to two column tiles,
  // measured 6-13% slower) with a ring of two k-blocks (three: 1-3.5% slower, int4 fp16 within
  // 0.5%).
  constexpr bool kOrdered = DT == HQ_DTYPE_F16 && RT == 8 && !GEN && TW == 4;
  constexpr int kRing = kOrdered || TW == 2 ? 2 : 3;
  // Partial tiles are stored and loaded with the sc1 cache policy: agent-coherent, so a
  // store that has completed is visible to loads from any XCD.
  constexpr int kCoherent = 16;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  uint32_t* const sh_last = reinterpret_cast<uint32_t*>(smem + 2u * KS * kStageBytes);

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t kh = KS > 1 ? wave_all / (4u * WM) : 0u;           // K half (KS = 2)
  const uint32_t wave = KS > 1 ? wave_all % (4u * WM) : wave_all;    // wavefront within its half
  char* const stages = smem + kh * 2u * kStageBytes;                 // this half's two LDS stages
  const uint32_t c16 = lane & 15u, g4 = lane >> 4;
  const uint32_t wm = wave / 4u, wn = wave % 4u;
  const uint32_t wrow0 = wm * 16u * RT;  // first tile row of this wavefront
  const uint32_t nkb = d.nkb;

  const uint32_t bid = blockIdx.x;

  // KS = 2: the two K halves meet separately at every k-block, so that the wavefronts sharing
  // a SIMD (one per half) drift apart and hide each other's waits (a workgroup barrier kept
  // them in step: the fused QKV tile ran at half the MFMA rate of two independent workgroups
  // on a CU). A half's barrier is an LDS arrival count (sh_last[kh]): each wavefront adds one
  // once its own copies of the k-block have landed and its reads of the previous stage are
  // done, and waits until the half's four have arrived. The wait is bounded: every wavefront
  // of a half executes the same steps, so a correct launch never reaches the bound; one that
  // gives up sets the host-visible fault word (reported as HQ_ERR_DEVICE) and carries on.
  uint32_t arrivals = 0;
  const uint32_t harr = (uint32_t)(uintptr_t)(sh_last + kh);
  if constexpr (KS > 1) {
    if (threadIdx.x < 2u) sh_last[threadIdx.x] = 0u;
    __syncthreads();
  }
  auto kblock_barrier = [&]() {
    if constexpr (KS == 1) {
      __syncthreads();
    } else {
      arrivals += 4u;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) asm volatile("ds_add_u32 %0, %1" ::"v"(harr), "v"(1u) : "memory");
      bool met = false;
      for (uint32_t spin = 0; spin < pp.spin; ++spin) {
        uint32_t got;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(got) : "v"(harr) : "memory");
        if (__builtin_amdgcn_readfirstlane(got) >= arrivals) {
          met = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!met && lane == 0 && pp.fault) __hip_atomic_store(pp.fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  };

  // The wave's RT activation load instructions per k-block (BM / 4 in all): instruction i
  // fills LDS rows 4q..4q+3, q = wave * RT + i; lane -> row 4q + g4, 16-byte slot c16
  // holding unit c16 ^ (row & 15). The k-block goes in the uniform offset; the row stays
  // in the per-lane offset, which the descriptor's range check covers (rows >= M read 0).
  uint32_t aoff[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const uint32_t r = 4u * (wave * RT + i) + g4;
    aoff[i] = (r * (uint32_t)d.ldx + 8u * (c16 ^ (r & 15u))) * 2u;
  }
  // LDS fragment addresses: row 16 r + c16, unit (4 c + g4) ^ c16.
  uint32_t ldsoff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) ldsoff[c] = c16 * 256u + (((4u * c + g4) ^ c16) * 16u);
  const DqConst dqk = dq_const_f16();
  const uint32_t tile_bytes = nkb * 64u * (FMT == HQ_FORMAT_INT4 ? 16u : 8u);
  const __amdgpu_buffer_rsrc_t partr = make_rsrc(pp.part, pp.part ? pp.psk * 2u * kPartBytes : 0u);

  f4 acc[RT][kTilesPerWave];

  // Epilogue of a finished tile. The MFMAs take the weight fragment as their A operand and the
  // activations as B, so each 16 x 16 result is the transposed tile: lane -> activation row
  // 16 r + c16 and the four consecutive output columns 16 (ct0 + t) + 4 g4 + v. When the
  // wavefront's 64 columns lie inside N and rows are 16-byte aligned, the results go through
  // the wavefront's own LDS area (16 RT rows x 128 bytes, 16-byte units XOR-swizzled by row)
  // and leave as 16-byte stores, eight lanes per row: each instruction writes whole 128-byte
  // row segments (8-byte stores straight from the MFMA layout wrote each line in four 32-byte
  // pieces: 1.6x the output bytes in HBM writes). The area overlaps the activation stages: the
  // caller guarantees every wavefront is done reading them. Otherwise one 8-byte store per
  // lane, and 2-byte stores for columns past N or rows that are not 8-byte aligned. Rows past M
  // fall outside the descriptor. Only row tiles r0 <= r < r1 (compile-time after unrolling).
  auto store_tile = [&](uint32_t s, uint32_t m0, uint32_t ct0, int r0 = 0, int r1 = RT) {
    constexpr float post = (FMT == HQ_FORMAT_TERNARY2 && DT == HQ_DTYPE_F16) ? 0.5f : 1.0f;
    const SegDesc& sg = d.seg[s];
    const uint32_t rows = min(BM, d.M - m0);
    const __amdgpu_buffer_rsrc_t yr =
        make_rsrc(reinterpret_cast<char*>(sg.Y) + (size_t)m0 * (size_t)sg.ldy * 2u, rows * (uint32_t)sg.ldy * 2u);
    const uint32_t align = (uint32_t)reinterpret_cast<uintptr_t>(sg.Y) | ((uint32_t)sg.ldy * 2u);
    // RB: bytes of a wavefront's output row (16 TW columns), in 2 TW 16-byte units.
    constexpr uint32_t RB = 32u * TW, UM = 2u * TW - 1u;
    if ((align & 15u) == 0u && ct0 * 16u + 16u * TW <= sg.N) {  // uniform
      char* const area = smem + wave * (16u * RT * RB);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (r < r0 || r >= r1) continue;
        const uint32_t row = 16u * r + c16;
#pragma unroll
        for (int t = 0; t < kTilesPerWave; ++t) {
          const f4 v = acc[r][t] * post;
          const u2 packed = {(uint32_t)f32_to_out<DT>(v[0]) | ((uint32_t)f32_to_out<DT>(v[1]) << 16),
                             (uint32_t)f32_to_out<DT>(v[2]) | ((uint32_t)f32_to_out<DT>(v[3]) << 16)};
          const uint32_t unit = 2u * t + (g4 >> 1);
          *reinterpret_cast<u2*>(area + row * RB + ((unit ^ (row & UM)) * 16u) + (g4 & 1u) * 8u) = packed;
        }
      }
      // Read back in row order (this wavefront's own area: its LDS operations complete in
      // order): lane -> row (32 / TW) i + lane / (2 TW), columns 8 (lane % (2 TW)) .. + 7.
      const uint32_t j = lane & UM;
      constexpr int kRowsPer = 32 / TW;  // rows per read instruction
#pragma unroll
      for (int i = 0; i < RT * TW / 2; ++i) {
        if (i < r0 * TW / 2 || i >= r1 * TW / 2) continue;
        const uint32_t row = (uint32_t)kRowsPer * i + lane / (2u * TW);
        const u4 v = *reinterpret_cast<const u4*>(area + row * RB + ((j ^ (row & UM)) * 16u));
        __builtin_amdgcn_raw_buffer_store_b128(v, yr, ((wrow0 + row) * (uint32_t)sg.ldy + ct0 * 16u + 8u * j) * 2u, 0, 0);
      }
      return;
    }
    const bool wide = (align & 7u) == 0u;  // uniform
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) {
      const uint32_t n0 = (ct0 + t) * 16u + 4u * g4;
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (r < r0 || r >= r1) continue;
        const uint32_t row = wrow0 + 16u * r + c16;
        const uint32_t o = (row * (uint32_t)sg.ldy + n0) * 2u;
        const f4 v = acc[r][t] * post;
        if (wide && n0 + 3u < sg.N) {
          const u2 packed = {(uint32_t)f32_to_out<DT>(v[0]) | ((uint32_t)f32_to_out<DT>(v[1]) << 16),
                             (uint32_t)f32_to_out<DT>(v[2]) | ((uint32_t)f32_to_out<DT>(v[3]) << 16)};
          __builtin_amdgcn_raw_buffer_store_b64(packed, yr, o, 0, 0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_out<DT>(v[e]), yr, n0 + e < sg.N ? o + 2u * e : kOutOfRange,
                                                  0, 0);
        }
      }
    }
  };

  // k-blocks [ka, kz) of one tile into acc.
  auto run_piece = [&](uint32_t s, uint32_t m0, uint32_t ct0, uint32_t ka, uint32_t kz) {
    const SegDesc& sg = d.seg[s];
    // Activation rows [m0, m0 + BM) of X; rows >= M read as zero.
    const uint32_t rows = min(BM, d.M - m0);
    const __amdgpu_buffer_rsrc_t xr =
        make_rsrc(reinterpret_cast<const char*>(d.X) + (size_t)m0 * (size_t)d.ldx * 2u, rows * (uint32_t)d.ldx * 2u);
    // Prefetches past the piece re-read its last k-block (in range, never computed on), so
    // every step issues the same loads and the wait counts stay exact.
    auto load_a = [&](uint32_t stage, uint32_t kb) {
      const uint32_t ko = min(kb, kz - 1u) * 256u;
#pragma unroll
      for (int i = 0; i < RT; ++i)
        buffer_to_lds16(xr, stages + stage * kStageBytes + (wave * RT + i) * 1024u, aoff[i], ko);
    };
    // Weights: one descriptor per column tile of this wavefront.
    __amdgpu_buffer_rsrc_t wrs[kTilesPerWave];
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) {
      const uint32_t ct = ct0 + t;
      const bool ok = ct < sg.ntiles;
      wrs[t] = make_rsrc(reinterpret_cast<const char*>(sg.Wp) + (size_t)(ok ? ct : 0u) * tile_bytes, ok ? tile_bytes : 0u);
    }
    // Scale of column 16 ct + c16 (clamped to N - 1: columns past N are not stored). GEN: the
    // scale (and bias) of that column in chunk g4 of the k-block, row (4 kb + g4) / g32.
    const uint32_t srows = GEN ? 4u * nkb / d.g32 : nkb / d.gkb;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(sg.S, ((srows - 1u) * sg.lds + sg.N) * 2u);
    const __amdgpu_buffer_rsrc_t brs = make_rsrc(sg.B, GEN && sg.B ? ((srows - 1u) * sg.lds + sg.N) * 4u : 0u);
    uint32_t soff[kTilesPerWave];
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) soff[t] = min((ct0 + t) * 16u + c16, sg.N - 1u) * 2u;
    // Weights and scales: a register ring of kRing k-blocks, kRing - 1 ahead of the one
    // computed.
    // Column tiles past the segment have an empty descriptor and read zero.
    u4 wr[kRing][kTilesPerWave];
    uint32_t sr[kRing][kTilesPerWave];
    uint32_t br[GEN ? kRing : 1][kTilesPerWave];
    auto load_b = [&](int slot, uint32_t kb) {
      const uint32_t kc = min(kb, kz - 1u);
      const uint32_t so = kc / d.gkb * sg.lds * 2u;
      const uint32_t grow = GEN ? plan_div(4u * kc + g4, d.g32, d.g32_m) : 0u;
#pragma unroll
      for (int t = 0; t < kTilesPerWave; ++t) {
        if constexpr (FMT == HQ_FORMAT_INT4) {
          wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b128(wrs[t], lane * 16u, kc * 1024u, 0);
        } else {
          const u2 v = __builtin_amdgcn_raw_buffer_load_b64(wrs[t], lane * 8u, kc * 512u, 0);
          wr[slot][t] = u4{v[0], v[1], 0u, 0u};
        }
        if constexpr (GEN) {
          sr[slot][t] = __builtin_amdgcn_raw_buffer_load_b16(srs, soff[t] + grow * sg.lds * 2u, 0, 0);
          br[slot][t] = __builtin_amdgcn_raw_buffer_load_b32(brs, soff[t] * 2u + grow * sg.lds * 4u, 0, 0);
        } else {
          sr[slot][t] = __builtin_amdgcn_raw_buffer_load_b16(srs, soff[t], so, 0);
        }
      }
    };
    const bool has_bias = GEN && sg.B != nullptr;

#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int t = 0; t < kTilesPerWave; ++t) acc[r][t] = f4{0.f, 0.f, 0.f, 0.f};

    // One k-block. Issue order per step: A(kb + 1) to LDS, then B(kb + kRing - 1) to
    // registers, so at the top of the next step vmcnt((kRing - 2) * kBLoads) leaves only the
    // B loads of later k-blocks in flight (none with a ring of two).
    constexpr int kBLoads = (GEN ? 3 : 2) * kTilesPerWave;  // weight, scale (and bias) loads per k-block
    auto step = [&](uint32_t kb, int slot) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((kRing - 2) * kBLoads));  // A(kb), B(kb) landed for this wave
      kblock_barrier();  // ... for every wave (of the half); stage (kb+1)&1 is free
      load_a((kb + 1) & 1u, kb + 1);
      load_b((slot + kRing - 1) % kRing, kb + kRing - 1);
      // Keep this step's loads ahead of its compute: vmcnt retires in issue order, so a load
      // sunk below the first use of this step's weights would be waited for with them.
      __builtin_amdgcn_sched_barrier(0);
      if (kb < kz) {  // uniform; no loads inside
        const char* sbase = stages + (kb & 1u) * kStageBytes;
        // Ternary: a group whose scale is not finite contributes nothing (its scale reads as 0).
        uint32_t sc[kTilesPerWave];
#pragma unroll
        for (int t = 0; t < kTilesPerWave; ++t)
          sc[t] = FMT == HQ_FORMAT_TERNARY2 && (sr[slot][t] & 0x7C00u) == 0x7C00u ? 0u : sr[slot][t];
        // GEN: chunk c's scale and addend of tile t come from lane 16 c + c16 of the loads.
        uint32_t gsc[GEN ? 4 : 1][kTilesPerWave], gadd[GEN ? 4 : 1][kTilesPerWave];
        if constexpr (GEN) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < kTilesPerWave; ++t) {
              const uint32_t sv = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((16u * c + c16) * 4u), (int)sc[t]) & 0xFFFFu;
              const uint32_t bv = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((16u * c + c16) * 4u), (int)br[slot][t]);
              gsc[c][t] = sv;
              if constexpr (FMT == HQ_FORMAT_INT4) {
                const float s32 = f16_to_f32((uint16_t)sv);
                if constexpr (DT == HQ_DTYPE_F16)  // e = 8 s + b (0 without a bias), as fp16
                  gadd[c][t] = has_bias ? f32_to_out<HQ_DTYPE_F16>(__builtin_fmaf(8.0f, s32, __builtin_bit_cast(float, bv))) : 0u;
                else  // the bias b (or -8 s), fp32
                  gadd[c][t] = has_bias ? bv : __builtin_bit_cast(uint32_t, -8.0f * s32);
              } else {
                gadd[c][t] = 0u;
              }
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u4 b[kTilesPerWave];
#pragma unroll
          for (int t = 0; t < kTilesPerWave; ++t) {
            if constexpr (GEN) b[t] = dq_scaled<FMT, DT, true>(wr[slot][t], c, gsc[c][t], dqk, gadd[c][t]);
            else b[t] = dq_scaled<FMT, DT>(wr[slot][t], c, sc[t], dqk);
          }
#pragma unroll
          for (int r = 0; r < RT; ++r) {
            const u4 a = *reinterpret_cast<const u4*>(sbase + (wrow0 + 16u * r) * 256u + ldsoff[c]);
#pragma unroll
            for (int t = 0; t < kTilesPerWave; ++t) acc[r][t] = mfma16x16x32<DT>(b[t], a, acc[r][t]);
          }
        }
        if constexpr (kOrdered) {
          // Instruction order of the k-block (fragment i = c * RT + r): the first kReadAhead
          // LDS reads and the first chunk's dequantisation, then per fragment the LDS read of
          // fragment i + kReadAhead, the four MFMAs of fragment i and a share of the next
          // chunk's dequantisation, so that no LDS round trip stands between MFMAs.
          // (Masks: 0x100 LDS reads, 0x008 MFMA, 0x002 VALU.)
          __builtin_amdgcn_sched_group_barrier(0x100, kReadAhead, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kValuFirst, 0);
#pragma unroll
          for (int i = 0; i < 4 * RT; ++i) {
            if (i + kReadAhead < 4 * RT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, kTilesPerWave, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, kValuPerFrag, 0);
          }
        }
      }
    };

    // Every wave is past the previous piece's last reads of both LDS stages.
    __syncthreads();
    // Prologue in ring order (no reordering across the barriers): the loop header's wait
    // counts assume slot kRing - 2 holds the youngest loads, as at the loop latch.
    load_a(ka & 1u, ka);
    load_b(0, ka);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kRing == 3) load_b(1, ka + 1);
    __builtin_amdgcn_sched_barrier(0);
    for (uint32_t kb = ka; kb < kz; kb += kRing) {
#pragma unroll
      for (int s = 0; s < kRing; ++s) step(kb + s, s);
    }
    __builtin_amdgcn_s_waitcnt(0);  // drain the prefetches past the piece
  };

  if constexpr (!SKP) {
    // Whole tiles, renumbered so that each XCD (consecutive workgroup ids go round-robin
    // over the 8 XCDs) owns a contiguous range of the visiting order, and visited in groups
    // of gb row bands (4 by default), column-block major inside a group: an XCD keeps the
    // group's activation rows near (its L2 and the MALL), and the gb tiles of one column
    // block run at about the same time, so their weight reads after the first hit L2.
    uint32_t tile = pp.xcd ? (bid % 8u) * (pp.dp / 8u) + bid / 8u : bid;
    if (pp.gb > 1u) {
      const uint32_t span = pp.gb * pp.nb;
      const uint32_t g = tile / span, r = tile - g * span;
      const uint32_t nbg = min(pp.gb, pp.bands - g * pp.gb);  // bands in this group
      const uint32_t cb = r / nbg;
      tile = (g * pp.gb + (r - cb * nbg)) * pp.nb + cb;
    }
    uint32_t s, m0, ct0;
    tile_geom<BM, TW>(d, pp.nb, tile, wn, s, m0, ct0);
    if constexpr (KS == 1) {
      run_piece(s, m0, ct0, 0u, nkb);
      __syncthreads();  // the output goes through the activation stages' LDS
      store_tile(s, m0, ct0);
    } else {
      // Halves of equal length (nkb even, checked by the host), so both meet every barrier.
      const uint32_t kmid = nkb / 2u;
      run_piece(s, m0, ct0, kh ? kmid : 0u, kh ? nkb : kmid);
      __syncthreads();  // both halves are done reading their stages
      f4* const part = reinterpret_cast<f4*>(smem) + wave * (RT * kTilesPerWave * 64u);
      if (kh) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
          for (int t = 0; t < kTilesPerWave; ++t) part[(r * kTilesPerWave + t) * 64u + lane] = acc[r][t];
      }
      __syncthreads();
      if (!kh) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
          for (int t = 0; t < kTilesPerWave; ++t) acc[r][t] += part[(r * kTilesPerWave + t) * 64u + lane];
      }
      __syncthreads();  // every partial is read before the output reuses the LDS
      if (!kh) store_tile(s, m0, ct0);
    }
    return;
  }

  // This workgroup's stream-K units (unit = tile * nkb + kb).
  const uint32_t u0 = pp.dp * nkb + plan_begin(pp.L, pp.rem, bid);
  const uint32_t u1 = pp.dp * nkb + plan_begin(pp.L, pp.rem, bid + 1u);

  // Stream-K pieces: the tiles of [u0, u1), at most two since a range is shorter than a
  // tile (L < nkb). Each goes to workspace slot 0 (first piece of the range) or 1 (last
  // piece); the fix-up stores every tile, also one that a range holds whole (its only
  // contributor is then the last). Keeping the output stores out of the piece loop keeps
  // their addresses out of the k-loop's registers.
  uint32_t ptile0 = ~0u, ptile1 = ~0u;
  for (uint32_t u = u0; u < u1;) {  // uniform
    const uint32_t tile = plan_div(u, nkb, pp.nkb_m);
    const uint32_t ka = u - tile * nkb;
    const uint32_t kz = min(nkb, u1 - tile * nkb);
    const bool first = u == u0;
    u = tile * nkb + kz;
    uint32_t s, m0, ct0;
    tile_geom<BM, TW>(d, pp.nb, tile, wn, s, m0, ct0);
    run_piece(s, m0, ct0, ka, kz);
    const uint32_t slot = first ? 0u : 1u;
    if (first) ptile0 = tile;
    else ptile1 = tile;
    const uint32_t base = (bid * 2u + slot) * kPartBytes + wave * kWavePart + lane * 16u;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int t = 0; t < kTilesPerWave; ++t)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[r][t]), partr,
                                               base + (uint32_t)(r * kTilesPerWave + t) * 1024u, 0, kCoherent);
  }


  // Fix-up: count arrivals per split tile; the last contributor sums every contributor's
  // partial in workgroup order (so the result does not depend on arrival order) and
  // stores the tile. Waiting for the coherent partial stores to complete before the
  // barrier orders them before the arrival count.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x < 2u) {
    const uint32_t tile = threadIdx.x == 0u ? ptile0 : ptile1;
    uint32_t last = 0;
    if (tile != ~0u) {
      const uint32_t rel = tile - pp.dp;
      const uint32_t bf = plan_wg_of_unit(pp.L, pp.rem, rel * nkb);
      const uint32_t bl = plan_wg_of_unit(pp.L, pp.rem, (rel + 1u) * nkb - 1u);
      const uint32_t old = __hip_atomic_fetch_add(pp.cnt + rel, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == bl - bf) {
        last = 1u;
        __hip_atomic_store(pp.cnt + rel, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    sh_last[threadIdx.x] = last;
  }
  __syncthreads();
  const uint32_t last0 = sh_last[0], last1 = sh_last[1];
  for (uint32_t i = 0; i < 2u; ++i) {
    if (!(i == 0u ? last0 : last1)) continue;
    const uint32_t tile = i == 0u ? ptile0 : ptile1;
    const uint32_t rel = tile - pp.dp;
    const uint32_t bf = plan_wg_of_unit(pp.L, pp.rem, rel * nkb);
    const uint32_t bl = plan_wg_of_unit(pp.L, pp.rem, (rel + 1u) * nkb - 1u);
    uint32_t s, m0, ct0;
    tile_geom<BM, TW>(d, pp.nb, tile, wn, s, m0, ct0);
    // The sum runs over the contributors in workgroup order from zero (this workgroup's
    // own partial is read back too: keeping it in registers across the fix-up would cost
    // the k-loop registers). Four row tiles at a time: all 16 loads of a contributor in
    // flight before the adds.
    constexpr int kRG = 4;
#pragma unroll
    for (int rg = 0; rg < RT; rg += kRG) {
#pragma unroll
      for (int r = rg; r < rg + kRG; ++r)
#pragma unroll
        for (int t = 0; t < kTilesPerWave; ++t) acc[r][t] = f4{0.f, 0.f, 0.f, 0.f};
      for (uint32_t c = bf; c <= bl; ++c) {  // contributors in workgroup order
        const uint32_t cslot = plan_div(plan_begin(pp.L, pp.rem, c), nkb, pp.nkb_m) == rel ? 0u : 1u;
        const uint32_t base = (c * 2u + cslot) * kPartBytes + wave * kWavePart + lane * 16u;
        u4 part[kRG][kTilesPerWave];
#pragma unroll
        for (int r = 0; r < kRG; ++r)
#pragma unroll
          for (int t = 0; t < kTilesPerWave; ++t)
            part[r][t] = __builtin_amdgcn_raw_buffer_load_b128(
                partr, base + (uint32_t)((rg + r) * kTilesPerWave + t) * 1024u, 0, kCoherent);
#pragma unroll
        for (int r = 0; r < kRG; ++r)
#pragma unroll
          for (int t = 0; t < kTilesPerWave; ++t) acc[rg + r][t] += __builtin_bit_cast(f4, part[r][t]);
      }
      store_tile(s, m0, ct0, rg, rg + kRG);
    }
  }
}

template <int FMT, int DT, int RT, int WM, int KS = 1>
constexpr size_t prefill_lds() {
  return 2u * KS * (16u * RT * WM) * 256u + 16u;
}

// Whole-tile workgroups one CU holds at once (1 if the device cannot be queried).
template <int FMT, int DT, int RT, int WM>
int prefill_occupancy() {
  static const int occ = [] {
    const void* f = reinterpret_cast<const void*>(&hq_prefill_kernel<FMT, DT, RT, WM, false>);
    int n = 0;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)prefill_lds<FMT, DT, RT, WM>()) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 256 * WM, prefill_lds<FMT, DT, RT, WM>()) != hipSuccess ||
        n < 1) {
      (void)hipGetLastError();
      n = 1;
    }
    return n;
  }();
  return occ;
}

// Column blocks: blk_begin = first column block (64 TW columns: 256, or 128 for TW = 2) of
// each segment in the global block order. Returns the number of blocks.
uint32_t assign_blocks(GemmDesc& d, int TW = kTilesPerWave) {
  uint32_t nb = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    d.seg[i].blk_begin = nb;
    d.seg[i].blk_count = (d.seg[i].ntiles + 4u * TW - 1u) / (4u * TW);
    nb += d.seg[i].blk_count;
  }
  return nb;
}

int env_int(const char* name, int dflt);

template <int FMT, int DT, int RT, int WM, bool GEN = false>
hipError_t launch_rt(const PrefillLaunch& c, void* ws, hipStream_t stream) {
  constexpr uint32_t BM = 16u * RT * WM;
  GemmDesc d = c.d;
  PrefillPlan pp{};
  pp.nb = assign_blocks(d);
  if ((d.M + BM - 1) / BM * pp.nb != c.tiles || c.dp + (c.psk ? 1u : 0u) > c.tiles) return hipErrorInvalidValue;
  pp.psk = c.psk;
  pp.dp = c.dp;
  pp.xcd = c.dp % 8u == 0u ? 1u : 0u;
  pp.bands = (d.M + BM - 1) / BM;
  // Band groups reorder whole-tile launches only (every tile of the launch is whole).
  pp.gb = c.dp == pp.bands * pp.nb ? (uint32_t)std::max(1, env_int("HQ_PREFILL_GB", 4)) : 1u;
  pp.nkb_m = plan_div_magic(d.nkb);
  if (c.psk) {
    if (!ws) return hipErrorInvalidValue;
    const uint32_t units = (c.tiles - c.dp) * d.nkb;
    pp.L = units / c.psk;
    pp.rem = units % c.psk;
    pp.cnt = static_cast<uint32_t*>(ws);
    pp.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  }
  const size_t lds = prefill_lds<FMT, DT, RT, WM>();
  // More than the default 64 KiB of dynamic LDS needs an opt-in per kernel (idempotent).
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_prefill_kernel<FMT, DT, RT, WM, false, GEN>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess
          ? hipErrorInvalidConfiguration
          : hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_prefill_kernel<FMT, DT, RT, WM, true, GEN>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  // Stream-K part first, then the whole tiles (stream order: one after the other).
  if (c.psk) {
    hipLaunchKernelGGL((hq_prefill_kernel<FMT, DT, RT, WM, true, GEN>), dim3(c.psk), dim3(256 * WM), lds, stream, d, pp);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (c.dp)
    hipLaunchKernelGGL((hq_prefill_kernel<FMT, DT, RT, WM, false, GEN>), dim3(c.dp), dim3(256 * WM), lds, stream, d, pp);
  return hipGetLastError();
}

// Whole 128-row tiles with the K split inside the workgroup (KS = 2): one tile per workgroup.
template <int FMT, int DT>
hipError_t launch_ks2(const PrefillLaunch& c, uint32_t* fault, uint32_t spin, hipStream_t stream) {
  GemmDesc d = c.d;
  PrefillPlan pp{};
  pp.fault = fault;
  pp.spin = spin;
  pp.nb = assign_blocks(d);
  if ((d.M + 127u) / 128u * pp.nb != c.tiles || c.psk != 0 || c.dp != c.tiles || d.nkb % 2u != 0 || d.nkb < 2u)
    return hipErrorInvalidValue;
  pp.dp = c.dp;
  pp.xcd = c.dp % 8u == 0u ? 1u : 0u;
  pp.bands = (d.M + 127u) / 128u;
  pp.gb = (uint32_t)std::max(1, env_int("HQ_PREFILL_GB", 4));
  pp.nkb_m = plan_div_magic(d.nkb);
  const size_t lds = prefill_lds<FMT, DT, 8, 1, 2>();
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_prefill_kernel<FMT, DT, 8, 1, false, false, 2>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((hq_prefill_kernel<FMT, DT, 8, 1, false, false, 2>), dim3(c.dp), dim3(512), lds, stream, d, pp);
  return hipGetLastError();
}

// Whole 128-row x 128-column tiles (TW = 2): one workgroup per tile, two per CU.
template <int FMT, int DT>
hipError_t launch_tw2(const PrefillLaunch& c, hipStream_t stream) {
  GemmDesc d = c.d;
  PrefillPlan pp{};
  pp.nb = assign_blocks(d, 2);
  if ((d.M + 127u) / 128u * pp.nb != c.tiles || c.psk != 0 || c.dp != c.tiles) return hipErrorInvalidValue;
  pp.dp = c.dp;
  pp.xcd = c.dp % 8u == 0u ? 1u : 0u;
  pp.bands = (d.M + 127u) / 128u;
  pp.gb = (uint32_t)std::max(1, env_int("HQ_PREFILL_GB", 4));
  pp.nkb_m = plan_div_magic(d.nkb);
  const size_t lds = prefill_lds<FMT, DT, 8, 1>();
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_prefill_kernel<FMT, DT, 8, 1, false, false, 1, 2>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((hq_prefill_kernel<FMT, DT, 8, 1, false, false, 1, 2>), dim3(c.dp), dim3(256), lds, stream, d, pp);
  return hipGetLastError();
}

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

// Tile height: 64 rows (RT 4, WM 1) up to M = 64, else 128 rows (8, 1), two workgroups per
// CU. Measured on MI355X at K = 5120, N = 27648: 128-row tiles two to a CU beat 256-row tiles
// (two row waves, one workgroup per CU) by 3-8% from M = 512 to 4096.
void prefill_shape(uint32_t M, int& RT, int& WM) {
  const int eWM = env_int("HQ_PREFILL_WM", 0);  // tuning override: 128 (1) or 256 (2) rows
  const int eRT = env_int("HQ_PREFILL_RT", 0);  // tuning override: 4 = 64 rows
  if (eRT == 4) {
    RT = 4;
    WM = 1;
  } else if (eWM == 1 || eWM == 2) {
    RT = 8;
    WM = eWM;
  } else if (M <= 64) {
    RT = 4;
    WM = 1;
  } else {
    RT = 8;
    WM = 1;
  }
}

// Concurrent workgroups of the chosen shape on this device. The f16 instantiation stands
// for both dtypes, so that the plan (and the workspace size) does not depend on the dtype.
int prefill_slots(int fmt, int RT, int WM) {
  int occ = 1;
  if (fmt == HQ_FORMAT_INT4) {
    occ = RT == 4 ? prefill_occupancy<HQ_FORMAT_INT4, HQ_DTYPE_F16, 4, 1>()
                  : (WM == 1 ? prefill_occupancy<HQ_FORMAT_INT4, HQ_DTYPE_F16, 8, 1>()
                             : prefill_occupancy<HQ_FORMAT_INT4, HQ_DTYPE_F16, 8, 2>());
  } else {
    occ = RT == 4 ? prefill_occupancy<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16, 4, 1>()
                  : (WM == 1 ? prefill_occupancy<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16, 8, 1>()
                             : prefill_occupancy<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16, 8, 2>());
  }
  return cu_count() * occ;
}

template <int FMT, int DT>
hipError_t launch_fd(const PrefillLaunch& c, void* ws, uint32_t* fault, uint32_t spin, hipStream_t stream) {
  if (c.d.gen) return c.RT == 4 && c.WM == 1 ? launch_rt<FMT, DT, 4, 1, true>(c, ws, stream) : hipErrorInvalidConfiguration;
  if (c.KS == 2) return c.RT == 8 && c.WM == 1 ? launch_ks2<FMT, DT>(c, fault, spin, stream) : hipErrorInvalidConfiguration;
  if (c.TW == 2) return c.RT == 8 && c.WM == 1 ? launch_tw2<FMT, DT>(c, stream) : hipErrorInvalidConfiguration;
  if (c.RT == 4) return launch_rt<FMT, DT, 4, 1>(c, ws, stream);
  if (c.WM == 1) return launch_rt<FMT, DT, 8, 1>(c, ws, stream);
  return launch_rt<FMT, DT, 8, 2>(c, ws, stream);
}

// Global column blocks [cb0, cb1) of d as a descriptor of their own: segments outside
// dropped, the others' weight, scale and output pointers advanced to their first column.
GemmDesc column_range(int fmt, const GemmDesc& d, uint32_t cb0, uint32_t cb1) {
  GemmDesc out = d;
  out.nseg = 0;
  const size_t tile_words = (size_t)d.nkb * 64u * words_per_lane(fmt);
  uint32_t cb = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    const SegDesc& g = d.seg[i];
    const uint32_t nb = (g.ntiles + 15u) / 16u;
    const uint32_t lo = std::max(cb0, cb) - cb, hi = std::min(cb1, cb + nb);
    if (cb + lo < hi) {
      SegDesc t = g;
      const uint32_t c0 = lo * 256u;
      t.Wp = g.Wp + (size_t)lo * 16u * tile_words;
      t.S = g.S + c0;
      t.B = g.B ? g.B + c0 : nullptr;
      t.Y = static_cast<char*>(g.Y) + (size_t)c0 * 2u;
      t.N = std::min<uint32_t>(g.N, (hi - cb) * 256u) - c0;
      t.ntiles = col_tiles(t.N);
      out.seg[out.nseg++] = t;
    }
    cb += nb;
  }
  return out;
}

uint32_t count_blocks(const GemmDesc& d, int TW = kTilesPerWave) {
  GemmDesc t = d;
  return assign_blocks(t, TW);
}

PrefillLaunch make_launch(int RT, int WM, const GemmDesc& d, int TW = kTilesPerWave) {
  PrefillLaunch l{};
  l.RT = RT;
  l.WM = WM;
  l.KS = 1;
  l.TW = TW;
  l.d = d;
  l.tiles = (d.M + 16u * RT * WM - 1) / (16u * RT * WM) * count_blocks(d, TW);
  l.dp = l.tiles;
  l.psk = 0;
  return l;
}

}  // namespace

// Tiling of a prefill call (tile heights 128 / 64 rows as M allows; 256 on request):
//  * A grid of at most half the workgroup slots is split s ways along K (stream-K,
//    s = floor(slots / tiles), at most nkb / 4 so that a range keeps 4 k-blocks): s *
//    tiles workgroups, each one aligned tile fraction, each tile s contributors.
//  * Otherwise, for 256-row tiles, when the last round of whole tiles would be part-empty,
//    the last k column blocks (just enough to empty that round) run as a second launch of
//    half-height tiles, if those fit in one round: the tail then takes half a round.
//  * Otherwise whole tiles.
namespace {
PrefillConfig choose_prefill_256(int fmt, const GemmDesc& d, size_t ws_cap) {
  PrefillConfig c{};
  int RT = 8, WM = 2;
  prefill_shape(d.M, RT, WM);
  if (d.gen) {  // the general kernels: 64-row tiles only
    RT = 4;
    WM = 1;
  }
  // 128-row tiles too few for the slots would be split along K; when those pieces would be
  // short (under 64 k-blocks) 64-row tiles do better: twice the tiles, split half as often
  // or not at all. Measured on MI355X: fused QKV (N = 7168) M = 256..1024 7-38% faster,
  // 27648 x 4096 at M = 192..512 2-33% faster, 28672 x 8192 at M = 192 and 320 7-20%
  // faster; with long pieces (K = 27648, M = 1024) the 128-row split stays (64-row tiles
  // there: 40% slower). Except over a long K (64 k-blocks or more) where the 64-row tiles
  // would cover three quarters of the CUs and so run whole (no stream-K), each streaming all
  // of K: there the 128-row split (at most eight ways) measured 8-39% faster in every case
  // (best of two alternated runs, M = 384..512: 8192 x 8192 87.2 -> 77.6 us, 10240 x 8192
  // 107 -> 75-90, 16384 x 8192 168 -> 118-127, 28672 x 8192 289 -> 177-195).
  const uint32_t cus = (uint32_t)cu_count();
  if (RT == 8 && WM == 1 && env_int("HQ_PREFILL_RT", 0) == 0 && env_int("HQ_PREFILL_WM", 0) == 0) {
    const uint32_t t128 = make_launch(8, 1, d).tiles, s128 = (uint32_t)prefill_slots(fmt, 8, 1);
    const uint32_t split = std::min<uint32_t>(s128 / std::max(t128, 1u), d.nkb / 4u);
    if (4u * t128 >= 3u * cus && 2u * t128 <= s128) {
      // One round of 128-row tiles covering at least three quarters of the CUs: whole tiles.
      // Measured on MI355X (K = 5120, alternated runs): fused QKV (N = 7168) M = 1024, 224
      // tiles: 77.5 us against 82.5 with 448 64-row tiles; N = 27648 M = 256, 216 tiles: 75.9
      // against 80.9.
    } else if (split >= 2u && d.nkb / split < 64u) {
      const uint32_t t64 = make_launch(4, 1, d).tiles;
      if (!(d.nkb >= 64u && split <= 8u && 4u * t64 >= 3u * cus)) RT = 4;
    } else if (split < 2u) {
      // Whole tiles either way: compare rounds, in units of a full 128-row round. A part-empty
      // last round that leaves at most one workgroup per CU costs 0.35 + 0.45 x its fill (its
      // lone workgroups run faster); a fuller one 0.35 + 0.65 x its fill with 128-row tiles
      // and a whole round with 64-row tiles (several per CU). A 64-row tile computes its
      // rows at 0.76 (int4: its dequantisation is shared by half as many rows) or 0.915
      // (ternary) of a 128-row tile's rate, so a round of s64 64-row tiles costs
      // (s64 * 64) / (s128 * 128) / rate. Measured on MI355X (K = 5120; ternary N = 27648,
      // 34816, 55296 and int4 N = 27648, 55296 at M = 384..2048): this picks the faster
      // height in every case, e.g. ternary N = 34816 at M = 512 (544 128-row tiles) 64-row
      // tiles 7% faster, at M = 2048 128-row tiles 10% faster; int4 N = 27648 at M = 384
      // 128-row tiles 12% faster.
      const uint32_t t64 = make_launch(4, 1, d).tiles, s64 = (uint32_t)prefill_slots(fmt, 4, 1);
      // 128-row tiles a few past one per CU, when 64-row tiles fit two per CU: the CUs that
      // take a second 128-row tile set the time. Measured on MI355X (best of three alternated
      // runs, M = 136..192): int4 5120 x 34816 / 36864 and 4096 x 40960 (272-320 128-row
      // tiles) 17-20% faster with 64-row tiles (4096 x 40960 M = 160: 80.3 -> 64.8 us); at
      // M = 224, 256 (64-row tiles past two per CU) 128-row tiles stay 4% ahead.
      if (t128 > cus && t64 <= 2u * cus) RT = 4;
      const double rate64 = fmt == HQ_FORMAT_INT4 ? 0.76 : 0.915;
      const double round64 = (double)s64 * 64.0 / ((double)s128 * 128.0) / rate64;
      auto rounds = [](uint32_t t, uint32_t sl, double full) {
        const double f = (double)(t % sl) / (double)sl;
        return (double)(t / sl) + (t % sl ? (f <= 0.5 ? 0.35 + 0.45 * f : full * (0.35 + 0.65 * f) + (1.0 - full)) : 0.0);
      };
      if (round64 * rounds(t64, s64, 0.0) < rounds(t128, s128, 1.0)) RT = 4;
    }
  }
  c.n = 1;
  c.l[0] = make_launch(RT, WM, d);
  PrefillLaunch& l = c.l[0];
  // One round of whole 128-row tiles, at most one per CU and at least three quarters of them:
  // the K split inside the workgroup (KS = 2) keeps two wavefronts on every SIMD.
  // HQ_PREFILL_KS = 1 turns it off, = 2 forces it for any whole-tile fast call (tests).
  const int eks = env_int("HQ_PREFILL_KS", 0);
  if (RT == 8 && WM == 1 && !d.gen && d.nkb % 2u == 0u && d.nkb >= 8u && eks != 1 &&
      (eks == 2 || (l.tiles <= cus && 4u * l.tiles >= 3u * cus))) {
    l.KS = 2;
    return c;
  }
  const uint32_t slots = (uint32_t)prefill_slots(fmt, RT, WM);
  const int epsk = env_int("HQ_PREFILL_PSK", 0);  // tuning / test override: stream-K grid
  if (env_int("HQ_PREFILL_SK", 1) != 0 && d.nkb >= 8u && l.tiles <= kMaxCounters &&
      (uint64_t)l.tiles * d.nkb < (1ull << 31)) {
    uint32_t psk = std::min<uint32_t>(slots / l.tiles, d.nkb / 4u) * l.tiles;
    if (epsk > 0) psk = std::min<uint32_t>((uint32_t)epsk, l.tiles * d.nkb);
    // Under a workspace cap: as many whole s-way splits as the partial tiles fit in.
    const size_t per_wg = 2u * (16u * RT * WM) * 256u * sizeof(float);
    if (ws_cap != SIZE_MAX) {
      const size_t fit = ws_cap > kCounterBytes ? (ws_cap - kCounterBytes) / per_wg : 0u;
      if (psk > fit) psk = epsk > 0 ? (uint32_t)fit : (uint32_t)(fit / l.tiles) * l.tiles;
    }
    // Stream-K only for grids that leave more than a quarter of the CUs idle: whole tiles
    // covering three quarters of them or more measured faster (fused QKV M = 512, 224 64-row
    // tiles: 58.2 against 66.3 us split two ways; N = 27648 M = 128, 216 tiles: 58.2 against
    // 62.0); at 112 tiles and fewer the split still wins (QKV M = 256: 46.2 against 56.3).
    if (psk > l.tiles && ((psk >= 2u * l.tiles && 4u * l.tiles < 3u * cus) || epsk > 0)) {
      l.psk = psk;
      l.dp = 0;
      return c;
    }
  }
  // Part-empty last rounds of 128-row tiles (two per CU) cost little: a lone workgroup has
  // its CU to itself. Measured on MI355X (M = 1024, 2048, 4096 at N = 27648) and slower
  // than whole tiles: 64-row tail tiles (their dequantisation is shared by half as many
  // rows) and a stream-K launch over the last round's tiles (its partial-tile traffic).
  // Only 256-row tiles get the half-height tail launch.
  const uint32_t r = l.tiles % slots;
  if (WM == 1) return c;
  if (env_int("HQ_PREFILL_TAIL", 1) == 0 || r == 0u) return c;
  const int hRT = RT * WM / 2;  // half-height tiles of one row wave: 256 -> 128, 128 -> 64 rows
  const uint32_t bands = (d.M + 16u * RT * WM - 1) / (16u * RT * WM);
  const uint32_t nb = count_blocks(d);
  const uint32_t k = (r + bands - 1) / bands;
  if (k >= nb) return c;
  const PrefillLaunch tail = make_launch(hRT, 1, column_range(fmt, d, nb - k, nb));
  if (tail.tiles > (uint32_t)prefill_slots(fmt, hRT, 1)) return c;
  c.n = 2;
  c.l[0] = make_launch(RT, WM, column_range(fmt, d, 0, nb - k));
  c.l[1] = tail;
  return c;
}

bool env_set(const char* name) {
  const char* v = std::getenv(name);
  return v && *v;
}
}  // namespace

// The plan over 256-column tiles, then 128-row x 128-column whole tiles (TW = 2, four
// wavefronts of 32 columns, two workgroups per CU) in place of a one-round whole-tile grid
// that leaves the CUs one workgroup each or uneven: at the same tile count as 64-row tiles
// each dequantised weight serves twice the rows, and against a 128-row tile split in two K
// halves the CU holds two independent tiles. The choice depends on the activation type (the
// fp16 256-column kernel runs an explicit instruction order, the bf16 one forms its weights
// in fp32) but not the workspace: every plan it swaps needs none. Measured on MI355X (best of
// two alternated runs, K = 4096..5120, M = 81..1536):
//  * in place of 64-row whole tiles (216-344): 8-18% faster for int4 fp16 (5120 x 7168
//    M = 768 79.6 -> 68.9 us), 7-30% for bf16 (5120 x 34816 M = 96 104.6 -> 80.5 us), 5-11%
//    for ternary fp16 where the 64-row tiles outnumber the CUs (216 tiles at 5120 x 27648:
//    -4..+2%);
//  * in place of the K split (192-256 tiles): fp16 3-6% faster (the fused QKV width at M =
//    1024, int4: 72.8 -> 68.8 us), bf16 within -4..+2%;
//  * in place of 272-336 128-row whole tiles (544-672 128-column tiles): bf16 8-11% faster,
//    also over a long K (27648 x 5120, 17408 x 5120, 16384 x 6144, 8192 x 8192 at M = 1152..
//    2048: 8-13%), fp16 6-13% slower; bf16 at 408 (816) 8% slower, at 432-1728 (864-3456) up
//    to 11% slower.
// Stream-K plans (short grids, long K) stay: 128-column tiles there were 1-40% slower.
PrefillConfig choose_prefill(int fmt, const GemmDesc& d, size_t ws_cap, int dtype) {
  PrefillConfig c = choose_prefill_256(fmt, d, ws_cap);
  if (d.gen || c.n != 1) return c;
  PrefillLaunch& l = c.l[0];
  const int etw = env_int("HQ_PREFILL_TW", 0);  // tuning / test override: 2 forces, 1 forbids
  if (etw == 2) {
    if (l.RT == 8 && l.WM == 1) l = make_launch(8, 1, d, 2);
    return c;
  }
  if (etw == 1 || d.M <= 64u || l.psk != 0 || l.dp != l.tiles) return c;
  for (const char* e : {"HQ_PREFILL_RT", "HQ_PREFILL_WM", "HQ_PREFILL_KS", "HQ_PREFILL_PSK", "HQ_PREFILL_SK"})
    if (env_set(e)) return c;  // a forced 256-column plan stays
  const uint32_t cus = (uint32_t)cu_count();
  const PrefillLaunch t2 = make_launch(8, 1, d, 2);
  const bool f16 = dtype == HQ_DTYPE_F16;
  const bool one_round = t2.tiles <= 2u * cus;
  // In place of 64-row tiles only while the 128-row bands add at most a quarter more rows
  // (M = 136..192 would compute up to a third more).
  // Ternary fp16 keeps 64-row tiles that all fit one per CU (5120 x 27648 at M = 81..128, 216
  // tiles: 4% faster than 128-column tiles at M = 128, within 2% below).
  const bool rows_ok = 8u * ((d.M + 127u) / 128u) <= 5u * ((d.M + 63u) / 64u) &&
                       !(fmt == HQ_FORMAT_TERNARY2 && f16 && l.tiles <= cus);
  const bool use = (l.RT == 4 && l.WM == 1 && one_round && rows_ok) || (l.KS == 2 && f16 && one_round) ||
                   (!f16 && l.RT == 8 && l.WM == 1 && l.KS == 1 && l.tiles > cus && 4u * t2.tiles <= 11u * cus);
  if (use) l = t2;
  return c;
}

size_t prefill_workspace_bytes(const GemmDesc& d, const PrefillConfig& c) {
  (void)d;
  size_t b = 0;
  for (int i = 0; i < c.n; ++i)
    if (c.l[i].psk)
      b = std::max(b, kCounterBytes + (size_t)c.l[i].psk * 2u * (16u * c.l[i].RT * c.l[i].WM) * 256u * sizeof(float));
  return b;
}

hipError_t launch_prefill(int fmt, int dtype, const PrefillConfig& c, void* ws, uint32_t* fault, uint32_t spin,
                          hipStream_t stream) {
  for (int i = 0; i < c.n; ++i) {
    const PrefillLaunch& l = c.l[i];
    hipError_t e;
    if (fmt == HQ_FORMAT_INT4)
      e = dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_F16>(l, ws, fault, spin, stream)
                                : launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_BF16>(l, ws, fault, spin, stream);
    else
      e = dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16>(l, ws, fault, spin, stream)
                                : launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_BF16>(l, ws, fault, spin, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace hq

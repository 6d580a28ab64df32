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
// already is the v_mfma_f32_16x16x32 B-fragment order. Accumulation is fp32 (AGPRs).
// Workgroups are renumbered so that each XCD owns a contiguous band of row blocks and
// keeps its activation rows resident in its own L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "hq_device.hpp"
#include "hq_internal.hpp"

namespace hq {
namespace {

constexpr int kTilesPerWave = 4;  // 64 columns per wavefront, 256 per workgroup

// Dequantised B fragment with the group scale applied. s2 holds the fp16 scale twice.
template <int FMT, int DT>
__device__ __forceinline__ u4 dq_scaled(const u4& w, int c, uint32_t s_f16, const DqConst& k) {
  if constexpr (DT == HQ_DTYPE_F16) {
    const h2 s2 = bits_h2(s_f16 | (s_f16 << 16));
    u4 q;
    if constexpr (FMT == HQ_FORMAT_INT4) {
      q = dq_int4_f16(w[c], k);  // exact q - 8
    } else {
      const uint32_t word = w[c >> 1];
      q = (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);  // exact 2t; the epilogue halves
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
      const float ms = -8.0f * s;
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

template <int FMT, int DT, int RT, int WM>
__global__ void __launch_bounds__(256 * WM) hq_prefill_kernel(const GemmDesc d, uint32_t mtiles, uint32_t total_wg) {
  constexpr uint32_t BM = 16u * RT * WM;
  constexpr uint32_t kStageBytes = BM * 256u;  // BM rows x 128 fp16
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t c16 = lane & 15u, g4 = lane >> 4;

  // XCD-aware renumbering: consecutive workgroup ids are spread round-robin over the 8
  // XCDs; give each XCD a contiguous range of logical tiles (row-block major).
  uint32_t lid = blockIdx.x;
  if (total_wg % 8u == 0u) lid = (blockIdx.x % 8u) * (total_wg / 8u) + blockIdx.x / 8u;
  uint32_t s = 0;
#pragma unroll
  for (uint32_t i = 1; i < HQ_MAX_SEGMENTS; ++i)
    if (i < d.nseg && lid >= d.seg[i].blk_begin) s = i;
  const SegDesc sg = d.seg[s];
  const uint32_t nblk = (sg.ntiles + 15u) / 16u;
  const uint32_t local = lid - sg.blk_begin;
  const uint32_t mt = local / nblk, nt = local % nblk;
  const uint32_t m0 = mt * BM;
  const uint32_t wm = wave / 4u, wn = wave % 4u;
  const uint32_t ct0 = nt * 16u + wn * kTilesPerWave;
  const uint32_t wrow0 = wm * 16u * RT;  // first workgroup row of this wavefront

  // Activation rows [m0, m0 + BM) of X; rows >= M read as zero.
  const uint32_t rows = min(BM, d.M - m0);
  const __amdgpu_buffer_rsrc_t xr =
      make_rsrc(reinterpret_cast<const char*>(d.X) + (size_t)m0 * (size_t)d.ldx * 2u, rows * (uint32_t)d.ldx * 2u);
  // This lane's part of the wave's RT load instructions per k-block (BM / 4 in all): instruction
  // i fills LDS rows 4q..4q+3, q = wave * RT + i; lane -> row 4q + g4, 16-byte slot c16
  // holding unit c16 ^ (row & 15).
  uint32_t aoff[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const uint32_t q = wave * RT + i;
    const uint32_t r = 4u * q + g4;
    aoff[i] = (r * (uint32_t)d.ldx + 8u * (c16 ^ (r & 15u))) * 2u;
  }
  auto load_a = [&](uint32_t stage, uint32_t kb) {
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const uint32_t q = wave * RT + i;
      buffer_to_lds16(xr, smem + stage * kStageBytes + q * 1024u, aoff[i] + kb * 256u);
    }
  };

  // Weights: one descriptor per column tile of this wavefront.
  __amdgpu_buffer_rsrc_t wrs[kTilesPerWave];
  uint32_t soff[kTilesPerWave];
  const uint32_t tile_bytes = d.nkb * 64u * (FMT == HQ_FORMAT_INT4 ? 16u : 8u);
#pragma unroll
  for (int t = 0; t < kTilesPerWave; ++t) {
    const uint32_t ct = ct0 + t;
    const bool ok = ct < sg.ntiles;
    wrs[t] = make_rsrc(reinterpret_cast<const char*>(sg.Wp) + (size_t)(ok ? ct : 0u) * tile_bytes, ok ? tile_bytes : 0u);
    soff[t] = min(ct * 16u + c16, sg.N - 1u) * 2u;
  }
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(sg.S, (d.nkb / d.gkb) * sg.N * 2u);
  // Weights and scales: a register ring of 3 k-blocks, two ahead of the one computed.
  // Loads past the last k-block read zero (empty range) instead of branching.
  u4 wr[3][kTilesPerWave];
  uint32_t sr[3][kTilesPerWave];
  auto load_b = [&](int slot, uint32_t kb) {
    const bool ok = kb < d.nkb;
    const uint32_t grp = min(kb, d.nkb - 1u) / d.gkb;
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) {
      if constexpr (FMT == HQ_FORMAT_INT4) {
        wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b128(wrs[t], ok ? (kb * 64u + lane) * 16u : kOutOfRange, 0, 0);
      } else {
        const u2 v = __builtin_amdgcn_raw_buffer_load_b64(wrs[t], ok ? (kb * 64u + lane) * 8u : kOutOfRange, 0, 0);
        wr[slot][t] = u4{v[0], v[1], 0u, 0u};
      }
      sr[slot][t] = __builtin_amdgcn_raw_buffer_load_b16(srs, grp * sg.N * 2u + soff[t], 0, 0);
    }
  };

  const DqConst dqk = dq_const_f16();
  f4 acc[RT][kTilesPerWave];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < kTilesPerWave; ++t) acc[r][t] = f4{0.f, 0.f, 0.f, 0.f};

  // LDS fragment addresses: row 16 r + c16, unit (4 c + g4) ^ c16.
  uint32_t ldsoff[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) ldsoff[c] = c16 * 256u + (((4u * c + g4) ^ c16) * 16u);

  const uint32_t nkb = d.nkb;
  // One k-block. Issue order per step: A(kb + 1) to LDS, then B(kb + 2) to registers, so
  // at the top of the next step vmcnt(2 * kTilesPerWave) leaves only B(kb + 2) in flight.
  auto step = [&](uint32_t kb, int slot) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kTilesPerWave));  // A(kb), B(kb) landed for this wave
    __syncthreads();                                            // ... for every wave; stage (kb+1)&1 is free
    load_a((kb + 1) & 1u, kb + 1);
    load_b((slot + 2) % 3, kb + 2);
    // Keep this step's loads ahead of its compute: vmcnt retires in issue order, so a load
    // sunk below the first use of this step's weights would be waited for with them.
    __builtin_amdgcn_sched_barrier(0);
    if (kb < nkb) {  // uniform; no loads inside
      const char* sbase = smem + (kb & 1u) * kStageBytes;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        u4 b[kTilesPerWave];
#pragma unroll
        for (int t = 0; t < kTilesPerWave; ++t) b[t] = dq_scaled<FMT, DT>(wr[slot][t], c, sr[slot][t], dqk);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const u4 a = *reinterpret_cast<const u4*>(sbase + (wrow0 + 16u * r) * 256u + ldsoff[c]);
#pragma unroll
          for (int t = 0; t < kTilesPerWave; ++t) acc[r][t] = mfma16x16x32<DT>(a, b[t], acc[r][t]);
        }
      }
    }
  };

  // Prologue in ring order (no reordering across the barriers): the loop header's wait
  // counts assume slot 1 holds the youngest loads, as at the loop latch.
  load_a(0, 0);
  load_b(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_b(1, 1);
  __builtin_amdgcn_sched_barrier(0);
  for (uint32_t kb = 0; kb < nkb; kb += 3) {
    step(kb, 0);
    step(kb + 1, 1);
    step(kb + 2, 2);
  }
  __builtin_amdgcn_s_waitcnt(0);  // drain the out-of-range prefetches before the stores

  // Epilogue: tile (r, t), lane -> column 16 (ct0 + t) + c16, rows 16 r + 4 g4 + v. Rows past M
  // fall outside the descriptor; columns past N get an out-of-range offset.
  constexpr float post = (FMT == HQ_FORMAT_TERNARY2 && DT == HQ_DTYPE_F16) ? 0.5f : 1.0f;
  const __amdgpu_buffer_rsrc_t yr =
      make_rsrc(reinterpret_cast<char*>(sg.Y) + (size_t)m0 * (size_t)sg.ldy * 2u, rows * (uint32_t)sg.ldy * 2u);
#pragma unroll
  for (int t = 0; t < kTilesPerWave; ++t) {
    const uint32_t n = (ct0 + t) * 16u + c16;
    const uint32_t cbase = n < sg.N ? n * 2u : kOutOfRange;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t row = wrow0 + 16u * r + 4u * g4 + v;
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_out<DT>(acc[r][t][v] * post), yr,
                                              cbase == kOutOfRange ? kOutOfRange : cbase + row * (uint32_t)sg.ldy * 2u, 0, 0);
      }
  }
}

template <int FMT, int DT, int RT, int WM>
hipError_t launch_rt(GemmDesc d, hipStream_t stream) {
  constexpr uint32_t BM = 16u * RT * WM;
  const uint32_t mtiles = (d.M + BM - 1) / BM;
  uint32_t blk = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    d.seg[i].blk_begin = blk;
    d.seg[i].blk_count = mtiles * ((d.seg[i].ntiles + 15u) / 16u);
    blk += d.seg[i].blk_count;
  }
  const size_t lds = 2u * BM * 256u;
  // More than the default 64 KiB of dynamic LDS needs an opt-in per kernel (idempotent).
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_prefill_kernel<FMT, DT, RT, WM>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((hq_prefill_kernel<FMT, DT, RT, WM>), dim3(blk), dim3(256 * WM), lds, stream, d, mtiles, blk);
  return hipGetLastError();
}

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

template <int FMT, int DT>
hipError_t launch_fd(GemmDesc d, hipStream_t stream) {
  const int eWM = env_int("HQ_PREFILL_WM", 0);  // tuning override: workgroup height 128 (1) or 256 (2) rows
  if (eWM == 1) return launch_rt<FMT, DT, 8, 1>(d, stream);
  if (eWM == 2) return launch_rt<FMT, DT, 8, 2>(d, stream);
  if (d.M <= 64) return launch_rt<FMT, DT, 4, 1>(d, stream);
  if (d.M <= 128) return launch_rt<FMT, DT, 8, 1>(d, stream);
  return launch_rt<FMT, DT, 8, 2>(d, stream);
}

}  // namespace

hipError_t launch_prefill(int fmt, int dtype, GemmDesc d, hipStream_t stream) {
  if (fmt == HQ_FORMAT_INT4) {
    return dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_F16>(d, stream)
                                 : launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_BF16>(d, stream);
  }
  return dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16>(d, stream)
                               : launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_BF16>(d, stream);
}

}  // namespace hq

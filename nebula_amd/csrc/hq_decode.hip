// hq_decode.hip — memory-bound qGEMM for M <= 16 (decode), gfx950.
//
// Replaces kernel_marlin_gemm_int4_templated / _dynamic
// (hydrogen/src/model/marlin_gemm.cu:130-237, 242-322). The reference gives each
// thread one output column and does 32 x M scalar FMAs per 16-byte weight load,
// then merges 16 fixed K-splits with fp32 atomics into a pre-zeroed Y. Here:
//   * one wavefront streams T column tiles (16 columns each) over its K range, one
//     fully coalesced wave load (1 KiB int4 / 512 B ternary) per tile and k-block,
//     with U k-blocks of weights, scales and activations in flight in a register ring
//     (HBM latency is ~2 us, so bytes in flight, not wave count, set the bandwidth);
//   * weights are dequantised in registers straight into MFMA B fragments and
//     multiplied against the activation rows (M padded to 16) with
//     v_mfma_f32_16x16x32_{f16,bf16}: the k reduction happens inside the matrix core
//     instead of lane-by-lane FMAs and shuffles;
//   * the group scale multiplies the fp32 group sum once per (column, group);
//   * WK wavefronts of a workgroup split K and are reduced through LDS in a fixed
//     order, so the result is deterministic and Y needs no zero-fill or atomics.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "hq_device.hpp"
#include "hq_internal.hpp"

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

template <int FMT, int DT>
__device__ __forceinline__ u4 dequant_chunk(const typename WTraits<FMT>::V& w, int c, const DqConst& k) {
  if constexpr (FMT == HQ_FORMAT_INT4) {
    if constexpr (DT == HQ_DTYPE_F16) return dq_int4_f16(w[c], k);
    else return dq_int4_bf16_biased(w[c], k);
  } else {
    const uint32_t word = w[c >> 1];
    return (c & 1) ? dq_tern2<1>(word) : dq_tern2<0>(word);
  }
}

// Constant bf16 -1.5 in every B element: MFMA(x, this) = -1.5 * sum_k x over the chunk.
constexpr uint32_t kBf16NegOneHalf2 = 0xBFC0BFC0u;

// Largest workgroup (in wavefronts) per tile width: the deep register rings of T >= 2 need
// more than the 128 VGPRs a 16-wave workgroup leaves each lane.
constexpr int max_wk(int T) { return T >= 2 ? 8 : 16; }

template <int FMT, int DT, int T, int U>
__global__ void __launch_bounds__(64 * max_wk(T)) hq_decode_kernel(const GemmDesc d, uint32_t kb_per_wave) {
  using W = typename WTraits<FMT>::V;
  constexpr uint32_t WPL = WTraits<FMT>::wpl;
  constexpr bool kBiased = (FMT == HQ_FORMAT_INT4 && DT == HQ_DTYPE_BF16);
  extern __shared__ float red[];

  const uint32_t lane = threadIdx.x & 63u;
  // Wave index through readfirstlane so the compiler keeps all k-block arithmetic scalar.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t nwave = blockDim.x >> 6;
  const uint32_t c16 = lane & 15u;
  const uint32_t g4 = lane >> 4;

  // Segment of this workgroup (segments are few; the scan is uniform).
  uint32_t s = 0;
#pragma unroll
  for (uint32_t i = 1; i < HQ_MAX_SEGMENTS; ++i)
    if (i < d.nseg && blockIdx.x >= d.seg[i].blk_begin) s = i;
  const SegDesc sg = d.seg[s];
  const uint32_t ct0 = (blockIdx.x - sg.blk_begin) * T;

  const uint32_t kb0 = wave * kb_per_wave;
  const uint32_t kb1 = min(d.nkb, kb0 + kb_per_wave);

  // A operand: row c16 of X, k-slice g4 of each chunk. Rows >= M fall outside the
  // descriptor and read as zero.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(d.X, d.M * (uint32_t)d.ldx * 2u);
  const uint32_t xoff = c16 * (uint32_t)d.ldx * 2u + g4 * 16u;

  // One descriptor per column tile; tiles past the segment get an empty descriptor.
  __amdgpu_buffer_rsrc_t wrs[T];
  uint32_t soff[T];
  const uint32_t tile_bytes = d.nkb * 64u * WPL * 4u;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t ct = ct0 + t;
    const bool ok = ct < sg.ntiles;
    wrs[t] = make_rsrc(sg.Wp + (size_t)(ok ? ct : 0u) * d.nkb * 64u * WPL, ok ? tile_bytes : 0u);
    // Padding columns read column N-1's scale; their outputs are never stored.
    soff[t] = min(ct * 16u + c16, sg.N - 1u) * 2u;
  }
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(sg.S, (d.nkb / d.gkb) * sg.N * 2u);
  const uint32_t srow = sg.N * 2u;

  // Register ring: slot u holds k-block kb0 + u (mod U) of weights, scales and activations,
  // issued together. vmcnt retires loads in issue order, so anything fetched later than
  // the weights it is used with would drain the whole ring; one issue point per k-block
  // keeps U - 1 k-blocks in flight. Loads past the wave's range read zero.
  W wr[U][T];
  uint16_t sr[U][T];
  u4 ar[U][4];
  auto load = [&](int slot, uint32_t kb) {
    const bool ok = kb < kb1;
    // Scales past the range re-read the last group (2 bytes, cached) instead of branching.
    const uint32_t grp = min(kb, kb1 - 1u) / d.gkb;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t wo = ok ? (kb * 64u + lane) * WPL * 4u : kOutOfRange;
      if constexpr (WPL == 4) wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b128(wrs[t], wo, 0, kStreamAux);
      else wr[slot][t] = __builtin_amdgcn_raw_buffer_load_b64(wrs[t], wo, 0, kStreamAux);
      sr[slot][t] = __builtin_amdgcn_raw_buffer_load_b16(srs, grp * srow + soff[t], 0, 0);
    }
    const uint32_t base = ok ? xoff + kb * 256u : kOutOfRange;
#pragma unroll
    for (int c = 0; c < 4; ++c) ar[slot][c] = __builtin_amdgcn_raw_buffer_load_b128(xr, base, c * 64u, 0);
  };

  const DqConst dqk = DT == HQ_DTYPE_F16 ? dq_const_f16() : dq_const_bf16();
  f4 acc[T], gacc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    gacc[t] = f4{0.f, 0.f, 0.f, 0.f};
  }
  f4 corr = f4{0.f, 0.f, 0.f, 0.f};

  // Issue the prologue in slot order (no reordering across the barriers): the loop
  // header's wait count is the worst case over both paths into it, so the preheader
  // must leave slot 0 as the oldest load, as the loop latch does.
#pragma unroll
  for (int u = 0; u < U; ++u) {
    load(u, kb0 + u);
    __builtin_amdgcn_sched_barrier(0);
  }

  for (uint32_t kb = kb0; kb < kb1; kb += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t k = kb + u;
      if (k < kb1) {  // uniform; no loads inside, so waitcnt stays exact across it
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            gacc[t] = mfma16x16x32<DT>(ar[u][c], dequant_chunk<FMT, DT>(wr[u][t], c, dqk), gacc[t]);
        }
        if constexpr (kBiased) {
          const u4 neg = u4{kBf16NegOneHalf2, kBf16NegOneHalf2, kBf16NegOneHalf2, kBf16NegOneHalf2};
#pragma unroll
          for (int c = 0; c < 4; ++c) corr = mfma16x16x32<DT>(ar[u][c], neg, corr);
        }
        if ((k + 1u) % d.gkb == 0u) {
#pragma unroll
          for (int t = 0; t < T; ++t) {
            float sc = f16_to_f32(sr[u][t]);
            if constexpr (FMT == HQ_FORMAT_TERNARY2) {
              // A non-finite block scale drops the block (native_decoder.cu:174); fields hold 2t.
              sc = __builtin_isfinite(sc) ? 0.5f * sc : 0.0f;
            }
            if constexpr (kBiased) {
              sc *= 16.0f;
              gacc[t] += corr;
            }
            acc[t] += gacc[t] * sc;
            gacc[t] = f4{0.f, 0.f, 0.f, 0.f};
          }
          corr = f4{0.f, 0.f, 0.f, 0.f};
        }
      }
      load(u, k + U);
    }
  }

  // Output element e = (t * 4 + v) * 64 + ln: row 4 * (ln / 16) + v, column 16 * (ct0 + t) + ln % 16.
  auto store = [&](uint32_t e, float val) {
    const uint32_t t = e >> 8, v = (e >> 6) & 3u, ln = e & 63u;
    const uint32_t row = 4u * (ln >> 4) + v;
    const uint32_t n = (ct0 + t) * 16u + (ln & 15u);
    if (row < d.M && n < sg.N && ct0 + t < sg.ntiles)
      reinterpret_cast<uint16_t*>(sg.Y)[(size_t)row * sg.ldy + n] = f32_to_out<DT>(val);
  };

  if (nwave == 1) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) store((t * 4 + v) * 64 + lane, acc[t][v]);
    return;
  }
  constexpr uint32_t per_wave = T * 4 * 64;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave * per_wave + (t * 4 + v) * 64 + lane] = acc[t][v];
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < per_wave; e += blockDim.x) {
    float sum = 0.0f;
    for (uint32_t w = 0; w < nwave; ++w) sum += red[w * per_wave + e];
    store(e, sum);
  }
}

struct DecodeConfig {
  int T;
  int WK;
};

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

// Tiling choice (measured on MI355X over the 27B-class decode shapes): wide tiles (T=4)
// amortise the activation fragments over 64 columns when N offers >= 1024 tiles, T=2
// for mid-size N, T=1 below; four wavefronts per workgroup split K.
DecodeConfig choose_decode(const GemmDesc& d) {
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) tiles += d.seg[i].ntiles;
  const uint32_t groups = d.nkb / d.gkb;
  int T = tiles >= 1024 ? 4 : (tiles >= 300 ? 2 : 1);
  int WK = 4;
  const int eT = env_int("HQ_DECODE_T", 0), eWK = env_int("HQ_DECODE_WK", 0);
  if (eT == 1 || eT == 2 || eT == 4) T = eT;
  if (eWK >= 1) WK = eWK;
  WK = std::max(1, std::min<int>(std::min<int>(WK, max_wk(T)), (int)groups));
  return {T, WK};
}

template <int FMT, int DT, int T, int U>
hipError_t launch_t(GemmDesc d, int WK, hipStream_t stream) {
  uint32_t blk = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    d.seg[i].blk_begin = blk;
    d.seg[i].blk_count = (d.seg[i].ntiles + T - 1) / T;
    blk += d.seg[i].blk_count;
  }
  const uint32_t groups = d.nkb / d.gkb;
  const uint32_t gpw = (groups + WK - 1) / WK;
  const uint32_t kb_per_wave = gpw * d.gkb;
  const size_t lds = WK > 1 ? (size_t)WK * T * 4 * 64 * sizeof(float) : 0;
  hipLaunchKernelGGL((hq_decode_kernel<FMT, DT, T, U>), dim3(blk), dim3(64 * WK), lds, stream, d, kb_per_wave);
  return hipGetLastError();
}

template <int FMT, int DT>
hipError_t launch_fd(GemmDesc d, hipStream_t stream) {
  const DecodeConfig cfg = choose_decode(d);
  switch (cfg.T) {
    case 4: return launch_t<FMT, DT, 4, 4>(d, cfg.WK, stream);
    case 2: return launch_t<FMT, DT, 2, 4>(d, cfg.WK, stream);
    default: return launch_t<FMT, DT, 1, 4>(d, cfg.WK, stream);
  }
}

}  // namespace

hipError_t launch_decode(int fmt, int dtype, GemmDesc d, hipStream_t stream) {
  if (fmt == HQ_FORMAT_INT4) {
    return dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_F16>(d, stream)
                                 : launch_fd<HQ_FORMAT_INT4, HQ_DTYPE_BF16>(d, stream);
  }
  return dtype == HQ_DTYPE_F16 ? launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_F16>(d, stream)
                               : launch_fd<HQ_FORMAT_TERNARY2, HQ_DTYPE_BF16>(d, stream);
}

}  // namespace hq

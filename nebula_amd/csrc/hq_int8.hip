// hq_int8.hip — the int8 path: int8 weights x activations quantised to int8, gfx950 i8 MFMA.
//
// Replaces kernel_cutlass_int8_gemm / forward_cutlass_int8 (hydrogen/src/model/marlin_gemm.cu:
// 327-377, 603-617), which the reference never launches: activations quantised as
// int8(clamp(x * 127, -128, 127)) converted toward zero (:356-359), int8 weights [K][N]
// (q * 16 - 128 of its int4 codes, :508), y = scale[n] * sum_k xq w / 127 with one scale per
// column (:371-375). Two launches, or one when a workgroup's activation rows are small:
//   1. hq_quantize_x_kernel: the M x K activations once to int8 (the workspace), so the GEMM
//      copies 1 byte per element instead of re-reading fp32 rows in every workgroup; when the
//      rows of a workgroup's K piece are at most one 16-element unit per thread (M = 1 at
//      K = 5120), the GEMM reads them as fp32 and quantises them itself (QX);
//   2. hq_w8a8_kernel: the X-resident structure of the int4 decode kernel (hq_decode.hip): one
//      workgroup per (slab of T column tiles, piece of K), the piece's int8 rows copied into
//      LDS by LDS-DMA, then a barrier-free register ring of weight steps (T tiles x one
//      128-deep k-block, 2 KiB per tile) into v_mfma_i32_16x16x64_i8. Sums are int32 and exact,
//      across wavefronts (LDS) and K pieces (workspace, last arriver), so the result does not
//      depend on the decomposition; the reference's fp32 quad-by-quad accumulation differs from
//      it by at most its own rounding.
//
// Weight tile layout: column tile ct (16 columns) x k-block kb (128) is 2 KiB at byte
// (ct * nkb + kb) * 2048; lane l holds 32 bytes: chunk c (64 k) at 16 c, elements
// k = 128 kb + 64 c + 16 (l / 16) + i (i = 0..15) of column 16 ct + l % 16, the B operand of
// the MFMA (lane l: column l % 16, k-slice l / 16). N is padded to 16 columns of zeros.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "hq_device.hpp"
#include "hq_internal.hpp"
#include "hq_plan.hpp"

namespace hq {
namespace {

typedef int32_t i4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) hq_quantize_x_kernel(const float* __restrict__ X, uint32_t ldx,
                                                            int8_t* __restrict__ Xq, uint32_t M, uint32_t K) {
  // Four consecutive elements per thread (K is a multiple of 128).
  const uint32_t i = (blockIdx.x * 256u + threadIdx.x) * 4u;
  if (i >= M * K) return;
  const uint32_t r = i / K, k = i % K;
  const float4 x = *reinterpret_cast<const float4*>(X + (size_t)r * ldx + k);
  uint32_t packed = 0;
  const float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // fminf(fmaxf(x * 127, -128), 127) converted toward zero; NaN -> -128 (fmaxf).
    const float t = fminf(fmaxf(v[e] * 127.0f, -128.0f), 127.0f);
    packed |= ((uint32_t)(int32_t)t & 0xFFu) << (8 * e);
  }
  *reinterpret_cast<uint32_t*>(Xq + (size_t)r * K + k) = packed;
}

struct W8Plan {
  const int8_t* Xq;  // [M][K] int8 activations
  const float* X;    // [M][ldx] fp32 activations (QX)
  uint32_t ldx;
  const int8_t* Wp;  // tile layout
  const float* S;    // [N] scales
  float* Y;
  uint32_t ldy, M, K, N, nkb, ntiles;
  uint32_t wk;       // wavefronts per workgroup
  uint32_t S_;       // pieces per slab (grid y)
  uint32_t kq, kr;   // piece p: k-blocks [p * kq + min(p, kr), ...), kq + (p < kr) of them
  uint32_t m_lo, m_hi;  // plan_div_magic(8 * kq), plan_div_magic(8 * (kq + 1))
  uint32_t* cnt;     // [slabs] arrival counters (S_ > 1)
  int32_t* part;     // [slabs][S_][M * 16 * T] partial sums (S_ > 1)
};

constexpr int w8_max_wk(int T) { return T >= 4 ? 8 : 16; }

// LDS layout of a piece's activation rows (nkbp k-blocks): 16-byte units, unit
// (r * nkbp + kb - kb0) * 8 + (j ^ (r & 7)) holds elements 16 j .. 16 j + 15 of k-block kb of row
// r (j = 0..7); an A fragment read of chunk c (piece j = 4 c + g4) spreads eight rows over every
// bank. Lanes of rows >= M read row M - 1 (their output rows are never stored).
// The quantiser of hq_quantize_x_kernel on one value: clamp(x * 127) toward zero, NaN -> -128.
__device__ __forceinline__ uint32_t quantize_int8(float v) {
  const float t = fminf(fmaxf(v * 127.0f, -128.0f), 127.0f);
  return (uint32_t)(int32_t)t & 0xFFu;
}

template <int T, int U, bool QX>
__global__ void __launch_bounds__(64 * w8_max_wk(T)) hq_w8a8_kernel(const W8Plan pl) {
  constexpr uint32_t kCols = 16u * T;
  extern __shared__ __attribute__((aligned(16))) char xs[];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t c16 = lane & 15u, g4 = lane >> 4;
  const uint32_t g = blockIdx.x, p = blockIdx.y;
  const uint32_t WK = pl.wk, nkb = pl.nkb, M = pl.M, K = pl.K, N = pl.N;
  const uint32_t kq = pl.kq, kr = pl.kr, m_lo = pl.m_lo, m_hi = pl.m_hi;
  const int8_t* const Xq = pl.Xq;
  asm volatile("" ::"s"(WK), "s"(nkb), "s"(M), "s"(K), "s"(kq), "s"(kr), "s"(m_lo), "s"(m_hi), "s"(Xq));
  const uint32_t kb0 = p * kq + min(p, kr);
  const uint32_t nkbp = kq + (p < kr ? 1u : 0u);
  const uint32_t ct0 = g * T;
  const uint32_t nv = min((uint32_t)T, pl.ntiles - ct0);

  // 1. The piece's int8 rows -> LDS (64 units of 16 bytes per LDS-DMA instruction), or (QX)
  //    each thread's unit of fp32 elements into registers, quantised once the ring is issued.
  const uint32_t xu = threadIdx.x;  // QX: this thread's unit (LDS bytes 16 xu .. 16 xu + 15)
  bool xlive = false;
  f4 xv[4];
  if constexpr (QX) {
    const uint32_t nkb8 = nkbp * 8u;
    const uint32_t m8 = p < kr ? m_hi : m_lo;
    const uint32_t r = plan_div(xu, nkb8, m8);
    const uint32_t rem = xu - r * nkb8;
    xlive = r < M;
    const uint32_t voff =
        xlive ? (r * pl.ldx + (kb0 + (rem >> 3)) * 128u + (((rem & 7u) ^ (r & 7u)) * 16u)) * 4u : kOutOfRange;
    const __amdgpu_buffer_rsrc_t xf = make_rsrc(pl.X, M * pl.ldx * 4u);
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(xf, voff, 16u * i, 0));
  } else {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(Xq, M * K);
    const uint32_t nkb8 = nkbp * 8u;
    const uint32_t m8 = p < kr ? m_hi : m_lo;
    const uint32_t nq = (M * nkb8 + 63u) / 64u;
    for (uint32_t q = wave; q < nq; q += WK) {
      const uint32_t u = q * 64u + lane;
      const uint32_t r = plan_div(u, nkb8, m8);
      const uint32_t rem = u - r * nkb8;
      const uint32_t voff = r < M ? r * K + (kb0 + (rem >> 3)) * 128u + (((rem & 7u) ^ (r & 7u)) * 16u) : kOutOfRange;
      buffer_to_lds16(xr, xs + q * 1024u, voff);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. Weight ring: step j is k-block kb0 + wave + j * WK, T tiles of 32 bytes per lane.
  const uint32_t nj = wave < nkbp ? (nkbp - wave + WK - 1u) / WK : 0u;
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(pl.Wp + (size_t)ct0 * nkb * 2048u, __builtin_amdgcn_readfirstlane(nv * nkb * 2048u));
  uint32_t wvo[T];
#pragma unroll
  for (int t = 0; t < T; ++t) wvo[t] = lane * 32u + (uint32_t)t * nkb * 2048u;
  u4 wr[U][T][2];
  auto load = [&](int slot, uint32_t j) {
    const bool live = j < nj;
    const uint32_t kbo = __builtin_amdgcn_readfirstlane(live ? (kb0 + wave + j * WK) * 2048u : 0u);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t vo = live ? wvo[t] : kOutOfRange;
      wr[slot][t][0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, vo, kbo, kStreamAux);
      wr[slot][t][1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, vo + 16u, kbo, kStreamAux);
    }
  };
#pragma unroll
  for (int u = 0; u < U; ++u) load(u, (uint32_t)u);
  __builtin_amdgcn_sched_barrier(0);
  // Wait for this wavefront's copies only (the ring's 2 T U loads were issued after them).
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * T * U));
  if constexpr (QX) {
    if (xlive) {
      u4 q;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        q[i] = quantize_int8(xv[i][0]) | (quantize_int8(xv[i][1]) << 8) | (quantize_int8(xv[i][2]) << 16) |
               (quantize_int8(xv[i][3]) << 24);
      *reinterpret_cast<u4*>(xs + xu * 16u) = q;
    }
  }
  __syncthreads();

  const uint32_t xrow = min(c16, M - 1u);
  uint32_t xa[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) xa[c] = (xrow * nkbp * 8u + ((4u * c + g4) ^ (xrow & 7u))) * 16u;
  i4 acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = i4{0, 0, 0, 0};
  auto compute = [&](int u, uint32_t j) {
    const uint32_t kbl = wave + j * WK;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const i4 a = *reinterpret_cast<const i4*>(xs + xa[c] + kbl * 128u);
#pragma unroll
      for (int t = 0; t < T; ++t)
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, __builtin_bit_cast(i4, wr[u][t][c]), acc[t], 0, 0, 0);
    }
  };
  for (uint32_t j = 0; j < nj; j += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j + u < nj) compute(u, j + u);  // uniform; no loads inside, so waitcnt stays exact across it
      load(u, j + u + U);
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // 3. Exact int32 sums over the wavefronts (LDS, over the rows), then over the pieces.
  __syncthreads();
  const uint32_t SL = M * kCols;
  int32_t* red = reinterpret_cast<int32_t*>(xs);
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint32_t row = 4u * g4 + v;
      if (row < M) red[wave * SL + row * kCols + t * 16u + c16] = acc[t][v];
    }
  __syncthreads();
  const uint32_t nthr = WK * 64u;
  constexpr int kCoherent = 16;  // sc1: agent-coherent partials
  const uint32_t S = pl.S_;
  const __amdgpu_buffer_rsrc_t partr = make_rsrc(pl.part, S > 1u ? gridDim.x * S * SL * 4u : 0u);
  if (S > 1u) {
    for (uint32_t o4 = threadIdx.x; o4 < SL / 4u; o4 += nthr) {
      i4 v = i4{0, 0, 0, 0};
      for (uint32_t w = 0; w < WK; ++w) v += *reinterpret_cast<const i4*>(red + w * SL + 4u * o4);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), partr, ((g * S + p) * SL + 4u * o4) * 4u, 0,
                                             kCoherent);
    }
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
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(pl.S, N * 4u);
  for (uint32_t o4 = threadIdx.x; o4 < SL / 4u; o4 += nthr) {
    i4 v = i4{0, 0, 0, 0};
    if (S > 1u) {
      for (uint32_t q = 0; q < S; ++q)
        v += __builtin_bit_cast(i4, __builtin_amdgcn_raw_buffer_load_b128(partr, ((g * S + q) * SL + 4u * o4) * 4u,
                                                                          0, kCoherent));
    } else {
      for (uint32_t w = 0; w < WK; ++w) v += *reinterpret_cast<const i4*>(red + w * SL + 4u * o4);
    }
    const uint32_t o = 4u * o4, row = o / kCols, lc = o % kCols, n = ct0 * 16u + lc;
    if (lc >= nv * 16u) continue;
    float* y = pl.Y + (size_t)row * pl.ldy + n;
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
      if (n + e < N) {
        const float s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srs, (n + e) * 4u, 0, 0));
        y[e] = (float)v[e] * (1.0f / 127.0f) * s;
      }
    }
  }
}

int w8_env(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

uint32_t w8_x_bytes(uint32_t M, uint32_t nkb, int S) {
  const uint32_t nkbp = (nkb + (uint32_t)S - 1u) / (uint32_t)S;
  return (M * nkbp * 8u + 63u) / 64u * 1024u;
}

uint32_t w8_lds_bytes(uint32_t M, uint32_t nkb, int T, int WK, int S) {
  return std::max(w8_x_bytes(M, nkb, S), (uint32_t)WK * M * 16u * (uint32_t)T * 4u);
}

template <int T, int U, bool QX>
hipError_t w8_launch_t(const W8Config& c, W8Plan pl, hipStream_t stream) {
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hq_w8a8_kernel<T, U, QX>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kXrLdsMax);
  if (attr != hipSuccess) return attr;
  if (c.WK < 1 || c.WK > w8_max_wk(T)) return hipErrorInvalidValue;
  // QX: every unit of a piece's rows has a thread (the kernel quantises one unit per thread).
  if (QX && pl.M * (pl.kq + (pl.kr ? 1u : 0u)) * 8u > 64u * (uint32_t)c.WK) return hipErrorInvalidValue;
  const uint32_t G = (pl.ntiles + T - 1) / T;
  hipLaunchKernelGGL((hq_w8a8_kernel<T, U, QX>), dim3(G, pl.S_), dim3(64 * c.WK), c.lds, stream, pl);
  return hipGetLastError();
}

}  // namespace

// Tiling, as for the X-resident int4 kernel: the fewest K pieces whose int8 rows fit in LDS,
// then the narrowest slabs (T = 2 or 4 tiles; a step is 4 or 8 KiB of weights per wavefront)
// whose grid fits on the CUs in one round with eight wavefronts per workgroup, two steps in
// flight; pieces also when whole slabs leave more than half of the CUs idle.
// HQ_W8_T / _WK / _S override (tuning and tests).
W8Config choose_w8a8(uint32_t M, uint32_t K, uint32_t N) {
  W8Config c{2, 2, 8, 1, 0, false};
  if (M < 1 || M > 16 || K % 128 || N == 0) return c;
  const uint32_t nkb = K / 128, ntiles = (N + 15) / 16;
  const uint32_t cus = (uint32_t)cu_count();
  bool found = false;
  for (int s = 1; s <= 16 && !found; ++s) {
    if ((uint32_t)s > nkb || w8_x_bytes(M, nkb, s) > kXrLdsMax) continue;
    for (int t : {2, 4}) {
      const uint32_t lds = w8_lds_bytes(M, nkb, t, 8, s);
      const uint32_t per_cu = std::min<uint32_t>(2u, kXrLdsMax / lds);  // 2 x 8 waves (<= 128 VGPRs)
      const uint32_t slabs = (ntiles + t - 1) / t, wgs = slabs * (uint32_t)s;
      if (per_cu < 1 || wgs > cus * per_cu) continue;
      if (s == 1 && wgs * 2u < cus && nkb >= 2) break;  // whole slabs leave most CUs idle
      c = W8Config{t, 2, 8, s, lds, false};
      found = true;
      break;
    }
  }
  const int eT = w8_env("HQ_W8_T", 0), eWK = w8_env("HQ_W8_WK", 0), eS = w8_env("HQ_W8_S", 0);
  if (eT == 2 || eT == 4) c.T = eT;
  if (eWK >= 1) c.WK = std::min(eWK, w8_max_wk(c.T));
  if (eS >= 1) c.S = std::min<int>(eS, (int)nkb);
  if (!found && !(eT || eWK || eS)) return c;
  c.lds = w8_lds_bytes(M, nkb, c.T, c.WK, c.S);
  c.ok = c.lds <= kXrLdsMax && (ntiles + c.T - 1) / c.T <= kMaxCounters;
  // One launch when each thread has at most one 16-element unit of its piece's rows to
  // quantise (M = 1 at K = 5120: the separate launch cost ~2 us of 31.8); HQ_W8_QX = 0 keeps
  // the quantisation launch.
  const uint32_t nkbp = (nkb + (uint32_t)c.S - 1u) / (uint32_t)c.S;
  c.qx = c.ok && M * nkbp * 8u <= 64u * (uint32_t)c.WK && w8_env("HQ_W8_QX", 1) != 0;
  return c;
}

// Workspace: the counter area, the pieces' partial sums, then the int8 activations.
size_t w8a8_workspace_bytes(uint32_t M, uint32_t K, uint32_t N, const W8Config& c) {
  const size_t slabs = ((N + 15) / 16 + c.T - 1) / c.T;
  const size_t part = c.S > 1 ? (size_t)slabs * c.S * M * 16u * c.T * 4u : 0u;
  const size_t xq = ((size_t)M * K + 255u) / 256u * 256u;
  return kCounterBytes + (part + 255u) / 256u * 256u + xq;
}

hipError_t launch_w8a8(const float* X, uint32_t ldx, const int8_t* Wp, const float* scales, float* Y, uint32_t ldy,
                       uint32_t M, uint32_t K, uint32_t N, const W8Config& c, void* ws, hipStream_t stream) {
  if (!c.ok || !ws) return hipErrorInvalidValue;
  const uint32_t nkb = K / 128;
  const size_t slabs = ((N + 15) / 16 + c.T - 1) / c.T;
  const size_t part = c.S > 1 ? (size_t)slabs * c.S * M * 16u * c.T * 4u : 0u;
  char* w = static_cast<char*>(ws);
  int8_t* Xq = reinterpret_cast<int8_t*>(w + kCounterBytes + (part + 255u) / 256u * 256u);
  // 32-bit buffer offsets: the int8 rows, a slab's weights and the partials.
  if ((uint64_t)M * K >= (1ull << 31) || (uint64_t)c.T * nkb * 2048u >= (1ull << 31) || part >= (1ull << 31) ||
      (uint64_t)N * 4u >= (1ull << 31))
    return hipErrorInvalidValue;
  if (!c.qx) {
    const uint32_t n4 = M * K / 4u;
    hipLaunchKernelGGL(hq_quantize_x_kernel, dim3((n4 + 255u) / 256u), dim3(256), 0, stream, X, ldx, Xq, M, K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  W8Plan pl{};
  pl.Xq = Xq;
  pl.X = X;
  pl.ldx = ldx;
  pl.Wp = Wp;
  pl.S = scales;
  pl.Y = Y;
  pl.ldy = ldy;
  pl.M = M;
  pl.K = K;
  pl.N = N;
  pl.nkb = nkb;
  pl.ntiles = (N + 15) / 16;
  pl.wk = (uint32_t)c.WK;
  pl.S_ = (uint32_t)c.S;
  pl.kq = nkb / pl.S_;
  pl.kr = nkb % pl.S_;
  pl.m_lo = plan_div_magic(8u * pl.kq);
  pl.m_hi = plan_div_magic(8u * (pl.kq + 1u));
  pl.cnt = static_cast<uint32_t*>(ws);
  pl.part = reinterpret_cast<int32_t*>(w + kCounterBytes);
  switch (c.T) {
    case 2: return c.qx ? w8_launch_t<2, 2, true>(c, pl, stream) : w8_launch_t<2, 2, false>(c, pl, stream);
    case 4: return c.qx ? w8_launch_t<4, 2, true>(c, pl, stream) : w8_launch_t<4, 2, false>(c, pl, stream);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace hq

// hq_bench_qgemm — benchmark and acceptance tool for the gfx950 weight-only qGEMM.
//
// The MI355X counterpart of hydrogen/src/tools/bench_marlin_gemm.cpp (the reference's only
// caller of MarlinGemmEngine, BENCH:26-155): same options (--json --k --n --group --iters
// --warmups -h) and the same JSON keys, driven through the library's C ABI
// (include/hq_qgemm.h). Differences, all deliberate:
//   * "marlin" is hq_gemm_w4a16 (or hq_gemm_w2a16 with --format ternary2); "baseline" is a
//     plain HIP kernel of the reference's naive int4 GEMM shape (one thread per column,
//     dequantise then fp32 FMA; MG.cu:76-117);
//   * the numerical reference is a plain fp32 dequantise-then-matmul kernel on the GPU, as
//     in the reference (MG.cu:52-70); activations and outputs are fp16 (bf16 with
//     --dtype bf16), so the gate is the normwise relative error <= 1e-2 (the reference's
//     1e-3 absolute gate does not transfer to fp16 outputs of magnitude ~6); max_abs_error
//     and mse are reported as in MG.cu:619-644;
//   * bytes per launch are the packed weights + fp16 scales + X + Y actually moved
//     (the reference counts its fp32 scales, biases, X and Y, MG.cu:673-675), against the
//     MI355X HBM peak of 8 TB/s;
//   * weights rotate over >= 640 MiB of copies by default (--rotate-mib 0 reuses one copy,
//     as the reference does), so the 256 MiB Infinity Cache cannot serve them.
// Exit status 0 iff every acceptance check passes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "hq_qgemm.h"

namespace {

#define HIP_OK(x)                                                                                 \
  do {                                                                                            \
    hipError_t e_ = (x);                                                                          \
    if (e_ != hipSuccess) {                                                                       \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(2);                                                                               \
    }                                                                                             \
  } while (0)

#define HQ_OK(x)                                                                                   \
  do {                                                                                             \
    hq_status s_ = (x);                                                                            \
    if (s_ != HQ_OK) {                                                                             \
      std::fprintf(stderr, "hq error %d (%s) at %s:%d\n", (int)s_, hq_last_error(), __FILE__, __LINE__); \
      std::exit(2);                                                                                \
    }                                                                                              \
  } while (0)

constexpr double kHbmPeakGBs = 8000.0;

void print_help(const char* prog) {
  std::printf(
      "Usage: %s [options]\n\n"
      "Options:\n"
      "  --json             Output structured JSON telemetry\n"
      "  --k <N>            Matrix dimension K (default: 4096)\n"
      "  --n <N>            Matrix dimension N (default: 4096)\n"
      "  --group <N>        Quantization group size (default: 128)\n"
      "  --iters <N>        Timed benchmark iterations (default: 20)\n"
      "  --warmups <N>      Warmup iterations (default: 5)\n"
      "  --m <list>         Comma-separated batch sizes (default: 1,2,4,8)\n"
      "  --format <f>       int4 (default) or ternary2\n"
      "  --dtype <d>        f16 (default) or bf16 activations and outputs\n"
      "  --rotate-mib <N>   Distinct weight copies totalling >= N MiB (default: 640; 0 = one copy)\n"
      "  -h, --help         Display this help message\n",
      prog);
}

// splitmix64 stream for the synthetic data.
struct Rng {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
  double normal() { return std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform()); }
};

uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  u += 0x7FFFu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
  return (uint16_t)(u >> 16);
}
float bf16_to_f32(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

// ---- comparison kernels (not part of the library) --------------------------------------

__device__ float act_to_f32(uint16_t v, int bf16) {
  return bf16 ? __builtin_bit_cast(float, (uint32_t)v << 16) : (float)__builtin_bit_cast(_Float16, v);
}

// Dequantised weight of the linear layouts: int4 [K/8][N] (nibble i = k % 8, value q - 8)
// or ternary [K/16][N] (2-bit code c = t + 1 at bits 2 (k % 16)).
__device__ float weight_of(const uint32_t* W, int fmt, uint32_t k, uint32_t n, uint32_t N) {
  if (fmt == HQ_FORMAT_INT4) return (float)((int)((W[(size_t)(k / 8) * N + n] >> (4 * (k % 8))) & 15u) - 8);
  return (float)((int)((W[(size_t)(k / 16) * N + n] >> (2 * (k % 16))) & 3u) - 1);
}

// Reference: Y[m][n] = sum_k x[m][k] * w(k, n) * s(k / g, n), fp32, k ascending.
__global__ void reference_gemm(const uint16_t* X, int bf16, const uint32_t* W, int fmt, const uint16_t* S, float* Y,
                               uint32_t M, uint32_t K, uint32_t N, uint32_t group) {
  const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.0f;
  for (uint32_t k = 0; k < K; ++k) {
    float s = (float)__builtin_bit_cast(_Float16, S[(size_t)(k / group) * N + n]);
    if (fmt == HQ_FORMAT_TERNARY2 && !__builtin_isfinite(s)) s = 0.0f;
    acc = __builtin_fmaf(act_to_f32(X[(size_t)m * K + k], bf16), weight_of(W, fmt, k, n, N) * s, acc);
  }
  Y[(size_t)m * N + n] = acc;
}

// Baseline: one thread per column streams its linear weight words and keeps M fp32
// accumulators (the naive int4 kernel shape of the reference).
template <int MB>
__global__ void baseline_gemm(const uint16_t* X, int bf16, const uint32_t* W, int fmt, const uint16_t* S, uint16_t* Y,
                              uint32_t M, uint32_t K, uint32_t N, uint32_t group) {
  const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float acc[MB];
  for (int m = 0; m < MB; ++m) acc[m] = 0.0f;
  const uint32_t per = fmt == HQ_FORMAT_INT4 ? 8u : 16u, bits = fmt == HQ_FORMAT_INT4 ? 4u : 2u;
  const uint32_t mask = (1u << bits) - 1u, zero = fmt == HQ_FORMAT_INT4 ? 8u : 1u;
  for (uint32_t kw = 0; kw < K / per; ++kw) {
    const uint32_t word = W[(size_t)kw * N + n];
    const float s = (float)__builtin_bit_cast(_Float16, S[(size_t)(kw * per / group) * N + n]);
    for (uint32_t i = 0; i < per; ++i) {
      const float w = (float)((int)((word >> (bits * i)) & mask) - (int)zero) * s;
      const uint32_t k = kw * per + i;
      for (int m = 0; m < MB; ++m)
        if ((uint32_t)m < M) acc[m] = __builtin_fmaf(act_to_f32(X[(size_t)m * K + k], bf16), w, acc[m]);
    }
  }
  for (int m = 0; m < MB; ++m)
    if ((uint32_t)m < M) {
      const float v = acc[m];
      Y[(size_t)m * N + n] = bf16 ? (uint16_t)(__builtin_bit_cast(uint32_t, v) >> 16)
                                  : __builtin_bit_cast(uint16_t, (_Float16)v);
    }
}

struct SweepResult {
  uint32_t M;
  double latency_ms, baseline_ms, speedup, gbs, util_pct, tflops, max_abs, mse, normwise;
  bool numerical, latency_ok;
};

}  // namespace

int main(int argc, char** argv) {
  bool json = false;
  uint32_t K = 4096, N = 4096, group = 128;
  int iters = 20, warmups = 5;
  std::vector<uint32_t> Ms = {1, 2, 4, 8};
  hq_format fmt = HQ_FORMAT_INT4;
  hq_dtype dt = HQ_DTYPE_F16;
  double rotate_mib = 640.0;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "missing value for %s\n", a.c_str());
        std::exit(2);
      }
      return argv[++i];
    };
    if (a == "--json") json = true;
    else if (a == "--k") K = (uint32_t)std::stoul(next());
    else if (a == "--n") N = (uint32_t)std::stoul(next());
    else if (a == "--group") group = (uint32_t)std::stoul(next());
    else if (a == "--iters") iters = std::stoi(next());
    else if (a == "--warmups") warmups = std::stoi(next());
    else if (a == "--rotate-mib") rotate_mib = std::stod(next());
    else if (a == "--format") {
      const std::string f = next();
      fmt = f == "ternary2" ? HQ_FORMAT_TERNARY2 : HQ_FORMAT_INT4;
    } else if (a == "--dtype") {
      dt = std::string(next()) == "bf16" ? HQ_DTYPE_BF16 : HQ_DTYPE_F16;
    } else if (a == "--m") {
      Ms.clear();
      std::string s = next();
      size_t p = 0;
      while (p < s.size()) {
        size_t q = s.find(',', p);
        if (q == std::string::npos) q = s.size();
        Ms.push_back((uint32_t)std::stoul(s.substr(p, q - p)));
        p = q + 1;
      }
    } else if (a == "-h" || a == "--help") {
      print_help(argv[0]);
      return 0;
    }
  }
  const uint32_t Mmax = *std::max_element(Ms.begin(), Ms.end());
  if (Mmax > 16 || Ms.empty()) {
    std::fprintf(stderr, "--m values must be in 1..16 (decode sweep)\n");
    return 2;
  }
  const int bf16 = dt == HQ_DTYPE_BF16;

  // ---- synthetic data: X ~ N(0, 1), codes uniform (int4) or P(-1, 0, 1) = (.25, .5, .25),
  // scales |N(0, 0.02)|, all fp16 (X in the activation dtype). ----
  Rng rng{42};
  const size_t lin_words = hq_linear_words(fmt, K, N), packed_words = hq_packed_words(fmt, K, N);
  if (packed_words == 0) {
    std::fprintf(stderr, "unsupported shape K=%u N=%u\n", K, N);
    return 2;
  }
  std::vector<uint32_t> lin(lin_words);
  for (auto& w : lin) {
    if (fmt == HQ_FORMAT_INT4) {
      w = (uint32_t)rng.next();
    } else {
      uint32_t v = 0;
      for (int i = 0; i < 16; ++i) {
        const uint32_t r = (uint32_t)(rng.next() & 3u);
        v |= (r >= 2 ? 1u : (r == 1 ? 2u : 0u)) << (2 * i);
      }
      w = v;
    }
  }
  std::vector<uint16_t> S((size_t)(K / group) * N), X((size_t)Mmax * K);
  for (auto& s : S) s = f32_to_f16((float)std::fabs(rng.normal() * 0.02));
  for (auto& x : X) x = bf16 ? f32_to_bf16((float)rng.normal()) : f32_to_f16((float)rng.normal());

  // ---- repack timing (host, one-time at load; reference: benchmark_repacking MG.cu:646-657) ----
  std::vector<uint32_t> packed(packed_words);
  double repack_ms = 1e30;
  for (int r = 0; r < 3; ++r) {
    const auto t0 = std::chrono::steady_clock::now();
    HQ_OK(fmt == HQ_FORMAT_INT4 ? hq_repack_int4(lin.data(), packed.data(), K, N)
                                : hq_repack_ternary2(lin.data(), packed.data(), K, N));
    const auto t1 = std::chrono::steady_clock::now();
    repack_ms = std::min(repack_ms, std::chrono::duration<double, std::milli>(t1 - t0).count());
  }
  const bool repack_ok = repack_ms < 1000.0;

  // ---- device buffers ----
  const size_t wbytes = packed_words * 4, sbytes = S.size() * 2;
  const int copies = rotate_mib > 0 ? std::max(1, (int)std::ceil(rotate_mib * 1048576.0 / (double)(wbytes + sbytes))) : 1;
  std::vector<uint32_t*> dWp(copies);
  std::vector<uint16_t*> dS(copies);
  for (int c = 0; c < copies; ++c) {
    HIP_OK(hipMalloc(&dWp[c], wbytes));
    HIP_OK(hipMalloc(&dS[c], sbytes));
    HIP_OK(hipMemcpy(dWp[c], packed.data(), wbytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dS[c], S.data(), sbytes, hipMemcpyHostToDevice));
  }
  uint32_t* dLin;
  uint16_t *dX, *dY;
  float* dRef;
  HIP_OK(hipMalloc(&dLin, lin_words * 4));
  HIP_OK(hipMalloc(&dX, X.size() * 2));
  HIP_OK(hipMalloc(&dY, (size_t)Mmax * N * 2));
  HIP_OK(hipMalloc(&dRef, (size_t)Mmax * N * 4));
  HIP_OK(hipMemcpy(dLin, lin.data(), lin_words * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dX, X.data(), X.size() * 2, hipMemcpyHostToDevice));
  size_t ws_bytes = 0;
  HQ_OK(hq_workspace_bytes(fmt, Mmax, K, N, group, &ws_bytes));
  void* dWs = nullptr;
  if (ws_bytes) {
    HIP_OK(hipMalloc(&dWs, ws_bytes));
    HIP_OK(hipMemset(dWs, 0, ws_bytes));
  }
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));

  auto gemm = [&](uint32_t M, int c) {
    if (fmt == HQ_FORMAT_INT4)
      HQ_OK(hq_gemm_w4a16(dX, dt, K, dWp[c], dS[c], nullptr, dY, N, M, K, N, group, dWs, ws_bytes, stream));
    else
      HQ_OK(hq_gemm_w2a16(dX, dt, K, dWp[c], dS[c], dY, N, M, K, N, group, dWs, ws_bytes, stream));
  };
  auto baseline = [&](uint32_t M, int c) {
    (void)c;
    hipLaunchKernelGGL(baseline_gemm<16>, dim3((N + 255) / 256), dim3(256), 0, stream, dX, bf16, dLin, (int)fmt,
                       dS[0], dY, M, K, N, group);
    HIP_OK(hipGetLastError());
  };
  auto time_ms = [&](auto&& launch, uint32_t M) {
    for (int w = 0; w < warmups; ++w) launch(M, w % copies);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipEventRecord(e0, stream));
    for (int it = 0; it < iters; ++it) launch(M, it % copies);
    HIP_OK(hipEventRecord(e1, stream));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    return (double)ms / std::max(1, iters);
  };

  std::vector<SweepResult> results;
  std::vector<uint16_t> Y((size_t)Mmax * N);
  std::vector<float> R((size_t)Mmax * N);
  for (uint32_t M : Ms) {
    SweepResult r{};
    r.M = M;
    hipLaunchKernelGGL(reference_gemm, dim3((N + 255) / 256, M), dim3(256), 0, stream, dX, bf16, dLin, (int)fmt, dS[0],
                       dRef, M, K, N, group);
    HIP_OK(hipGetLastError());
    gemm(M, 0);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipMemcpy(Y.data(), dY, (size_t)M * N * 2, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(R.data(), dRef, (size_t)M * N * 4, hipMemcpyDeviceToHost));
    double maxabs = 0.0, se = 0.0, rmax = 0.0;
    for (size_t i = 0; i < (size_t)M * N; ++i) {
      const double y = bf16 ? bf16_to_f32(Y[i]) : f16_to_f32(Y[i]), ref = R[i];
      const double d = std::fabs(y - ref);
      maxabs = std::max(maxabs, std::isfinite(d) ? d : 1e30);
      se += d * d;
      rmax = std::max(rmax, std::fabs(ref));
    }
    r.max_abs = maxabs;
    r.mse = se / ((double)M * N);
    r.normwise = rmax > 0 ? maxabs / rmax : maxabs;
    r.numerical = r.normwise <= 1e-2;
    r.latency_ms = time_ms(gemm, M);
    r.baseline_ms = time_ms(baseline, M);
    r.speedup = r.baseline_ms / r.latency_ms;
    const double bytes = (double)wbytes + (double)sbytes + 2.0 * M * K + 2.0 * M * N;
    r.gbs = bytes / (r.latency_ms * 1e-3) / 1e9;
    r.util_pct = 100.0 * r.gbs / kHbmPeakGBs;
    r.tflops = 2.0 * M * K * N / (r.latency_ms * 1e-3) / 1e12;
    r.latency_ok = r.latency_ms <= 0.15;
    results.push_back(r);
  }

  bool numerical_ok = true, latency_ok = true, speedup_ok = true;
  double peak_util = 0.0;
  for (const auto& r : results) {
    numerical_ok &= r.numerical;
    latency_ok &= r.latency_ok;
    speedup_ok &= r.speedup >= 1.8;
    peak_util = std::max(peak_util, r.util_pct);
  }
  // The reference's gate (BENCH:80-94): peak bus utilisation >= 80% when K, N >= 4096; the
  // MI355X decode target (>= 70% of 8 TB/s) is reported beside it.
  const bool bw_ok = peak_util >= 80.0, bw70_ok = peak_util >= 70.0;
  const bool check_bw = K >= 4096 && N >= 4096;
  const bool all_ok = repack_ok && numerical_ok && latency_ok && speedup_ok && (!check_bw || bw_ok);

  if (json) {
    std::printf("{\n  \"status\": \"%s\",\n  \"K\": %u,\n  \"N\": %u,\n  \"group_size\": %u,\n", all_ok ? "PASS" : "FAIL", K,
                N, group);
    std::printf("  \"format\": \"%s\",\n  \"dtype\": \"%s\",\n  \"weight_copies\": %d,\n",
                fmt == HQ_FORMAT_INT4 ? "int4" : "ternary2", bf16 ? "bf16" : "f16", copies);
    std::printf("  \"repack_time_ms\": %.2f,\n  \"repack_under_1s\": %s,\n", repack_ms, repack_ok ? "true" : "false");
    std::printf("  \"numerical_match_passed\": %s,\n  \"latency_le_0_15ms_passed\": %s,\n", numerical_ok ? "true" : "false",
                latency_ok ? "true" : "false");
    std::printf("  \"speedup_gt_1_8x_passed\": %s,\n  \"bandwidth_gt_80pct_passed\": %s,\n", speedup_ok ? "true" : "false",
                bw_ok ? "true" : "false");
    std::printf("  \"bandwidth_gt_70pct_passed\": %s,\n  \"peak_bandwidth_util_pct\": %.1f,\n  \"sweep\": [\n",
                bw70_ok ? "true" : "false", peak_util);
    for (size_t i = 0; i < results.size(); ++i) {
      const auto& r = results[i];
      std::printf(
          "    {\n      \"M\": %u,\n      \"marlin_latency_ms\": %.4f,\n      \"baseline_latency_ms\": %.4f,\n"
          "      \"speedup_ratio\": %.2f,\n      \"bandwidth_gbs\": %.1f,\n      \"bandwidth_util_pct\": %.1f,\n"
          "      \"tflops\": %.3f,\n      \"max_abs_error\": %.6e,\n      \"mse\": %.6e,\n      \"normwise_error\": %.6e\n    }%s\n",
          r.M, r.latency_ms, r.baseline_ms, r.speedup, r.gbs, r.util_pct, r.tflops, r.max_abs, r.mse, r.normwise,
          i + 1 < results.size() ? "," : "");
    }
    std::printf("  ]\n}\n");
  } else {
    std::printf("\n===================================================\n");
    std::printf("gfx950 weight-only qGEMM (%s, %s activations)\n", fmt == HQ_FORMAT_INT4 ? "int4" : "ternary 2-bit",
                bf16 ? "bf16" : "fp16");
    std::printf("===================================================\n");
    std::printf("Matrix Geometry:           K=%u, N=%u (%uM params)\n", K, N, (uint32_t)((uint64_t)K * N / 1048576));
    std::printf("Quantization Format:       gfx950 tile layout | Group size=%u\n", group);
    std::printf("Startup Weight Repacking:  %.2f ms (%s)\n", repack_ms, repack_ok ? "PASS < 1.0s" : "FAIL");
    std::printf("Peak Bus Theoretical:      8000.0 GB/s (MI355X HBM3E)\n");
    std::printf("Weight copies rotated:     %d\n", copies);
    std::printf("---------------------------------------------------\nBatch Sweep Results:\n");
    std::printf("   M   | qGEMM (ms) | Baseline (ms) | Speedup | Bandwidth | Bus Util | Max Abs Err | Status\n");
    for (const auto& r : results)
      std::printf("  M=%2u | %8.4f ms | %10.4f ms | %5.2fx  | %7.1f GB/s | %5.1f%%  | %.2e  | %s\n", r.M, r.latency_ms,
                  r.baseline_ms, r.speedup, r.gbs, r.util_pct, r.max_abs,
                  r.numerical && r.latency_ok && r.speedup >= 1.8 ? "PASS" : "FAIL");
    std::printf("---------------------------------------------------\nAcceptance Criteria Verification:\n");
    std::printf("  Weight Repacking (<1.0s):  %s (%.2f ms)\n", repack_ok ? "PASS" : "FAIL", repack_ms);
    std::printf("  GEMM Speedup (>1.8x):      %s\n", speedup_ok ? "PASS (> 1.8x vs naive int4 kernel)" : "FAIL");
    std::printf("  Execution Time (<=0.15ms): %s\n", latency_ok ? "PASS (<= 0.15 ms per GEMM)" : "FAIL");
    std::printf("  Memory Bus Saturation (>80%%): %s (peak %.1f%% of 8 TB/s%s)\n", bw_ok ? "PASS" : "FAIL", peak_util,
                check_bw ? "" : ", not gated below K, N = 4096");
    std::printf("  Numerical Accuracy (normwise <= 1e-2): %s\n", numerical_ok ? "PASS" : "FAIL");
    std::printf("===================================================\n");
    std::printf("Overall Status:            %s\n\n", all_ok ? "PASS (All Invariants Verified)" : "FAIL");
  }

  for (int c = 0; c < copies; ++c) {
    HIP_OK(hipFree(dWp[c]));
    HIP_OK(hipFree(dS[c]));
  }
  HIP_OK(hipFree(dLin));
  HIP_OK(hipFree(dX));
  HIP_OK(hipFree(dY));
  HIP_OK(hipFree(dRef));
  if (dWs) HIP_OK(hipFree(dWs));
  HIP_OK(hipStreamDestroy(stream));
  return all_ok ? 0 : 1;
}

// hq_stream_ceiling — the practical HBM read ceiling of this device for one launch of a
// given size: the shortest time in which a plain streaming kernel reads N bytes once.
//
// The decode GEMMs read their packed weights once per call; this tool measures, on the same
// device and in the same run, what a kernel that does nothing but read those bytes achieves
// (grid-stride 16-byte loads, XOR-folded, one guarded store per thread), so that a decode
// launch can be compared with the stream rate its size allows and not only with the 8 TB/s
// peak. Launches are timed inside a HIP graph (40 per graph, the graph replayed 3 times) and
// rotate over enough buffers (>= 1 GiB in total) that no launch reads data a recent launch
// left in the last-level cache. Several launch shapes are tried per size; the fastest counts.
//
// usage: hq_stream_ceiling BYTES [BYTES ...]
// output: one JSON object on stdout.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                            \
  do {                                                                                      \
    hipError_t e_ = (x);                                                                    \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "hq_stream_ceiling: %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                         \
    }                                                                                       \
  } while (0)

// Reads n16 16-byte words once. Thread i reads words i, i + S, i + 2S, ... (S = threads in
// the grid), UNR of them per loop trip; every index is below n16.
template <int UNR>
__global__ void __launch_bounds__(256) hq_stream_read(const u4* __restrict__ p, size_t n16, uint32_t* out) {
  u4 acc = {0u, 0u, 0u, 0u};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (UNR - 1) * stride < n16; i += UNR * stride) {
    u4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < UNR; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9E3779B9u) out[blockIdx.x] = x;  // keeps the loads; the buffers never hold this
}

struct Best {
  double us = 0.0;
  int wg_per_cu = 0;
  int unroll = 0;
};

double time_config(const std::vector<u4*>& bufs, size_t n16, int grid, int unroll, uint32_t* out, hipStream_t s) {
  const int nb = (int)bufs.size();
  constexpr int kPerGraph = 40, kReplays = 3;
  auto launch = [&](int r) {
    if (unroll == 2) hipLaunchKernelGGL(hq_stream_read<2>, dim3(grid), dim3(256), 0, s, bufs[r % nb], n16, out);
    else if (unroll == 4) hipLaunchKernelGGL(hq_stream_read<4>, dim3(grid), dim3(256), 0, s, bufs[r % nb], n16, out);
    else hipLaunchKernelGGL(hq_stream_read<8>, dim3(grid), dim3(256), 0, s, bufs[r % nb], n16, out);
  };
  for (int r = 0; r < 8; ++r) launch(r);
  CHECK(hipGetLastError());
  CHECK(hipStreamSynchronize(s));
  hipGraph_t g;
  hipGraphExec_t ge;
  CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  for (int r = 0; r < kPerGraph; ++r) launch(r);
  CHECK(hipStreamEndCapture(s, &g));
  CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  CHECK(hipGraphLaunch(ge, s));  // warm-up replay
  CHECK(hipStreamSynchronize(s));
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  CHECK(hipEventRecord(a, s));
  for (int k = 0; k < kReplays; ++k) CHECK(hipGraphLaunch(ge, s));
  CHECK(hipEventRecord(b, s));
  CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  CHECK(hipGraphExecDestroy(ge));
  CHECK(hipGraphDestroy(g));
  return (double)ms * 1e3 / (kPerGraph * kReplays);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s BYTES [BYTES ...]\n", argv[0]);
    return 2;
  }
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  uint32_t* out = nullptr;
  CHECK(hipMalloc(&out, (size_t)cus * 8u * sizeof(uint32_t)));
  hipStream_t s;
  CHECK(hipStreamCreate(&s));
  std::printf("{\"arch\": \"%s\", \"cus\": %d, \"sizes\": [", prop.gcnArchName, cus);
  for (int a = 1; a < argc; ++a) {
    const long long req = std::atoll(argv[a]);
    if (req < 16 || req > (16ll << 30)) {
      std::fprintf(stderr, "hq_stream_ceiling: size %s out of range (16 B .. 16 GiB)\n", argv[a]);
      return 2;
    }
    const size_t bytes = (size_t)req / 16u * 16u;
    const size_t n16 = bytes / 16u;
    size_t nb = (size_t(1) << 30) / bytes + 1u;
    if (nb < 2u) nb = 2u;
    std::vector<u4*> bufs(nb);
    for (auto& p : bufs) {
      CHECK(hipMalloc(&p, bytes));
      CHECK(hipMemsetAsync(p, 1, bytes, s));
    }
    CHECK(hipStreamSynchronize(s));
    Best best;
    for (int wpc : {1, 2, 4, 8}) {
      for (int unroll : {2, 4, 8}) {
        const double us = time_config(bufs, n16, cus * wpc, unroll, out, s);
        if (best.us == 0.0 || us < best.us) best = Best{us, wpc, unroll};
      }
    }
    for (auto& p : bufs) CHECK(hipFree(p));
    std::printf("%s{\"bytes\": %zu, \"us\": %.3f, \"GBps\": %.1f, \"workgroups_per_cu\": %d, \"unroll\": %d}",
                a > 1 ? ", " : "", bytes, best.us, (double)bytes / best.us / 1e3, best.wg_per_cu, best.unroll);
    std::fflush(stdout);
  }
  std::printf("]}\n");
  CHECK(hipFree(out));
  CHECK(hipStreamDestroy(s));
  return 0;
}

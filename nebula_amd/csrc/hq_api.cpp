// hq_api.cpp — the C ABI (include/hq_qgemm.h): argument validation, host repacks,
// kernel dispatch and per-thread error strings. No exception crosses the ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "hq_internal.hpp"
#include "hq_layout.hpp"
#include "hq_plan.hpp"
#include "hq_qgemm.h"

namespace {

thread_local std::string g_last_error;

hq_status fail(hq_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return s;
}

hq_status ok() {
  g_last_error.clear();
  return HQ_OK;
}

}  // namespace

hq_status hq_set_error(hq_status s, const char* fmt, ...) {
  if (s == HQ_OK) {
    g_last_error.clear();
    return s;
  }
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return s;
}

namespace {

hq_status from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(HQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

bool valid_fmt(int f) { return f == HQ_FORMAT_INT4 || f == HQ_FORMAT_TERNARY2; }
bool valid_dtype(int d) { return d == HQ_DTYPE_F16 || d == HQ_DTYPE_BF16; }

hq_status check_repack_shape(hq_format fmt, uint32_t K, uint32_t N) {
  if (!valid_fmt(fmt)) return fail(HQ_ERR_INVALID_ARG, "unknown format %d", (int)fmt);
  if (K == 0 || N == 0) return fail(HQ_ERR_SHAPE, "K=%u N=%u must be positive", K, N);
  if (K % hq::kBlockK) return fail(HQ_ERR_SHAPE, "K=%u must be a multiple of 128", K);
  return HQ_OK;
}

// Parallel-for over [0, n) on host threads (the repacks are memory-bound word gathers).
template <class F>
void parallel_for(size_t n, F f) {
  unsigned nt = std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > 16) nt = 16;
  if (n < (1u << 16) || nt == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  const size_t chunk = (n + nt - 1) / nt;
  for (unsigned i = 0; i < nt; ++i) {
    const size_t b = i * chunk, e = std::min(n, b + chunk);
    if (b < e) th.emplace_back([=] { f(b, e); });
  }
  for (auto& t : th) t.join();
}

// Library-owned workspace, one per (device, stream), used when the caller passes
// none. It is zero-filled when allocated (the kernels leave its counters at zero), grows
// when a larger shape needs it, and is never allocated while the stream is capturing.
// Buffers that were outgrown stay allocated until the process ends: a launch still in
// flight may use them.
struct InternalWorkspace {
  std::mutex mu;
  std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> live;
  std::vector<void*> retired;
};
InternalWorkspace& internal_ws() {
  static InternalWorkspace* w = new InternalWorkspace();  // never destroyed: see above
  return *w;
}

hq_status get_internal_ws(hipStream_t stream, size_t need, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HQ_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  InternalWorkspace& w = internal_ws();
  std::lock_guard<std::mutex> lock(w.mu);
  auto& slot = w.live[{dev, stream}];
  if (slot.second >= need) {
    *out = slot.first;
    return HQ_OK;
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) return fail(HQ_ERR_DEVICE, "hipStreamIsCapturing: %s", hipGetErrorString(e));
  if (cap != hipStreamCaptureStatusNone)
    return fail(HQ_ERR_WORKSPACE,
                "this shape needs %zu workspace bytes; pass a workspace (hq_workspace_bytes) or run "
                "the shape once before capturing the stream",
                need);
  const size_t bytes = std::max(need, (size_t)1 << 20);
  void* p = nullptr;
  if ((e = hipMalloc(&p, bytes)) != hipSuccess) return fail(HQ_ERR_DEVICE, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  if ((e = hipMemsetAsync(p, 0, bytes, stream)) != hipSuccess) {
    (void)hipFree(p);
    return fail(HQ_ERR_DEVICE, "hipMemsetAsync: %s", hipGetErrorString(e));
  }
  if (slot.first) w.retired.push_back(slot.first);
  slot = {p, bytes};
  *out = p;
  return HQ_OK;
}

// Streaming kernel family for the calls the X-resident kernel does not take (rows of all of
// K that do not fit in LDS even in pieces, pieces beyond a workspace cap, more than 16 rows,
// the general kernels). With at most four activation rows the activation traffic is
// small and the per-wavefront kernel (hq_decode.hip) is as fast or faster (M = 4, same-run
// order-swapped timings on MI355X: 5120 x 5120 7.7 against 8.1 us, 5120 x 27648 15.9 against
// 16.15 us, 27648 x 5120 even); from five rows on, the lockstep kernel (hq_decode_ls.hip),
// which fetches each activation k-block once per workgroup, is, and above 16 rows only the
// lockstep kernel takes them. With ternary weights the lockstep kernel's
// four-k-group configuration is faster from one row on (5120 x 27648 at M = 1: 12.8 us
// against 14.7 us), so it is taken whenever the lockstep planner picks it. The general
// kernels (bias, groups that are not multiples of 128) exist in the lockstep family only.
// HQ_DECODE_KERNEL=0 / 1 forces one of them for M <= 16 (tuning and tests).
bool use_lockstep(int fmt, const hq::GemmDesc& d) {
  if (d.M > 16 || d.gen) return true;  // only the lockstep kernel takes several row tiles
  const char* v = std::getenv("HQ_DECODE_KERNEL");
  if (v && *v) return std::atoi(v) != 0;
  if (d.M >= 5) return true;
  return fmt == HQ_FORMAT_TERNARY2 && hq::choose_decode_ls(fmt, d).KG == 4;
}

// The X-resident kernel (hq_decode.hip) takes every call with at most 16 rows whose
// activation rows fit in LDS, outside the general kernels. HQ_DECODE_KERNEL=2 forces it
// where it fits, 0 or 1 keeps it off (tuning and tests).
bool use_resident(int fmt, const hq::GemmDesc& d, size_t cap, hq::XrConfig* c) {
  if (d.M > 16 || d.gen) return false;
  const char* v = std::getenv("HQ_DECODE_KERNEL");
  if (v && *v && std::atoi(v) != 2) return false;
  *c = hq::choose_decode_xr(fmt, d, cap);
  return c->ok;
}

// Slabs of the X-resident grid over the segments of d (up to T tiles each; at least G in
// all when G > 0, as hq::assign_slabs cuts them).
uint32_t xr_slabs(const hq::GemmDesc& d, int T, uint32_t G) {
  uint32_t tiles = 0, g = 0;
  for (uint32_t i = 0; i < d.nseg; ++i) tiles += d.seg[i].ntiles;
  for (uint32_t i = 0; i < d.nseg; ++i) {
    const uint32_t nt = d.seg[i].ntiles;
    uint32_t ns = (nt + T - 1) / T;
    if (G) ns = std::max<uint32_t>(ns, (uint32_t)(((uint64_t)G * nt + tiles - 1) / tiles));
    g += std::min(ns, nt);
  }
  return g;
}

// Rows up to which the streaming (decode) kernels run; the MFMA tile kernel above. The
// lockstep kernel takes up to 16 * kLsMaxRowTiles rows: a split-fuse step (16 decode
// tokens and a 64-token prefill chunk) stays a weight stream. HQ_DECODE_MAX_M overrides
// (16 .. 80; tuning and tests).
uint32_t decode_max_m() {
  const char* v = std::getenv("HQ_DECODE_MAX_M");
  const int e = v && *v ? std::atoi(v) : 0;
  const uint32_t top = 16u * hq::kLsMaxRowTiles;
  return e >= 16 && (uint32_t)e <= top ? (uint32_t)e : top;
}

// The general kernels on request for groups and calls the fast kernels also take (tests
// compare the two): HQ_GENERAL=1.
bool force_general() {
  const char* v = std::getenv("HQ_GENERAL");
  return v && *v && std::atoi(v) != 0;
}

// Shape validation shared by the GEMM entry points and the workspace queries.
hq_status check_shape(int fmt, uint32_t M, uint32_t K, uint32_t group, bool bias) {
  if (!valid_fmt(fmt)) return fail(HQ_ERR_INVALID_ARG, "unknown format %d", fmt);
  if (M == 0) return fail(HQ_ERR_SHAPE, "M must be >= 1");
  if (K == 0 || K % hq::kBlockK) return fail(HQ_ERR_SHAPE, "K=%u must be a positive multiple of 128", K);
  if (group == 0 || group % 32)
    return fail(HQ_ERR_SHAPE, "group=%u must be a positive multiple of 32", group);
  if (K % group) return fail(HQ_ERR_SHAPE, "K=%u must be a multiple of group=%u", K, group);
  if (bias && fmt != HQ_FORMAT_INT4) return fail(HQ_ERR_UNSUPPORTED, "a bias is supported for int4 weights only");
  return HQ_OK;
}

// Validation of the activation operand.
hq_status check_x(const void* X, int dtype, int64_t ldx, uint32_t K) {
  if (!X) return fail(HQ_ERR_INVALID_ARG, "X is null");
  if (!valid_dtype(dtype)) return fail(HQ_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  if (ldx < (int64_t)K) return fail(HQ_ERR_SHAPE, "ldx=%lld < K=%u", (long long)ldx, K);
  if (ldx % 8) return fail(HQ_ERR_ALIGNMENT, "ldx=%lld must be a multiple of 8 elements", (long long)ldx);
  if (reinterpret_cast<uintptr_t>(X) % 16) return fail(HQ_ERR_ALIGNMENT, "X must be 16-byte aligned");
  return HQ_OK;
}

// Every operand a kernel reads or writes is addressed through a buffer descriptor with 32-bit
// byte offsets: an operand of 2 GiB or more would wrap, and loads past the wrapped range read
// zero (silently wrong results), so such calls are rejected. ldx = 0 / ldy = 0: not known yet
// (the workspace and plan queries check the shape-derived operands only).
hq_status check_ranges(int fmt, uint32_t M, uint32_t K, uint32_t group, uint32_t N, uint32_t seg, int64_t ldx,
                       int64_t ldy, bool bias) {
  constexpr uint64_t kRange = 1ull << 31;
  const uint64_t rows = K / group, tiles = hq::col_tiles(N);
  const uint64_t x = (uint64_t)M * (uint64_t)(ldx ? ldx : K) * 2u;
  const uint64_t y = (uint64_t)M * (uint64_t)(ldy ? ldy : N) * 2u;
  const uint64_t sc = ((rows - 1u) * N + N) * 2u;
  const uint64_t w = tiles * (K / hq::kBlockK) * (fmt == HQ_FORMAT_INT4 ? 1024u : 512u);
  if (x >= kRange)
    return fail(HQ_ERR_SHAPE, "X spans %llu bytes (M * ldx * 2): operands must stay below 2 GiB", (unsigned long long)x);
  if (y >= kRange)
    return fail(HQ_ERR_SHAPE, "segment %u: Y spans %llu bytes (M * ldy * 2): operands must stay below 2 GiB", seg,
                (unsigned long long)y);
  if (sc >= kRange || (bias && sc * 2u >= kRange))
    return fail(HQ_ERR_SHAPE, "segment %u: the scales%s of K=%u, N=%u, group=%u span 2 GiB or more", seg,
                bias ? " or bias" : "", K, N, group);
  if (w >= kRange)
    return fail(HQ_ERR_SHAPE, "segment %u: the packed weights of K=%u, N=%u span %llu bytes (2 GiB or more)", seg, K,
                N, (unsigned long long)w);
  return HQ_OK;
}

hq_status check_segment(const hq_segment& s, uint32_t i) {
  if (!s.Wp || !s.scales || !s.Y) return fail(HQ_ERR_INVALID_ARG, "segment %u: null pointer", i);
  if (s.N == 0) return fail(HQ_ERR_SHAPE, "segment %u: N must be >= 1", i);
  if (s.ldy < (int64_t)s.N) return fail(HQ_ERR_SHAPE, "segment %u: ldy=%lld < N=%u", i, (long long)s.ldy, s.N);
  if (reinterpret_cast<uintptr_t>(s.Wp) % 16) return fail(HQ_ERR_ALIGNMENT, "segment %u: Wp must be 16-byte aligned", i);
  if (reinterpret_cast<uintptr_t>(s.scales) % 2) return fail(HQ_ERR_ALIGNMENT, "segment %u: scales must be 2-byte aligned", i);
  if (reinterpret_cast<uintptr_t>(s.bias) % 4) return fail(HQ_ERR_ALIGNMENT, "segment %u: bias must be 4-byte aligned", i);
  if (reinterpret_cast<uintptr_t>(s.Y) % 2) return fail(HQ_ERR_ALIGNMENT, "segment %u: Y must be 2-byte aligned", i);
  return HQ_OK;
}

// Descriptor of a call from its shape (pointers filled by the caller when it has them).
hq::GemmDesc make_desc(uint32_t M, uint32_t K, uint32_t group, const uint32_t* Ns, uint32_t nseg, bool bias) {
  hq::GemmDesc d{};
  d.M = M;
  d.K = K;
  d.nkb = K / hq::kBlockK;
  d.gkb = group % hq::kBlockK == 0 ? group / hq::kBlockK : 1u;
  d.nseg = nseg;
  d.gen = (bias || group % hq::kBlockK != 0 || force_general()) ? 1u : 0u;
  d.g32 = group / 32u;
  d.g32_m = hq::plan_div_magic(d.g32);
  d.has_bias = bias ? 1u : 0u;
  for (uint32_t i = 0; i < nseg; ++i) {
    d.seg[i].N = Ns[i];
    d.seg[i].lds = Ns[i];
    d.seg[i].ntiles = hq::col_tiles(Ns[i]);
  }
  return d;
}

// What a call runs: the kernel family, its tiling and the workspace it needs.
enum class Kind { kDecode, kLockstep, kPrefill, kResident };
struct Plan {
  Kind kind;
  hq::XrConfig xc{};
  hq::DecodeConfig c{};
  hq::LsConfig lc{};
  hq::PrefillConfig pc{};
  size_t need = 0;
};

// cap: the largest workspace the plan may use (the no-allocation entry point's scratch).
// dtype: the activation type (the prefill tile width depends on it, the workspace does not,
// so the workspace queries plan without it).
Plan make_plan(int fmt, const hq::GemmDesc& d, size_t cap = SIZE_MAX, int dtype = HQ_DTYPE_F16) {
  Plan p{};
  if (d.M > decode_max_m()) {
    p.kind = Kind::kPrefill;
    p.pc = hq::choose_prefill(fmt, d, cap, dtype);
    p.need = hq::prefill_workspace_bytes(d, p.pc);
    return p;
  }
  if (use_resident(fmt, d, cap, &p.xc)) {
    p.kind = Kind::kResident;
    p.need = hq::decode_xr_workspace_bytes(d, p.xc);
    return p;
  }
  if (!use_lockstep(fmt, d)) {
    p.kind = Kind::kDecode;
    p.c = hq::choose_decode(fmt, d);
    p.need = hq::decode_workspace_bytes(d, p.c);
    if (p.need <= cap) return p;
  }
  // The lockstep kernel takes every decode shape; under a cap with fewer pieces per slab.
  p.kind = Kind::kLockstep;
  p.lc = hq::choose_decode_ls(fmt, d, cap);
  p.need = hq::decode_ls_workspace_bytes(d, p.lc);
  return p;
}

// Host-visible fault word of kernels whose bounded waits gave up (pinned, mapped host
// memory, one word for every device; allocated on the first call outside stream capture).
struct FaultWord {
  std::mutex mu;
  uint32_t* host = nullptr;  // also the device address (unified addressing)
};
FaultWord& fault_word() {
  static FaultWord* f = new FaultWord();  // never destroyed: kernels may still write it
  return *f;
}
uint32_t* fault_ptr(hipStream_t s) {
  FaultWord& f = fault_word();
  std::lock_guard<std::mutex> lock(f.mu);
  if (f.host) return f.host;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  void* p = nullptr;
  if (hipHostMalloc(&p, 256, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::memset(p, 0, 256);
  void* dp = nullptr;
  if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess || dp != p) {
    (void)hipGetLastError();
    (void)hipHostFree(p);
    return nullptr;
  }
  f.host = static_cast<uint32_t*>(p);
  return f.host;
}
// The fault word if it exists already (never allocates).
uint32_t* fault_ptr_if_any() { return __atomic_load_n(&fault_word().host, __ATOMIC_ACQUIRE); }
// Reads and clears the fault word: true if a kernel reported a fault since the last check.
bool take_fault() {
  FaultWord& f = fault_word();
  uint32_t* w = __atomic_load_n(&f.host, __ATOMIC_ACQUIRE);
  if (!w) return false;
  return __atomic_exchange_n(w, 0u, __ATOMIC_ACQ_REL) != 0u;
}
hq_status fault_status() {
  return fail(HQ_ERR_DEVICE,
              "a launch gave up waiting at a k-group barrier (the lockstep decode kernel's k-groups, or the "
              "two K halves of a prefill tile): the outputs of that launch are wrong (fault word reported by "
              "the device)");
}
uint32_t ls_spin() {
  // Polls of the kernels' bounded barriers (lockstep k-groups, prefill K halves); tests: a
  // small limit forces the fault path.
  const char* v = std::getenv("HQ_DECODE_LS_SPIN");
  return v && *v ? (uint32_t)std::strtoul(v, nullptr, 10) : hq::kLsSpinLimit;
}

// Validates a call and builds its descriptor (pointers included).
hq_status prepare(const void* X, hq_dtype dtype, int64_t ldx, hq_format fmt, const hq_segment* segs, uint32_t nseg,
                  uint32_t M, uint32_t K, uint32_t group, hq::GemmDesc* out) {
  if (take_fault()) return fault_status();
  if (!segs || nseg == 0 || nseg > HQ_MAX_SEGMENTS)
    return fail(HQ_ERR_INVALID_ARG, "need 1..%d segments, got %u", HQ_MAX_SEGMENTS, nseg);
  bool bias = false;
  uint32_t Ns[HQ_MAX_SEGMENTS];
  hq_status st;
  for (uint32_t i = 0; i < nseg; ++i) {
    if ((st = check_segment(segs[i], i)) != HQ_OK) return st;
    bias |= segs[i].bias != nullptr;
    Ns[i] = segs[i].N;
  }
  if ((st = check_shape(fmt, M, K, group, bias)) != HQ_OK) return st;
  if ((st = check_x(X, dtype, ldx, K)) != HQ_OK) return st;
  for (uint32_t i = 0; i < nseg; ++i)
    if ((st = check_ranges(fmt, M, K, group, Ns[i], i, ldx, segs[i].ldy, segs[i].bias != nullptr)) != HQ_OK) return st;
  hq::GemmDesc d = make_desc(M, K, group, Ns, nseg, bias);
  if (d.gen && !hq::kGeneralKernels)
    return fail(HQ_ERR_UNSUPPORTED, "group=%u%s needs the general kernels, which this build lacks", group,
                bias ? " with a bias" : "");
  d.X = X;
  d.ldx = ldx;
  for (uint32_t i = 0; i < nseg; ++i) {
    d.seg[i].Wp = segs[i].Wp;
    d.seg[i].S = segs[i].scales;
    d.seg[i].B = segs[i].bias;
    d.seg[i].Y = segs[i].Y;
    d.seg[i].ldy = segs[i].ldy;
  }
  *out = d;
  return HQ_OK;
}

hq_status launch_plan(int fmt, int dtype, const hq::GemmDesc& d, const Plan& p, void* w, uint32_t* fault,
                      hipStream_t s) {
  switch (p.kind) {
    case Kind::kPrefill: return from_hip(hq::launch_prefill(fmt, dtype, p.pc, w, fault, ls_spin(), s), "prefill launch");
    case Kind::kLockstep:
      return from_hip(hq::launch_decode_ls(fmt, dtype, d, p.lc, w, fault, ls_spin(), s), "decode launch");
    case Kind::kResident: return from_hip(hq::launch_decode_xr(fmt, dtype, d, p.xc, w, s), "decode launch");
    case Kind::kDecode: break;
  }
  return from_hip(hq::launch_decode(fmt, dtype, d, p.c, w, s), "decode launch");
}

hq_status run_gemm(const void* X, hq_dtype dtype, int64_t ldx, hq_format fmt, const hq_segment* segs,
                   uint32_t nseg, uint32_t M, uint32_t K, uint32_t group, void* ws, size_t ws_bytes,
                   hq_stream stream) {
  hq::GemmDesc d;
  hq_status st = prepare(X, dtype, ldx, fmt, segs, nseg, M, K, group, &d);
  if (st != HQ_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const Plan p = make_plan(fmt, d, SIZE_MAX, dtype);
  void* w = nullptr;
  if (p.need > 0) {
    if (ws) {
      if (ws_bytes < p.need)
        return fail(HQ_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu this call needs", ws_bytes, p.need);
      if (reinterpret_cast<uintptr_t>(ws) % 256)
        return fail(HQ_ERR_ALIGNMENT, "workspace must be 256-byte aligned");
      w = ws;
    } else if ((st = get_internal_ws(s, p.need, &w)) != HQ_OK) {
      return st;
    }
  }
  return launch_plan(fmt, dtype, d, p, w, fault_ptr(s), s);
}

// ---- the no-allocation entry point's scratch ----
// A file-scope device array is the workspace of hq_gemm_fused_noalloc: each GPU the library
// runs on holds its own copy, at its own address, until the process ends. Host code never
// passes the array's name to a kernel (on the host it only names the symbol): the per-device
// address comes from hipGetSymbolAddress, taken once per device at that device's first call.
constexpr size_t kScratchBytes = HQ_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void hq_zero_words(uint32_t* p, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

// The scratch array's address on the current device. The first call on a device resolves it
// and clears the arrival counters at its start with a fill kernel on `s` (kernels leave them
// at zero after every call; a fill kernel, not a memset, so that a captured first call still
// replays correctly).
hq_status scratch_ptr(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return from_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(HQ_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  ScratchSlot& sl = g_scratch[dev];
  std::call_once(sl.once, [&] {
    sl.err = hipGetSymbolAddress(&sl.ptr, HIP_SYMBOL(scratch));
    if (sl.err != hipSuccess) return;
    const uint32_t n = (uint32_t)(hq::kCounterBytes / 4u);
    hipLaunchKernelGGL(hq_zero_words, dim3((n + 255u) / 256u), dim3(256), 0, s, static_cast<uint32_t*>(sl.ptr), n);
    sl.err = hipGetLastError();
  });
  if (sl.err != hipSuccess) return from_hip(sl.err, "scratch set-up (hipGetSymbolAddress)");
  *out = sl.ptr;
  return HQ_OK;
}

const char* fmt_name(int fmt) { return fmt == HQ_FORMAT_INT4 ? "int4" : "ternary2"; }
const char* dt_name(int dt) { return dt == HQ_DTYPE_F16 ? "f16" : "bf16"; }

// Ring depth the per-wavefront launcher instantiates for slab width T (and an override U).
int decode_ring(int T, int U) {
  if (T == 8) return U == 3 ? 3 : 2;
  if (T == 4 || T == 2) return (U == 2 || U == 4) ? U : 3;
  return 4;
}

std::string describe(int fmt, int dtype, const hq::GemmDesc& d, const Plan& p) {
  char b[512];
  if (p.kind == Kind::kResident && p.xc.SG > 1) {
    const uint32_t slabs = xr_slabs(d, p.xc.T, p.xc.G);
    std::snprintf(b, sizeof b,
                  "hq_decode_xr_kernel<%s,%s,T=%d,U=%d,SG=%d> workgroups=%u of %d slabs (%u slabs) x %d pieces x %d "
                  "wavefronts per slab lds=%u ws=%zu",
                  fmt_name(fmt), dt_name(dtype), p.xc.T, p.xc.U, p.xc.SG, (slabs + p.xc.SG - 1) / p.xc.SG, p.xc.SG,
                  slabs, p.xc.S, p.xc.WK, p.xc.lds, p.need);
  } else if (p.kind == Kind::kResident) {
    std::snprintf(b, sizeof b,
                  "hq_decode_xr_kernel<%s,%s,T=%d,U=%d> workgroups=%u slabs x %d pieces x %d wavefronts lds=%u ws=%zu",
                  fmt_name(fmt), dt_name(dtype), p.xc.T, p.xc.U, xr_slabs(d, p.xc.T, p.xc.G), p.xc.S, p.xc.WK, p.xc.lds,
                  p.need);
  } else if (p.kind == Kind::kDecode) {
    std::snprintf(b, sizeof b, "hq_decode_kernel<%s,%s,T=%d,U=%d> workgroups=%d x %d wavefronts%s%s ws=%zu",
                  fmt_name(fmt), dt_name(dtype), p.c.T, decode_ring(p.c.T, p.c.U), p.c.SK, p.c.WK,
                  p.c.G ? " variable-width slabs" : "", p.need ? " cut slabs (fix-up)" : "", p.need);
  } else if (p.kind == Kind::kLockstep) {
    std::snprintf(b, sizeof b,
                  "hq_decode_ls_kernel<%s,%s,KG=%d,GW=%d,T=%d,U=%d,MT=%d%s> grid=%d pieces x slabs of %d tiles, "
                  "%d wavefronts%s ws=%zu",
                  fmt_name(fmt), dt_name(dtype), p.lc.KG, p.lc.GW, p.lc.T, p.lc.U, p.lc.MT, d.gen ? ",general" : "",
                  p.lc.S, p.lc.SW, p.lc.KG * p.lc.GW, p.lc.P > 0 ? " balanced grid" : "", p.need);
  } else {
    int n = std::snprintf(b, sizeof b, "hq_prefill_kernel<%s,%s%s>", fmt_name(fmt), dt_name(dtype),
                          d.gen ? ",general" : "");
    for (int i = 0; i < p.pc.n && n > 0 && (size_t)n < sizeof b; ++i) {
      const hq::PrefillLaunch& l = p.pc.l[i];
      n += std::snprintf(b + n, sizeof b - n, "%s launch %d: %u-row%s tiles=%u whole=%u stream-K workgroups=%u%s",
                         i ? ";" : "", i, 16u * l.RT * l.WM, l.TW == 2 ? " 128-column" : "", l.tiles, l.dp, l.psk,
                         l.KS == 2 ? " k-split in workgroup" : "");
    }
    if (n > 0 && (size_t)n < sizeof b) std::snprintf(b + n, sizeof b - n, " ws=%zu", p.need);
  }
  return b;
}

}  // namespace

namespace {
// Byte of the tile layout holding w[k][n] (column tile n / 16, k-block k / 128; lane
// 16 ((k % 64) / 16) + n % 16 holds 16 consecutive k of chunk (k % 128) / 64 at byte 16 c).
inline size_t int8_tile_byte(uint32_t k, uint32_t n, uint32_t nkb) {
  const uint32_t ct = n / 16u, kb = k / 128u, c = (k % 128u) / 64u, s = (k % 64u) / 16u, i = k % 16u;
  const uint32_t lane = 16u * s + n % 16u;
  return ((size_t)ct * nkb + kb) * 2048u + lane * 32u + c * 16u + i;
}

hq_status check_int8_shape(uint32_t K, uint32_t N) {
  if (K == 0 || K % hq::kBlockK) return fail(HQ_ERR_SHAPE, "K=%u must be a positive multiple of 128", K);
  if (K > 131072u) return fail(HQ_ERR_SHAPE, "K=%u exceeds 131072 (the int32 sum could overflow)", K);
  if (N == 0) return fail(HQ_ERR_SHAPE, "N must be >= 1");
  return HQ_OK;
}
}  // namespace

extern "C" {

const char* hq_version(void) { return "nebula-hq 0.2.0 (gfx950, ABI 2)"; }

const char* hq_last_error(void) { return g_last_error.c_str(); }

const char* hq_status_string(hq_status s) {
  switch (s) {
    case HQ_OK: return "ok";
    case HQ_ERR_INVALID_ARG: return "invalid argument";
    case HQ_ERR_SHAPE: return "unsupported shape";
    case HQ_ERR_ALIGNMENT: return "misaligned pointer or leading dimension";
    case HQ_ERR_UNSUPPORTED: return "unsupported";
    case HQ_ERR_WORKSPACE: return "workspace too small";
    case HQ_ERR_BAD_CODE: return "invalid ternary code";
    case HQ_ERR_DEVICE: return "device error";
    case HQ_ERR_INTERNAL: return "internal error";
    case HQ_ERR_FORMAT: return "malformed or unsupported GGUF data";
    case HQ_ERR_NOT_FOUND: return "not found";
    case HQ_ERR_IO: return "file error";
  }
  return "unknown status";
}

size_t hq_linear_words(hq_format fmt, uint32_t K, uint32_t N) {
  if (fmt == HQ_FORMAT_INT4) return (size_t)(K / 8) * N;
  if (fmt == HQ_FORMAT_TERNARY2) return (size_t)(K / 16) * N;
  return 0;
}

size_t hq_packed_words(hq_format fmt, uint32_t K, uint32_t N) {
  if (!valid_fmt(fmt) || K == 0 || N == 0 || K % hq::kBlockK) return 0;
  return (size_t)hq::col_tiles(N) * (K / hq::kBlockK) * 64u * hq::words_per_lane(fmt);
}

hq_status hq_workspace_bytes(hq_format fmt, uint32_t M, uint32_t K, uint32_t N, uint32_t group, size_t* bytes) {
  if (!bytes) return fail(HQ_ERR_INVALID_ARG, "bytes is null");
  hq_status st = check_shape(fmt, M, K, group, false);
  if (st != HQ_OK) return st;
  if (N == 0) return fail(HQ_ERR_SHAPE, "N must be >= 1");
  if ((st = check_ranges(fmt, M, K, group, N, 0, 0, 0, false)) != HQ_OK) return st;
  *bytes = 0;
  // The larger of the plans without and (int4) with a bias: exactly what a one-projection call
  // of this shape needs, at any M.
  for (int b = 0; b < (fmt == HQ_FORMAT_INT4 ? 2 : 1); ++b) {
    const hq::GemmDesc d = make_desc(M, K, group, &N, 1, b != 0);
    *bytes = std::max(*bytes, make_plan(fmt, d).need);
  }
  return ok();
}

hq_status hq_workspace_bytes_fused(hq_format fmt, uint32_t M, uint32_t K, uint32_t group, const uint32_t* Ns,
                                   uint32_t nseg, int with_bias, size_t* bytes) {
  if (!bytes || !Ns) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  if (nseg == 0 || nseg > HQ_MAX_SEGMENTS) return fail(HQ_ERR_INVALID_ARG, "need 1..%d segments, got %u", HQ_MAX_SEGMENTS, nseg);
  hq_status st = check_shape(fmt, M, K, group, with_bias != 0);
  if (st != HQ_OK) return st;
  for (uint32_t i = 0; i < nseg; ++i) {
    if (Ns[i] == 0) return fail(HQ_ERR_SHAPE, "segment %u: N must be >= 1", i);
    if ((st = check_ranges(fmt, M, K, group, Ns[i], i, 0, 0, with_bias != 0)) != HQ_OK) return st;
  }
  *bytes = make_plan(fmt, make_desc(M, K, group, Ns, nseg, with_bias != 0)).need;
  return ok();
}

hq_status hq_describe_gemm(hq_format fmt, hq_dtype dtype, uint32_t M, uint32_t K, uint32_t N, uint32_t group,
                           int with_bias, char* buf, size_t buf_len) {
  if (!buf || buf_len == 0) return fail(HQ_ERR_INVALID_ARG, "buf is null or empty");
  if (!valid_dtype(dtype)) return fail(HQ_ERR_INVALID_ARG, "unknown dtype %d", (int)dtype);
  hq_status st = check_shape(fmt, M, K, group, with_bias != 0);
  if (st != HQ_OK) return st;
  if (N == 0) return fail(HQ_ERR_SHAPE, "N must be >= 1");
  const hq::GemmDesc d = make_desc(M, K, group, &N, 1, with_bias != 0);
  const std::string s = describe(fmt, dtype, d, make_plan(fmt, d, SIZE_MAX, dtype));
  std::snprintf(buf, buf_len, "%s", s.c_str());
  return ok();
}

hq_status hq_device_status(hq_stream stream) {
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return from_hip(e, "hipStreamSynchronize");
  if (take_fault()) return fault_status();
  return ok();
}

hq_status hq_repack_int4_ref(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N) {
  if (!src || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  if (K == 0 || N == 0 || K % 32) return fail(HQ_ERR_SHAPE, "K=%u must be a positive multiple of 32, N=%u > 0", K, N);
  const uint32_t nkq = K / 32;
  parallel_for(nkq, [=](size_t b, size_t e) {
    for (size_t kq = b; kq < e; ++kq)
      for (uint32_t n = 0; n < N; ++n) {
        const size_t o = (kq * N + n) * 4;
        for (uint32_t j = 0; j < 4; ++j) dst[o + j] = src[(4 * kq + j) * N + n];
      }
  });
  return ok();
}

hq_status hq_repack_int4(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N) {
  if (!src || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_repack_shape(HQ_FORMAT_INT4, K, N);
  if (st != HQ_OK) return st;
  const uint32_t nkb = K / hq::kBlockK, nt = hq::col_tiles(N);
  parallel_for((size_t)nt * nkb, [=](size_t b, size_t e) {
    for (size_t blk = b; blk < e; ++blk) {
      const uint32_t ct = (uint32_t)(blk / nkb), kb = (uint32_t)(blk % nkb);
      uint32_t* o = dst + blk * 256;
      for (uint32_t lane = 0; lane < 64; ++lane) {
        const uint32_t n = ct * 16 + (lane & 15);
        for (uint32_t w = 0; w < 4; ++w) {
          const uint32_t lin = n < N ? src[(size_t)hq::int4_linear_kw(kb, lane, w) * N + n] : 0x88888888u;
          o[lane * 4 + w] = hq::int4_linear_to_tile(lin);
        }
      }
    }
  });
  return ok();
}

hq_status hq_unpack_int4(const uint32_t* packed, uint32_t* dst, uint32_t K, uint32_t N) {
  if (!packed || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_repack_shape(HQ_FORMAT_INT4, K, N);
  if (st != HQ_OK) return st;
  const uint32_t nkb = K / hq::kBlockK, nt = hq::col_tiles(N);
  parallel_for((size_t)nt * nkb, [=](size_t b, size_t e) {
    for (size_t blk = b; blk < e; ++blk) {
      const uint32_t ct = (uint32_t)(blk / nkb), kb = (uint32_t)(blk % nkb);
      const uint32_t* p = packed + blk * 256;
      for (uint32_t lane = 0; lane < 64; ++lane) {
        const uint32_t n = ct * 16 + (lane & 15);
        if (n >= N) continue;
        for (uint32_t w = 0; w < 4; ++w)
          dst[(size_t)hq::int4_linear_kw(kb, lane, w) * N + n] = hq::int4_tile_to_linear(p[lane * 4 + w]);
      }
    }
  });
  return ok();
}

hq_status hq_repack_ternary2(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N) {
  if (!src || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_repack_shape(HQ_FORMAT_TERNARY2, K, N);
  if (st != HQ_OK) return st;
  const uint32_t nkb = K / hq::kBlockK, nt = hq::col_tiles(N);
  std::vector<char> bad_by_chunk(nt, 0);
  char* badp = bad_by_chunk.data();
  parallel_for(nt, [=](size_t b, size_t e) {
    for (size_t ct = b; ct < e; ++ct) {
      bool bad = false;
      for (uint32_t kb = 0; kb < nkb; ++kb) {
        uint32_t* o = dst + ((size_t)ct * nkb + kb) * 128;
        for (uint32_t lane = 0; lane < 64; ++lane) {
          const uint32_t n = (uint32_t)ct * 16 + (lane & 15), g4 = lane >> 4;
          for (uint32_t w = 0; w < 2; ++w) {
            uint32_t out = 0;
            if (n < N) {
              const size_t kw0 = (size_t)8 * kb + 4 * w + (g4 >> 1);
              out = hq::tern_pack_word(src[kw0 * N + n], src[(kw0 + 2) * N + n], g4 & 1, &bad);
            }
            o[lane * 2 + w] = out;
          }
        }
      }
      badp[ct] = bad;
    }
  });
  for (uint32_t i = 0; i < nt; ++i)
    if (bad_by_chunk[i]) return fail(HQ_ERR_BAD_CODE, "ternary code 3 in column tile %u", i);
  return ok();
}

hq_status hq_unpack_ternary2(const uint32_t* packed, uint32_t* dst, uint32_t K, uint32_t N) {
  if (!packed || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_repack_shape(HQ_FORMAT_TERNARY2, K, N);
  if (st != HQ_OK) return st;
  const uint32_t nkb = K / hq::kBlockK;
  // Each linear word (kw, n) gathers 8 codes from each of two packed words.
  parallel_for((size_t)(K / 16), [=](size_t b, size_t e) {
    for (size_t kw = b; kw < e; ++kw) {
      for (uint32_t n = 0; n < N; ++n) {
        uint32_t lin = 0;
        for (uint32_t i = 0; i < 16; ++i) {
          const uint32_t k = (uint32_t)kw * 16 + i;
          const uint32_t kb = k / 128, r = k % 128, c = r / 32, g4 = (r % 32) / 8, el = r % 8;
          const uint32_t lane = g4 * 16 + (n % 16), w = c >> 1, cw = c & 1;
          const uint32_t word = packed[(((size_t)(n / 16) * nkb + kb) * 64 + lane) * 2 + w];
          const uint32_t f = (word >> hq::tern_field_bit(cw, el)) & 3u;
          lin |= hq::tern_field_to_c(f) << (2 * i);
        }
        dst[kw * N + n] = lin;
      }
    }
  });
  return ok();
}

size_t hq_tq1_0_bytes(uint32_t K, uint32_t N) {
  if (K == 0 || N == 0 || K % hq::kTq1K) return 0;
  return (size_t)N * (K / hq::kTq1K) * hq::kTq1Bytes;
}

hq_status hq_convert_tq1_0(const void* blocks, uint32_t K, uint32_t N, uint32_t* codes, uint16_t* scales) {
  if (!blocks || !codes || !scales) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  if (hq_tq1_0_bytes(K, N) == 0) return fail(HQ_ERR_SHAPE, "K=%u must be a positive multiple of 256, N=%u > 0", K, N);
  const uint32_t nb = K / hq::kTq1K;
  const uint8_t* src = static_cast<const uint8_t*>(blocks);
  parallel_for(N, [=](size_t b, size_t e) {
    for (size_t n = b; n < e; ++n)
      for (uint32_t blk = 0; blk < nb; ++blk) {
        const uint8_t* p = src + (n * nb + blk) * hq::kTq1Bytes;
        scales[(size_t)blk * N + n] = (uint16_t)(p[0] | (p[1] << 8));
        for (uint32_t w = 0; w < hq::kTq1K / 16; ++w) {
          uint32_t lin = 0;
          for (uint32_t i = 0; i < 16; ++i) lin |= hq::tq1_code(p + 2, 16 * w + i) << (2 * i);
          codes[((size_t)blk * (hq::kTq1K / 16) + w) * N + n] = lin;
        }
      }
  });
  return ok();
}

hq_status hq_repack_tq1_0_device(const void* blocks, uint32_t K, uint32_t N, uint32_t* packed, uint16_t* scales,
                                 hq_stream stream) {
  if (!blocks || !packed || !scales) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  if (hq_tq1_0_bytes(K, N) == 0) return fail(HQ_ERR_SHAPE, "K=%u must be a positive multiple of 256, N=%u > 0", K, N);
  if (reinterpret_cast<uintptr_t>(blocks) % 8 || reinterpret_cast<uintptr_t>(packed) % 4 ||
      reinterpret_cast<uintptr_t>(scales) % 2)
    return fail(HQ_ERR_ALIGNMENT, "blocks must be 8-byte, packed 4-byte and scales 2-byte aligned");
  return from_hip(hq::launch_repack_tq1_0(static_cast<const uint8_t*>(blocks), packed, scales, K, N,
                                          reinterpret_cast<hipStream_t>(stream)),
                  "repack launch");
}

hq_status hq_repack_int4_device(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N, hq_stream stream) {
  if (!src || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_repack_shape(HQ_FORMAT_INT4, K, N);
  if (st != HQ_OK) return st;
  return from_hip(hq::launch_repack_int4(src, dst, K, N, reinterpret_cast<hipStream_t>(stream)), "repack launch");
}

hq_status hq_repack_ternary2_device(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N, uint32_t* bad,
                                    hq_stream stream) {
  if (!src || !dst) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_repack_shape(HQ_FORMAT_TERNARY2, K, N);
  if (st != HQ_OK) return st;
  return from_hip(hq::launch_repack_ternary2(src, dst, K, N, bad, reinterpret_cast<hipStream_t>(stream)),
                  "repack launch");
}

hq_status hq_gemm_w4a16(const void* X, hq_dtype dtype, int64_t ldx, const uint32_t* Wp, const uint16_t* scales,
                        const float* bias, void* Y, int64_t ldy, uint32_t M, uint32_t K, uint32_t N, uint32_t group,
                        void* ws, size_t ws_bytes, hq_stream stream) {
  hq_segment s{Wp, scales, bias, Y, ldy, N};
  return run_gemm(X, dtype, ldx, HQ_FORMAT_INT4, &s, 1, M, K, group, ws, ws_bytes, stream);
}

hq_status hq_gemm_w2a16(const void* X, hq_dtype dtype, int64_t ldx, const uint32_t* Wp, const uint16_t* scales,
                        void* Y, int64_t ldy, uint32_t M, uint32_t K, uint32_t N, uint32_t group, void* ws,
                        size_t ws_bytes, hq_stream stream) {
  hq_segment s{Wp, scales, nullptr, Y, ldy, N};
  return run_gemm(X, dtype, ldx, HQ_FORMAT_TERNARY2, &s, 1, M, K, group, ws, ws_bytes, stream);
}

hq_status hq_gemm_fused(const void* X, hq_dtype dtype, int64_t ldx, hq_format fmt, const hq_segment* segs,
                        uint32_t nseg, uint32_t M, uint32_t K, uint32_t group, void* ws, size_t ws_bytes,
                        hq_stream stream) {
  return run_gemm(X, dtype, ldx, fmt, segs, nseg, M, K, group, ws, ws_bytes, stream);
}

// ---- the int8 path (hq_int8.hip) ----
size_t hq_int8_packed_bytes(uint32_t K, uint32_t N) {
  if (K == 0 || N == 0 || K % hq::kBlockK) return 0;
  return (size_t)K * hq::col_tiles(N) * 16u;
}

hq_status hq_repack_int8(const int8_t* w, uint32_t K, uint32_t N, int8_t* packed) {
  if (!w || !packed) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_int8_shape(K, N);
  if (st != HQ_OK) return st;
  const uint32_t nkb = K / hq::kBlockK, nt = hq::col_tiles(N);
  parallel_for((size_t)nt * nkb, [=](size_t b, size_t e) {
    for (size_t blk = b; blk < e; ++blk) {
      const uint32_t ct = (uint32_t)(blk / nkb), kb = (uint32_t)(blk % nkb);
      for (uint32_t kk = 0; kk < 128u; ++kk)
        for (uint32_t c16 = 0; c16 < 16u; ++c16) {
          const uint32_t k = kb * 128u + kk, n = ct * 16u + c16;
          packed[int8_tile_byte(k, n, nkb)] = n < N ? w[(size_t)k * N + n] : (int8_t)0;
        }
    }
  });
  return HQ_OK;
}

hq_status hq_unpack_int8(const int8_t* packed, uint32_t K, uint32_t N, int8_t* w) {
  if (!w || !packed) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_int8_shape(K, N);
  if (st != HQ_OK) return st;
  const uint32_t nkb = K / hq::kBlockK;
  parallel_for((size_t)K, [=](size_t b, size_t e) {
    for (size_t k = b; k < e; ++k)
      for (uint32_t n = 0; n < N; ++n) w[k * N + n] = packed[int8_tile_byte((uint32_t)k, n, nkb)];
  });
  return HQ_OK;
}

hq_status hq_workspace_bytes_w8a8(uint32_t M, uint32_t K, uint32_t N, size_t* bytes) {
  if (!bytes) return fail(HQ_ERR_INVALID_ARG, "bytes is null");
  hq_status st = check_int8_shape(K, N);
  if (st != HQ_OK) return st;
  if (M == 0 || M > 16) return fail(HQ_ERR_UNSUPPORTED, "the int8 path takes 1..16 rows, got M=%u", M);
  const hq::W8Config c = hq::choose_w8a8(M, K, N);
  if (!c.ok) return fail(HQ_ERR_UNSUPPORTED, "no int8 plan for M=%u K=%u N=%u", M, K, N);
  *bytes = hq::w8a8_workspace_bytes(M, K, N, c);
  return HQ_OK;
}

hq_status hq_gemm_w8a8(const float* X, int64_t ldx, const int8_t* Wp, const float* scales, float* Y, int64_t ldy,
                       uint32_t M, uint32_t K, uint32_t N, void* ws, size_t ws_bytes, hq_stream stream) {
  if (take_fault()) return fault_status();
  if (!X || !Wp || !scales || !Y) return fail(HQ_ERR_INVALID_ARG, "null pointer");
  hq_status st = check_int8_shape(K, N);
  if (st != HQ_OK) return st;
  if (M == 0 || M > 16) return fail(HQ_ERR_UNSUPPORTED, "the int8 path takes 1..16 rows, got M=%u", M);
  if (ldx < (int64_t)K || ldx % 4) return fail(HQ_ERR_SHAPE, "ldx=%lld must be >= K=%u and a multiple of 4", (long long)ldx, K);
  if (ldy < (int64_t)N) return fail(HQ_ERR_SHAPE, "ldy=%lld < N=%u", (long long)ldy, N);
  if ((uint64_t)M * (uint64_t)ldx >= (1ull << 29) || (uint64_t)M * (uint64_t)ldy >= (1ull << 31))
    return fail(HQ_ERR_SHAPE, "X or Y too large for 32-bit offsets");
  if (reinterpret_cast<uintptr_t>(X) % 16 || reinterpret_cast<uintptr_t>(Wp) % 16)
    return fail(HQ_ERR_ALIGNMENT, "X and Wp must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(scales) % 4 || reinterpret_cast<uintptr_t>(Y) % 4)
    return fail(HQ_ERR_ALIGNMENT, "scales and Y must be 4-byte aligned");
  const hq::W8Config c = hq::choose_w8a8(M, K, N);
  if (!c.ok) return fail(HQ_ERR_UNSUPPORTED, "no int8 plan for M=%u K=%u N=%u", M, K, N);
  const size_t need = hq::w8a8_workspace_bytes(M, K, N, c);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* w = nullptr;
  if (ws) {
    if (ws_bytes < need)
      return fail(HQ_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu this call needs", ws_bytes, need);
    if (reinterpret_cast<uintptr_t>(ws) % 256) return fail(HQ_ERR_ALIGNMENT, "workspace must be 256-byte aligned");
    w = ws;
  } else if ((st = get_internal_ws(s, need, &w)) != HQ_OK) {
    return st;
  }
  return from_hip(hq::launch_w8a8(X, (uint32_t)ldx, Wp, scales, Y, (uint32_t)ldy, M, K, N, c, w, s), "int8 launch");
}

hq_status hq_gemm_fused_noalloc(const void* X, hq_dtype dtype, int64_t ldx, hq_format fmt, const hq_segment* segs,
                                uint32_t nseg, uint32_t M, uint32_t K, uint32_t group, hq_stream stream) {
  hq::GemmDesc d;
  hq_status st = prepare(X, dtype, ldx, fmt, segs, nseg, M, K, group, &d);
  if (st != HQ_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const Plan p = make_plan(fmt, d, kScratchBytes, dtype);
  if (p.need > kScratchBytes)
    return fail(HQ_ERR_WORKSPACE, "this call needs %zu workspace bytes, more than the %zu-byte static scratch",
                p.need, kScratchBytes);
  void* w = nullptr;
  if (p.need > 0 && (st = scratch_ptr(s, &w)) != HQ_OK) return st;
  return launch_plan(fmt, dtype, d, p, w, fault_ptr_if_any(), s);
}

}  // extern "C"

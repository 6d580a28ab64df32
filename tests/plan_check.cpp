// CPU check of the decode work decomposition (nebula_amd/csrc/hq_plan.hpp), built with g++
// by tests/test_plan.py. For each (G, nkb, P, WK) it walks every workgroup and wavefront
// exactly as the kernel does and checks that
//   * every unit (slab, k-block) is computed by exactly one (workgroup, wavefront);
//   * the pieces of a workgroup are its slabs, each once, and only pieces 0 and 1 can be
//     partial;
//   * for every partial slab, the contributors found by plan_wg_of_unit are exactly the
//     workgroups that hold a partial piece of it, and the workspace slot each reader
//     derives equals the slot its writer used;
//   * the piece count never exceeds plan_np_max and the wavefronts counted by the
//     reduction (min(WK, kz - ka)) are exactly those with units in the piece;
//   * plan_group_of_kb equals kb / gkb.
// Prints "ok <cases>" or the first failure.
#include <cstdint>
#include <cstdio>
#include <map>
#include <set>
#include <vector>

#include "hq_plan.hpp"

using namespace hq;

static int fail(const char* what, uint32_t G, uint32_t nkb, uint32_t P, uint32_t WK) {
  std::printf("FAIL %s G=%u nkb=%u P=%u WK=%u\n", what, G, nkb, P, WK);
  return 1;
}

static int check(uint32_t G, uint32_t nkb, uint32_t P, uint32_t WK) {
  const uint32_t utot = G * nkb;
  if (P > utot) return 0;
  const uint32_t L = utot / P, rem = utot % P;
  std::vector<int> seen(utot, 0);
  std::map<uint32_t, std::set<uint32_t>> writers;        // slab -> workgroups with a partial piece
  std::map<std::pair<uint32_t, uint32_t>, uint32_t> slot_of;  // (wg, slab) -> slot written
  const uint32_t npmax = plan_np_max(utot, P, nkb);
  for (uint32_t b = 0; b < P; ++b) {
    const uint32_t u0 = plan_begin(L, rem, b), u1 = plan_begin(L, rem, b + 1);
    if (u1 <= u0) return fail("empty range", G, nkb, P, WK);
    if (u1 - u0 > L + 1 || u1 - u0 < L) return fail("unbalanced range", G, nkb, P, WK);
    if (plan_wg_of_unit(L, rem, u0) != b || plan_wg_of_unit(L, rem, u1 - 1) != b)
      return fail("wg_of_unit", G, nkb, P, WK);
    const uint32_t gfirst = u0 / nkb, glast = (u1 - 1) / nkb, np = glast - gfirst + 1;
    if (np > npmax) return fail("np_max", G, nkb, P, WK);
    std::set<uint32_t> slabs;
    for (uint32_t i = 0; i < np; ++i) {
      const uint32_t g = plan_piece_slab(gfirst, glast, i);
      if (!slabs.insert(g).second) return fail("slab twice", G, nkb, P, WK);
      const uint32_t ka = g == gfirst ? u0 - g * nkb : 0, kz = g == glast ? u1 - g * nkb : nkb;
      const bool full = ka == 0 && kz == nkb;
      if (!full && i >= 2) return fail("partial piece >= 2", G, nkb, P, WK);
      if (!full && !plan_has_partial(G, P)) return fail("has_partial", G, nkb, P, WK);
      if (!full) {
        writers[g].insert(b);
        slot_of[{b, g}] = i;
      }
      uint32_t with_units = 0;
      for (uint32_t w = 0; w < WK; ++w) {
        bool any = false;
        for (uint32_t kb = ka + w; kb < kz; kb += WK) {
          const uint32_t u = g * nkb + kb;
          if (u < u0 || u >= u1) return fail("unit outside range", G, nkb, P, WK);
          ++seen[u];
          any = true;
        }
        if (any) {
          if (w != with_units) return fail("wavefronts with units not a prefix", G, nkb, P, WK);
          ++with_units;
        }
      }
      if (with_units != (WK < kz - ka ? WK : kz - ka)) return fail("nw", G, nkb, P, WK);
    }
    if (slabs.size() != np) return fail("slab count", G, nkb, P, WK);
  }
  if (plan_begin(L, rem, P) != utot) return fail("ranges do not end at utot", G, nkb, P, WK);
  for (uint32_t u = 0; u < utot; ++u)
    if (seen[u] != 1) return fail("coverage", G, nkb, P, WK);
  for (auto& kv : writers) {
    const uint32_t g = kv.first;
    const uint32_t bf = plan_wg_of_unit(L, rem, g * nkb), bl = plan_wg_of_unit(L, rem, (g + 1) * nkb - 1);
    std::set<uint32_t> expect;
    for (uint32_t c = bf; c <= bl; ++c) expect.insert(c);
    if (expect != kv.second || bl == bf) return fail("contributors", G, nkb, P, WK);
    for (uint32_t c = bf; c <= bl; ++c) {
      const uint32_t reader_slot = plan_begin(L, rem, c) / nkb == g ? 0u : 1u;
      if (slot_of[{c, g}] != reader_slot) return fail("slot", G, nkb, P, WK);
    }
  }
  return 0;
}

int main() {
  int cases = 0;
  const uint32_t Gs[] = {1, 2, 3, 5, 16, 80, 81, 432, 433};
  const uint32_t nkbs[] = {1, 2, 3, 8, 40, 216};
  const uint32_t Ps[] = {1, 2, 3, 7, 64, 255, 256, 257, 512, 1000};
  const uint32_t WKs[] = {1, 3, 8, 16};
  for (uint32_t G : Gs)
    for (uint32_t nkb : nkbs)
      for (uint32_t P : Ps)
        for (uint32_t WK : WKs) {
          if (check(G, nkb, P, WK)) return 1;
          ++cases;
        }
  {
    const uint32_t ds[] = {1, 2, 3, 5, 7, 8, 16, 40, 216, 1000, 65535, 65536, 0x7FFFFFFFu, 0xFFFFFFFFu};
    const uint32_t us[] = {0, 1, 2, 3, 39, 40, 41, 215, 216, 217, 65535, 65536, 0x7FFFFFFEu, 0x7FFFFFFFu, 0x80000000u,
                           0xFFFFFFFEu, 0xFFFFFFFFu};
    for (uint32_t d : ds) {
      const uint32_t m = plan_div_magic(d);
      for (uint32_t u : us)
        for (int64_t du = -2; du <= 2; ++du) {
          const uint32_t x = (uint32_t)((int64_t)u + du);
          if (plan_div(x, d, m) != x / d) {
            std::printf("FAIL div u=%u d=%u\n", x, d);
            return 1;
          }
        }
      for (uint32_t x = 0; x < 200000; ++x)
        if (plan_div(x, d, m) != x / d) {
          std::printf("FAIL div u=%u d=%u\n", x, d);
          return 1;
        }
    }
  }
  for (uint32_t gkb = 1; gkb <= 40; ++gkb) {
    const uint32_t gmul = plan_gmul(gkb);
    for (uint32_t kb = 0; kb < 100000; ++kb)
      if (plan_group_of_kb(kb, gmul) != kb / gkb) {
        std::printf("FAIL group_of_kb kb=%u gkb=%u\n", kb, gkb);
        return 1;
      }
  }
  std::printf("ok %d\n", cases);
  return 0;
}

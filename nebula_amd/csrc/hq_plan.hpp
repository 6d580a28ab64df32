// hq_plan.hpp — work decomposition of the decode kernel, shared by host and device code.
//
// The output columns of all segments are cut into "slabs" of T column tiles (16 columns
// each); a unit of work is one slab times one 128-deep k-block, and units are numbered
// slab-major: u = g * nkb + kb. The grid has P workgroups and workgroup b owns the
// contiguous unit range [begin(b), begin(b + 1)) with begin(b) = b * L + min(b, rem),
// L = utot / P, rem = utot % P (the first rem workgroups take one unit more), so every
// workgroup streams the same number of weight bytes (+-1 unit) whatever N and K are;
// the kernel computes its range without a division. A slab whose k range is cut by a range boundary ("partial piece") is finished by
// a fix-up: every contributing workgroup writes its fp32 partial tile to the workspace,
// and the last one to arrive (per-slab counter) sums the partials in workgroup order and
// stores the output, so the result does not depend on arrival order.
//
// Inside a workgroup, pieces are numbered: 0 = the slab of the first unit, 1 = the slab
// of the last unit (when different), 2.. = the slabs in between (always whole). Only
// pieces 0 and 1 can be partial; their partials go to workspace slots 0 and 1 of the
// workgroup.
#pragma once
#include <stdint.h>

#include "hq_layout.hpp"

namespace hq {

struct DecodePlan {
  uint32_t G;     // slabs over all segments
  uint32_t utot;  // G * nkb
  uint32_t P;     // workgroups
  uint32_t WK;    // wavefronts per workgroup
  uint32_t L;     // utot / P
  uint32_t rem;   // utot % P
  uint32_t nkb_m; // plan_div_magic(nkb)
  uint32_t wk_m;  // plan_div_magic(WK)
  uint32_t np_max;  // largest number of pieces of one workgroup
  uint32_t gmul;    // ceil(2^32 / gkb) for the k-block -> scale-group division (0 when gkb == 1)
  uint32_t contig;  // 1: wavefront w takes k-blocks [ka + w*len/WK, ka + (w+1)*len/WK) of a piece;
                    // 0: k-blocks ka + w, ka + w + WK, ...
  float* part;      // [P][2][M * 16 * T] partial tiles (null when no piece is partial)
  uint32_t* cnt;    // [G] arrival counters, zero between launches
};

HQ_HD uint32_t plan_begin(uint32_t L, uint32_t rem, uint32_t b) { return b * L + (b < rem ? b : rem); }

// Workgroup whose range holds unit u: the largest b with begin(b) <= u.
HQ_HD uint32_t plan_wg_of_unit(uint32_t L, uint32_t rem, uint32_t u) {
  const uint32_t head = rem * (L + 1u);  // units of the workgroups with L + 1 units
  return u < head ? u / (L + 1u) : rem + (u - head) / L;
}

// Largest piece count of any workgroup: a range of at most L + (rem > 0) units touches
// at most floor((Lmax - 1) / nkb) + 2 slabs.
HQ_HD uint32_t plan_np_max(uint32_t utot, uint32_t P, uint32_t nkb) {
  if (utot % P == 0 && (utot / P) % nkb == 0) return utot / P / nkb;  // ranges aligned to slabs
  const uint32_t L = (utot + P - 1) / P;
  const uint32_t n = (L - 1) / nkb + 2;
  const uint32_t g = utot / nkb;
  return n < g ? n : g;
}

// Slab of piece i of a workgroup whose slabs run from gfirst to glast.
HQ_HD uint32_t plan_piece_slab(uint32_t gfirst, uint32_t glast, uint32_t i) {
  return i == 0 ? gfirst : (i == 1 ? glast : gfirst + i - 1);
}

// Prefill grid: the first psk workgroups share the last (tiles - dp) output tiles along K
// (stream-K over units (tile - dp) * nkb + kb, ranges as above); the dp workgroups after
// them own one whole tile each. Splitting only the tiles that would leave the last round
// of the grid part-empty keeps the fix-up traffic to that round.
struct PrefillPlan {
  uint32_t psk;     // stream-K workgroups (grid x indices [0, psk))
  uint32_t dp;      // whole-tile workgroups after them (logical tiles [0, dp))
  uint32_t xcd;     // 1: number the whole-tile workgroups XCD-major (dp % 8 == 0)
  uint32_t L, rem;  // stream-K ranges: begin(s) = s * L + min(s, rem)
  uint32_t nkb_m;   // plan_div_magic(nkb)
  uint32_t nb;      // 256-column blocks over all segments (tile = row band * nb + block)
  uint32_t bands;   // row bands (tiles = bands * nb)
  uint32_t gb;      // whole tiles are visited in groups of gb row bands, column-block major
  float* part;      // [psk][2][tile] fp32 partial tiles (null when psk == 0)
  uint32_t* cnt;    // [tiles - dp] arrival counters, zero between launches
  uint32_t* fault;  // host-visible word set to 1 when a bounded wait gives up (may be null)
  uint32_t spin;    // polls before the K halves' k-block barrier gives up (KS = 2)
};

// Exact u / d for any 32-bit u without a divide instruction: m = floor((2^32 - 1) / d)
// makes mulhi(u, m) at most one below the quotient, and one step corrects it.
HQ_HD uint32_t plan_div_magic(uint32_t d) { return (uint32_t)(0xFFFFFFFFu / d); }
HQ_HD uint32_t plan_div(uint32_t u, uint32_t d, uint32_t m) {
  const uint32_t q = (uint32_t)(((uint64_t)u * m) >> 32);  // q * d <= u
  return u - q * d >= d ? q + 1u : q;
}

// Whether some workgroup range boundary falls inside a slab.
HQ_HD bool plan_has_partial(uint32_t G, uint32_t P) { return G % P != 0; }

// k-block -> scale group with the multiplier of DecodePlan::gmul (exact for kb * gkb < 2^32).
HQ_HD uint32_t plan_group_of_kb(uint32_t kb, uint32_t gmul) {
  return gmul == 0 ? kb : (uint32_t)(((uint64_t)kb * gmul) >> 32);
}
HQ_HD uint32_t plan_gmul(uint32_t gkb) {
  return gkb == 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + gkb - 1) / gkb);
}

}  // namespace hq

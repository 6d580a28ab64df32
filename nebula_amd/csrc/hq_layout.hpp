// hq_layout.hpp — the gfx950 packed-weight tile layouts, shared by host and device code.
//
// Both formats are cut into "k-blocks" of 16 output columns x 128 reduction indices,
// one per column tile (ct) and k-block (kb), stored column-tile-major:
//     block (ct, kb) starts at word (ct * nkb + kb) * 64 * WPL, nkb = K / 128,
// where WPL (words per lane) is 4 for int4 and 2 for ternary. Inside a block, lane
// l (0..63) of a wavefront owns WPL consecutive words, so one wavefront load of
// 64 x (4 * WPL) bytes is a single contiguous, fully coalesced 1 KiB (int4) or
// 512 B (ternary) read. Lane l serves output column n = 16*ct + (l % 16) and the
// 8-wide k slice g4 = l / 16 of every 32-wide chunk, which is exactly the B-operand
// fragment of v_mfma_f32_16x16x32_{f16,bf16}: chunk c (0..3) of a block covers
// k = 128*kb + 32*c + 8*g4 + e, e = 0..7.
//
// int4: word w of lane l holds chunk c = w. The nibble of element e sits at nibble
//   position P_OF_E[e] = {0,4,1,5,2,6,3,7}[e], so that (word & 0x000F000F) yields the
//   pair (e=0, e=1) in the two fp16 halves, (word & 0x00F000F0) yields (2, 3), and the
//   same two masks on (word >> 8) yield (4, 5) and (6, 7). Codes are the reference's
//   unsigned nibbles q (value (q - 8) * scale). Each packed word is one linear word
//   (kw = 16*kb + 4*c + g4, n) with its nibbles permuted.
// ternary: word w of lane l holds chunks 2w and 2w+1 (cw = 0, 1). Element (cw, e)
//   occupies the 2-bit field whose low bit is 14 - 8*cw - e (e even) or
//   30 - 8*cw - (e - 1) (e odd), so (word << 2a) & 0xC000C000, a = 4*cw + e/2, moves
//   the pair (e, e+1) of chunk cw to bits 14..15 and 30..31. The field is
//   (sign, nonzero): +1 -> 01, 0 -> 00, -1 -> 11, i.e. exactly the top two bits of the
//   fp16 / bf16 encodings of +2, 0 and -2.
//
// Columns past N (up to the next multiple of 16) are padding that decodes to zero
// (int4 code 8, ternary 00). K must be a multiple of 128.
#pragma once
#include <stdint.h>

#ifdef __HIPCC__
#define HQ_HD __host__ __device__ __forceinline__
#else
#define HQ_HD inline
#endif

namespace hq {

constexpr uint32_t kTileN = 16;   // output columns per tile
constexpr uint32_t kBlockK = 128; // reduction indices per k-block
constexpr uint32_t kLanes = 64;   // wavefront size

HQ_HD uint32_t words_per_lane(int fmt) { return fmt == 1 ? 4u : 2u; }
HQ_HD uint32_t col_tiles(uint32_t N) { return (N + kTileN - 1) / kTileN; }

// Nibble unshuffle: linear nibble e -> position P_OF_E[e] (even e to 0..3, odd e to 4..7).
HQ_HD uint32_t int4_linear_to_tile(uint32_t x) {
  uint32_t t = (x ^ (x >> 4)) & 0x00F000F0u;  // swap nibbles 1<->2 and 5<->6
  x ^= t ^ (t << 4);
  t = (x ^ (x >> 8)) & 0x0000FF00u;           // swap bytes 1<->2
  x ^= t ^ (t << 8);
  return x;
}
HQ_HD uint32_t int4_tile_to_linear(uint32_t x) {
  uint32_t t = (x ^ (x >> 8)) & 0x0000FF00u;
  x ^= t ^ (t << 8);
  t = (x ^ (x >> 4)) & 0x00F000F0u;
  x ^= t ^ (t << 4);
  return x;
}

// Linear int4 word index for packed word (ct, kb, lane, w), and its column.
HQ_HD uint32_t int4_linear_kw(uint32_t kb, uint32_t lane, uint32_t w) { return 16u * kb + 4u * w + lane / 16u; }

// Bit offset of ternary element (cw, e) inside its packed word.
HQ_HD uint32_t tern_field_bit(uint32_t cw, uint32_t e) {
  return (e & 1u) ? (30u - 8u * cw - (e - 1u)) : (14u - 8u * cw - e);
}
// Reference code c = t + 1 (0, 1, 2) -> (sign, nonzero) field; 3 is invalid.
HQ_HD uint32_t tern_c_to_field(uint32_t c) { return c == 0u ? 3u : (c == 2u ? 1u : 0u); }
HQ_HD uint32_t tern_field_to_c(uint32_t f) { return f == 3u ? 0u : (f == 1u ? 2u : 1u); }

// Build packed ternary word (kb, lane, w) from the two linear words holding its chunks.
// lin0 holds chunk 2w, lin1 chunk 2w+1; half = (lane/16) % 2 selects the 8 codes.
// Sets *bad when a code 3 is met.
HQ_HD uint32_t tern_pack_word(uint32_t lin0, uint32_t lin1, uint32_t half, bool* bad) {
  uint32_t out = 0;
  for (uint32_t cw = 0; cw < 2; ++cw) {
    uint32_t lin = cw ? lin1 : lin0;
    for (uint32_t e = 0; e < 8; ++e) {
      uint32_t c = (lin >> (2u * (8u * half + e))) & 3u;
      if (c == 3u) *bad = true;
      out |= tern_c_to_field(c) << tern_field_bit(cw, e);
    }
  }
  return out;
}


// GGUF TQ1_0 (the PrismML block, GGML type 143; hydrogen/src/model/native_decoder.cu:31-36):
// 256 weights in 56 bytes: fp16 d (bytes 0..1), 52 bytes of base-3 trits (2..53), 2 padding
// bytes. Element i < 250 is digit i % 5 of trit byte i / 5, element 250 + j is digit j % 3 of
// trit byte 50 + j / 3, digit j of a byte being (byte / 3^j) % 3 for any byte value
// (native_decoder.cu:87-101). The digit is the ternary code c = t + 1 of the element.
constexpr uint32_t kTq1Bytes = 56;
constexpr uint32_t kTq1K = 256;
HQ_HD uint32_t tq1_code(const uint8_t* trits, uint32_t i) {
  const uint32_t byte = i < 250u ? i / 5u : 50u + (i - 250u) / 3u;
  const uint32_t digit = i < 250u ? i % 5u : (i - 250u) % 3u;
  uint32_t v = trits[byte];
  for (uint32_t j = 0; j < digit; ++j) v /= 3u;
  return v % 3u;
}
}  // namespace hq

/*
 * hq_oracle.h — CPU restatement of hydrogen's weight-only quantized GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle: tests, the smoke
 * check and the CPU-baseline leg of the benchmark call it. Nothing in the
 * product library (nebula_amd/) links or loads it.
 *
 * Every function restates one piece of the reference (paths relative to the
 * reference repository root):
 *   hqo_repack_ref        hydrogen/src/model/marlin_gemm.cu:432-467 (loop 446-455)
 *   hqo_dequant_int4      hydrogen/src/model/marlin_gemm.cu:495-512 (w = q*s + b, b = -8*s, :483-488)
 *   hqo_dequant_int4_bias the same with a caller-given fp32 bias per group (marlin_gemm.hpp:100-107,
 *                         the forward's d_biases; marlin_gemm.cu:195-196 reads it per 32-wide chunk)
 *   hqo_dequant_ternary2  hydrogen/src/model/native_decoder.cu:184-186 (w = d * t)
 *   hqo_gemm_f32          hydrogen/src/model/marlin_gemm.cu:52-70 (fp32, k ascending, FMA)
 *   hqo_qgemm             the two above fused row by row (bit-identical to running them in turn)
 *   hqo_qgemm_bias        hqo_qgemm with the bias of hqo_dequant_int4_bias (NULL: hqo_qgemm)
 *   hqo_fidelity          hydrogen/src/model/marlin_gemm.cu:619-644 (max |d|, MSE in fp64)
 *   hqo_tq1_0_code        hydrogen/src/model/native_decoder.cu:31-36, 87-101 (base-3 trits of a TQ1_0 block)
 *   hqo_gemv_tq1_0        hydrogen/src/model/native_decoder.cu:155-206 (kernel_gemv_tq1_0, any M)
 *   hqo_dequant_q4_k      GGML's published Q4_K block (dequantize_row_q4_K of GGML / llama.cpp); the
 *                         reference names the type (hydrogen/include/gguf_parser.hpp:44, 130) but has
 *                         no decoder for it, so this one is pinned by the published layout only
 *   hqo_int8_from_int4    hydrogen/src/model/marlin_gemm.cu:508 (h_W_int8 = q * 16 - 128)
 *   hqo_quantize_x_int8   hydrogen/src/model/marlin_gemm.cu:356-359 (int8(clamp(x * 127, -128, 127)))
 *   hqo_gemm_int8         hydrogen/src/model/marlin_gemm.cu:327-377 (kernel_cutlass_int8_gemm, any M)
 *
 * The generator (hqo_rng_*, hqo_gen_*) is this build's own specification, not
 * the reference's: the reference seeds std::mt19937 with implementation-defined
 * distributions (marlin_gemm.cu:470-472), which no other compiler reproduces.
 *
 * Numeric types cross this interface as raw IEEE bit patterns: uint16_t for
 * fp16 and bf16, float for fp32.
 */
#ifndef HQ_ORACLE_H
#define HQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { HQO_F16 = 1, HQO_BF16 = 2 };
enum { HQO_INT4 = 1, HQO_TERNARY2 = 2 };

/* ---- counter-based generator: splitmix64 finaliser over (seed, stream, index) ---- */
uint64_t hqo_rng_u64(uint64_t seed, uint64_t stream, uint64_t idx);
/* Uniform double in (0, 1]: ((r >> 11) + 1) * 2^-53. */
double hqo_rng_uniform(uint64_t seed, uint64_t stream, uint64_t idx);
/* N(0, sigma) by Box-Muller on draws (2i, 2i+1); |.| when absval != 0; rounded (RNE) to dtype. */
void hqo_gen_normal(uint64_t seed, uint64_t stream, double sigma, int absval, int dtype,
                    uint16_t* out, size_t n);
/* int4 codes uniform on {0..15}: u32 [K/8][N], nibble i of word (kw, n) is k = 8*kw + i. */
void hqo_gen_int4_linear(uint64_t seed, uint64_t stream, uint32_t* out, uint32_t K, uint32_t N);
/* Ternary t in {-1,0,+1} with P = {0.25, 0.5, 0.25}: u32 [K/16][N], bits 2i..2i+1 hold c = t + 1
 * for k = 16*kw + i. */
void hqo_gen_ternary2_linear(uint64_t seed, uint64_t stream, uint32_t* out, uint32_t K, uint32_t N);

/* ---- IEEE conversions (round to nearest even), written from the format definitions ---- */
uint16_t hqo_f32_to_f16(float f);
float hqo_f16_to_f32(uint16_t h);
uint16_t hqo_f32_to_bf16(float f);
float hqo_bf16_to_f32(uint16_t h);
void hqo_to_f32(const uint16_t* in, int dtype, float* out, size_t n);
void hqo_from_f32(const float* in, int dtype, uint16_t* out, size_t n);

/* ---- the reference algorithm ---- */
/* marlin_gemm.cu:446-455: dst[(kq*N + n)*4 + j] = src[(4*kq + j)*N + n], kq < K/32, j < 4. */
void hqo_repack_ref(const uint32_t* src_linear, uint32_t* dst, uint32_t K, uint32_t N);
/* marlin_gemm.cu:495-512 with scale = fp16 scale widened to fp32, bias = -8 * scale:
 * Wdq[k*N + n] = (float)q * scale + bias, evaluated without contraction. */
void hqo_dequant_int4(const uint32_t* w_linear, const uint16_t* scales_f16, uint32_t K, uint32_t N,
                      uint32_t group, float* wdq);
/* marlin_gemm.cu:495-512 with the caller's fp32 bias [K/group][N] (NULL: -8 * scale):
 * Wdq[k*N + n] = (float)q * scale + bias[(k/group)*N + n], evaluated without contraction. Any group
 * that divides K (the reference takes one per 32-wide chunk: group % 32 == 0). */
void hqo_dequant_int4_bias(const uint32_t* w_linear, const uint16_t* scales_f16, const float* bias,
                           uint32_t K, uint32_t N, uint32_t group, float* wdq);
/* native_decoder.cu:184-186: Wdq[k*N + n] = scale * (float)t, t = c - 1. Returns -1 if a code 3 is present. */
int hqo_dequant_ternary2(const uint32_t* w_linear, const uint16_t* scales_f16, uint32_t K, uint32_t N,
                         uint32_t group, float* wdq);
/* marlin_gemm.cu:60-69: Y[m*N + n] = sum_k X[m*K + k] * W[k*N + n], fp32, FMA, k ascending. */
void hqo_gemm_f32(const float* X, const float* W, float* Y, uint32_t M, uint32_t K, uint32_t N,
                  int threads);
/* Dequantize-then-matmul over fp16/bf16 activation bits. X is [M][ldx] (elements), Y is fp32 [M][N].
 * Bit-identical to hqo_dequant_* followed by hqo_gemm_f32 on the widened activations.
 * Returns -1 on an invalid ternary code, 0 otherwise. */
int hqo_qgemm(const uint16_t* X, int xdtype, size_t ldx, int fmt, const uint32_t* w_linear,
              const uint16_t* scales_f16, uint32_t M, uint32_t K, uint32_t N, uint32_t group,
              float* Y, int threads);
/* hqo_qgemm with an int4 bias (hqo_dequant_int4_bias semantics; NULL gives hqo_qgemm). */
int hqo_qgemm_bias(const uint16_t* X, int xdtype, size_t ldx, int fmt, const uint32_t* w_linear,
                   const uint16_t* scales_f16, const float* bias, uint32_t M, uint32_t K, uint32_t N,
                   uint32_t group, float* Y, int threads);
/* marlin_gemm.cu:619-644: max |a - b| and mean squared difference, accumulated in fp64. */
void hqo_fidelity(const float* a, const float* b, size_t count, double* max_abs, double* mse);

/* ---- GGUF TQ1_0 (the reference's PrismML block, GGML type 143): 256 weights in 56 bytes,
 *      fp16 d at bytes 0..1, 52 bytes of base-3 trits at 2..53, 2 padding bytes ---- */
/* native_decoder.cu:87-101: code c = t + 1 (0, 1, 2) of element i (0..255) of one block.
 * Elements 0..249 are digit i % 5 of packed byte i / 5, elements 250..255 digit (i - 250) % 3
 * of packed byte 50 + (i - 250) / 3; digit j of a byte is (byte / 3^j) % 3, by repeated
 * division, for any byte value. */
uint32_t hqo_tq1_0_code(const uint8_t* block, uint32_t i);
/* The block's d as fp16 bits (little-endian bytes 0..1). */
uint16_t hqo_tq1_0_scale(const uint8_t* block);
/* native_decoder.cu:155-206 (kernel_gemv_tq1_0) for M activation rows: W holds N rows of
 * K/256 blocks ([out][in/256], :167). Y[m*N + n] = sum over blocks b of row n whose d is finite
 * (non-finite d: the block is skipped, :174) of sum_i fma(d * t_i, X[m*K + 256 b + i], .), fp32,
 * blocks and elements ascending (the reference splits blocks over 32 lanes and sums the lanes
 * in a tree; results agree within fp32 reassociation). */
void hqo_gemv_tq1_0(const float* X, const uint8_t* W, float* Y, uint32_t M, uint32_t K, uint32_t N,
                    int threads);

/* ---- GGML Q4_K: 144 bytes per 256 weights: fp16 d, fp16 dmin, 12 bytes of 6-bit sub-block
 *      scales and mins, 128 bytes of 4-bit codes ---- */
/* W holds N rows of K/256 blocks. Sub-block j of a block (weights 32 j .. 32 j + 31) has scale
 * sc_j and min m_j: for j < 4, sc = s[j] & 63, m = s[j + 4] & 63; else sc = (s[j + 4] & 15) |
 * ((s[j - 4] >> 6) << 4), m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4). Weight 64 c + l (l < 32) has
 * code q[32 c + l] & 15, weight 64 c + 32 + l the high nibble; w = (d * sc) * q - dmin * m in fp32
 * (separate roundings). Output fp32 Wdq[k*N + n]. */
void hqo_dequant_q4_k(const uint8_t* blocks, uint32_t K, uint32_t N, float* wdq);

/* ---- the int8 path (kernel_cutlass_int8_gemm; never launched by the reference) ---- */
/* out[k*N + n] = q * 16 - 128 for the int4 code q of (k, n) in the linear layout. */
void hqo_int8_from_int4(const uint32_t* w_linear, uint32_t K, uint32_t N, int8_t* out);
/* fminf(fmaxf(x * 127, -128), 127) converted toward zero (NaN -> -128, as fmaxf returns the
 * other operand). */
int8_t hqo_quantize_x_int8(float x);
/* Y[m*N + n] = acc * scales[n], acc accumulating, quad by quad over k (4 q .. 4 q + 3, K / 4
 * quads), fmaf((float)dot, 1.0f / 127.0f, acc) with dot the exact integer product of the
 * quantised activations and W[k*N + n] (int8, [K][N]); X fp32 [M][ldx]; scales fp32 [N] (the
 * reference passes its scale matrix and reads row 0). */
void hqo_gemm_int8(const float* X, size_t ldx, const int8_t* W, const float* scales, uint32_t M, uint32_t K,
                   uint32_t N, float* Y, int threads);

#ifdef __cplusplus
}
#endif
#endif

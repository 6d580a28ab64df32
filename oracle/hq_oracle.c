/*
 * hq_oracle.c — CPU restatement of hydrogen's weight-only quantized GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle). See hq_oracle.h for the function-by-
 * function map to the reference. Build with -ffp-contract=off: the reference's
 * host dequantisation (marlin_gemm.cu:506) is a separate multiply and add, and
 * the only fused multiply-adds are the explicit fmaf() calls of the matmul,
 * which nvcc's default contraction produces in kernel_reference_gemm
 * (marlin_gemm.cu:66).
 */
#include "hq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* generator                                                                 */
/* ------------------------------------------------------------------------- */

static inline uint64_t mix64(uint64_t z) {
    /* splitmix64 finaliser (Steele, Lea, Flood 2014). */
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t hqo_rng_u64(uint64_t seed, uint64_t stream, uint64_t idx) {
    uint64_t key = mix64(seed * 0x9E3779B97F4A7C15ULL + stream * 0xD1B54A32D192ED03ULL + 0x632BE59BD9B4E019ULL);
    return mix64(key + (idx + 1) * 0x9E3779B97F4A7C15ULL);
}

double hqo_rng_uniform(uint64_t seed, uint64_t stream, uint64_t idx) {
    return (double)((hqo_rng_u64(seed, stream, idx) >> 11) + 1) * 0x1.0p-53;
}

void hqo_gen_normal(uint64_t seed, uint64_t stream, double sigma, int absval, int dtype,
                    uint16_t* out, size_t n) {
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) {
        double u1 = hqo_rng_uniform(seed, stream, 2 * (uint64_t)i);
        double u2 = hqo_rng_uniform(seed, stream, 2 * (uint64_t)i + 1);
        double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2) * sigma;
        if (absval) z = fabs(z);
        float f = (float)z;
        out[i] = (dtype == HQO_BF16) ? hqo_f32_to_bf16(f) : hqo_f32_to_f16(f);
    }
}

void hqo_gen_int4_linear(uint64_t seed, uint64_t stream, uint32_t* out, uint32_t K, uint32_t N) {
    size_t words = (size_t)(K / 8) * N;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)words; ++i)
        out[i] = (uint32_t)hqo_rng_u64(seed, stream, (uint64_t)i);
}

void hqo_gen_ternary2_linear(uint64_t seed, uint64_t stream, uint32_t* out, uint32_t K, uint32_t N) {
    size_t words = (size_t)(K / 16) * N;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)words; ++i) {
        uint64_t r = hqo_rng_u64(seed, stream, (uint64_t)i);
        uint32_t w = 0;
        for (int j = 0; j < 16; ++j) {
            uint32_t b0 = (uint32_t)(r >> (2 * j)) & 1u;      /* P = 1/2: t = 0  */
            uint32_t b1 = (uint32_t)(r >> (2 * j + 1)) & 1u;  /* else sign       */
            uint32_t c = b0 ? 1u : (b1 ? 2u : 0u);            /* c = t + 1       */
            w |= c << (2 * j);
        }
        out[i] = w;
    }
}

/* ------------------------------------------------------------------------- */
/* IEEE-754 binary16 / bfloat16 conversions, round to nearest, ties to even   */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t hqo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {                       /* inf or NaN */
        if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                        /* below 2^-14: subnormal result */
        if (a <= 0x33000000u) return (uint16_t)sign;          /* <= 2^-25 rounds to 0 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                /* value / 2^-24 = m >> shift */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((a >> 23) - 112u) << 10) | ((a >> 13) & 0x3FFu);
    uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float hqo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 0x1.0p-24f;          /* exact: m < 2^10 */
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t hqo_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t r = x + 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

float hqo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void hqo_to_f32(const uint16_t* in, int dtype, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = (dtype == HQO_BF16) ? hqo_bf16_to_f32(in[i]) : hqo_f16_to_f32(in[i]);
}

void hqo_from_f32(const float* in, int dtype, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = (dtype == HQO_BF16) ? hqo_f32_to_bf16(in[i]) : hqo_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------- */
/* reference algorithm                                                       */
/* ------------------------------------------------------------------------- */

void hqo_repack_ref(const uint32_t* src, uint32_t* dst, uint32_t K, uint32_t N) {
    uint32_t nkq = K / 32;
    for (uint32_t kq = 0; kq < nkq; ++kq) {
        size_t base_kw = (size_t)kq * 4;
        for (uint32_t n = 0; n < N; ++n) {
            size_t d = ((size_t)kq * N + n) * 4;
            for (uint32_t j = 0; j < 4; ++j) dst[d + j] = src[(base_kw + j) * N + n];
        }
    }
}

/* One dequantised weight, exactly as the reference's host loop forms it; b is the caller's
 * fp32 bias array [K/group][N], or NULL for the reference's own bias -8 * scale. */
static inline float dq_int4b(const uint32_t* w, const uint16_t* s, const float* b, uint32_t N,
                             uint32_t group, uint32_t k, uint32_t n) {
    uint32_t q = (w[(size_t)(k / 8) * N + n] >> (4 * (k % 8))) & 0xFu;
    float scale = hqo_f16_to_f32(s[(size_t)(k / group) * N + n]);
    float bias = b ? b[(size_t)(k / group) * N + n] : -8.0f * scale;
    float prod = (float)q * scale;   /* -ffp-contract=off keeps this a separate rounding */
    return prod + bias;
}
static inline float dq_int4(const uint32_t* w, const uint16_t* s, uint32_t N, uint32_t group,
                            uint32_t k, uint32_t n) {
    return dq_int4b(w, s, NULL, N, group, k, n);
}

/* Ternary: t = c - 1, w = d * t; a non-finite scale drops the group as in native_decoder.cu:174. */
static inline int dq_ternary(const uint32_t* w, const uint16_t* s, uint32_t N, uint32_t group,
                             uint32_t k, uint32_t n, float* out) {
    uint32_t c = (w[(size_t)(k / 16) * N + n] >> (2 * (k % 16))) & 3u;
    if (c == 3u) return -1;
    float d = hqo_f16_to_f32(s[(size_t)(k / group) * N + n]);
    if (isnan(d) || isinf(d)) { *out = 0.0f; return 0; }
    *out = d * (float)((int)c - 1);
    return 0;
}

void hqo_dequant_int4(const uint32_t* w, const uint16_t* s, uint32_t K, uint32_t N, uint32_t group,
                      float* wdq) {
#pragma omp parallel for schedule(static)
    for (long long k = 0; k < (long long)K; ++k)
        for (uint32_t n = 0; n < N; ++n) wdq[(size_t)k * N + n] = dq_int4(w, s, N, group, (uint32_t)k, n);
}

void hqo_dequant_int4_bias(const uint32_t* w, const uint16_t* s, const float* bias, uint32_t K, uint32_t N,
                           uint32_t group, float* wdq) {
#pragma omp parallel for schedule(static)
    for (long long k = 0; k < (long long)K; ++k)
        for (uint32_t n = 0; n < N; ++n) wdq[(size_t)k * N + n] = dq_int4b(w, s, bias, N, group, (uint32_t)k, n);
}

int hqo_dequant_ternary2(const uint32_t* w, const uint16_t* s, uint32_t K, uint32_t N, uint32_t group,
                         float* wdq) {
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(| : bad)
    for (long long k = 0; k < (long long)K; ++k)
        for (uint32_t n = 0; n < N; ++n)
            if (dq_ternary(w, s, N, group, (uint32_t)k, n, &wdq[(size_t)k * N + n])) bad = 1;
    return bad ? -1 : 0;
}

void hqo_gemm_f32(const float* X, const float* W, float* Y, uint32_t M, uint32_t K, uint32_t N,
                  int threads) {
    const uint32_t NB = 256;
    uint32_t nblk = (N + NB - 1) / NB;
    long long units = (long long)M * nblk;
    if (threads <= 0) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (long long u = 0; u < units; ++u) {
        uint32_t m = (uint32_t)(u / nblk);
        uint32_t n0 = (uint32_t)(u % nblk) * NB;
        uint32_t n1 = n0 + NB < N ? n0 + NB : N;
        float* y = Y + (size_t)m * N;
        for (uint32_t n = n0; n < n1; ++n) y[n] = 0.0f;
        for (uint32_t k = 0; k < K; ++k) {
            float xv = X[(size_t)m * K + k];
            const float* wr = W + (size_t)k * N;
            for (uint32_t n = n0; n < n1; ++n) y[n] = fmaf(xv, wr[n], y[n]);
        }
    }
}

int hqo_qgemm(const uint16_t* X, int xdtype, size_t ldx, int fmt, const uint32_t* w,
              const uint16_t* s, uint32_t M, uint32_t K, uint32_t N, uint32_t group, float* Y,
              int threads) {
    return hqo_qgemm_bias(X, xdtype, ldx, fmt, w, s, NULL, M, K, N, group, Y, threads);
}

int hqo_qgemm_bias(const uint16_t* X, int xdtype, size_t ldx, int fmt, const uint32_t* w,
                   const uint16_t* s, const float* bias, uint32_t M, uint32_t K, uint32_t N,
                   uint32_t group, float* Y, int threads) {
    const uint32_t NB = 128;
    uint32_t nblk = (N + NB - 1) / NB;
    int bad = 0;
    if (threads <= 0) threads = 1;
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K + 1);
    if (!xf) return -2;
    for (uint32_t m = 0; m < M; ++m)
        hqo_to_f32(X + (size_t)m * ldx, xdtype, xf + (size_t)m * K, K);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads) reduction(| : bad)
    for (long long b = 0; b < (long long)nblk; ++b) {
        uint32_t n0 = (uint32_t)b * NB;
        uint32_t n1 = n0 + NB < N ? n0 + NB : N;
        float wrow[128];
        for (uint32_t m = 0; m < M; ++m)
            for (uint32_t n = n0; n < n1; ++n) Y[(size_t)m * N + n] = 0.0f;
        for (uint32_t k = 0; k < K; ++k) {
            if (fmt == HQO_INT4) {
                for (uint32_t n = n0; n < n1; ++n) wrow[n - n0] = dq_int4b(w, s, bias, N, group, k, n);
            } else {
                for (uint32_t n = n0; n < n1; ++n)
                    if (dq_ternary(w, s, N, group, k, n, &wrow[n - n0])) bad = 1;
            }
            for (uint32_t m = 0; m < M; ++m) {
                float xv = xf[(size_t)m * K + k];
                float* y = Y + (size_t)m * N;
                for (uint32_t n = n0; n < n1; ++n) y[n] = fmaf(xv, wrow[n - n0], y[n]);
            }
        }
    }
    free(xf);
    return bad ? -1 : 0;
}

void hqo_fidelity(const float* a, const float* b, size_t count, double* max_abs, double* mse) {
    double mx = 0.0, sq = 0.0;
    for (size_t i = 0; i < count; ++i) {
        double d = fabs((double)a[i] - (double)b[i]);
        if (d > mx) mx = d;
        sq += d * d;
    }
    *max_abs = mx;
    *mse = count ? sq / (double)count : 0.0;
}

/* ---- GGUF TQ1_0 ---- */
uint32_t hqo_tq1_0_code(const uint8_t* block, uint32_t i) {
    const uint8_t* packed = block + 2;
    uint32_t byte_idx, digit;
    if (i < 250) {
        byte_idx = i / 5;
        digit = i % 5;
    } else {
        byte_idx = 50 + (i - 250) / 3;
        digit = (i - 250) % 3;
    }
    uint32_t val = packed[byte_idx];
    for (uint32_t s = 0; s < digit; ++s) val /= 3;
    return val % 3;
}

uint16_t hqo_tq1_0_scale(const uint8_t* block) {
    return (uint16_t)(block[0] | (block[1] << 8));
}

void hqo_gemv_tq1_0(const float* X, const uint8_t* W, float* Y, uint32_t M, uint32_t K, uint32_t N,
                    int threads) {
    const uint32_t nb = K / 256;
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; ++n) {
        for (uint32_t m = 0; m < M; ++m) {
            const float* x = X + (size_t)m * K;
            float sum = 0.0f;
            for (uint32_t b = 0; b < nb; ++b) {
                const uint8_t* blk = W + ((size_t)n * nb + b) * 56;
                const float d = hqo_f16_to_f32(hqo_tq1_0_scale(blk));
                if (!isfinite(d)) continue;
                for (uint32_t i = 0; i < 256; ++i) {
                    const float t = (float)((int)hqo_tq1_0_code(blk, i) - 1);
                    sum = fmaf(d * t, x[256 * b + i], sum);
                }
            }
            Y[(size_t)m * N + n] = sum;
        }
    }
}

/* ---- GGML Q4_K (the published block_q4_K of GGML / llama.cpp) ---- */
static void q4k_scale_min(uint32_t j, const uint8_t* q, uint32_t* d, uint32_t* m) {
    if (j < 4) {
        *d = q[j] & 63u;
        *m = q[j + 4] & 63u;
    } else {
        *d = (q[j + 4] & 0xFu) | ((uint32_t)(q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((uint32_t)(q[j - 0] >> 6) << 4);
    }
}

void hqo_dequant_q4_k(const uint8_t* blocks, uint32_t K, uint32_t N, float* w) {
    const uint32_t nb = K / 256;
#pragma omp parallel for schedule(static)
    for (long long n = 0; n < (long long)N; ++n) {
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t* x = blocks + ((size_t)n * nb + b) * 144;
            const float d = hqo_f16_to_f32((uint16_t)(x[0] | (x[1] << 8)));
            const float min = hqo_f16_to_f32((uint16_t)(x[2] | (x[3] << 8)));
            const uint8_t* sc = x + 4;
            const uint8_t* q = x + 16;
            uint32_t k = 256 * b;
            for (uint32_t j = 0; j < 256; j += 64) {
                uint32_t s1, m1, s2, m2;
                q4k_scale_min(j / 32, sc, &s1, &m1);
                q4k_scale_min(j / 32 + 1, sc, &s2, &m2);
                const float d1 = d * (float)s1, mm1 = min * (float)m1;
                const float d2 = d * (float)s2, mm2 = min * (float)m2;
                for (uint32_t l = 0; l < 32; ++l) w[(size_t)(k++) * N + n] = d1 * (float)(q[l] & 0xF) - mm1;
                for (uint32_t l = 0; l < 32; ++l) w[(size_t)(k++) * N + n] = d2 * (float)(q[l] >> 4) - mm2;
                q += 32;
            }
        }
    }
}

/* ---- the int8 path ---- */
void hqo_int8_from_int4(const uint32_t* w, uint32_t K, uint32_t N, int8_t* out) {
    for (uint32_t kw = 0; kw < K / 8; ++kw)
        for (uint32_t n = 0; n < N; ++n)
            for (uint32_t i = 0; i < 8; ++i) {
                const int q = (int)((w[(size_t)kw * N + n] >> (4 * i)) & 0xFu);
                out[(size_t)(8 * kw + i) * N + n] = (int8_t)(q * 16 - 128);
            }
}

int8_t hqo_quantize_x_int8(float x) {
    /* marlin_gemm.cu:356-359: static_cast<int8_t>(fminf(fmaxf(X * 127.0f, -128.0f), 127.0f)) */
    const float t = fminf(fmaxf(x * 127.0f, -128.0f), 127.0f);
    return (int8_t)t;
}

void hqo_gemm_int8(const float* X, size_t ldx, const int8_t* W, const float* scales, uint32_t M, uint32_t K,
                   uint32_t N, float* Y, int threads) {
    if (threads <= 0) threads = 1;
    const uint32_t nq = K / 4;
    int8_t* xq = (int8_t*)malloc((size_t)M * K + 1);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t k = 0; k < K; ++k) xq[(size_t)m * K + k] = hqo_quantize_x_int8(X[(size_t)m * ldx + k]);
#pragma omp parallel for schedule(static) num_threads(threads)
    for (long long u = 0; u < (long long)M * N; ++u) {
        const uint32_t m = (uint32_t)(u / N), n = (uint32_t)(u % N);
        const int8_t* x = xq + (size_t)m * K;
        float acc = 0.0f;
        for (uint32_t q = 0; q < nq; ++q) {
            int32_t dot = 0;
            for (uint32_t i = 0; i < 4; ++i) dot += (int32_t)x[4 * q + i] * (int32_t)W[(size_t)(4 * q + i) * N + n];
            acc = fmaf((float)dot, 1.0f / 127.0f, acc);
        }
        Y[(size_t)m * N + n] = acc * scales[n];
    }
    free(xq);
}

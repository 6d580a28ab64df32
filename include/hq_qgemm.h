/*
 * hq_qgemm.h — C ABI of the MI355X (gfx950) weight-only quantized GEMM.
 *
 * Drop-in for hydrogen's Marlin-style qGEMM path. The reference surface is the
 * C++ class hydrogen::MarlinGemmEngine (hydrogen/include/marlin_gemm.hpp:59-172,
 * hydrogen/src/model/marlin_gemm.cu:381-758); each entry point below names the
 * member it replaces. Differences from that surface, all required by the target
 * operator (fp16/bf16 activations, fp16 group scales, fp32 accumulation):
 *   - activations and outputs are fp16 or bf16 instead of fp32;
 *   - scales are fp16 [K/group][N]; the reference's per-group fp32 bias array
 *     (marlin_gemm.hpp:100-107, w = q * scale + bias, marlin_gemm.cu:195-196, 506) is an
 *     optional argument: NULL means the zero point 8 of the reference's own data
 *     (bias = -8 * scale, marlin_gemm.cu:486-487);
 *   - M is given per call and may be any value >= 1 (the reference's buffers fix a
 *     maximum M and its kernels are only valid for M <= 8, marlin_gemm.cu:260);
 *   - every call takes an explicit stream and returns a status instead of throwing
 *     (the reference throws std::runtime_error from CUDA_CHECK, marlin_gemm.cu:19-27).
 *
 * Conventions. All pointers passed to hq_gemm_* and *_device calls are device
 * pointers; hq_repack_* / hq_unpack_* without _device are host-to-host. The caller
 * owns every buffer. Calls are thread-safe; a call returns after enqueueing its
 * kernels on `stream` (a hipStream_t; NULL is the null stream). On error nothing is
 * enqueued, the status is returned, and hq_last_error() describes it (per thread).
 */
#ifndef HQ_QGEMM_H
#define HQ_QGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HQ_ABI_VERSION 2

/* The enums are int-sized. C++ gives them int as their underlying type, so that any value a C
 * caller passes (including invalid ones, which are rejected) is a valid enum value there. */
#ifdef __cplusplus
#define HQ_ENUM(name) enum name : int
#else
#define HQ_ENUM(name) enum name
#endif

typedef HQ_ENUM(hq_status) {
    HQ_OK = 0,
    HQ_ERR_INVALID_ARG = 1,  /* null pointer, bad enum */
    HQ_ERR_SHAPE = 2,        /* M, K, N, group or leading dimensions not supported */
    HQ_ERR_ALIGNMENT = 3,    /* a pointer or leading dimension breaks the alignment rules */
    HQ_ERR_UNSUPPORTED = 4,  /* valid request this build does not implement */
    HQ_ERR_WORKSPACE = 5,    /* workspace missing or smaller than hq_workspace_bytes() */
    HQ_ERR_BAD_CODE = 6,     /* ternary code 3 met while repacking */
    HQ_ERR_DEVICE = 7,       /* HIP runtime error */
    HQ_ERR_INTERNAL = 8,
    HQ_ERR_FORMAT = 9,       /* malformed or unsupported GGUF data */
    HQ_ERR_NOT_FOUND = 10,   /* no such GGUF tensor or metadata key */
    HQ_ERR_IO = 11           /* a file could not be opened or mapped */
} hq_status;

typedef HQ_ENUM(hq_dtype) { HQ_DTYPE_F16 = 1, HQ_DTYPE_BF16 = 2 } hq_dtype;

typedef HQ_ENUM(hq_format) {
    HQ_FORMAT_INT4 = 1,      /* u32 [K/8][N], nibble i of word (kw, n) is k = 8*kw + i, code q in
                                0..15, weight (q - 8) * scale (marlin_gemm.cu:495-512) */
    HQ_FORMAT_TERNARY2 = 2   /* u32 [K/16][N], bits 2i..2i+1 of word (kw, n) hold c = t + 1 for
                                k = 16*kw + i, t in {-1, 0, +1}, weight t * scale; c = 3 is invalid
                                (value semantics of native_decoder.cu:81-102, 184-186) */
} hq_format;

typedef void* hq_stream; /* hipStream_t */

/* One projection of a fused call: its own packed weight, scales, optional bias, width and
 * output. */
typedef struct hq_segment {
    const uint32_t* Wp;     /* packed (hq_repack_*) weight, device */
    const uint16_t* scales; /* fp16 [K/group][N], device */
    const float* bias;      /* int4 only: fp32 [K/group][N] per-group bias (weight q * scale + bias),
                               device, 4-byte aligned; NULL: zero point 8 (weight (q - 8) * scale) */
    void* Y;                /* [M][ldy] output in the activation dtype, device */
    int64_t ldy;            /* elements, >= N */
    uint32_t N;
} hq_segment;

#define HQ_MAX_SEGMENTS 8

/* ---- support ---- */
const char* hq_version(void);
/* Description of the last failure on the calling thread ("" if none). */
const char* hq_last_error(void);
const char* hq_status_string(hq_status s);

/* Words of the reference linear layout: (K/8)*N for int4, (K/16)*N for ternary. */
size_t hq_linear_words(hq_format fmt, uint32_t K, uint32_t N);
/* Words of the gfx950 tile layout (N padded up to a multiple of 16). 0 on a bad shape. */
size_t hq_packed_words(hq_format fmt, uint32_t K, uint32_t N);
/* Device workspace a GEMM call of this shape needs on the current device (0: none).
 * Calls whose work is split across workgroups along K need one (decode shapes with few
 * column tiles, prefill calls with few output tiles): a 256-byte aligned buffer,
 * zero-filled by the caller before its first use (every call leaves it zero-filled
 * again). Calls sharing one workspace must not overlap in time (same stream, or ordered
 * by events), and a workspace shared by calls of several shapes needs the largest of their
 * sizes. The value is exactly what a one-projection call of this shape needs, with or
 * without a bias; for a fused call use hq_workspace_bytes_fused, which plans the call's own
 * segment list. Shapes whose operands would span 2 GiB or more (M * K * 2 bytes of X, the
 * scales, the packed weights) are rejected with HQ_ERR_SHAPE, as the GEMM calls reject them,
 * since the kernels address each operand with 32-bit offsets. Passing NULL instead
 * makes the library use a buffer of its own per (device, stream), allocated on first need
 * outside stream capture; a call that would need to allocate it during capture fails with
 * HQ_ERR_WORKSPACE. The reference has no workspace: it allocates inside
 * MarlinGemmEngine (marlin_gemm.cu:381-416). */
hq_status hq_workspace_bytes(hq_format fmt, uint32_t M, uint32_t K, uint32_t N, uint32_t group,
                             size_t* bytes);
/* The workspace of one hq_gemm_fused call: Ns[0..nseg) are its segments' widths, with_bias
 * whether any segment has a bias. Exactly what that call asks for (the same planning). */
hq_status hq_workspace_bytes_fused(hq_format fmt, uint32_t M, uint32_t K, uint32_t group,
                                   const uint32_t* Ns, uint32_t nseg, int with_bias, size_t* bytes);
/* The plan a GEMM call of this shape runs on the current device, as text: kernel, tiling and
 * grid (for benchmarks and tests; no counterpart in the reference). Writes at most buf_len
 * bytes including the terminating zero. */
hq_status hq_describe_gemm(hq_format fmt, hq_dtype dtype, uint32_t M, uint32_t K, uint32_t N,
                           uint32_t group, int with_bias, char* buf, size_t buf_len);
/* Faults that kernels report after their launch returned: a bounded wait inside a kernel
 * (the lockstep decode kernel's k-group barrier, the barrier of a prefill tile's two K
 * halves) that gave up sets a host-visible fault
 * word, and that launch's outputs are wrong. This call waits for `stream`, then returns
 * HQ_ERR_DEVICE (and clears the word) if one was reported since the last check, HQ_OK
 * otherwise. Every hq_gemm_* call also checks the word first and fails with HQ_ERR_DEVICE
 * if it is set. The reference has no such waits (it reports launch errors only,
 * marlin_gemm.cu:600). */
hq_status hq_device_status(hq_stream stream);

/* ---- repack: replaces MarlinGemmEngine::repack_q4k_to_marlin (marlin_gemm.hpp:78-83) ---- */

/* The reference's own "Marlin" layout, bit-exact with marlin_gemm.cu:446-455:
 * dst[(kq*N + n)*4 + j] = src[(4*kq + j)*N + n], kq < K/32. Host to host, K % 32 == 0. */
hq_status hq_repack_int4_ref(const uint32_t* src_linear, uint32_t* dst, uint32_t K, uint32_t N);

/* Linear -> gfx950 tile layout (hq_packed_words words), host to host. K % 128 == 0. */
hq_status hq_repack_int4(const uint32_t* src_linear, uint32_t* dst_packed, uint32_t K, uint32_t N);
hq_status hq_repack_ternary2(const uint32_t* src_linear, uint32_t* dst_packed, uint32_t K, uint32_t N);
/* Inverse of the above (padding columns dropped), host to host. */
hq_status hq_unpack_int4(const uint32_t* packed, uint32_t* dst_linear, uint32_t K, uint32_t N);
hq_status hq_unpack_ternary2(const uint32_t* packed, uint32_t* dst_linear, uint32_t K, uint32_t N);

/* Same repacks on the device (one kernel, enqueued on `stream`). For ternary,
 * d_bad_flag (a device uint32, may be NULL) is set to 1 if a code 3 was met; the
 * caller zeroes it first and reads it after the stream completes. */
hq_status hq_repack_int4_device(const uint32_t* d_src_linear, uint32_t* d_dst_packed, uint32_t K,
                                uint32_t N, hq_stream stream);
hq_status hq_repack_ternary2_device(const uint32_t* d_src_linear, uint32_t* d_dst_packed, uint32_t K,
                                    uint32_t N, uint32_t* d_bad_flag, hq_stream stream);

/* ---- GGUF TQ1_0 import: the reference's ternary weight blocks (BlockTQ1_0,
 *      native_decoder.cu:31-36), read today by kernel_gemv_tq1_0 (native_decoder.cu:155-206) ----
 * A TQ1_0 tensor of N output rows and K inputs is N rows of K/256 blocks of 56 bytes
 * ([out][in/256], native_decoder.cu:167): fp16 d, 52 bytes of base-3 trits, 2 padding bytes.
 * Element i of a block is w = d * t_i, t_i in {-1, 0, 1}: digit i % 5 of trit byte i / 5 for
 * i < 250, digit (i - 250) % 3 of trit byte 50 + (i - 250) / 3 after (native_decoder.cu:87-101;
 * any byte value decodes digit by digit). The import is lossless: codes c = t + 1 and d are
 * kept as they are, one scale per 256 inputs, so an imported weight is used with group = 256.
 * A non-finite d is kept; the GEMM then drops its block, as kernel_gemv_tq1_0 skips it
 * (native_decoder.cu:174). K % 256 == 0. */
/* Bytes of such a tensor (0 on a bad shape). */
size_t hq_tq1_0_bytes(uint32_t K, uint32_t N);
/* Host to host: blocks -> ternary linear codes u32 [K/16][N] (the hq_repack_ternary2 input)
 * and fp16 scales [K/256][N]. */
hq_status hq_convert_tq1_0(const void* blocks, uint32_t K, uint32_t N, uint32_t* codes_linear,
                           uint16_t* scales);
/* On the device, one kernel on `stream`: blocks (8-byte aligned) -> the gfx950 ternary tile
 * layout (hq_packed_words(HQ_FORMAT_TERNARY2, K, N) words) and fp16 scales [K/256][N]; the
 * same words as hq_convert_tq1_0 followed by hq_repack_ternary2. */
hq_status hq_repack_tq1_0_device(const void* d_blocks, uint32_t K, uint32_t N, uint32_t* d_packed,
                                 uint16_t* d_scales, hq_stream stream);

/* ---- GGUF container: replaces hydrogen::ModelLoader / parse_gguf (tensor_loader.hpp:14-53,
 *      gguf_parser.hpp:33-145, tensor_loader.cpp) for the weights of this path ----
 * The parse follows the reference's rules: magic "GGUF", versions 2 and 3, 64-bit counts,
 * every metadata value type (arrays of any element type, nested), at most 4 tensor
 * dimensions, tensor data starting at the header's end rounded up to general.alignment
 * (default 32; 0 reads as 32), a tensor's byte size from its element count and its type's
 * block traits (gguf_parser.hpp:108-139; unlisted types one byte per element), and a null data
 * pointer for a tensor that extends past the end of the data. Malformed data gives
 * HQ_ERR_FORMAT (the reference throws std::runtime_error). A weight matrix is a 2-D tensor
 * with shape[0] = K (inputs, the contiguous dimension) and shape[1] = N (output rows), its
 * blocks stored row by row ([N][K/256] for the 256-weight block types). */
typedef struct hq_gguf hq_gguf; /* an open GGUF file or buffer */
typedef struct hq_gguf_header_info {
    uint32_t version;
    uint64_t tensor_count, kv_count;
    uint64_t alignment;            /* general.alignment, or 32 */
    uint64_t header_bytes;         /* end of the tensor directory */
    uint64_t tensor_data_offset;   /* start of the tensor data (aligned) */
    uint64_t total_tensor_bytes;   /* largest offset + size over the tensors */
    uint64_t file_bytes;
} hq_gguf_header_info;
typedef struct hq_gguf_tensor_info {
    const char* name;              /* valid until hq_gguf_close */
    uint32_t n_dims;
    uint64_t shape[4];
    uint32_t type;                 /* GGML type: 0 F32, 1 F16, 12 Q4_K, 34 / 143 TQ1_0, ... */
    uint64_t offset;               /* relative to the tensor data */
    uint64_t absolute_offset;
    uint64_t size_bytes;
    const void* data;              /* host address in the mapping, NULL past the end of the data */
} hq_gguf_tensor_info;
/* Memory-maps a file read-only and parses it (ModelLoader::load). */
hq_status hq_gguf_open(const char* path, hq_gguf** out);
/* Parses GGUF bytes the caller keeps alive until hq_gguf_close (parse_gguf). */
hq_status hq_gguf_parse(const void* data, size_t bytes, hq_gguf** out);
void hq_gguf_close(hq_gguf* g);
hq_status hq_gguf_header(const hq_gguf* g, hq_gguf_header_info* out);
hq_status hq_gguf_tensor_at(const hq_gguf* g, uint64_t index, hq_gguf_tensor_info* out);
/* GGUFModel::find_tensor; HQ_ERR_NOT_FOUND if absent (the last tensor of a repeated name wins). */
hq_status hq_gguf_find_tensor(const hq_gguf* g, const char* name, hq_gguf_tensor_info* out);
/* Typed metadata (GGUFValue::as_*): integers and bools, floats, strings (len gets the length;
 * buf receives at most buf_len - 1 bytes and a zero), arrays (element type and count). */
hq_status hq_gguf_get_int(const hq_gguf* g, const char* key, int64_t* out);
hq_status hq_gguf_get_float(const hq_gguf* g, const char* key, double* out);
hq_status hq_gguf_get_string(const hq_gguf* g, const char* key, char* buf, size_t buf_len, size_t* len);
hq_status hq_gguf_get_array(const hq_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count);
/* A TQ1_0 weight (type 34 or 143, the reference's 56-byte BlockTQ1_0) onto the device: its
 * blocks are copied into d_staging (>= size_bytes, device) and repacked there by
 * hq_repack_tq1_0_device into d_packed (hq_packed_words(HQ_FORMAT_TERNARY2, K, N) words) and
 * d_scales (fp16 [K/256][N]); *K, *N receive the shape. Enqueued on `stream`; keep g open until
 * the stream has passed the copy. The reference instead uploads the whole tensor section and
 * decodes the blocks at every token (native_decoder.cu:849-857, 155-206). */
hq_status hq_gguf_load_tq1_0(const hq_gguf* g, const char* name, void* d_staging, size_t staging_bytes,
                             uint32_t* d_packed, uint16_t* d_scales, uint32_t* K, uint32_t* N,
                             hq_stream stream);
/* GGML Q4_K blocks (144 bytes per 256 weights: fp16 d and dmin, 12 bytes of 6-bit sub-block
 * scales and mins, 128 bytes of 4-bit codes; weight = d * sc_j * q - dmin * m_j per 32-weight
 * sub-block j) -> int4 linear codes u32 [K/8][N] (the hq_repack_int4 input), fp16 scales
 * [K/32][N] (d * sc_j, rounded to fp16) and fp32 biases [K/32][N] (-dmin * m_j): use them with
 * hq_gemm_w4a16(..., bias, ..., group = 32). Host to host, K % 256 == 0. The layout is GGML's
 * published block_q4_K (the reference names the type, gguf_parser.hpp:44, 130, but has no
 * decoder for it). */
hq_status hq_convert_q4_k(const void* blocks, uint32_t K, uint32_t N, uint32_t* codes_linear,
                          uint16_t* scales, float* bias);
/* The same for a Q4_K tensor of an open GGUF (type 12, shape [K, N]). */
hq_status hq_gguf_convert_q4_k(const hq_gguf* g, const char* name, uint32_t* codes_linear,
                               uint16_t* scales, float* bias, uint32_t* K, uint32_t* N);

/* ---- forward: replaces MarlinGemmEngine::forward_marlin_int4 (marlin_gemm.hpp:100-107,
 *      marlin_gemm.cu:556-601) ----
 * Y[m, n] = sum_k X[m, k] * w(k, n), fp32 accumulation, Y rounded to the activation dtype.
 * X: [M][ldx] fp16/bf16, 16-byte aligned, ldx % 8 == 0, ldx >= K.
 * Wp: gfx950 packed weight, 16-byte aligned. scales: fp16 [K/group][N].
 * bias (int4): NULL, or fp32 [K/group][N], 4-byte aligned: w = q * scale + bias as in the
 *   reference (marlin_gemm.cu:195-196); NULL gives w = (q - 8) * scale.
 * Y: [M][ldy], 2-byte aligned, ldy >= N; written in full (no zero-fill needed).
 * K % 128 == 0, group % 32 == 0, K % group == 0, M >= 1, N >= 1 (the reference takes a
 *   group per 32-wide k chunk, marlin_gemm.cu:191-193). Groups that are multiples of 128
 *   without a bias run the fastest kernels; other groups and biased calls run kernels that
 *   apply one scale (and bias) per 32-wide k chunk.
 * workspace / workspace_bytes: see hq_workspace_bytes (NULL, 0 is always accepted).
 * Every operand must span less than 2 GiB (M * ldx * 2 bytes of X, M * ldy * 2 of Y, the
 *   scales, the bias, the packed weights; the kernels address them with 32-bit offsets):
 *   larger calls fail with HQ_ERR_SHAPE before any device work. (The reference drops a K
 *   tail silently, marlin_gemm.cu:156-159; this library never returns wrong results.)
 * Up to M = 80 (decode steps, split-fuse steps of decode tokens and a prefill chunk) the
 * HBM-streaming kernels run; larger M the MFMA tile kernel.
 * Results are deterministic: repeated calls with the same shapes give identical bits. */
hq_status hq_gemm_w4a16(const void* X, hq_dtype dtype, int64_t ldx, const uint32_t* Wp,
                        const uint16_t* scales, const float* bias, void* Y, int64_t ldy, uint32_t M,
                        uint32_t K, uint32_t N, uint32_t group, void* workspace, size_t workspace_bytes,
                        hq_stream stream);
/* Ternary weights (value semantics of kernel_gemv_tq1_0, native_decoder.cu:155-206): the same
 * contract without a bias; a group whose scale is not finite contributes nothing. */
hq_status hq_gemm_w2a16(const void* X, hq_dtype dtype, int64_t ldx, const uint32_t* Wp,
                        const uint16_t* scales, void* Y, int64_t ldy, uint32_t M, uint32_t K,
                        uint32_t N, uint32_t group, void* workspace, size_t workspace_bytes,
                        hq_stream stream);

/* Fused projections sharing one activation read (QKV, gate||up): nseg segments of one
 * format over the same X. Each output equals the hq_gemm_* call of its segment up to fp32
 * summation order (the fused launch may split K differently). Replaces the
 * separate GEMV launches of native_decoder.cu:1113-1115, 1149-1150, 1178-1179. */
hq_status hq_gemm_fused(const void* X, hq_dtype dtype, int64_t ldx, hq_format fmt,
                        const hq_segment* segs, uint32_t nseg, uint32_t M, uint32_t K,
                        uint32_t group, void* workspace, size_t workspace_bytes, hq_stream stream);

/* hq_gemm_fused for callers that cannot allocate (code under stream capture, tight serving
 * loops, harnesses that forbid allocation). No counterpart in the reference. It allocates
 * nothing: its workspace is a static device array of HQ_NOALLOC_SCRATCH_BYTES per GPU, held
 * from the library's load until the process ends, and it never creates the fault word (a
 * fault is still reported if another call created it). Plans are chosen to fit that array
 * (fewer K splits where a call would need more), so outputs equal hq_gemm_fused's up to fp32
 * summation order; a call that cannot fit fails with HQ_ERR_WORKSPACE. Every call on one GPU
 * shares that GPU's array, which keeps the last call's contents: calls that overlap in time
 * on one GPU (different streams without ordering) race and give wrong results. */
#define HQ_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
hq_status hq_gemm_fused_noalloc(const void* X, hq_dtype dtype, int64_t ldx, hq_format fmt,
                                const hq_segment* segs, uint32_t nseg, uint32_t M, uint32_t K,
                                uint32_t group, hq_stream stream);

/* ---- The int8 path --------------------------------------------------------------------
 * Replaces MarlinGemmEngine::forward_cutlass_int8 (hydrogen/src/model/marlin_gemm.cu:603-617)
 * and kernel_cutlass_int8_gemm (:327-377), which the reference builds but never launches.
 * Same operands and semantics: fp32 activations X [M][ldx] quantised per element to
 * int8(clamp(x * 127, -128, 127)) converted toward zero; int8 weights [K][N] (the reference's
 * W_int8: q * 16 - 128 of its int4 codes, :508), repacked once into the gfx950 tile layout;
 * one fp32 scale per column (the reference reads row 0 of its scale matrix); fp32 output
 * Y[m][n] = scales[n] * (sum_k xq[m][k] * w[k][n]) / 127. The products are summed exactly in
 * int32 (the reference sums fp32 quad by quad, which differs by its own rounding only).
 * M <= 16 (the reference's kernel takes M <= 8); K a multiple of 128, at most 131072 (the int32
 * sum cannot overflow); N >= 1. */

/* Bytes of the int8 tile layout of a K x N weight (N padded to 16 columns): K * ceil(N/16) * 16;
 * 0 if K is not a positive multiple of 128 or N is 0. */
size_t hq_int8_packed_bytes(uint32_t K, uint32_t N);

/* Host repack of int8 weights w_kn [K][N] into the tile layout (hq_int8_packed_bytes(K, N)
 * bytes, padding columns zero), and its inverse. Replaces the upload of h_W_int8
 * (marlin_gemm.cu:517): the tile layout is what hq_gemm_w8a8 streams. */
hq_status hq_repack_int8(const int8_t* w_kn, uint32_t K, uint32_t N, int8_t* packed);
hq_status hq_unpack_int8(const int8_t* packed, uint32_t K, uint32_t N, int8_t* w_kn);

/* Workspace bytes of an hq_gemm_w8a8 call (the quantised activations, and the partial sums when
 * the call splits K): a NULL workspace makes the library use its own. */
hq_status hq_workspace_bytes_w8a8(uint32_t M, uint32_t K, uint32_t N, size_t* bytes);

/* The int8 GEMM on `stream`. X 16-byte aligned with ldx >= K a multiple of 4; Wp (the tile
 * layout) 16-byte aligned; scales [N] fp32; Y [M][ldy] fp32, ldy >= N. workspace: NULL or
 * hq_workspace_bytes_w8a8 bytes, 256-byte aligned. */
hq_status hq_gemm_w8a8(const float* X, int64_t ldx, const int8_t* Wp, const float* scales, float* Y, int64_t ldy,
                       uint32_t M, uint32_t K, uint32_t N, void* workspace, size_t workspace_bytes,
                       hq_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* HQ_QGEMM_H */

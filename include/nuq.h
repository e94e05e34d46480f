/*
 * nuq — MI355X (gfx950) quantized-weight matmul path for nuclis.
 *
 * C ABI of libnuq.so: the drop-in for nuclis's Metal matmul backend
 * (inference/src/backends/metal/). The Zig engine keeps its `Backend`
 * entry points and its GGUF block layouts; it binds these functions with
 * @cImport instead of the nu_metal_* bridge (backends/metal/root.zig:29-44,
 * bridge.m). Weights are raw GGUF rows, read as-is from device memory and
 * never repacked: Q8_0 (encoding 8, 34-byte blocks of 32), Q4_K (12, 144-byte
 * blocks of 256), Q5_K (13, 176-byte blocks of 256), Q6_K (14, 210-byte blocks
 * of 256) and IQ4_XS (23, 136-byte blocks of 256).
 *
 * Conventions (mirroring the reference):
 *  - Every function returns 0 on success or a NUQ_* status. Validation happens
 *    before anything is launched or written (ops/matvec.zig:86-89).
 *  - Pointers to weights, activations and outputs are DEVICE pointers owned by
 *    the caller. Work is enqueued on the context's stream in order; nuq_sync
 *    blocks until it is done (the begin/dispatch/commit model of bridge.m:224-310).
 *  - A nuq_matrix mirrors `cpu.Matrix` (backends/cpu/root.zig:31-36): row r is
 *    bytes [r*stride, (r+1)*stride) with stride = byte_len / rows.
 *  - out[t][r] = sum_c W[r][c] * x[t][c]; x is [tokens][in_stride], out is
 *    [tokens][out_stride] F32 (ops/matmul.zig:51-61).
 *  - One context is used by one host thread at a time.
 */
#ifndef NUQ_H
#define NUQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The Zig error each maps to is named beside it. */
enum nuq_status {
    NUQ_OK = 0,
    NUQ_INVALID_SHAPE = 1,            /* error.InvalidShape */
    NUQ_UNSUPPORTED_ENCODING = 2,     /* error.UnsupportedTensorEncoding */
    NUQ_INVALID_ROW_LENGTH = 3,       /* error.InvalidRowLength */
    NUQ_INVALID_BYTE_LENGTH = 4,      /* error.InvalidByteLength */
    NUQ_NON_FINITE = 5,               /* error.NonFiniteResult (argmax) */
    NUQ_DEVICE_ERROR = 6,             /* error.MetalExecutionFailed */
    NUQ_INVALID_ARGUMENT = 7          /* null context or pointer */
};

/* GGML encoding ids (inference/src/tensor/encoding.zig:29-41). */
enum nuq_encoding { NUQ_Q8_0 = 8, NUQ_Q4_K = 12, NUQ_Q5_K = 13, NUQ_Q6_K = 14, NUQ_IQ4_XS = 23 };

/* Activation element type of nuq_matmul. The reference passes F32
 * (ops/matmul.zig:79); F16 activations are accepted as they are. */
enum nuq_dtype { NUQ_F32 = 0, NUQ_F16 = 1 };

/* Kernels nuq_matmul_kernel may force (measurement aid). */
enum nuq_kernel {
    NUQ_KERNEL_AUTO = 0,      /* the routing nuq_matmul uses */
    NUQ_KERNEL_ROWS = 1,      /* register-dequant multi-token GEMV (tokens <= 8) */
    NUQ_KERNEL_TILE = 2,      /* LDS-dequant f16 MFMA tile */
    NUQ_KERNEL_GENERIC = 3    /* one-row-per-wave F32 control, any alignment */
};

/* Pair epilogues of nuq_matvec_segments (ops/matvec.zig:224). */
enum nuq_segment_mode { NUQ_SEGMENT_PLAIN = 0, NUQ_SEGMENT_SILU_MUL_PAIR = 1 };

typedef struct nuq_context nuq_context;

/* cpu.Matrix (backends/cpu/root.zig:31-36); `bytes` is a device pointer. */
typedef struct nuq_matrix {
    uint32_t encoding;
    uint32_t reserved;
    uint64_t rows;
    uint64_t columns;
    const void *bytes;
    uint64_t byte_len;
} nuq_matrix;

/* One projection of nuq_matvec_segments (ops/matvec.zig:223, Segment). */
typedef struct nuq_segment {
    nuq_matrix matrix;
    float *output;
} nuq_segment;

/* Replaces nu_metal_create (bridge.m:74-96): opens `device`. On failure it
 * returns NULL and writes a message into err[0..cap). */
nuq_context *nuq_create(int device, char *err, size_t cap);
/* Replaces the backend's deinit. */
void nuq_destroy(nuq_context *ctx);
/* Work is enqueued on `stream` (a hipStream_t; NULL = the null stream).
 * When the stream changes, the new stream first waits for the work already
 * enqueued on the old one (the context's workspace is shared by its calls),
 * unless either stream is capturing a graph. The previous stream must still
 * be alive when this is called (an event is recorded on it). */
int nuq_set_stream(nuq_context *ctx, void *stream);
/* The context's device workspace (verify K-range partials, prefill split
 * partials, the SiLU pair's second GEMV) is allocated on the first call that
 * wants it and grown as needed; nuq_create allocates none. A call that would
 * grow it while a graph capture is active takes its no-workspace route
 * instead (same products). A workspace that a captured call used is never
 * freed on growth: it stays allocated until nuq_destroy, so graphs captured
 * earlier keep replaying into valid memory (they must not replay after
 * nuq_destroy). Callers that capture graphs may reserve it beforehand, so it
 * never grows after a capture. No counterpart in the reference (Metal buffers are created per
 * use, backends/metal/root.zig:62-86). */
int nuq_reserve_workspace(nuq_context *ctx, uint64_t bytes);
/* Bytes of workspace the context currently holds. */
uint64_t nuq_workspace_bytes(const nuq_context *ctx);
/* Replaces nu_metal_commit's wait (bridge.m:279-310): blocks until all work
 * enqueued on the context's stream has completed; reports device errors. */
int nuq_sync(nuq_context *ctx);
/* Text of the last failure on this context ("" if none). */
const char *nuq_last_error(const nuq_context *ctx);
/* When nonzero, every product runs the one-row-per-wave F32 control kernel
 * (Backend.generic_only, backends/metal/root.zig:99-102). */
int nuq_set_generic_only(nuq_context *ctx, int enabled);

/* decode.validateRow (quant/decode.zig:108-120); host only, no device work. */
int nuq_validate_row(uint32_t encoding, uint64_t byte_count, uint64_t element_count);

/* Backend.embed (ops/rowwise.zig:17-25): decode row `token` to F32,
 * bit-exact with the CPU decoder (quant/decode.zig:30). */
int nuq_embed(nuq_context *ctx, const nuq_matrix *m, uint32_t token, float *out);
/* Bulk form of embed: rows [first, first+count) to out[count][columns]. */
int nuq_dequant_range(nuq_context *ctx, const nuq_matrix *m, uint64_t first, uint64_t count, float *out);

/* Backend.matvec (ops/matvec.zig:32-34, 85-116): out[r] = sum_c W[r,c] x[c],
 * x and out F32. The decode GEMV. */
int nuq_matvec(nuq_context *ctx, const nuq_matrix *m, const float *x, float *out);

/* Backend.matvecRows (ops/matvec.zig:149-188): 2 <= tokens <= 8 activation
 * rows, F32 precision. Q4_K / Q5_K serve at most 4 token rows per pass over
 * the weights (5..8 rows: two passes); the other encodings decode each
 * weight once and dot it with every token row. */
int nuq_matvec_rows(nuq_context *ctx, const nuq_matrix *m, const float *x, uint64_t in_stride, float *out,
                    uint64_t out_stride, uint32_t tokens);

/* Backend.matmul (ops/matmul.zig:62-108): any token count; x is F32 or F16
 * ([tokens][in_stride] elements). Routes: tokens == 1 -> GEMV, tokens <= 3
 * -> multi-token GEMV (F16 x on Q4_K / Q5_K: the verify tile, exact in its
 * products), otherwise the f16 MFMA tile. Requires rows % 8 == 0 and
 * columns % 64 == 0 as the reference does. */
int nuq_matmul(nuq_context *ctx, const nuq_matrix *m, const void *x, uint32_t x_dtype, uint64_t in_stride, float *out,
               uint64_t out_stride, uint32_t tokens);
/* Backend.matmulKernel (ops/matmul.zig:73-75): same contract, forcing a
 * nuq_kernel (NUQ_KERNEL_ROWS needs tokens <= 8). */
int nuq_matmul_kernel(nuq_context *ctx, uint32_t kernel, const nuq_matrix *m, const void *x, uint32_t x_dtype,
                      uint64_t in_stride, float *out, uint64_t out_stride, uint32_t tokens);

/* Backend.matvecSegments (ops/matvec.zig:245-343): up to 4 projections that
 * read the same F32 input in one launch. PLAIN writes each segment's output;
 * SILU_MUL_PAIR takes exactly two segments of equal rows naming the same
 * output and writes silu(seg0) * seg1 there. */
int nuq_matvec_segments(nuq_context *ctx, const nuq_segment *segments, uint32_t count, const float *x,
                        uint32_t mode);

/* Largest SiLU pair (rows) nuq_matvec_segments_noalloc takes. */
#define NUQ_NOALLOC_MAX_PAIR_ROWS (1u << 20)
/* nuq_matvec_segments without any allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops). The SiLU pair's second GEMV goes to a
 * fixed 4 MiB scratch array in device memory, one per GPU, held until the
 * process ends, instead of the context workspace; pairs of more than
 * NUQ_NOALLOC_MAX_PAIR_ROWS rows are refused (NUQ_INVALID_SHAPE) before
 * anything is launched. Same validation, kernels and results as
 * nuq_matvec_segments otherwise. Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (other streams, other contexts of
 * the same process) race; calls in one stream are ordered. */
int nuq_matvec_segments_noalloc(nuq_context *ctx, const nuq_segment *segments, uint32_t count, const float *x,
                                uint32_t mode);

/* Greedy argmax over `count` device logits (sampling/root.zig:226-239: first
 * maximum wins; a non-finite logit gives NUQ_NON_FINITE). `index` is a host
 * pointer; the call synchronizes the context's stream. */
int nuq_argmax(nuq_context *ctx, const float *logits, uint64_t count, uint32_t *index);

/* Flat-argument forms of dequant / matvec / matmul over `rows` rows of
 * `stride` bytes at `w` (stride = the encoded row length, as cpu.Matrix
 * requires): the same validation, routing and kernels as nuq_dequant_range
 * (all rows), nuq_matvec and nuq_matmul. For callers that hold raw pointers
 * rather than a matrix descriptor (C / C++ harnesses). */
int nuq_dequant_rows(nuq_context *ctx, uint32_t encoding, const void *w, uint64_t stride, uint32_t rows,
                     uint32_t columns, float *out);
int nuq_gemv(nuq_context *ctx, uint32_t encoding, const void *w, uint64_t stride, uint32_t rows, uint32_t columns,
             const float *x, float *y);
int nuq_gemm(nuq_context *ctx, uint32_t encoding, const void *w, uint64_t stride, uint32_t rows, uint32_t columns,
             const void *x, uint32_t x_dtype, uint64_t in_stride, float *y, uint64_t out_stride, uint32_t tokens);

/* Device sampling: the partial top-k readback (Backend.topk,
 * backends/metal/ops/sampling.zig:15-57). `values` / `indices` receive the k
 * best logits by (value descending, index ascending); `sums` the
 * NUQ_TOPK_PARTIALS F32 partial sums of exp((l - max) / temperature) over
 * every logit, which the caller adds in F64 (sampling.TopK.total); `flags`
 * one word per partition, nonzero when it saw a non-finite logit. NaN never
 * enters the list. All four are device buffers (k floats, k u32,
 * NUQ_TOPK_PARTIALS floats, NUQ_TOPK_PARTIALS u32). */
enum { NUQ_TOPK_CAPACITY = 256, NUQ_TOPK_PARTIALS = 64, NUQ_TOPK_MAX_COUNT = 262144 };
typedef struct nuq_topk_buffers {
    float *values;
    uint32_t *indices;
    float *sums;
    uint32_t *flags;
} nuq_topk_buffers;
/* Backend.topk: InvalidShape unless 0 < count <= NUQ_TOPK_MAX_COUNT,
 * 0 < k <= min(NUQ_TOPK_CAPACITY, count) and the temperature is finite and
 * positive. Enqueued on the context's stream (no synchronization). */
int nuq_topk(nuq_context *ctx, const float *logits, uint64_t count, uint32_t k, float temperature,
             const nuq_topk_buffers *out);
/* Backend.penalize (ops/sampling.zig:58-71) = Sampler.penalize
 * (sampling/root.zig:375-381) in place on every logit whose id is set in
 * `history` (bit id of word id / 32; history_words >= ceil(count / 32)):
 * l / repetition for l > 0, else l * repetition, then minus presence. */
int nuq_penalize(nuq_context *ctx, float *logits, uint64_t count, const uint32_t *history, uint64_t history_words,
                 float repetition, float presence);

/* Weight preparation on the host (not part of the reference's backend):
 * quantize `rows` F32 rows of `columns` into GGUF rows in dst (host memory,
 * dst_len = rows * row bytes). Q8_0 is quant/encode.zig:17-36 exactly; the
 * reference has no K-quant or IQ4_XS quantizer (encode.zig:1-2), so Q4_K,
 * Q5_K, Q6_K and IQ4_XS use this library's own deterministic quantizers
 * producing legal blocks. */
int nuq_quantize_rows(uint32_t encoding, const float *src, uint64_t rows, uint64_t columns, void *dst,
                      uint64_t dst_len);

#ifdef __cplusplus
}
#endif
#endif

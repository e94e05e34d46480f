// C-ABI shim of libnuq.so (declared in include/nuq.h): validation with the
// reference's shape rules, routing, and launches on the context's stream.
//
// Validation mirrors, before anything is launched or written:
//   matvec       backends/metal/ops/matvec.zig:85-89
//   matvecRows   ops/matvec.zig:149-157
//   matmul       ops/matmul.zig:77-83
//   embed        ops/rowwise.zig:17-21
//   segments     ops/matvec.zig:265-311
//   validateRow  quant/decode.zig:108-120
// Routing mirrors the reference's specialised-vs-generic choice
// (ops/matvec.zig:196-219, ops/matmul.zig:114-123): the vectorised kernels
// need 16-byte aligned Q4_K rows (pointer and stride), even Q6_K / Q8_0 rows
// and a 16-byte aligned input; anything else runs the generic control.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/nuq.h"
#include "../../include/nuq_gguf.h"
#include "gguf_doc.h"
#include "formats.h"
#include "kernels.h"

struct nuq_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool generic_only = false;
    std::string last_error;
    uint32_t *argmax_buf = nullptr;  // device: {index, nonfinite flag}
    // F32 workspace of the verify K ranges, the prefill split partials and
    // the SiLU pair's second GEMV: allocated on the first call that wants it
    // and grown in whole 256 x 256 tiles (ensure_workspace)
    nuq::SplitScratch split{nullptr, 0};
    // The current workspace was handed to a launch recorded into a graph:
    // on growth it is kept (the graph may replay) rather than freed.
    bool split_captured = false;
    std::vector<float *> retired;  // such earlier workspaces, freed by nuq_destroy
    uint64_t *topk_keys = nullptr;  // partial top-k keys between passes
    hipEvent_t handoff = nullptr;   // orders work across a stream change
    float *static_scratch = nullptr;  // this device's copy of `scratch` (below)
};

// Scratch of the allocation-free entry point (nuq_matvec_segments_noalloc):
// the SiLU pair's second GEMV output. One copy per GPU, alive until the
// process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (nuq_create keeps it in
// the context), never through the array's name.
constexpr uint64_t NOALLOC_SCRATCH_FLOATS = NUQ_NOALLOC_MAX_PAIR_ROWS;  // 4 MiB
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_FLOATS];

namespace {

int fail(nuq_context *ctx, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(nuq_context *ctx, int code, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->last_error = buf;
    }
    return code;
}

int hip_check(nuq_context *ctx, hipError_t e, const char *what) {
    if (e == hipSuccess) return NUQ_OK;
    return fail(ctx, NUQ_DEVICE_ERROR, "%s: %s", what, hipGetErrorString(e));
}

// Whether work enqueued now on `stream` would be recorded into a graph, or
// a device-wide call now could disturb a capture: the context's stream is
// capturing, or a query fails (the legacy stream reports an implicit
// capture error while another stream captures in global mode).
bool capture_active(hipStream_t stream) {
    hipStreamCaptureStatus a = hipStreamCaptureStatusNone, b = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &a) != hipSuccess || a != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return true;
    }
    if (stream != nullptr && (hipStreamIsCapturing(nullptr, &b) != hipSuccess || b != hipStreamCaptureStatusNone)) {
        (void)hipGetLastError();
        return true;
    }
    return false;
}

// Grows the context workspace to at least `floats` F32 values (whole 256 x
// 256 tiles). Returns false, leaving it as it was, when the allocation fails
// or a graph capture is active (an allocation cannot be captured): the
// caller's route then takes its no-workspace form, or fewer splits of the
// workspace it has, which compute the same products. A call made while its
// stream captures marks the current workspace as captured; growing later
// then keeps that buffer alive until nuq_destroy (a graph replay writes to
// it), and otherwise frees it once the context's stream has finished with
// it (a stream change orders the new stream after the old, so that wait
// covers every call of the context).
bool ensure_workspace(nuq_context *ctx, uint64_t floats) {
    constexpr uint64_t TILE = 256 * 256;
    if (floats == 0) return true;
    const uint64_t tiles = (floats + TILE - 1) / TILE;
    if (capture_active(ctx->stream)) {
        if (ctx->split.work) ctx->split_captured = true;
        return tiles <= ctx->split.tiles;
    }
    if (tiles <= ctx->split.tiles) return true;
    if (tiles > 0xffffffffull) return false;
    float *p = nullptr;
    if (hipMalloc((void **)&p, tiles * TILE * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (ctx->split.work) {
        if (ctx->split_captured) {
            ctx->retired.push_back(ctx->split.work);
        } else {
            (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(ctx->split.work);
        }
    }
    ctx->split.work = p;
    ctx->split.tiles = (uint32_t)tiles;
    ctx->split_captured = false;
    return true;
}

int validate_row(uint32_t encoding, uint64_t byte_count, uint64_t element_count) {
    nuq::Layout l;
    if (!nuq::layout_of(encoding, &l)) return NUQ_UNSUPPORTED_ENCODING;
    if (element_count == 0 || element_count % l.elements != 0) return NUQ_INVALID_ROW_LENGTH;
    if (byte_count % l.bytes != 0 || byte_count / l.bytes != element_count / l.elements) return NUQ_INVALID_BYTE_LENGTH;
    return NUQ_OK;
}

const char *status_name(int code) {
    switch (code) {
    case NUQ_INVALID_SHAPE: return "InvalidShape";
    case NUQ_UNSUPPORTED_ENCODING: return "UnsupportedTensorEncoding";
    case NUQ_INVALID_ROW_LENGTH: return "InvalidRowLength";
    case NUQ_INVALID_BYTE_LENGTH: return "InvalidByteLength";
    default: return "error";
    }
}

// Shared matrix checks: descriptor present, rows and bytes consistent, whole
// blocks per row. Returns the row stride in *stride.
int check_matrix(nuq_context *ctx, const nuq_matrix *m, uint64_t *stride) {
    if (!m) return fail(ctx, NUQ_INVALID_ARGUMENT, "null matrix");
    if (m->rows == 0 || m->columns == 0) return fail(ctx, NUQ_INVALID_SHAPE, "empty matrix");
    if (m->byte_len % m->rows != 0) return fail(ctx, NUQ_INVALID_SHAPE, "byte length not a whole number of rows");
    *stride = m->byte_len / m->rows;
    int e = validate_row(m->encoding, *stride, m->columns);
    if (e) return fail(ctx, e, "%s: encoding %u, %llu bytes per row, %llu columns", status_name(e), m->encoding,
                       (unsigned long long)*stride, (unsigned long long)m->columns);
    if (!m->bytes) return fail(ctx, NUQ_INVALID_ARGUMENT, "null weights");
    if (m->rows > 0x7fffffffull || m->columns > 0x7fffffffull)
        return fail(ctx, NUQ_INVALID_SHAPE, "matrix dimensions exceed 2^31");
    return NUQ_OK;
}

// Whether the vectorised kernels may read this weight range and input
// (the reference's blockAligned plus its float4 input rule).
bool vector_aligned(const nuq_matrix *m, uint64_t stride, const void *x) {
    // ops/matmul.zig:114-123: Q4_K/Q5_K 16, IQ4_XS 8, Q6_K/Q8_0 2
    uintptr_t wp = (uintptr_t)m->bytes;
    uint64_t need = (m->encoding == NUQ_Q4_K || m->encoding == NUQ_Q5_K) ? 16 : m->encoding == NUQ_IQ4_XS ? 8 : 2;
    return wp % need == 0 && stride % need == 0 && ((uintptr_t)x % 16) == 0;
}

// Encodings with specialised multi-token GEMV kernels; the M=1 GEMV and the
// MFMA tiles take every supported encoding. The others run the generic
// decode-and-multiply kernels.
bool specialised(uint32_t encoding) {
    return encoding == NUQ_Q8_0 || encoding == NUQ_Q4_K || encoding == NUQ_Q6_K;
}

// Rows per wave of the M=1 GEMV: the number of rows a wave keeps in flight
// against one register copy of its x slice.
int gemv_rows_per_wave(uint32_t encoding, uint64_t rows) {
    if (encoding == NUQ_Q6_K) return rows >= 65536 ? 4 : 2;
    if (encoding == NUQ_Q8_0) return 2;
    return rows >= 8192 ? 4 : 2;
}

// The decode GEMV: every encoding on the integer-dot DMA kernel where its
// shape fits (Q8_0 needs K % 256 == 0), else the register kernel (Q4_K), the
// row-per-wave kernels (Q6_K, Q8_0) or the generic kernel (Q5_K, IQ4_XS).
int run_gemv(nuq_context *ctx, const nuq_matrix *m, uint64_t stride, const float *x, float *out) {
    if (m->encoding == NUQ_Q6_K || m->encoding == NUQ_Q8_0) {
        hipError_t e = nuq::launch_gemv_dma(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride,
                                            (uint32_t)m->rows, (uint32_t)m->columns, x, out);
        if (e != hipErrorInvalidValue) return hip_check(ctx, e, "gemv launch");
    }
    if (m->encoding == NUQ_Q5_K || m->encoding == NUQ_IQ4_XS) {
        hipError_t e = nuq::launch_gemv_dma(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride,
                                            (uint32_t)m->rows, (uint32_t)m->columns, x, out);
        if (e != hipErrorInvalidValue) return hip_check(ctx, e, "gemv launch");
        return hip_check(ctx,
                         nuq::launch_generic(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride,
                                             (uint32_t)m->rows, (uint32_t)m->columns, x, 0, m->columns, out, m->rows,
                                             1),
                         "generic kernel launch");
    }
    if (m->encoding == NUQ_Q4_K) {
        const int config = 0;  // DMA kernel, two ring slots; register kernel when LDS is short
        hipError_t e = nuq::launch_gemv_q4k_int(ctx->stream, (const uint8_t *)m->bytes, stride, (uint32_t)m->rows,
                                                (uint32_t)m->columns, x, out, config);
        if (e != hipErrorInvalidValue) return hip_check(ctx, e, "q4_k gemv launch");
    }
    return hip_check(ctx,
                     nuq::launch_gemv(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride, (uint32_t)m->rows,
                                      (uint32_t)m->columns, x, out, gemv_rows_per_wave(m->encoding, m->rows)),
                     "gemv launch");
}

// F32 activations of 2..8 tokens at F32 precision on the matrix cores
// (Q4_K / Q5_K); returns -1 when the shape is not one it takes (nothing is
// launched then). One launch serves at most 4 tokens, so 5..8 tokens run as
// two launches (5 = 4 + 1, ..., 8 = 4 + 4): each token's row sums do not
// depend on the others, and every launch streams the weights once.
int run_rows_mfma(nuq_context *ctx, const nuq_matrix *m, uint64_t stride, const float *x, uint64_t in_stride,
                  float *out, uint64_t out_stride, uint32_t tokens) {
    if (tokens < 2 || tokens > 8 || (m->encoding != NUQ_Q4_K && m->encoding != NUQ_Q5_K)) return -1;
    (void)ensure_workspace(ctx, nuq::tile_workspace_floats(m->encoding, (uint32_t)m->rows, (uint32_t)m->columns,
                                                           std::min(tokens, 4u), in_stride, true));
    for (uint32_t t0 = 0; t0 < tokens;) {
        const uint32_t c = std::min(tokens - t0, 4u);
        bool taken = false;
        const hipError_t e = nuq::launch_rows_mfma(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride,
                                                   (uint32_t)m->rows, (uint32_t)m->columns, x + t0 * in_stride,
                                                   in_stride, out + t0 * out_stride, out_stride, c, ctx->split, &taken);
        // a shape the form does not take is refused by the first launch,
        // before anything runs (later launches have the same or fewer tokens)
        if (!taken && t0 == 0) return -1;
        if (!taken) return fail(ctx, NUQ_DEVICE_ERROR, "multi-token gemv: a later pass of %u tokens was refused", c);
        const int r = hip_check(ctx, e, "multi-token gemv launch");
        if (r) return r;
        t0 += c;
    }
    return NUQ_OK;
}

int run_generic(nuq_context *ctx, const nuq_matrix *m, uint64_t stride, const void *x, uint32_t x_f16,
                uint64_t in_stride, float *out, uint64_t out_stride, uint32_t tokens) {
    return hip_check(ctx,
                     nuq::launch_generic(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride, (uint32_t)m->rows,
                                         (uint32_t)m->columns, x, x_f16, in_stride, out, out_stride, tokens),
                     "generic kernel launch");
}

int matmul_impl(nuq_context *ctx, uint32_t kernel, const nuq_matrix *m, const void *x, uint32_t x_dtype,
                uint64_t in_stride, float *out, uint64_t out_stride, uint32_t tokens) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    uint64_t stride;
    int e = check_matrix(ctx, m, &stride);
    if (e) return e;
    // ops/matmul.zig:77-83
    if (m->rows % 8 != 0 || m->columns % 64 != 0)
        return fail(ctx, NUQ_INVALID_SHAPE, "matmul needs rows %% 8 == 0 and columns %% 64 == 0");
    if (tokens == 0 || in_stride < m->columns || out_stride < m->rows)
        return fail(ctx, NUQ_INVALID_SHAPE, "matmul: tokens, in_stride or out_stride out of range");
    if (x_dtype != NUQ_F32 && x_dtype != NUQ_F16) return fail(ctx, NUQ_INVALID_ARGUMENT, "unknown activation dtype");
    if (!x || !out) return fail(ctx, NUQ_INVALID_ARGUMENT, "null activation or output");
    const uint64_t elem = x_dtype == NUQ_F16 ? 2 : 4;
    if ((uintptr_t)x % 16 != 0 || (in_stride * elem) % 16 != 0 || (uintptr_t)out % 4 != 0)
        return fail(ctx, NUQ_INVALID_SHAPE, "matmul: activations must be 16-byte aligned rows");
    if (kernel > NUQ_KERNEL_GENERIC) return fail(ctx, NUQ_INVALID_ARGUMENT, "unknown kernel %u", kernel);
    if (kernel == NUQ_KERNEL_ROWS && tokens > 8)
        return fail(ctx, NUQ_INVALID_SHAPE, "the multi-token GEMV serves at most 8 tokens");
    const uint32_t f16 = x_dtype == NUQ_F16;
    const bool aligned = vector_aligned(m, stride, x);
    if (ctx->generic_only || kernel == NUQ_KERNEL_GENERIC || !aligned)
        return run_generic(ctx, m, stride, x, f16, in_stride, out, out_stride, tokens);
    if (kernel == NUQ_KERNEL_AUTO) {
        if (tokens == 1 && !f16) return run_gemv(ctx, m, stride, (const float *)x, out);
        if (!f16 && tokens <= 3) {
            const int r = run_rows_mfma(ctx, m, stride, (const float *)x, in_stride, out, out_stride, tokens);
            if (r >= 0) return r;
        }
        // F16 activations on Q4_K / Q5_K take the streamed verify tile: it
        // multiplies the exact f16 activations by the exact f16 integers
        // q * sc and applies d and the minima in F32, so every product is
        // exact and the register GEMV's F32 precision holds while the
        // weights stream once for all tokens.
        const bool exact_tile = f16 && (m->encoding == NUQ_Q4_K || m->encoding == NUQ_Q5_K);
        kernel = tokens <= 3 && specialised(m->encoding) && !exact_tile ? NUQ_KERNEL_ROWS : NUQ_KERNEL_TILE;
    }
    // NUQ_KERNEL_ROWS forces the register-dequant multi-row GEMV (a
    // measurement aid, as the reference's matmulKernel forces a kernel).
    if (kernel == NUQ_KERNEL_ROWS && !specialised(m->encoding))
        return run_generic(ctx, m, stride, x, f16, in_stride, out, out_stride, tokens);
    if (kernel == NUQ_KERNEL_ROWS && f16 && m->encoding == NUQ_Q4_K) {
        // the K-split register kernel; rows longer than 24 blocks run as K
        // ranges into the workspace (at most 4 ranges)
        if (m->columns > 24 * 256) (void)ensure_workspace(ctx, 4ull * tokens * m->rows);
        hipError_t le = hipSuccess;
        if (nuq::launch_rows_q4k_f16(ctx->stream, (const uint8_t *)m->bytes, stride, (uint32_t)m->rows,
                                     (uint32_t)m->columns, (const _Float16 *)x, in_stride, out, out_stride, tokens,
                                     ctx->split.work, (uint64_t)ctx->split.tiles * 256 * 256, &le))
            return hip_check(ctx, le, "multi-token gemv launch");
    }
    if (kernel == NUQ_KERNEL_ROWS)
        return hip_check(ctx,
                         nuq::launch_rows(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride,
                                          (uint32_t)m->rows, (uint32_t)m->columns, x, f16, in_stride, out,
                                          out_stride, tokens),
                         "multi-token gemv launch");
    (void)ensure_workspace(ctx, nuq::tile_workspace_floats(m->encoding, (uint32_t)m->rows, (uint32_t)m->columns,
                                                           tokens, in_stride));
    return hip_check(ctx,
                     nuq::launch_tile(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride, (uint32_t)m->rows,
                                      (uint32_t)m->columns, x, f16, in_stride, out, out_stride, tokens, ctx->split),
                     "tile launch");
}

}  // namespace

extern "C" {

nuq_context *nuq_create(int device, char *err, size_t cap) {
    auto report = [&](const char *msg) {
        if (err && cap) {
            std::snprintf(err, cap, "%s", msg);
        }
    };
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        report("no HIP device available");
        return nullptr;
    }
    if (device < 0 || device >= count) {
        report("device index out of range");
        return nullptr;
    }
    if (hipSetDevice(device) != hipSuccess) {
        report("hipSetDevice failed");
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess || std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        char msg[256];
        std::snprintf(msg, sizeof msg, "libnuq is built for gfx950; device %d is %s", device, prop.gcnArchName);
        report(msg);
        return nullptr;
    }
    auto *ctx = new nuq_context();
    ctx->device = device;
    // this device's copy of the allocation-free scratch (device current)
    if (hipGetSymbolAddress((void **)&ctx->static_scratch, HIP_SYMBOL(scratch)) != hipSuccess ||
        !ctx->static_scratch) {
        (void)hipGetLastError();
        report("hipGetSymbolAddress of the allocation-free scratch failed");
        delete ctx;
        return nullptr;
    }
    if (hipMalloc((void **)&ctx->argmax_buf, 2 * sizeof(uint32_t)) != hipSuccess) {
        report("hipMalloc of the argmax result failed");
        delete ctx;
        return nullptr;
    }
    if (hipMalloc((void **)&ctx->topk_keys, nuq::topk_scratch_keys() * sizeof(uint64_t)) != hipSuccess) {
        report("hipMalloc of the top-k scratch failed");
        nuq_destroy(ctx);
        return nullptr;
    }
    return ctx;
}

void nuq_destroy(nuq_context *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->argmax_buf) (void)hipFree(ctx->argmax_buf);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->split.work) (void)hipFree(ctx->split.work);
    for (float *p : ctx->retired) (void)hipFree(p);
    if (ctx->topk_keys) (void)hipFree(ctx->topk_keys);
    if (ctx->handoff) (void)hipEventDestroy(ctx->handoff);
    delete ctx;
}

int nuq_set_stream(nuq_context *ctx, void *stream) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    hipStream_t next = (hipStream_t)stream;
    if (next != ctx->stream) {
        // The context's workspace is shared by its calls: work on the new
        // stream waits for what was enqueued on the old one. Skipped when
        // either stream is capturing a graph (a capture cannot wait on work
        // outside it); the caller orders captured work itself.
        hipStreamCaptureStatus a = hipStreamCaptureStatusNone, b = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(ctx->stream, &a) == hipSuccess && hipStreamIsCapturing(next, &b) == hipSuccess &&
            a == hipStreamCaptureStatusNone && b == hipStreamCaptureStatusNone) {
            if (!ctx->handoff) {
                int e = hip_check(ctx, hipEventCreateWithFlags(&ctx->handoff, hipEventDisableTiming), "event");
                if (e) return e;
            }
            int e = hip_check(ctx, hipEventRecord(ctx->handoff, ctx->stream), "stream handoff record");
            if (!e) e = hip_check(ctx, hipStreamWaitEvent(next, ctx->handoff, 0), "stream handoff wait");
            if (e) return e;
        }
        ctx->stream = next;
    }
    return NUQ_OK;
}

int nuq_reserve_workspace(nuq_context *ctx, uint64_t bytes) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    (void)hipSetDevice(ctx->device);
    if (!ensure_workspace(ctx, (bytes + sizeof(float) - 1) / sizeof(float)))
        return fail(ctx, NUQ_DEVICE_ERROR, "workspace of %llu bytes could not be allocated (or the stream is capturing)",
                    (unsigned long long)bytes);
    return NUQ_OK;
}

uint64_t nuq_workspace_bytes(const nuq_context *ctx) {
    return ctx ? (uint64_t)ctx->split.tiles * 256 * 256 * sizeof(float) : 0;
}

int nuq_sync(nuq_context *ctx) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    (void)hipSetDevice(ctx->device);
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
}

const char *nuq_last_error(const nuq_context *ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }

int nuq_set_generic_only(nuq_context *ctx, int enabled) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    ctx->generic_only = enabled != 0;
    return NUQ_OK;
}

int nuq_validate_row(uint32_t encoding, uint64_t byte_count, uint64_t element_count) {
    return validate_row(encoding, byte_count, element_count);
}

int nuq_dequant_range(nuq_context *ctx, const nuq_matrix *m, uint64_t first, uint64_t count, float *out) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    uint64_t stride;
    int e = check_matrix(ctx, m, &stride);
    if (e) return e;
    if (m->columns % 16 != 0) return fail(ctx, NUQ_INVALID_SHAPE, "columns must be a multiple of 16");
    if (count == 0 || first >= m->rows || count > m->rows - first)
        return fail(ctx, NUQ_INVALID_SHAPE, "row range outside the matrix");
    if (count > 0xffffffffull) return fail(ctx, NUQ_INVALID_SHAPE, "too many rows in one call");
    if (!out) return fail(ctx, NUQ_INVALID_ARGUMENT, "null output");
    return hip_check(ctx,
                     nuq::launch_dequant_rows(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride, first,
                                              (uint32_t)count, (uint32_t)m->columns, out),
                     "dequant launch");
}

int nuq_embed(nuq_context *ctx, const nuq_matrix *m, uint32_t token, float *out) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (m && token >= m->rows) return fail(ctx, NUQ_INVALID_SHAPE, "token %u outside %llu rows", token,
                                           (unsigned long long)m->rows);
    return nuq_dequant_range(ctx, m, token, 1, out);
}

int nuq_matvec(nuq_context *ctx, const nuq_matrix *m, const float *x, float *out) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    uint64_t stride;
    int e = check_matrix(ctx, m, &stride);
    if (e) return e;
    if (m->columns % 16 != 0) return fail(ctx, NUQ_INVALID_SHAPE, "columns must be a multiple of 16");
    if (!x || !out) return fail(ctx, NUQ_INVALID_ARGUMENT, "null input or output");
    if ((uintptr_t)x % 4 != 0 || (uintptr_t)out % 4 != 0)
        return fail(ctx, NUQ_INVALID_SHAPE, "input and output must be 4-byte aligned");
    if (ctx->generic_only || !vector_aligned(m, stride, x)) return run_generic(ctx, m, stride, x, 0, m->columns, out, m->rows, 1);
    return run_gemv(ctx, m, stride, x, out);
}

int nuq_matvec_rows(nuq_context *ctx, const nuq_matrix *m, const float *x, uint64_t in_stride, float *out,
                    uint64_t out_stride, uint32_t tokens) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    uint64_t stride;
    int e = check_matrix(ctx, m, &stride);
    if (e) return e;
    if (m->columns % 16 != 0) return fail(ctx, NUQ_INVALID_SHAPE, "columns must be a multiple of 16");
    if (tokens < 2 || tokens > 8) return fail(ctx, NUQ_INVALID_SHAPE, "matvecRows serves 2..8 tokens");
    if (in_stride < m->columns || out_stride < m->rows)
        return fail(ctx, NUQ_INVALID_SHAPE, "in_stride or out_stride too small");
    if (!x || !out) return fail(ctx, NUQ_INVALID_ARGUMENT, "null input or output");
    if ((uintptr_t)x % 16 != 0 || in_stride % 4 != 0 || (uintptr_t)out % 4 != 0)
        return fail(ctx, NUQ_INVALID_SHAPE, "input must be float4 aligned (offset and stride)");
    if (ctx->generic_only || !vector_aligned(m, stride, x))
        return run_generic(ctx, m, stride, x, 0, in_stride, out, out_stride, tokens);
    const int r = run_rows_mfma(ctx, m, stride, x, in_stride, out, out_stride, tokens);
    if (r >= 0) return r;
    if (!specialised(m->encoding)) return run_generic(ctx, m, stride, x, 0, in_stride, out, out_stride, tokens);
    return hip_check(ctx,
                     nuq::launch_rows(ctx->stream, m->encoding, (const uint8_t *)m->bytes, stride, (uint32_t)m->rows,
                                      (uint32_t)m->columns, x, 0, in_stride, out, out_stride, tokens),
                     "multi-token gemv launch");
}

int nuq_matmul(nuq_context *ctx, const nuq_matrix *m, const void *x, uint32_t x_dtype, uint64_t in_stride, float *out,
               uint64_t out_stride, uint32_t tokens) {
    return matmul_impl(ctx, NUQ_KERNEL_AUTO, m, x, x_dtype, in_stride, out, out_stride, tokens);
}

int nuq_matmul_kernel(nuq_context *ctx, uint32_t kernel, const nuq_matrix *m, const void *x, uint32_t x_dtype,
                      uint64_t in_stride, float *out, uint64_t out_stride, uint32_t tokens) {
    return matmul_impl(ctx, kernel, m, x, x_dtype, in_stride, out, out_stride, tokens);
}

// Flat-argument forms: a matrix of `rows` rows of `stride` bytes each, as
// the descriptor entry points validate it (stride must be the encoded row
// length, cpu/root.zig:31-36).
static nuq_matrix flat_matrix(uint32_t encoding, const void *w, uint64_t stride, uint32_t rows, uint32_t columns) {
    nuq_matrix m;
    m.encoding = encoding;
    m.reserved = 0;
    m.rows = rows;
    m.columns = columns;
    m.bytes = w;
    m.byte_len = stride * rows;
    return m;
}

int nuq_dequant_rows(nuq_context *ctx, uint32_t encoding, const void *w, uint64_t stride, uint32_t rows,
                     uint32_t columns, float *out) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (rows != 0 && stride > UINT64_MAX / rows) return fail(ctx, NUQ_INVALID_BYTE_LENGTH, "rows x stride overflows");
    const nuq_matrix m = flat_matrix(encoding, w, stride, rows, columns);
    return nuq_dequant_range(ctx, &m, 0, rows, out);
}

int nuq_gemv(nuq_context *ctx, uint32_t encoding, const void *w, uint64_t stride, uint32_t rows, uint32_t columns,
             const float *x, float *y) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (rows != 0 && stride > UINT64_MAX / rows) return fail(ctx, NUQ_INVALID_BYTE_LENGTH, "rows x stride overflows");
    const nuq_matrix m = flat_matrix(encoding, w, stride, rows, columns);
    return nuq_matvec(ctx, &m, x, y);
}

int nuq_gemm(nuq_context *ctx, uint32_t encoding, const void *w, uint64_t stride, uint32_t rows, uint32_t columns,
             const void *x, uint32_t x_dtype, uint64_t in_stride, float *y, uint64_t out_stride, uint32_t tokens) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (rows != 0 && stride > UINT64_MAX / rows) return fail(ctx, NUQ_INVALID_BYTE_LENGTH, "rows x stride overflows");
    const nuq_matrix m = flat_matrix(encoding, w, stride, rows, columns);
    return nuq_matmul(ctx, &m, x, x_dtype, in_stride, y, out_stride, tokens);
}

// Rows from which a SiLU pair runs as two decode GEMVs plus the epilogue.
constexpr uint64_t PAIR_SPLIT_ROWS = 4096;

// The body of both segment entry points. `fixed` (the allocation-free form)
// is a device buffer of `fixed_floats` floats that takes the SiLU pair's
// second GEMV instead of the context workspace; the form then never
// allocates and refuses pairs it cannot hold.
static int segments_impl(nuq_context *ctx, const nuq_segment *segments, uint32_t count, const float *x, uint32_t mode,
                         float *fixed, uint64_t fixed_floats) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (!segments || count == 0 || count > 4) return fail(ctx, NUQ_INVALID_SHAPE, "segments: 1..4 projections");
    if (mode > NUQ_SEGMENT_SILU_MUL_PAIR) return fail(ctx, NUQ_INVALID_ARGUMENT, "unknown segment mode");
    if (!x || (uintptr_t)x % 16 != 0) return fail(ctx, NUQ_INVALID_SHAPE, "input must be 16-byte aligned");
    const uint64_t columns = segments[0].matrix.columns;
    if (columns == 0 || columns % 16 != 0) return fail(ctx, NUQ_INVALID_SHAPE, "columns must be a multiple of 16");
    if (mode != NUQ_SEGMENT_PLAIN &&
        (count != 2 || segments[0].matrix.rows != segments[1].matrix.rows || segments[0].output != segments[1].output))
        return fail(ctx, NUQ_INVALID_SHAPE, "a pair needs two segments of equal rows naming one output");
    nuq::SegmentsArgs args;
    std::memset(&args, 0, sizeof args);
    args.count = count;
    args.mode = mode;
    const uint32_t rpw = (uint32_t)nuq::segment_rows_per_wave();
    uint32_t waves = 0;
    uint64_t strides[4];
    for (uint32_t i = 0; i < count; ++i) {
        const nuq_matrix &m = segments[i].matrix;
        uint64_t stride;
        int e = check_matrix(ctx, &m, &stride);
        if (e) return e;
        strides[i] = stride;
        if (m.rows % 16 != 0 || m.columns != columns)
            return fail(ctx, NUQ_INVALID_SHAPE, "segment %u: rows %% 16 and equal columns required", i);
        if (!segments[i].output || (uintptr_t)segments[i].output % 4 != 0)
            return fail(ctx, NUQ_INVALID_SHAPE, "segment %u: output null or misaligned", i);
        if (!vector_aligned(&m, stride, x))
            return fail(ctx, NUQ_INVALID_SHAPE, "segment %u: weights not aligned for the merged kernel", i);
        // Plain outputs must be disjoint from each other and from the input.
        const float *o = segments[i].output;
        if ((const void *)o < (const void *)(x + columns) && (const void *)x < (const void *)(o + m.rows))
            return fail(ctx, NUQ_INVALID_SHAPE, "segment %u: output overlaps the input", i);
        if (mode == NUQ_SEGMENT_PLAIN)
            for (uint32_t k = 0; k < i; ++k) {
                const float *p = segments[k].output;
                if (o < p + segments[k].matrix.rows && p < o + m.rows)
                    return fail(ctx, NUQ_INVALID_SHAPE, "segment %u: output overlaps segment %u", i, k);
            }
        nuq::Layout l;
        nuq::layout_of(m.encoding, &l);
        args.seg[i] = {(const uint8_t *)m.bytes, stride, segments[i].output, m.encoding, (uint32_t)m.rows,
                       (uint32_t)(columns / l.elements), 0};
        args.wave_start[i] = waves;
        waves += (uint32_t)((m.rows + rpw - 1) / rpw);
    }
    args.wave_start[count] = waves;
    if (fixed && mode == NUQ_SEGMENT_SILU_MUL_PAIR && segments[0].matrix.rows > fixed_floats)
        return fail(ctx, NUQ_INVALID_SHAPE,
                    "SiLU pair of %llu rows exceeds the allocation-free scratch (at most %llu rows)",
                    (unsigned long long)segments[0].matrix.rows, (unsigned long long)fixed_floats);
    // A large SiLU pair streams faster as decode GEMVs (gate into the output,
    // up into a workspace) and the elementwise epilogue than as one merged
    // row-per-wave pass.
    const bool pair_big = mode == NUQ_SEGMENT_SILU_MUL_PAIR && !ctx->generic_only &&
                          segments[0].matrix.rows >= PAIR_SPLIT_ROWS;
    const bool pair_split = pair_big && (fixed || ensure_workspace(ctx, segments[0].matrix.rows));
    float *up_buffer = fixed ? fixed : ctx->split.work;
    // Segments of one encoding and row stride (q/k/v, gate/up) run as one
    // launch of the decode GEMV, each matrix on its share of the workgroups.
    bool same = !ctx->generic_only && (mode == NUQ_SEGMENT_PLAIN || pair_split);
    for (uint32_t i = 1; i < count && same; ++i)
        same = segments[i].matrix.encoding == segments[0].matrix.encoding && strides[i] == strides[0];
    if (same) {
        const uint8_t *ws[4];
        uint32_t rs[4];
        float *ys[4];
        for (uint32_t i = 0; i < count; ++i) {
            ws[i] = (const uint8_t *)segments[i].matrix.bytes;
            rs[i] = (uint32_t)segments[i].matrix.rows;
            ys[i] = segments[i].output;
        }
        if (mode != NUQ_SEGMENT_PLAIN) ys[1] = up_buffer;
        const hipError_t he = nuq::launch_gemv_dma_segments(ctx->stream, segments[0].matrix.encoding, count, ws,
                                                            strides[0], rs, (uint32_t)columns, x, ys);
        if (he != hipErrorInvalidValue) {
            int e = hip_check(ctx, he, "segments gemv launch");
            if (e || mode == NUQ_SEGMENT_PLAIN) return e;
            return hip_check(ctx, nuq::launch_silu_mul(ctx->stream, segments[0].output, up_buffer, rs[0]),
                             "silu pair epilogue");
        }
    }
    if (pair_split) {
        const nuq_matrix &g = segments[0].matrix, &u = segments[1].matrix;
        float *up = up_buffer;
        int e = run_gemv(ctx, &g, g.byte_len / g.rows, x, segments[0].output);
        if (e) return e;
        e = run_gemv(ctx, &u, u.byte_len / u.rows, x, up);
        if (e) return e;
        return hip_check(ctx, nuq::launch_silu_mul(ctx->stream, segments[0].output, up, (uint32_t)g.rows),
                         "silu pair epilogue");
    }
    if (mode != NUQ_SEGMENT_PLAIN) args.wave_start[1] = (uint32_t)((segments[0].matrix.rows + rpw - 1) / rpw);
    return hip_check(ctx, nuq::launch_segments(ctx->stream, args, x), "segments launch");
}

int nuq_matvec_segments(nuq_context *ctx, const nuq_segment *segments, uint32_t count, const float *x, uint32_t mode) {
    return segments_impl(ctx, segments, count, x, mode, nullptr, 0);
}

int nuq_matvec_segments_noalloc(nuq_context *ctx, const nuq_segment *segments, uint32_t count, const float *x,
                                uint32_t mode) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    return segments_impl(ctx, segments, count, x, mode, ctx->static_scratch, NOALLOC_SCRATCH_FLOATS);
}

int nuq_argmax(nuq_context *ctx, const float *logits, uint64_t count, uint32_t *index) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (!logits || !index) return fail(ctx, NUQ_INVALID_ARGUMENT, "null logits or index");
    if (count == 0 || count > 0xffffffffull) return fail(ctx, NUQ_INVALID_SHAPE, "logit count out of range");
    int e = hip_check(ctx, nuq::launch_argmax(ctx->stream, logits, count, ctx->argmax_buf), "argmax launch");
    if (e) return e;
    uint32_t host[2];
    e = hip_check(ctx, hipMemcpyAsync(host, ctx->argmax_buf, sizeof host, hipMemcpyDeviceToHost, ctx->stream),
                  "argmax readback");
    if (e) return e;
    e = hip_check(ctx, hipStreamSynchronize(ctx->stream), "argmax synchronize");
    if (e) return e;
    if (host[1]) return fail(ctx, NUQ_NON_FINITE, "NonFiniteResult: a logit is not finite");
    *index = host[0];
    return NUQ_OK;
}

// Sampler.penalize on the device (backends/metal/ops/sampling.zig:63-71).
int nuq_penalize(nuq_context *ctx, float *logits, uint64_t count, const uint32_t *history, uint64_t history_words,
                 float repetition, float presence) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (!logits || !history) return fail(ctx, NUQ_INVALID_ARGUMENT, "null logits or history");
    if (count == 0 || count > 0xffffffffull) return fail(ctx, NUQ_INVALID_SHAPE, "logit count out of range");
    if (!std::isfinite(repetition) || repetition <= 0 || !std::isfinite(presence))
        return fail(ctx, NUQ_INVALID_SHAPE, "penalties must be finite and the repetition positive");
    if (history_words < (count + 31) / 32) return fail(ctx, NUQ_INVALID_SHAPE, "history shorter than the logits");
    return hip_check(ctx, nuq::launch_penalize(ctx->stream, logits, (uint32_t)count, history, repetition, presence),
                     "penalize launch");
}

// Backend.topk (backends/metal/ops/sampling.zig:44-57).
int nuq_topk(nuq_context *ctx, const float *logits, uint64_t count, uint32_t k, float temperature,
             const nuq_topk_buffers *out) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (!logits || !out || !out->values || !out->indices || !out->sums || !out->flags)
        return fail(ctx, NUQ_INVALID_ARGUMENT, "null logits or top-k buffers");
    if (count == 0 || count > nuq::TOPK_MAX_COUNT || k == 0 || k > nuq::TOPK_CAPACITY || k > count)
        return fail(ctx, NUQ_INVALID_SHAPE, "top-k of %u over %llu logits is out of range", k,
                    (unsigned long long)count);
    if (!std::isfinite(temperature) || temperature <= 0)
        return fail(ctx, NUQ_INVALID_SHAPE, "temperature must be finite and positive");
    return hip_check(ctx,
                     nuq::launch_topk(ctx->stream, logits, (uint32_t)count, k, temperature, ctx->topk_keys,
                                      out->values, out->indices, out->sums, out->flags),
                     "top-k launch");
}

// The tensor-data section of a GGUF file goes to the device unchanged
// (tensors keep their offsets). Host threads copy the mapping into one of
// two pinned staging buffers while the DMA engine drains the other, so the
// page-cache reads, the pinned copy and PCIe overlap.
int nuq_gguf_upload(nuq_context *ctx, const nuq_gguf *g, void *device, uint64_t device_len) {
    if (!ctx) return NUQ_INVALID_ARGUMENT;
    if (!g || (!device && device_len)) return fail(ctx, NUQ_INVALID_ARGUMENT, "null document or device pointer");
    const uint64_t total = g->file_bytes - g->data_offset;
    if (g->avail < g->file_bytes) return fail(ctx, NUQ_GGUF_END_OF_STREAM, "the tensor data is not all present");
    if (device_len < total)
        return fail(ctx, NUQ_INVALID_ARGUMENT, "device buffer of %llu bytes < data section of %llu",
                    (unsigned long long)device_len, (unsigned long long)total);
    if (total == 0) return NUQ_OK;
    constexpr uint64_t CHUNK = 64ull << 20;
    const uint64_t chunk = std::min(CHUNK, total);
    uint8_t *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = NUQ_OK;
    for (int b = 0; b < 2 && rc == NUQ_OK; ++b) {
        rc = hip_check(ctx, hipHostMalloc((void **)&stage[b], chunk, hipHostMallocDefault), "pinned staging");
        if (rc == NUQ_OK) rc = hip_check(ctx, hipEventCreateWithFlags(&done[b], hipEventDisableTiming), "event");
    }
    const unsigned threads = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    const uint8_t *src = g->bytes + g->data_offset;
    for (uint64_t off = 0, k = 0; rc == NUQ_OK && off < total; off += chunk, ++k) {
        const int b = (int)(k & 1);
        const uint64_t n = std::min(chunk, total - off);
        // the copy that last used this buffer must have drained it
        if (k >= 2) {
            rc = hip_check(ctx, hipEventSynchronize(done[b]), "staging wait");
            if (rc != NUQ_OK) break;
        }
        const uint64_t part = (n + threads - 1) / threads;
        std::vector<std::thread> pool;
        for (unsigned t = 1; t < threads && t * part < n; ++t)
            pool.emplace_back([&, t] { memcpy(stage[b] + t * part, src + off + t * part, std::min(part, n - t * part)); });
        memcpy(stage[b], src + off, std::min(part, n));
        for (auto &th : pool) th.join();
        rc = hip_check(ctx, hipMemcpyAsync((uint8_t *)device + off, stage[b], n, hipMemcpyHostToDevice, ctx->stream),
                       "upload copy");
        if (rc == NUQ_OK) rc = hip_check(ctx, hipEventRecord(done[b], ctx->stream), "upload event");
    }
    const int sync = hip_check(ctx, hipStreamSynchronize(ctx->stream), "upload synchronize");
    if (rc == NUQ_OK) rc = sync;
    for (int b = 0; b < 2; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (stage[b]) (void)hipHostFree(stage[b]);
    }
    return rc;
}

}  // extern "C"


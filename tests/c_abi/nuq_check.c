/*
 * The C ABI driven from C, as the Zig engine would drive it through
 * @cImport: plain C, include/nuq.h + include/nuq_gguf.h, device memory from
 * the HIP runtime, no Python. Checks each call against the CPU oracle
 * (oracle/oracle.h, test infrastructure) on seeded inputs:
 *   - nuq_dequant_rows bit-exact with orc_decode_row (Q4_K, Q6_K, Q8_0);
 *   - nuq_gemv / nuq_matvec within max relative error 2e-3 of orc_matvec;
 *   - nuq_gemm (M = 8, f16 activations) within 2e-3 of orc_matmul on the
 *     f16-rounded activations;
 *   - nuq_topk ids equal to orc_topk, nuq_argmax equal to orc_argmax;
 *   - refusals: a wrong stride is NUQ_INVALID_BYTE_LENGTH, a GGUF with a bad
 *     magic is NUQ_GGUF_INVALID_MAGIC.
 * Prints "nuq_check: OK" and exits 0, or names the failing check and exits 1.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nuq.h"
#include "nuq_gguf.h"
#include "oracle.h"

static int failures = 0;
#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            fprintf(stderr, "nuq_check: FAIL: " __VA_ARGS__); \
            fprintf(stderr, "\n");                        \
            ++failures;                                   \
        }                                                 \
    } while (0)
#define HIP(call)                                                         \
    do {                                                                  \
        hipError_t e_ = (call);                                           \
        if (e_ != hipSuccess) {                                           \
            fprintf(stderr, "nuq_check: %s: %s\n", #call, hipGetErrorString(e_)); \
            exit(1);                                                      \
        }                                                                 \
    } while (0)

/* splitmix64 -> two uniforms -> Box-Muller: seeded N(0, 1) floats */
static uint64_t state;
static uint64_t next_u64(void) {
    uint64_t z = (state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static void gaussian(uint64_t seed, float *out, size_t n, float std) {
    state = seed;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = ((next_u64() >> 11) + 1.0) / 9007199254740993.0;
        const double u2 = (next_u64() >> 11) / 9007199254740992.0;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(6.283185307179586 * u2) * std);
        if (i + 1 < n) out[i + 1] = (float)(r * sin(6.283185307179586 * u2) * std);
    }
}

static size_t row_bytes(uint32_t encoding, size_t columns) {
    switch (encoding) {
        case NUQ_Q8_0: return columns / 32 * 34;
        case NUQ_Q4_K: return columns / 256 * 144;
        case NUQ_Q6_K: return columns / 256 * 210;
        default: return 0;
    }
}

static void *to_device(const void *host, size_t n) {
    void *d = NULL;
    HIP(hipMalloc(&d, n));
    HIP(hipMemcpy(d, host, n, hipMemcpyHostToDevice));
    return d;
}

static double normwise(const float *got, const float *want, size_t n) {
    double err = 0, mag = 0;
    for (size_t i = 0; i < n; ++i) {
        if (!isfinite(got[i])) return INFINITY;
        const double e = fabs((double)got[i] - want[i]);
        if (e > err) err = e;
        if (fabs(want[i]) > mag) mag = fabs(want[i]);
    }
    return err / (mag > 0 ? mag : 1);
}

static void check_matrix(nuq_context *ctx, uint32_t encoding, uint32_t rows, uint32_t columns, uint64_t seed) {
    const size_t stride = row_bytes(encoding, columns), wbytes = stride * rows;
    float *wf = malloc(sizeof(float) * rows * columns), *x = malloc(sizeof(float) * 8 * columns);
    uint8_t *w = malloc(wbytes);
    gaussian(seed, wf, (size_t)rows * columns, 0.02f);
    gaussian(seed + 1, x, (size_t)8 * columns, 1.0f);
    CHECK(nuq_quantize_rows(encoding, wf, rows, columns, w, wbytes) == NUQ_OK, "quantize %u", encoding);
    void *dw = to_device(w, wbytes), *dx = to_device(x, sizeof(float) * columns);
    float *dy = NULL, *dd = NULL, *dyt = NULL;
    HIP(hipMalloc((void **)&dy, sizeof(float) * rows));
    HIP(hipMalloc((void **)&dd, sizeof(float) * rows * columns));
    HIP(hipMalloc((void **)&dyt, sizeof(float) * 8 * rows));

    /* dequant: bit-exact */
    CHECK(nuq_dequant_rows(ctx, encoding, dw, stride, rows, columns, dd) == NUQ_OK, "dequant %u: %s", encoding,
          nuq_last_error(ctx));
    /* GEMV through both entry forms */
    CHECK(nuq_gemv(ctx, encoding, dw, stride, rows, columns, dx, dy) == NUQ_OK, "gemv %u: %s", encoding,
          nuq_last_error(ctx));
    CHECK(nuq_sync(ctx) == NUQ_OK, "sync");
    float *dec = malloc(sizeof(float) * rows * columns), *dec_ref = malloc(sizeof(float) * columns);
    HIP(hipMemcpy(dec, dd, sizeof(float) * rows * columns, hipMemcpyDeviceToHost));
    size_t mismatched = 0;
    for (uint32_t r = 0; r < rows; ++r) {
        orc_decode_row(encoding, w + (size_t)r * stride, stride, dec_ref, columns);
        if (memcmp(dec + (size_t)r * columns, dec_ref, sizeof(float) * columns) != 0) ++mismatched;
    }
    CHECK(mismatched == 0, "dequant %u: %zu rows differ from the oracle", encoding, mismatched);
    float *y = malloc(sizeof(float) * rows), *yref = malloc(sizeof(float) * rows);
    HIP(hipMemcpy(y, dy, sizeof(float) * rows, hipMemcpyDeviceToHost));
    orc_matvec(encoding, rows, columns, w, wbytes, x, columns, yref, rows, 1);
    const double e1 = normwise(y, yref, rows);
    CHECK(e1 <= 2e-3, "gemv %u: normwise %.3e", encoding, e1);
    nuq_matrix m = {encoding, 0, rows, columns, dw, wbytes};
    CHECK(nuq_matvec(ctx, &m, dx, dy) == NUQ_OK && nuq_sync(ctx) == NUQ_OK, "matvec %u", encoding);
    float *y2 = malloc(sizeof(float) * rows);
    HIP(hipMemcpy(y2, dy, sizeof(float) * rows, hipMemcpyDeviceToHost));
    CHECK(memcmp(y, y2, sizeof(float) * rows) == 0, "gemv and matvec %u differ", encoding);

    /* M = 8 verify GEMM with f16 activations */
    uint16_t *x16 = malloc(sizeof(uint16_t) * 8 * columns);
    float *xr = malloc(sizeof(float) * 8 * columns);
    for (size_t i = 0; i < (size_t)8 * columns; ++i) {
        x16[i] = orc_f32_to_half(x[i]);
        xr[i] = orc_half_to_f32(x16[i]);
    }
    void *dx16 = to_device(x16, sizeof(uint16_t) * 8 * columns);
    CHECK(nuq_gemm(ctx, encoding, dw, stride, rows, columns, dx16, NUQ_F16, columns, dyt, rows, 8) == NUQ_OK,
          "gemm %u: %s", encoding, nuq_last_error(ctx));
    CHECK(nuq_sync(ctx) == NUQ_OK, "sync");
    float *yt = malloc(sizeof(float) * 8 * rows), *ytref = malloc(sizeof(float) * 8 * rows);
    HIP(hipMemcpy(yt, dyt, sizeof(float) * 8 * rows, hipMemcpyDeviceToHost));
    orc_matmul(encoding, rows, columns, w, wbytes, xr, columns, ytref, rows, 8, 0);
    const double e2 = normwise(yt, ytref, (size_t)8 * rows);
    CHECK(e2 <= 2e-3, "gemm %u: normwise %.3e", encoding, e2);

    /* refusal: a stride that is not the encoded row length */
    CHECK(nuq_gemv(ctx, encoding, dw, stride + 2, rows, columns, dx, dy) == NUQ_INVALID_BYTE_LENGTH,
          "gemv %u with a wrong stride was not refused", encoding);
    printf("nuq_check: encoding %u %ux%u: dequant exact, gemv %.2e, gemm M=8 %.2e\n", encoding, rows, columns, e1,
           e2);

    free(wf); free(x); free(w); free(dec); free(dec_ref); free(y); free(yref); free(y2);
    free(x16); free(xr); free(yt); free(ytref);
    HIP(hipFree(dw)); HIP(hipFree(dx)); HIP(hipFree(dy)); HIP(hipFree(dd)); HIP(hipFree(dyt)); HIP(hipFree(dx16));
}

static void check_sampling(nuq_context *ctx) {
    const size_t n = 151936;
    const uint32_t k = 256;
    float *logits = malloc(sizeof(float) * n);
    gaussian(77, logits, n, 3.0f);
    logits[4242] = 40.0f;
    float *dl = to_device(logits, sizeof(float) * n);
    nuq_topk_buffers b;
    HIP(hipMalloc((void **)&b.values, sizeof(float) * k));
    HIP(hipMalloc((void **)&b.indices, sizeof(uint32_t) * k));
    HIP(hipMalloc((void **)&b.sums, sizeof(float) * NUQ_TOPK_PARTIALS));
    HIP(hipMalloc((void **)&b.flags, sizeof(uint32_t) * NUQ_TOPK_PARTIALS));
    CHECK(nuq_topk(ctx, dl, n, k, 0.7f, &b) == NUQ_OK && nuq_sync(ctx) == NUQ_OK, "topk: %s", nuq_last_error(ctx));
    uint32_t ids[256], want_ids[256];
    float vals[256], want_vals[256];
    double total;
    int finite;
    HIP(hipMemcpy(ids, b.indices, sizeof ids, hipMemcpyDeviceToHost));
    orc_topk(logits, n, k, 0.7f, want_ids, want_vals, &total, &finite);
    CHECK(memcmp(ids, want_ids, sizeof ids) == 0, "topk ids differ from the oracle");
    HIP(hipMemcpy(vals, b.values, sizeof vals, hipMemcpyDeviceToHost));
    CHECK(memcmp(vals, want_vals, sizeof vals) == 0, "topk values differ from the oracle");
    uint32_t best = 0;
    size_t want_best = 0;
    CHECK(nuq_argmax(ctx, dl, n, &best) == NUQ_OK, "argmax");
    orc_argmax(logits, n, &want_best);
    CHECK(best == want_best && best == 4242, "argmax %u, oracle %zu", best, want_best);
    CHECK(nuq_topk(ctx, dl, n, 0, 0.7f, &b) == NUQ_INVALID_SHAPE, "topk k = 0 was not refused");
    printf("nuq_check: top-k 256 of %zu equal to the oracle, argmax %u\n", n, best);
    free(logits);
    HIP(hipFree(dl)); HIP(hipFree(b.values)); HIP(hipFree(b.indices)); HIP(hipFree(b.sums)); HIP(hipFree(b.flags));
}

static void check_gguf(void) {
    /* header only (magic, version 3, no tensors, no metadata), padded to the
     * 32-byte default alignment where the (empty) data section starts */
    uint8_t file[32] = {'G', 'G', 'U', 'F', 3, 0, 0, 0};
    nuq_gguf *g = NULL;
    CHECK(nuq_gguf_parse(file, sizeof file, sizeof file, NULL, &g, NULL) == NUQ_OK, "empty GGUF refused");
    nuq_gguf_info info;
    CHECK(g && nuq_gguf_info_get(g, &info) == NUQ_OK && info.version == 3 && info.tensor_count == 0, "GGUF info");
    nuq_gguf_close(g);
    CHECK(nuq_gguf_parse(file, 24, 24, NULL, &g, NULL) == NUQ_GGUF_END_OF_STREAM && g == NULL,
          "a GGUF ending before its data offset was not EndOfStream");
    file[0] = 'X';
    CHECK(nuq_gguf_parse(file, sizeof file, sizeof file, NULL, &g, NULL) == NUQ_GGUF_INVALID_MAGIC && g == NULL,
          "bad GGUF magic not refused");
}

int main(int argc, char **argv) {
    if (argc > 1 && strcmp(argv[1], "--host-only") == 0) {  /* the checks that need no GPU */
        check_gguf();
        printf(failures ? "nuq_check: host checks failed\n" : "nuq_check: host OK\n");
        return failures ? 1 : 0;
    }
    char err[256] = {0};
    nuq_context *ctx = nuq_create(0, err, sizeof err);
    if (!ctx) {
        fprintf(stderr, "nuq_check: nuq_create: %s\n", err);
        return 1;
    }
    hipStream_t stream;
    HIP(hipStreamCreate(&stream));
    CHECK(nuq_set_stream(ctx, stream) == NUQ_OK, "set stream");
    check_matrix(ctx, NUQ_Q4_K, 512, 5120, 10);
    check_matrix(ctx, NUQ_Q6_K, 264, 5120, 20);
    check_matrix(ctx, NUQ_Q8_0, 296, 4096, 30);
    check_sampling(ctx);
    check_gguf();
    nuq_destroy(ctx);
    HIP(hipStreamDestroy(stream));
    if (failures) {
        fprintf(stderr, "nuq_check: %d failure(s)\n", failures);
        return 1;
    }
    printf("nuq_check: OK\n");
    return 0;
}

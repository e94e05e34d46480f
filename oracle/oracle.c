/*
 * CPU oracle for the quantized-weight matmul path. TEST INFRASTRUCTURE ONLY:
 * the checker for tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg. The product never loads it. Function-by-function citations of the
 * nuclis sources are in oracle.h.
 *
 * Arithmetic discipline: compiled with -ffp-contract=off and without
 * -ffast-math, so each F32 multiply and subtract rounds on its own exactly as
 * the Zig decoders do, and the matvec sum is an F64 sum in column order with
 * one rounding to F32 at the end.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <stdatomic.h>
#include <string.h>
#include <unistd.h>

/* decode.zig:432-435: little-endian F16 widened exactly (subnormals, signed
 * zero, infinities and NaN payloads preserved). */
float orc_half_to_f32(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits >> 15) << 31;
    uint32_t exponent = (bits >> 10) & 31u;
    uint32_t mantissa = bits & 0x3ffu;
    uint32_t out;
    if (exponent == 0) {
        /* zero or subnormal: mantissa * 2^-24, exact in F32 */
        float magnitude = ldexpf((float)mantissa, -24);
        memcpy(&out, &magnitude, 4);
        out |= sign;
    } else if (exponent == 31) {
        out = sign | 0x7f800000u | (mantissa << 13);
    } else {
        out = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float value;
    memcpy(&value, &out, 4);
    return value;
}

/* F32 -> F16, round to nearest even, overflow to infinity, NaN stays NaN:
 * the narrowing `@floatCast` performs in encode.zig:29. */
uint16_t orc_f32_to_half(float value) {
    uint32_t u;
    memcpy(&u, &value, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {
        /* below 2^-14: subnormal half; value * 2^24 is exact, rintf rounds to even */
        float magnitude;
        memcpy(&magnitude, &a, 4);
        return (uint16_t)(sign | (uint16_t)rintf(magnitude * 16777216.0f));
    }
    uint32_t rounded = a + 0xfffu + ((a >> 13) & 1u);
    return (uint16_t)(sign | (uint16_t)((rounded - 0x38000000u) >> 13));
}

static int layout(uint32_t encoding, size_t *elements, size_t *bytes) {
    /* inference/src/tensor/encoding.zig:29-41 */
    switch (encoding) {
    case 0: *elements = 1; *bytes = 4; return 1;
    case 1: *elements = 1; *bytes = 2; return 1;
    case 8: *elements = 32; *bytes = 34; return 1;
    case 12: *elements = 256; *bytes = 144; return 1;
    case 13: *elements = 256; *bytes = 176; return 1;
    case 14: *elements = 256; *bytes = 210; return 1;
    case 23: *elements = 256; *bytes = 136; return 1;
    default: return 0;
    }
}

int orc_validate_row(uint32_t encoding, size_t byte_count, size_t element_count) {
    size_t elements, block_bytes;
    if (!layout(encoding, &elements, &block_bytes)) return ORC_UNSUPPORTED_ENCODING;
    if (element_count == 0 || element_count % elements != 0) return ORC_INVALID_ROW_LENGTH;
    if (byte_count % block_bytes != 0 || byte_count / block_bytes != element_count / elements)
        return ORC_INVALID_BYTE_LENGTH;
    return ORC_OK;
}

static float half_at(const uint8_t *p) { return orc_half_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* decode.zig:147-170, kBlock: Q4_K (fifth_bit 0, codes at 16) and Q5_K
 * (fifth_bit 1: codes at 48, and byte 16 + c of the high-bit plane gives
 * bit g of column c as bit 4 of group g's code). */
static void k_block(int fifth_bit, const uint8_t *block, float *out) {
    float d = half_at(block);
    float dmin = half_at(block + 2);
    const uint8_t *s = block + 4;
    const uint8_t *low = block + (fifth_bit ? 48 : 16);
    for (int g = 0; g < 8; ++g) {
        unsigned scale, minimum;
        if (g < 4) {
            scale = s[g] & 63u;
            minimum = s[g + 4] & 63u;
        } else {
            scale = (s[g + 4] & 15u) | ((unsigned)(s[g - 4] >> 6) << 4);
            minimum = (unsigned)(s[g + 4] >> 4) | ((unsigned)(s[g] >> 6) << 4);
        }
        float multiplier = d * (float)scale;
        float offset = dmin * (float)minimum;
        for (int c = 0; c < 32; ++c) {
            uint8_t byte = low[g / 2 * 32 + c];
            unsigned q = (g % 2 == 0) ? (byte & 15u) : (unsigned)(byte >> 4);
            if (fifth_bit) q |= (unsigned)((block[16 + c] >> g) & 1u) << 4;
            float scaled = multiplier * (float)q;
            out[g * 32 + c] = scaled - offset;
        }
    }
}

/* decode.zig:198-211, Q6_K. */
static void q6k_block(const uint8_t *block, float *out) {
    float d = half_at(block + 208);
    for (int i = 0; i < 256; ++i) {
        int quarter = (i % 128) / 32;
        int column = i % 32;
        int low_shift = (quarter / 2) * 4;
        int high_shift = quarter * 2;
        int low = (block[(i / 128) * 64 + (quarter % 2) * 32 + column] >> low_shift) & 15;
        int high = (block[128 + (i / 128) * 32 + column] >> high_shift) & 3;
        int value = (low | (high << 4)) - 32;
        int8_t scale = (int8_t)block[192 + i / 16];
        float multiplier = d * (float)scale;
        out[i] = multiplier * (float)value;
    }
}

/* decode.zig:437, the IQ4_NL / IQ4_XS nonlinear code values. */
static const int8_t iq4_values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* decode.zig:213-228, IQ4_XS: [d:f16][scales_h:u16][scales_l:4 B][qs:128 B].
 * Group g's six-bit scale is nibble g%2 of scales_l[g/2] plus bits 2g..2g+1
 * of scales_h, biased by -32; qs[16g + j] holds values 32g + j (low nibble)
 * and 32g + j + 16 (high nibble). */
static void iq4xs_block(const uint8_t *block, float *out) {
    float d = half_at(block);
    unsigned high = (unsigned)block[2] | ((unsigned)block[3] << 8);
    for (int g = 0; g < 8; ++g) {
        unsigned low = (block[4 + g / 2] >> (4 * (g % 2))) & 15u;
        int scale = (int)(low | (((high >> (2 * g)) & 3u) << 4)) - 32;
        float multiplier = d * (float)scale;
        for (int j = 0; j < 16; ++j) {
            uint8_t byte = block[8 + g * 16 + j];
            out[g * 32 + j] = multiplier * (float)iq4_values[byte & 15];
            out[g * 32 + j + 16] = multiplier * (float)iq4_values[byte >> 4];
        }
    }
}

int orc_decode_row(uint32_t encoding, const uint8_t *bytes, size_t byte_count, float *out, size_t element_count) {
    int err = orc_validate_row(encoding, byte_count, element_count);
    if (err) return err;
    size_t elements = 1, block_bytes = 1;
    layout(encoding, &elements, &block_bytes);
    for (size_t offset = 0, o = 0; offset < byte_count; offset += block_bytes, o += elements) {
        const uint8_t *block = bytes + offset;
        switch (encoding) {
        case 0: memcpy(&out[o], block, 4); break;
        case 1: out[o] = half_at(block); break;
        case 8: {
            float scale = half_at(block);
            for (int j = 0; j < 32; ++j) out[o + j] = scale * (float)(int8_t)block[2 + j];
            break;
        }
        case 12: k_block(0, block, out + o); break;
        case 13: k_block(1, block, out + o); break;
        case 14: q6k_block(block, out + o); break;
        case 23: iq4xs_block(block, out + o); break;
        }
    }
    return ORC_OK;
}

/* encode.zig:17-36. */
int orc_q8_0_row(const float *input, size_t count, uint8_t *out, size_t out_len) {
    if (count == 0 || count % 32 != 0) return ORC_INVALID_ROW_LENGTH;
    if (out_len != count / 32 * 34) return ORC_INVALID_BYTE_LENGTH;
    for (size_t b = 0; b < count / 32; ++b) {
        const float *v = input + b * 32;
        uint8_t *block = out + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j)
            if (!isnan(v[j])) amax = fmaxf(amax, fabsf(v[j]));
        uint16_t dbits = orc_f32_to_half(amax / 127.0f);
        block[0] = (uint8_t)(dbits & 0xff);
        block[1] = (uint8_t)(dbits >> 8);
        float scale = orc_half_to_f32(dbits);
        for (int j = 0; j < 32; ++j) {
            float q;
            if (scale == 0.0f || !isfinite(scale) || isnan(v[j])) {
                q = 0.0f;
            } else {
                q = roundf(v[j] / scale); /* half away from zero, as Zig's @round */
                if (q < -127.0f) q = -127.0f;
                if (q > 127.0f) q = 127.0f;
            }
            block[2 + j] = (uint8_t)(int8_t)q;
        }
    }
    return ORC_OK;
}

int orc_default_threads(void) {
    /* cpu/root.zig:84-87: one task per core, at most 64 */
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    return n > 64 ? 64 : (int)n;
}

typedef struct {
    uint32_t encoding;
    size_t columns, row_bytes, rows, chunk;
    const uint8_t *bytes;
    const float *input;
    float *output;
    atomic_size_t *next;
} rows_job;

/* cpu/root.zig:144-152 (Rows.run): decode a row, widen both operands to F64,
 * sum in column order, round once. */
static void rows_run(const rows_job *job, size_t first, size_t last, float *decoded) {
    for (size_t r = first; r < last; ++r) {
        orc_decode_row(job->encoding, job->bytes + r * job->row_bytes, job->row_bytes, decoded, job->columns);
        double sum = 0.0;
        for (size_t c = 0; c < job->columns; ++c) sum += (double)decoded[c] * (double)job->input[c];
        job->output[r] = (float)sum;
    }
}

typedef struct {
    const rows_job *job;
    float *decoded;
} rows_task_arg;

/* cpu/root.zig:155-164 (Rows.task): pull chunks from an atomic counter. */
static void *rows_task(void *p) {
    rows_task_arg *arg = (rows_task_arg *)p;
    const rows_job *job = arg->job;
    for (;;) {
        size_t first = atomic_fetch_add(job->next, job->chunk);
        if (first >= job->rows) return NULL;
        size_t last = first + job->chunk < job->rows ? first + job->chunk : job->rows;
        rows_run(job, first, last, arg->decoded);
    }
}

/* cpu/root.zig:112-135 (matvec): validation before any write, then the rows
 * split across at most `threads` tasks in chunks of rows/(tasks*8). The
 * result does not depend on the split. */
int orc_matvec(uint32_t encoding, size_t rows, size_t columns, const uint8_t *bytes, size_t byte_len,
               const float *input, size_t input_len, float *output, size_t output_len, int threads) {
    if (rows == 0 || columns == 0 || input_len != columns || output_len != rows) return ORC_INVALID_SHAPE;
    if (byte_len % rows != 0) return ORC_INVALID_BYTE_LENGTH;
    size_t row_bytes = byte_len / rows;
    int err = orc_validate_row(encoding, row_bytes, columns);
    if (err) return err;
    if (threads < 1) threads = orc_default_threads();
    size_t tasks = (rows * columns < (1u << 16)) ? 1 : (size_t)threads;
    if (tasks > rows) tasks = rows;
    atomic_size_t next = 0;
    size_t chunk = rows / (tasks * 8);
    if (chunk < 1) chunk = 1;
    rows_job job = {encoding, columns, row_bytes, rows, chunk, bytes, input, output, &next};
    float *scratch = (float *)malloc(sizeof(float) * columns * tasks);
    if (!scratch) return ORC_INVALID_SHAPE;
    if (tasks == 1) {
        rows_run(&job, 0, rows, scratch);
    } else {
        pthread_t tid[64];
        rows_task_arg args[64];
        size_t spawned = 0;
        for (size_t t = 0; t < tasks; ++t) {
            args[t].job = &job;
            args[t].decoded = scratch + t * columns;
            if (pthread_create(&tid[t], NULL, rows_task, &args[t]) == 0) spawned++;
            else break;
        }
        if (spawned == 0) rows_task(&args[0]);
        for (size_t t = 0; t < spawned; ++t) pthread_join(tid[t], NULL);
    }
    free(scratch);
    return ORC_OK;
}

/* Batched product as the reference checks it: one matvec per token row
 * (metal-check.zig:4410-4424). */
int orc_matmul(uint32_t encoding, size_t rows, size_t columns, const uint8_t *bytes, size_t byte_len,
               const float *input, size_t in_stride, float *output, size_t out_stride, size_t tokens,
               int threads) {
    if (tokens == 0 || in_stride < columns || out_stride < rows) return ORC_INVALID_SHAPE;
    for (size_t t = 0; t < tokens; ++t) {
        int err = orc_matvec(encoding, rows, columns, bytes, byte_len, input + t * in_stride, columns,
                             output + t * out_stride, rows, threads);
        if (err) return err;
    }
    return ORC_OK;
}

/* sampling/root.zig:226-239: first index of the maximum (strict `>`), any
 * non-finite value is an error. */
int orc_argmax(const float *logits, size_t count, size_t *index) {
    if (count == 0) return ORC_INVALID_SHAPE;
    size_t best = 0;
    float best_value = 0.0f;
    for (size_t i = 0; i < count; ++i) {
        float v = logits[i];
        if (!isfinite(v)) return ORC_NON_FINITE;
        if (i == 0 || v > best_value) {
            best = i;
            best_value = v;
        }
    }
    *index = best;
    return ORC_OK;
}

/* Sampler.penalize (inference/src/sampling/root.zig:375-381) for every id:
 * ids in the history bit set (bit id of word id / 32) get l / r for l > 0,
 * else l * r, then minus presence; the others are copied. */
int orc_penalize(const float *logits, size_t count, const uint32_t *history, size_t words, float repetition,
                 float presence, float *out) {
    if (count == 0 || words < (count + 31) / 32) return ORC_INVALID_SHAPE;
    for (size_t i = 0; i < count; ++i) {
        const float value = logits[i];
        if (!(history[i / 32] & (1u << (i % 32)))) {
            out[i] = value;
            continue;
        }
        const float scaled = value > 0 ? value / repetition : value * repetition;
        out[i] = scaled - presence;
    }
    return ORC_OK;
}

typedef struct {
    uint32_t id;
    float weight;
} orc_candidate;

/* Sampler.lessThan (sampling/root.zig:385-387): weight descending, id ascending. */
static int orc_candidate_order(const void *pa, const void *pb) {
    const orc_candidate *a = (const orc_candidate *)pa, *b = (const orc_candidate *)pb;
    if (a->weight > b->weight) return -1;
    if (a->weight < b->weight) return 1;
    return a->id < b->id ? -1 : (a->id > b->id ? 1 : 0);
}

/* The readback a correct device produces (referenceTopK, sampling/root.zig:
 * 701-715, with the device's non-finite rule of kernels/sampling.metal:58-67):
 * the first k of the reference sort over the non-NaN logits, padded with
 * (-inf, 0xffffffff) when fewer remain; total = sum over every logit of
 * exp((l - max) / T) in F64 with max the first value; finite = no logit is
 * NaN or infinite. */
int orc_topk(const float *logits, size_t count, size_t k, float temperature, uint32_t *ids, float *values,
             double *total, int *finite) {
    if (count == 0 || k == 0 || k > count) return ORC_INVALID_SHAPE;
    orc_candidate *c = (orc_candidate *)malloc(count * sizeof *c);
    if (!c) return ORC_INVALID_SHAPE;
    size_t n = 0;
    int all_finite = 1;
    for (size_t i = 0; i < count; ++i) {
        if (!isfinite(logits[i])) all_finite = 0;
        if (isnan(logits[i])) continue;
        c[n].id = (uint32_t)i;
        c[n].weight = logits[i];
        ++n;
    }
    qsort(c, n, sizeof *c, orc_candidate_order);
    for (size_t r = 0; r < k; ++r) {
        ids[r] = r < n ? c[r].id : 0xffffffffu;
        values[r] = r < n ? c[r].weight : -INFINITY;
    }
    const double maximum = values[0];
    double sum = 0.0;
    for (size_t i = 0; i < count; ++i) sum += exp(((double)logits[i] - maximum) / (double)temperature);
    *total = sum;
    *finite = all_finite;
    free(c);
    return ORC_OK;
}

/*
 * CPU oracle for the quantized-weight matmul path. TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of nuclis's CPU reference for the GGUF
 * dequantize-and-multiply path. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker. The
 * product (nuclis_amd/libnuq.so) never links, loads or calls it.
 *
 * Reference functions restated (paths relative to the nuclis tree):
 *   orc_half_to_f32      inference/src/quant/decode.zig:432-435   (half)
 *   orc_f32_to_half      the f32 -> f16 narrowing Zig's @floatCast performs
 *                        in inference/src/quant/encode.zig:29 (round to
 *                        nearest even, overflow to infinity)
 *   orc_validate_row     inference/src/quant/decode.zig:108-120  (validateRow)
 *   orc_decode_row       inference/src/quant/decode.zig:30-106   (row), arms
 *                        0 (F32), 1 (F16), 8 (Q8_0, :57-63), 12 (Q4_K) and
 *                        13 (Q5_K) (kBlock :147-170), 14 (Q6_K, q6Block
 *                        :198-211) and 23 (IQ4_XS, iq4XsBlock :213-228 with
 *                        the iq4_values table :437)
 *   orc_q8_0_row         inference/src/quant/encode.zig:17-36    (q8_0Row)
 *   orc_matvec           inference/src/backends/cpu/root.zig:97-165 (matvec,
 *                        Rows.run, Rows.task)
 *   orc_matmul           M independent matvecs: the reference's oracle form
 *                        for batched products (inference/metal-check.zig:4410-4424)
 *   orc_argmax           inference/src/sampling/root.zig:226-239 (first
 *                        maximum wins, a non-finite logit is an error)
 *   orc_penalize         inference/src/sampling/root.zig:375-381 (penalize)
 *                        over a history bit set (History.writeWords layout)
 *   orc_topk             the readback referenceTopK builds
 *                        (inference/src/sampling/root.zig:701-715: the
 *                        Sampler.lessThan sort, F64 exp-sum) with the device
 *                        rule that NaN never enters the list
 *                        (backends/metal/kernels/sampling.metal:58-67)
 *
 * Every function is pinned by tests/test_oracle.py against the llama.cpp
 * fixtures the reference holds (tests/golden/), the reference's own
 * known-answer tests, and independent closed forms (numpy's float16 for the
 * half conversions, brute-force f64 sums for matvec).
 */
#ifndef NUCLIS_ORACLE_H
#define NUCLIS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_INVALID_SHAPE = 1,
    ORC_UNSUPPORTED_ENCODING = 2,
    ORC_INVALID_ROW_LENGTH = 3,
    ORC_INVALID_BYTE_LENGTH = 4,
    ORC_NON_FINITE = 5,
};

float orc_half_to_f32(uint16_t bits);
uint16_t orc_f32_to_half(float value);
int orc_validate_row(uint32_t encoding, size_t byte_count, size_t element_count);
int orc_decode_row(uint32_t encoding, const uint8_t *bytes, size_t byte_count, float *out, size_t element_count);
int orc_q8_0_row(const float *input, size_t count, uint8_t *out, size_t out_len);
int orc_matvec(uint32_t encoding, size_t rows, size_t columns, const uint8_t *bytes, size_t byte_len,
               const float *input, size_t input_len, float *output, size_t output_len, int threads);
int orc_matmul(uint32_t encoding, size_t rows, size_t columns, const uint8_t *bytes, size_t byte_len,
               const float *input, size_t in_stride, float *output, size_t out_stride, size_t tokens,
               int threads);
int orc_argmax(const float *logits, size_t count, size_t *index);
int orc_penalize(const float *logits, size_t count, const uint32_t *history, size_t words, float repetition,
                 float presence, float *out);
int orc_topk(const float *logits, size_t count, size_t k, float temperature, uint32_t *ids, float *values,
             double *total, int *finite);
int orc_default_threads(void);

#ifdef __cplusplus
}
#endif
#endif

// Launchers shared between the kernel translation units and the C-ABI shim.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nuq {

struct SegmentDesc {
    const uint8_t *w;
    uint64_t stride;
    float *out;
    uint32_t encoding;
    uint32_t rows;
    uint32_t nblocks;
    uint32_t pad;
};

struct SegmentsArgs {
    SegmentDesc seg[4];
    uint32_t wave_start[5];  // prefix sums of each segment's wave count
    uint32_t count;
    uint32_t mode;  // 0 plain, 1 silu(seg0) * seg1
};

// Device workspace for the K-split partial tiles of the prefill kernel:
// room for `tiles` partial 256x256 F32 tiles.
struct SplitScratch {
    float *work;
    uint32_t tiles;
};

hipError_t launch_dequant_rows(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint64_t first,
                               uint32_t count, uint32_t columns, float *out);
hipError_t launch_gemv(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const float *x, float *y, int rows_per_wave);
hipError_t launch_gemv_q4k_int(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                               const float *x, float *y, int config);
// Up to GD_MAX_SEGMENTS matrices of one encoding and row stride against one
// x in one DMA GEMV launch (y[q] = W_q x). hipErrorInvalidValue when the
// shape does not fit it.
constexpr uint32_t GD_MAX_SEGMENTS = 4;
struct GdSegments {
    const uint8_t *w[GD_MAX_SEGMENTS];
    float *y[GD_MAX_SEGMENTS];
    uint32_t rows[GD_MAX_SEGMENTS];
    uint32_t rows_per_wg[GD_MAX_SEGMENTS];
    uint32_t wg_end[GD_MAX_SEGMENTS];
    uint32_t count;  // 0: one matrix, from the kernel's own arguments
};
hipError_t launch_gemv_dma_segments(hipStream_t s, uint32_t encoding, uint32_t count, const uint8_t *const *w,
                                    uint64_t stride, const uint32_t *rows, uint32_t columns, const float *x,
                                    float *const *y);
hipError_t launch_gemv_dma(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                           uint32_t columns, const float *x, float *y);
hipError_t launch_generic(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                          uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                          uint64_t out_stride, uint32_t tokens);
hipError_t launch_rows(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                       uint64_t out_stride, uint32_t tokens);
hipError_t launch_segments(hipStream_t s, const SegmentsArgs &args, const float *x);
int segment_rows_per_wave();
hipError_t launch_argmax(hipStream_t s, const float *logits, uint64_t count, uint32_t *result);
hipError_t launch_silu_mul(hipStream_t s, float *out, const float *up, uint32_t n);

// Device sampling (sampling.hip). The partial top-k keeps at most
// TOPK_CAPACITY entries of at most TOPK_MAX_COUNT logits and writes
// TOPK_PARTIALS exp-sum partials (backends/metal/ops/sampling.zig:15-22).
constexpr uint32_t TOPK_CAPACITY = 256, TOPK_PARTIALS = 64, TOPK_MAX_COUNT = TOPK_PARTIALS * 256 * 16;
uint64_t topk_scratch_keys();
hipError_t launch_penalize(hipStream_t s, float *logits, uint32_t count, const uint32_t *history, float repetition,
                           float presence);
hipError_t launch_topk(hipStream_t s, const float *logits, uint32_t count, uint32_t k, float temperature,
                       uint64_t *scratch, float *values, uint32_t *indices, float *sums, uint32_t *flags);
hipError_t launch_tile(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                       uint64_t out_stride, uint32_t tokens, const SplitScratch &scratch);
uint32_t split_scratch_tiles();
// Adds `ranges` K-range partial outputs ws[(k * tokens + t) * rows + r] in
// range order into y[t * out_stride + r].
hipError_t launch_verify_reduce(hipStream_t s, const float *ws, uint32_t ranges, uint32_t rows, uint32_t tokens,
                                float *y, uint64_t out_stride);
// Register-dequant multi-token GEMV (KERNEL_ROWS) for Q4_K with f16
// activations, 1..8 tokens; `ws` (ws_floats floats) takes the K ranges of
// rows longer than 24 blocks. False (nothing launched) for shapes it does
// not take; otherwise *err is the launch status.
bool launch_rows_q4k_f16(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                         const _Float16 *x, uint64_t in_stride, float *y, uint64_t out_stride, uint32_t tokens,
                         float *ws, uint64_t ws_floats, hipError_t *err);
// Multi-token GEMV of F32 activations (1..4 tokens) at F32 precision on the
// matrix cores (the streamed verify tile with each token's activations as
// three f16 parts); Q4_K / Q5_K. *taken is false (and nothing launched)
// for shapes it does not take; otherwise the launch's own status returns.
hipError_t launch_rows_mfma(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                            uint32_t columns, const float *x, uint64_t in_stride, float *y, uint64_t out_stride,
                            uint32_t tokens, const SplitScratch &scratch, bool *taken);
// F32 workspace the tile route of this call would use (verify K ranges or
// prefill split partials); 0 when it needs none. A smaller workspace makes
// the route fall back (fewer splits, or the register verify tile).
uint64_t tile_workspace_floats(uint32_t encoding, uint32_t rows, uint32_t columns, uint32_t tokens,
                               uint64_t in_stride, bool xs3 = false);

}  // namespace nuq

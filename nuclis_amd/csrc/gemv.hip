// Decode-side kernels: bit-exact dequantisation, the M=1 GEMV for Q4_K /
// Q6_K / Q8_0, the multi-token register-dequant GEMV (M = 2..8), the merged
// segments GEMV and the greedy argmax. All are HBM-bound integer/FP32 work on
// wave64: no MFMA.
//
// GEMV geometry (one wave = 64 lanes; a workgroup = 4 waves):
//   each wave owns R consecutive weight rows and walks the whole K range.
//   Q4_K: 8 lanes per 144-byte block, each lane one 16-byte qs chunk (32
//         values: 16 of group 2j and 16 of group 2j+1) -> 8 blocks in flight
//         per row per wave, coalesced 16-byte loads.
//   Q6_K: 16 lanes per 210-byte block, each lane 16 values (4 columns x 4
//         quarters) from three dwords of ql/qh -> 4 blocks per row per wave.
//   Q8_0: 4 lanes per 34-byte block, each lane 8 int8 codes.
// A lane holds its x slice in registers and reuses it for all R rows, so x
// is read from L1/L2 once per R rows. Per-group sums of x fold the Q4_K
// minimum and the Q6_K -32 bias out of the inner loop:
//   sum_i (d*sc*q_i - dmin*m) x_i = d*sc*sum_i q_i x_i - dmin*m*sum_i x_i.
// The result differs from the CPU reference only by FP32 rounding order.
#include "formats.h"
#include "kernels.h"

namespace nuq {

__device__ __forceinline__ float wave_sum(float v) {
    // Butterfly over the 64 lanes; every lane ends with the total.
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Bit-exact dequantisation (Backend.embed, ops/rowwise.zig:17-25). One thread
// per 16 consecutive values of a row.
__global__ void __launch_bounds__(256) dequant_rows_kernel(uint32_t encoding, const uint8_t *__restrict__ w,
                                                            uint64_t stride, uint32_t block_values,
                                                            uint32_t block_bytes, uint64_t first, uint32_t count,
                                                            uint32_t columns, float *__restrict__ out) {
    uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t segments = columns / 16;
    if (t >= (uint64_t)count * segments) return;
    uint32_t r = (uint32_t)(t / segments);
    uint32_t c0 = (uint32_t)(t % segments) * 16;
    const uint8_t *row = w + (first + r) * stride;
    float *o = out + (uint64_t)r * columns + c0;
    uint32_t block = c0 / block_values;
    const uint8_t *b = row + (uint64_t)block * block_bytes;
    uint32_t i0 = c0 % block_values;
#pragma unroll 4
    for (uint32_t k = 0; k < 16; ++k) o[k] = decode_value(encoding, b, i0 + k);
}

// ---------------------------------------------------------------------------
// Q4_K. A half-wave (32 lanes) covers 4 consecutive blocks of R rows: lane
// (slot, c) holds 16-byte qs chunk c of block slot, i.e. columns 16*(c&1)..+16
// of groups 2j and 2j+1 (j = c>>1), whose low / high nibbles share the bytes.
// The two half-waves of a wave take different rows and the same columns, so
// every block count that is a multiple of 4 (20, 24, 68 at the configs)
// keeps all lanes busy. High nibbles are converted in place (x16) and the
// 1/16 folded into their scale, so each value costs one v_cvt_f32_ubyteN and
// one FMA.

// Pair (sa, ma, sb, mb) of six-bit scales/minima for groups 2j, 2j+1 without
// branches (lanes of one wave take both forms): quant/decode.zig:155-158.
struct PairShift {
    uint32_t shift;
    bool direct;
};

__device__ __forceinline__ void q4k_pair(uint32_t s0, uint32_t s1, uint32_t s2, PairShift ps, float *sa, float *ma,
                                         float *sb, float *mb) {
    const uint32_t x = s0 >> ps.shift, y = s1 >> ps.shift, z = s2 >> ps.shift;
    const uint32_t a = ps.direct ? (x & 63u) : ((z & 15u) | (((x >> 6) & 3u) << 4));
    const uint32_t m = ps.direct ? (y & 63u) : (((z >> 4) & 15u) | (((y >> 6) & 3u) << 4));
    const uint32_t b = ps.direct ? ((x >> 8) & 63u) : (((z >> 8) & 15u) | (((x >> 14) & 3u) << 4));
    const uint32_t n = ps.direct ? ((y >> 8) & 63u) : (((z >> 12) & 15u) | (((y >> 14) & 3u) << 4));
    *sa = (float)a;
    *ma = (float)m;
    *sb = (float)b;
    *mb = (float)n;
}

__device__ __forceinline__ PairShift pair_shift(uint32_t j) {
    PairShift p;
    p.direct = j < 2;
    p.shift = p.direct ? 16 * j : 16 * j - 32;
    return p;
}

// Low nibbles against xa, high nibbles (kept at x16) against xb.
__device__ __forceinline__ void q4k_dot16(const uint4 qs, const float *xa, const float *xb, float *lo_out,
                                          float *hi_out) {
    const uint32_t words[4] = {qs.x, qs.y, qs.z, qs.w};
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t l4 = opaque_and<0x0f0f0f0fu>(words[k]);
        const uint32_t h4 = opaque_and<0xf0f0f0f0u>(words[k]);
        lo = fmaf(ubyte_f<0>(l4), xa[4 * k + 0], lo);
        lo = fmaf(ubyte_f<1>(l4), xa[4 * k + 1], lo);
        lo = fmaf(ubyte_f<2>(l4), xa[4 * k + 2], lo);
        lo = fmaf(ubyte_f<3>(l4), xa[4 * k + 3], lo);
        hi = fmaf(ubyte_f<0>(h4), xb[4 * k + 0], hi);
        hi = fmaf(ubyte_f<1>(h4), xb[4 * k + 1], hi);
        hi = fmaf(ubyte_f<2>(h4), xb[4 * k + 2], hi);
        hi = fmaf(ubyte_f<3>(h4), xb[4 * k + 3], hi);
    }
    *lo_out = lo;
    *hi_out = hi;
}

__device__ __forceinline__ float q4k_chunk_dot(const uint4 hdr, const uint4 qs, const float *xa, const float *xb,
                                               float sxa, float sxb, PairShift ps) {
    float d = half_bits(hdr.x & 0xffffu);
    float dmin = half_bits(hdr.x >> 16);
    float sa, ma, sb, mb;
    q4k_pair(hdr.y, hdr.z, hdr.w, ps, &sa, &ma, &sb, &mb);
    float lo, hi;
    q4k_dot16(qs, xa, xb, &lo, &hi);
    float r = (d * sa) * lo + (d * sb * 0.0625f) * hi;
    return r - dmin * (ma * sxa + mb * sxb);
}

__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
    for (int offset = 16; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

template <int R>
__global__ void __launch_bounds__(256) gemv_q4k_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                        uint32_t nblocks, const float *__restrict__ x,
                                                        float *__restrict__ y) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (wave * 2 * R >= rows) return;
    const uint32_t rg = lane >> 5, slot = (lane >> 3) & 3, c = lane & 7;
    const uint32_t j = c >> 1, half16 = (c & 1) * 16;
    const uint32_t row0 = wave * 2 * R + rg * R;
    const PairShift ps = pair_shift(j);
    const uint8_t *hp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) hp[r] = w + (uint64_t)min(row0 + r, rows - 1) * stride + slot * 144;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;

    uint4 hdr[R], qs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        hdr[r] = *(const uint4 *)hp[r];
        qs[r] = *(const uint4 *)(hp[r] + 16 + c * 16);
    }
    for (uint32_t b = slot; b < nblocks; b += 4) {
        const float *xp = x + b * 256 + j * 64 + half16;
        float xa[16], xb[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float4 a = *(const float4 *)(xp + 4 * k);
            float4 bb = *(const float4 *)(xp + 32 + 4 * k);
            xa[4 * k] = a.x; xa[4 * k + 1] = a.y; xa[4 * k + 2] = a.z; xa[4 * k + 3] = a.w;
            xb[4 * k] = bb.x; xb[4 * k + 1] = bb.y; xb[4 * k + 2] = bb.z; xb[4 * k + 3] = bb.w;
        }
        // prefetch the next block of every row before computing this one
        uint4 nhdr[R], nqs[R];
        const bool more = b + 4 < nblocks;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            hp[r] += 4 * 144;
            if (more) {
                nhdr[r] = *(const uint4 *)hp[r];
                nqs[r] = *(const uint4 *)(hp[r] + 16 + c * 16);
            }
        }
        float sxa = ((xa[0] + xa[1]) + (xa[2] + xa[3])) + ((xa[4] + xa[5]) + (xa[6] + xa[7])) +
                    (((xa[8] + xa[9]) + (xa[10] + xa[11])) + ((xa[12] + xa[13]) + (xa[14] + xa[15])));
        float sxb = ((xb[0] + xb[1]) + (xb[2] + xb[3])) + ((xb[4] + xb[5]) + (xb[6] + xb[7])) +
                    (((xb[8] + xb[9]) + (xb[10] + xb[11])) + ((xb[12] + xb[13]) + (xb[14] + xb[15])));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += q4k_chunk_dot(hdr[r], qs[r], xa, xb, sxa, sxb, ps);
        if (more) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                hdr[r] = nhdr[r];
                qs[r] = nqs[r];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v = half_wave_sum(acc[r]);
        if ((lane & 31) == 0 && row0 + r < rows) y[row0 + r] = v;
    }
}

// ---------------------------------------------------------------------------
// Q6_K: lane = (half h, column quad l4) of a block; 16 lanes per block.
__device__ __forceinline__ float q6k_lane_dot(const uint8_t *blk, uint32_t h, uint32_t l, const float (*xq)[4],
                                              const float *sxq) {
    uint32_t ql0 = load_u32_unaligned(blk + h * 64 + l);       // quarters 0 (low) and 2 (high nibble)
    uint32_t ql1 = load_u32_unaligned(blk + h * 64 + 32 + l);  // quarters 1 and 3
    uint32_t qh = load_u32_unaligned(blk + 128 + h * 32 + l);
    // scales sc[h*8 + 2q + (l >= 16)], q = 0..3: bytes at even/odd positions
    uint32_t s0 = load_u32_unaligned(blk + 192 + h * 8);
    uint32_t s1 = load_u32_unaligned(blk + 196 + h * 8);
    uint32_t d16 = (uint32_t)load_u16_bytes(blk + 208);
    float d = half_bits(d16);
    uint32_t odd = (l >= 16) ? 8u : 0u;
    int sc[4];
    sc[0] = (int8_t)((s0 >> odd) & 0xff);
    sc[1] = (int8_t)((s0 >> (16 + odd)) & 0xff);
    sc[2] = (int8_t)((s1 >> odd) & 0xff);
    sc[3] = (int8_t)((s1 >> (16 + odd)) & 0xff);
    float total = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t low = ((q & 1) ? ql1 : ql0);
        low = (q >= 2 ? (low >> 4) : low) & 0x0f0f0f0fu;
        uint32_t u = low | (((qh >> (2 * q)) & 0x03030303u) << 4);
        float s = ubyte_f<0>(u) * xq[q][0];
        s = fmaf(ubyte_f<1>(u), xq[q][1], s);
        s = fmaf(ubyte_f<2>(u), xq[q][2], s);
        s = fmaf(ubyte_f<3>(u), xq[q][3], s);
        s = fmaf(-32.f, sxq[q], s);
        total = fmaf((float)sc[q], s, total);
    }
    return d * total;
}

template <int R>
__global__ void __launch_bounds__(256) gemv_q6k_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                        uint32_t nblocks, const float *__restrict__ x,
                                                        float *__restrict__ y) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t row0 = wave * R;
    if (row0 >= rows) return;
    const uint32_t slot = lane >> 4, h = (lane >> 3) & 1, l = (lane & 7) * 4;
    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowp[r] = w + (uint64_t)min(row0 + r, rows - 1) * stride;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (uint32_t b = slot; b < nblocks; b += 4) {
        float xq[4][4], sxq[4];
        const float *xp = x + b * 256 + h * 128 + l;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float4 v = *(const float4 *)(xp + q * 32);
            xq[q][0] = v.x; xq[q][1] = v.y; xq[q][2] = v.z; xq[q][3] = v.w;
            sxq[q] = (v.x + v.y) + (v.z + v.w);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += q6k_lane_dot(rowp[r] + (uint64_t)b * 210, h, l, xq, sxq);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < rows) y[row0 + r] = v;
    }
}

// ---------------------------------------------------------------------------
// Q8_0: lane = quarter k of a block (8 codes); 16 blocks per wave step.
// Codes are biased to unsigned bytes (q ^ 0x80 = q + 128) so one
// v_cvt_f32_ubyte converts each; the bias is removed with the slice sum of x.
__device__ __forceinline__ float q8_lane_dot(const uint8_t *blk, uint32_t k, const float *xv, float sx) {
    float d = half_bits(load_u16_bytes(blk));
    uint32_t q0 = load_u32_unaligned(blk + 2 + 8 * k) ^ 0x80808080u;
    uint32_t q1 = load_u32_unaligned(blk + 6 + 8 * k) ^ 0x80808080u;
    float s = ubyte_f<0>(q0) * xv[0];
    s = fmaf(ubyte_f<1>(q0), xv[1], s);
    s = fmaf(ubyte_f<2>(q0), xv[2], s);
    s = fmaf(ubyte_f<3>(q0), xv[3], s);
    s = fmaf(ubyte_f<0>(q1), xv[4], s);
    s = fmaf(ubyte_f<1>(q1), xv[5], s);
    s = fmaf(ubyte_f<2>(q1), xv[6], s);
    s = fmaf(ubyte_f<3>(q1), xv[7], s);
    s = fmaf(-128.f, sx, s);
    return d * s;
}

template <int R>
__global__ void __launch_bounds__(256) gemv_q8_0_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                         uint32_t nblocks, const float *__restrict__ x,
                                                         float *__restrict__ y) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t row0 = wave * R;
    if (row0 >= rows) return;
    const uint32_t slot = lane >> 2, k = lane & 3;
    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowp[r] = w + (uint64_t)min(row0 + r, rows - 1) * stride;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (uint32_t b = slot; b < nblocks; b += 16) {
        const float *xp = x + b * 32 + 8 * k;
        float4 a = *(const float4 *)xp, c = *(const float4 *)(xp + 4);
        float xv[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        float sx = ((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += q8_lane_dot(rowp[r] + (uint64_t)b * 34, k, xv, sx);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < rows) y[row0 + r] = v;
    }
}

// ---------------------------------------------------------------------------
// Generic control (the reference's nu_matvec, kernels/matvec.metal:4-21): one
// wave per row, exact scalar decode of each value, F32 activations of any
// alignment, T tokens. Serves misaligned weights and the generic_only mode.
__global__ void __launch_bounds__(256) generic_rows_kernel(uint32_t encoding, const uint8_t *__restrict__ w,
                                                            uint64_t stride, uint32_t rows, uint32_t columns,
                                                            uint32_t block_values, uint32_t block_bytes,
                                                            const void *__restrict__ x, uint32_t x_f16,
                                                            uint64_t in_stride, float *__restrict__ y,
                                                            uint64_t out_stride, uint32_t tokens) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint8_t *rowp = w + (uint64_t)row * stride;
    for (uint32_t t = 0; t < tokens; ++t) {
        float acc = 0.f;
        for (uint32_t col = lane; col < columns; col += 64) {
            float wv = decode_value(encoding, rowp + (uint64_t)(col / block_values) * block_bytes, col % block_values);
            float xv = x_f16 ? __half2float(((const __half *)x)[t * in_stride + col])
                             : ((const float *)x)[t * in_stride + col];
            acc = fmaf(wv, xv, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) y[t * out_stride + row] = acc;
    }
}

// ---------------------------------------------------------------------------
// Multi-token register-dequant GEMV (Backend.matvecRows, ops/matvec.zig:149).
// One wave per row; lanes hold 32 decoded Q4_K values (or 16 Q6_K / 8 Q8_0)
// of a block in registers and dot them with every token's x slice, so each
// weight byte is read once for all T tokens.
template <typename XT>
__device__ __forceinline__ float load_x(const XT *p);
template <>
__device__ __forceinline__ float load_x<float>(const float *p) { return *p; }
template <>
__device__ __forceinline__ float load_x<__half>(const __half *p) { return __half2float(*p); }

template <int T, typename XT>
__global__ void __launch_bounds__(256) rows_q4k_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                        uint32_t nblocks, const XT *__restrict__ x, uint64_t in_stride,
                                                        float *__restrict__ y, uint64_t out_stride) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t c = lane & 7, slot = lane >> 3;
    const uint32_t j = c >> 1, half16 = (c & 1) * 16;
    const uint8_t *rowp = w + (uint64_t)row * stride;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
    for (uint32_t b = slot; b < nblocks; b += 8) {
        const uint8_t *blk = rowp + (uint64_t)b * 144;
        uint4 hdr = *(const uint4 *)blk;
        uint4 qs = *(const uint4 *)(blk + 16 + c * 16);
        float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * j, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        q4k_scale_min(2 * j + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        float mul0 = d * (float)sc0, off0 = dmin * (float)m0;
        float mul1 = d * (float)sc1, off1 = dmin * (float)m1;
        float wa[16], wb[16];
        const uint32_t words[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wa[4 * k + e] = fmaf(mul0, (float)((words[k] >> (8 * e)) & 15u), -off0);
                wb[4 * k + e] = fmaf(mul1, (float)((words[k] >> (8 * e + 4)) & 15u), -off1);
            }
        }
        const uint32_t col = b * 256 + j * 64 + half16;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const XT *xp = x + t * in_stride + col;
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                s = fmaf(wa[k], load_x<XT>(xp + k), s);
                s = fmaf(wb[k], load_x<XT>(xp + 32 + k), s);
            }
            acc[t] += s;
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float v = wave_sum(acc[t]);
        if (lane == 0) y[t * out_stride + row] = v;
    }
}

template <int T, typename XT>
__global__ void __launch_bounds__(256) rows_q6k_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                        uint32_t nblocks, const XT *__restrict__ x, uint64_t in_stride,
                                                        float *__restrict__ y, uint64_t out_stride) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t slot = lane >> 4, h = (lane >> 3) & 1, l = (lane & 7) * 4;
    const uint8_t *rowp = w + (uint64_t)row * stride;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
    for (uint32_t b = slot; b < nblocks; b += 4) {
        const uint8_t *blk = rowp + (uint64_t)b * 210;
        uint32_t ql0 = load_u32_unaligned(blk + h * 64 + l);
        uint32_t ql1 = load_u32_unaligned(blk + h * 64 + 32 + l);
        uint32_t qh = load_u32_unaligned(blk + 128 + h * 32 + l);
        uint32_t s0 = load_u32_unaligned(blk + 192 + h * 8);
        uint32_t s1 = load_u32_unaligned(blk + 196 + h * 8);
        float d = half_bits(load_u16_bytes(blk + 208));
        uint32_t odd = (l >= 16) ? 8u : 0u;
        float wv[4][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t sw = (q < 2) ? s0 : s1;
            float mul = d * (float)(int8_t)((sw >> (16 * (q & 1) + odd)) & 0xff);
            uint32_t low = ((q & 1) ? ql1 : ql0);
            low = (q >= 2 ? (low >> 4) : low) & 0x0f0f0f0fu;
            uint32_t u = low | (((qh >> (2 * q)) & 0x03030303u) << 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) wv[q][e] = mul * (float)((int)((u >> (8 * e)) & 0xffu) - 32);
        }
        const uint32_t col = b * 256 + h * 128 + l;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const XT *xp = x + t * in_stride + col;
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) s = fmaf(wv[q][e], load_x<XT>(xp + q * 32 + e), s);
            acc[t] += s;
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float v = wave_sum(acc[t]);
        if (lane == 0) y[t * out_stride + row] = v;
    }
}

template <int T, typename XT>
__global__ void __launch_bounds__(256) rows_q8_0_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                         uint32_t nblocks, const XT *__restrict__ x,
                                                         uint64_t in_stride, float *__restrict__ y,
                                                         uint64_t out_stride) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint32_t slot = lane >> 2, k = lane & 3;
    const uint8_t *rowp = w + (uint64_t)row * stride;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
    for (uint32_t b = slot; b < nblocks; b += 16) {
        const uint8_t *blk = rowp + (uint64_t)b * 34;
        float d = half_bits(load_u16_bytes(blk));
        uint32_t q0 = load_u32_unaligned(blk + 2 + 8 * k);
        uint32_t q1 = load_u32_unaligned(blk + 6 + 8 * k);
        float wv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            wv[e] = d * (float)(int8_t)((q0 >> (8 * e)) & 0xff);
            wv[4 + e] = d * (float)(int8_t)((q1 >> (8 * e)) & 0xff);
        }
        const uint32_t col = b * 32 + 8 * k;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const XT *xp = x + t * in_stride + col;
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf(wv[e], load_x<XT>(xp + e), s);
            acc[t] += s;
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float v = wave_sum(acc[t]);
        if (lane == 0) y[t * out_stride + row] = v;
    }
}

// ---------------------------------------------------------------------------
// Greedy argmax (sampling/root.zig:226-239): the first index of the maximum;
// a non-finite logit is reported through a flag. Single workgroup of 1024
// threads; each keeps the best (value, lowest index) of its strided slice,
// then a tree reduction prefers the larger value, the lower index on ties.
__global__ void __launch_bounds__(1024) argmax_kernel(const float *__restrict__ logits, uint64_t count,
                                                      uint32_t *__restrict__ result) {
    __shared__ float best_v[1024];
    __shared__ uint32_t best_i[1024];
    __shared__ uint32_t bad[1024];
    const uint32_t t = threadIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    uint32_t nonfinite = 0;
    for (uint64_t i = t; i < count; i += blockDim.x) {
        float v = logits[i];
        if (!isfinite(v)) nonfinite = 1;
        if (bi == 0xffffffffu || v > bv) {
            bv = v;
            bi = (uint32_t)i;
        }
    }
    best_v[t] = bv;
    best_i[t] = bi;
    bad[t] = nonfinite;
    __syncthreads();
    for (uint32_t s = blockDim.x / 2; s > 0; s >>= 1) {
        if (t < s) {
            float ov = best_v[t + s];
            uint32_t oi = best_i[t + s];
            if (oi != 0xffffffffu &&
                (best_i[t] == 0xffffffffu || ov > best_v[t] || (ov == best_v[t] && oi < best_i[t]))) {
                best_v[t] = ov;
                best_i[t] = oi;
            }
            bad[t] |= bad[t + s];
        }
        __syncthreads();
    }
    if (t == 0) {
        result[0] = best_i[0];
        result[1] = bad[0];
    }
}

// ---------------------------------------------------------------------------
// Merged segments GEMV (Backend.matvecSegments, ops/matvec.zig:245-343): up
// to four Q4_K/Q6_K/Q8_0 projections that share one input in one launch. The
// wave index is mapped to (segment, row group) through prefix sums of each
// segment's row-group count. In SILU_MUL_PAIR mode a wave computes row r of
// both segments and writes silu(a) * b.
template <int R>
__device__ __forceinline__ void gemv_rows_any(uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                                              uint32_t nblocks, const float *x, uint32_t row0, float *out_acc) {
    const uint32_t lane = threadIdx.x & 63;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowp[r] = w + (uint64_t)min(row0 + r, rows - 1) * stride;
    if (encoding == 12) {
        const uint32_t c = lane & 7, slot = lane >> 3, j = c >> 1, half16 = (c & 1) * 16;
        for (uint32_t b = slot; b < nblocks; b += 8) {
            const float *xp = x + b * 256 + j * 64 + half16;
            float xa[16], xb[16], sxa = 0.f, sxb = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                xa[k] = xp[k];
                xb[k] = xp[32 + k];
                sxa += xa[k];
                sxb += xb[k];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t *blk = rowp[r] + (uint64_t)b * 144;
                acc[r] += q4k_chunk_dot(*(const uint4 *)blk, *(const uint4 *)(blk + 16 + c * 16), xa, xb, sxa, sxb, pair_shift(j));
            }
        }
    } else if (encoding == 14) {
        const uint32_t slot = lane >> 4, h = (lane >> 3) & 1, l = (lane & 7) * 4;
        for (uint32_t b = slot; b < nblocks; b += 4) {
            float xq[4][4], sxq[4];
            const float *xp = x + b * 256 + h * 128 + l;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 v = *(const float4 *)(xp + q * 32);
                xq[q][0] = v.x; xq[q][1] = v.y; xq[q][2] = v.z; xq[q][3] = v.w;
                sxq[q] = (v.x + v.y) + (v.z + v.w);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] += q6k_lane_dot(rowp[r] + (uint64_t)b * 210, h, l, xq, sxq);
        }
    } else if (encoding != 8) {
        // Q5_K / IQ4_XS (256-value blocks): exact decode, 4 values per lane per pass
        Layout l;
        layout_of(encoding, &l);
        for (uint32_t c0 = 4 * lane; c0 < nblocks * 256; c0 += 256) {
            const uint32_t blk = c0 / 256, i = c0 % 256;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t *bp = rowp[r] + (uint64_t)blk * l.bytes;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[r] = fmaf(decode_value(encoding, bp, i + e), x[c0 + e], acc[r]);
            }
        }
    } else {
        const uint32_t slot = lane >> 2, k = lane & 3;
        for (uint32_t b = slot; b < nblocks; b += 16) {
            const float *xp = x + b * 32 + 8 * k;
            float4 a = *(const float4 *)xp, c = *(const float4 *)(xp + 4);
            float xv[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            float sx = ((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w));
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] += q8_lane_dot(rowp[r] + (uint64_t)b * 34, k, xv, sx);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) out_acc[r] = wave_sum(acc[r]);
}

constexpr int SEG_ROWS = 2;

__global__ void __launch_bounds__(256) segments_kernel(SegmentsArgs args, const float *__restrict__ x) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (args.mode == 0) {
        uint32_t s = 0;
        while (s + 1 < args.count && wave >= args.wave_start[s + 1]) ++s;
        if (wave >= args.wave_start[args.count]) return;
        const SegmentDesc &d = args.seg[s];
        uint32_t row0 = (wave - args.wave_start[s]) * SEG_ROWS;
        float acc[SEG_ROWS];
        gemv_rows_any<SEG_ROWS>(d.encoding, d.w, d.stride, d.rows, d.nblocks, x, row0, acc);
#pragma unroll
        for (int r = 0; r < SEG_ROWS; ++r)
            if (lane == 0 && row0 + r < d.rows) d.out[row0 + r] = acc[r];
    } else {
        if (wave >= args.wave_start[1]) return;
        uint32_t row0 = wave * SEG_ROWS;
        const SegmentDesc &a = args.seg[0];
        const SegmentDesc &b = args.seg[1];
        float ga[SEG_ROWS], ub[SEG_ROWS];
        gemv_rows_any<SEG_ROWS>(a.encoding, a.w, a.stride, a.rows, a.nblocks, x, row0, ga);
        gemv_rows_any<SEG_ROWS>(b.encoding, b.w, b.stride, b.rows, b.nblocks, x, row0, ub);
#pragma unroll
        for (int r = 0; r < SEG_ROWS; ++r) {
            if (lane == 0 && row0 + r < a.rows) {
                float g = ga[r];
                // silu as cpu/vector.zig:178-181: -inf maps to -0
                float silu = (g == -INFINITY) ? -0.f : g / (1.f + expf(-g));
                a.out[row0 + r] = silu * ub[r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host-side launchers.
static inline uint32_t div_up(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

hipError_t launch_dequant_rows(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint64_t first,
                               uint32_t count, uint32_t columns, float *out) {
    Layout l;
    layout_of(encoding, &l);
    uint64_t threads = (uint64_t)count * (columns / 16);
    hipLaunchKernelGGL(dequant_rows_kernel, dim3(div_up(threads, 256)), dim3(256), 0, s, encoding, w, stride,
                       l.elements, l.bytes, first, count, columns, out);
    return hipGetLastError();
}

template <int R>
static hipError_t launch_gemv_r(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                                uint32_t nblocks, const float *x, float *y) {
    uint32_t waves = div_up(rows, encoding == 12 ? 2 * R : R);
    dim3 grid(div_up(waves, 4)), block(256);
    switch (encoding) {
    case 12: hipLaunchKernelGGL(gemv_q4k_kernel<R>, grid, block, 0, s, w, stride, rows, nblocks, x, y); break;
    case 14: hipLaunchKernelGGL(gemv_q6k_kernel<R>, grid, block, 0, s, w, stride, rows, nblocks, x, y); break;
    default: hipLaunchKernelGGL(gemv_q8_0_kernel<R>, grid, block, 0, s, w, stride, rows, nblocks, x, y); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const float *x, float *y, int rows_per_wave) {
    Layout l;
    layout_of(encoding, &l);
    uint32_t nblocks = columns / l.elements;
    switch (rows_per_wave) {
    case 1: return launch_gemv_r<1>(s, encoding, w, stride, rows, nblocks, x, y);
    case 2: return launch_gemv_r<2>(s, encoding, w, stride, rows, nblocks, x, y);
    case 8: return launch_gemv_r<8>(s, encoding, w, stride, rows, nblocks, x, y);
    default: return launch_gemv_r<4>(s, encoding, w, stride, rows, nblocks, x, y);
    }
}

hipError_t launch_generic(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                          uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                          uint64_t out_stride, uint32_t tokens) {
    Layout l;
    layout_of(encoding, &l);
    hipLaunchKernelGGL(generic_rows_kernel, dim3(div_up(rows, 4)), dim3(256), 0, s, encoding, w, stride, rows, columns,
                       l.elements, l.bytes, x, x_f16, in_stride, y, out_stride, tokens);
    return hipGetLastError();
}

template <int T, typename XT>
static hipError_t launch_rows_t(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                                uint32_t nblocks, const XT *x, uint64_t in_stride, float *y, uint64_t out_stride) {
    dim3 grid(div_up(rows, 4)), block(256);
    switch (encoding) {
    case 12:
        hipLaunchKernelGGL((rows_q4k_kernel<T, XT>), grid, block, 0, s, w, stride, rows, nblocks, x, in_stride, y,
                           out_stride);
        break;
    case 14:
        hipLaunchKernelGGL((rows_q6k_kernel<T, XT>), grid, block, 0, s, w, stride, rows, nblocks, x, in_stride, y,
                           out_stride);
        break;
    default:
        hipLaunchKernelGGL((rows_q8_0_kernel<T, XT>), grid, block, 0, s, w, stride, rows, nblocks, x, in_stride, y,
                           out_stride);
        break;
    }
    return hipGetLastError();
}

template <typename XT>
static hipError_t launch_rows_x(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                                uint32_t nblocks, const XT *x, uint64_t in_stride, float *y, uint64_t out_stride,
                                uint32_t tokens) {
    switch (tokens) {
    case 1: return launch_rows_t<1, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    case 2: return launch_rows_t<2, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    case 3: return launch_rows_t<3, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    case 4: return launch_rows_t<4, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    case 5: return launch_rows_t<5, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    case 6: return launch_rows_t<6, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    case 7: return launch_rows_t<7, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    default: return launch_rows_t<8, XT>(s, encoding, w, stride, rows, nblocks, x, in_stride, y, out_stride);
    }
}

hipError_t launch_rows(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                       uint64_t out_stride, uint32_t tokens) {
    Layout l;
    layout_of(encoding, &l);
    uint32_t nblocks = columns / l.elements;
    if (x_f16)
        return launch_rows_x<__half>(s, encoding, w, stride, rows, nblocks, (const __half *)x, in_stride, y,
                                     out_stride, tokens);
    return launch_rows_x<float>(s, encoding, w, stride, rows, nblocks, (const float *)x, in_stride, y, out_stride,
                                tokens);
}

hipError_t launch_segments(hipStream_t s, const SegmentsArgs &args, const float *x) {
    uint32_t waves = args.wave_start[args.mode == 0 ? args.count : 1];
    hipLaunchKernelGGL(segments_kernel, dim3(div_up(waves, 4)), dim3(256), 0, s, args, x);
    return hipGetLastError();
}

int segment_rows_per_wave() { return SEG_ROWS; }

hipError_t launch_argmax(hipStream_t s, const float *logits, uint64_t count, uint32_t *result) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, logits, count, result);
    return hipGetLastError();
}

// The SiLU pair epilogue over two finished products: out[r] = silu(out[r])
// * up[r], with the segments kernel's silu (cpu/vector.zig:178-181).
__global__ void __launch_bounds__(256) silu_mul_kernel(float *__restrict__ out, const float *__restrict__ up,
                                                       uint32_t n) {
    const uint32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= n) return;
    const float g = out[r];
    const float silu = (g == -INFINITY) ? -0.f : g / (1.f + expf(-g));
    out[r] = silu * up[r];
}

hipError_t launch_silu_mul(hipStream_t s, float *out, const float *up, uint32_t n) {
    hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, out, up, n);
    return hipGetLastError();
}

}  // namespace nuq

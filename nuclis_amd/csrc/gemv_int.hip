// Decode GEMV (M = 1) on the integer dot-product pipe.
//
// Why: at M=1 the GEMV must stream 50 MB in ~9 us, and F32 dequant-and-FMA
// costs >= 2 VALU ops per weight value (convert + FMA) plus scale handling,
// which on 256 CUs x 64 lanes is ~7 us of VALU time alone. Here each weight
// code meets the activations in v_dot4c_i32_i8 (4 MACs per op) with exact
// int32 accumulation.
//
// Activations: every lane keeps a fixed slice of x for the whole kernel
// (the K-split below), so it quantises that slice once: per 32-value slice,
// scale s = max|x| / 32639 and x16 = rint(x / s), split exactly into two
// signed bytes x16 = 256*xh + xl (xl in [-128, 127], xh in [-128, 127]).
// A code q then contributes q * x16 = 256 * (q * xh) + q * xl, i.e. two
// dot4 accumulations. The only approximation against the F32 reference is
// x's rounding to 16 bits relative to its slice maximum (|error| <=
// max|x| / 65278 per element); sums of codes are exact and the per-group
// affine terms (scale, minimum) are applied in F32. Non-finite activations
// make the affected outputs NaN.
//
// Layout (K-split, persistent rows): a workgroup of W waves owns a range of
// rows; wave w owns the block range [4P*w, 4P*w + 4P) of every row, so its
// x slices are quantised once and reused for every row the workgroup
// streams. Per-wave row partials meet in LDS and are summed in wave order.
#include "formats.h"
#include "kernels.h"

namespace nuq {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 stream16(const uint8_t *p) {
    u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 32 consecutive activations as two byte planes (8 dwords each), with the
// slice scale and the F32 sum of the original values.
struct XSlice {
    uint32_t hi[8], lo[8];
    float scale;
    float sum;
    int isum;      // sum of x16 (used by biased codes)
    float poison;  // NaN when the slice holds a non-finite value, else 0
};

// LDS image of one quantised slice: 16 plane dwords + scale, sum, isum, poison.
constexpr int SLICE_WORDS = 20;

// Cooperative quantisation: lane pair (2s, 2s+1) quantises slice s (32
// values at xs[s]) of the wave's slice list, 16 values per lane; the two
// halves agree on the slice maximum through one lane exchange. Writes the
// slice image to lds[s * SLICE_WORDS ..]. Every lane of the wave must call
// this (the exchanges are wave-wide).
__device__ __forceinline__ void quantize_half_slice(const float *__restrict__ xp, uint32_t half, uint32_t *lds) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float4 f = *(const float4 *)(xp + 16 * half + 4 * k);
        v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
    float amax = 0.f, sum = 0.f;
    bool finite = true;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        finite = finite && isfinite(v[k]);
        amax = fmaxf(amax, fabsf(v[k]));
        sum += v[k];
    }
    // the pair's halves: lane ^ 1
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    const float other_sum = __shfl_xor(sum, 1, 64);
    finite = finite && (__shfl_xor((int)finite, 1, 64) != 0);
    const float scale = amax / 32639.f;
    const float inv = amax > 0.f ? 32639.f / amax : 0.f;
    int isum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t h = 0, l = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int q = finite ? (int)rintf(v[4 * k + e] * inv) : 0;
            isum += q;
            const int lo = ((q + 128) & 255) - 128;
            const int hi = (q - lo) >> 8;
            h |= (uint32_t)(hi & 255) << (8 * e);
            l |= (uint32_t)(lo & 255) << (8 * e);
        }
        lds[4 * half + k] = h;
        lds[8 + 4 * half + k] = l;
    }
    isum += __shfl_xor(isum, 1, 64);
    if (half == 0) {
        lds[16] = __float_as_uint(scale);
        lds[17] = __float_as_uint(sum + other_sum);  // lower half first, as the summation order
        lds[18] = (uint32_t)isum;
        lds[19] = finite ? 0u : 0x7fc00000u;
    }
}

__device__ __forceinline__ void read_slice(const uint32_t *lds, XSlice &s) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        s.hi[k] = lds[k];
        s.lo[k] = lds[8 + k];
    }
    s.scale = __uint_as_float(lds[16]);
    s.sum = __uint_as_float(lds[17]);
    s.isum = (int)lds[18];
    s.poison = __uint_as_float(lds[19]);
}

// Q4_K scales/minima of the pair (2j, 2j+1) as floats (quant/decode.zig:155-158).
__device__ __forceinline__ void q4k_pair_f(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t shift, bool direct,
                                           float &sa, float &ma, float &sb, float &mb) {
    const uint32_t x = s0 >> shift, y = s1 >> shift, z = s2 >> shift;
    const uint32_t a = direct ? (x & 63u) : ((z & 15u) | (((x >> 6) & 3u) << 4));
    const uint32_t m = direct ? (y & 63u) : (((z >> 4) & 15u) | (((y >> 6) & 3u) << 4));
    const uint32_t b = direct ? ((x >> 8) & 63u) : (((z >> 8) & 15u) | (((x >> 14) & 3u) << 4));
    const uint32_t n = direct ? ((y >> 8) & 63u) : (((z >> 12) & 15u) | (((y >> 14) & 3u) << 4));
    sa = (float)a;
    ma = (float)m;
    sb = (float)b;
    mb = (float)n;
}

// One lane's 64 values of one Q4_K block (qs pair j: 32 bytes) against its
// two x slices: returns d*sa*sum(q x) - dmin*ma*sum(x) + (same for group b).
__device__ __forceinline__ float q4k_lane(const uint4 hdr, const uint4 q0, const uint4 q1, const XSlice &A,
                                          const XSlice &B, uint32_t shift, bool direct) {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int ah = 0, al = 0, bh = 0, bl = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t lo = w[k] & 0x0f0f0f0fu;
        const uint32_t hi = (w[k] >> 4) & 0x0f0f0f0fu;
        ah = dot4(lo, A.hi[k], ah);
        al = dot4(lo, A.lo[k], al);
        bh = dot4(hi, B.hi[k], bh);
        bl = dot4(hi, B.lo[k], bl);
    }
    const float ia = (float)(ah * 256 + al);
    const float ib = (float)(bh * 256 + bl);
    const float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
    float sa, ma, sb, mb;
    q4k_pair_f(hdr.y, hdr.z, hdr.w, shift, direct, sa, ma, sb, mb);
    const float dot = fmaf(sa * A.scale, ia, (sb * B.scale) * ib);
    const float off = fmaf(ma, A.sum, mb * B.sum);
    return fmaf(d, dot, -(dmin * off));
}


__device__ __forceinline__ float quarter_sum(float v) {
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    return v;
}

// Lane = (row group g: 0..3, block slot: 0..3, pair j: 0..3). A quarter-wave
// (16 lanes) covers 4 consecutive blocks of R rows; the 4 quarter-waves take
// different rows. W = ceil(nblocks / 4) waves cover a row (a wave set): wave
// kw of a set owns blocks [4kw, 4kw + 4) of every row, so its x slices are
// read once and stay in registers. A workgroup holds M wave sets (up to 16
// waves) that share one quantised copy of x in LDS and take alternate row
// steps; the next step's weights are loaded before the current step is
// computed. Per-wave row partials meet in LDS and are summed in wave order,
// so the result does not depend on timing.
constexpr int GI_WG_THREADS = 1024;
constexpr uint32_t GI_MAX_SET_WAVES = 16;  // nblocks <= 128 (K <= 32768)

template <int R, int SLOTS>
__global__ void __launch_bounds__(GI_WG_THREADS) gemv_q4k_int_kernel(const uint8_t *__restrict__ w, uint64_t stride,
                                                                      uint32_t rows, uint32_t nblocks,
                                                                      uint32_t rows_per_wg, uint32_t set_waves,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ y) {
    extern __shared__ uint32_t lds[];
    const uint32_t nslices = nblocks * 8;
    uint32_t *slices = lds;                                   // nslices * SLICE_WORDS
    float *partial = (float *)(lds + nslices * SLICE_WORDS);  // rows_per_wg * set_waves

    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sets = (blockDim.x >> 6) / set_waves;
    const uint32_t set = wv / set_waves, kw = wv % set_waves;
    // lane = (row group g, block slot, pair j); a group of 4*SLOTS lanes
    // covers SLOTS consecutive blocks
    const uint32_t g = lane / (4 * SLOTS), slot = (lane >> 2) % SLOTS, j = lane & 3;
    constexpr uint32_t GROUPS = 64 / (4 * SLOTS);
    const bool direct = j < 2;
    const uint32_t shift = direct ? 16 * j : 16 * j - 32;
    const uint32_t row_begin = blockIdx.x * rows_per_wg;
    const uint32_t row_end = min(row_begin + rows_per_wg, rows);
    const uint32_t step_rows = GROUPS * R;
    const uint32_t b = SLOTS * kw + slot;
    const bool live = b < nblocks;
    const uint32_t boff = (live ? b : 0) * 144;

    uint4 hA[R], aA[R], bA[R], hB[R], aB[R], bB[R];
    auto load_step = [&](uint32_t r0, uint4 (&h)[R], uint4 (&q0)[R], uint4 (&q1)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = w + (uint64_t)min(r0 + g * R + r, rows - 1) * stride + boff;
            h[r] = stream16(blk);
            q0[r] = stream16(blk + 16 + 32 * j);
            q1[r] = stream16(blk + 32 + 32 * j);
        }
    };
    // The first step's weights are in flight while x is quantised.
    const uint32_t first = row_begin + set * step_rows;
    const uint32_t set_stride = sets * step_rows;
    if (first < row_end) load_step(first, hA, aA, bA);

    // Cooperative quantisation of all of x: lane pair (2s, 2s+1) -> slice s.
    for (uint32_t t = threadIdx.x; t < 2 * nslices; t += blockDim.x)
        quantize_half_slice(x + (uint64_t)(t >> 1) * 32, t & 1, slices + (t >> 1) * SLICE_WORDS);
    __syncthreads();

    XSlice xa, xb;
    const uint32_t bb = live ? b : 0;
    read_slice(slices + (bb * 8 + 2 * j) * SLICE_WORDS, xa);
    read_slice(slices + (bb * 8 + 2 * j + 1) * SLICE_WORDS, xb);
    if (!live) {
        xa.scale = xb.scale = 0.f;
        xa.sum = xb.sum = 0.f;
        xa.poison = xb.poison = 0.f;
    }
    const float poison = xa.poison + xb.poison;

    auto compute_step = [&](uint32_t r0, const uint4 (&h)[R], const uint4 (&q0)[R], const uint4 (&q1)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = poison + q4k_lane(h[r], q0[r], q1[r], xa, xb, shift, direct);
#pragma unroll
            for (uint32_t off = 2 * SLOTS; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            const uint32_t row = r0 + g * R + r;
            if ((lane & (4 * SLOTS - 1)) == 0 && row < row_end) partial[(row - row_begin) * set_waves + kw] = v;
        }
    };
    uint32_t r0 = first;
    while (r0 < row_end) {
        const uint32_t r1 = r0 + set_stride;
        if (r1 < row_end) load_step(r1, hB, aB, bB);
        compute_step(r0, hA, aA, bA);
        if (r1 >= row_end) break;
        const uint32_t r2 = r1 + set_stride;
        if (r2 < row_end) load_step(r2, hA, aA, bA);
        compute_step(r1, hB, aB, bB);
        r0 = r2;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < row_end - row_begin; i += blockDim.x) {
        float t = 0.f;
        for (uint32_t k = 0; k < set_waves; ++k) t += partial[i * set_waves + k];
        y[row_begin + i] = t;
    }
}

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

template <int R, int SLOTS>
static hipError_t launch_q4k_int(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t nblocks,
                                 const float *x, float *y, uint32_t sets_wanted, uint32_t wgs_per_cu) {
    const uint32_t set_waves = cdiv(nblocks, SLOTS);
    uint32_t sets = (GI_WG_THREADS / 64) / set_waves;
    if (sets_wanted && sets_wanted < sets) sets = sets_wanted;
    const uint32_t step_rows = (64 / (4 * SLOTS)) * R;
    const uint32_t rows_per_wg = cdiv(cdiv(rows, 256 * wgs_per_cu), step_rows) * step_rows;
    const size_t lds = (size_t)nblocks * 8 * SLICE_WORDS * 4 + (size_t)rows_per_wg * set_waves * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_q4k_int_kernel<R, SLOTS>), dim3(cdiv(rows, rows_per_wg)), dim3(64 * set_waves * sets), lds, s,
                       w, stride, rows, nblocks, rows_per_wg, set_waves, x, y);
    return hipGetLastError();
}

// config = R*100 + sets*10 + workgroups per CU (0 = defaults: R=2, as many
// wave sets as fit in 16 waves, one workgroup per CU). Returns
// hipErrorInvalidValue when the shape does not fit (more than 64 blocks per
// row): the caller then uses the row-per-wave kernel.
hipError_t launch_gemv_q4k_int(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                               const float *x, float *y, int config) {
    const uint32_t nblocks = columns / 256;
    if (cdiv(nblocks, 8) > GI_MAX_SET_WAVES) return hipErrorInvalidValue;
    int R = config / 100, sets = (config / 10) % 10, per_cu = config % 10;
    if (config <= 0) {
        R = 2;
        sets = 0;
        per_cu = 1;
    }
    if (per_cu == 0) per_cu = 1;
    // 4 blocks per row group while a row fits in 16 waves, else 8
    if (cdiv(nblocks, 4) <= GI_MAX_SET_WAVES) {
        if (R == 1) return launch_q4k_int<1, 4>(s, w, stride, rows, nblocks, x, y, sets, per_cu);
        return launch_q4k_int<2, 4>(s, w, stride, rows, nblocks, x, y, sets, per_cu);
    }
    if (R == 1) return launch_q4k_int<1, 8>(s, w, stride, rows, nblocks, x, y, sets, per_cu);
    return launch_q4k_int<2, 8>(s, w, stride, rows, nblocks, x, y, sets, per_cu);
}

}  // namespace nuq

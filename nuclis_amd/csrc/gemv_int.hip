// Decode GEMV (M = 1) on the integer dot-product pipe.
//
// Why: at M=1 the GEMV must stream 50 MB in ~9 us, and F32 dequant-and-FMA
// costs >= 2 VALU ops per weight value (convert + FMA) plus scale handling,
// which on 256 CUs x 64 lanes is ~7 us of VALU time alone. Here each weight
// code meets the activations in v_dot4c_i32_i8 (4 MACs per op) with exact
// int32 accumulation.
//
// Activations: every lane keeps a fixed slice of x for the whole kernel
// (the K-split below), so it converts that slice once to fixed point with
// 23 significant bits (an F32 mantissa has 24): per 32-value slice, a
// power-of-two scale s = 2^-k is picked so that max|x| / s lies in
// (4194303, 8355711], and x24 = rint(x / s) (an exact ldexp, then one
// rounding) is split exactly into three signed bytes x24 = 65536*xh +
// 256*xm + xl (each in [-128, 127]). A code q then contributes q*x24 =
// 65536*(q*xh) + 256*(q*xm) + q*xl: three dot4 accumulations, each exact in
// int32. The only approximation before the F32 scale and accumulate is x's
// rounding, |error| <= s/2 <= max|x| * 1.2e-7 (2.4e-7 when max|x| sits just
// above a power of two); the per-group affine terms (scale, minimum) are
// applied in F32. The scale is a power of two at every finite magnitude, so
// nothing overflows: slices of any size keep their relative precision down
// to max|x| = 2^-127, below which s underflows and the slice reads as zero.
//
// Non-finite activations take no part in the fixed-point planes (their
// codes are 0 and they are left out of the slice sum); two 32-bit masks per
// slice mark +Inf/NaN and -Inf/NaN, and the lanes whose slices hold any add
// decoded_weight * x for those values in F32, so a row's output is +-Inf or
// NaN exactly as cpu.matvec's F64 products make it (w * +-Inf = +-Inf,
// 0 * Inf = NaN, w * NaN = NaN; backends/cpu/root.zig:144-152).
//
// Layout (K-split, persistent rows): a workgroup of W waves owns a range of
// rows; wave w owns the block range [4P*w, 4P*w + 4P) of every row, so its
// x slices are quantised once and reused for every row the workgroup
// streams. Per-wave row partials meet in LDS and are summed in wave order.
#include <algorithm>

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

// 32 consecutive activations as three byte planes (8 dwords each), with the
// slice scale and the F32 sum of the original values.
struct XSlice {
    uint32_t hi[8], mid[8], lo[8];
    float scale;
    float sum;                // F32 sum of the slice's finite values
    uint32_t pos, neg;        // bit c: x[c] is +Inf or NaN (pos), -Inf or NaN (neg)
    // Q6_K only (registers): 32 * sum(x24) over values 0-15 and 16-31
    float bias[2];
};

// LDS image of one quantised slice: 24 plane dwords + scale, sum, pos, neg.
constexpr int SLICE_WORDS = 28;
constexpr float X24_MAX = 8355711.f;  // 127 * (65536 + 256 + 1): every byte of the split in [-128, 127]

// q*x24 from the three plane sums: 65536*h + (256*m + l); the parenthesis
// is an exact int32 for every encoding's codes, then one F32 rounding.
__device__ __forceinline__ float combine3(int h, int m, int l) { return fmaf((float)h, 65536.f, (float)(m * 256 + l)); }

// Cooperative quantisation: lane pair (2s, 2s+1) quantises slice s (32
// values at xs[s]) of the wave's slice list, 16 values per lane; the two
// halves agree on the slice maximum through one lane exchange. Writes the
// slice image to lds[s * SLICE_WORDS ..]. Every lane of the wave must call
// this (the exchanges are wave-wide).
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct XHalf {
    f32x4_t f[4];
};

__device__ __forceinline__ void load_half_slice(const float *__restrict__ xp, uint32_t half, XHalf &h) {
#pragma unroll
    for (int k = 0; k < 4; ++k) h.f[k] = *(const f32x4_t *)(xp + 16 * half + 4 * k);
}

typedef __attribute__((address_space(3))) uint32_t lds_u32_t;

// LDS accesses written as asm, for kernels that also copy into LDS with
// global_load_lds: the compiler cannot tell the copies' destination apart
// from other LDS data and would wait for every copy in flight before a
// plain LDS access. The caller orders these with explicit lgkmcnt waits.
__device__ __forceinline__ uint32_t lds_addr(const uint32_t *p) { return (uint32_t)(uintptr_t)(const lds_u32_t *)p; }
__device__ __forceinline__ void lds_store4(uint32_t *p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    asm volatile("ds_write_b128 %0, %1" : : "v"(lds_addr(p)), "v"(v) : "memory");
}

// x loads as asm, for the same reason: with copies into LDS in flight the
// compiler waits for all of them before using any load it issued. The
// caller waits with xhalf_wait<N>, N = loads issued after these.
__device__ __forceinline__ void load_half_slice_asm(const float *__restrict__ xp, uint32_t half, XHalf &h) {
    const float *p = xp + 16 * half;
    asm volatile(
        "global_load_dwordx4 %0, %4, off\n\t"
        "global_load_dwordx4 %1, %4, off offset:16\n\t"
        "global_load_dwordx4 %2, %4, off offset:32\n\t"
        "global_load_dwordx4 %3, %4, off offset:48"
        : "=&v"(h.f[0]), "=&v"(h.f[1]), "=&v"(h.f[2]), "=&v"(h.f[3])
        : "v"(p)
        : "memory");
}
template <int N>
__device__ __forceinline__ void xhalf_wait(XHalf &h) {
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(h.f[0]), "+v"(h.f[1]), "+v"(h.f[2]), "+v"(h.f[3]) : "n"(N) : "memory");
}

template <bool ASM_LDS = false>
__device__ __forceinline__ void quantize_half_slice(const XHalf &xh, uint32_t half, uint32_t *lds) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const f32x4_t f = xh.f[k];
        v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        amax = fmaxf(amax, fabsf(v[k]));
        sum += v[k];
    }
    uint32_t pos = 0, neg = 0;
    if (!isfinite(sum)) {
        // rare: a non-finite value (the sum of finite ones cannot reach Inf
        // unless it overflows, which this path handles the same way): mark
        // them and leave them out of the slice
        amax = 0.f;
        sum = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const bool fin = isfinite(v[k]);
            pos |= (uint32_t)(!fin && !(v[k] < 0.f)) << k;  // +Inf, NaN
            neg |= (uint32_t)(!fin && !(v[k] > 0.f)) << k;  // -Inf, NaN
            v[k] = fin ? v[k] : 0.f;
            amax = fmaxf(amax, fabsf(v[k]));
            sum += v[k];
        }
    }
    // the pair's halves: lane ^ 1 (every lane takes part in each exchange)
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    const float other_sum = __shfl_xor(sum, 1, 64);
    const uint32_t other_pos = (uint32_t)__shfl_xor((int)pos, 1, 64);
    const uint32_t other_neg = (uint32_t)__shfl_xor((int)neg, 1, 64);
    const uint32_t sh = 16 * half;
    const uint32_t pos32 = (pos << sh) | (other_pos << (16 - sh)), neg32 = (neg << sh) | (other_neg << (16 - sh));
    // scale 2^-k: amax * 2^k = f * 2^(e + k) with f in [0.5, 1) from frexp;
    // k = 23 - e unless that passes X24_MAX (f > 0.99608), then 22 - e
    int ex;
    (void)frexpf(amax, &ex);
    int kx = 23 - ex;
    if (ldexpf(amax, kx) > X24_MAX) kx -= 1;
    const float scale = amax > 0.f ? ldexpf(1.f, -kx) : 0.f;
    uint32_t hw[4], mw[4], lw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t h = 0, m = 0, l = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // |q| <= 8355711: q = 65536*hi + 256*mi + lo with every part in [-128, 127]
            const int q = (int)rintf(ldexpf(v[4 * k + e], kx));
            const int lo = ((q + 128) & 255) - 128;
            const int q1 = (q - lo) >> 8;
            const int mi = ((q1 + 128) & 255) - 128;
            const int hi = (q1 - mi) >> 8;
            h |= (uint32_t)(hi & 255) << (8 * e);
            m |= (uint32_t)(mi & 255) << (8 * e);
            l |= (uint32_t)(lo & 255) << (8 * e);
        }
        hw[k] = h;
        mw[k] = m;
        lw[k] = l;
    }
    // words: hi plane 0..7, mid plane 8..15, lo plane 16..23, then scale, sum
    // (lower half first, as the summation order), the non-finite masks
    const uint32_t t0 = __float_as_uint(scale),
                   t1 = __float_as_uint(half == 0 ? sum + other_sum : other_sum + sum), t2 = pos32, t3 = neg32;
    if constexpr (ASM_LDS) {
        lds_store4(lds + 4 * half, hw[0], hw[1], hw[2], hw[3]);
        lds_store4(lds + 8 + 4 * half, mw[0], mw[1], mw[2], mw[3]);
        lds_store4(lds + 16 + 4 * half, lw[0], lw[1], lw[2], lw[3]);
        if (half == 0) lds_store4(lds + 24, t0, t1, t2, t3);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            lds[4 * half + k] = hw[k];
            lds[8 + 4 * half + k] = mw[k];
            lds[16 + 4 * half + k] = lw[k];
        }
        if (half == 0) {
            lds[24] = t0;
            lds[25] = t1;
            lds[26] = t2;
            lds[27] = t3;
        }
    }
}

// read_slice through asm (see lds_store4); waits for its own reads.
__device__ __forceinline__ void read_slice_asm(const uint32_t *lds, XSlice &s) {
    u32x4_t p[7];
    asm volatile(
        "ds_read_b128 %0, %7\n\t"
        "ds_read_b128 %1, %7 offset:16\n\t"
        "ds_read_b128 %2, %7 offset:32\n\t"
        "ds_read_b128 %3, %7 offset:48\n\t"
        "ds_read_b128 %4, %7 offset:64\n\t"
        "ds_read_b128 %5, %7 offset:80\n\t"
        "ds_read_b128 %6, %7 offset:96\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(p[0]), "=&v"(p[1]), "=&v"(p[2]), "=&v"(p[3]), "=&v"(p[4]), "=&v"(p[5]), "=&v"(p[6])
        : "v"(lds_addr(lds))
        : "memory");
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        s.hi[4 * k] = p[k].x; s.hi[4 * k + 1] = p[k].y; s.hi[4 * k + 2] = p[k].z; s.hi[4 * k + 3] = p[k].w;
        s.mid[4 * k] = p[2 + k].x; s.mid[4 * k + 1] = p[2 + k].y; s.mid[4 * k + 2] = p[2 + k].z; s.mid[4 * k + 3] = p[2 + k].w;
        s.lo[4 * k] = p[4 + k].x; s.lo[4 * k + 1] = p[4 + k].y; s.lo[4 * k + 2] = p[4 + k].z; s.lo[4 * k + 3] = p[4 + k].w;
    }
    s.scale = __uint_as_float(p[6].x);
    s.sum = __uint_as_float(p[6].y);
    s.pos = p[6].z;
    s.neg = p[6].w;
}

__device__ __forceinline__ void read_slice(const uint32_t *lds, XSlice &s) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        s.hi[k] = lds[k];
        s.mid[k] = lds[8 + k];
        s.lo[k] = lds[16 + k];
    }
    s.scale = __uint_as_float(lds[24]);
    s.sum = __uint_as_float(lds[25]);
    s.pos = lds[26];
    s.neg = lds[27];
}

// Q6_K's -32 bias per 16-value half of a slice: 32 * sum(x24), from the
// planes' exact integer sums, rounded once to F32.
__device__ __forceinline__ void plane_sums(XSlice &s) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        int h = 0, m = 0, l = 0;
#pragma unroll
        for (int k = 4 * half; k < 4 * half + 4; ++k) {
            h = dot4(s.hi[k], 0x01010101u, h);
            m = dot4(s.mid[k], 0x01010101u, m);
            l = dot4(s.lo[k], 0x01010101u, l);
        }
        s.bias[half] = 32.f * combine3(h, m, l);
    }
}

// The non-finite activations against one row's decoded weights: the sum of
// w[c] * x[c] over the columns c that the slice masks mark, in F32.
// cpu.matvec multiplies each F64 weight by its activation
// (backends/cpu/root.zig:144-152); with x = +-Inf or NaN the class of each
// product (w * +-Inf = +-Inf, 0 * Inf = NaN, w * NaN = NaN) and of their sum
// with the finite rest does not depend on the precision. Taken only when a
// workgroup's x holds such values; `unit_bytes` is 272 for Q8_0 (eight
// blocks), else the block size.
__device__ __noinline__ float nonfinite_row(uint32_t enc, const uint8_t *row, uint32_t unit_bytes,
                                            const uint32_t *slices, uint32_t nslices) {
    float t = 0.f;
    for (uint32_t s = 0; s < nslices; ++s) {
        const uint32_t pos = slices[s * SLICE_WORDS + 26], neg = slices[s * SLICE_WORDS + 27];
        uint32_t m = pos | neg;
        while (m) {
            const uint32_t c = __builtin_ctz(m);
            m &= m - 1;
            const float xv = ((pos & neg) >> c) & 1u ? __builtin_nanf("") : ((pos >> c) & 1u ? INFINITY : -INFINITY);
            const uint32_t col = 32 * s + c;
            const float wv = enc == 8 ? decode_q8_0(row + (col / 32) * 34, col % 32)
                                      : decode_value(enc, row + (col / 256) * unit_bytes, col % 256);
            t += wv * xv;
        }
    }
    return t;
}

// Q4_K scales/minima of the pair (2j, 2j+1) as floats (quant/decode.zig:155-158),
// without branches: with shift = 16*(j&1), the pair's two scale bytes are
// bytes 0-1 of A = s0>>shift (and the minima of M = s1>>shift). Pairs 0 and 1
// use their 6 low bits; pairs 2 and 3 take the low (scales) or high (minima)
// nibble of Z = s2>>shift plus bits 6-7 of A (or M) as bits 4-5. Both forms
// are computed on the two bytes at once and selected with a lane mask.
__device__ __forceinline__ void q4k_pair_f(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t shift, bool direct,
                                           float &sa, float &ma, float &sb, float &mb) {
    const uint32_t A = s0 >> shift, M = s1 >> shift, Z = s2 >> shift;
    const uint32_t dm = 0u - (uint32_t)direct;
    const uint32_t sc = ((A & 0x3f3fu) & dm) | (((Z & 0x0f0fu) | ((A >> 2) & 0x3030u)) & ~dm);
    const uint32_t mn = ((M & 0x3f3fu) & dm) | ((((Z >> 4) & 0x0f0fu) | ((M >> 2) & 0x3030u)) & ~dm);
    sa = ubyte_f<0>(sc);
    sb = ubyte_f<1>(sc);
    ma = ubyte_f<0>(mn);
    mb = ubyte_f<1>(mn);
}

// One lane's 64 values of one Q4_K block (qs pair j: 32 bytes) against its
// two x slices: returns d*sa*sum(q x) - dmin*ma*sum(x) + (same for group b).
__device__ __forceinline__ float q4k_lane(const uint4 hdr, const uint4 q0, const uint4 q1, const XSlice &A,
                                          const XSlice &B, uint32_t shift, bool direct) {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t lo = w[k] & 0x0f0f0f0fu;
        const uint32_t hi = (w[k] >> 4) & 0x0f0f0f0fu;
        ah = dot4(lo, A.hi[k], ah);
        am = dot4(lo, A.mid[k], am);
        al = dot4(lo, A.lo[k], al);
        bh = dot4(hi, B.hi[k], bh);
        bm = dot4(hi, B.mid[k], bm);
        bl = dot4(hi, B.lo[k], bl);
    }
    const float ia = combine3(ah, am, al);
    const float ib = combine3(bh, bm, bl);
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

template <int R, int SLOTS, int D>
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
    const uint32_t first = row_begin + set * step_rows;
    const uint32_t set_stride = sets * step_rows;
    const uint32_t nsteps = first < row_end ? (row_end - first + set_stride - 1) / set_stride : 0;

    // Issue order: this thread's first half-slice of x, then the weights of
    // the first D steps (everything a wave streams, for the shapes this
    // kernel is sized for), so the quantisation below waits only for x.
    const uint32_t t0 = threadIdx.x;
    XHalf xh;
    if (t0 < 2 * nslices) load_half_slice(x + (uint64_t)(t0 >> 1) * 32, t0 & 1, xh);

    uint4 hq[D][R], aq[D][R], bq[D][R];
#define NUQ_GI_LOAD(SLOT_, STEP_)                                                              \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                                            \
        const uint32_t row_ = first + (STEP_) * set_stride + g * R + r;                        \
        const uint8_t *blk = w + (uint64_t)min(row_, row_end - 1) * stride + boff;             \
        hq[SLOT_][r] = stream16(blk);                                                          \
        aq[SLOT_][r] = stream16(blk + 16 + 32 * j);                                            \
        bq[SLOT_][r] = stream16(blk + 32 + 32 * j);                                            \
    }
    // Loads are unconditional (rows past the range re-read the workgroup's
    // last row, a cache hit): a load behind a branch makes the compiler's
    // wait counts conservative and drains every outstanding load.
#pragma unroll
    for (int d = 0; d < D; ++d) NUQ_GI_LOAD(d, (uint32_t)d)

    // Cooperative quantisation of all of x: lane pair (2s, 2s+1) -> slice s.
    if (t0 < 2 * nslices) quantize_half_slice(xh, t0 & 1, slices + (t0 >> 1) * SLICE_WORDS);
    for (uint32_t t = t0 + blockDim.x; t < 2 * nslices; t += blockDim.x) {
        load_half_slice(x + (uint64_t)(t >> 1) * 32, t & 1, xh);
        quantize_half_slice(xh, t & 1, slices + (t >> 1) * SLICE_WORDS);
    }
    __syncthreads();

    XSlice xa, xb;
    const uint32_t bb = live ? b : 0;
    read_slice(slices + (bb * 8 + 2 * j) * SLICE_WORDS, xa);
    read_slice(slices + (bb * 8 + 2 * j + 1) * SLICE_WORDS, xb);
    if (!live) {
        xa.scale = xb.scale = 0.f;
        xa.sum = xb.sum = 0.f;
        xa.pos = xa.neg = xb.pos = xb.neg = 0u;
    }
    // wave-uniform: does any slice this wave reads hold a non-finite value
    const bool nonfinite = __ballot((xa.pos | xa.neg | xb.pos | xb.neg) != 0u) != 0;

    // Step i lives in register slot i % D; once computed, the slot takes
    // step i + D. The main loop runs while every refill is a real step, so
    // its loads need no branch; the last 2D steps are peeled.
#define NUQ_GI_COMPUTE(SLOT_, STEP_)                                                                         \
    {                                                                                                        \
        const uint32_t r0_ = first + (STEP_) * set_stride;                                                   \
        _Pragma("unroll") for (int r = 0; r < R; ++r) {                                                      \
            float v = q4k_lane(hq[SLOT_][r], aq[SLOT_][r], bq[SLOT_][r], xa, xb, shift, direct);              \
            _Pragma("unroll") for (uint32_t off = 2 * SLOTS; off > 0; off >>= 1) v += __shfl_xor(v, off, 64); \
            const uint32_t row = r0_ + g * R + r;                                                            \
            if ((lane & (4 * SLOTS - 1)) == 0 && row < row_end) partial[(row - row_begin) * set_waves + kw] = v; \
        }                                                                                                    \
    }
    uint32_t i = 0;
    for (; i + 2 * D <= nsteps; i += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            NUQ_GI_COMPUTE(d, i + d)
            NUQ_GI_LOAD(d, i + d + D)
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (i + d < nsteps) NUQ_GI_COMPUTE(d, i + d)
        if (i + d + D < nsteps) NUQ_GI_LOAD(d, i + d + D)
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (i + D + d < nsteps) NUQ_GI_COMPUTE(d, i + D + d)
#undef NUQ_GI_COMPUTE
#undef NUQ_GI_LOAD
    // every slice is read by some live lane, so this is "x holds a non-finite value"
    const bool any_nonfinite = __syncthreads_or(nonfinite);
    for (uint32_t i = threadIdx.x; i < row_end - row_begin; i += blockDim.x) {
        float t = 0.f;
        for (uint32_t k = 0; k < set_waves; ++k) t += partial[i * set_waves + k];
        if (any_nonfinite) t += nonfinite_row(12, w + (uint64_t)(row_begin + i) * stride, 144, slices, nslices);
        y[row_begin + i] = t;
    }
}

// DMA variant (R = 1), for Q4_K, Q5_K and IQ4_XS. Instead of each lane
// loading its header and code chunks straight from HBM (scattered loads that
// touch every cache line of the step about three times), each wave copies
// the step's bytes -- GROUPS rows x SLOTS blocks, as many contiguous 16-byte
// chunks as a block has bytes (144, 176, 136) whatever SLOTS is -- into a
// private LDS ring with three global_load_lds_dwordx4 (lane i of
// instruction n moves chunk 64n + i), and the lanes then read their bytes
// from LDS. Waves never read
// another wave's ring, so only the wave's own vmcnt orders DMA and reads.
// A ring slot holds INSTRS copy instructions of 64 lanes x 16 bytes.

typedef __attribute__((address_space(3))) void gd_lds_void_t;
typedef __attribute__((address_space(3))) uint8_t gd_lds_u8_t;

// Per-encoding pieces of the DMA kernel. `read<VM>` fetches a lane's bytes
// of one block from its wave's ring once at most VM younger copies are
// outstanding, and waits for the reads: one asm block, because the compiler
// cannot tell ring slots apart and would otherwise wait for every copy in
// flight. `dot` is the lane's contribution: pair j = groups 2j (x slice A)
// and 2j+1 (slice B) of the block.
__device__ __forceinline__ uint32_t lds_u8_addr(const uint8_t *p) { return (uint32_t)(uintptr_t)(const gd_lds_u8_t *)p; }

template <uint32_t ENC>
struct GdEnc;

template <>
struct GdEnc<12> {  // Q4_K: header + the pair's 32 code bytes
    static constexpr uint32_t BYTES = 144, INSTRS = (BYTES + 63) / 64;
    u32x4_t h, q0, q1;
    template <int VM>
    __device__ __forceinline__ void read(const uint8_t *blk, uint32_t j) {
        const uint32_t a = lds_u8_addr(blk), b = a + 16 + 32 * j;
        asm volatile(
            "s_waitcnt vmcnt(%3)\n\t"
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %5\n\t"
            "ds_read_b128 %2, %5 offset:16\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(h), "=&v"(q0), "=&v"(q1)
            : "n"(VM), "v"(a), "v"(b)
            : "memory");
    }
    __device__ __forceinline__ float dot(const XSlice &A, const XSlice &B, uint32_t, uint32_t shift,
                                         bool direct) const {
        return q4k_lane(make_uint4(h.x, h.y, h.z, h.w), make_uint4(q0.x, q0.y, q0.z, q0.w),
                        make_uint4(q1.x, q1.y, q1.z, q1.w), A, B, shift, direct);
    }
};

template <>
struct GdEnc<13> {  // Q5_K: header, the 32 high-plane bytes, the pair's 32 code bytes
    static constexpr uint32_t BYTES = 176, INSTRS = (BYTES + 63) / 64;
    u32x4_t h, qh0, qh1, q0, q1;
    template <int VM>
    __device__ __forceinline__ void read(const uint8_t *blk, uint32_t j) {
        const uint32_t a = lds_u8_addr(blk), b = a + 48 + 32 * j;
        asm volatile(
            "s_waitcnt vmcnt(%5)\n\t"
            "ds_read_b128 %0, %6\n\t"
            "ds_read_b128 %1, %6 offset:16\n\t"
            "ds_read_b128 %2, %6 offset:32\n\t"
            "ds_read_b128 %3, %7\n\t"
            "ds_read_b128 %4, %7 offset:16\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(h), "=&v"(qh0), "=&v"(qh1), "=&v"(q0), "=&v"(q1)
            : "n"(VM), "v"(a), "v"(b)
            : "memory");
    }
    // codes are 5-bit: nibble plus bit 2j (group 2j) or 2j+1 of high-plane
    // byte c for column c (quant/decode.zig:162-166)
    __device__ __forceinline__ float dot(const XSlice &A, const XSlice &B, uint32_t j, uint32_t shift,
                                         bool direct) const {
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[8] = {qh0.x, qh0.y, qh0.z, qh0.w, qh1.x, qh1.y, qh1.z, qh1.w};
        int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t lo = (w[k] & 0x0f0f0f0fu) | (((hb[k] >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t hi = ((w[k] >> 4) & 0x0f0f0f0fu) | (((hb[k] >> (2 * j + 1)) & 0x01010101u) << 4);
            ah = dot4(lo, A.hi[k], ah);
            am = dot4(lo, A.mid[k], am);
            al = dot4(lo, A.lo[k], al);
            bh = dot4(hi, B.hi[k], bh);
            bm = dot4(hi, B.mid[k], bm);
            bl = dot4(hi, B.lo[k], bl);
        }
        const float ia = combine3(ah, am, al), ib = combine3(bh, bm, bl);
        const float d = half_bits(h.x & 0xffffu), dmin = half_bits(h.x >> 16);
        float sa, ma, sb, mb;
        q4k_pair_f(h.y, h.z, h.w, shift, direct, sa, ma, sb, mb);
        const float dt = fmaf(sa * A.scale, ia, (sb * B.scale) * ib);
        const float off = fmaf(ma, A.sum, mb * B.sum);
        return fmaf(d, dt, -(dmin * off));
    }
};

template <>
struct GdEnc<14> {  // Q6_K: the half's 64 code bytes, its 32 high-bit bytes, 4 scales, d
    static constexpr uint32_t BYTES = 210, INSTRS = (BYTES + 63) / 64;
    u32x4_t l0, l1, l2, l3, h0, h1;
    uint32_t sc, d16;
    // Blocks sit at 2-byte offsets in the ring. Misaligned LDS reads return
    // the right bytes but stall, so the fields are read as 4-byte aligned
    // dword pairs one dword longer than needed and shifted into place with
    // one funnel shift each (v_alignbit_b32): by the block's offset mod 4
    // in bytes, plus 4 bits for the lanes that take the high nibbles (and
    // the matching high-bit pairs), so the code words need no other shift.
    template <int VM>
    __device__ __forceinline__ void read(const uint8_t *blk, uint32_t j) {
        typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
        const uint32_t a = lds_u8_addr(blk), sh = a & 3u;
        const uint32_t ql = (a + 64 * (j >> 1)) & ~3u, qh = (a + 128 + 32 * (j >> 1)) & ~3u;
        const uint32_t sca = (a + 192 + 4 * j) & ~3u, da = (a + 208) & ~3u;
        u32x2_t q[9], hq[5], sp;
        uint32_t dw;
        asm volatile(
            "s_waitcnt vmcnt(%16)\n\t"
            "ds_read2_b32 %0, %17 offset1:1\n\t"
            "ds_read2_b32 %1, %17 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %2, %17 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %3, %17 offset0:6 offset1:7\n\t"
            "ds_read2_b32 %4, %17 offset0:8 offset1:9\n\t"
            "ds_read2_b32 %5, %17 offset0:10 offset1:11\n\t"
            "ds_read2_b32 %6, %17 offset0:12 offset1:13\n\t"
            "ds_read2_b32 %7, %17 offset0:14 offset1:15\n\t"
            "ds_read2_b32 %8, %17 offset0:16 offset1:17\n\t"
            "ds_read2_b32 %9, %18 offset1:1\n\t"
            "ds_read2_b32 %10, %18 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %11, %18 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %12, %18 offset0:6 offset1:7\n\t"
            "ds_read2_b32 %13, %18 offset0:8 offset1:9\n\t"
            "ds_read2_b32 %14, %19 offset1:1\n\t"
            "ds_read_b32 %15, %20\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]),
              "=&v"(q[7]), "=&v"(q[8]), "=&v"(hq[0]), "=&v"(hq[1]), "=&v"(hq[2]), "=&v"(hq[3]), "=&v"(hq[4]),
              "=&v"(sp), "=&v"(dw)
            : "n"(VM), "v"(ql), "v"(qh), "v"(sca), "v"(da)
            : "memory");
        uint32_t r[18], t[10];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            r[2 * k] = q[k].x;
            r[2 * k + 1] = q[k].y;
        }
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            t[2 * k] = hq[k].x;
            t[2 * k + 1] = hq[k].y;
        }
        uint32_t o[16], p[8];
        const uint32_t bits = 8 * sh + 4 * (j & 1);
#pragma unroll
        for (int k = 0; k < 16; ++k) o[k] = __builtin_amdgcn_alignbit(r[k + 1], r[k], bits);
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = __builtin_amdgcn_alignbit(t[k + 1], t[k], bits);
        l0 = u32x4_t{o[0], o[1], o[2], o[3]};
        l1 = u32x4_t{o[4], o[5], o[6], o[7]};
        l2 = u32x4_t{o[8], o[9], o[10], o[11]};
        l3 = u32x4_t{o[12], o[13], o[14], o[15]};
        h0 = u32x4_t{p[0], p[1], p[2], p[3]};
        h1 = u32x4_t{p[4], p[5], p[6], p[7]};
        sc = __builtin_amdgcn_alignbyte(sp.y, sp.x, sh);
        d16 = (dw >> (8 * sh)) & 0xffffu;
    }
    // lane j: quarters q0 = 2(j&1) (x slice A) and q0+1 (slice B) of half
    // j>>1; code of column c = nibble j&1 of ql[c] (ql[32 + c] for q0+1) |
    // bits 2q of qh[c] as bits 4-5, minus 32 (quant/decode.zig:198-211);
    // scale bytes: A columns 0-15, 16-31, then B's. read() has already
    // shifted the code and high-bit words by 4 (j&1) bits.
    __device__ __forceinline__ float dot(const XSlice &A, const XSlice &B, uint32_t, uint32_t, bool) const {
        const uint32_t la[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
        const uint32_t lb[8] = {l2.x, l2.y, l2.z, l2.w, l3.x, l3.y, l3.z, l3.w};
        const uint32_t hb[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        // Codes stay unsigned (0..63, also valid signed bytes); the -32 bias
        // comes off each 16-value sum in F32 as 32 * sum(x24) of those values.
        int a0[3] = {0, 0, 0}, a1[3] = {0, 0, 0}, b0[3] = {0, 0, 0}, b1[3] = {0, 0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t hq = hb[k];
            const uint32_t ua = (la[k] & 0x0f0f0f0fu) | ((hq << 4) & 0x30303030u);
            const uint32_t ub = (lb[k] & 0x0f0f0f0fu) | ((hq << 2) & 0x30303030u);
            int *ra = k < 4 ? a0 : a1, *rb = k < 4 ? b0 : b1;
            ra[0] = dot4(ua, A.hi[k], ra[0]);
            ra[1] = dot4(ua, A.mid[k], ra[1]);
            ra[2] = dot4(ua, A.lo[k], ra[2]);
            rb[0] = dot4(ub, B.hi[k], rb[0]);
            rb[1] = dot4(ub, B.mid[k], rb[1]);
            rb[2] = dot4(ub, B.lo[k], rb[2]);
        }
        const float s0 = (float)(int8_t)(sc & 0xffu), s1 = (float)(int8_t)((sc >> 8) & 0xffu);
        const float s2 = (float)(int8_t)((sc >> 16) & 0xffu), s3 = (float)(int8_t)(sc >> 24);
        const float ia0 = combine3(a0[0], a0[1], a0[2]) - A.bias[0];
        const float ia1 = combine3(a1[0], a1[1], a1[2]) - A.bias[1];
        const float ib0 = combine3(b0[0], b0[1], b0[2]) - B.bias[0];
        const float ib1 = combine3(b1[0], b1[1], b1[2]) - B.bias[1];
        const float ta = fmaf(s0, ia0, s1 * ia1);
        const float tb = fmaf(s2, ib0, s3 * ib1);
        return half_bits(d16) * fmaf(A.scale, ta, B.scale * tb);
    }
};

template <>
struct GdEnc<8> {  // Q8_0: eight 34-byte blocks (256 values) as one unit; lane j: blocks 2j, 2j+1
    static constexpr uint32_t BYTES = 272, INSTRS = (BYTES + 63) / 64;
    uint32_t qa[8], qb[8], da, db;
    // The pair's 68 bytes start 4-byte aligned (units are 16-byte aligned in
    // the ring, 68j into the unit): block 2j's codes sit 2 bytes in and are
    // shifted into dwords with v_alignbyte_b32; block 2j+1's are aligned.
    template <int VM>
    __device__ __forceinline__ void read(const uint8_t *blk, uint32_t j) {
        typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
        const uint32_t a = lds_u8_addr(blk) + 68 * j;
        u32x2_t q[8];
        uint32_t last;
        asm volatile(
            "s_waitcnt vmcnt(%9)\n\t"
            "ds_read2_b32 %0, %10 offset1:1\n\t"
            "ds_read2_b32 %1, %10 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %2, %10 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %3, %10 offset0:6 offset1:7\n\t"
            "ds_read2_b32 %4, %10 offset0:8 offset1:9\n\t"
            "ds_read2_b32 %5, %10 offset0:10 offset1:11\n\t"
            "ds_read2_b32 %6, %10 offset0:12 offset1:13\n\t"
            "ds_read2_b32 %7, %10 offset0:14 offset1:15\n\t"
            "ds_read_b32 %8, %10 offset:64\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]),
              "=&v"(q[7]), "=&v"(last)
            : "n"(VM), "v"(a)
            : "memory");
        uint32_t r[17];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            r[2 * k] = q[k].x;
            r[2 * k + 1] = q[k].y;
        }
        r[16] = last;
#pragma unroll
        for (int k = 0; k < 8; ++k) qa[k] = __builtin_amdgcn_alignbyte(r[k + 1], r[k], 2);
#pragma unroll
        for (int k = 0; k < 8; ++k) qb[k] = r[9 + k];
        da = r[0] & 0xffffu;
        db = r[8] >> 16;
    }
    // w = d * q per 32-value block (quant/decode.zig:57-63): the exact
    // integer sums of q * x16 scaled by d and the slice scale in F32
    __device__ __forceinline__ float dot(const XSlice &A, const XSlice &B, uint32_t, uint32_t, bool) const {
        int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            ah = dot4(qa[k], A.hi[k], ah);
            am = dot4(qa[k], A.mid[k], am);
            al = dot4(qa[k], A.lo[k], al);
            bh = dot4(qb[k], B.hi[k], bh);
            bm = dot4(qb[k], B.mid[k], bm);
            bl = dot4(qb[k], B.lo[k], bl);
        }
        // d * sum first, then the slice scale (a power of two): d * scale
        // alone could fall below the F32 range for tiny activations
        const float ta = half_bits(da) * combine3(ah, am, al), tb = half_bits(db) * combine3(bh, bm, bl);
        return fmaf(ta, A.scale, tb * B.scale);
    }
};

template <>
struct GdEnc<23> {  // IQ4_XS: 8-byte header + the pair's 32 code bytes (8-byte aligned)
    static constexpr uint32_t BYTES = 136, INSTRS = (BYTES + 63) / 64;
    uint32_t h0, h1;
    u32x4_t qa, qb;
    template <int VM>
    __device__ __forceinline__ void read(const uint8_t *blk, uint32_t j) {
        const uint32_t a = lds_u8_addr(blk), b = a + 8 + 32 * j;
        u32x4_t hh;
        asm volatile(
            "s_waitcnt vmcnt(%3)\n\t"
            "ds_read_b64 %0, %4\n\t"
            "ds_read2_b64 %1, %5 offset1:1\n\t"
            "ds_read2_b64 %2, %5 offset0:2 offset1:3\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hh.xy), "=&v"(qa), "=&v"(qb)
            : "n"(VM), "v"(a), "v"(b)
            : "memory");
        h0 = hh.x;
        h1 = hh.y;
    }
    // group 2j: code bytes 0-15 (qa), group 2j+1: bytes 16-31 (qb); byte k's
    // low nibble is value k and its high nibble value 16+k of the group
    // (quant/decode.zig:213-228); codes map to signed bytes by iq4_lookup.
    __device__ __forceinline__ float dot(const XSlice &A, const XSlice &B, uint32_t j, uint32_t, bool) const {
        const uint32_t wa[4] = {qa.x, qa.y, qa.z, qa.w}, wb[4] = {qb.x, qb.y, qb.z, qb.w};
        int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t la = iq4_lookup(wa[m] & 0x0f0f0f0fu), ua = iq4_lookup((wa[m] >> 4) & 0x0f0f0f0fu);
            const uint32_t lb = iq4_lookup(wb[m] & 0x0f0f0f0fu), ub = iq4_lookup((wb[m] >> 4) & 0x0f0f0f0fu);
            ah = dot4(la, A.hi[m], ah);
            am = dot4(la, A.mid[m], am);
            al = dot4(la, A.lo[m], al);
            ah = dot4(ua, A.hi[4 + m], ah);
            am = dot4(ua, A.mid[4 + m], am);
            al = dot4(ua, A.lo[4 + m], al);
            bh = dot4(lb, B.hi[m], bh);
            bm = dot4(lb, B.mid[m], bm);
            bl = dot4(lb, B.lo[m], bl);
            bh = dot4(ub, B.hi[4 + m], bh);
            bm = dot4(ub, B.mid[4 + m], bm);
            bl = dot4(ub, B.lo[4 + m], bl);
        }
        const float ia = combine3(ah, am, al), ib = combine3(bh, bm, bl);
        const uint32_t sl = (h1 >> (8 * j)) & 0xffu, sh = h0 >> 16;
        const int sa = (int)((sl & 15u) | (((sh >> (4 * j)) & 3u) << 4)) - 32;
        const int sb = (int)((sl >> 4) | (((sh >> (4 * j + 2)) & 3u) << 4)) - 32;
        const float d = half_bits(h0 & 0xffffu);
        return d * fmaf((float)sa * A.scale, ia, ((float)sb * B.scale) * ib);
    }
};
typedef __attribute__((address_space(1))) void gd_global_void_t;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of N lanes (16 or 32), left in every lane of the
// group: four DPP adds within a 16-lane row (xor 1, xor 2, half-row mirror,
// row mirror), then one lane exchange between rows for N = 32.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    if (N == 32) v += __shfl_xor(v, 16, 64);
    return v;
}

// Workgroup size cap of the DMA kernel: 16 waves, except Q6_K, whose lanes
// hold more bytes per block (the alignment shifts) and so take 12 waves,
// keeping its registers (up to 170) clear of spills.
template <uint32_t ENC>
constexpr int gd_threads() { return ENC == 14 ? 768 : GI_WG_THREADS; }

// TWO: x takes two rounds of half-slices (a template parameter, so each
// form is straight-line code: the asm loads' registers must not be touched
// before their explicit waits, and a branch merging two forms made the
// compiler copy them early).
// WX: every wave quantises its own blocks' x slices (one wave set).
template <uint32_t ENC, int SLOTS, int D, bool TWO = false, bool WX = false>
__global__ void __launch_bounds__(gd_threads<ENC>()) gemv_dma_kernel(const uint8_t *__restrict__ w, uint64_t stride,
                                                                      uint32_t rows, uint32_t nblocks,
                                                                      uint32_t rows_per_wg, uint32_t set_waves,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ y, uint32_t tail,
                                                                      GdSegments segs) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    // Segments: workgroups [wg_end[q-1], wg_end[q]) run matrix q. Each entry
    // is read with a constant index, so the table stays in scalar registers.
    uint32_t blk = blockIdx.x;
    if (segs.count) {
        w = segs.w[0];
        y = segs.y[0];
        rows = segs.rows[0];
        rows_per_wg = segs.rows_per_wg[0];
#pragma unroll
        for (uint32_t q = 1; q < GD_MAX_SEGMENTS; ++q)
            if (q < segs.count && blockIdx.x >= segs.wg_end[q - 1]) {
                w = segs.w[q];
                y = segs.y[q];
                rows = segs.rows[q];
                rows_per_wg = segs.rows_per_wg[q];
                blk = blockIdx.x - segs.wg_end[q - 1];
            }
    }
    if (tail && blockIdx.x == gridDim.x - 1) {
        // The matrix's last row (rows is the count without it), when a row
        // ends mid-chunk: its last copy would read past the weights, so this
        // extra workgroup decodes it exactly against F32 x instead.
        const uint8_t *rowp = w + (uint64_t)rows * stride;
        float acc = 0.f;
        for (uint32_t c = threadIdx.x; c < nblocks * 256; c += blockDim.x)
            acc = fmaf(decode_value(ENC, rowp + (uint64_t)(c / 256) * GdEnc<ENC>::BYTES, c % 256), x[c], acc);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
        float *sums = (float *)lds;
        if ((threadIdx.x & 63) == 0) sums[threadIdx.x >> 6] = acc;
        __syncthreads();
        if (threadIdx.x == 0) {
            float t = 0.f;
            for (uint32_t k = 0; k < (blockDim.x >> 6); ++k) t += sums[k];
            y[rows] = t;
        }
        return;
    }
    constexpr uint32_t GD_DMA_INSTRS = GdEnc<ENC>::INSTRS, GD_SLOT_BYTES = GD_DMA_INSTRS * 64 * 16;
    const uint32_t nslices = nblocks * 8;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    uint8_t *rings = (uint8_t *)lds;                                          // nwaves * D * GD_SLOT_BYTES
    uint32_t *slices = lds + nwaves * D * (GD_SLOT_BYTES / 4);                // nslices * SLICE_WORDS
    // rows_per_wg * set_waves partial sums, one spare per wave, then one
    // row-step counter per K range
    float *partial = (float *)(slices + nslices * SLICE_WORDS);
    uint8_t *ring = rings + wv * D * GD_SLOT_BYTES;
#define NUQ_GD_RING(SLOT_) (ring + (SLOT_) * GD_SLOT_BYTES)
    const uint32_t sets = nwaves / set_waves;
    const uint32_t set = wv / set_waves, kw = wv % set_waves;
    const uint32_t g = lane / (4 * SLOTS), slot = (lane >> 2) % SLOTS, j = lane & 3;
    constexpr uint32_t GROUPS = 64 / (4 * SLOTS);
    constexpr uint32_t BYTES = GdEnc<ENC>::BYTES;
    constexpr uint32_t ROW_CHUNKS = SLOTS * BYTES / 16;  // a row's SLOTS blocks (SLOTS even for IQ4_XS)
    static_assert(GROUPS * ROW_CHUNKS == BYTES && SLOTS * BYTES % 16 == 0, "one step is BYTES chunks");
    const bool direct = j < 2;
    const uint32_t shift = direct ? 16 * j : 16 * j - 32;
    const uint32_t row_begin = blk * rows_per_wg;
    const uint32_t row_end = min(row_begin + rows_per_wg, rows);
    const uint32_t b = SLOTS * kw + slot;
    const bool live = b < nblocks;
    const uint32_t first = row_begin + set * GROUPS;
    const uint32_t set_stride = sets * GROUPS;
    const uint32_t nsteps = first < row_end ? (row_end - first + set_stride - 1) / set_stride : 0;

    // This lane's chunk in each DMA instruction: row q within the step and
    // byte offset within the row (chunks past the step repeat the last one;
    // chunks that start past the row's last block read the row's first bytes,
    // so every byte copied is real data). When a row is not a whole number of
    // chunks its last chunk also copies the first bytes after it, which the
    // host keeps inside the weights (see launch_gemv_dma).
    uint32_t dq[GD_DMA_INSTRS], doff[GD_DMA_INSTRS];
#pragma unroll
    for (uint32_t n = 0; n < GD_DMA_INSTRS; ++n) {
        const uint32_t k = min(64 * n + lane, BYTES - 1);
        const uint32_t off = SLOTS * kw * BYTES + 16 * (k % ROW_CHUNKS);
        dq[n] = k / ROW_CHUNKS;
        doff[n] = off < nblocks * BYTES ? off : 0;
    }
#define NUQ_GD_DMA(SLOT_, STEP_)                                                                              \
    _Pragma("unroll") for (uint32_t n = 0; n < GD_DMA_INSTRS; ++n) {                                          \
        const uint32_t lrow_ = min(first_local + (STEP_) * set_stride + dq[n], last_local);                   \
        __builtin_amdgcn_global_load_lds((gd_global_void_t *)(wg_base + (lrow_ * stride32 + doff[n])),        \
                                         (gd_lds_void_t *)(NUQ_GD_RING(SLOT_) + n * 1024), 16, 0, 2);         \
    }

    // Copy addresses: a uniform workgroup base plus a 32-bit offset (the
    // host keeps a workgroup's rows within 4 GiB).
    const uint8_t *wg_base = w + (uint64_t)row_begin * stride;
    const uint32_t stride32 = (uint32_t)stride;
    const uint32_t first_local = first - row_begin, last_local = row_end - 1 - row_begin;

    const uint32_t t0 = threadIdx.x;
    if constexpr (WX) {
        // Each wave quantises the slices of its own blocks (SLOTS / 4 rounds
        // of one half-slice per lane) and reads them back after its own LDS
        // writes: no workgroup barrier before the steps. Taken with one wave
        // set (gd_wave_x); with several, each set would quantise all of x
        // again (17408 x 5120 took 14.7 against 13.1-13.3 us).
        constexpr uint32_t R = SLOTS / 4;
        const uint32_t hbase = 16 * SLOTS * kw, hend = 2 * nslices;
        XHalf xr[R];
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            const uint32_t h = min(hbase + 64 * r + lane, hend - 1);
            load_half_slice_asm(x + (uint64_t)(h >> 1) * 32, h & 1, xr[r]);
        }
#pragma unroll
        for (int d = 0; d < D; ++d) NUQ_GD_DMA(d, (uint32_t)d)
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            const uint32_t h = hbase + 64 * r + lane;
            if (r == 0) xhalf_wait<GD_DMA_INSTRS * D + 4 * (R - 1)>(xr[r]);
            else xhalf_wait<GD_DMA_INSTRS * D>(xr[r]);
            if (h < hend) quantize_half_slice<true>(xr[r], h & 1, slices + (h >> 1) * SLICE_WORDS);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    } else {
    XHalf xh;
    if (t0 < 2 * nslices) load_half_slice_asm(x + (uint64_t)(t0 >> 1) * 32, t0 & 1, xh);
    // When x takes a second round of half-slices (long rows: 1088 for
    // K = 17408 over 576 threads), its loads go out with the first, before
    // the copies, instead of after the first round's quantisation. The
    // condition is uniform, and every thread issues the loads (clamped to
    // the last half-slice) so the wait counts below are exact.
    constexpr bool two_rounds = TWO;
    XHalf xh2;
    const uint32_t t1 = min(t0 + blockDim.x, 2 * nslices - 1);
    if constexpr (two_rounds) load_half_slice_asm(x + (uint64_t)(t1 >> 1) * 32, t1 & 1, xh2);
    // With two rounds, every wave's x loads go out before any wave's copies
    // (5120 x 17408: 16.2 -> 15.6 us for Q4_K, 19.5 -> 18.8 us for Q5_K).
    if constexpr (two_rounds) __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int d = 0; d < D; ++d) NUQ_GD_DMA(d, (uint32_t)d)

    // The slice image goes to LDS through asm and the barrier carries no
    // fence, so the copies in flight keep flying while x is quantised.
    if constexpr (two_rounds) {
        xhalf_wait<GD_DMA_INSTRS * D + 4>(xh);  // x is older than the second round and the copies
        if (t0 < 2 * nslices) quantize_half_slice<true>(xh, t0 & 1, slices + (t0 >> 1) * SLICE_WORDS);
        xhalf_wait<GD_DMA_INSTRS * D>(xh2);
        if (t0 + blockDim.x < 2 * nslices) quantize_half_slice<true>(xh2, t1 & 1, slices + (t1 >> 1) * SLICE_WORDS);
    } else {
        xhalf_wait<GD_DMA_INSTRS * D>(xh);  // x is older than the D steps' copies
        if (t0 < 2 * nslices) quantize_half_slice<true>(xh, t0 & 1, slices + (t0 >> 1) * SLICE_WORDS);
    }
    for (uint32_t t = t0 + 2 * blockDim.x; t < 2 * nslices; t += blockDim.x) {
        load_half_slice_asm(x + (uint64_t)(t >> 1) * 32, t & 1, xh);
        xhalf_wait<0>(xh);
        quantize_half_slice<true>(xh, t & 1, slices + (t >> 1) * SLICE_WORDS);
    }
    // the row-step counters of the K ranges (D * sets steps are assigned statically)
    if (t0 < set_waves) ((uint32_t *)(partial + rows_per_wg * set_waves + nwaves))[t0] = D * sets;
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    __builtin_amdgcn_s_barrier();
    }

    XSlice xa, xb;
    const uint32_t bb = live ? b : 0;
    read_slice_asm(slices + (bb * 8 + 2 * j) * SLICE_WORDS, xa);
    read_slice_asm(slices + (bb * 8 + 2 * j + 1) * SLICE_WORDS, xb);
    if constexpr (ENC == 14) {
        plane_sums(xa);
        plane_sums(xb);
    }
    if (!live) {
        xa.scale = xb.scale = 0.f;
        xa.sum = xb.sum = 0.f;
        xa.pos = xa.neg = xb.pos = xb.neg = 0u;
    }
    // wave-uniform: does any slice this wave reads hold a non-finite value
    const bool nonfinite = __ballot((xa.pos | xa.neg | xb.pos | xb.neg) != 0u) != 0;
    const uint32_t role = g * ROW_CHUNKS * 16 + slot * BYTES;
    const uint32_t spare = rows_per_wg * set_waves + wv;  // one spare partial per wave

    // Each ring slot holds one step. As soon as a slot's bytes are in
    // registers the slot is refilled with the wave's next step, before the
    // arithmetic. While every slot is refilled, the D-1 younger steps'
    // copies may still be in flight when slot d is read; once refills stop,
    // the remaining slots wait for all copies.
#define NUQ_GD_COMPUTE(SLOT_, STEP_, VM_, REFILL_)                                                                     \
    {                                                                                                       \
        GdEnc<ENC> e_;                                                                                      \
        e_.template read<VM_>(NUQ_GD_RING(SLOT_) + role, j);                                                \
        REFILL_                                                                                             \
        /* lanes past the row's last block read arbitrary copied bytes: select zero */                     \
        const float v = group_sum<4 * SLOTS>(live ? e_.dot(xa, xb, j, shift, direct) : 0.f);                \
        const uint32_t row = first + (STEP_) * set_stride + g;                                              \
        /* every lane of the group holds the sum; rows past the range go to a spare slot */               \
        partial[row < row_end ? (row - row_begin) * set_waves + kw : spare] = v;                            \
    }
    if constexpr (!WX) {
#define NUQ_GD_DMA2(SLOT_, C_)                                                                                \
    _Pragma("unroll") for (uint32_t n = 0; n < GD_DMA_INSTRS; ++n) {                                          \
        const uint32_t lrow_ = min((C_) * GROUPS + dq[n], last_local);                                        \
        __builtin_amdgcn_global_load_lds((gd_global_void_t *)(wg_base + (lrow_ * stride32 + doff[n])),        \
                                         (gd_lds_void_t *)(NUQ_GD_RING(SLOT_) + n * 1024), 16, 0, 2);         \
    }
#define NUQ_GD_COMPUTE2(SLOT_, C_, VM_, REFILL_)                                                            \
    {                                                                                                       \
        GdEnc<ENC> e_;                                                                                      \
        e_.template read<VM_>(NUQ_GD_RING(SLOT_) + role, j);                                                \
        REFILL_                                                                                             \
        const float v = group_sum<4 * SLOTS>(live ? e_.dot(xa, xb, j, shift, direct) : 0.f);                \
        const uint32_t row = row_begin + (C_) * GROUPS + g;                                                 \
        partial[row < row_end ? (row - row_begin) * set_waves + kw : spare] = v;                            \
    }
        // Waves of one K range (one per wave set) claim row steps from a
        // shared LDS counter, so waves that start late take fewer steps.
        const uint32_t tsteps = (row_end - row_begin + GROUPS - 1) / GROUPS;
        const uint32_t claim_addr =
            lds_u8_addr((const uint8_t *)(partial + rows_per_wg * set_waves + nwaves + kw));
        uint32_t sid[D];
        bool claiming = true;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            sid[d] = set + d * sets;
            if (sid[d] >= tsteps) claiming = false;
        }
        while (claiming) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (claiming) {
                    // The claim is issued before the ring read, whose
                    // lgkmcnt(0) also covers it (asm: the compiler would
                    // wait for every copy before an LDS atomic).
                    uint32_t c_ = 0;
                    if (lane == 0)
                        asm volatile("ds_add_rtn_u32 %0, %1, %2" : "=v"(c_) : "v"(claim_addr), "v"(1u) : "memory");
                    NUQ_GD_COMPUTE2(d, sid[d], GD_DMA_INSTRS * (D - 1),
                                    asm volatile("" : "+v"(c_));
                                    c_ = __builtin_amdgcn_readfirstlane(c_);
                                    if (c_ < tsteps) { NUQ_GD_DMA2(d, c_) } else claiming = false;)
                    sid[d] = c_;
                }
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (sid[d] < tsteps) NUQ_GD_COMPUTE2(d, sid[d], 0, )
#undef NUQ_GD_COMPUTE2
#undef NUQ_GD_DMA2
    } else {  // one wave set: each K range has one wave, steps in order
    uint32_t i = 0;
    for (; i + 2 * D <= nsteps; i += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            NUQ_GD_COMPUTE(d, i + d, GD_DMA_INSTRS * (D - 1), NUQ_GD_DMA(d, i + d + D))
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (i + d < nsteps) NUQ_GD_COMPUTE(d, i + d, 0, if (i + d + D < nsteps) { NUQ_GD_DMA(d, i + d + D) })
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (i + D + d < nsteps) NUQ_GD_COMPUTE(d, i + D + d, 0, )
    }
#undef NUQ_GD_COMPUTE
#undef NUQ_GD_DMA
#undef NUQ_GD_RING
    // Copies issued for steps past the range (when nsteps < D) must land
    // before the workgroup ends.
    __builtin_amdgcn_s_waitcnt(0x0f70);
    // Each wave's spare partial now holds its non-finite flag; every slice is
    // read by some live lane, so their OR is "x holds a non-finite value".
    if (lane == 0) partial[spare] = nonfinite ? 1.f : 0.f;
    __syncthreads();
    const bool any_nonfinite = __ballot(partial[rows_per_wg * set_waves + lane % nwaves] != 0.f) != 0;
    for (uint32_t r = threadIdx.x; r < row_end - row_begin; r += blockDim.x) {
        float t = 0.f;
        for (uint32_t k = 0; k < set_waves; ++k) t += partial[r * set_waves + k];
        if (any_nonfinite) t += nonfinite_row(ENC, w + (uint64_t)(row_begin + r) * stride, BYTES, slices, nslices);
        y[row_begin + r] = t;
    }
}

// Wave-local x quantisation (the kernel's WX form) where it measured faster
// with one wave set: 8-block lane groups of Q4_K (5120 x 17408: 15.8 -> 15.4 us,
// mean of 4 A/B pairs) and Q6_K (21.3 -> 21.1); Q5_K was 1 % slower.
template <uint32_t ENC, int SLOTS>
constexpr bool gd_wave_x() { return SLOTS == 8 && (ENC == 12 || ENC == 14); }

template <uint32_t ENC, int SLOTS, int D>
static hipError_t launch_dma(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t nblocks,
                                 const float *x, float *y, uint32_t sets_wanted, uint32_t wgs_per_cu,
                                 bool tail = false) {
    // tail: the last row goes to one extra workgroup (see the kernel)
    if (tail) {
        if (rows < 2) return hipErrorInvalidValue;
        rows -= 1;
    }
    const uint32_t cus = 256 * wgs_per_cu - (tail ? 1 : 0);
    const uint32_t set_waves = (nblocks + SLOTS - 1) / SLOTS;
    const uint32_t step_rows = 64 / (4 * SLOTS);
    if (set_waves > (uint32_t)gd_threads<ENC>() / 64) return hipErrorInvalidValue;
    uint32_t sets = (gd_threads<ENC>() / 64) / set_waves;
    // Fewer wave sets for small matrices, so the grid still covers the CUs
    // and each wave streams at least two steps: Q8_0 4096 x 4096 (16 rows
    // per workgroup) took 6.1 us with four sets of one step and 5.5 us with
    // two or one on MI355X. The wider shapes stay at their LDS-bound cap.
    // Q8_0 and Q6_K prefer half as many sets again (about four steps per
    // wave): Q8_0 4096 x 4096 5.73 -> 5.46 us, 8192 x 4096 8.9 -> 8.5, Q6_K
    // 4096 x 4096 6.24 -> 5.9; Q4_K, Q5_K and IQ4_XS measured 2-4 % slower so.
    const uint32_t per_set = (ENC == 8 || ENC == 14 ? 4 : 2) * cus * step_rows;
    if (!sets_wanted) sets_wanted = std::max(1u, rows / per_set);
    if (sets_wanted < sets) sets = sets_wanted;
    // Rows per workgroup need not be whole set steps (each set guards its
    // last step), so the grid is the CU count and each CU streams the same
    // share of the bytes.
    const uint32_t rows_per_wg = std::max(1u, (rows + cus - 1) / cus);
    // Fewer wave sets when the rings, x slices and partials exceed the LDS.
    auto lds_for = [&](uint32_t st) {
        const size_t wv = (size_t)set_waves * st;
        return wv * D * GdEnc<ENC>::INSTRS * 1024 + (size_t)nblocks * 8 * SLICE_WORDS * 4 +
               ((size_t)rows_per_wg * set_waves + wv + set_waves) * 4;
    };
    while (sets > 1 && lds_for(sets) > 160 * 1024) --sets;
    const uint32_t waves = set_waves * sets;
    const size_t lds = lds_for(sets);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if ((uint64_t)rows_per_wg * stride > 0xffffffffull) return hipErrorInvalidValue;  // 32-bit copy offsets
    const dim3 grid((rows + rows_per_wg - 1) / rows_per_wg + (tail ? 1 : 0)), block(64 * waves);
    if constexpr (gd_wave_x<ENC, SLOTS>()) {
        if (sets == 1) {  // each wave quantises its own slices
            hipLaunchKernelGGL((gemv_dma_kernel<ENC, SLOTS, D, false, true>), grid, block, lds, s, w, stride, rows,
                               nblocks, rows_per_wg, set_waves, x, y, tail ? 1u : 0u, GdSegments{});
            return hipGetLastError();
        }
    }
    if (2 * nblocks * 8 > 64 * waves)  // x in two rounds of half-slices (or more)
        hipLaunchKernelGGL((gemv_dma_kernel<ENC, SLOTS, D, true>), grid, block, lds, s, w, stride, rows, nblocks,
                           rows_per_wg, set_waves, x, y, tail ? 1u : 0u, GdSegments{});
    else
        hipLaunchKernelGGL((gemv_dma_kernel<ENC, SLOTS, D, false>), grid, block, lds, s, w, stride, rows, nblocks,
                           rows_per_wg, set_waves, x, y, tail ? 1u : 0u, GdSegments{});
    return hipGetLastError();
}

// Several matrices of one encoding and row stride against one x in a single
// launch: each gets whole workgroups, in proportion to its rows (at least
// one), and streams as it would alone. A row's sum does not depend on the
// workgroup split, so each output equals the matrix's own GEMV bit for bit.
template <uint32_t ENC, int SLOTS, int D>
static hipError_t launch_dma_segments(hipStream_t s, uint32_t count, const uint8_t *const *w, uint64_t stride,
                                      const uint32_t *rows, uint32_t nblocks, const float *x, float *const *y) {
    if (count == 0 || count > GD_MAX_SEGMENTS) return hipErrorInvalidValue;
    constexpr uint32_t cus = 256;
    uint64_t total = 0;
    for (uint32_t q = 0; q < count; ++q) {
        if (rows[q] == 0) return hipErrorInvalidValue;
        total += rows[q];
    }
    GdSegments segs{};
    segs.count = count;
    uint32_t wgs = 0, max_rpw = 0;
    for (uint32_t q = 0; q < count; ++q) {
        const uint32_t share = std::max<uint32_t>(1, (uint32_t)((cus * (uint64_t)rows[q] + total / 2) / total));
        const uint32_t rpw = (rows[q] + share - 1) / share;
        if ((uint64_t)rpw * stride > 0xffffffffull) return hipErrorInvalidValue;  // 32-bit copy offsets
        segs.w[q] = w[q];
        segs.y[q] = y[q];
        segs.rows[q] = rows[q];
        segs.rows_per_wg[q] = rpw;
        wgs += (rows[q] + rpw - 1) / rpw;
        segs.wg_end[q] = wgs;
        max_rpw = std::max(max_rpw, rpw);
    }
    const uint32_t set_waves = (nblocks + SLOTS - 1) / SLOTS;
    const uint32_t step_rows = 64 / (4 * SLOTS);
    if (set_waves > (uint32_t)gd_threads<ENC>() / 64) return hipErrorInvalidValue;
    uint32_t sets = (gd_threads<ENC>() / 64) / set_waves;
    sets = std::min(sets, std::max(1u, (uint32_t)(total / (2 * cus * step_rows))));  // as in launch_dma
    auto lds_for = [&](uint32_t st) {
        const size_t wv = (size_t)set_waves * st;
        return wv * D * GdEnc<ENC>::INSTRS * 1024 + (size_t)nblocks * 8 * SLICE_WORDS * 4 +
               ((size_t)max_rpw * set_waves + wv + set_waves) * 4;
    };
    while (sets > 1 && lds_for(sets) > 160 * 1024) --sets;
    const size_t lds = lds_for(sets);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if constexpr (gd_wave_x<ENC, SLOTS>()) {
        if (sets == 1) {  // each wave quantises its own slices
            hipLaunchKernelGGL((gemv_dma_kernel<ENC, SLOTS, D, false, true>), dim3(wgs), dim3(64 * set_waves), lds, s,
                               w[0], stride, rows[0], nblocks, max_rpw, set_waves, x, y[0], 0u, segs);
            return hipGetLastError();
        }
    }
    if (2 * nblocks * 8 > 64 * set_waves * sets)
        hipLaunchKernelGGL((gemv_dma_kernel<ENC, SLOTS, D, true>), dim3(wgs), dim3(64 * set_waves * sets), lds, s,
                           w[0], stride, rows[0], nblocks, max_rpw, set_waves, x, y[0], 0u, segs);
    else
        hipLaunchKernelGGL((gemv_dma_kernel<ENC, SLOTS, D, false>), dim3(wgs), dim3(64 * set_waves * sets), lds, s,
                           w[0], stride, rows[0], nblocks, max_rpw, set_waves, x, y[0], 0u, segs);
    return hipGetLastError();
}

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

template <int R, int SLOTS, int D>
static hipError_t launch_q4k_int(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t nblocks,
                                 const float *x, float *y, uint32_t sets_wanted, uint32_t wgs_per_cu) {
    const uint32_t set_waves = cdiv(nblocks, SLOTS);
    uint32_t sets = (GI_WG_THREADS / 64) / set_waves;
    if (sets_wanted && sets_wanted < sets) sets = sets_wanted;
    const uint32_t step_rows = (64 / (4 * SLOTS)) * R;
    const uint32_t rows_per_wg = cdiv(cdiv(rows, 256 * wgs_per_cu), step_rows) * step_rows;
    const size_t lds = (size_t)nblocks * 8 * SLICE_WORDS * 4 + (size_t)rows_per_wg * set_waves * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_q4k_int_kernel<R, SLOTS, D>), dim3(cdiv(rows, rows_per_wg)), dim3(64 * set_waves * sets), lds, s,
                       w, stride, rows, nblocks, rows_per_wg, set_waves, x, y);
    return hipGetLastError();
}

// config 0: the DMA kernel with two ring slots, or the register kernel (two
// slots, one row per lane group) when x and the rings do not fit in LDS.
// config >= 10000 forces the DMA kernel: 10000 + D*1000 + sets*10 + WGs/CU;
// other values force the register kernel: D*1000 + R*100 + sets*10 + WGs/CU.
// Returns hipErrorInvalidValue when the shape does not fit (more than 128
// blocks per row): the caller then uses the row-per-wave kernel.
hipError_t launch_gemv_q4k_int(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                               const float *x, float *y, int config) {
    const uint32_t nblocks = columns / 256;
    if (cdiv(nblocks, 8) > GI_MAX_SET_WAVES) return hipErrorInvalidValue;
    if (config >= 10000 || config <= 0) {
        // DMA kernel: config = 10000 + D*1000 + sets*10 + workgroups per CU
        const int c = config <= 0 ? 12000 : config;
        const int dd = (c / 1000) % 10, st = (c / 10) % 10, pc = c % 10 ? c % 10 : 1;
        hipError_t e = hipErrorInvalidValue;
        if (cdiv(nblocks, 4) <= GI_MAX_SET_WAVES) {
            if (dd == 2) e = launch_dma<12, 4, 2>(s, w, stride, rows, nblocks, x, y, st, pc);
            else if (dd == 3) e = launch_dma<12, 4, 3>(s, w, stride, rows, nblocks, x, y, st, pc);
        } else {
            if (dd == 2) e = launch_dma<12, 8, 2>(s, w, stride, rows, nblocks, x, y, st, pc);
            else if (dd == 3) e = launch_dma<12, 8, 3>(s, w, stride, rows, nblocks, x, y, st, pc);
        }
        if (e != hipErrorInvalidValue || config > 0) return e;
        config = 0;  // the LDS does not fit: register kernel
    }
    int D = config / 1000, R = (config / 100) % 10, sets = (config / 10) % 10, per_cu = config % 10;
    if (config <= 0) {
        D = 2;
        R = 1;
        sets = 0;
        per_cu = 1;
    }
    if (per_cu == 0) per_cu = 1;
#define NUQ_GI_CASE(D_, R_, S_) \
    if (D == D_ && R == R_) return launch_q4k_int<R_, S_, D_>(s, w, stride, rows, nblocks, x, y, sets, per_cu);
    // 4 blocks per row group while a row fits in 16 waves, else 8
    if (cdiv(nblocks, 4) <= GI_MAX_SET_WAVES) {
        NUQ_GI_CASE(2, 2, 4) NUQ_GI_CASE(2, 1, 4)
    } else {
        NUQ_GI_CASE(2, 2, 8) NUQ_GI_CASE(2, 1, 8)
    }
#undef NUQ_GI_CASE
    return hipErrorInvalidValue;
}

// Q5_K / Q6_K / IQ4_XS decode GEMV on the DMA kernel (two ring slots; Q6_K
// always with 8-block lane groups, so a row's segment is whole chunks). Returns
// hipErrorInvalidValue when the shape does not fit (more than 128 blocks per
// row, x and the rings beyond LDS, or IQ4_XS rows of an odd block count,
// whose 136-byte blocks would end mid-chunk): the caller then uses the
// generic kernel.
hipError_t launch_gemv_dma(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                           uint32_t columns, const float *x, float *y) {
    const uint32_t nblocks = columns / 256;
    if (cdiv(nblocks, 8) > GI_MAX_SET_WAVES) return hipErrorInvalidValue;
    const bool four = cdiv(nblocks, 4) <= GI_MAX_SET_WAVES;
    if (encoding == 13)
        return four ? launch_dma<13, 4, 2>(s, w, stride, rows, nblocks, x, y, 0, 1)
                    : launch_dma<13, 8, 2>(s, w, stride, rows, nblocks, x, y, 0, 1);
    if (encoding == 14)
        // A Q6_K row of nblocks % 8 != 0 blocks ends mid-chunk, so its last
        // copy reads up to 8 bytes past it: the next row for all but the
        // matrix's last row, which an extra workgroup computes directly.
        return launch_dma<14, 8, 2>(s, w, stride, rows, nblocks, x, y, 0, 1, nblocks * 210u % 16 != 0);
    if (encoding == 8 && columns % 256 == 0)  // nblocks counts 256-value units of eight Q8_0 blocks
        return four ? launch_dma<8, 4, 2>(s, w, stride, rows, nblocks, x, y, 0, 1)
                    : launch_dma<8, 8, 2>(s, w, stride, rows, nblocks, x, y, 0, 1);
    if (encoding == 23 && nblocks % 2 == 0)
        return four ? launch_dma<23, 4, 2>(s, w, stride, rows, nblocks, x, y, 0, 1)
                    : launch_dma<23, 8, 2>(s, w, stride, rows, nblocks, x, y, 0, 1);
    return hipErrorInvalidValue;
}

// The segment form of the DMA GEMV for every encoding launch_gemv_dma and
// the Q4_K DMA path take, when no row needs the separate last-row workgroup.
hipError_t launch_gemv_dma_segments(hipStream_t s, uint32_t encoding, uint32_t count, const uint8_t *const *w,
                                    uint64_t stride, const uint32_t *rows, uint32_t columns, const float *x,
                                    float *const *y) {
    const uint32_t nblocks = columns / 256;
    if (columns % 256 != 0 || cdiv(nblocks, 8) > GI_MAX_SET_WAVES) return hipErrorInvalidValue;
    const bool four = cdiv(nblocks, 4) <= GI_MAX_SET_WAVES;
#define NUQ_GD_SEG(E_) \
    return four ? launch_dma_segments<E_, 4, 2>(s, count, w, stride, rows, nblocks, x, y) \
                : launch_dma_segments<E_, 8, 2>(s, count, w, stride, rows, nblocks, x, y);
    if (encoding == 12) NUQ_GD_SEG(12)
    if (encoding == 13) NUQ_GD_SEG(13)
    if (encoding == 8) NUQ_GD_SEG(8)
    if (encoding == 23 && nblocks % 2 == 0) NUQ_GD_SEG(23)
#undef NUQ_GD_SEG
    if (encoding == 14 && nblocks * 210u % 16 == 0)
        return launch_dma_segments<14, 8, 2>(s, count, w, stride, rows, nblocks, x, y);
    return hipErrorInvalidValue;
}


// ---------------------------------------------------------------------------
// Register-dequant multi-token GEMV (matvecRows form, backends/metal/kernels/
// matvec_rows.metal:34-130: decode each weight once, dot it with every token)
// for Q4_K with f16 activations, 1..8 tokens: KERNEL_ROWS.
//
// Each weight is decoded once into registers as the exact f16 integer q*sc
// (at most 15*63 = 945) and meets every token's f16 activations in
// v_dot2_f32_f16 (two exact products per op, F32 accumulation), so the
// products are exact and only the F32 sums round, as in an F32 FMA chain;
// the block's d and the minimum term dmin*m*sum(x) are applied in F32.
//
// Layout: the K-split of the decode GEMV. Lane = (block slot 0..7, sub s
// 0..7): s / 2 is the block's nibble pair j (groups 2j and 2j+1), and the
// lane takes code bytes 16*(s%2) .. +15 of the pair, i.e. 16 values of each
// of the two groups. Wave kw of a wave set owns blocks [8kw, 8kw + 8) of
// every row of its K range, so each lane keeps its 32 activations of every
// token in registers (16 f16 pairs per token) with their per-group F32 sums
// for the whole launch. A step is 4 rows x the wave's 8 blocks, copied
// global -> LDS into a private two-slot ring as the decode GEMV copies its
// steps; the lanes then take the 4 rows in turn. A row's token partials are
// reduced across the wave with a reduce-scatter (each row-swap or DPP stage
// halves the values a lane holds), so lane (64 / NT) * t ends with token t's
// sum; per-wave partials meet in LDS and are added in wave order. Rows
// longer than 24 blocks run as K ranges (blockIdx.y) whose sums
// verify_reduce_kernel adds.

// 8 tokens hold 128 registers of activations: 8 waves (256 registers) there
template <int NT>
constexpr int rd_threads() { return NT == 8 ? 512 : NT == 4 ? 768 : 1024; }
constexpr uint32_t RD_ROW_CHUNKS = 8 * 144 / 16;                        // 72: a row's 8 blocks
constexpr uint32_t RD_INSTRS = (4 * RD_ROW_CHUNKS + 63) / 64;           // 5 copies per 4-row step
constexpr uint32_t RD_SLOT_BYTES = RD_INSTRS * 1024;

typedef _Float16 rd_half2_t __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ __forceinline__ float rd_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the wave's 64 lanes of each of a lane's NT token values, as a
// reduce-scatter: each stage halves the values a lane holds, the lanes
// whose bit is clear keeping the first half. Bits 32 and 16 swap rows with
// v_permlane32_swap / v_permlane16_swap (one swap and one add per value),
// bit 8 pairs lanes with a DPP row mirror; the lanes left holding one token
// then add the rest of their group. Returns the total of token
// (lane / (64 / NT)) % NT, held by every lane of that group.
__device__ __forceinline__ void rd_swap32(float &a, float &b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ void rd_swap16(float &a, float &b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
template <int NT>
__device__ __forceinline__ float rd_reduce(float *v, uint32_t lane) {
#pragma unroll
    for (int k = 0; k < NT / 2; ++k) rd_swap32(v[k], v[k + NT / 2]);
    if constexpr (NT >= 4) {
#pragma unroll
        for (int k = 0; k < NT / 4; ++k) rd_swap16(v[k], v[k + NT / 4]);
    }
    float r = v[0];
    if constexpr (NT == 8) {  // bit 8: row_mirror pairs lane i with 15 - i
        const bool lower = (lane & 8) == 0;
        const float send = lower ? v[1] : v[0], keep = lower ? v[0] : v[1];
        r = keep + rd_dpp<0x140>(send);
    }
    if constexpr (NT == 2) {  // the other half of the 32 lanes
        float t = r;
        rd_swap16(r, t);
    }
    if constexpr (NT <= 4) r += rd_dpp<0x140>(r);  // row_mirror
    r += rd_dpp<0x141>(r);                       // row_half_mirror
    r += rd_dpp<0x4e>(r);                        // quad_perm [2,3,0,1]
    r += rd_dpp<0xb1>(r);                        // quad_perm [1,0,3,2]
    return r;
}

// q*sc of 4 low (or high) nibbles as two exact f16 pairs: bytes (1024 + q)
// via v_perm_b32 from the nibble word and 0x64 bytes, then (1024 + q)*sc -
// 1024*sc in one v_pk_fma_f16 (the product is exact before the one rounding).
__device__ __forceinline__ void rd_codes(uint32_t nib, rd_half2_t sc, rd_half2_t nsc, rd_half2_t &p0, rd_half2_t &p1) {
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u);
    p0 = __builtin_elementwise_fma(__builtin_bit_cast(rd_half2_t, a), sc, nsc);
    p1 = __builtin_elementwise_fma(__builtin_bit_cast(rd_half2_t, b), sc, nsc);
}

template <int NT>
__global__ void __launch_bounds__(rd_threads<NT>()) rows_dma_kernel(const uint8_t *__restrict__ w, uint64_t stride,
                                                                      uint32_t rows, uint32_t nblocks_all,
                                                                      uint32_t ranges, uint32_t rows_per_wg,
                                                                      uint32_t set_waves,
                                                                      const _Float16 *__restrict__ x,
                                                                      uint64_t in_stride, uint32_t tokens,
                                                                      float *__restrict__ y, uint64_t out_stride) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    constexpr uint32_t BYTES = 144, ROW_CHUNKS = RD_ROW_CHUNKS, INSTRS = RD_INSTRS;
    const uint32_t range = blockIdx.y;
    const uint32_t b0 = range * nblocks_all / ranges, kb = (range + 1) * nblocks_all / ranges - b0;
    w += (uint64_t)b0 * BYTES;
    x += (uint64_t)b0 * 256;

    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    uint8_t *ring = (uint8_t *)lds + wv * 2 * RD_SLOT_BYTES;
    // rows_per_wg * set_waves * NT partials, 64 spare words per wave, then
    // one row-step counter per K range
    float *partial = (float *)(lds + nwaves * 2 * (RD_SLOT_BYTES / 4));
    const uint32_t sets = nwaves / set_waves;
    const uint32_t set = wv / set_waves, kw = wv % set_waves;
    const uint32_t slot = lane >> 3, sub = lane & 7, j = sub >> 1, c0 = 16 * (sub & 1);
    const bool direct = j < 2;
    const uint32_t shift = direct ? 16 * j : 16 * j - 32;
    const uint32_t b = 8 * kw + slot;
    const bool live = b < kb;
    const uint32_t row_begin = blockIdx.x * rows_per_wg;
    const uint32_t row_end = min(row_begin + rows_per_wg, rows);
    // Step c covers rows row_begin + 4c .. 4c + 3. The waves of one K range
    // (one per wave set) take steps set and set + sets, then claim further
    // steps from their range's LDS counter, so waves that share a SIMD with
    // another take fewer steps than waves alone on theirs.
    const uint32_t first = row_begin, set_stride = 4;
    const uint32_t tsteps = (row_end - row_begin + 3) / 4;
    const uint32_t counters = lds_u8_addr((const uint8_t *)(partial + rows_per_wg * set_waves * NT + nwaves * 64));
    if (threadIdx.x < set_waves) ((uint32_t *)(partial + rows_per_wg * set_waves * NT + nwaves * 64))[threadIdx.x] = 2 * sets;
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    __builtin_amdgcn_s_barrier();

    // DMA: lane i of copy n moves chunk 64n + i of the step (4 rows x 8 blocks)
    uint32_t dq[INSTRS], doff[INSTRS];
#pragma unroll
    for (uint32_t n = 0; n < INSTRS; ++n) {
        const uint32_t k = min(64 * n + lane, 4 * ROW_CHUNKS - 1);
        const uint32_t off = 8 * kw * BYTES + 16 * (k % ROW_CHUNKS);
        dq[n] = k / ROW_CHUNKS;
        doff[n] = off < kb * BYTES ? off : 0;
    }
    const uint8_t *wg_base = w + (uint64_t)row_begin * stride;
    const uint32_t stride32 = (uint32_t)stride;
    const uint32_t first_local = first - row_begin, last_local = row_end - 1 - row_begin;
#define NUQ_RD_DMA(SLOT_, STEP_)                                                                           \
    _Pragma("unroll") for (uint32_t n = 0; n < INSTRS; ++n) {                                              \
        const uint32_t lrow_ = min(first_local + (STEP_) * set_stride + dq[n], last_local);                \
        __builtin_amdgcn_global_load_lds((gd_global_void_t *)(wg_base + (lrow_ * stride32 + doff[n])),     \
                                         (gd_lds_void_t *)(ring + (SLOT_) * RD_SLOT_BYTES + n * 1024), 16, 0, 2); \
    }
    uint32_t sid0 = set, sid1 = set + sets;
    NUQ_RD_DMA(0, sid0)
    NUQ_RD_DMA(1, sid1)

    // this lane's 16 + 16 activations of every token, and their F32 sums
    uint4 xa[NT][2], xb[NT][2];
    float sa_x[NT], sb_x[NT];
    {
        const uint32_t col = (live ? b : 0) * 256 + 64 * j + c0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const _Float16 *p = x + (uint64_t)min((uint32_t)t, tokens - 1) * in_stride + col;
            xa[t][0] = *(const uint4 *)p;
            xa[t][1] = *(const uint4 *)(p + 8);
            xb[t][0] = *(const uint4 *)(p + 32);
            xb[t][1] = *(const uint4 *)(p + 40);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            // group sums: 1*x0 + 1*x1 per v_dot2_f32_f16, the products exact
            const rd_half2_t one = {(_Float16)1.f, (_Float16)1.f};
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if ((uint32_t)t >= tokens || !live) xa[t][h] = xb[t][h] = make_uint4(0, 0, 0, 0);
                const uint32_t wa[4] = {xa[t][h].x, xa[t][h].y, xa[t][h].z, xa[t][h].w};
                const uint32_t wb[4] = {xb[t][h].x, xb[t][h].y, xb[t][h].z, xb[t][h].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    s0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(rd_half2_t, wa[k]), one, s0, false);
                    s1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(rd_half2_t, wb[k]), one, s1, false);
                }
            }
            sa_x[t] = s0;
            sb_x[t] = s1;
        }
    }
    const uint32_t spare = rows_per_wg * set_waves * NT + wv * 64;
    const uint32_t hdr_base = lds_u8_addr(ring) + slot * BYTES;
    const uint32_t code_base = hdr_base + 16 + 32 * j + c0;

    // A row's header and code chunk are read from the ring one row ahead
    // (the first row of a step right after its copies land), so the LDS
    // latency of row q + 1 hides under row q's arithmetic.
    u32x4_t hn_, cn_;
#define NUQ_RD_READ(SLOT_, Q_)                                                                              \
    asm volatile("ds_read_b128 %0, %2 offset:%4\n\t"                                                        \
                 "ds_read_b128 %1, %3 offset:%4"                                                            \
                 : "=&v"(hn_), "=&v"(cn_)                                                                   \
                 : "v"(hdr_base), "v"(code_base), "n"((SLOT_) * RD_SLOT_BYTES + (Q_) * (ROW_CHUNKS * 16))   \
                 : "memory");
#define NUQ_RD_ROW(SLOT_, STEP_, Q_, NEXT_)                                                                 \
    {                                                                                                       \
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(hn_), "+v"(cn_) : : "memory");                           \
        const u32x4_t h_ = hn_, c_ = cn_;                                                                   \
        NEXT_                                                                                               \
        /* lanes past the row's last block read arbitrary copied bytes: their d and dmin are zero (their */ \
        /* activations are zero too, and the q*sc from any bytes are finite) */                             \
        const float d_ = live ? half_bits(h_.x & 0xffffu) : 0.f;                                            \
        const float dmin_ = live ? half_bits(h_.x >> 16) : 0.f;                                             \
        float sa_, ma_, sb_, mb_;                                                                           \
        q4k_pair_f(h_.y, h_.z, h_.w, shift, direct, sa_, ma_, sb_, mb_);                                    \
        const float dma_ = -(dmin_ * ma_), dmb_ = -(dmin_ * mb_);                                           \
        const rd_half2_t sca_ = {(_Float16)sa_, (_Float16)sa_}, scb_ = {(_Float16)sb_, (_Float16)sb_};      \
        const rd_half2_t nsa_ = sca_ * (_Float16)-1024.f, nsb_ = scb_ * (_Float16)-1024.f;                   \
        const uint32_t cw_[4] = {c_.x, c_.y, c_.z, c_.w};                                                   \
        rd_half2_t wa_[8], wb_[8];                                                                          \
        _Pragma("unroll") for (int k = 0; k < 4; ++k) {                                                     \
            rd_codes(cw_[k] & 0x0f0f0f0fu, sca_, nsa_, wa_[2 * k], wa_[2 * k + 1]);                         \
            rd_codes((cw_[k] >> 4) & 0x0f0f0f0fu, scb_, nsb_, wb_[2 * k], wb_[2 * k + 1]);                  \
        }                                                                                                   \
        float v_[NT];                                                                                       \
        _Pragma("unroll") for (int t = 0; t < NT; ++t) {                                                    \
            float acc = 0.f;                                                                                \
            _Pragma("unroll") for (int h = 0; h < 2; ++h) {                                                 \
                acc = __builtin_amdgcn_fdot2(wa_[4 * h + 0], __builtin_bit_cast(rd_half2_t, xa[t][h].x), acc, false); \
                acc = __builtin_amdgcn_fdot2(wa_[4 * h + 1], __builtin_bit_cast(rd_half2_t, xa[t][h].y), acc, false); \
                acc = __builtin_amdgcn_fdot2(wa_[4 * h + 2], __builtin_bit_cast(rd_half2_t, xa[t][h].z), acc, false); \
                acc = __builtin_amdgcn_fdot2(wa_[4 * h + 3], __builtin_bit_cast(rd_half2_t, xa[t][h].w), acc, false); \
                acc = __builtin_amdgcn_fdot2(wb_[4 * h + 0], __builtin_bit_cast(rd_half2_t, xb[t][h].x), acc, false); \
                acc = __builtin_amdgcn_fdot2(wb_[4 * h + 1], __builtin_bit_cast(rd_half2_t, xb[t][h].y), acc, false); \
                acc = __builtin_amdgcn_fdot2(wb_[4 * h + 2], __builtin_bit_cast(rd_half2_t, xb[t][h].z), acc, false); \
                acc = __builtin_amdgcn_fdot2(wb_[4 * h + 3], __builtin_bit_cast(rd_half2_t, xb[t][h].w), acc, false); \
            }                                                                                               \
            v_[t] = fmaf(d_, acc, fmaf(dma_, sa_x[t], dmb_ * sb_x[t]));                                     \
        }                                                                                                   \
        const float tot_ = rd_reduce<NT>(v_, lane);                                                         \
        const uint32_t row_ = first + (STEP_) * set_stride + (Q_);                                          \
        /* lane (64 / NT) t holds token t's total; the other lanes write to this wave's spare words */     \
        const bool writer_ = (lane & (64 / NT - 1)) == 0 && row_ < row_end;                                 \
        partial[writer_ ? ((row_ - row_begin) * set_waves + kw) * NT + lane / (64 / NT) : spare + lane] = tot_; \
    }
    // Each ring slot holds one step; once its 4 rows are read the slot is
    // refilled with the wave's next claimed step. The claim (an LDS atomic
    // in asm: as a compiler atomic it would first wait for every copy in
    // flight) is issued before the step's reads, whose waits cover it.
#define NUQ_RD_STEP(SLOT_, STEP_, VM_, CLAIM_, REFILL_)                                                      \
    {                                                                                                        \
        asm volatile("s_waitcnt vmcnt(%0)" : : "n"(VM_) : "memory");                                        \
        CLAIM_                                                                                               \
        NUQ_RD_READ(SLOT_, 0)                                                                                \
        NUQ_RD_ROW(SLOT_, STEP_, 0, NUQ_RD_READ(SLOT_, 1))                                                   \
        NUQ_RD_ROW(SLOT_, STEP_, 1, NUQ_RD_READ(SLOT_, 2))                                                   \
        NUQ_RD_ROW(SLOT_, STEP_, 2, NUQ_RD_READ(SLOT_, 3))                                                   \
        NUQ_RD_ROW(SLOT_, STEP_, 3, )                                                                        \
        asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); /* the slot's reads are done */                \
        REFILL_                                                                                              \
    }
#define NUQ_RD_CLAIM                                                                                         \
    if (lane == 0) asm volatile("ds_add_rtn_u32 %0, %1, %2" : "=v"(c_) : "v"(claim_addr), "v"(1u) : "memory");
#define NUQ_RD_NEXT(SLOT_, SID_)                                                                             \
    asm volatile("" : "+v"(c_));                                                                             \
    c_ = __builtin_amdgcn_readfirstlane(c_);                                                                 \
    if (c_ < tsteps) {                                                                                       \
        NUQ_RD_DMA(SLOT_, c_)                                                                                \
    } else {                                                                                                 \
        claiming = false;                                                                                    \
    }                                                                                                        \
    SID_ = c_;
    // the x loads were issued after the first two steps' copies: wait for all
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    const uint32_t claim_addr = counters + 4 * kw;
    bool claiming = sid0 < tsteps && sid1 < tsteps;
    while (claiming) {
        uint32_t c_ = 0;
        NUQ_RD_STEP(0, sid0, INSTRS, NUQ_RD_CLAIM, NUQ_RD_NEXT(0, sid0))
        if (!claiming) break;
        c_ = 0;
        NUQ_RD_STEP(1, sid1, INSTRS, NUQ_RD_CLAIM, NUQ_RD_NEXT(1, sid1))
    }
    // the steps still held, with full waits (fewer copies are in flight)
    if (sid0 < tsteps) NUQ_RD_STEP(0, sid0, 0, , )
    if (sid1 < tsteps) NUQ_RD_STEP(1, sid1, 0, , )
#undef NUQ_RD_NEXT
#undef NUQ_RD_CLAIM
#undef NUQ_RD_STEP
#undef NUQ_RD_ROW
#undef NUQ_RD_READ
#undef NUQ_RD_DMA
    __builtin_amdgcn_s_waitcnt(0x0f70);  // copies issued for steps past the range land before the end
    __syncthreads();
    const uint32_t n = (row_end - row_begin) * tokens;
    for (uint32_t e = threadIdx.x; e < n; e += blockDim.x) {
        const uint32_t t = e / (row_end - row_begin), r = e % (row_end - row_begin);
        float v = 0.f;
        for (uint32_t k = 0; k < set_waves; ++k) v += partial[(r * set_waves + k) * NT + t];
        if (ranges == 1) y[(uint64_t)t * out_stride + row_begin + r] = v;
        else y[((uint64_t)range * tokens + t) * rows + row_begin + r] = v;
    }
}

// KERNEL_ROWS for Q4_K with f16 activations (1..8 tokens). `ws` (rows *
// tokens * ranges floats, or null) takes the K ranges of rows longer than
// 24 blocks. Returns false (nothing launched) for shapes it does not take.
bool launch_rows_q4k_f16(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                         const _Float16 *x, uint64_t in_stride, float *y, uint64_t out_stride, uint32_t tokens,
                         float *ws, uint64_t ws_floats, hipError_t *err) {
    if (tokens < 1 || tokens > 8 || columns % 256 != 0 || rows < 4) return false;
    if (((uintptr_t)x & 15) != 0 || (in_stride * 2) % 16 != 0) return false;
    const uint32_t nb = columns / 256;
    // K ranges: one when a wave set (8 blocks per wave) holds the row in at
    // most 3 waves, else the range count up to 4 with the fewest idle block
    // slots (68 blocks: 3 ranges of 22-23 blocks, 3 waves each)
    uint32_t ranges = 0, best_waste = ~0u;
    for (uint32_t r = 1; r <= 4; ++r) {
        const uint32_t kb = (nb + r - 1) / r, sw = (kb + 7) / 8;
        if (sw > 3) continue;
        const uint32_t waste = sw * 8 * r - nb;
        if (ranges == 0 || waste < best_waste) {
            ranges = r;
            best_waste = waste;
        }
        if (r == 1) break;  // one range needs no reduce pass
    }
    if (ranges == 0) return false;
    if (ranges > 1 && (!ws || (uint64_t)ranges * tokens * rows > ws_floats)) return false;
    const uint32_t set_waves = ((nb + ranges - 1) / ranges + 7) / 8;
    const uint32_t nt = tokens <= 2 ? 2 : tokens <= 4 ? 4 : 8;
    const uint32_t max_waves = (nt == 8 ? rd_threads<8>() : nt == 4 ? rd_threads<4>() : rd_threads<2>()) / 64;
    const uint32_t sets = std::max(1u, max_waves / set_waves);
    const uint32_t nwaves = sets * set_waves;
    const uint32_t wgs = std::max(1u, 256 / ranges);
    const uint32_t rows_per_wg = std::max(4u, (rows + wgs - 1) / wgs);
    if ((uint64_t)rows_per_wg * stride > 0xffffffffull) return false;
    const size_t lds =
        (size_t)nwaves * 2 * RD_SLOT_BYTES + ((size_t)rows_per_wg * set_waves * nt + nwaves * 64 + set_waves) * 4;
    if (lds > 160 * 1024) return false;
    const dim3 grid((rows + rows_per_wg - 1) / rows_per_wg, ranges), block(64 * nwaves);
    float *out = ranges > 1 ? ws : y;
#define NUQ_RD_LAUNCH(NT_)                                                                                   \
    hipLaunchKernelGGL((rows_dma_kernel<NT_>), grid, block, lds, s, w, stride, rows, nb, ranges, rows_per_wg, \
                       set_waves, x, in_stride, tokens, out, out_stride)
    if (nt == 2) NUQ_RD_LAUNCH(2);
    else if (nt == 4) NUQ_RD_LAUNCH(4);
    else NUQ_RD_LAUNCH(8);
#undef NUQ_RD_LAUNCH
    *err = hipGetLastError();
    if (*err == hipSuccess && ranges > 1) *err = launch_verify_reduce(s, ws, ranges, rows, tokens, y, out_stride);
    return true;
}

}  // namespace nuq

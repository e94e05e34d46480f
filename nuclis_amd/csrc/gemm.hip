// LDS-dequant f16 MFMA tile for verify (M = 4..) and prefill (M = 512 / 4096).
//
// out[t][r] = sum_c W[r][c] * x[t][c]: A = activations (tokens x K), B = W^T
// (K x rows), D = tokens x rows, F32 accumulate on v_mfma_f32_32x32x16_f16.
//
// Workgroup tile: BM tokens x BN weight rows, K stepped by 64 columns.
// Per K step every thread dequantises 32 weight values of one row straight
// from the raw GGUF bytes (Q4_K: one 16-byte qs chunk = 16 values of group 2p
// and 16 of group 2p+1; Q6_K: one 32-column quarter; Q8_0: one block) in
// the CPU decoder's operation order, rounds them to f16 and writes them to
// LDS; activations are staged beside them as f16. Both LDS tiles are
// K-contiguous per row, which is exactly the per-lane operand layout of the
// 32x32x16 MFMA (lane l: row l%32, k = 8*(l/32)..+8), so each operand
// fragment is one 16-byte LDS read. Rows are padded by 8 halves to spread
// the 32 rows of a fragment over the LDS banks.
#include <algorithm>
#include <type_traits>

#include "formats.h"
#include "kernels.h"

namespace nuq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int LDS_PITCH = BK + 8;  // halves

// Dequantise the 32 values a thread owns for K step `ks` of one row into
// `out` (f16, the LDS row base for that row), placing them at their local k.
template <uint32_t ENC>
__device__ __forceinline__ void dequant_step(const uint8_t *__restrict__ row, uint32_t ks, uint32_t part,
                                             _Float16 *__restrict__ out) {
#pragma clang fp contract(off)
    if constexpr (ENC == 12) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 144;
        const uint32_t p = ks & 3;
        uint4 hdr = *(const uint4 *)blk;
        uint4 qs = *(const uint4 *)(blk + 16 + p * 32 + part * 16);
        float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * p, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        q4k_scale_min(2 * p + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        float mul0 = d * (float)sc0, off0 = dmin * (float)m0;
        float mul1 = d * (float)sc1, off1 = dmin * (float)m1;
        const uint32_t words[4] = {qs.x, qs.y, qs.z, qs.w};
        half8 lo[2], hi[2];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float a = mul0 * (float)((words[k] >> (8 * e)) & 15u);
                float b = mul1 * (float)((words[k] >> (8 * e + 4)) & 15u);
                lo[k >> 1][(k & 1) * 4 + e] = (_Float16)(a - off0);
                hi[k >> 1][(k & 1) * 4 + e] = (_Float16)(b - off1);
            }
        }
        *(half8 *)(out + part * 16) = lo[0];
        *(half8 *)(out + part * 16 + 8) = lo[1];
        *(half8 *)(out + 32 + part * 16) = hi[0];
        *(half8 *)(out + 32 + part * 16 + 8) = hi[1];
    } else if constexpr (ENC == 14) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 210;
        const uint32_t h = (ks & 3) >> 1;
        const uint32_t q = 2 * (ks & 1) + part;  // quarter 0..3 within half h
        const uint8_t *ql = blk + h * 64 + (q & 1) * 32;
        const uint8_t *qh = blk + 128 + h * 32;
        const uint32_t lshift = (q >> 1) * 4, hshift = 2 * q;
        float d = half_bits(load_u16_bytes(blk + 208));
        float mul_a = d * (float)(int8_t)blk[192 + h * 8 + 2 * q];
        float mul_b = d * (float)(int8_t)blk[192 + h * 8 + 2 * q + 1];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t lw = load_u32_unaligned(ql + 4 * k);
            uint32_t hw = load_u32_unaligned(qh + 4 * k);
            uint32_t u = ((lw >> lshift) & 0x0f0f0f0fu) | (((hw >> hshift) & 0x03030303u) << 4);
            float mul = k < 4 ? mul_a : mul_b;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                out[part * 32 + 4 * k + e] = (_Float16)(mul * (float)((int)((u >> (8 * e)) & 0xffu) - 32));
        }
    } else if constexpr (ENC == 13) {
        // Q5_K: as Q4_K, with bit 2p (low-nibble group) or 2p+1 of high-plane
        // byte c as bit 4 of column c's code
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 176;
        const uint32_t p = ks & 3;
        uint4 hdr = *(const uint4 *)blk;
        uint4 qh = *(const uint4 *)(blk + 16 + part * 16);
        uint4 qs = *(const uint4 *)(blk + 48 + p * 32 + part * 16);
        float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * p, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        q4k_scale_min(2 * p + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        float mul0 = d * (float)sc0, off0 = dmin * (float)m0;
        float mul1 = d * (float)sc1, off1 = dmin * (float)m1;
        const uint32_t words[4] = {qs.x, qs.y, qs.z, qs.w}, highs[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = (words[k] & 0x0f0f0f0fu) | (((highs[k] >> (2 * p)) & 0x01010101u) << 4);
            const uint32_t hi = ((words[k] >> 4) & 0x0f0f0f0fu) | (((highs[k] >> (2 * p + 1)) & 0x01010101u) << 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float a = mul0 * (float)((lo >> (8 * e)) & 0xffu);
                float b = mul1 * (float)((hi >> (8 * e)) & 0xffu);
                out[part * 16 + 4 * k + e] = (_Float16)(a - off0);
                out[32 + part * 16 + 4 * k + e] = (_Float16)(b - off1);
            }
        }
    } else if constexpr (ENC == 23) {
        // IQ4_XS: this thread owns group 2p + part (32 values)
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 136;
        const uint32_t g = 2 * (ks & 3) + part;
        const uint2 hdr = *(const uint2 *)blk;
        const uint32_t low = (hdr.y >> (8 * (g / 2) + 4 * (g % 2))) & 15u;
        const int sc = (int)(low | (((hdr.x >> (16 + 2 * g)) & 3u) << 4)) - 32;
        const float mul = half_bits(hdr.x & 0xffffu) * (float)sc;
        const uint2 q01 = *(const uint2 *)(blk + 8 + 16 * g), q23 = *(const uint2 *)(blk + 16 + 16 * g);
        const uint32_t words[4] = {q01.x, q01.y, q23.x, q23.y};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t tl = iq4_lookup(words[k] & 0x0f0f0f0fu), th = iq4_lookup((words[k] >> 4) & 0x0f0f0f0fu);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                out[part * 32 + 4 * k + e] = (_Float16)(mul * (float)(int8_t)((tl >> (8 * e)) & 0xffu));
                out[part * 32 + 16 + 4 * k + e] = (_Float16)(mul * (float)(int8_t)((th >> (8 * e)) & 0xffu));
            }
        }
    } else {
        const uint8_t *blk = row + (uint64_t)(2 * ks + part) * 34;
        float d = half_bits(load_u16_bytes(blk));
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t wv = load_u32_unaligned(blk + 2 + 4 * k);
#pragma unroll
            for (int e = 0; e < 4; ++e) out[part * 32 + 4 * k + e] = (_Float16)(d * (float)(int8_t)((wv >> (8 * e)) & 0xff));
        }
    }
}

// BM x BN = 128 x 128, 256 threads as 2 x 2 waves of 64 x 64.
template <uint32_t ENC, bool XF16>
__global__ void __launch_bounds__(256) tile_kernel(const uint8_t *__restrict__ w, uint64_t stride, uint32_t rows,
                                                    uint32_t columns, const void *__restrict__ xv,
                                                    uint64_t in_stride, float *__restrict__ y, uint64_t out_stride,
                                                    uint32_t tokens) {
    constexpr int BM = 128, BN = 128;
    __shared__ __attribute__((aligned(16))) _Float16 xs[BM * LDS_PITCH];
    __shared__ __attribute__((aligned(16))) _Float16 ws[BN * LDS_PITCH];

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t n_base = blockIdx.x * BN, m_base = blockIdx.y * BM;

    // staging roles: thread -> (row, part)
    const uint32_t srow = tid >> 1, part = tid & 1;
    const uint32_t wrow = min(n_base + srow, rows - 1);
    const uint8_t *wrow_ptr = w + (uint64_t)wrow * stride;
    const uint32_t xtok = m_base + srow;
    const bool xvalid = xtok < tokens;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const uint32_t ksteps = columns / BK;
    for (uint32_t ks = 0; ks < ksteps; ++ks) {
        // activations: 32 values of token row xtok at k = 32*part
        half8 xr[4];
        if (xvalid) {
            if constexpr (XF16) {
                const half8 *src = (const half8 *)((const _Float16 *)xv + (uint64_t)xtok * in_stride + ks * BK + part * 32);
#pragma unroll
                for (int k = 0; k < 4; ++k) xr[k] = src[k];
            } else {
                const float4 *src = (const float4 *)((const float *)xv + (uint64_t)xtok * in_stride + ks * BK + part * 32);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float4 a = src[2 * k], b = src[2 * k + 1];
                    xr[k][0] = (_Float16)a.x; xr[k][1] = (_Float16)a.y; xr[k][2] = (_Float16)a.z; xr[k][3] = (_Float16)a.w;
                    xr[k][4] = (_Float16)b.x; xr[k][5] = (_Float16)b.y; xr[k][6] = (_Float16)b.z; xr[k][7] = (_Float16)b.w;
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int e = 0; e < 8; ++e) xr[k][e] = (_Float16)0.f;
        }
        __syncthreads();  // previous step's fragments have been read
#pragma unroll
        for (int k = 0; k < 4; ++k) *(half8 *)(xs + srow * LDS_PITCH + part * 32 + 8 * k) = xr[k];
        dequant_step<ENC>(wrow_ptr, ks, part, ws + srow * LDS_PITCH);
        __syncthreads();

#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const uint32_t koff = kk * 16 + 8 * (lane >> 5);
            half8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *(const half8 *)(xs + (wm * 64 + i * 32 + (lane & 31)) * LDS_PITCH + koff);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *(const half8 *)(ws + (wn * 64 + j * 32 + (lane & 31)) * LDS_PITCH + koff);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }

    // D layout: lane holds column n = lane%32; register r holds row
    // m = 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n_base + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m_base + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < tokens && n < rows) y[(uint64_t)m * out_stride + n] = acc[i][j][r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill tile: BM x BN = 256 tokens x 256 weight rows, 512 threads as 2 x 4
// waves of 128 x 64 (4 x 2 MFMA 32x32 blocks, 128 F32 accumulators a lane).
// LDS holds two K slabs (double buffer): while the MFMAs of slab k run, the
// raw GGUF bytes and activations of slab k+1 are in flight in registers;
// they are dequantised into the other buffer after the MFMAs, so there is
// one barrier per slab.
//
// Workgroup order: the hardware deals workgroups to the 8 XCDs round-robin,
// each XCD with its own L2. The linear id is first regrouped so that every
// XCD owns a contiguous range of tiles, then walked GROUP_M tiles down the
// token axis before moving across rows, so the ~32 workgroups resident on
// one XCD share a few activation panels and weight panels in its L2.
template <typename XT>
struct XLoad;
template <>
struct XLoad<_Float16> {
    half8 v[4];
    __device__ __forceinline__ void load(const _Float16 *p, bool valid) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (valid) v[k] = ((const half8 *)p)[k];
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) v[k][e] = (_Float16)0.f;
        }
    }
    __device__ __forceinline__ void store(_Float16 *dst, uint32_t c) const { *(half8 *)(dst + 8 * c) = v[c]; }
};
template <>
struct XLoad<float> {
    float4 v[8];
    __device__ __forceinline__ void load(const float *p, bool valid) {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = valid ? ((const float4 *)p)[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __device__ __forceinline__ void store(_Float16 *dst, uint32_t k) const {
        half8 h;
        h[0] = (_Float16)v[2 * k].x; h[1] = (_Float16)v[2 * k].y; h[2] = (_Float16)v[2 * k].z; h[3] = (_Float16)v[2 * k].w;
        h[4] = (_Float16)v[2 * k + 1].x; h[5] = (_Float16)v[2 * k + 1].y; h[6] = (_Float16)v[2 * k + 1].z; h[7] = (_Float16)v[2 * k + 1].w;
        *(half8 *)(dst + 8 * k) = h;
    }
};

typedef _Float16 half4v_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Two f16 values 1024 + v from bytes i and j of t (each v < 1024): the
// byte goes into the low mantissa byte of 1024.0 (0x6400, ulp 1) by one
// v_perm_b32 whose second source supplies the 0x64 exponent bytes.
template <int I, int J>
__device__ __forceinline__ half2v f16_biased(uint32_t t) {
    constexpr uint32_t sel = (uint32_t)I | (4u << 8) | ((uint32_t)J << 16) | (4u << 24);
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, t, sel));
}

// Four weights mul*(b - bias) + add, rounded to f16, from the four bytes b of
// t: the bytes become exact f16 integers b - bias (one v_perm_b32 and one
// v_pk_add_f16 per pair), and the F32 product-sum is rounded to f16 by
// v_fma_mix (the F32 FMA's value, converted).
__device__ __forceinline__ half4v_t pf_four(uint32_t t, _Float16 bias, float mul, float add) {
    const half2v p = f16_biased<0, 1>(t) - (half2v){bias, bias};
    const half2v q = f16_biased<2, 3>(t) - (half2v){bias, bias};
    half4v_t r;
    r[0] = (_Float16)fmaf((float)p[0], mul, add);
    r[1] = (_Float16)fmaf((float)p[1], mul, add);
    r[2] = (_Float16)fmaf((float)q[0], mul, add);
    r[3] = (_Float16)fmaf((float)q[1], mul, add);
    return r;
}

// Raw bytes of the 32 weight values a thread owns in one K slab, kept in
// registers between the global load and the dequantisation. `dequant(c)`
// writes chunk c (0..3) of the 32 values, so the work can be spread between
// the MFMA sub-steps. Values are (d*sc)*q - dmin*m (Q4_K), (d*sc)*(q-32)
// (Q6_K) and d*q (Q8_0) in F32 with one FMA, then rounded to f16; the
// decoders' separate rounding of the product is not kept here (the tile
// rounds every weight to f16 anyway).
template <uint32_t ENC>
struct WRaw;
template <>
struct WRaw<12> {
    u32x4 hdr, qs;
    float mul0, off0, mul1, off1;
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 144;
        hdr = *(const u32x4 *)blk;
        qs = *(const u32x4 *)(blk + 16 + (ks & 3) * 32 + part * 16);
    }
    // The same two loads as asm, which the compiler does not track: the
    // caller waits with wait<N>(), N = vector memory ops issued after them.
    __device__ __forceinline__ void load_asm(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 144;
        const uint8_t *q = blk + 16 + (ks & 3) * 32 + part * 16;
        asm volatile("global_load_dwordx4 %0, %2, off\n\tglobal_load_dwordx4 %1, %3, off"
                     : "=&v"(hdr), "=&v"(qs) : "v"(blk), "v"(q) : "memory");
    }
    template <int N>
    __device__ __forceinline__ void wait() {
        asm volatile("s_waitcnt vmcnt(%2)" : "+v"(hdr), "+v"(qs) : "n"(N) : "memory");
    }

    __device__ __forceinline__ void dequant(uint32_t ks, uint32_t part, uint32_t c, _Float16 *out) {
        if (c == 0) {
            const uint32_t p = ks & 3;
            const float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
            uint32_t sc0, m0, sc1, m1;
            q4k_scale_min(2 * p, hdr.y, hdr.z, hdr.w, &sc0, &m0);
            q4k_scale_min(2 * p + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
            mul0 = d * (float)sc0;
            off0 = dmin * (float)m0;
            mul1 = d * (float)sc1 * 0.0625f;  // high nibbles are converted in place (x16)
            off1 = dmin * (float)m1;
        }
        const uint32_t word = c == 0 ? qs.x : c == 1 ? qs.y : c == 2 ? qs.z : qs.w;
        const uint32_t lo = opaque_and<0x0f0f0f0fu>(word), hi = opaque_and<0xf0f0f0f0u>(word);
        *(half4v_t *)(out + part * 16 + 4 * c) = pf_four(lo, (_Float16)1024.f, mul0, -off0);
        *(half4v_t *)(out + 32 + part * 16 + 4 * c) = pf_four(hi, (_Float16)1024.f, mul1, -off1);
    }
};
// Q6_K slabs are not 64 consecutive columns: slab ks of block ks / 4 holds
// quarters qa and qa + 2 (qa = ks & 1) of half (ks & 3) / 2, the two
// quarters whose 6-bit codes share their ql bytes (low and high nibbles) and
// their qh bytes (bits 2qa and 2qa + 4). Part p = values 16p .. 16p + 15 of
// both quarters (slab columns 16p.. and 32 + 16p..), so a thread loads 16
// ql bytes, 16 qh bytes, the scales and d once for 32 values.
template <>
struct WRaw<14> {
    u32x4 ql, qh, sc16;
    uint32_t d16;
    float mul_lo, mul_hi;
    // load() as asm (three unaligned 16-byte loads and one 2-byte load),
    // untracked by the compiler: wait<N>() as for WRaw<12>
    __device__ __forceinline__ void load_asm(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 210;
        const uint32_t h = (ks & 3) >> 1, qa = ks & 1;
        const uint8_t *pa = blk + h * 64 + qa * 32 + 16 * part, *pb = blk + 128 + h * 32 + 16 * part;
        asm volatile(
            "global_load_dwordx4 %0, %4, off\n\t"
            "global_load_dwordx4 %1, %5, off\n\t"
            "global_load_dwordx4 %2, %6, off offset:192\n\t"
            "global_load_ushort %3, %6, off offset:208"
            : "=&v"(ql), "=&v"(qh), "=&v"(sc16), "=&v"(d16)
            : "v"(pa), "v"(pb), "v"(blk)
            : "memory");
    }
    template <int N>
    __device__ __forceinline__ void wait() {
        asm volatile("s_waitcnt vmcnt(%4)" : "+v"(ql), "+v"(qh), "+v"(sc16), "+v"(d16) : "n"(N) : "memory");
    }
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 210;
        const uint32_t h = (ks & 3) >> 1, qa = ks & 1;
        // 2-byte aligned blocks: unaligned 16-byte loads (ROCm runs global
        // memory in unaligned mode)
        typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
        const u32x4_a2 a = *(const u32x4_a2 *)(blk + h * 64 + qa * 32 + 16 * part);
        const u32x4_a2 b = *(const u32x4_a2 *)(blk + 128 + h * 32 + 16 * part);
        const u32x4_a2 c = *(const u32x4_a2 *)(blk + 192);
        ql = u32x4{a.x, a.y, a.z, a.w};
        qh = u32x4{b.x, b.y, b.z, b.w};
        sc16 = u32x4{c.x, c.y, c.z, c.w};
        d16 = load_u16_bytes(blk + 208);
    }
    __device__ __forceinline__ void dequant(uint32_t ks, uint32_t part, uint32_t c, _Float16 *out) {
        const uint32_t h = (ks & 3) >> 1, qa = ks & 1;
        if (c == 0) {
            // scales of values 16 part.. of quarters qa and qa + 2: bytes
            // idx = 8h + 2qa + part and idx + 4 (dwords 2h and 2h + 1)
            const float d = half_bits(d16);
            const uint32_t lo_word = h ? sc16.z : sc16.x, hi_word = h ? sc16.w : sc16.y;
            const uint32_t sh = 8 * (2 * qa + part);
            mul_lo = d * (float)(int8_t)((lo_word >> sh) & 0xffu);
            mul_hi = d * (float)(int8_t)((hi_word >> sh) & 0xffu);
        }
        const uint32_t l = c == 0 ? ql.x : c == 1 ? ql.y : c == 2 ? ql.z : ql.w;
        const uint32_t hb = c == 0 ? qh.x : c == 1 ? qh.y : c == 2 ? qh.z : qh.w;
        const uint32_t s0 = 2 * qa;
        const uint32_t ulo = opaque_and<0x0f0f0f0fu>(l) | (opaque_and<0x03030303u>(hb >> s0) << 4);
        const uint32_t uhi = opaque_and<0x0f0f0f0fu>(l >> 4) | (opaque_and<0x03030303u>(hb >> (s0 + 4)) << 4);
        // mul * (u - 32): the product of the exact f16 integer u - 32
        *(half4v_t *)(out + part * 16 + 4 * c) = pf_four(ulo, (_Float16)1056.f, mul_lo, 0.f);
        *(half4v_t *)(out + 32 + part * 16 + 4 * c) = pf_four(uhi, (_Float16)1056.f, mul_hi, 0.f);
    }
};
template <>
struct WRaw<13> {
    u32x4 hdr, qh, qs;
    uint32_t p2;  // 2 * pair: the high-plane bit of the low-nibble group
    float mul0, off0, mul1, off1;
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 176;
        hdr = *(const u32x4 *)blk;
        qh = *(const u32x4 *)(blk + 16 + part * 16);
        qs = *(const u32x4 *)(blk + 48 + (ks & 3) * 32 + part * 16);
    }
    // load() as asm, untracked by the compiler: wait<N>() as for WRaw<12>
    __device__ __forceinline__ void load_asm(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 176;
        const uint8_t *ph = blk + 16 + part * 16, *pq = blk + 48 + (ks & 3) * 32 + part * 16;
        asm volatile(
            "global_load_dwordx4 %0, %3, off\n\t"
            "global_load_dwordx4 %1, %4, off\n\t"
            "global_load_dwordx4 %2, %5, off"
            : "=&v"(hdr), "=&v"(qh), "=&v"(qs)
            : "v"(blk), "v"(ph), "v"(pq)
            : "memory");
    }
    template <int N>
    __device__ __forceinline__ void wait() {
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(hdr), "+v"(qh), "+v"(qs) : "n"(N) : "memory");
    }
    __device__ __forceinline__ void dequant(uint32_t ks, uint32_t part, uint32_t c, _Float16 *out) {
        if (c == 0) {
            const uint32_t p = ks & 3;
            const float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
            uint32_t sc0, m0, sc1, m1;
            q4k_scale_min(2 * p, hdr.y, hdr.z, hdr.w, &sc0, &m0);
            q4k_scale_min(2 * p + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
            mul0 = d * (float)sc0;
            off0 = dmin * (float)m0;
            mul1 = d * (float)sc1;
            off1 = dmin * (float)m1;
            p2 = 2 * p;
        }
        const uint32_t word = c == 0 ? qs.x : c == 1 ? qs.y : c == 2 ? qs.z : qs.w;
        const uint32_t high = c == 0 ? qh.x : c == 1 ? qh.y : c == 2 ? qh.z : qh.w;
        const uint32_t lo = (word & 0x0f0f0f0fu) | (((high >> p2) & 0x01010101u) << 4);
        const uint32_t hi = ((word >> 4) & 0x0f0f0f0fu) | (((high >> (p2 + 1)) & 0x01010101u) << 4);
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
        half4 l, h;
        l[0] = (_Float16)fmaf(mul0, ubyte_f<0>(lo), -off0);
        l[1] = (_Float16)fmaf(mul0, ubyte_f<1>(lo), -off0);
        l[2] = (_Float16)fmaf(mul0, ubyte_f<2>(lo), -off0);
        l[3] = (_Float16)fmaf(mul0, ubyte_f<3>(lo), -off0);
        h[0] = (_Float16)fmaf(mul1, ubyte_f<0>(hi), -off1);
        h[1] = (_Float16)fmaf(mul1, ubyte_f<1>(hi), -off1);
        h[2] = (_Float16)fmaf(mul1, ubyte_f<2>(hi), -off1);
        h[3] = (_Float16)fmaf(mul1, ubyte_f<3>(hi), -off1);
        *(half4 *)(out + part * 16 + 4 * c) = l;
        *(half4 *)(out + 32 + part * 16 + 4 * c) = h;
    }
};
template <>
struct WRaw<23> {
    u32x2 hdr, q01, q23;  // d, scales_h, scales_l; the group's 16 code bytes
    float mul;
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 136;
        const uint32_t g = 2 * (ks & 3) + part;
        hdr = *(const u32x2 *)blk;
        q01 = *(const u32x2 *)(blk + 8 + 16 * g);
        q23 = *(const u32x2 *)(blk + 16 + 16 * g);
    }
    // load() as asm, untracked by the compiler: wait<N>() as for WRaw<12>
    __device__ __forceinline__ void load_asm(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(ks >> 2) * 136;
        const uint8_t *pq = blk + 8 + 16 * (2 * (ks & 3) + part);
        asm volatile(
            "global_load_dwordx2 %0, %3, off\n\t"
            "global_load_dwordx2 %1, %4, off\n\t"
            "global_load_dwordx2 %2, %4, off offset:8"
            : "=&v"(hdr), "=&v"(q01), "=&v"(q23)
            : "v"(blk), "v"(pq)
            : "memory");
    }
    template <int N>
    __device__ __forceinline__ void wait() {
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(hdr), "+v"(q01), "+v"(q23) : "n"(N) : "memory");
    }
    // this thread owns group 2(ks&3) + part: chunk c = byte dword c, values
    // 4c..4c+3 (low nibbles) and 16+4c.. (high nibbles)
    __device__ __forceinline__ void dequant(uint32_t ks, uint32_t part, uint32_t c, _Float16 *out) {
        if (c == 0) {
            const uint32_t g = 2 * (ks & 3) + part;
            const uint32_t low = (hdr.y >> (8 * (g / 2) + 4 * (g % 2))) & 15u;
            const int sc = (int)(low | (((hdr.x >> (16 + 2 * g)) & 3u) << 4)) - 32;
            mul = half_bits(hdr.x & 0xffffu) * (float)sc;
        }
        const uint32_t word = c == 0 ? q01.x : c == 1 ? q01.y : c == 2 ? q23.x : q23.y;
        const uint32_t tl = iq4_lookup(word & 0x0f0f0f0fu), th = iq4_lookup((word >> 4) & 0x0f0f0f0fu);
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
        half4 l, h;
        l[0] = (_Float16)(mul * sbyte_f<0>(tl));
        l[1] = (_Float16)(mul * sbyte_f<1>(tl));
        l[2] = (_Float16)(mul * sbyte_f<2>(tl));
        l[3] = (_Float16)(mul * sbyte_f<3>(tl));
        h[0] = (_Float16)(mul * sbyte_f<0>(th));
        h[1] = (_Float16)(mul * sbyte_f<1>(th));
        h[2] = (_Float16)(mul * sbyte_f<2>(th));
        h[3] = (_Float16)(mul * sbyte_f<3>(th));
        *(half4 *)(out + part * 32 + 4 * c) = l;
        *(half4 *)(out + part * 32 + 16 + 4 * c) = h;
    }
};
template <>
struct WRaw<8> {
    u32x4 qa, qb;  // the block's 32 codes
    uint32_t d16;
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(2 * ks + part) * 34;
        // 2-byte aligned blocks: unaligned 16-byte loads (ROCm runs global
        // memory in unaligned mode)
        typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
        d16 = load_u16_bytes(blk);
        const u32x4_a2 a = *(const u32x4_a2 *)(blk + 2), b = *(const u32x4_a2 *)(blk + 18);
        qa = u32x4{a.x, a.y, a.z, a.w};
        qb = u32x4{b.x, b.y, b.z, b.w};
    }
    // load() as asm, untracked by the compiler: wait<N>() as for WRaw<12>
    __device__ __forceinline__ void load_asm(const uint8_t *row, uint32_t ks, uint32_t part) {
        const uint8_t *blk = row + (uint64_t)(2 * ks + part) * 34;
        asm volatile(
            "global_load_ushort %0, %3, off\n\t"
            "global_load_dwordx4 %1, %3, off offset:2\n\t"
            "global_load_dwordx4 %2, %3, off offset:18"
            : "=&v"(d16), "=&v"(qa), "=&v"(qb)
            : "v"(blk)
            : "memory");
    }
    template <int N>
    __device__ __forceinline__ void wait() {
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(d16), "+v"(qa), "+v"(qb) : "n"(N) : "memory");
    }
    __device__ __forceinline__ void dequant(uint32_t, uint32_t part, uint32_t c, _Float16 *out) {
        const float d = half_bits(d16);
        const uint32_t w0 = c == 0 ? qa.x : c == 1 ? qa.z : c == 2 ? qb.x : qb.z;
        const uint32_t w1 = c == 0 ? qa.y : c == 1 ? qa.w : c == 2 ? qb.y : qb.w;
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (_Float16)(d * (float)(int8_t)(((e < 4 ? w0 : w1) >> (8 * (e & 3))) & 0xff));
        *(half8 *)(out + part * 32 + 8 * c) = v;
    }
};

constexpr int PF_BM = 256, PF_BN = 256, PF_GROUP_M = 4;

// Step order per encoding with F32 activations (f16 activations always copy
// first, see PF_ASMW): the activation loads before the weight prefetch for
// Q8_0, Q5_K and Q6_K, after it for Q4_K and IQ4_XS, as measured with the
// f16 copies before the weight loads left the compiler's tracking (8 %, 2 %,
// 7 % gained; 2-2.5 % lost). Bit e of the mask is encoding e.
#ifndef NUQ_PF_COPY_FIRST_MASK
#define NUQ_PF_COPY_FIRST_MASK ((1u << 8) | (1u << 13) | (1u << 14))
#endif
template <uint32_t ENC> struct PF_COPY_FIRST { static constexpr bool value = (NUQ_PF_COPY_FIRST_MASK >> (ENC & 31)) & 1u; };
// With f16 activations the weight prefetch is asm loads the compiler does
// not track, issued after the activation copies: the step's end then waits
// for the copies only and the weights keep their two-step distance (the
// compiler's own waits fall back to vmcnt(0) behind LDS copies). A/B on one
// box, M=4096 / M=512 TFLOP/s: Q4_K 848-861 -> 857-858 / 562-569 -> 585-589,
// Q6_K 779-781 -> 807-809 / 577-591 -> 588-601, Q5_K 794-806 -> 844-850 /
// 606-614 -> 630-637, IQ4_XS 850-860 -> 870-881 / 614-629 -> 652-670, Q8_0
// 860-863 -> 880-892 / 599-616 -> 639-653.
template <uint32_t ENC, typename XT> struct PF_ASMW {
    static constexpr bool value = sizeof(XT) == 2;
    static constexpr int LOADS = ENC == 14 ? 4 : ENC == 12 ? 2 : 3;  // WRaw<ENC>::load_asm's instructions
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// f16 activations go global -> LDS without registers (global_load_lds_dwordx4):
// lane i of wave instruction q fills 16-byte slot 64q + i of the padded
// tile (9 slots a row: 8 of data, 1 of padding, so rows keep the 144-byte
// pitch the fragment reads want). Padding slots load a valid address and
// are never read. Rows past `tokens` re-read the last token: their outputs
// are never stored. Wave w of NW issues instructions q = w, w + NW, ...
// A lane's byte offsets from the tile's first row are fixed
// for the whole K loop, so they are computed once (XDma::init) and each
// slab's copies are a uniform base plus those offsets.
constexpr uint32_t XD_INSTRS = PF_BM * 9 / 64;  // 36

// First column of K slab ks, and the offset of slab chunk c (8 columns)
// from it: 64 consecutive columns, except Q6_K (see WRaw<14>), whose slab
// is two 32-column pieces 64 columns apart.
template <uint32_t ENC>
__device__ __forceinline__ uint32_t slab_k0(uint32_t ks) {
    return ENC == 14 ? (ks >> 2) * 256 + ((ks & 3) >> 1) * 128 + (ks & 1) * 32 : ks * BK;
}
template <uint32_t ENC>
__device__ __forceinline__ uint32_t slab_chunk_col(uint32_t c) {
    return ENC == 14 && c >= 4 ? 64 + 8 * (c - 4) : 8 * c;
}
template <uint32_t NW, uint32_t ENC>
struct XDma {
    static constexpr uint32_t PER_WAVE = (XD_INSTRS + NW - 1) / NW;
    uint32_t off[PER_WAVE];
    uint32_t first;  // this wave's first instruction (scalar)
    __device__ __forceinline__ void init(uint64_t in_stride, uint32_t m_base, uint32_t tokens, uint32_t wave,
                                         uint32_t lane) {
        first = __builtin_amdgcn_readfirstlane(wave);
        const uint32_t last_row = tokens - 1 - m_base;
#pragma unroll
        for (uint32_t t = 0; t < PER_WAVE; ++t) {
            const uint32_t slot = 64 * min(first + t * NW, XD_INSTRS - 1) + lane;
            const uint32_t row = min(slot / 9, last_row), chunk = slot % 9;
            off[t] = (uint32_t)(((uint64_t)row * in_stride + slab_chunk_col<ENC>(chunk == 8 ? 0 : chunk)) * 2);
        }
    }
    // copies slab columns (k0 + slab_chunk_col) of the tile's rows into lds_tile
    __device__ __forceinline__ void copy(const _Float16 *__restrict__ x, uint64_t in_stride, uint32_t m_base,
                                         uint32_t k0, _Float16 *lds_tile) const {
        const char *base = (const char *)(x + (uint64_t)m_base * in_stride + k0);
#pragma unroll
        for (uint32_t t = 0; t < PER_WAVE; ++t) {
            const uint32_t q = first + t * NW;
            if (XD_INSTRS % NW != 0 && q >= XD_INSTRS) break;
            __builtin_amdgcn_global_load_lds((global_void_t *)(base + off[t]), (lds_void_t *)(lds_tile + 64 * q * 8),
                                             16, 0, 0);
        }
    }
};

__device__ __forceinline__ void tile_coords(uint32_t id, uint32_t tm, uint32_t tn, uint32_t *pid_m, uint32_t *pid_n) {
    const uint32_t total = tm * tn;
    if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;  // contiguous range per XCD
    const uint32_t per_group = PF_GROUP_M * tn;
    const uint32_t group = id / per_group;
    const uint32_t first_m = group * PF_GROUP_M;
    const uint32_t gm = min(tm - first_m, (uint32_t)PF_GROUP_M);
    const uint32_t in_group = id % per_group;
    *pid_m = first_m + in_group % gm;
    *pid_n = in_group / gm;
}

// NW = 8: 2 x 4 waves of 128 x 64 (each thread stages half a weight row);
// NW = 4: 2 x 2 waves of 128 x 128, 256 accumulators per lane (each thread
// stages a whole weight row). The larger wave tile halves the LDS fragment
// reads per MFMA.
// Instruction groups of the K step (sched_group_barrier): MFMA 1, LDS read 1,
// VALU PF_SCHED_VALU, repeated. Left to itself the scheduler bunched the
// MFMAs and the dequantisation apart; interleaved, Q4_K 17408 x 5120 went
// from ~815 to ~845 TFLOP/s at 4096 tokens and 532 to 555 at 512 on MI355X
// (4, 12, 16 and 20 were no better; Q6_K is unchanged).
constexpr int PF_SCHED_VALU = 8;
template <uint32_t ENC, typename XT, uint32_t NW>
__global__ void __launch_bounds__(64 * NW) prefill_kernel(const uint8_t *__restrict__ w, uint64_t stride,
                                                              uint32_t rows, uint32_t columns,
                                                              const XT *__restrict__ x, uint64_t in_stride,
                                                              float *__restrict__ y, uint64_t out_stride,
                                                              uint32_t tokens, uint32_t full, uint32_t tail,
                                                              uint32_t splits, float *__restrict__ work) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_smem[];
    // buffer b: activations at pf_smem + b*XS, weights at pf_smem + 2*XS + b*WS
    constexpr uint32_t XS = PF_BM * LDS_PITCH, WS = PF_BN * LDS_PITCH;

    const uint32_t tm = (tokens + PF_BM - 1) / PF_BM, tn = (rows + PF_BN - 1) / PF_BN;
    // Workgroups [0, full) each own a whole tile. The `tail` tiles after
    // them are split along K into `splits` column ranges of whole 256-column
    // blocks, one workgroup each (workgroup full + s*tail + t takes range s
    // of tile full + t), so a partial last round still spreads over the CUs.
    uint32_t tile = blockIdx.x, split = 0;
    const bool split_k = tile >= full;
    if (split_k) {
        tile = full + (blockIdx.x - full) % tail;
        split = (blockIdx.x - full) / tail;
        constexpr uint32_t BLOCK256 = ENC == 12 ? 144 : ENC == 13 ? 176 : ENC == 14 ? 210 : ENC == 23 ? 136 : 272;  // bytes per 256 columns
        const uint32_t nb = columns / 256;
        const uint32_t b0 = split * nb / splits, b1 = (split + 1) * nb / splits;
        w += (uint64_t)b0 * BLOCK256;
        x += (uint64_t)b0 * 256;
        columns = (b1 - b0) * 256;
    }
    uint32_t pid_m, pid_n;
    tile_coords(tile, tm, tn, &pid_m, &pid_n);
    const uint32_t m_base = pid_m * PF_BM, n_base = pid_n * PF_BN;

    constexpr uint32_t THREADS = 64 * NW, WN = NW == 8 ? 4 : 2, TJ = NW == 8 ? 2 : 4, NSPAN = PF_BN / WN;
    constexpr uint32_t SP = 2 * PF_BM / THREADS;  // (row, half) staging units per thread
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave / WN, wn = wave % WN;
    // staging unit u = SP*tid + s: row u/2, 32-column half u%2 of the slab
    const uint32_t srow = (SP * tid) >> 1;
    const uint8_t *wrow = w + (uint64_t)min(n_base + srow, rows - 1) * stride;
    const uint32_t xtok = m_base + srow;
    const bool xvalid = xtok < tokens;
    const XT *xrow = x + (uint64_t)(xvalid ? xtok : 0) * in_stride;
#define NUQ_PF_PART(s_) ((SP * tid + (s_)) & 1)

    floatx16 acc[4][TJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < (int)TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Pipeline. Activations: slab ks+1 is copied global -> LDS during step
    // ks (f16 input; F32 input is converted through registers after the
    // MFMAs). Weights: two register sets hold the raw GGUF bytes of slabs
    // ks+1 and ks+2; slab ks+1 is dequantised chunk by chunk between the
    // MFMA sub-steps of slab ks (so one wave keeps both the matrix core and
    // the VALU busy), while slab ks+2 is in flight.
    constexpr bool DMA = sizeof(XT) == 2;
    XLoad<XT> xr[SP];
    WRaw<ENC> wA[SP], wB[SP];
    const uint32_t ksteps = columns / BK;
    XDma<NW, ENC> xd;
    if constexpr (DMA) {
        xd.init(in_stride, m_base, tokens, wave, lane);
        xd.copy((const _Float16 *)x, in_stride, m_base, 0, pf_smem);
    } else {
#pragma unroll
        for (uint32_t s_ = 0; s_ < SP; ++s_) xr[s_].load(xrow + slab_chunk_col<ENC>(4 * NUQ_PF_PART(s_)), xvalid);
    }
#pragma unroll
    for (uint32_t s_ = 0; s_ < SP; ++s_) wA[s_].load(wrow, 0, NUQ_PF_PART(s_));
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c)
#pragma unroll
        for (uint32_t s_ = 0; s_ < SP; ++s_) {
            if constexpr (!DMA) xr[s_].store(pf_smem + srow * LDS_PITCH + NUQ_PF_PART(s_) * 32, c);
            wA[s_].dequant(0, NUQ_PF_PART(s_), c, pf_smem + 2 * XS + srow * LDS_PITCH);
        }
    if (ksteps > 1) {
#pragma unroll
        for (uint32_t s_ = 0; s_ < SP; ++s_) {
            if constexpr (PF_ASMW<ENC, XT>::value) wA[s_].load_asm(wrow, 1, NUQ_PF_PART(s_));
            else wA[s_].load(wrow, 1, NUQ_PF_PART(s_));
        }
    }
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();

    // One K step; a macro rather than a lambda so the accumulators stay in
    // registers (a capturing lambda takes their address).
#define NUQ_PF_STEP(KS, WNEXT, WFAR, WAITN)                                                                        \
    {                                                                                                              \
        const uint32_t ks_ = (KS);                                                                                 \
        const uint32_t cur = ks_ & 1;                                                                              \
        const bool next = ks_ + 1 < ksteps;                                                                        \
        const _Float16 *xa = pf_smem + cur * XS + (wm * 128 + (lane & 31)) * LDS_PITCH + 8 * (lane >> 5);         \
        const _Float16 *wb = pf_smem + 2 * XS + cur * WS + (wn * NSPAN + (lane & 31)) * LDS_PITCH + 8 * (lane >> 5); \
        _Float16 *wdst = pf_smem + 2 * XS + (cur ^ 1) * WS + srow * LDS_PITCH;                                     \
        half8 fa[2][4], fb[2][TJ];                                                                                 \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) fa[0][i] = *(const half8 *)(xa + i * 32 * LDS_PITCH);        \
        _Pragma("unroll") for (int j = 0; j < (int)TJ; ++j) fb[0][j] = *(const half8 *)(wb + j * 32 * LDS_PITCH);  \
        const bool far_ = ks_ + 2 < ksteps;                                                                        \
        /* PF_COPY_FIRST: the activation copy is issued before the weight prefetch */                            \
        if (!(PF_COPY_FIRST<ENC>::value || PF_ASMW<ENC, XT>::value) && far_) {                                    \
            _Pragma("unroll") for (uint32_t s_ = 0; s_ < SP; ++s_) WFAR[s_].load(wrow, ks_ + 2, NUQ_PF_PART(s_));  \
        }                                                                                                          \
        if (next) {                                                                                                \
            if constexpr (DMA) {                                                                                   \
                xd.copy((const _Float16 *)x, in_stride, m_base, slab_k0<ENC>(ks_ + 1), pf_smem + (cur ^ 1) * XS);  \
            } else {                                                                                               \
                _Pragma("unroll") for (uint32_t s_ = 0; s_ < SP; ++s_)                                             \
                    xr[s_].load(xrow + slab_chunk_col<ENC>(4 * NUQ_PF_PART(s_)) + slab_k0<ENC>(ks_ + 1), xvalid);  \
            }                                                                                                      \
        }                                                                                                          \
        if ((PF_COPY_FIRST<ENC>::value || PF_ASMW<ENC, XT>::value) && far_) {                                     \
            /* the weight loads stay behind the copies, so the step's end can wait for the copies alone */         \
            asm volatile("" ::: "memory");                                                                         \
            __builtin_amdgcn_sched_barrier(0);                                                                     \
            _Pragma("unroll") for (uint32_t s_ = 0; s_ < SP; ++s_) {                                               \
                if constexpr (PF_ASMW<ENC, XT>::value) WFAR[s_].load_asm(wrow, ks_ + 2, NUQ_PF_PART(s_));          \
                else WFAR[s_].load(wrow, ks_ + 2, NUQ_PF_PART(s_));                                                \
            }                                                                                                      \
        }                                                                                                          \
        if constexpr (PF_ASMW<ENC, XT>::value) {                                                                   \
            /* the previous step's weight loads are older than this step's copies and loads (WAITN of them at */  \
            /* least) */                                                                                           \
            _Pragma("unroll") for (uint32_t s_ = 0; s_ < SP; ++s_) WNEXT[s_].template wait<WAITN>();               \
        }                                                                                                          \
        _Pragma("unroll") for (uint32_t kk = 0; kk < BK / 16; ++kk) {                                              \
            const uint32_t p_ = kk & 1;                                                                            \
            if (kk + 1 < BK / 16) {                                                                                \
                _Pragma("unroll") for (int i = 0; i < 4; ++i)                                                      \
                    fa[p_ ^ 1][i] = *(const half8 *)(xa + i * 32 * LDS_PITCH + (kk + 1) * 16);                     \
                _Pragma("unroll") for (int j = 0; j < (int)TJ; ++j)                                                \
                    fb[p_ ^ 1][j] = *(const half8 *)(wb + j * 32 * LDS_PITCH + (kk + 1) * 16);                     \
            }                                                                                                      \
            _Pragma("unroll") for (int i = 0; i < 4; ++i) _Pragma("unroll") for (int j = 0; j < (int)TJ; ++j)      \
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[p_][i], fb[p_][j], acc[i][j], 0, 0, 0);      \
            /* the last step dequantises into the idle buffer; harmless */                                         \
            _Pragma("unroll") for (uint32_t s_ = 0; s_ < SP; ++s_)                                                 \
                WNEXT[s_].dequant(ks_ + 1, NUQ_PF_PART(s_), kk, wdst);                                             \
            /* scheduling: each MFMA, then one fragment read, then up to PF_SCHED_VALU */                        \
            /* dequantisation VALU ops, so they issue under the MFMA's 32 cycles */                                  \
            _Pragma("unroll") for (int q_ = 0; q_ < 4 * (int)TJ; ++q_) {                                           \
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                 \
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                 \
                __builtin_amdgcn_sched_group_barrier(0x002, PF_SCHED_VALU, 0);                                     \
            }                                                                                                      \
        }                                                                                                          \
        if (!DMA && next) {                                                                                        \
            _Pragma("unroll") for (uint32_t s_ = 0; s_ < SP; ++s_) {                                               \
                _Float16 *xdst = pf_smem + (cur ^ 1) * XS + srow * LDS_PITCH + NUQ_PF_PART(s_) * 32;               \
                _Pragma("unroll") for (uint32_t c = 0; c < 4; ++c) xr[s_].store(xdst, c);                          \
            }                                                                                                      \
        }                                                                                                          \
        if (DMA && (PF_COPY_FIRST<ENC>::value || PF_ASMW<ENC, XT>::value)) {                                      \
            /* this step's copies have landed and the dequantised weights are written; the barrier */             \
            /* carries no fence */                                                                                \
            if (PF_ASMW<ENC, XT>::value && far_) /* the weight loads may stay in flight */                         \
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" : : "n"(SP * PF_ASMW<ENC, XT>::LOADS) : "memory");   \
            else                                                                                                   \
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" : : : "memory");                                     \
            __builtin_amdgcn_s_barrier();                                                                          \
        } else {                                                                                                   \
            if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0x0f70); /* vmcnt(0): this step's DMA has landed */     \
            __syncthreads();                                                                                       \
        }                                                                                                          \
    }
    if constexpr (PF_ASMW<ENC, XT>::value) {
        // Two steps per iteration, the register sets trading roles (no copy
        // of registers an untracked load may still be filling). Every step of
        // the loop issues at least XD_INSTRS / NW activation copies per wave
        // and then its two weight loads, all younger than the previous step's
        // weight loads: waiting for all but YOUNG of them leaves those landed.
        // The last one to three steps wait for everything.
        constexpr int YOUNG = XD_INSTRS / NW + PF_ASMW<ENC, XT>::LOADS * SP;
        uint32_t ks = 0;
        for (; ks + 3 < ksteps; ks += 2) {
            NUQ_PF_STEP(ks, wA, wB, YOUNG)
            NUQ_PF_STEP(ks + 1, wB, wA, YOUNG)
        }
        if (ks < ksteps) NUQ_PF_STEP(ks, wA, wB, 0)
        if (ks + 1 < ksteps) NUQ_PF_STEP(ks + 1, wB, wA, 0)
        if (ks + 2 < ksteps) NUQ_PF_STEP(ks + 2, wA, wB, 0)
    } else {
        for (uint32_t ks = 0; ks < ksteps; ++ks) {
            NUQ_PF_STEP(ks, wA, wB, 0)
#pragma unroll
            for (uint32_t s_ = 0; s_ < SP; ++s_) wA[s_] = wB[s_];
        }
    }
#undef NUQ_PF_STEP
#undef NUQ_PF_PART

    // Output element (i, j, r) of a lane: tile row (token) and column (weight row).
#define NUQ_PF_M(i, r) (wm * 128 + (i) * 32 + 8 * ((r) >> 2) + 4 * (lane >> 5) + ((r) & 3))
#define NUQ_PF_N(j) (wn * NSPAN + (j) * 32 + (lane & 31))
    if (split_k) {
        // A split stores its partial tile row-major; split_reduce_kernel adds
        // the splits in order afterwards.
        float *mine = work + (uint64_t)((tile - full) * splits + split) * (PF_BM * PF_BN);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < (int)TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) mine[NUQ_PF_M(i, r) * PF_BN + NUQ_PF_N(j)] = acc[i][j][r];
        return;
    }

#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < (int)TJ; ++j) {
            const uint32_t n = n_base + NUQ_PF_N(j);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m_base + NUQ_PF_M(i, r);
                if (m < tokens && n < rows) y[(uint64_t)m * out_stride + n] = acc[i][j][r];
            }
        }
#undef NUQ_PF_M
#undef NUQ_PF_N
}

// Sums the K-split partial tiles of prefill_kernel (row-major 256 x 256
// each) in split order -- the order is fixed, so results do not depend on
// which split ran first -- and stores them.
__global__ void __launch_bounds__(256) split_reduce_kernel(const float *__restrict__ work, float *__restrict__ y,
                                                           uint64_t out_stride, uint32_t rows, uint32_t tokens,
                                                           uint32_t full, uint32_t splits) {
    constexpr uint32_t TILE_F = PF_BM * PF_BN;
    const uint32_t t = blockIdx.x / (TILE_F / 256);
    const uint32_t e = (blockIdx.x % (TILE_F / 256)) * 256 + threadIdx.x;
    const uint32_t tm = (tokens + PF_BM - 1) / PF_BM, tn = (rows + PF_BN - 1) / PF_BN;
    uint32_t pid_m, pid_n;
    tile_coords(full + t, tm, tn, &pid_m, &pid_n);
    const uint32_t m = pid_m * PF_BM + e / PF_BN, n = pid_n * PF_BN + e % PF_BN;
    const float *p = work + (uint64_t)t * splits * TILE_F + e;
    float v = p[0];
    for (uint32_t q = 1; q < splits; ++q) v += p[(uint64_t)q * TILE_F];
    if (m < tokens && n < rows) y[(uint64_t)m * out_stride + n] = v;
}

static uint32_t compute_units() {
    static uint32_t cached = 0;
    if (!cached) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cached = (uint32_t)n;
        else
            cached = 256;
    }
    return cached;
}

// The prefill's K-split plan (see launch_prefill): `full` whole tiles, then
// `tail` tiles split `splits` ways, needing tail * splits partial tiles of
// workspace; no split when the workspace holds fewer than that
// (max_tiles = 0: none).
static void prefill_split_plan(uint32_t tiles, uint32_t columns, uint32_t cus, uint64_t max_tiles, uint32_t *full,
                               uint32_t *tail, uint32_t *splits) {
    *full = tiles;
    *tail = 0;
    *splits = 1;
    const uint32_t rem = tiles % cus;
    if (rem == 0 || columns % 256 != 0 || max_tiles == 0) return;
    const uint32_t nb = columns / 256;
    const double whole = (double)nb + 1.0;
    double best = 0.85 * whole;
    for (uint32_t sp = 2; sp <= std::min(nb, 16u); ++sp) {
        if ((uint64_t)rem * sp > max_tiles) break;
        const double rounds = (double)((rem * sp + cus - 1) / cus);
        const double cost = rounds * ((double)((nb + sp - 1) / sp) + 1.0) + (double)rem * sp / 100.0 + 0.3;
        if (cost < best) {
            best = cost;
            *splits = sp;
        }
    }
    if (*splits > 1) {
        *full = tiles - rem;
        *tail = rem;
    }
}

template <uint32_t ENC>
static hipError_t launch_prefill(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                                 const void *x, uint32_t x_f16, uint64_t in_stride, float *y, uint64_t out_stride,
                                 uint32_t tokens, const SplitScratch &scratch, uint32_t cus) {
    const uint32_t tiles = ((tokens + PF_BM - 1) / PF_BM) * ((rows + PF_BN - 1) / PF_BN);
    // Tiles that fill whole rounds (one tile per CU) run whole. The rest
    // (all of them when there are fewer tiles than CUs) may be split along
    // K into s ranges of whole 256-column blocks, picked by a cost model in
    // units of one tile's work on one 256-column block:
    //   rounds(s) * (ceil(nb / s) + 1) + reduce(s),
    // where rounds(s) = ceil(rem * s / cus), the +1 is a workgroup's fixed
    // cost (pipeline fill, epilogue) and the reduce pass reads s partial
    // tiles of 256 KiB per split tile (about 1/100 of a unit each, plus a
    // launch). A split is taken only when it is predicted 15% faster (on
    // MI355X it does not pay for Q4_K 17408 x 5120 at 512 tokens).
    uint32_t full, tail, splits;
    prefill_split_plan(tiles, columns, cus, scratch.work != nullptr ? scratch.tiles : 0, &full, &tail, &splits);
    const uint32_t grid = full + tail * splits;
    const size_t lds = (size_t)2 * (PF_BM + PF_BN) * LDS_PITCH * sizeof(_Float16);
#define NUQ_PF_LAUNCH(NW_)                                                                                       \
    if (x_f16)                                                                                                   \
        hipLaunchKernelGGL((prefill_kernel<ENC, _Float16, NW_>), dim3(grid), dim3(64 * NW_), lds, s, w, stride,  \
                           rows, columns, (const _Float16 *)x, in_stride, y, out_stride, tokens, full, tail,     \
                           splits, scratch.work);                                                                \
    else                                                                                                         \
        hipLaunchKernelGGL((prefill_kernel<ENC, float, NW_>), dim3(grid), dim3(64 * NW_), lds, s, w, stride, rows, \
                           columns, (const float *)x, in_stride, y, out_stride, tokens, full, tail, splits,      \
                           scratch.work);
    // 8 waves: NW = 4 (1 wave per SIMD) measured slower on MI355X, 693 vs
    // 753 TFLOP/s for Q4_K 17408 x 5120 at 4096 tokens
    NUQ_PF_LAUNCH(8)
#undef NUQ_PF_LAUNCH
    if (tail != 0)
        hipLaunchKernelGGL(split_reduce_kernel, dim3(tail * (PF_BM * PF_BN / 256)), dim3(256), 0, s, scratch.work, y,
                           out_stride, rows, tokens, full, splits);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Verify tile (tokens <= 16): weights dequantised straight into MFMA
// A-fragment registers, no LDS for weights.
//
// v_mfma_f32_16x16x32_f16: A = 16 weight rows x 32 k (lane l: row l%16,
// 8 consecutive k slots 8*(l/16)..+8), B = 32 k x 16 tokens (lane l: token
// l%16, the same 8 k slots), D = 16 rows x 16 tokens. The k index is a sum
// index, so any permutation applied to both operands leaves D unchanged:
// lane (row r, quarter h = l/16) takes 64 values of block b that are cheap
// for it to decode (Q4_K: qs pair h, both nibbles; Q6_K: half h/2, columns
// 16*(h&1)..+16 of all four quarters; Q8_0: the two 32-blocks 2h, 2h+1) as
// 8 chunks of 8 consecutive columns, and the B fragment loads the same
// columns of x. A workgroup covers 16 rows; its waves take interleaved
// blocks and meet in LDS.
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <uint32_t ENC>
struct VLane;

template <>
struct VLane<12> {
    static constexpr uint32_t BLOCK_BYTES = 144, BLOCK_VALUES = 256;
    // first column (within the block) of chunk c for quarter h
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) { return 32 * (2 * h + (c >> 2)) + 8 * (c & 3); }
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&a)[8]) {
        const uint4 hdr = *(const uint4 *)blk;
        const uint4 q0 = *(const uint4 *)(blk + 16 + 32 * h), q1 = *(const uint4 *)(blk + 32 + 32 * h);
        const float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * h, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        q4k_scale_min(2 * h + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        const float mul0 = d * (float)sc0, off0 = dmin * (float)m0;
        const float mul1 = d * (float)sc1 * 0.0625f, off1 = dmin * (float)m1;
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // chunk c: columns 8c..8c+7 of group 2h (low nibbles), c+4: group 2h+1
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t lo = opaque_and<0x0f0f0f0fu>(w[2 * c + k]), hi = opaque_and<0xf0f0f0f0u>(w[2 * c + k]);
                a[c][4 * k + 0] = (_Float16)fmaf(mul0, ubyte_f<0>(lo), -off0);
                a[c][4 * k + 1] = (_Float16)fmaf(mul0, ubyte_f<1>(lo), -off0);
                a[c][4 * k + 2] = (_Float16)fmaf(mul0, ubyte_f<2>(lo), -off0);
                a[c][4 * k + 3] = (_Float16)fmaf(mul0, ubyte_f<3>(lo), -off0);
                a[c + 4][4 * k + 0] = (_Float16)fmaf(mul1, ubyte_f<0>(hi), -off1);
                a[c + 4][4 * k + 1] = (_Float16)fmaf(mul1, ubyte_f<1>(hi), -off1);
                a[c + 4][4 * k + 2] = (_Float16)fmaf(mul1, ubyte_f<2>(hi), -off1);
                a[c + 4][4 * k + 3] = (_Float16)fmaf(mul1, ubyte_f<3>(hi), -off1);
            }
        }
    }
};

template <>
struct VLane<14> {
    static constexpr uint32_t BLOCK_BYTES = 210, BLOCK_VALUES = 256;
    // chunk c: quarter q = c/2, columns 16*(h&1) + 8*(c&1) .. +8 of half h/2
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) {
        return 128 * (h >> 1) + 32 * (c >> 1) + 16 * (h & 1) + 8 * (c & 1);
    }
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&a)[8]) {
        const uint32_t hf = h >> 1, l0 = 16 * (h & 1);
        uint32_t qa[4], qb[4], qh[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            qa[k] = load_u32_unaligned(blk + hf * 64 + l0 + 4 * k);       // quarters 0 (low) / 2 (high nibble)
            qb[k] = load_u32_unaligned(blk + hf * 64 + 32 + l0 + 4 * k);  // quarters 1 / 3
            qh[k] = load_u32_unaligned(blk + 128 + hf * 32 + l0 + 4 * k);
        }
        const uint32_t s0 = load_u32_unaligned(blk + 192 + hf * 8), s1 = load_u32_unaligned(blk + 196 + hf * 8);
        const float d = half_bits(load_u16_bytes(blk + 208));
        const uint32_t odd = (h & 1) ? 8u : 0u;
        float mul[4];
        mul[0] = d * (float)(int8_t)((s0 >> odd) & 0xff);
        mul[1] = d * (float)(int8_t)((s0 >> (16 + odd)) & 0xff);
        mul[2] = d * (float)(int8_t)((s1 >> odd) & 0xff);
        mul[3] = d * (float)(int8_t)((s1 >> (16 + odd)) & 0xff);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t low = (q & 1) ? qb[k] : qa[k];
                const uint32_t u = opaque_and<0x0f0f0f0fu>(q >= 2 ? (low >> 4) : low) |
                                   opaque_and<0x30303030u>((qh[k] >> (2 * q)) << 4);
                const int c = 2 * q + (k >> 1), e0 = 4 * (k & 1);
                a[c][e0 + 0] = (_Float16)fmaf(mul[q], ubyte_f<0>(u), -32.f * mul[q]);
                a[c][e0 + 1] = (_Float16)fmaf(mul[q], ubyte_f<1>(u), -32.f * mul[q]);
                a[c][e0 + 2] = (_Float16)fmaf(mul[q], ubyte_f<2>(u), -32.f * mul[q]);
                a[c][e0 + 3] = (_Float16)fmaf(mul[q], ubyte_f<3>(u), -32.f * mul[q]);
            }
        }
    }
};

template <>
struct VLane<13> {
    static constexpr uint32_t BLOCK_BYTES = 176, BLOCK_VALUES = 256;
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) { return 32 * (2 * h + (c >> 2)) + 8 * (c & 3); }
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&a)[8]) {
        const uint4 hdr = *(const uint4 *)blk;
        const uint4 h0 = *(const uint4 *)(blk + 16), h1 = *(const uint4 *)(blk + 32);
        const uint4 q0 = *(const uint4 *)(blk + 48 + 32 * h), q1 = *(const uint4 *)(blk + 64 + 32 * h);
        const float d = half_bits(hdr.x & 0xffffu), dmin = half_bits(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * h, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        q4k_scale_min(2 * h + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        const float mul0 = d * (float)sc0, off0 = dmin * (float)m0;
        const float mul1 = d * (float)sc1, off1 = dmin * (float)m1;
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // chunk c: columns 8c..8c+7 of group 2h (low nibbles), c+4: group 2h+1
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t wd = w[2 * c + k], hd = hb[2 * c + k];
                const uint32_t lo = (wd & 0x0f0f0f0fu) | (((hd >> (2 * h)) & 0x01010101u) << 4);
                const uint32_t hi = ((wd >> 4) & 0x0f0f0f0fu) | (((hd >> (2 * h + 1)) & 0x01010101u) << 4);
                a[c][4 * k + 0] = (_Float16)fmaf(mul0, ubyte_f<0>(lo), -off0);
                a[c][4 * k + 1] = (_Float16)fmaf(mul0, ubyte_f<1>(lo), -off0);
                a[c][4 * k + 2] = (_Float16)fmaf(mul0, ubyte_f<2>(lo), -off0);
                a[c][4 * k + 3] = (_Float16)fmaf(mul0, ubyte_f<3>(lo), -off0);
                a[c + 4][4 * k + 0] = (_Float16)fmaf(mul1, ubyte_f<0>(hi), -off1);
                a[c + 4][4 * k + 1] = (_Float16)fmaf(mul1, ubyte_f<1>(hi), -off1);
                a[c + 4][4 * k + 2] = (_Float16)fmaf(mul1, ubyte_f<2>(hi), -off1);
                a[c + 4][4 * k + 3] = (_Float16)fmaf(mul1, ubyte_f<3>(hi), -off1);
            }
        }
    }
};

template <>
struct VLane<23> {
    static constexpr uint32_t BLOCK_BYTES = 136, BLOCK_VALUES = 256;
    // quarter h = groups 2h, 2h+1; chunk c of group 2h + c/4: values
    // 8*(c%4)..+8, i.e. low nibbles of bytes 0-7 / 8-15, then high nibbles
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) { return 32 * (2 * h + (c >> 2)) + 8 * (c & 3); }
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&a)[8]) {
        const uint2 hdr = *(const uint2 *)blk;
        const float d = half_bits(hdr.x & 0xffffu);
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            const uint32_t g = 2 * h + gg;
            const uint32_t low = (hdr.y >> (8 * (g / 2) + 4 * (g % 2))) & 15u;
            const int sc = (int)(low | (((hdr.x >> (16 + 2 * g)) & 3u) << 4)) - 32;
            const float mul = d * (float)sc;
            const uint2 qa = *(const uint2 *)(blk + 8 + 16 * g), qb = *(const uint2 *)(blk + 16 + 16 * g);
            const uint32_t wd[4] = {qa.x, qa.y, qb.x, qb.y};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t tl = iq4_lookup(wd[k] & 0x0f0f0f0fu), th = iq4_lookup((wd[k] >> 4) & 0x0f0f0f0fu);
                // bytes 4k..4k+3: chunk k/2 (low) and 2 + k/2 (high), elements 4*(k&1)..
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[4 * gg + (k >> 1)][4 * (k & 1) + e] = (_Float16)(mul * (float)(int8_t)((tl >> (8 * e)) & 0xffu));
                    a[4 * gg + 2 + (k >> 1)][4 * (k & 1) + e] = (_Float16)(mul * (float)(int8_t)((th >> (8 * e)) & 0xffu));
                }
            }
        }
    }
};

template <>
struct VLane<8> {
    // a "block" here is 8 Q8_0 blocks (256 columns); quarter h = 32-blocks 2h, 2h+1
    static constexpr uint32_t BLOCK_BYTES = 8 * 34, BLOCK_VALUES = 256;
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) { return 64 * h + 8 * c; }
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&a)[8]) {
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            const uint8_t *p = blk + (2 * h + bb) * 34;
            const float d = half_bits(load_u16_bytes(p));
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t v = load_u32_unaligned(p + 2 + 4 * k);
#pragma unroll
                for (int e = 0; e < 4; ++e) a[4 * bb + (k >> 1)][4 * (k & 1) + e] = (_Float16)(d * (float)(int8_t)((v >> (8 * e)) & 0xff));
            }
        }
    }
};


// Two f16 values 1024 + (t & M) from the halves of t (M keeps at most bits
// 0-9 of each half): (t & M) | 0x64006400 as one v_and_or_b32.
__device__ __forceinline__ half2v f16_masked(uint32_t t, uint32_t m) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(t), "s"(m), "v"(0x64006400u));
    return __builtin_bit_cast(half2v, r);
}

// The streamed verify tile's element order within each 8-value chunk,
// [0, 2, 1, 3, 4, 6, 5, 7]: activations go through this once per launch so
// that the weight pairs can be built from bytes (0, 2) and (1, 3) of a code
// word without moving bytes.
__device__ __forceinline__ half8 vd_swizzle(half8 v) {
    const u32x4 u = __builtin_bit_cast(u32x4, v);
    u32x4 r;
    r[0] = __builtin_amdgcn_perm(u[1], u[0], 0x05040100u);
    r[1] = __builtin_amdgcn_perm(u[1], u[0], 0x07060302u);
    r[2] = __builtin_amdgcn_perm(u[3], u[2], 0x05040100u);
    r[3] = __builtin_amdgcn_perm(u[3], u[2], 0x07060302u);
    return __builtin_bit_cast(half8, r);
}

// (1024 + v) * s - 1024 * s, fused (v_pk_fma_f16): v * s rounded once, and
// exact when |v * s| <= 2048.
__device__ __forceinline__ uint32_t scaled_codes(half2v biased, half2v s, half2v c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(biased, s, c));
}

// Six-bit scales and minima of Q4_K groups 2h and 2h+1 (the 12 scale bytes
// in s0, s1, s2; quant/decode.zig:155-158) without a branch on h: both
// groups sit in adjacent bytes 2(h&1), 2(h&1)+1 of each word, so the byte
// pairs are combined at once and the h >= 2 form is selected. Returns
// (sc0 | sc1 << 8) in *sc and (m0 | m1 << 8) in *m.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t h, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t *sc,
                                                   uint32_t *m) {
    const uint32_t sh = 16 * (h & 1);
    const uint32_t b0 = s0 >> sh, b1 = s1 >> sh, b2 = s2 >> sh;
    const uint32_t sc_lo = b0 & 0x3f3fu, m_lo = b1 & 0x3f3fu;
    const uint32_t sc_hi = (b2 & 0x0f0fu) | ((b0 >> 2) & 0x3030u);
    const uint32_t m_hi = ((b2 >> 4) & 0x0f0fu) | ((b1 >> 2) & 0x3030u);
    *sc = h >= 2 ? sc_hi : sc_lo;
    *m = h >= 2 ? m_hi : m_lo;
}

// Q4_K and Q5_K for the split-product verify tile: lane (row, quarter h)
// turns groups 2h and 2h+1 into the exact f16 integers q * sc (at most
// 31 * 63 = 1953), returns the block scale d, applied to the F32 block sum,
// and -dmin * m of its two groups, the F32 weights of the minimum term. The
// decoded value d * sc * q - dmin * m (quant/decode.zig:163-170, 240-250) is
// thereby split into two sums that each round nothing but the activations.
template <uint32_t ENC>
struct VSplit;

template <>
struct VSplit<12> {
    static constexpr uint32_t BLOCK_BYTES = 144, BLOCK_VALUES = 256;
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) { return VLane<12>::col(h, c); }
    // 16-byte reads of lane quarter h: NH header reads at 16 j, then two code
    // reads at CODE + 32 h and CODE + 32 h + 16
    static constexpr uint32_t NH = 1, CODE = 16;
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&b)[8], float &d,
                                                   float &nm0, float &nm1) {
        const uint4 hdr[NH] = {*(const uint4 *)blk};
        decode<false>(hdr, *(const uint4 *)(blk + CODE + 32 * h), *(const uint4 *)(blk + CODE + 16 + 32 * h), h, b, d,
                      nm0, nm1);
    }
    // PAIR: the streamed tile's form, with the branch-free scale unpack and
    // the element order of vd_swizzle; the register tile keeps the natural
    // order and the per-group scale unpack, which measured faster there
    template <bool PAIR>
    __device__ __forceinline__ static void decode(const uint4 (&hr)[NH], uint4 q0, uint4 q1, uint32_t h,
                                                  half8 (&b)[8], float &d, float &nm0, float &nm1) {
        const uint4 hdr = hr[0];
        d = half_bits(hdr.x & 0xffffu);
        const float dmin = half_bits(hdr.x >> 16);
        uint32_t scp, mp;
        if constexpr (PAIR) {
            q4k_scale_min_pair(h, hdr.y, hdr.z, hdr.w, &scp, &mp);
        } else {
            uint32_t a0, n0, a1, n1;
            q4k_scale_min(2 * h, hdr.y, hdr.z, hdr.w, &a0, &n0);
            q4k_scale_min(2 * h + 1, hdr.y, hdr.z, hdr.w, &a1, &n1);
            scp = a0 | (a1 << 8);
            mp = n0 | (n1 << 8);
        }
        const uint32_t sc0 = scp & 0xffu, sc1 = scp >> 8;
        nm0 = -dmin * (float)(mp & 0xffu);
        nm1 = -dmin * (float)(mp >> 8);
        // low nibbles at 1024 + q (scale sc), high nibbles at 1024 + 16 q (scale sc / 16)
        const _Float16 s0 = (_Float16)(float)sc0, s1 = (_Float16)((float)sc1 * 0.0625f);
        const half2v S0 = {s0, s0}, C0 = {(_Float16)(-1024.f * (float)sc0), (_Float16)(-1024.f * (float)sc0)};
        const half2v S1 = {s1, s1}, C1 = {(_Float16)(-64.f * (float)sc1), (_Float16)(-64.f * (float)sc1)};
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // chunk c: group 2h, c + 4: group 2h + 1 (VLane<12> order)
            u32x4 lo, hi;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if constexpr (PAIR) {  // streamed order: bytes (0, 2), then (1, 3)
                    const uint32_t w0 = w[2 * c + k], w1 = w0 >> 8;
                    lo[2 * k] = scaled_codes(f16_masked(w0, 0x000f000fu), S0, C0);
                    lo[2 * k + 1] = scaled_codes(f16_masked(w1, 0x000f000fu), S0, C0);
                    hi[2 * k] = scaled_codes(f16_masked(w0, 0x00f000f0u), S1, C1);
                    hi[2 * k + 1] = scaled_codes(f16_masked(w1, 0x00f000f0u), S1, C1);
                } else {
                    const uint32_t l4 = w[2 * c + k] & 0x0f0f0f0fu, u4 = w[2 * c + k] & 0xf0f0f0f0u;
                    lo[2 * k] = scaled_codes(f16_biased<0, 1>(l4), S0, C0);
                    lo[2 * k + 1] = scaled_codes(f16_biased<2, 3>(l4), S0, C0);
                    hi[2 * k] = scaled_codes(f16_biased<0, 1>(u4), S1, C1);
                    hi[2 * k + 1] = scaled_codes(f16_biased<2, 3>(u4), S1, C1);
                }
            }
            b[c] = __builtin_bit_cast(half8, lo);
            b[c + 4] = __builtin_bit_cast(half8, hi);
        }
    }
};

template <>
struct VSplit<13> {
    static constexpr uint32_t BLOCK_BYTES = 176, BLOCK_VALUES = 256;
    __device__ __forceinline__ static uint32_t col(uint32_t h, uint32_t c) { return VLane<13>::col(h, c); }
    static constexpr uint32_t NH = 3, CODE = 48;  // header + qh, codes (as VSplit<12>)
    __device__ __forceinline__ static void dequant(const uint8_t *blk, uint32_t h, half8 (&b)[8], float &d,
                                                   float &nm0, float &nm1) {
        const uint4 hdr[NH] = {*(const uint4 *)blk, *(const uint4 *)(blk + 16), *(const uint4 *)(blk + 32)};
        decode<false>(hdr, *(const uint4 *)(blk + CODE + 32 * h), *(const uint4 *)(blk + CODE + 16 + 32 * h), h, b, d,
                      nm0, nm1);
    }
    // PAIR: the streamed tile's form, with the branch-free scale unpack and
    // the element order of vd_swizzle; the register tile keeps the natural
    // order and the per-group scale unpack, which measured faster there
    template <bool PAIR>
    __device__ __forceinline__ static void decode(const uint4 (&hr)[NH], uint4 q0, uint4 q1, uint32_t h,
                                                  half8 (&b)[8], float &d, float &nm0, float &nm1) {
        const uint4 hdr = hr[0], h0 = hr[1], h1 = hr[2];
        d = half_bits(hdr.x & 0xffffu);
        const float dmin = half_bits(hdr.x >> 16);
        uint32_t scp, mp;
        if constexpr (PAIR) {
            q4k_scale_min_pair(h, hdr.y, hdr.z, hdr.w, &scp, &mp);
        } else {
            uint32_t a0, n0, a1, n1;
            q4k_scale_min(2 * h, hdr.y, hdr.z, hdr.w, &a0, &n0);
            q4k_scale_min(2 * h + 1, hdr.y, hdr.z, hdr.w, &a1, &n1);
            scp = a0 | (a1 << 8);
            mp = n0 | (n1 << 8);
        }
        const uint32_t sc0 = scp & 0xffu, sc1 = scp >> 8;
        nm0 = -dmin * (float)(mp & 0xffu);
        nm1 = -dmin * (float)(mp >> 8);
        const _Float16 s0 = (_Float16)(float)sc0, s1 = (_Float16)(float)sc1;
        const half2v S0 = {s0, s0}, C0 = {(_Float16)(-1024.f * (float)sc0), (_Float16)(-1024.f * (float)sc0)};
        const half2v S1 = {s1, s1}, C1 = {(_Float16)(-1024.f * (float)sc1), (_Float16)(-1024.f * (float)sc1)};
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hb[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            u32x4 lo, hi;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t wd = w[2 * c + k], hd = hb[2 * c + k];
                const uint32_t l5 = (wd & 0x0f0f0f0fu) | (((hd >> (2 * h)) & 0x01010101u) << 4);
                const uint32_t u5 = ((wd >> 4) & 0x0f0f0f0fu) | (((hd >> (2 * h + 1)) & 0x01010101u) << 4);
                constexpr int A0 = PAIR ? 0 : 0, A1 = PAIR ? 2 : 1, B0 = PAIR ? 1 : 2, B1 = 3;  // streamed order
                lo[2 * k] = scaled_codes(f16_biased<A0, A1>(l5), S0, C0);
                lo[2 * k + 1] = scaled_codes(f16_biased<B0, B1>(l5), S0, C0);
                hi[2 * k] = scaled_codes(f16_biased<A0, A1>(u5), S1, C1);
                hi[2 * k + 1] = scaled_codes(f16_biased<B0, B1>(u5), S1, C1);
            }
            b[c] = __builtin_bit_cast(half8, lo);
            b[c + 4] = __builtin_bit_cast(half8, hi);
        }
    }
};

constexpr int VF_MAX_WAVES = 16;

// RG row groups of 16 per wave: the x fragments of a block are loaded once
// and feed RG MFMA chains, so a workgroup reads x once per 16*RG rows.
template <uint32_t ENC, typename XT, int RG>
__global__ void __launch_bounds__(64 * VF_MAX_WAVES) verify_kernel(const uint8_t *__restrict__ w, uint64_t stride,
                                                                    uint32_t rows, uint32_t nblocks,
                                                                    const XT *__restrict__ x, uint64_t in_stride,
                                                                    float *__restrict__ y, uint64_t out_stride,
                                                                    uint32_t tokens) {
    __shared__ float part_sums[VF_MAX_WAVES][RG][16][16];
    using L = VLane<ENC>;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const uint32_t r16 = lane & 15, h = lane >> 4;
    const uint32_t row0 = blockIdx.x * 16 * RG;
    const bool tok_ok = r16 < tokens;
    const XT *xrow = x + (uint64_t)(tok_ok ? r16 : 0) * in_stride;

    floatx4 acc[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) acc[g] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t b = wv; b < nblocks; b += nwaves) {
        half8 bx[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t col = b * L::BLOCK_VALUES + L::col(h, c);
            if constexpr (sizeof(XT) == 2) {
                bx[c] = tok_ok ? *(const half8 *)((const _Float16 *)xrow + col) : half8{};
            } else {
                float4 f0 = tok_ok ? *(const float4 *)((const float *)xrow + col) : make_float4(0.f, 0.f, 0.f, 0.f);
                float4 f1 = tok_ok ? *(const float4 *)((const float *)xrow + col + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                bx[c][0] = (_Float16)f0.x; bx[c][1] = (_Float16)f0.y; bx[c][2] = (_Float16)f0.z; bx[c][3] = (_Float16)f0.w;
                bx[c][4] = (_Float16)f1.x; bx[c][5] = (_Float16)f1.y; bx[c][6] = (_Float16)f1.z; bx[c][7] = (_Float16)f1.w;
            }
        }
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            const uint8_t *wrow = w + (uint64_t)min(row0 + 16 * g + r16, rows - 1) * stride;
            half8 a[8];
            L::dequant(wrow + (uint64_t)b * L::BLOCK_BYTES, h, a);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c], bx[c], acc[g], 0, 0, 0);
        }
    }
    // D layout: lane l holds token l%16, rows 4*(l/16) + i
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) part_sums[wv][g][4 * h + i][r16] = acc[g][i];
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < 256 * RG; idx += blockDim.x) {
        const uint32_t g = idx >> 8, rr = (idx >> 4) & 15, t = idx & 15;
        float v = 0.f;
        for (uint32_t k = 0; k < nwaves; ++k) v += part_sums[k][g][rr][t];
        const uint32_t row = row0 + 16 * g + rr;
        if (t < tokens && row < rows) y[(uint64_t)t * out_stride + row] = v;
    }
}

// The split-product verify tile (Q4_K, Q5_K). The activations are the A
// operand (16 tokens x 32 k) and the weights the B operand, so lane
// (row r16, quarter h) holds D for its own row and tokens 4h..4h+3 and
// applies its own block scale d. Per block: eight f16 MFMAs of x against
// q * sc into a zeroed block sum, one F32 FMA by d, and two F32 MFMAs
// (16x16x4) of the group sums of x against -dmin * m.
template <uint32_t ENC, typename XT, int RG>
__global__ void __launch_bounds__(64 * VF_MAX_WAVES) verify_split_kernel(const uint8_t *__restrict__ w,
                                                                          uint64_t stride, uint32_t rows,
                                                                          uint32_t nblocks,
                                                                          const XT *__restrict__ x,
                                                                          uint64_t in_stride, float *__restrict__ y,
                                                                          uint64_t out_stride, uint32_t tokens) {
    __shared__ float part_sums[VF_MAX_WAVES][RG][16][16];
    using L = VSplit<ENC>;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const uint32_t r16 = lane & 15, h = lane >> 4;
    const uint32_t row0 = blockIdx.x * 16 * RG;
    const bool tok_ok = r16 < tokens;
    const XT *xrow = x + (uint64_t)(tok_ok ? r16 : 0) * in_stride;
    const half2v ones = {(_Float16)1.f, (_Float16)1.f};
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

    floatx4 acc[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) acc[g] = zero;
    for (uint32_t b = wv; b < nblocks; b += nwaves) {
        half8 bx[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t col = b * L::BLOCK_VALUES + L::col(h, c);
            // A rows past `tokens` (lanes reading token 0) only reach D rows
            // that are never stored, so the loads need no guard.
            if constexpr (sizeof(XT) == 2) {
                bx[c] = *(const half8 *)((const _Float16 *)xrow + col);
            } else {
                const float4 f0 = *(const float4 *)((const float *)xrow + col);
                const float4 f1 = *(const float4 *)((const float *)xrow + col + 4);
                bx[c][0] = (_Float16)f0.x; bx[c][1] = (_Float16)f0.y; bx[c][2] = (_Float16)f0.z; bx[c][3] = (_Float16)f0.w;
                bx[c][4] = (_Float16)f1.x; bx[c][5] = (_Float16)f1.y; bx[c][6] = (_Float16)f1.z; bx[c][7] = (_Float16)f1.w;
            }
        }
        // F32 sums of the (f16) activations of groups 2h and 2h+1, token r16
        float sx0 = 0.f, sx1 = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sx0 = __builtin_amdgcn_fdot2(half2v{bx[c][2 * e], bx[c][2 * e + 1]}, ones, sx0, false);
                sx1 = __builtin_amdgcn_fdot2(half2v{bx[c + 4][2 * e], bx[c + 4][2 * e + 1]}, ones, sx1, false);
            }
        }
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            const uint8_t *wrow = w + (uint64_t)min(row0 + 16 * g + r16, rows - 1) * stride;
            half8 bq[8];
            float d, nm0, nm1;
            L::dequant(wrow + (uint64_t)b * L::BLOCK_BYTES, h, bq, d, nm0, nm1);
            floatx4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[0], bq[0], zero, 0, 0, 0);
#pragma unroll
            for (int c = 1; c < 8; ++c) part = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[c], bq[c], part, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(d, part[i], acc[g][i]);
            acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx0, nm0, acc[g], 0, 0, 0);
            acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx1, nm1, acc[g], 0, 0, 0);
        }
    }
    // D layout: lane l holds weight row l%16, tokens 4*(l/16) + i
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) part_sums[wv][g][r16][4 * h + i] = acc[g][i];
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < 256 * RG; idx += blockDim.x) {
        const uint32_t g = idx >> 8, rr = (idx >> 4) & 15, t = idx & 15;
        float v = 0.f;
        for (uint32_t k = 0; k < nwaves; ++k) v += part_sums[k][g][rr][t];
        const uint32_t row = row0 + 16 * g + rr;
        if (t < tokens && row < rows) y[(uint64_t)t * out_stride + row] = v;
    }
}

// The streamed verify tile (Q4_K, Q5_K; K up to 24 blocks). Weights go
// global -> LDS with global_load_lds_dwordx4 into a two-slot ring per wave,
// as contiguous whole-row spans, instead of every lane loading its own
// scattered 16-byte pieces. Each wave owns a fixed run of at most NB blocks
// of every row: its x fragments and group sums stay in registers for the
// whole launch. A step is 16 rows x NB blocks. Per-wave partial sums of
// each (row, token) go to LDS and are added in wave order at the end, so
// results are the same run to run; the arithmetic is that of
// verify_split_kernel.
//
// With f16 activations each wave first copies the activations of its own
// blocks, contiguous per token, into LDS and reads its fragments from
// there: a lane's fragments are 16-byte pieces of 16 token rows, which as
// direct loads cost one cache line each. LDS layouts (STAGE):
//   0, 1: one region per wave (its slot 0, its slot 1 and, for 1, the extra
//         bytes its activations need past slot 1), then the partial sums
//         [row][wave][token]. No other wave touches a wave's region, so its
//         step-1 copies follow its fragment reads at once.
//   2:    every wave's slot 0, every wave's slot 1, the partial sums; the
//         activations are staged over the slot-1s and partial sums, so a
//         barrier separates the fragment reads from the step-1 copies.
// waves per workgroup: runs of 2 blocks fit 170 registers (3 waves per
// SIMD), runs of 3 need 256 (2 per SIMD)
template <uint32_t NB>
constexpr uint32_t vd_max_waves() { return NB == 2 ? 12 : 8; }
// Blocks per K range of the streamed verify tile. The F32 multi-token form
// (xs3) stages three f16 part rows per token in each wave's region: at 20
// blocks its 10 waves take 10 x 13.8 KB with three ring slots, and a CU's
// rows' partial sums still fit beside them (K = 5120 runs as one range).
constexpr uint32_t vd_max_kb(bool xs3) { return xs3 ? 20 : 2 * vd_max_waves<2>(); }

typedef __attribute__((address_space(3))) uint8_t vd_lds_u8_t;
__device__ __forceinline__ uint32_t vd_lds_addr(const uint8_t *p) { return (uint32_t)(uintptr_t)(const vd_lds_u8_t *)p; }

template <uint32_t ENC, uint32_t NB>
struct VDma {
    using L = VSplit<ENC>;
    static constexpr uint32_t BYTES = L::BLOCK_BYTES, ROW_BYTES = NB * BYTES;
    static constexpr uint32_t STEP_CHUNKS = 16 * ROW_BYTES / 16, INSTRS = (STEP_CHUNKS + 63) / 64;
    static constexpr uint32_t SLOT = STEP_CHUNKS * 16;  // the last copy runs on the lanes it needs
};

// Ring reads of block S of a step for one lane (row r16, quarter h): the
// header reads at a + S * BYTES + 16 j, the code reads at c + S * BYTES and
// + 16, where c = a + CODE + 32 h. No wait: vd_ring_wait follows.
template <uint32_t ENC, uint32_t S>
__device__ __forceinline__ void vd_read_block(uint32_t a, uint32_t c, u32x4 (&r)[VSplit<ENC>::NH], u32x4 (&q)[2]) {
    constexpr uint32_t O = S * VSplit<ENC>::BLOCK_BYTES;
    if constexpr (VSplit<ENC>::NH == 1) {
        asm volatile(
            "ds_read_b128 %0, %3 offset:%5\n\t"
            "ds_read_b128 %1, %4 offset:%5\n\t"
            "ds_read_b128 %2, %4 offset:%6"
            : "=&v"(r[0]), "=&v"(q[0]), "=&v"(q[1])
            : "v"(a), "v"(c), "n"(O), "n"(O + 16)
            : "memory");
    } else {
        static_assert(VSplit<ENC>::NH == 3, "header reads");
        asm volatile(
            "ds_read_b128 %0, %5 offset:%7\n\t"
            "ds_read_b128 %1, %5 offset:%8\n\t"
            "ds_read_b128 %2, %5 offset:%9\n\t"
            "ds_read_b128 %3, %6 offset:%7\n\t"
            "ds_read_b128 %4, %6 offset:%8"
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(q[0]), "=&v"(q[1])
            : "v"(a), "v"(c), "n"(O), "n"(O + 16), "n"(O + 32)
            : "memory");
    }
}

template <uint32_t ENC, uint32_t NB, int VM>
__device__ __forceinline__ void vd_ring_read(uint32_t a, uint32_t c, uint4 (&hd)[NB][VSplit<ENC>::NH],
                                             uint4 (&cq)[NB][2]) {
    constexpr uint32_t NH = VSplit<ENC>::NH;
    u32x4 r[NB][NH], q[NB][2];
    // the ring slot's copies are older than the VM copies of younger steps
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(VM) : "memory");
    vd_read_block<ENC, 0>(a, c, r[0], q[0]);
    vd_read_block<ENC, 1>(a, c, r[1], q[1]);
    if constexpr (NB > 2) vd_read_block<ENC, 2>(a, c, r[2], q[2]);
    static_assert(NB == 2 || NB == 3, "blocks per wave");
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    // the registers are defined after the wait, as far as the compiler knows
#pragma unroll
    for (uint32_t s = 0; s < NB; ++s) {
#pragma unroll
        for (uint32_t j = 0; j < NH; ++j) {
            asm volatile("" : "+v"(r[s][j]));
            hd[s][j] = make_uint4(r[s][j].x, r[s][j].y, r[s][j].z, r[s][j].w);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            asm volatile("" : "+v"(q[s][j]));
            cq[s][j] = make_uint4(q[s][j].x, q[s][j].y, q[s][j].z, q[s][j].w);
        }
    }
}

// The arithmetic of one streamed-verify step over NL live blocks: per
// block an independent chain of eight f16 MFMAs against q * sc, scaled by
// the block's d, plus one chain of F32 MFMAs for the minimum terms.
// With XS = 3 each D row m is one f16 part of a token's activations scaled
// by a power of two per (token, block); sfm[s][e] undoes it for D row 4h+e.
template <typename L, uint32_t NB, uint32_t NL, uint32_t XS>
__device__ __forceinline__ floatx4 vd_step_blocks(const uint4 (&hd)[NB][L::NH], const uint4 (&cq)[NB][2], uint32_t h,
                                                  const half8 (&bx)[NB][8], const float (&sx)[NB][2],
                                                  const float (&sfm)[NB][4]) {
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    floatx4 part[NL], accm = zero;
    float d[NL];
#pragma unroll
    for (uint32_t s = 0; s < NL; ++s) {
        half8 bq[8];
        float nm0, nm1;
        L::template decode<true>(hd[s], cq[s][0], cq[s][1], h, bq, d[s], nm0, nm1);
        part[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[s][0], bq[0], zero, 0, 0, 0);
#pragma unroll
        for (int c = 1; c < 8; ++c) part[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bx[s][c], bq[c], part[s], 0, 0, 0);
        accm = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[s][0], nm0, accm, 0, 0, 0);
        accm = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[s][1], nm1, accm, 0, 0, 0);
    }
    floatx4 acc = accm;
#pragma unroll
    for (uint32_t s = 0; s < NL; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(XS == 3 ? d[s] * sfm[s][e] : d[s], part[s][e], acc[e]);
    return acc;
}

// One 16-byte-per-lane copy global -> LDS as a buffer load: base in a
// buffer resource (scalar), lane offset voff, uniform offset soff, LDS
// destination lds (uniform, the lane's 16 bytes at lds + 16 lane), with the
// non-temporal hint. The record count is the maximum: callers keep every
// offset inside their rows.
__device__ __forceinline__ void vd_copy(const uint8_t *base, uint32_t lds, uint32_t voff, uint32_t soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, 0xffffffff, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(uintptr_t)lds, 16, voff, soff, 0, 2);
}

// Fragment reads of one block of staged activations: the lane's 128
// contiguous bytes at a + O (chunks c = 0..7 at 16 c). No wait.
template <uint32_t O>
__device__ __forceinline__ void vd_read_x(uint32_t a, u32x4 (&r)[8]) {
    asm volatile(
        "ds_read_b128 %0, %8 offset:%9\n\t"
        "ds_read_b128 %1, %8 offset:%10\n\t"
        "ds_read_b128 %2, %8 offset:%11\n\t"
        "ds_read_b128 %3, %8 offset:%12\n\t"
        "ds_read_b128 %4, %8 offset:%13\n\t"
        "ds_read_b128 %5, %8 offset:%14\n\t"
        "ds_read_b128 %6, %8 offset:%15\n\t"
        "ds_read_b128 %7, %8 offset:%16"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(a), "n"(O), "n"(O + 16), "n"(O + 32), "n"(O + 48), "n"(O + 64), "n"(O + 80), "n"(O + 96),
          "n"(O + 112)
        : "memory");
}

// Cross-lane reductions on the VALU (DPP within a 16-lane row, the gfx950
// row swaps across rows), no LDS round trips. Every lane ends with the same
// bits, added in the same order.
template <int CTRL>
__device__ __forceinline__ float vd_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// sum over the four rows: lanes l, l ^ 16, l ^ 32, l ^ 48
__device__ __forceinline__ float vd_rows_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// maximum over the whole wave
__device__ __forceinline__ float vd_wave_max(float v) {
    v = fmaxf(v, vd_dpp<0xb1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, vd_dpp<0x4e>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, vd_dpp<0x141>(v));  // row_half_mirror
    v = fmaxf(v, vd_dpp<0x140>(v));  // row_mirror
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// XS = 3 (F32 activations, at most 3 tokens): A row 4p + t is part p of
// token t's activations, x * 2^e = p0 + p1 + p2 (each part the f16 rounding
// of what the earlier ones leave, so the sum holds every bit of x), with
// 2^e per (token, wave run) putting the run's largest |x| in [2^14, 2^15).
// The weights are exact f16 integers, so every product is exact and the
// MFMA sums carry F32 rounding only: the F32 precision of the multi-token
// GEMV (ops/matvec.zig:149-188) on the matrix cores. A lane's D rows 4h + e
// are part h of token e, so adding the four h lanes gives the token's sum;
// the partial sums then hold 4 tokens per (row, wave). The parts are staged
// per wave (STAGE 1), part p of token t at staging row pT + t.
template <uint32_t ENC, uint32_t NB, typename XT, int STAGE, uint32_t DEPTH, uint32_t XS = 1>
__global__ void __launch_bounds__(64 * vd_max_waves<NB>()) verify_dma_kernel(const uint8_t *__restrict__ w_all,
                                                                        uint64_t stride, uint32_t rows,
                                                                        uint32_t nblocks_all,
                                                                        const XT *__restrict__ x_all,
                                                                        uint64_t in_stride, float *__restrict__ y_all,
                                                                        uint64_t out_stride, uint32_t tokens,
                                                                        uint32_t tpad, uint32_t region,
                                                                        uint32_t slot_gap, uint32_t part_off,
                                                                        uint32_t kb, uint64_t y_range) {
    using L = VSplit<ENC>;
    using V = VDma<ENC, NB>;
    // K ranges (gridDim.y > 1): workgroup (bx, by) takes blocks
    // [by kb, (by + 1) kb) and stores its sums y_range floats further on
    const uint32_t kb0 = blockIdx.y * kb;
    const uint32_t nblocks = gridDim.y > 1 ? min(kb, nblocks_all - kb0) : nblocks_all;
    const uint8_t *__restrict__ w = w_all + (uint64_t)kb0 * L::BLOCK_BYTES;
    const XT *__restrict__ x = x_all + (uint64_t)kb0 * L::BLOCK_VALUES;
    float *__restrict__ y = y_all + blockIdx.y * y_range;
    extern __shared__ __attribute__((aligned(16))) uint8_t vd_lds[];
    const uint32_t lane = threadIdx.x & 63, kw = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const uint32_t r16 = lane & 15, h = lane >> 4;
    uint8_t *ring = vd_lds + __builtin_amdgcn_readfirstlane(kw * region);  // slot d at + d * slot_gap
    const uint32_t slot_stride = slot_gap;
    float *partial = (float *)(vd_lds + part_off);  // [row][wave][tpad]
    // balanced row ranges: every workgroup holds at least 16 rows (the host
    // launches at most rows / 16 workgroups)
    const uint32_t row_begin = (uint32_t)((uint64_t)blockIdx.x * rows / gridDim.x);
    const uint32_t nrow = (uint32_t)((uint64_t)(blockIdx.x + 1) * rows / gridDim.x) - row_begin;
    const uint32_t nsteps = (nrow + 15) / 16;
    // wave kw owns blocks [kw nblocks / nwaves, (kw + 1) nblocks / nwaves)
    // NB = 3: runs of 3 blocks on the first nblocks - 2 nwaves waves, 2 on the
    // rest, so with 8 waves each SIMD's two waves (kw, kw + 4) hold 5 blocks
    const uint32_t x3 = NB == 3 ? nblocks - 2 * nwaves : 0;
    const uint32_t b0 = __builtin_amdgcn_readfirstlane(NB == 3 ? 2 * kw + min(kw, x3) : kw * nblocks / nwaves);
    const uint32_t nlive = __builtin_amdgcn_readfirstlane(NB == 3 ? 2 + (kw < x3 ? 1 : 0)
                                                                   : (kw + 1) * nblocks / nwaves - b0);  // 1 .. NB

    // This lane's chunk of each copy: row q of the step and byte offset in
    // the row (chunks past the step repeat the last one; a block past the
    // row's end copies the wave's first block again, so every copy stays in
    // the row).
    // A step's 16 rows start at row min(16 i, nrow - 16) of the range: the
    // last step moves back to end at the range's last row, and stores only
    // the rows no earlier step stored. So every copy is a uniform step base
    // plus this lane's fixed 32-bit offset (16 rows span < 4 GiB).
    uint32_t doff[V::INSTRS];
#pragma unroll
    for (uint32_t n = 0; n < V::INSTRS; ++n) {
        const uint32_t k = min(64 * n + lane, V::STEP_CHUNKS - 1);
        const uint32_t in_row = 16 * (k % (V::ROW_BYTES / 16)), sblk = in_row / V::BYTES;
        doff[n] = (k / (V::ROW_BYTES / 16)) * (uint32_t)stride + b0 * V::BYTES +
                  (sblk < nlive ? in_row : in_row - sblk * V::BYTES);
    }
    const uint8_t *wg_base = w + (uint64_t)row_begin * stride;
    // The copies run as buffer loads: the workgroup's base in a buffer
    // resource, the step's row offset as the scalar offset and the lane's
    // fixed 32-bit offset, so a copy costs no VALU. Every offset stays in
    // the workgroup's rows, so the record count is left at its maximum.
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(vd_lds_addr(ring));
    // DEPTH 1 (VS): one register set per wave instead of ring slots: step
    // i + 1's 16-byte pieces are loaded into registers while step i computes
    // and written to the wave's single slot at the top of step i + 1.
    constexpr bool VS = DEPTH == 1;
    u32x4 vr[V::INSTRS];
#define NUQ_VD_DMA(SLOT_, STEP_)                                                                          \
    {                                                                                                   \
    if constexpr (VS) {                                                                                 \
        const uint32_t soff_ = min(16 * (STEP_), nrow - 16) * (uint32_t)stride;                         \
        _Pragma("unroll") for (uint32_t n = 0; n < V::INSTRS; ++n) vr[n] =                              \
            __builtin_nontemporal_load((const u32x4 *)(wg_base + soff_ + doff[n]));                     \
    } else {                                                                                            \
        const uint32_t soff_ = min(16 * (STEP_), nrow - 16) * (uint32_t)stride;                         \
        const uint32_t dst_ = ring_lds + (SLOT_) * slot_stride;                                         \
        _Pragma("unroll") for (uint32_t n = 0; n < V::INSTRS; ++n) {                                    \
            if (64 * (n + 1) <= V::STEP_CHUNKS || 64 * n + lane < V::STEP_CHUNKS)                          \
                vd_copy(wg_base, dst_ + n * 1024, doff[n], soff_);                                      \
        }                                                                                               \
    }                                                                                                   \
    }
    half8 bx[NB][8];
    float sx3[NB][2], sft[4];  // XS = 3: F32 group sums; each token's scale back
    float gs3[2][2] = {{0.f, 0.f}, {0.f, 0.f}};  // XS = 3: staged group sums of this lane's token
    u32x4 xr3[NB][8] = {};  // XS = 3: this lane's part fragments, read during the staging
    if constexpr (STAGE != 0) {
        // this wave's activations, [token][its blocks' 512 bytes], copied
        // before the step-0 weights so that they are waited for alone
        static_assert(NB <= 2 || (XS == 1 && STAGE == 1), "a run's activations are 32, 64 or 96 chunks per token");
        const uint32_t span = nlive * 512, xchunks = tokens * span / 16;
        const uint32_t span_log2 = nlive == 2 ? 6 : 5;  // log2(span / 16)
        // (VS: in the slot itself, whose first step waits in registers until
        // the activations are read)
        uint8_t *xs = STAGE == 1 ? (VS ? ring : ring + V::SLOT) : vd_lds + nwaves * V::SLOT + b0 * tokens * 512;
        if constexpr (XS == 3) {
            // F32 activations: lane k converts values [8k, 8k + 8) of the
            // wave's run of each token into its three f16 parts, the F32
            // sums of 32-value groups go to the lanes that need them, and the
            // wave agrees on the token's scale 2^e. Tokens go through the
            // staging two at a time (part p of the phase's token tt at
            // staging row 2p + tt), each lane reading its fragments in its
            // token's phase, so four tokens stage in the room of two.
            static_assert(STAGE == 1, "F32 activations are staged in the wave's own region");
            (void)xchunks;
            (void)span_log2;
            // (LDS accesses as asm: see vd_read_x)
            const bool live_k = 8 * lane < nlive * 256;
            // every token's values are loaded before the step-0 copies; lanes
            // past the run and tokens past `tokens` load valid bytes and drop them
            float4 fl[4][2];
#pragma unroll
            for (uint32_t t = 0; t < 4; ++t) {
                const float *src = (const float *)x + (uint64_t)min(t, tokens - 1) * in_stride + b0 * L::BLOCK_VALUES +
                                   8 * (live_k ? lane : 0);
                fl[t][0] = *(const float4 *)src;
                fl[t][1] = *(const float4 *)(src + 4);
            }
            NUQ_VD_DMA(0, 0)
#pragma unroll
            for (uint32_t t = 0; t < 4; ++t) sft[t] = 0.f;
            const uint32_t ap3 = r16 >> 2, at3 = r16 & 3;
#pragma unroll
            for (uint32_t ph = 0; ph < 2; ++ph) {
                if (2 * ph >= tokens) break;
#pragma unroll
                for (uint32_t tt = 0; tt < 2; ++tt) {
                    const uint32_t t = 2 * ph + tt;
                    if (t >= tokens) continue;
                    const float f[8] = {fl[t][0].x, fl[t][0].y, fl[t][0].z, fl[t][0].w,
                                        fl[t][1].x, fl[t][1].y, fl[t][1].z, fl[t][1].w};
                    float amax = 0.f, cs = 0.f;
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        amax = fmaxf(amax, fabsf(f[k]));
                        cs += f[k];
                    }
                    if (!live_k) amax = cs = 0.f;
                    amax = vd_wave_max(amax);
                    // group sums: the four lanes of a 32-value group
                    cs += vd_dpp<0xb1>(cs);
                    cs += vd_dpp<0x4e>(cs);
                    // lane (r16, h) of part 0 of this token keeps the sums of
                    // groups 2h, 2h + 1 of each block: lanes 32s + 8h + 4q
#pragma unroll
                    for (uint32_t sb = 0; sb < 2; ++sb)
#pragma unroll
                        for (uint32_t q = 0; q < 2; ++q) {
                            const float g = __shfl(cs, 32 * sb + 8 * h + 4 * q, 64);
                            if (at3 == t) gs3[sb][q] = g;
                        }
                    // 2^e with the run's largest |x| * 2^e in [2^14, 2^15); 1 for
                    // zero or non-finite runs (non-finite values reach the MFMA)
                    int ex = 0;
                    if (amax > 0.f && amax <= 3.0e38f) {
                        (void)frexpf(amax, &ex);
                        ex = 15 - ex;
                    }
                    sft[t] = ldexpf(1.f, -ex);
                    half8 p0, p1, p2;
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const float xv = ldexpf(f[k], ex);
                        p0[k] = (_Float16)xv;
                        const float r1 = xv - (float)p0[k];
                        p1[k] = (_Float16)r1;
                        p2[k] = (_Float16)(r1 - (float)p1[k]);
                    }
                    if (live_k) {
                        uint32_t dst = vd_lds_addr(xs + tt * span + 16 * lane);
                        const uint32_t pst = 2 * span;
                        asm volatile("ds_write_b128 %0, %1\n\t"
                                     "v_add_u32 %0, %0, %4\n\t"
                                     "ds_write_b128 %0, %2\n\t"
                                     "v_add_u32 %0, %0, %4\n\t"
                                     "ds_write_b128 %0, %3"
                                     : "+&v"(dst)
                                     : "v"(__builtin_bit_cast(u32x4, p0)), "v"(__builtin_bit_cast(u32x4, p1)),
                                       "v"(__builtin_bit_cast(u32x4, p2)), "v"(pst)
                                     : "memory");
                    }
                }
                // this phase's part rows are written (one wave: its LDS
                // accesses complete in order); its lanes read their fragments
                asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
                if (ap3 < 3 && at3 < tokens && (at3 >> 1) == ph) {
                    const uint32_t xa = vd_lds_addr(xs) + (2 * ap3 + (at3 & 1)) * span + 128 * h;
                    vd_read_x<0>(xa, xr3[0]);
                    if (nlive > 1) vd_read_x<512>(xa, xr3[1]);
                    // the reads land before the next phase writes over the
                    // rows, and before anything reads the registers
                    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
#pragma unroll
                    for (uint32_t s = 0; s < NB; ++s)
#pragma unroll
                        for (int c = 0; c < 8; ++c) asm volatile("" : "+v"(xr3[s][c]));
                }
            }
        } else {
            for (uint32_t jx = 0; 64 * jx < xchunks; ++jx) {
                const uint32_t k = 64 * jx + lane;
                if (k < xchunks) {
                    const uint32_t t = nlive == 3 ? k / 96 : k >> span_log2;
                    const uint32_t rem = k - t * (span / 16);
                    const uint8_t *src = (const uint8_t *)x + ((uint64_t)t * in_stride + b0 * L::BLOCK_VALUES) * 2 + rem * 16;
                    __builtin_amdgcn_global_load_lds((global_void_t *)src, (lds_void_t *)(xs + 1024 * jx), 16, 0, 0);
                }
            }
            NUQ_VD_DMA(0, 0)
        }
        asm volatile("s_waitcnt vmcnt(%0)" : : "n"(V::INSTRS) : "memory");
        // lanes of tokens past `tokens` read token 0: they reach only D rows
        // that are never stored. XS = 3: A row r16 = 4p + t is part p of
        // token t; rows of p = 3 or t >= tokens are zero (they are added
        // into the stored sums).
        const uint32_t ap = r16 >> 2, at = r16 & 3;
        const bool arow = XS == 3 ? ap < 3 && at < tokens : r16 < tokens;
        u32x4 xr[NB][8] = {};  // a wave's block past the row's end stays zero
        if constexpr (XS == 3) {
#pragma unroll
            for (uint32_t s = 0; s < NB; ++s)
#pragma unroll
                for (int c = 0; c < 8; ++c) xr[s][c] = xr3[s][c];
        } else {
            const uint32_t srow = arow ? r16 : 0;
            const uint32_t xa = vd_lds_addr(xs) + srow * span + 128 * h;
            vd_read_x<0>(xa, xr[0]);
            if (nlive > 1) vd_read_x<512>(xa, xr[1]);
            if constexpr (NB > 2) {
                if (nlive > 2) vd_read_x<1024>(xa, xr[2]);
            }
        }
        if constexpr (XS == 3) {
            // F32 group sums 2h, 2h + 1 of each block, for part 0 of a token
#pragma unroll
            for (uint32_t s = 0; s < NB; ++s) {
                const bool ok = arow && ap == 0 && s < nlive;
                sx3[s][0] = ok ? gs3[s][0] : 0.f;
                sx3[s][1] = ok ? gs3[s][1] : 0.f;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
#pragma unroll
        for (uint32_t s = 0; s < NB; ++s)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                asm volatile("" : "+v"(xr[s][c]));
                if (XS == 3 && !arow) xr[s][c] = u32x4{0u, 0u, 0u, 0u};
                bx[s][c] = __builtin_bit_cast(half8, xr[s][c]);
            }
        // the fragments are in registers: slots 1.. take their first steps
        if constexpr (STAGE == 2) __builtin_amdgcn_s_barrier();
#pragma unroll
        for (uint32_t d = 1; d < DEPTH; ++d)
            if (d < nsteps) NUQ_VD_DMA(d, d)
    } else {
        // x fragments of the wave's blocks, loaded directly and before the
        // first copies, so that they are waited for alone (loads return in
        // order). Every lane loads (lanes of tokens past `tokens` read token
        // 0) and those A rows are zeroed afterwards: they reach only D rows
        // that are never stored. The loads are unconditional so that they all
        // go out before the first wait.
        const bool tok_ok = r16 < tokens;
        const XT *xrow = x + (uint64_t)(tok_ok ? r16 : 0) * in_stride;
        using XV = typename std::conditional<sizeof(XT) == 2, half8, float4>::type;
        constexpr int XP = sizeof(XT) == 2 ? 1 : 2;  // 16-byte loads per chunk
        XV xv[NB][8][XP];
#pragma unroll
        for (uint32_t s = 0; s < NB; ++s) {
            const uint32_t blk = s < nlive ? b0 + s : b0;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t col = blk * L::BLOCK_VALUES + L::col(h, c);
#pragma unroll
                for (int p = 0; p < XP; ++p) xv[s][c][p] = *(const XV *)(xrow + col + 8 / XP * p);
            }
        }
        // (every slot takes a step, real or not, so that the compiler counts
        // the copies exactly and waits for the x loads alone)
#pragma unroll
        for (uint32_t d = 0; d < DEPTH; ++d) NUQ_VD_DMA(d, d)
#pragma unroll
        for (uint32_t s = 0; s < NB; ++s)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                if constexpr (sizeof(XT) == 2) {
                    bx[s][c] = xv[s][c][0];
                } else {
                    const float4 f0 = xv[s][c][0], f1 = xv[s][c][1];
                    bx[s][c] = half8{(_Float16)f0.x, (_Float16)f0.y, (_Float16)f0.z, (_Float16)f0.w,
                                     (_Float16)f1.x, (_Float16)f1.y, (_Float16)f1.z, (_Float16)f1.w};
                }
                if (!tok_ok) bx[s][c] = half8{};
            }
    }

#pragma unroll
    for (uint32_t s = 0; s < NB; ++s)
#pragma unroll
        for (int c = 0; c < 8; ++c) bx[s][c] = vd_swizzle(bx[s][c]);

    // F32 sums of the f16 activations of groups 2h and 2h+1 of each block
    const half2v ones = {(_Float16)1.f, (_Float16)1.f};
    float sx[NB][2], sfm[NB][4];
#pragma unroll
    for (uint32_t s = 0; s < NB; ++s) {
        if constexpr (XS == 3) {
            sx[s][0] = sx3[s][0];
            sx[s][1] = sx3[s][1];
            // D row 4h + e is part h of token e
#pragma unroll
            for (int e = 0; e < 4; ++e) sfm[s][e] = sft[e];
            continue;
        }
        sx[s][0] = sx[s][1] = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sx[s][0] = __builtin_amdgcn_fdot2(half2v{bx[s][c][2 * e], bx[s][c][2 * e + 1]}, ones, sx[s][0], false);
                sx[s][1] = __builtin_amdgcn_fdot2(half2v{bx[s][c + 4][2 * e], bx[s][c + 4][2 * e + 1]}, ones,
                                                  sx[s][1], false);
            }
    }

    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    const uint32_t ring_a = vd_lds_addr(ring) + r16 * V::ROW_BYTES;
    const uint32_t part_a = vd_lds_addr((const uint8_t *)partial) + ((r16 * nwaves + kw) * tpad + 4 * h) * 4;
    const uint32_t part_step = 16 * nwaves * tpad * 4;
    const bool store_tokens = 4 * h < tpad;
    uint32_t slot = 0;  // i % DEPTH
    for (uint32_t i = 0; i < nsteps; ++i) {
        uint4 hd[NB][L::NH], cq[NB][2];
        const uint32_t a = ring_a + slot * slot_stride;
        if constexpr (VS) {
            // the step's pieces go to the slot (the compiler waits for their
            // loads), the next step's loads go out, and the slot is read back
            // (LDS operations of a wave complete in order)
#pragma unroll
            for (uint32_t n = 0; n < V::INSTRS; ++n)
                if (64 * (n + 1) <= V::STEP_CHUNKS || 64 * n + lane < V::STEP_CHUNKS)
                    *(u32x4 *)(ring + n * 1024 + 16 * lane) = vr[n];
            if (i + 1 < nsteps) NUQ_VD_DMA(0, i + 1)
            vd_ring_read<ENC, NB, 63>(a, a + L::CODE + 32 * h, hd, cq);
        } else {
            // the copies of up to DEPTH - 1 younger steps may still be in flight
            const uint32_t ahead = min(DEPTH - 1, nsteps - 1 - i);
            if (DEPTH > 2 && ahead >= 2)
                vd_ring_read<ENC, NB, 2 * V::INSTRS>(a, a + L::CODE + 32 * h, hd, cq);
            else if (ahead >= 1)
                vd_ring_read<ENC, NB, V::INSTRS>(a, a + L::CODE + 32 * h, hd, cq);
            else
                vd_ring_read<ENC, NB, 0>(a, a + L::CODE + 32 * h, hd, cq);
        }
        // one copy of the step body per live block count (wave-uniform), so
        // the per-block results need no merging
        static_assert(NB == 2 || NB == 3, "live block counts 1 and 2, or 2 and 3");
        const floatx4 acc = nlive == NB ? vd_step_blocks<L, NB, NB, XS>(hd, cq, h, bx, sx, sfm)
                                        : vd_step_blocks<L, NB, NB - 1, XS>(hd, cq, h, bx, sx, sfm);
        // D: lane holds row base + r16 (base = min(16 i, nrow - 16)), tokens
        // 4h..4h+3; rows an earlier step stored are skipped (written through
        // asm: the compiler would otherwise wait for every ring copy in flight)
        const uint32_t base = min(16 * i, nrow - 16);
        if constexpr (XS == 3) {
            // the token's three parts (and the zero rows of h = 3) add up
            floatx4 sum = acc;
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[e] = vd_rows_sum(sum[e]);
            if (h == 0 && base + r16 >= 16 * i)
                asm volatile("ds_write_b128 %0, %1" : : "v"(part_a + base * (part_step / 16)), "v"(sum) : "memory");
        } else if (store_tokens && base + r16 >= 16 * i) {
            asm volatile("ds_write_b128 %0, %1" : : "v"(part_a + base * (part_step / 16)), "v"(acc) : "memory");
        }
        // the slot's refill goes out after the step's arithmetic: a copy that
        // waits for room in the memory queue then holds up no arithmetic
        // (17408 x 5120: M=8 17.9 -> 17.5 us, T=2 18.3 -> 17.5 us)
        if constexpr (!VS) {
            if (i + DEPTH < nsteps) NUQ_VD_DMA(slot, i + DEPTH)
            slot = slot + 1 == DEPTH ? 0 : slot + 1;
        }
    }
#undef NUQ_VD_DMA
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" : : : "memory");
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < nrow * tokens; idx += blockDim.x) {
        const uint32_t t = idx / nrow, r = idx - t * nrow;
        float v = 0.f;
        for (uint32_t k = 0; k < nwaves; ++k) v += partial[(r * nwaves + k) * tpad + t];
        y[(uint64_t)t * out_stride + row_begin + r] = v;
    }
}

// The LDS layout of one launch (see verify_dma_kernel).
struct VdLayout {
    int stage;          // 0 direct activation loads, 1 private staging, 2 shared staging
    uint32_t depth;     // ring slots per wave (2 or 3)
    uint32_t region;    // per-wave stride of slot 0
    uint32_t slot_gap;  // slot 1 - slot 0
    uint32_t part_off;  // partial sums
    size_t per_row;     // partial-sum bytes per row
    size_t lds;         // for rows_per_wg rows
};

template <uint32_t ENC, uint32_t NB>
static hipError_t launch_verify_dma_nb(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows,
                                       uint32_t nblocks, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                                       uint64_t out_stride, uint32_t tokens, uint32_t tpad, uint32_t wgs,
                                       const VdLayout &L, uint32_t waves, uint32_t ranges, uint32_t kb,
                                       uint64_t y_range, bool xs3) {
    const dim3 grid(wgs, ranges), block(64 * waves);
#define NUQ_VD_LAUNCH(XT_, MODE_, D_, XS_)                                                                   \
    hipLaunchKernelGGL((verify_dma_kernel<ENC, NB, XT_, MODE_, D_, XS_>), grid, block, L.lds, s, w, stride, rows, \
                       nblocks, (const XT_ *)x, in_stride, y, out_stride, tokens, tpad, L.region, L.slot_gap,      \
                       L.part_off, kb, y_range)
#define NUQ_VD_LAUNCH_D(XT_, MODE_, XS_)                                                                     \
    if (L.depth == 3)                                                                                       \
        NUQ_VD_LAUNCH(XT_, MODE_, 3, XS_);                                                                  \
    else if (L.depth == 2)                                                                                  \
        NUQ_VD_LAUNCH(XT_, MODE_, 2, XS_);                                                                  \
    else                                                                                                    \
        NUQ_VD_LAUNCH(XT_, MODE_, 1, XS_);
    if (xs3) {
        NUQ_VD_LAUNCH_D(float, 1, 3)
    } else if (x_f16 && L.stage == 1) {
        NUQ_VD_LAUNCH_D(_Float16, 1, 1)
    } else if (x_f16 && L.stage == 2) {
        NUQ_VD_LAUNCH_D(_Float16, 2, 1)
    } else if (x_f16) {
        NUQ_VD_LAUNCH_D(_Float16, 0, 1)
    } else {
        NUQ_VD_LAUNCH_D(float, 0, 1)
    }
#undef NUQ_VD_LAUNCH_D
#undef NUQ_VD_LAUNCH
    return hipGetLastError();
}

// Adds the K ranges' partial sums in range order: y[t][r] = sum over k of
// ws[k][t][r] (ws rows x tokens per range, rows contiguous).
__global__ void verify_reduce_kernel(const float *__restrict__ ws, uint32_t nranges, uint32_t rows, uint32_t tokens,
                                     float *__restrict__ y, uint64_t out_stride) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * tokens) return;
    const uint32_t t = i / rows, r = i - t * rows;
    float v = 0.f;
    for (uint32_t k = 0; k < nranges; ++k) v += ws[((uint64_t)k * tokens + t) * rows + r];
    y[(uint64_t)t * out_stride + r] = v;
}

hipError_t launch_verify_reduce(hipStream_t s, const float *ws, uint32_t ranges, uint32_t rows, uint32_t tokens,
                                float *y, uint64_t out_stride) {
    const uint32_t n = rows * tokens;
    hipLaunchKernelGGL(verify_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, s, ws, ranges, rows, tokens, y,
                       out_stride);
    return hipGetLastError();
}

// Streams when the row's blocks fit 12 waves of at most 2 blocks, or, with a
// workspace, in K ranges of at most 24 blocks whose sums verify_reduce_kernel
// adds; returns false (nothing launched) otherwise.
// xs3: F32 activations of at most 4 tokens as three f16 parts each (the
// kernel's XS = 3): F32 precision.
template <uint32_t ENC>
static bool launch_verify_dma(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t nblocks_all,
                              const void *x, uint32_t x_f16, uint64_t in_stride, float *y_out,
                              uint64_t out_stride_out, uint32_t out_tokens, hipError_t *err,
                              const SplitScratch *scratch = nullptr, bool xs3 = false) {
    if (xs3 && (x_f16 || out_tokens > 4)) return false;
    const uint32_t tokens = out_tokens;
    constexpr uint32_t MAXW = vd_max_waves<2>();
    constexpr size_t LDS = 160 * 1024;
    if (rows < 16) return false;
    // K ranges: longer rows (the down projection) run as `ranges` ranges of
    // kb blocks over the workgroups, into the prefill workspace
    uint32_t ranges = 1, kb = nblocks_all;
    const uint32_t max_kb = vd_max_kb(xs3);
    if (nblocks_all > max_kb) {
        ranges = (nblocks_all + max_kb - 1) / max_kb;
        kb = (nblocks_all + ranges - 1) / ranges;
        if (!scratch || !scratch->work ||
            (uint64_t)ranges * out_tokens * rows > (uint64_t)scratch->tiles * 256 * 256)
            return false;
    }
    const uint32_t nblocks = kb;
    float *y = ranges > 1 ? scratch->work : y_out;
    const uint64_t out_stride = ranges > 1 ? rows : out_stride_out;
    // One wave per 2 blocks: equal work per wave and up to 3 waves per SIMD.
    // At K = 20 blocks this measured faster than 8 waves of 3 + 2 blocks per
    // SIMD (one wave left alone on its SIMD at the end) and than 12 waves of
    // 1 or 2 blocks (5 blocks on every SIMD, but more per-wave overhead).
    // Q4_K rows split into K ranges of 17-24 blocks (the down projection's
    // 68 blocks: 23 + 23 + 22) with f16 activations run on 8 waves of 3- and
    // 2-block runs (NB = 3, register-staged): 5120 x 17408 at M=8 went from
    // 19.6 to 18.4-18.6 us. At K = 5120 (one range of 20 blocks) it measured
    // no better than 10 waves of 2 blocks, which keep that shape.
    if constexpr (ENC == 12) {
        const uint32_t last = nblocks_all - (ranges - 1) * kb;  // the last range's blocks
        if (!xs3 && x_f16 && ranges > 1 && kb >= 17 && kb <= 24 && last >= 17) {
            constexpr uint32_t W3 = 8;
            const uint32_t tpad3 = (tokens + 3) & ~3u;
            const size_t slot3 = VDma<ENC, 3>::SLOT;
            const size_t region3 = std::max(slot3, (size_t)tokens * 3 * 512);
            const size_t rings3 = W3 * region3;
            const size_t per_row3 = (size_t)W3 * tpad3 * 4;
            if (rings3 + 16 * per_row3 <= LDS) {
                const uint32_t fit = (uint32_t)((LDS - rings3) / per_row3);
                const uint32_t steps16 = (rows + 15) / 16, cap = std::max(1u, 256 / ranges);
                const uint32_t per_wg = (steps16 + cap - 1) / cap;
                uint32_t wgs = std::max((steps16 + per_wg - 1) / per_wg, (rows + fit - 1) / fit);
                wgs = std::min(wgs, rows / 16);
                const uint32_t rpw = (rows + wgs - 1) / wgs;
                if (rpw <= fit && (uint64_t)rpw * stride <= 0xffffffffull) {
                    const size_t lds = rings3 + rpw * per_row3;
                    hipLaunchKernelGGL((verify_dma_kernel<ENC, 3, _Float16, 1, 1, 1>), dim3(wgs, ranges), dim3(64 * W3),
                                       lds, s, w, stride, rows, nblocks_all, (const _Float16 *)x, in_stride, y,
                                       out_stride, tokens, tpad3, (uint32_t)region3, (uint32_t)slot3, (uint32_t)rings3,
                                       kb, (uint64_t)out_tokens * rows);
                    *err = hipGetLastError();
                    if (*err == hipSuccess && ranges > 1) {
                        const uint32_t n = rows * out_tokens;
                        hipLaunchKernelGGL(verify_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, s, scratch->work,
                                           ranges, rows, out_tokens, y_out, out_stride_out);
                        *err = hipGetLastError();
                    }
                    return true;
                }
            }
        }
    }
    const uint32_t waves = (nblocks + 1) / 2;
    const uint32_t tpad = xs3 ? 4 : (tokens + 3) & ~3u;
    const size_t slot = VDma<ENC, 2>::SLOT;
    // wave kw's run: [kw nblocks / waves, (kw + 1) nblocks / waves)
    uint32_t max_run = 0;
    for (uint32_t k = 0; k < waves; ++k) max_run = std::max(max_run, (k + 1) * nblocks / waves - k * nblocks / waves);
    // staged activations per wave: f16 rows, or (xs3) three part rows per
    // token of a staging phase (two tokens)
    const size_t xwave = (size_t)(xs3 ? 3 * std::min(tokens, 2u) : tokens) * max_run * 512;
    const size_t xall = (size_t)tokens * nblocks * 512;
    const size_t per_row = (size_t)waves * tpad * 4;
    // One workgroup per CU when the partial sums of its rows fit, else more,
    // shorter row ranges; never more than rows / 16 workgroups, so each range
    // holds at least 16 rows (the kernel's steps assume it). Ranges differ by
    // at most one row.
    const uint32_t want_rows = std::max(16u, (rows * ranges + 255) / 256);
    // Candidates in order of preference: three ring slots (two steps in
    // flight while one computes), then two (Q4_K without xs3: the single
    // register-staged slot); within each, private staging,
    // shared staging, direct loads (the only one for F32 activations). The
    // first whose rings and partial sums hold want_rows rows wins, else the
    // one holding the most.
    VdLayout L{}, best{};
    uint32_t best_rows = 0;
    const int modes_f16[3] = {1, 2, 0}, modes_f32[1] = {0}, modes_xs3[1] = {1};
    const int *modes = xs3 ? modes_xs3 : x_f16 ? modes_f16 : modes_f32;
    bool found = false;
    // Q4_K with one token row per MFMA row (not xs3) stages each step through
    // registers (depth 1): 17408 x 5120 at M=8 took 16.3-16.7 us against
    // 17.7 with the three-slot ring. The register set spills on Q5_K and
    // with xs3, which keep the rings.
    const bool vs = ENC == 12 && !xs3;
    for (uint32_t depth = vs ? 1 : 3; depth >= (vs ? 1u : 2u) && !found; --depth) {
        for (int m = 0; m < (x_f16 ? 3 : 1); ++m) {
            const int mode = modes[m];
            VdLayout c{};
            c.stage = mode;
            c.depth = depth;
            c.per_row = per_row;
            const size_t ahead = (depth - 1) * slot;  // staging room from slot 1 on
            c.region = (uint32_t)(mode == 1 ? (depth == 1 ? std::max(slot, xwave)
                                                          : depth * slot + (xwave > ahead ? xwave - ahead : 0))
                                            : mode == 2 ? slot : depth * slot);
            c.slot_gap = (uint32_t)(mode == 2 ? waves * slot : slot);
            const size_t rings = mode == 2 ? depth * waves * slot : (size_t)waves * c.region;
            c.part_off = (uint32_t)rings;
            if (mode == 2 && waves * slot + xall > LDS) continue;
            if (rings + 16 * per_row > LDS) continue;
            const uint32_t fit = (uint32_t)((LDS - rings) / per_row);
            if (fit > best_rows) {
                best = c;
                best_rows = fit;
            }
            if (fit >= want_rows) {
                best = c;
                best_rows = fit;
                found = true;
                break;
            }
        }
    }
    if (best_rows < 16) return false;
    L = best;
    const uint32_t rings_end = L.part_off;
    // As few workgroups as keep the longest row range at the same number of
    // 16-row steps: ranges then end near a multiple of 16 rows, so the last
    // step (moved back to end at the range's last row) re-reads few rows.
    // 17408 rows: 218 workgroups of 80 rows instead of 256 of 68 (5 steps
    // either way, 12 rows re-read per range).
    const uint32_t steps16 = (rows + 15) / 16, cap = std::max(1u, 256 / ranges);
    const uint32_t per_wg = (steps16 + cap - 1) / cap;
    uint32_t wgs = std::max((steps16 + per_wg - 1) / per_wg, (rows + best_rows - 1) / best_rows);
    wgs = std::min(wgs, rows / 16);
    const uint32_t rows_per_wg = (rows + wgs - 1) / wgs;  // the longest range
    if (rows_per_wg > best_rows) return false;
    // a range's copy offsets (step base + lane offset) are 32-bit
    if ((uint64_t)rows_per_wg * stride > 0xffffffffull) return false;
    const size_t xall_lds = L.stage == 2 ? waves * slot + xall : 0;
    L.lds = std::max(rings_end + rows_per_wg * L.per_row, xall_lds);
    *err = launch_verify_dma_nb<ENC, 2>(s, w, stride, rows, nblocks_all, x, x_f16, in_stride, y, out_stride, tokens,
                                        tpad, wgs, L, waves, ranges, kb, (uint64_t)out_tokens * rows, xs3);
    if (*err == hipSuccess && ranges > 1) {
        const uint32_t n = rows * out_tokens;
        hipLaunchKernelGGL(verify_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, s, scratch->work, ranges, rows,
                           out_tokens, y_out, out_stride_out);
        *err = hipGetLastError();
    }
    return true;
}

template <uint32_t ENC, int RG>
static hipError_t launch_verify_rg(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t nblocks,
                                   uint32_t waves, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                                   uint64_t out_stride, uint32_t tokens) {
    dim3 grid((rows + 16 * RG - 1) / (16 * RG)), block(64 * waves);
    if constexpr (ENC == 12 || ENC == 13) {
        if (x_f16)
            hipLaunchKernelGGL((verify_split_kernel<ENC, _Float16, RG>), grid, block, 0, s, w, stride, rows, nblocks,
                               (const _Float16 *)x, in_stride, y, out_stride, tokens);
        else
            hipLaunchKernelGGL((verify_split_kernel<ENC, float, RG>), grid, block, 0, s, w, stride, rows, nblocks,
                               (const float *)x, in_stride, y, out_stride, tokens);
    } else {
        if (x_f16)
            hipLaunchKernelGGL((verify_kernel<ENC, _Float16, RG>), grid, block, 0, s, w, stride, rows, nblocks,
                               (const _Float16 *)x, in_stride, y, out_stride, tokens);
        else
            hipLaunchKernelGGL((verify_kernel<ENC, float, RG>), grid, block, 0, s, w, stride, rows, nblocks,
                               (const float *)x, in_stride, y, out_stride, tokens);
    }
    return hipGetLastError();
}

template <uint32_t ENC>
static hipError_t launch_verify_enc(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows,
                                    uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                                    uint64_t out_stride, uint32_t tokens, const SplitScratch &scratch) {
    const uint32_t nblocks = columns / 256;
    if constexpr (ENC == 12 || ENC == 13) {
        hipError_t err;
        if (launch_verify_dma<ENC>(s, w, stride, rows, nblocks, x, x_f16, in_stride, y, out_stride, tokens, &err,
                                   &scratch))
            return err;
    }
    // About five blocks per wave (at most VF_MAX_WAVES waves), split evenly:
    // measured best at K = 5120 (4 waves) and K = 17408 (14 waves).
    const uint32_t per_wave = std::max(5u, (nblocks + VF_MAX_WAVES - 1) / VF_MAX_WAVES);
    const uint32_t waves = (nblocks + per_wave - 1) / per_wave;
    // Two row groups per wave halve the x reads once there are enough rows
    // to keep 160 or more workgroups.
    if (rows >= 32u * 160)
        return launch_verify_rg<ENC, 2>(s, w, stride, rows, nblocks, waves, x, x_f16, in_stride, y, out_stride, tokens);
    return launch_verify_rg<ENC, 1>(s, w, stride, rows, nblocks, waves, x, x_f16, in_stride, y, out_stride, tokens);
}

template <uint32_t ENC>
static hipError_t launch_tile_enc(hipStream_t s, const uint8_t *w, uint64_t stride, uint32_t rows, uint32_t columns,
                                  const void *x, uint32_t x_f16, uint64_t in_stride, float *y, uint64_t out_stride,
                                  uint32_t tokens) {
    dim3 grid((rows + 127) / 128, (tokens + 127) / 128), block(256);
    if (x_f16)
        hipLaunchKernelGGL((tile_kernel<ENC, true>), grid, block, 0, s, w, stride, rows, columns, x, in_stride, y,
                           out_stride, tokens);
    else
        hipLaunchKernelGGL((tile_kernel<ENC, false>), grid, block, 0, s, w, stride, rows, columns, x, in_stride, y,
                           out_stride, tokens);
    return hipGetLastError();
}


hipError_t launch_rows_mfma(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                            uint32_t columns, const float *x, uint64_t in_stride, float *y, uint64_t out_stride,
                            uint32_t tokens, const SplitScratch &scratch, bool *taken) {
    *taken = false;
    if (tokens < 1 || tokens > 4 || columns % 256 != 0) return hipSuccess;
    hipError_t err = hipSuccess;
    bool launched = false;
    if (encoding == 12)
        launched = launch_verify_dma<12>(s, w, stride, rows, columns / 256, x, 0, in_stride, y, out_stride, tokens,
                                         &err, &scratch, true);
    else if (encoding == 13)
        launched = launch_verify_dma<13>(s, w, stride, rows, columns / 256, x, 0, in_stride, y, out_stride, tokens,
                                         &err, &scratch, true);
    *taken = launched;
    return launched ? err : hipSuccess;
}

uint32_t split_scratch_tiles() { return 4 * compute_units(); }

// Q4_K / Q5_K with up to VF_PASS_MAX tokens (K a multiple of 256) run on the
// streamed verify tile in passes of at most 16 tokens, each pass reading the
// weights once; more tokens, and the other encodings past 16 tokens, go to
// the prefill tile. 17408 x 5120 Q4_K: 17 / 24 / 32 / 48 tokens 0.033 /
// 0.034 / 0.047 / 0.070 ms in passes against 0.075-0.078 on the prefill
// tile (and 0.108-0.126 on the 128 x 128 tile); Q6_K 5120 x 17408, whose
// verify tile is the register form, 0.083 in passes at 17 tokens against
// 0.078.
constexpr uint32_t VF_PASS_MAX = 48;
static bool vf_passes(uint32_t encoding, uint32_t tokens, uint32_t columns) {
    return (encoding == 12 || encoding == 13) && tokens > 16 && tokens <= VF_PASS_MAX && columns % 256 == 0;
}
static uint32_t vf_pass_tokens(uint32_t tokens) {
    const uint32_t passes = (tokens + 15) / 16;
    return (tokens + passes - 1) / passes;
}

uint64_t tile_workspace_floats(uint32_t encoding, uint32_t rows, uint32_t columns, uint32_t tokens,
                               uint64_t in_stride, bool xs3) {
    if (vf_passes(encoding, tokens, columns)) tokens = vf_pass_tokens(tokens);
    if (tokens <= 16 && columns % 256 == 0) {
        // the streamed verify tile's K ranges (Q4_K / Q5_K rows longer than
        // 2 * MAXW blocks, or 20 for the F32 multi-token form), one F32
        // partial per range, token and row
        constexpr uint32_t MAXW = vd_max_waves<2>();
        const uint32_t nblocks = columns / 256, max_kb = vd_max_kb(xs3);
        if ((encoding != 12 && encoding != 13) || nblocks <= max_kb || rows < 16) return 0;
        return (uint64_t)((nblocks + max_kb - 1) / max_kb) * tokens * rows;
    }
    if (tokens > 16 && (uint64_t)PF_BM * in_stride * 2 + 256 <= 0xffffffffull) {  // as launch_tile routes
        const uint32_t cus = compute_units();
        const uint32_t tiles = ((tokens + PF_BM - 1) / PF_BM) * ((rows + PF_BN - 1) / PF_BN);
        uint32_t full, tail, splits;
        prefill_split_plan(tiles, columns, cus, split_scratch_tiles(), &full, &tail, &splits);
        return (uint64_t)tail * splits * PF_BM * PF_BN;
    }
    return 0;
}

hipError_t launch_tile(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                       uint64_t out_stride, uint32_t tokens, const SplitScratch &scratch) {
    if (vf_passes(encoding, tokens, columns)) {
        const uint32_t chunk = vf_pass_tokens(tokens);
        const size_t xe = x_f16 ? 2 : 4;
        for (uint32_t t0 = 0; t0 < tokens; t0 += chunk) {
            const hipError_t e = launch_tile(s, encoding, w, stride, rows, columns,
                                             (const uint8_t *)x + (uint64_t)t0 * in_stride * xe, x_f16, in_stride,
                                             y + (uint64_t)t0 * out_stride, out_stride, std::min(chunk, tokens - t0),
                                             scratch);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (tokens <= 16 && columns % 256 == 0) {
        switch (encoding) {
        case 12: return launch_verify_enc<12>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch);
        case 13: return launch_verify_enc<13>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch);
        case 14: return launch_verify_enc<14>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch);
        case 23: return launch_verify_enc<23>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch);
        default: return launch_verify_enc<8>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch);
        }
    }
    // (the prefill tile's activation copies use 32-bit offsets within a tile)
    if (tokens > 16 && (uint64_t)PF_BM * in_stride * 2 + 256 <= 0xffffffffull) {
        const uint32_t cus = compute_units();
        switch (encoding) {
        case 12: return launch_prefill<12>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch, cus);
        case 13: return launch_prefill<13>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch, cus);
        case 14: return launch_prefill<14>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch, cus);
        case 23: return launch_prefill<23>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch, cus);
        default: return launch_prefill<8>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens, scratch, cus);
        }
    }
    switch (encoding) {
    case 12: return launch_tile_enc<12>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    case 13: return launch_tile_enc<13>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    case 14: return launch_tile_enc<14>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    case 23: return launch_tile_enc<23>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    default: return launch_tile_enc<8>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    }
}

}  // namespace nuq

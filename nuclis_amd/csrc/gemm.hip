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

hipError_t launch_tile(hipStream_t s, uint32_t encoding, const uint8_t *w, uint64_t stride, uint32_t rows,
                       uint32_t columns, const void *x, uint32_t x_f16, uint64_t in_stride, float *y,
                       uint64_t out_stride, uint32_t tokens) {
    switch (encoding) {
    case 12: return launch_tile_enc<12>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    case 14: return launch_tile_enc<14>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    default: return launch_tile_enc<8>(s, w, stride, rows, columns, x, x_f16, in_stride, y, out_stride, tokens);
    }
}

}  // namespace nuq

// Host-side weight preparation: F32 rows -> GGUF Q8_0 / Q4_K / Q5_K / Q6_K /
// IQ4_XS rows.
//
// Q8_0 restates nuclis's only encoder, quant/encode.zig:17-36 (q8_0Row):
// d = f16(max|x| / 127) rounded to nearest even; q = clamp(round(x / d),
// -127, 127) rounding half away from zero; a zero or non-finite d stores zero
// codes and a NaN value codes as zero.
//
// nuclis has no K-quant or IQ quantizer (encode.zig:1-2); the ones below are
// this library's own, deterministic and simple (no error search). They write
// legal blocks in the layouts quant/decode.zig:147-170, :198-211 and :213-228
// read:
//   Q4_K: per 32-value group g, scale s_g = (max - min') / 15 and offset
//         o_g = -min' with min' = min(min, 0); d = f16(max s_g / 63),
//         dmin = f16(max o_g / 63); sc_g = round(s_g / d), m_g = round(o_g /
//         dmin) in 0..63; q = clamp(round((x + dmin*m_g) / (d*sc_g)), 0, 15).
//   Q5_K: as Q4_K with 32 levels (s_g = (max - min') / 31, q in 0..31); bit
//         4 of group g's code goes to bit g of high-plane byte c.
//   IQ4_XS: per 32-value group, s_g = max|x| / 127; d = f16(max s_g / 31);
//         scale_g = round(s_g / d) in 0..31 (stored +32 as six bits); each
//         value takes the nearest of the 16 nonlinear code values times
//         d*scale_g.
//   Q6_K: per 16-value group, s_g = max|x| / 31; d = f16(max s_g / 127);
//         sc_g = round(s_g / d) in 0..127; q = clamp(round(x / (d*sc_g)),
//         -32, 31) + 32 split into a low nibble (ql) and two high bits (qh).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/nuq.h"

namespace {

uint16_t f32_to_f16(float value) {
    uint32_t u;
    std::memcpy(&u, &value, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        float magnitude;
        std::memcpy(&magnitude, &a, 4);
        return (uint16_t)(sign | (uint16_t)std::nearbyint(magnitude * 16777216.0f));
    }
    uint32_t rounded = a + 0xfffu + ((a >> 13) & 1u);
    return (uint16_t)(sign | (uint16_t)((rounded - 0x38000000u) >> 13));
}

float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 31u, mantissa = h & 0x3ffu;
    uint32_t out;
    if (exponent == 0) {
        float m = std::ldexp((float)mantissa, -24);
        std::memcpy(&out, &m, 4);
        out |= sign;
    } else if (exponent == 31) {
        out = sign | 0x7f800000u | (mantissa << 13);
    } else {
        out = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float v;
    std::memcpy(&v, &out, 4);
    return v;
}

void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}

void q8_0_row(const float *x, uint64_t n, uint8_t *out) {
    for (uint64_t b = 0; b < n / 32; ++b) {
        const float *v = x + b * 32;
        uint8_t *blk = out + b * 34;
        float amax = 0.f;
        for (int j = 0; j < 32; ++j)
            if (!std::isnan(v[j])) amax = std::fmax(amax, std::fabs(v[j]));
        uint16_t dbits = f32_to_f16(amax / 127.0f);
        put16(blk, dbits);
        float scale = f16_to_f32(dbits);
        for (int j = 0; j < 32; ++j) {
            float q = 0.f;
            if (scale != 0.f && std::isfinite(scale) && !std::isnan(v[j])) {
                q = std::round(v[j] / scale);
                q = q < -127.f ? -127.f : (q > 127.f ? 127.f : q);
            }
            blk[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}

int clampi(long v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : (int)v); }

// Q4_K (levels 15, codes at 16) and Q5_K (levels 31, high plane at 16,
// codes at 48) share the affine group scheme.
void k_row(bool fifth_bit, const float *x, uint64_t n, uint8_t *out) {
    const uint64_t bb = fifth_bit ? 176 : 144;
    const float levels = fifth_bit ? 31.f : 15.f;
    for (uint64_t b = 0; b < n / 256; ++b) {
        const float *v = x + b * 256;
        uint8_t *blk = out + b * bb;
        float scale[8], offset[8];
        float max_scale = 0.f, max_offset = 0.f;
        for (int g = 0; g < 8; ++g) {
            float lo = 0.f, hi = -INFINITY;
            for (int c = 0; c < 32; ++c) {
                float t = v[g * 32 + c];
                lo = std::fmin(lo, t);
                hi = std::fmax(hi, t);
            }
            scale[g] = (hi - lo) / levels;
            offset[g] = -lo;
            max_scale = std::fmax(max_scale, scale[g]);
            max_offset = std::fmax(max_offset, offset[g]);
        }
        uint16_t dbits = f32_to_f16(max_scale / 63.f), mbits = f32_to_f16(max_offset / 63.f);
        float d = f16_to_f32(dbits), dmin = f16_to_f32(mbits);
        uint8_t sc[8], mn[8];
        for (int g = 0; g < 8; ++g) {
            sc[g] = (uint8_t)(d > 0.f ? clampi(std::lround(scale[g] / d), 0, 63) : 0);
            mn[g] = (uint8_t)(dmin > 0.f ? clampi(std::lround(offset[g] / dmin), 0, 63) : 0);
        }
        put16(blk, dbits);
        put16(blk + 2, mbits);
        uint8_t *s = blk + 4;
        // inverse of decode.zig:155-158
        for (int g = 0; g < 4; ++g) {
            s[g] = (uint8_t)((sc[g] & 63) | ((sc[g + 4] >> 4) << 6));
            s[g + 4] = (uint8_t)((mn[g] & 63) | ((mn[g + 4] >> 4) << 6));
            s[g + 8] = (uint8_t)((sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4));
        }
        uint8_t *qh = blk + 16, *qs = blk + (fifth_bit ? 48 : 16);
        std::memset(blk + 16, 0, bb - 16);
        for (int g = 0; g < 8; ++g) {
            float mul = d * (float)sc[g], off = dmin * (float)mn[g];
            for (int c = 0; c < 32; ++c) {
                int q = mul > 0.f ? clampi(std::lround((v[g * 32 + c] + off) / mul), 0, (int)levels) : 0;
                qs[g / 2 * 32 + c] |= (uint8_t)(g % 2 == 0 ? (q & 15) : ((q & 15) << 4));
                if (fifth_bit) qh[c] |= (uint8_t)(((q >> 4) & 1) << g);
            }
        }
    }
}

const int kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

void iq4_xs_row(const float *x, uint64_t n, uint8_t *out) {
    for (uint64_t b = 0; b < n / 256; ++b) {
        const float *v = x + b * 256;
        uint8_t *blk = out + b * 136;
        float scale[8], max_scale = 0.f;
        for (int g = 0; g < 8; ++g) {
            float amax = 0.f;
            for (int c = 0; c < 32; ++c) amax = std::fmax(amax, std::fabs(v[g * 32 + c]));
            scale[g] = amax / 127.f;
            max_scale = std::fmax(max_scale, scale[g]);
        }
        uint16_t dbits = f32_to_f16(max_scale / 31.f);
        float d = f16_to_f32(dbits);
        std::memset(blk, 0, 136);
        put16(blk, dbits);
        uint16_t high = 0;
        for (int g = 0; g < 8; ++g) {
            const int si = d > 0.f ? clampi(std::lround(scale[g] / d), 0, 31) : 0;
            const unsigned stored = (unsigned)(si + 32);
            blk[4 + g / 2] |= (uint8_t)((stored & 15) << (4 * (g % 2)));
            high |= (uint16_t)(((stored >> 4) & 3) << (2 * g));
            const float mul = d * (float)si;
            for (int j = 0; j < 32; ++j) {
                int best = 0;
                float err = INFINITY;
                for (int c = 0; c < 16; ++c) {
                    const float e = std::fabs(v[g * 32 + j] - mul * (float)kIq4Values[c]);
                    if (e < err) {
                        err = e;
                        best = c;
                    }
                }
                uint8_t &byte = blk[8 + g * 16 + (j & 15)];
                byte |= (uint8_t)(j < 16 ? best : (best << 4));
            }
        }
        put16(blk + 2, high);
    }
}

void q6_k_row(const float *x, uint64_t n, uint8_t *out) {
    for (uint64_t b = 0; b < n / 256; ++b) {
        const float *v = x + b * 256;
        uint8_t *blk = out + b * 210;
        float scale[16], max_scale = 0.f;
        for (int g = 0; g < 16; ++g) {
            float amax = 0.f;
            for (int c = 0; c < 16; ++c) amax = std::fmax(amax, std::fabs(v[g * 16 + c]));
            scale[g] = amax / 31.f;
            max_scale = std::fmax(max_scale, scale[g]);
        }
        uint16_t dbits = f32_to_f16(max_scale / 127.f);
        float d = f16_to_f32(dbits);
        int8_t sc[16];
        for (int g = 0; g < 16; ++g) sc[g] = (int8_t)(d > 0.f ? clampi(std::lround(scale[g] / d), 0, 127) : 0);
        std::memset(blk, 0, 192);
        for (int i = 0; i < 256; ++i) {
            float mul = d * (float)sc[i / 16];
            int q = mul > 0.f ? clampi(std::lround(v[i] / mul), -32, 31) : 0;
            int u = q + 32;
            int quarter = (i % 128) / 32, column = i % 32;
            blk[(i / 128) * 64 + (quarter % 2) * 32 + column] |= (uint8_t)((u & 15) << ((quarter / 2) * 4));
            blk[128 + (i / 128) * 32 + column] |= (uint8_t)(((u >> 4) & 3) << (quarter * 2));
        }
        for (int g = 0; g < 16; ++g) blk[192 + g] = (uint8_t)sc[g];
        put16(blk + 208, dbits);
    }
}

}  // namespace

extern "C" int nuq_quantize_rows(uint32_t encoding, const float *src, uint64_t rows, uint64_t columns, void *dst,
                                 uint64_t dst_len) {
    uint64_t elements, bytes;
    switch (encoding) {
    case NUQ_Q8_0: elements = 32; bytes = 34; break;
    case NUQ_Q4_K: elements = 256; bytes = 144; break;
    case NUQ_Q5_K: elements = 256; bytes = 176; break;
    case NUQ_Q6_K: elements = 256; bytes = 210; break;
    case NUQ_IQ4_XS: elements = 256; bytes = 136; break;
    default: return NUQ_UNSUPPORTED_ENCODING;
    }
    if (!src || !dst) return NUQ_INVALID_ARGUMENT;
    if (rows == 0 || columns == 0 || columns % elements != 0) return NUQ_INVALID_ROW_LENGTH;
    const uint64_t row_bytes = columns / elements * bytes;
    if (dst_len / rows != row_bytes || dst_len % rows != 0) return NUQ_INVALID_BYTE_LENGTH;
    unsigned hw = std::thread::hardware_concurrency();
    unsigned threads = hw == 0 ? 1 : (hw > 32 ? 32 : hw);
    if (rows * columns < (1u << 20)) threads = 1;
    auto work = [&](unsigned t) {
        for (uint64_t r = t; r < rows; r += threads) {
            const float *x = src + r * columns;
            uint8_t *o = (uint8_t *)dst + r * row_bytes;
            switch (encoding) {
            case NUQ_Q8_0: q8_0_row(x, columns, o); break;
            case NUQ_Q4_K: k_row(false, x, columns, o); break;
            case NUQ_Q5_K: k_row(true, x, columns, o); break;
            case NUQ_IQ4_XS: iq4_xs_row(x, columns, o); break;
            default: q6_k_row(x, columns, o); break;
            }
        }
    };
    if (threads == 1) {
        work(0);
    } else {
        std::vector<std::thread> pool;
        for (unsigned t = 0; t < threads; ++t) pool.emplace_back(work, t);
        for (auto &th : pool) th.join();
    }
    return NUQ_OK;
}

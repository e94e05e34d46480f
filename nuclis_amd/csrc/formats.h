// GGUF block formats on gfx950: geometry, exact scalar decoders and the
// vectorised per-lane decoders the product kernels use.
//
// Block layouts are facts of the GGML storage formats, as nuclis decodes them:
//   Q8_0 (id 8):  [d:f16][q:i8 x32]                          34 B / 32 values
//                 quant/decode.zig:57-63
//   Q4_K (id 12): [d:f16][dmin:f16][scales:12 B][qs:128 B]     144 B / 256 values
//                 quant/decode.zig:147-170 (kBlock, fifth_bit false)
//   Q5_K (id 13): [d:f16][dmin:f16][scales:12 B][qh:32 B][qs:128 B] 176 B / 256
//                 quant/decode.zig:147-170 (kBlock, fifth_bit true)
//   Q6_K (id 14): [ql:128 B][qh:64 B][sc:i8 x16][d:f16]        210 B / 256 values
//                 quant/decode.zig:198-211 (q6Block)
//   IQ4_XS (id 23): [d:f16][scales_h:u16][scales_l:4 B][qs:128 B] 136 B / 256
//                 quant/decode.zig:213-228 (iq4XsBlock), values :437
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nuq {

struct Layout {
    uint32_t elements;
    uint32_t bytes;
};

// inference/src/tensor/encoding.zig:29-41
__host__ __device__ inline bool layout_of(uint32_t encoding, Layout *l) {
    switch (encoding) {
    case 8: *l = {32, 34}; return true;
    case 12: *l = {256, 144}; return true;
    case 13: *l = {256, 176}; return true;
    case 14: *l = {256, 210}; return true;
    case 23: *l = {256, 136}; return true;
    default: return false;
    }
}

// Exact F16 -> F32 widening from the bits (subnormals, infinities and NaN
// payloads preserved), independent of the hardware denormal mode.
__device__ __forceinline__ float half_bits_exact(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 31u;
    uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0) {
        // mantissa * 2^-24 is exact in F32
        return __uint_as_float(sign | __float_as_uint((float)mantissa * 5.9604644775390625e-8f));
    }
    if (exponent == 31) return __uint_as_float(sign | 0x7f800000u | (mantissa << 13));
    return __uint_as_float(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

// Hardware widening (v_cvt_f32_f16); exact for every input while F16
// denormals are enabled, which is the HIP default on gfx950.
__device__ __forceinline__ float half_bits(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}

// Q4_K six-bit scale and minimum of group g (0..7) from the 12 scale bytes
// held little-endian in s0 (bytes 0-3), s1 (4-7), s2 (8-11).
// quant/decode.zig:155-158.
__device__ __forceinline__ void q4k_scale_min(uint32_t g, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t *scale,
                                              uint32_t *minimum) {
    if (g < 4) {
        *scale = (s0 >> (8 * g)) & 63u;
        *minimum = (s1 >> (8 * g)) & 63u;
    } else {
        uint32_t k = g - 4;
        uint32_t b8 = (s2 >> (8 * k)) & 0xffu;     // scales[g + 4]
        uint32_t lo = (s0 >> (8 * k)) & 0xffu;     // scales[g - 4]
        uint32_t hi = (s1 >> (8 * k)) & 0xffu;     // scales[g]
        *scale = (b8 & 15u) | ((lo >> 6) << 4);
        *minimum = (b8 >> 4) | ((hi >> 6) << 4);
    }
}

__device__ __forceinline__ uint32_t load_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t load_u16_bytes(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Exact scalar decoders: value i of a block, in the CPU decoder's operation
// order, each F32 multiply and subtract rounded separately (no contraction).
#pragma clang fp contract(off)
__device__ __forceinline__ float decode_q8_0(const uint8_t *block, uint32_t i) {
    float d = half_bits_exact(load_u16_bytes(block));
    return d * (float)(int8_t)block[2 + i];
}

__device__ __forceinline__ float decode_q4_k(const uint8_t *block, uint32_t i) {
    float d = half_bits_exact(load_u16_bytes(block));
    float dmin = half_bits_exact(load_u16_bytes(block + 2));
    const uint8_t *s = block + 4;
    uint32_t g = i / 32, c = i % 32;
    uint32_t scale, minimum;
    if (g < 4) {
        scale = s[g] & 63u;
        minimum = s[g + 4] & 63u;
    } else {
        scale = (s[g + 4] & 15u) | ((uint32_t)(s[g - 4] >> 6) << 4);
        minimum = (uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4);
    }
    float multiplier = d * (float)scale;
    float offset = dmin * (float)minimum;
    uint32_t byte = block[16 + g / 2 * 32 + c];
    uint32_t q = (g % 2 == 0) ? (byte & 15u) : (byte >> 4);
    float scaled = multiplier * (float)q;
    return scaled - offset;
}

__device__ __forceinline__ float decode_q5_k(const uint8_t *block, uint32_t i) {
    float d = half_bits_exact(load_u16_bytes(block));
    float dmin = half_bits_exact(load_u16_bytes(block + 2));
    const uint8_t *s = block + 4;
    uint32_t g = i / 32, c = i % 32;
    uint32_t scale, minimum;
    if (g < 4) {
        scale = s[g] & 63u;
        minimum = s[g + 4] & 63u;
    } else {
        scale = (s[g + 4] & 15u) | ((uint32_t)(s[g - 4] >> 6) << 4);
        minimum = (uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4);
    }
    float multiplier = d * (float)scale;
    float offset = dmin * (float)minimum;
    uint32_t byte = block[48 + g / 2 * 32 + c];
    uint32_t q = (g % 2 == 0) ? (byte & 15u) : (byte >> 4);
    q |= ((uint32_t)(block[16 + c] >> g) & 1u) << 4;  // bit g of high-plane byte c
    float scaled = multiplier * (float)q;
    return scaled - offset;
}

// quant/decode.zig:437
__constant__ static const int8_t kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                                   1,    13,   25,  38,  53,  69,  89,  113};

__device__ __forceinline__ float decode_iq4_xs(const uint8_t *block, uint32_t i) {
    float d = half_bits_exact(load_u16_bytes(block));
    uint32_t high = load_u16_bytes(block + 2);
    uint32_t g = i / 32, j = i % 32;
    uint32_t low = (block[4 + g / 2] >> (4 * (g % 2))) & 15u;
    int scale = (int)(low | (((high >> (2 * g)) & 3u) << 4)) - 32;
    float multiplier = d * (float)scale;
    uint32_t byte = block[8 + g * 16 + (j & 15)];
    uint32_t code = j < 16 ? (byte & 15u) : (byte >> 4);
    return multiplier * (float)kIq4Values[code];
}

__device__ __forceinline__ float decode_q6_k(const uint8_t *block, uint32_t i) {
    float d = half_bits_exact(load_u16_bytes(block + 208));
    uint32_t quarter = (i % 128) / 32;
    uint32_t column = i % 32;
    uint32_t low = (block[(i / 128) * 64 + (quarter % 2) * 32 + column] >> ((quarter / 2) * 4)) & 15u;
    uint32_t high = (block[128 + (i / 128) * 32 + column] >> (quarter * 2)) & 3u;
    int value = (int)(low | (high << 4)) - 32;
    float multiplier = d * (float)(int8_t)block[192 + i / 16];
    return multiplier * (float)value;
}
#pragma clang fp contract(on)

__device__ __forceinline__ float decode_value(uint32_t encoding, const uint8_t *block, uint32_t i) {
    switch (encoding) {
    case 8: return decode_q8_0(block, i);
    case 12: return decode_q4_k(block, i);
    case 13: return decode_q5_k(block, i);
    case 23: return decode_iq4_xs(block, i);
    default: return decode_q6_k(block, i);
    }
}

// IQ4_XS / IQ4_NL code lookup for four codes at once: byte e of `codes`
// (0..15) -> byte e of the result = kIq4Values[code] as a signed byte. Two
// v_perm_b32 pick from table entries 0-7 and 8-15 (selectors 0-7 address the
// eight bytes of a dword pair, low dword first); a third picks byte e of
// the second when bit 3 of code e is set (selector e + 4), else of the first
// (selector e).
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t codes) {
    // entries 0-3, 4-7, 8-11, 12-15 of kIq4Values as little-endian bytes
    constexpr uint32_t T0 = 0xbfad9881u, T1 = 0xf6eaddcfu, T2 = 0x26190d01u, T3 = 0x71594535u;
    const uint32_t sel = codes & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    const uint32_t pick = ((codes >> 1) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(hi, lo, pick);
}

// Byte E of a dword as a signed value in F32.
template <int E>
__device__ __forceinline__ float sbyte_f(uint32_t w) { return (float)(int8_t)((w >> (8 * E)) & 0xffu); }

// Byte E of a dword as F32; the backend selects v_cvt_f32_ubyteE.
template <int E>
__device__ __forceinline__ float ubyte_f(uint32_t w) { return (float)((w >> (8 * E)) & 0xffu); }

// a & M through an instruction the compiler cannot see into, so the
// following byte extractions select v_cvt_f32_ubyteN on the masked word
// instead of re-deriving each nibble with v_bfe_u32.
template <uint32_t M>
__device__ __forceinline__ uint32_t opaque_and(uint32_t a) {
    uint32_t r;
    asm("v_and_b32_e32 %0, %2, %1" : "=v"(r) : "v"(a), "n"(M));
    return r;
}

// Unaligned 32-bit load. gfx9 global memory runs in unaligned access mode
// under ROCm, so a dword load at a 2-byte aligned address returns the four
// bytes at that address.
__device__ __forceinline__ uint32_t load_u32_unaligned(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}

}  // namespace nuq

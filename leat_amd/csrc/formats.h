// Every GGUF block format the dequantizer decodes (leat/quant.py:94-231): block geometry, and the
// f32 weights of one piece of 32 weights in ggml's float operation order (each product and sum
// rounded on its own: no fused multiply-add), so decoded weights equal ggml's and gguf-py's bit
// for bit. A piece is a block of the 32-weight types; for the 256-weight types, weights
// 32p..32p+31 of the block.
//
//   Q4_0   18 B: f16 d, 16 B of nibbles (value i < 16 the low nibble of byte i, i + 16 the high)
//                w = d * (q - 8)
//   Q4_1   20 B: f16 d, f16 m, nibbles                              w = d * q + m
//   Q5_0   22 B: f16 d, 4 B of fifth bits (bit i of value i), nibbles w = d * (q - 16)
//   Q5_1   24 B: f16 d, f16 m, fifth bits, nibbles                  w = d * q + m
//   Q8_0   34 B: f16 d, int8 q[32]                                  w = d * q
//   IQ4_NL 18 B: f16 d, nibbles indexing IQ4 values                 w = d * v[q]
//   MXFP4  17 B: exponent byte e, nibbles indexing doubled E2M1     w = 2^(e - 128) * v[q]
//   Q2_K   84 B: scales u8[16], 2-bit q[64 B], f16 d, f16 dmin; per 16 weights
//                w = (d * (s & 15)) * q - (dmin * (s >> 4))
//   Q3_K  110 B: hmask u8[32], 2-bit q[64 B], 6-bit scales in 12 B, f16 d; per 16 weights
//                w = (d * (s - 32)) * (q - 4 * !hbit)
//   Q4_K  144 B: f16 d, f16 dmin, 6-bit scales and mins in 12 B, nibbles[128]
//                w = (d * sc) * q - (dmin * m)
//   Q5_K  176 B: as Q4_K with qh[32] before the nibbles, bit s of qh[l] the fifth bit of value l
//                of sub-block s
//   Q6_K  210 B: ql[128], qh[64], int8 scales[16], f16 d; w = (d * sc) * (q - 32)
//   IQ4_XS 136 B: f16 d, 16 high scale bits, 4 B of low scale nibbles, nibbles[128];
//                w = (d * (s - 32)) * v[q] per sub-block of 32
#pragma once

#include "common.h"

namespace leat {

template <int TYPE> struct Format;
template <> struct Format<Q4_0> { static constexpr int BYTES = 18, WEIGHTS = 32; };
template <> struct Format<Q4_1> { static constexpr int BYTES = 20, WEIGHTS = 32; };
template <> struct Format<Q5_0> { static constexpr int BYTES = 22, WEIGHTS = 32; };
template <> struct Format<Q5_1> { static constexpr int BYTES = 24, WEIGHTS = 32; };
template <> struct Format<Q8_0> { static constexpr int BYTES = 34, WEIGHTS = 32; };
template <> struct Format<IQ4_NL> { static constexpr int BYTES = 18, WEIGHTS = 32; };
template <> struct Format<MXFP4> { static constexpr int BYTES = 17, WEIGHTS = 32; };
template <> struct Format<Q2_K> { static constexpr int BYTES = 84, WEIGHTS = 256; };
template <> struct Format<Q3_K> { static constexpr int BYTES = 110, WEIGHTS = 256; };
template <> struct Format<Q4_K> { static constexpr int BYTES = 144, WEIGHTS = 256; };
template <> struct Format<Q5_K> { static constexpr int BYTES = 176, WEIGHTS = 256; };
template <> struct Format<Q6_K> { static constexpr int BYTES = 210, WEIGHTS = 256; };
template <> struct Format<IQ4_XS> { static constexpr int BYTES = 136, WEIGHTS = 256; };

// the 16 values IQ4_NL's and IQ4_XS's nibbles index, and MXFP4's E2M1 values doubled
__device__ __forceinline__ int iq4_value(int q) {
    constexpr int8_t v[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    return v[q];
}
__device__ __forceinline__ int fp4_value(int q) {
    constexpr int8_t v[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    return v[q];
}

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8)));
}

// 2^(e - 128) of an exponent byte: the f32 bits (e - 1) << 23, or the denormal 0x00200000 << e
// below e = 2 (ggml's e8m0_to_fp32_half)
__device__ __forceinline__ float e8m0_half(uint32_t e) {
    return __builtin_bit_cast(float, e < 2 ? 0x00200000u << e : (e - 1) << 23);
}

// get_scale_min_k4 (leat/quant.py:182-187): the 6-bit scale and min of sub-block s of 8
__device__ __forceinline__ void scale_min_k4(const uint8_t* q, int s, int* sc, int* m) {
    if (s < 4) {
        *sc = q[s] & 63;
        *m = q[s + 4] & 63;
    } else {
        *sc = (q[s + 4] & 0xF) | ((q[s - 4] >> 6) << 4);
        *m = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
    }
}

// nibble l (0..31) of a 32-weight run of 16 bytes: low nibbles first, then high ones
__device__ __forceinline__ int nibble(const uint8_t* qs, int l) { return l < 16 ? qs[l] & 0xF : qs[l - 16] >> 4; }

template <int TYPE>
__device__ void dequant_piece(const uint8_t* __restrict__ blk, int p, float y[32]) {
#pragma clang fp contract(off)
    if constexpr (TYPE == Q4_0 || TYPE == Q5_0 || TYPE == IQ4_NL) {
        const float d = f16_at(blk);
        const uint8_t* qs = blk + (TYPE == Q5_0 ? 6 : 2);
#pragma unroll
        for (int l = 0; l < 32; l++) {
            int q = nibble(qs, l);
            if (TYPE == Q4_0) q -= 8;
            if (TYPE == Q5_0) q = (q | (((blk[2 + l / 8] >> (l % 8)) & 1) << 4)) - 16;
            if (TYPE == IQ4_NL) q = iq4_value(q);
            y[l] = d * (float)q;
        }
    } else if constexpr (TYPE == Q4_1 || TYPE == Q5_1) {
        const float d = f16_at(blk), m = f16_at(blk + 2);
        const uint8_t* qs = blk + (TYPE == Q5_1 ? 8 : 4);
#pragma unroll
        for (int l = 0; l < 32; l++) {
            int q = nibble(qs, l);
            if (TYPE == Q5_1) q |= ((blk[4 + l / 8] >> (l % 8)) & 1) << 4;
            y[l] = d * (float)q + m;
        }
    } else if constexpr (TYPE == Q8_0) {
        const float d = f16_at(blk);
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = d * (float)(int8_t)blk[2 + l];
    } else if constexpr (TYPE == MXFP4) {
        const float d = e8m0_half(blk[0]);
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = d * (float)fp4_value(nibble(blk + 1, l));
    } else if constexpr (TYPE == Q2_K) {
        const float d = f16_at(blk + 80), dmin = f16_at(blk + 82);
        const int half = p >> 2, k = p & 3;  // bits 2k of qs[32 half + l]
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const int s = blk[2 * p + l / 16];
            const float dl = d * (float)(s & 15), ml = dmin * (float)(s >> 4);
            y[l] = dl * (float)((blk[16 + 32 * half + l] >> (2 * k)) & 3) - ml;
        }
    } else if constexpr (TYPE == Q3_K) {
        const float d = f16_at(blk + 108);
        const int half = p >> 2, k = p & 3;
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const int j = 2 * p + l / 16;  // the value's scale: low 4 bits from the nibbles, top 2 from byte 8 + j % 4
            const int low = j < 8 ? blk[96 + j] & 15 : blk[96 + j - 8] >> 4;
            const int high = (blk[104 + j % 4] >> (2 * (j / 4))) & 3;
            const float dl = d * (float)((low | (high << 4)) - 32);
            const int q = ((blk[32 + 32 * half + l] >> (2 * k)) & 3) - (((blk[l] >> p) & 1) ? 0 : 4);
            y[l] = dl * (float)q;
        }
    } else if constexpr (TYPE == Q4_K || TYPE == Q5_K) {
        const float d = f16_at(blk), dmin = f16_at(blk + 2);
        int sc, m;
        scale_min_k4(blk + 4, p, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t* qs = blk + (TYPE == Q5_K ? 48 : 16) + 32 * (p >> 1);
        const int shift = 4 * (p & 1);
#pragma unroll
        for (int l = 0; l < 32; l++) {
            int q = (qs[l] >> shift) & 0xF;
            if (TYPE == Q5_K) q |= ((blk[16 + l] >> p) & 1) << 4;
            y[l] = d1 * (float)q - m1;
        }
    } else if constexpr (TYPE == Q6_K) {
        const float d = f16_at(blk + 208);
        const int n = p >> 2, k = p & 3;
        const uint8_t* ql = blk + 64 * n + 32 * (k & 1);
        const uint8_t* qh = blk + 128 + 32 * n;
        const int8_t* sc = (const int8_t*)(blk + 192 + 8 * n + 2 * k);
        const int lshift = 4 * (k >> 1), hshift = 2 * k;
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const int q = (((ql[l] >> lshift) & 0xF) | (((qh[l] >> hshift) & 3) << 4)) - 32;
            y[l] = d * (float)sc[l >> 4] * (float)q;
        }
    } else if constexpr (TYPE == IQ4_XS) {
        const float d = f16_at(blk);
        const int low = (blk[4 + p / 2] >> (4 * (p & 1))) & 0xF;
        const int high = ((blk[2] | (blk[3] << 8)) >> (2 * p)) & 3;
        const float dl = d * (float)((low | (high << 4)) - 32);
        const uint8_t* qs = blk + 8 + 16 * p;
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = dl * (float)iq4_value(nibble(qs, l));
    }
}

// X(TYPE) for every type above: `switch (type) { LEAT_FORMATS(CASE) }` dispatches on a run-time id
#define LEAT_FORMATS(X) X(Q4_0) X(Q4_1) X(Q5_0) X(Q5_1) X(Q8_0) X(Q2_K) X(Q3_K) X(Q4_K) X(Q5_K) X(Q6_K) X(IQ4_NL) X(IQ4_XS) X(MXFP4)

}  // namespace leat

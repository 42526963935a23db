// The v_dot4 decode tasks of the other storage types the decode kernels take (leat/kernels/
// matvec.py:184-303), in the shape of blocks.h's: a task's weights become int8 words for two
// scale spans, whose int32 dot products with the q8 activations are combined in f32.
//
//   32-weight blocks (Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL, MXFP4): a task is two blocks, each one
//     activation group (spans 2 task and 2 task + 1, 8 words each). A pair starts at an even byte
//     (every pair of blocks is an even number of bytes), so it is read as 16-bit halfwords;
//     a block's 16 bytes of nibbles give words 0..3 (low nibbles, values 0..15) and 4..7 (high
//     nibbles, values 16..31).
//       Q4_0   q - 8                         u = d xd dot
//       Q4_1   q (0..15)                     u = d xd dot + m xs
//       Q5_0   (q | fifth bit << 4) - 16     u = d xd dot
//       Q5_1   q | fifth bit << 4            u = d xd dot + m xs
//       IQ4_NL IQ4 values[q]                 u = d xd dot
//       MXFP4  doubled E2M1 values[q]        u = 2^(e - 128) xd dot
//   Q5_K: Q4_K's tasks (half h of sub-blocks 2j and 2j + 1) with the fifth bits, bit s of qh[l]
//     for value l of sub-block s: qh bytes [16h, +16) of the task's values.
//   IQ4_XS: a task is sub-block s of a block (32 weights, one activation group): span 0 its
//     values 0..15 (low nibbles of its 16 bytes), span 1 values 16..31 (high nibbles), words 0..3
//     and 4..7 of the group; u = d (sc - 32) xd (dot0 + dot1).
#pragma once

#include "formats.h"

namespace leat {

// 4 nibble-valued bytes (0..15 each) replaced by entries of a 16-byte table held as 4 words:
// v_perm_b32 picks entries 0..7 and 8..15 by the low 3 bits, the top bit chooses between them
__device__ __forceinline__ uint32_t lookup16(uint32_t q, const uint32_t (&t)[4]) {
    const uint32_t sel = q & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], sel);
    const uint32_t top = ((q >> 3) & 0x01010101u) * 0xFFu;
    return (hi & top) | (lo & ~top);
}

// the table words of IQ4_NL's values and of MXFP4's doubled E2M1 values (int8, little-endian)
template <int TYPE>
__device__ __forceinline__ void table_words(uint32_t (&t)[4]) {
    if (TYPE == MXFP4) {
        t[0] = 0x03020100u, t[1] = 0x0C080604u, t[2] = 0xFDFEFF00u, t[3] = 0xF4F8FAFCu;
    } else {  // -127 -104 -83 -65 | -49 -35 -22 -10 | 1 13 25 38 | 53 69 89 113
        t[0] = 0xBFAD9881u, t[1] = 0xF6EADDCFu, t[2] = 0x26190D01u, t[3] = 0x71594535u;
    }
}

// 4 bits (bits 0..3 of x) as bit 4 of each of 4 bytes
__device__ __forceinline__ uint32_t fifth_bits(uint32_t x) {
    return ((x & 1u) | ((x & 2u) << 7) | ((x & 4u) << 14) | ((x & 8u) << 21)) << 4;
}

template <int TYPE>
struct Task32 {
    static constexpr int BYTES = Format<TYPE>::BYTES, WEIGHTS = 32, TASK_W = 64, PER_BLOCK = 1, WORDS = 8;
    static constexpr bool NEEDS_S = TYPE == Q4_1 || TYPE == Q5_1;
    static constexpr int WORD_SKIP = 0;
    // the first byte of the nibbles within a block
    static constexpr int QS = TYPE == Q4_1 ? 4 : TYPE == Q5_0 ? 6 : TYPE == Q5_1 ? 8 : TYPE == MXFP4 ? 1 : 2;
    struct Raw {
        uint16_t h[BYTES];  // the pair's 2 * BYTES bytes
    };
    struct Dec {
        uint32_t w0[8], w1[8];
        float c0, c1, m0, m1;
    };
    __device__ static Raw load(const uint8_t* w, int64_t row, int cols, int task) {
        const int nb = cols / WEIGHTS;
        const uint16_t* p = (const uint16_t*)(w + ((int64_t)row * nb + 2 * task) * BYTES);
        Raw r;
#pragma unroll
        for (int i = 0; i < BYTES; i++) r.h[i] = p[i];
        return r;
    }
    // byte k of the pair (k known at compile time after unrolling)
    __device__ static uint32_t byte(const Raw& r, int k) { return (uint32_t)(r.h[k >> 1] >> (8 * (k & 1))) & 0xFFu; }
    __device__ static uint32_t word(const Raw& r, int k) {
        return byte(r, k) | (byte(r, k + 1) << 8) | (byte(r, k + 2) << 16) | (byte(r, k + 3) << 24);
    }
    __device__ static void block(const Raw& r, int b, uint32_t (&out)[8], float* c, float* m) {
        const int at = b * BYTES;
        uint32_t table[4];
        table_words<TYPE>(table);
        const uint32_t qh = TYPE == Q5_0 ? word(r, at + 2) : TYPE == Q5_1 ? word(r, at + 4) : 0u;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = word(r, at + QS + 4 * i);
            uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
            if (TYPE == Q5_0 || TYPE == Q5_1) {
                lo |= fifth_bits((qh >> (4 * i)) & 15u);
                hi |= fifth_bits((qh >> (16 + 4 * i)) & 15u);
            }
            if (TYPE == Q4_0) lo = minus_bytes(lo, 8), hi = minus_bytes(hi, 8);
            if (TYPE == Q5_0) lo = minus_bytes(lo, 16), hi = minus_bytes(hi, 16);
            if (TYPE == IQ4_NL || TYPE == MXFP4) lo = lookup16(lo, table), hi = lookup16(hi, table);
            out[i] = lo;
            out[4 + i] = hi;
        }
        if (TYPE == MXFP4) {
            *c = e8m0_half(byte(r, at));
        } else {
            *c = (float)__builtin_bit_cast(_Float16, (uint16_t)(byte(r, at) | (byte(r, at + 1) << 8)));
        }
        *m = NEEDS_S ? (float)__builtin_bit_cast(_Float16, (uint16_t)(byte(r, at + 2) | (byte(r, at + 3) << 8))) : 0.0f;
    }
    __device__ static Dec decode(const Raw& r, int task) {
        Dec d;
        block(r, 0, d.w0, &d.c0, &d.m0);
        block(r, 1, d.w1, &d.c1, &d.m1);
        return d;
    }
    __device__ static void act_at(int cols, int task, int* g0, int* g1, int* word) {
        *g0 = 2 * task;
        *g1 = 2 * task + 1;
        *word = 0;
    }
    __device__ static Dots dots(const Dec& d, const ActQ& x) {
        int a = 0, b = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            a = dot4(d.w0[i], x.x0[i], a);
            b = dot4(d.w1[i], x.x1[i], b);
        }
        return {a, b};
    }
    __device__ static float combine(const Dec& d, const ActQ& x, Dots s) {
        float u = d.c0 * x.d0 * (float)s.a + d.c1 * x.d1 * (float)s.b;
        if (NEEDS_S) u += d.m0 * x.s0 + d.m1 * x.s1;
        return u;
    }
};

template <> struct Task<Q4_0> : Task32<Q4_0> {};
template <> struct Task<Q4_1> : Task32<Q4_1> {};
template <> struct Task<Q5_0> : Task32<Q5_0> {};
template <> struct Task<Q5_1> : Task32<Q5_1> {};
template <> struct Task<IQ4_NL> : Task32<IQ4_NL> {};
template <> struct Task<MXFP4> : Task32<MXFP4> {};

template <>
struct Task<Q5_K> {
    static constexpr int BYTES = 176, WEIGHTS = 256, TASK_W = 32, PER_BLOCK = 8, WORDS = 4;
    static constexpr bool NEEDS_S = true;
    static constexpr int WORD_SKIP = 0;
    struct Raw {
        u32x4 hdr, qh, qs;
    };
    using Dec = Task<Q4_K>::Dec;
    __device__ static Raw load(const uint8_t* w, int64_t row, int cols, int task) {
        const int nb = cols / WEIGHTS, b = task >> 3, k = task & 7;
        const uint8_t* blk = w + ((int64_t)row * nb + b) * BYTES;
        Raw r;
        r.hdr = stream_load((const u32x4*)blk);
        r.qh = stream_load((const u32x4*)(blk + 16 + 16 * (k & 1)));
        r.qs = stream_load((const u32x4*)(blk + 48 + 16 * k));
        return r;
    }
    __device__ static Dec decode(const Raw& r, int task) {
        const int j = (task & 7) >> 1;
        Task<Q4_K>::Raw q4 = {r.hdr, r.qs};
        Dec d = Task<Q4_K>::decode(q4, task);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w0[i] |= ((r.qh[i] >> (2 * j)) & 0x01010101u) << 4;
            d.w1[i] |= ((r.qh[i] >> (2 * j + 1)) & 0x01010101u) << 4;
        }
        return d;
    }
    __device__ static void act_at(int cols, int task, int* g0, int* g1, int* word) {
        Task<Q4_K>::act_at(cols, task, g0, g1, word);
    }
    __device__ static Dots dots(const Dec& d, const ActQ& x) { return Task<Q4_K>::dots(d, x); }
    __device__ static float combine(const Dec& d, const ActQ& x, Dots s) { return Task<Q4_K>::combine(d, x, s); }
};

template <>
struct Task<IQ4_XS> {
    static constexpr int BYTES = 136, WEIGHTS = 256, TASK_W = 32, PER_BLOCK = 8, WORDS = 4;
    static constexpr bool NEEDS_S = false;
    static constexpr int WORD_SKIP = 4;  // span 1 is words 4..7 of the same group
    struct Raw {
        u32x2 hdr;
        u32x4 qs;
    };
    struct Dec {
        uint32_t w0[4], w1[4];
        float c;
    };
    __device__ static Raw load(const uint8_t* w, int64_t row, int cols, int task) {
        const int nb = cols / WEIGHTS, b = task >> 3, s = task & 7;
        const uint8_t* blk = w + ((int64_t)row * nb + b) * BYTES;
        Raw r;
        r.hdr = stream_load((const u32x2*)blk);
        r.qs = stream_load((const u32x4_a4*)(blk + 8 + 16 * s));
        return r;
    }
    __device__ static Dec decode(const Raw& r, int task) {
        const int s = task & 7;
        uint32_t table[4];
        table_words<IQ4_NL>(table);
        Dec d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w0[i] = lookup16(r.qs[i] & 0x0F0F0F0Fu, table);
            d.w1[i] = lookup16((r.qs[i] >> 4) & 0x0F0F0F0Fu, table);
        }
        const uint32_t low = (r.hdr[1] >> (4 * s)) & 15u, high = (r.hdr[0] >> (16 + 2 * s)) & 3u;
        d.c = f16_lo(r.hdr[0]) * (float)((int)(low | (high << 4)) - 32);
        return d;
    }
    __device__ static void act_at(int cols, int task, int* g0, int* g1, int* word) {
        *g0 = *g1 = 8 * (task >> 3) + (task & 7);
        *word = 0;
    }
    __device__ static Dots dots(const Dec& d, const ActQ& x) {
        int a = 0, b = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a = dot4(d.w0[i], x.x0[i], a);
            b = dot4(d.w1[i], x.x1[i], b);
        }
        return {a, b};
    }
    __device__ static float combine(const Dec& d, const ActQ& x, Dots s) { return d.c * x.d0 * (float)(s.a + s.b); }
};

}  // namespace leat

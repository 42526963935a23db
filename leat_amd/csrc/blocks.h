// Per-type decoding of one "task": 32 weights of one row for Q4_K and Q6_K, 64 (two blocks) for
// Q8_0, to int8 words for two scale spans, and the f32 combine of their int32 dot products with
// q8 activations. Shared by the matvec, GLU, expert and debug (group-sum) kernels, so the
// integer path the parity tests pin is the one the hot kernels run.
//
// Task decomposition (the reference's "units" of 64 weights, leat/kernels/matvec.py:107-181,
// halved for Q4_K/Q6_K so a row of 4096 or 14336 weights is a whole number of wave64 turns):
//   Q4_K task k of block b (k = 0..7): pair j = k/2 of sub-blocks (2j, 2j+1), half h = k%2:
//        qs bytes [32j + 16h, +16): low nibbles are sub-block 2j's weights 16h..16h+15, high
//        nibbles sub-block 2j+1's. Spans: activation groups 8b+2j and 8b+2j+1, words 4h..4h+3.
//        u = d*sc0*xd0*dot0 + d*sc1*xd1*dot1 - [h==0] dmin*(m0*xs0 + m1*xs1)
//   Q6_K task k of block b: half n = k/4, row pair kk = (k/2)%2 (rows kk and kk+2 of the half),
//        a = k%2 (l in 16a..16a+15): ql bytes [64n + 32kk + 16a, +16) (low nibble row kk, high
//        row kk+2), qh bytes [128 + 32n + 16a, +16) (bits 2kk and 2kk+4). Spans: groups
//        8b+4n+kk and +2, words 4a..4a+3, scales sc[8n+2kk+a] and sc[8n+2kk+4+a].
//        u = d * (sc0*xd0*dot0 + sc1*xd1*dot1)
//   Q8_0 task p: blocks 2p and 2p+1 (68 bytes, always 4-byte aligned). Spans: groups 2p, 2p+1.
//        u = d0*xd0*dot0 + d1*xd1*dot1
#pragma once

#include "common.h"

namespace leat {

template <int TYPE> struct Task;

// activations of one token for one task: 4 words per span (8 for Q8_0), d and s per span
struct ActQ {
    uint32_t x0[8], x1[8];
    float d0, d1, s0, s1;
};

struct Dots {
    int a, b;
};

template <>
struct Task<Q4_K> {
    static constexpr int BYTES = 144, WEIGHTS = 256, TASK_W = 32, PER_BLOCK = 8, WORDS = 4;
    static constexpr bool NEEDS_S = true;  // the mins enter through s = d * sum(q)
    static constexpr int WORD_SKIP = 0;    // span 1's words start where span 0's do, in its own group
    struct Raw {
        u32x4 hdr, qs;
    };
    struct Dec {
        uint32_t w0[4], w1[4];
        float c0, c1, m0, m1;
    };
    __device__ static Raw load(const uint8_t* w, int64_t row, int cols, int task) {
        const int nb = cols / WEIGHTS, b = task >> 3, k = task & 7;
        const uint8_t* blk = w + ((int64_t)row * nb + b) * BYTES;
        Raw r;
        r.hdr = stream_load((const u32x4*)blk);
        r.qs = stream_load((const u32x4*)(blk + 16 + 16 * k));  // 32j + 16h = 16k
        return r;
    }
    // get_scale_min_k4 for sub-blocks s and s+1 (s even), leat/quant.py:182-187
    __device__ static Dec decode(const Raw& r, int task) {
        const int k = task & 7, j = k >> 1, h = k & 1;
        Dec d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w0[i] = r.qs[i] & 0x0F0F0F0Fu;
            d.w1[i] = (r.qs[i] >> 4) & 0x0F0F0F0Fu;
        }
        const float dd = f16_lo(r.hdr[0]), dmin = f16_hi(r.hdr[0]);
        const uint32_t q0 = r.hdr[1], q1 = r.hdr[2], q2 = r.hdr[3];
        float sc[2], mn[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int s = 2 * j + e;
            const uint32_t sh = 8u * (uint32_t)(s & 3);
            const uint32_t a = q0 >> sh, bm = q1 >> sh, c = q2 >> sh;
            const uint32_t scv = s < 4 ? (a & 63u) : ((c & 15u) | ((a >> 2) & 0x30u));
            const uint32_t mv = s < 4 ? (bm & 63u) : (((c >> 4) & 15u) | ((bm >> 2) & 0x30u));
            sc[e] = dd * (float)scv;
            mn[e] = h == 0 ? dmin * (float)mv : 0.0f;
        }
        d.c0 = sc[0];
        d.c1 = sc[1];
        d.m0 = mn[0];
        d.m1 = mn[1];
        return d;
    }
    __device__ static void act_at(int cols, int task, int* g0, int* g1, int* word) {
        const int b = task >> 3, k = task & 7, j = k >> 1, h = k & 1;
        *g0 = 8 * b + 2 * j;
        *g1 = *g0 + 1;
        *word = 4 * h;
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
    __device__ static float combine(const Dec& d, const ActQ& x, Dots s) {
        return d.c0 * x.d0 * (float)s.a + d.c1 * x.d1 * (float)s.b - (d.m0 * x.s0 + d.m1 * x.s1);
    }
};

template <>
struct Task<Q6_K> {
    static constexpr int BYTES = 210, WEIGHTS = 256, TASK_W = 32, PER_BLOCK = 8, WORDS = 4;
    static constexpr bool NEEDS_S = false;
    static constexpr int WORD_SKIP = 0;
    struct Raw {
        uint32_t ql[4], qh[4];
        uint32_t sc;  // the two int8 scales, in bytes 0 and 1
        uint32_t dbits;
    };
    struct Dec {
        uint32_t w0[4], w1[4];
        float c0, c1;
    };
    __device__ static Raw load(const uint8_t* w, int64_t row, int cols, int task) {
        const int nb = cols / WEIGHTS, b = task >> 3, k = task & 7;
        const int n = k >> 2, kk = (k >> 1) & 1, a = k & 1;
        const uint64_t off = ((uint64_t)row * nb + b) * BYTES;
        Raw r;
        load16_even(w, off + 64 * n + 32 * kk + 16 * a, r.ql);
        load16_even(w, off + 128 + 32 * n + 16 * a, r.qh);
        const uint32_t s0 = w[off + 192 + 8 * n + 2 * kk + a];
        const uint32_t s1 = w[off + 192 + 8 * n + 2 * kk + 4 + a];
        r.sc = s0 | (s1 << 8);
        r.dbits = *(const uint16_t*)(w + off + 208);
        return r;
    }
    __device__ static Dec decode(const Raw& r, int task) {
        const int kk = (task >> 1) & 1;
        const uint32_t sh0 = 2u * kk, sh1 = 2u * kk + 4u;
        Dec d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = r.ql[i] & 0x0F0F0F0Fu, hi = (r.ql[i] >> 4) & 0x0F0F0F0Fu;
            const uint32_t h0 = (r.qh[i] >> sh0) & 0x03030303u, h1 = (r.qh[i] >> sh1) & 0x03030303u;
            d.w0[i] = minus_bytes(lo | (h0 << 4), 32);
            d.w1[i] = minus_bytes(hi | (h1 << 4), 32);
        }
        const float dd = f16_lo(r.dbits);
        d.c0 = dd * (float)(int8_t)(r.sc & 0xFF);
        d.c1 = dd * (float)(int8_t)(r.sc >> 8);
        return d;
    }
    __device__ static void act_at(int cols, int task, int* g0, int* g1, int* word) {
        const int b = task >> 3, k = task & 7;
        const int n = k >> 2, kk = (k >> 1) & 1, a = k & 1;
        *g0 = 8 * b + 4 * n + kk;
        *g1 = *g0 + 2;
        *word = 4 * a;
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
    // the reference's order (matvec.py:157-163): d * sum of xd * sc * dot
    __device__ static float combine(const Dec& d, const ActQ& x, Dots s) {
        return x.d0 * d.c0 * (float)s.a + x.d1 * d.c1 * (float)s.b;
    }
};

template <>
struct Task<Q8_0> {
    static constexpr int BYTES = 34, WEIGHTS = 32, TASK_W = 64, PER_BLOCK = 1, WORDS = 8;
    static constexpr bool NEEDS_S = false;
    static constexpr int WORD_SKIP = 0;
    struct Raw {
        uint32_t v[17];
    };
    struct Dec {
        uint32_t w0[8], w1[8];
        float c0, c1;
    };
    __device__ static Raw load(const uint8_t* w, int64_t row, int cols, int task) {
        const int nb = cols / WEIGHTS;
        const uint32_t* p = (const uint32_t*)(w + ((int64_t)row * nb + 2 * task) * BYTES);
        Raw r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u32x4 q = stream_load((const u32x4_a4*)(p + 4 * i));
            r.v[4 * i] = q[0];
            r.v[4 * i + 1] = q[1];
            r.v[4 * i + 2] = q[2];
            r.v[4 * i + 3] = q[3];
        }
        r.v[16] = stream_load(p + 16);
        return r;
    }
    __device__ static Dec decode(const Raw& r, int task) {
        Dec d;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            d.w0[i] = align_bytes(r.v[i + 1], r.v[i], 2);  // block 0's bytes 2..33
            d.w1[i] = r.v[9 + i];                          // block 1's bytes 36..67 of the pair
        }
        d.c0 = f16_lo(r.v[0]);
        d.c1 = f16_hi(r.v[8]);
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
        return d.c0 * x.d0 * (float)s.a + d.c1 * x.d1 * (float)s.b;
    }
};

}  // namespace leat

#include "tasks.h"

namespace leat {

// token t's activations for a task: xq (tokens * cols/4 words), xd/xs (tokens * cols/32)
template <int TYPE, bool SCALES = true>
__device__ __forceinline__ ActQ load_act(const int32_t* xq, const float* xd, const float* xs, int cols,
                                         int t, int task) {
    using T = Task<TYPE>;
    int g0, g1, word;
    T::act_at(cols, task, &g0, &g1, &word);
    const uint32_t* q = (const uint32_t*)xq + (int64_t)t * (cols / 4);
    const float* dd = xd + (int64_t)t * (cols / GROUP);
    ActQ a;
#pragma unroll
    for (int i = 0; i < T::WORDS; i += 4) {
        u32x4 v0 = *(const u32x4*)(q + g0 * 8 + word + i);
        u32x4 v1 = *(const u32x4*)(q + g1 * 8 + word + T::WORD_SKIP + i);
        a.x0[i] = v0[0], a.x0[i + 1] = v0[1], a.x0[i + 2] = v0[2], a.x0[i + 3] = v0[3];
        a.x1[i] = v1[0], a.x1[i + 1] = v1[1], a.x1[i + 2] = v1[2], a.x1[i + 3] = v1[3];
    }
    a.d0 = a.d1 = a.s0 = a.s1 = 0.0f;
    if (!SCALES) return a;
    a.d0 = dd[g0];
    a.d1 = dd[g1];
    if (T::NEEDS_S) {
        const float* ss = xs + (int64_t)t * (cols / GROUP);
        a.s0 = ss[g0];
        a.s1 = ss[g1];
    }
    return a;
}

// the same from LDS, where a workgroup staged B tokens' activations: xq words (B * cols/4),
// then d (B * cols/32), then s (B * cols/32)
template <int TYPE>
__device__ __forceinline__ ActQ load_act_lds(const uint32_t* lds, int tokens, int cols, int t, int task) {
    using T = Task<TYPE>;
    int g0, g1, word;
    T::act_at(cols, task, &g0, &g1, &word);
    const uint32_t* q = lds + t * (cols / 4);
    const float* dd = (const float*)(lds + tokens * (cols / 4)) + t * (cols / GROUP);
    const float* ss = dd + tokens * (cols / GROUP);
    ActQ a;
#pragma unroll
    for (int i = 0; i < T::WORDS; i += 4) {
        u32x4 v0 = *(const u32x4*)(q + g0 * 8 + word + i);
        u32x4 v1 = *(const u32x4*)(q + g1 * 8 + word + T::WORD_SKIP + i);
        a.x0[i] = v0[0], a.x0[i + 1] = v0[1], a.x0[i + 2] = v0[2], a.x0[i + 3] = v0[3];
        a.x1[i] = v1[0], a.x1[i + 1] = v1[1], a.x1[i + 2] = v1[2], a.x1[i + 3] = v1[3];
    }
    a.d0 = dd[g0];
    a.d1 = dd[g1];
    a.s0 = a.s1 = 0.0f;
    if (T::NEEDS_S) {
        a.s0 = ss[g0];
        a.s1 = ss[g1];
    }
    return a;
}

}  // namespace leat

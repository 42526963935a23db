// Row-streaming task decoders, shared by the row-streaming matvec kernels (rows.hip) and the
// mixture-of-experts decode kernels (experts.hip): a lane owns the same task of every row it
// streams, so one set of byte offsets (RowTask::at) serves every row.
#pragma once

#include "blocks.h"

namespace leat {

// A task's weight bytes, read with 32-bit offsets from the row's (uniform) start.
template <int TYPE> struct RowTask;

// Q4_K: a lane's task k = task % 8 is the same in every row (task = lane + 64 i), so its
// sub-block pair j = k / 2 and half h = k % 2 are lane constants, and get_scale_min_k4
// (leat/quant.py:182-187) for sub-blocks 2j and 2j+1 becomes two masked byte pairs per row:
//   j < 2:  scales = bytes 2j, 2j+1 of q0 & 63,  mins = the same of q1
//   j >= 2: scales = (bytes 2j-4, 2j-3 of q2 & 15) | (top 2 bits of those of q0) << 4,
//           mins   = (the same bytes of q2 >> 4)   | (top 2 bits of those of q1) << 4
// (q0, q1, q2 the header's scale words). The mins enter once per sub-block, through the h = 0
// lanes; the h = 1 lanes hold zero activation sums instead of a branch.
template <>
struct RowTask<Q4_K> {
    using Raw = Task<Q4_K>::Raw;
    static constexpr uint32_t STRIDE = 8 * 144;  // bytes from a lane's task i to its task i + 1
    struct Off {
        uint32_t hdr, qs;
        bool high;                      // sub-blocks 4..7
        uint32_t sh_sc, sh_m, sh_top;  // shifts of the scale nibbles, the min nibbles, the top bits
    };
    __device__ static Off at(int task) {
        const uint32_t b = (uint32_t)task >> 3, k = (uint32_t)task & 7, j = k >> 1;
        Off o;
        o.hdr = b * 144u;
        o.qs = b * 144u + 16u + 16u * k;
        o.high = j >= 2;
        const uint32_t base = 16u * (j & 1);
        o.sh_sc = base;
        o.sh_m = o.high ? base + 4 : base;
        o.sh_top = o.high ? base + 2 : base;
        return o;
    }
    __device__ static Raw load(const uint8_t* row, const Off& o) {
        Raw r;
        r.hdr = stream_load((const u32x4*)(row + o.hdr));
        r.qs = stream_load((const u32x4*)(row + o.qs));
        return r;
    }
    // the lane's activations for the task, with s zeroed on the h = 1 lanes
    __device__ static ActQ act(ActQ a, int task) {
        if (task & 1) a.s0 = a.s1 = 0.0f;
        return a;
    }
    // the task's share of the row's product with one token
    __device__ static float dot(const Raw& r, const Off& o, const ActQ& x) {
        const uint32_t q0 = r.hdr[1], q1 = r.hdr[2], q2 = r.hdr[3];
        const uint32_t xs = o.high ? q2 : q0, xm = o.high ? q2 : q1;
        const uint32_t sc = ((xs >> o.sh_sc) & 0x0F0Fu) | ((q0 >> o.sh_top) & 0x3030u);
        const uint32_t mn = ((xm >> o.sh_m) & 0x0F0Fu) | ((q1 >> o.sh_top) & 0x3030u);
        int d0 = 0, d1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d0 = dot4(r.qs[i] & 0x0F0F0F0Fu, x.x0[i], d0);
            d1 = dot4((r.qs[i] >> 4) & 0x0F0F0F0Fu, x.x1[i], d1);
        }
        const float d = f16_lo(r.hdr[0]), dmin = f16_hi(r.hdr[0]);
        const float scaled = (float)(sc & 0xFF) * (x.d0 * (float)d0) + (float)(sc >> 8) * (x.d1 * (float)d1);
        const float mins = (float)(mn & 0xFF) * x.s0 + (float)(mn >> 8) * x.s1;
        return d * scaled - dmin * mins;
    }
};

// Q6_K: 210-byte blocks, so within a row a block starts 2 bytes off a 4-byte boundary when its
// index is odd; a lane's task (and so that alignment) is the same in every row. Each 16-byte run
// (ql, qh) is read as 5 aligned dwords and realigned. The 6-bit values enter the dot products
// unsigned (0..63) and the q - 32 of leat/quant.py:213-223 comes back as 32 * (sum of the
// activations), a lane constant computed once.
template <>
struct RowTask<Q6_K> {
    static constexpr uint32_t STRIDE = 8 * 210;  // a multiple of 4: every task of a lane aligns alike
    struct Raw {
        uint32_t ql[5], qh[5];
        uint32_t sc0, sc1;  // the task's two int8 scales, as bytes
        uint32_t dword;     // the dword holding d
    };
    struct Off {
        uint32_t ql, qh, sc0, sc1, dword;  // dword-aligned runs, scale bytes
        uint32_t shift;                    // bytes to realign the runs: 0 or 2
        bool d_high;                       // d in the upper half of its dword
        uint32_t sh0, sh1;                 // qh bit shifts of the task's rows kk and kk + 2
    };
    __device__ static Off at(int task) {
        const uint32_t b = (uint32_t)task >> 3, k = (uint32_t)task & 7;
        const uint32_t n = k >> 2, kk = (k >> 1) & 1, a = k & 1;
        const uint32_t blk = 210u * b;
        Off o;
        o.shift = blk & 3u;  // 0 or 2
        o.ql = (blk + 64 * n + 32 * kk + 16 * a) & ~3u;
        o.qh = (blk + 128 + 32 * n + 16 * a) & ~3u;
        o.sc0 = blk + 192 + 8 * n + 2 * kk + a;
        o.sc1 = o.sc0 + 4;
        o.dword = (blk + 208) & ~3u;
        o.d_high = ((blk + 208) & 2u) != 0;
        o.sh0 = 2 * kk;
        o.sh1 = 2 * kk + 4;
        return o;
    }
    __device__ static Raw load(const uint8_t* row, const Off& o) {
        Raw r;
        const u32x4 a = stream_load((const u32x4_a4*)(row + o.ql));
        const u32x4 c = stream_load((const u32x4_a4*)(row + o.qh));
        r.ql[0] = a[0], r.ql[1] = a[1], r.ql[2] = a[2], r.ql[3] = a[3];
        r.qh[0] = c[0], r.qh[1] = c[1], r.qh[2] = c[2], r.qh[3] = c[3];
        r.ql[4] = stream_load((const uint32_t*)(row + o.ql + 16));
        r.qh[4] = stream_load((const uint32_t*)(row + o.qh + 16));
        r.sc0 = row[o.sc0];
        r.sc1 = row[o.sc1];
        r.dword = stream_load((const uint32_t*)(row + o.dword));
        return r;
    }
    // the activations, with each span's 32 * sum in s0 and s1 (integer bits)
    __device__ static ActQ act(ActQ a, int) {
        int sum0 = 0, sum1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sum0 = dot4(0x01010101u, a.x0[i], sum0);
            sum1 = dot4(0x01010101u, a.x1[i], sum1);
        }
        a.s0 = __builtin_bit_cast(float, 32 * sum0);
        a.s1 = __builtin_bit_cast(float, 32 * sum1);
        return a;
    }
    __device__ static float dot(const Raw& r, const Off& o, const ActQ& x) {
        int d0 = 0, d1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t ql = align_bytes(r.ql[i + 1], r.ql[i], o.shift);
            const uint32_t qh = align_bytes(r.qh[i + 1], r.qh[i], o.shift);
            const uint32_t w0 = (ql & 0x0F0F0F0Fu) | (((qh >> o.sh0) & 0x03030303u) << 4);
            const uint32_t w1 = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> o.sh1) & 0x03030303u) << 4);
            d0 = dot4(w0, x.x0[i], d0);
            d1 = dot4(w1, x.x1[i], d1);
        }
        d0 -= __builtin_bit_cast(int, x.s0);
        d1 -= __builtin_bit_cast(int, x.s1);
        const float d = o.d_high ? f16_hi(r.dword) : f16_lo(r.dword);
        const float s0 = (float)(int8_t)r.sc0, s1 = (float)(int8_t)r.sc1;
        return d * (x.d0 * s0 * (float)d0 + x.d1 * s1 * (float)d1);
    }
};

template <>
struct RowTask<Q8_0> {
    using Raw = Task<Q8_0>::Raw;
    static constexpr uint32_t STRIDE = 64 * 68;
    struct Off {
        uint32_t first;
    };
    __device__ static Off at(int task) { return {(uint32_t)task * 68u}; }
    __device__ static Raw load(const uint8_t* row, const Off& o) {
        const uint32_t* p = (const uint32_t*)(row + o.first);
        Raw r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u32x4 q = stream_load((const u32x4_a4*)(p + 4 * i));
            r.v[4 * i] = q[0], r.v[4 * i + 1] = q[1], r.v[4 * i + 2] = q[2], r.v[4 * i + 3] = q[3];
        }
        r.v[16] = stream_load(p + 16);
        return r;
    }
    __device__ static ActQ act(ActQ a, int) { return a; }
    __device__ static float dot(const Raw& r, const Off&, const ActQ& x) {
        const Task<Q8_0>::Dec dec = Task<Q8_0>::decode(r, 0);
        return Task<Q8_0>::combine(dec, x, Task<Q8_0>::dots(dec, x));
    }
};

}  // namespace leat

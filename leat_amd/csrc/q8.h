// The activation quantizer's arithmetic (leat/kernels/quantize.py:25-49), shared by the
// standalone quantizer and the kernels that quantize their own input, so that every path gives
// the same bits:
//   per group of 32 values  d = max|x| / 127,  q = roundf(x / d) (0 where d = 0),  s = d * sum(q)
// with both quotients IEEE f32 divisions and roundf rounding half away from zero. The values are
// packed four to an int32 word, byte i of word w holding value 4w + i.
//
// Layout of the work: a 256-thread block takes a row 1024 values at a time, thread `tid` the 4
// consecutive values at 4 * tid, so the 8 threads of an aligned octet hold one group of 32.
#pragma once

#include "common.h"

namespace leat {

// 1 / sqrt(mean(x^2) + eps) over the n values of row xr, the same in every thread of a block of
// THREADS >= 256 threads (n a multiple of 4). `partial` is THREADS / 64 floats of the block's
// shared memory. The summation order is that of a 256-thread block whatever THREADS is, so every
// kernel normalizes to the same bits: threads 0..255 sum float4 runs strided by 1024, each wave
// reduces with DPP moves (wave_sum_dpp), then (w0 + w1) + (w2 + w3); further waves contribute nothing.
// a float4's sum of squares, and its values normalized (times inv, times the norm weight): the
// expressions every path uses, so all of them round alike
__device__ __forceinline__ float sum_sq4(float4 v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }
__device__ __forceinline__ float4 normed4(float4 v, float inv, float4 w) {
    return make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
}

template <int THREADS = 256>
__device__ __forceinline__ float block_inv_rms(const float* __restrict__ xr, int n, float eps, float* partial) {
    const int tid = threadIdx.x;
    float ss = 0.0f;
    if (tid < 256)
        for (int at0 = tid * 4; at0 < n; at0 += 4 * 1024) {
            // 4 loads in flight, summed in order
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (at0 + 1024 * u < n) v[u] = *(const float4*)(xr + at0 + 1024 * u);
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (at0 + 1024 * u < n) ss += sum_sq4(v[u]);
        }
    ss = wave_sum_dpp(ss);
    __syncthreads();  // `partial` may still be read from a previous row
    if ((tid & (WAVE - 1)) == 0) partial[tid / WAVE] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    return 1.0f / sqrtf(total / (float)n + eps);
}

// v of a lane's aligned octet of lanes combined with `op` over the octet, by DPP lane moves (no
// LDS traffic): xor 1 and xor 2 within quads, then xor 4 as a left shift by 4 into banks 0 and 2
// of each row of 16 and a right shift by 4 into banks 1 and 3
template <typename Op>
__device__ __forceinline__ float octet_reduce(float v, Op op) {
    v = op(v, LEAT_DPP(v, 0xB1, 0xF, 0xF));  // quad_perm [1,0,3,2]
    v = op(v, LEAT_DPP(v, 0x4E, 0xF, 0xF));  // quad_perm [2,3,0,1]
    const int bits = __builtin_bit_cast(int, v);
    int other = __builtin_amdgcn_update_dpp(bits, bits, 0x104, 0xF, 0x5, false);  // row_shl:4, banks 0, 2
    other = __builtin_amdgcn_update_dpp(other, bits, 0x114, 0xF, 0xA, false);      // row_shr:4, banks 1, 3
    return op(v, __builtin_bit_cast(float, other));
}

// roundf(v / scale) (IEEE quotient, halves away from zero) for scale > 0, from a reciprocal:
// with r = rcp(scale) (within 1 ulp) the product a = v * r is within |v / scale| * 2^-21 <= 7e-5
// of the correctly rounded quotient (|v / scale| <= 127 here), so both round to the same integer
// unless a lies within that of a half-integer; those rare values, and scales too small for the
// reciprocal, take the division itself.
__device__ __forceinline__ int round_quotient(float v, float scale, float r) {
    const float a = v * r;
    const float frac = fabsf(a - truncf(a));
    if (fabsf(frac - 0.5f) < 1e-4f || !(scale > 1e-30f)) return (int)roundf(v / scale);
    return (int)rintf(a);
}

// Quantizes the 4 values v (positions 4 * (tid % 8) .. + 3 of their group) together with the
// other 7 threads of the aligned octet. Returns the packed word; every thread of the octet also
// gets the group's d and s.
__device__ __forceinline__ uint32_t quantize4(float4 v, float* d_out, float* s_out) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = octet_reduce(amax, [](float a, float b) { return fmaxf(a, b); });
    const float scale = amax / 127.0f;
    int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
    if (scale > 0.0f) {
        const float r = __builtin_amdgcn_rcpf(scale);
        q0 = round_quotient(v.x, scale, r);
        q1 = round_quotient(v.y, scale, r);
        q2 = round_quotient(v.z, scale, r);
        q3 = round_quotient(v.w, scale, r);
    }
    // the octet's sum of q: small integers, exact in f32 whatever the order
    const float total = octet_reduce((float)(q0 + q1 + q2 + q3), [](float a, float b) { return a + b; });
    *d_out = scale;
    *s_out = scale * total;
    return (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
           ((uint32_t)(q3 & 0xFF) << 24);
}

// v of each lane combined with `op` over its aligned 32 lanes, by DPP moves and the gfx950
// permlane16 swap (no LDS traffic): xor 1, 2, 4 as octet_reduce, xor 8 as a rotation of the row
// of 16 by 8, then the two rows of 16 exchanged (each lane gets its own value and its partner's,
// in an order that depends on the lane: op must commute)
template <typename Op>
__device__ __forceinline__ float lane32_reduce(float v, Op op) {
    v = octet_reduce(v, op);
    v = op(v, LEAT_DPP(v, 0x128, 0xF, 0xF));  // row_ror:8
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const uint32_t lo = r[0], hi = r[1];
    return op(__uint_as_float(lo), __uint_as_float(hi));
}

// The q8 of a group of 32 values held one a lane by an aligned 32 lanes of a wave (all of them
// active), bit for bit as quantize4 and the standalone quantizer write it: returns, for lanes
// 4j of the group, the word of the values of lanes 4j .. 4j + 3 (other lanes: unspecified); every
// lane gets the group's d and s.
__device__ __forceinline__ uint32_t quantize_lane32(float v, float* d_out, float* s_out) {
    const float amax = lane32_reduce(fabsf(v), [](float a, float b) { return fmaxf(a, b); });
    const float scale = amax / 127.0f;
    const int q = scale > 0.0f ? round_quotient(v, scale, __builtin_amdgcn_rcpf(scale)) : 0;
    // small integers, exact in f32 whatever the order
    const float total = lane32_reduce((float)q, [](float a, float b) { return a + b; });
    *d_out = scale;
    *s_out = scale * total;
    // lanes 4j take the bytes of lanes 4j + 1 .. 4j + 3 (row_shl:k reads lane l + k within the row of 16)
    const int b0 = q & 0xFF;
    const int b1 = __builtin_amdgcn_update_dpp(0, b0, 0x101, 0xF, 0xF, false);
    const int b2 = __builtin_amdgcn_update_dpp(0, b0, 0x102, 0xF, 0xF, false);
    const int b3 = __builtin_amdgcn_update_dpp(0, b0, 0x103, 0xF, 0xF, false);
    return (uint32_t)b0 | ((uint32_t)b1 << 8) | ((uint32_t)b2 << 16) | ((uint32_t)b3 << 24);
}

// One row of n values (after RMSNorm when `weight` is set, `inv` its 1/rms) into q words, d and s
// (pointers to the row's first word and group), by a block of THREADS threads. Any address space.
template <int THREADS = 256, typename Q, typename F>
__device__ __forceinline__ void quantize_row(const float* __restrict__ xr, int n, const float* __restrict__ weight,
                                             float inv, Q* q, F* d, F* s) {
    const int tid = threadIdx.x;
    // n % 32 == 0: an octet is all in or all out; 4 float4 (and their norm weights) in flight
    for (int at0 = tid * 4; at0 < n; at0 += 16 * THREADS) {
        float4 v[4], w[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int at = at0 + 4 * THREADS * u;
            if (at < n) {
                v[u] = *(const float4*)(xr + at);
                if (weight) w[u] = *(const float4*)(weight + at);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int at = at0 + 4 * THREADS * u;
            if (at >= n) break;
            float dv, sv;
            const uint32_t word = quantize4(weight ? normed4(v[u], inv, w[u]) : v[u], &dv, &sv);
            q[at / 4] = word;
            if ((tid & 7) == 0) {
                d[at / GROUP] = dv;
                s[at / GROUP] = sv;
            }
        }
    }
}

// B rows of n <= 1024 * NX f32 values (and the norm weight), held in registers by threads
// 0..255 of a block, the float4 at 4 tid + 1024 j: loaded before anything else the block asks
// of memory, so that the norm and quantization wait for x alone. quantize() then writes what
// block_inv_rms and quantize_row write, bit for bit: the same sums in the same order and the
// same quantize4 of every float4.
template <int B, int NX>
struct RowsInRegs {
    float4 v[B][NX], w[NX];

    __device__ __forceinline__ void load(const float* __restrict__ x, const float* __restrict__ weight, int n) {
        const int tid = threadIdx.x;
        if (tid >= 256) return;
#pragma unroll
        for (int j = 0; j < NX; j++) {
            const int at = 4 * tid + 1024 * j;
            if (at >= n) break;
#pragma unroll
            for (int t = 0; t < B; t++) v[t][j] = *(const float4*)(x + (int64_t)t * n + at);
            if (weight) w[j] = *(const float4*)(weight + at);
        }
    }

    // token t's 1/rms and q8 into q (words), d and s (the token's first word and group); every
    // thread of the block (THREADS of them) calls it; `partial` as block_inv_rms's
    template <int THREADS>
    __device__ __forceinline__ void quantize(int t, const float* weight, float eps, int n, float* partial, uint32_t* q,
                                             float* d, float* s) {
        const int tid = threadIdx.x;
        float inv = 1.0f;
        if (weight) {
            float ss = 0.0f;
            if (tid < 256)
#pragma unroll
                for (int j = 0; j < NX; j++)
                    if (4 * tid + 1024 * j < n) ss += sum_sq4(v[t][j]);
            ss = wave_sum_dpp(ss);
            __syncthreads();  // `partial` may still be read from a previous row
            if ((tid & (WAVE - 1)) == 0) partial[tid / WAVE] = ss;
            __syncthreads();
            const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
            inv = 1.0f / sqrtf(total / (float)n + eps);
        }
        if (tid >= 256) return;
#pragma unroll
        for (int j = 0; j < NX; j++) {
            const int at = 4 * tid + 1024 * j;  // n % 32 == 0: an octet is all in or all out
            if (at >= n) break;
            const float4 u = weight ? normed4(v[t][j], inv, w[j]) : v[t][j];
            float dv, sv;
            q[at / 4] = quantize4(u, &dv, &sv);
            if ((tid & 7) == 0) {
                d[at / GROUP] = dv;
                s[at / GROUP] = sv;
            }
        }
    }
};

// The q8 of one group of 32 consecutive outputs per token, as quantize_q8 would write it: value i
// of token t is vals[t][i] (shared memory, 16-byte aligned), and the aligned octet of threads
// 8t .. 8t + 7 of the block (t < B) quantizes it with quantize4, a float4 a thread (DPP moves
// only), into group `group` of the token's row of `rows` values (hq words, hd and hs per group).
template <int B>
__device__ __forceinline__ void store_group_q8(const float (*vals)[32], int rows, int group, uint32_t* hq, float* hd,
                                               float* hs) {
    if (threadIdx.x >= 8 * B) return;
    const int t = threadIdx.x >> 3, o = threadIdx.x & 7;
    float dv, sv;
    const uint32_t word = quantize4(((const float4*)vals[t])[o], &dv, &sv);
    const int64_t first = (int64_t)t * rows + 32 * group;
    hq[first / 4 + o] = word;
    if (o == 0) {
        hd[first / GROUP] = dv;
        hs[first / GROUP] = sv;
    }
}

}  // namespace leat

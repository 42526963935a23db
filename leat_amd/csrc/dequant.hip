// Dequantization (leat/quant.py:117-119, 182-197, 213-223, in ggml's float operation order:
// Q8_0 d*q, Q4_K (d*sc)*q - (dmin*m), Q6_K (d*sc)*q, each product and difference rounded on its
// own, no fused multiply-add), the LEAT_KERNELS=ref linear layer on it (leat/ops.py:35-38: f32
// activations, not quantized), and the exact int32 span sums of the int8 path for parity tests.
#include "blocks.h"

namespace leat {

// the 32 weights of piece p of a row: Q4_K sub-block p, Q6_K row-of-32 p (half p/4, k = p%4),
// Q8_0 block p
template <int TYPE>
__device__ void dequant_piece(const uint8_t* __restrict__ blk, int p, float y[32]) {
#pragma clang fp contract(off)
    if (TYPE == Q8_0) {
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[0] | (blk[1] << 8)));
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = d * (float)(int8_t)blk[2 + l];
    } else if (TYPE == Q4_K) {
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[0] | (blk[1] << 8)));
        const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[2] | (blk[3] << 8)));
        const uint8_t* q = blk + 4;
        int sc, m;
        if (p < 4) {
            sc = q[p] & 63;
            m = q[p + 4] & 63;
        } else {
            sc = (q[p + 4] & 0xF) | ((q[p - 4] >> 6) << 4);
            m = (q[p + 4] >> 4) | ((q[p] >> 6) << 4);
        }
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t* qs = blk + 16 + 32 * (p >> 1);
        const int shift = 4 * (p & 1);
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = d1 * (float)((qs[l] >> shift) & 0xF) - m1;
    } else {
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(blk[208] | (blk[209] << 8)));
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
    }
}

template <int TYPE>
constexpr int block_bytes() {
    return TYPE == Q8_0 ? 34 : TYPE == Q4_K ? 144 : 210;
}
template <int TYPE>
constexpr int block_weights() {
    return TYPE == Q8_0 ? 32 : 256;
}

template <int TYPE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ blocks, int64_t pieces,
                                                      float* __restrict__ out) {
    constexpr int PER = block_weights<TYPE>() / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pieces) return;
    const int64_t b = i / PER;
    const int p = (int)(i % PER);
    float y[32];
    dequant_piece<TYPE>(blocks + b * block_bytes<TYPE>(), p, y);
    float* o = out + i * 32;
#pragma unroll
    for (int l = 0; l < 32; l += 4) *(float4*)(o + l) = make_float4(y[l], y[l + 1], y[l + 2], y[l + 3]);
}

// out[t, :] = row ids[t] of W decoded (ids outside the matrix give zeros): a thread per 32 weights
template <int TYPE>
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t* __restrict__ w, int rows, int cols,
                                                        const int32_t* __restrict__ ids, float* __restrict__ out) {
    constexpr int PER = block_weights<TYPE>() / 32;
    const int t = blockIdx.y, pieces = cols / 32;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= pieces) return;
    const int id = ids[t];
    float y[32];
    if (id >= 0 && id < rows) {
        const int64_t nb = cols / block_weights<TYPE>();
        dequant_piece<TYPE>(w + ((int64_t)id * nb + p / PER) * block_bytes<TYPE>(), p % PER, y);
    } else {
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = 0.0f;
    }
    float* o = out + (int64_t)t * cols + (int64_t)p * 32;
#pragma unroll
    for (int l = 0; l < 32; l += 4) *(float4*)(o + l) = make_float4(y[l], y[l + 1], y[l + 2], y[l + 3]);
}

// out[t * rows + row] = sum_c x[t, c] * W[row, c] (+ residual): one wave per row, lanes over
// pieces of 32 weights, each decoded exactly as above then multiplied into f32 sums
template <int TYPE, int B>
__global__ __launch_bounds__(256) void matvec_f32x_kernel(const uint8_t* __restrict__ w, int rows, int cols,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ residual,
                                                          float* __restrict__ out) {
    constexpr int PER = block_weights<TYPE>() / 32;
    const int lane = threadIdx.x & (WAVE - 1);
    const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE);
    if (row >= rows) return;
    const int nb = cols / block_weights<TYPE>(), pieces = cols / 32;
    float acc[B];
#pragma unroll
    for (int t = 0; t < B; t++) acc[t] = 0.0f;
    for (int p = lane; p < pieces; p += WAVE) {
        float y[32];
        dequant_piece<TYPE>(w + ((int64_t)row * nb + p / PER) * block_bytes<TYPE>(), p % PER, y);
#pragma unroll
        for (int t = 0; t < B; t++) {
            const float* xt = x + (int64_t)t * cols + (int64_t)p * 32;
#pragma unroll
            for (int l = 0; l < 32; l += 4) {
                const float4 v = *(const float4*)(xt + l);
                acc[t] += y[l] * v.x + y[l + 1] * v.y + y[l + 2] * v.z + y[l + 3] * v.w;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < B; t++) acc[t] = wave_sum(acc[t]);
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < B; t++) {
            const int64_t at = (int64_t)t * rows + row;
            out[at] = acc[t] + (residual ? residual[at] : 0.0f);
        }
    }
}

// exact int32 sums per scale span (Q4_K/Q8_0: groups of 32; Q6_K: halves of 16), by the matvec
// kernels' own task decode: out[(t * rows + row) * spans + span]
template <int TYPE>
__global__ __launch_bounds__(256) void group_dots_kernel(const uint8_t* __restrict__ w, int rows, int cols,
                                                         const int32_t* __restrict__ xq, int tokens,
                                                         int32_t* __restrict__ out) {
    using T = Task<TYPE>;
    const int tasks = cols / T::TASK_W;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)tokens * rows * tasks) return;
    const int task = (int)(i % tasks);
    const int row = (int)((i / tasks) % rows);
    const int t = (int)(i / ((int64_t)tasks * rows));
    const ActQ act = load_act<TYPE, false>(xq, nullptr, nullptr, cols, t, task);
    const Dots dd = T::dots(T::decode(T::load(w, row, cols, task), task), act);
    int g0, g1, word;
    T::act_at(cols, task, &g0, &g1, &word);
    if (TYPE == Q6_K) {
        const int spans = cols / 16;
        int32_t* o = out + ((int64_t)t * rows + row) * spans;
        o[2 * g0 + word / 4] = dd.a;
        o[2 * g1 + word / 4] = dd.b;
    } else if (TYPE == Q4_K) {  // two tasks (halves h) add up to a group: the h = 1 lane adds
        const int spans = cols / 32;
        int32_t* o = out + ((int64_t)t * rows + row) * spans;
        atomicAdd(o + g0, dd.a);
        atomicAdd(o + g1, dd.b);
    } else {
        const int spans = cols / 32;
        int32_t* o = out + ((int64_t)t * rows + row) * spans;
        o[g0] = dd.a;
        o[g1] = dd.b;
    }
}

__global__ void zero_kernel(int32_t* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

int check_cols(int type, int cols);
int check_ptrs(int type, const void* w, const void* xq);

}  // namespace leat

using namespace leat;

extern "C" int leat_dequantize(int type, const void* blocks, int64_t n_blocks, float* out, void* stream) {
    LEAT_REQUIRE(blocks && out && n_blocks >= 0, "dequantize: null pointer");
    if (n_blocks == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* b = (const uint8_t*)blocks;
    int64_t pieces;
    switch (type) {
    case Q8_0:
        pieces = n_blocks;
        hipLaunchKernelGGL(dequant_kernel<Q8_0>, dim3((pieces + 255) / 256), dim3(256), 0, st, b, pieces, out);
        break;
    case Q4_K:
        pieces = n_blocks * 8;
        hipLaunchKernelGGL(dequant_kernel<Q4_K>, dim3((pieces + 255) / 256), dim3(256), 0, st, b, pieces, out);
        break;
    case Q6_K:
        pieces = n_blocks * 8;
        hipLaunchKernelGGL(dequant_kernel<Q6_K>, dim3((pieces + 255) / 256), dim3(256), 0, st, b, pieces, out);
        break;
    default: set_error("dequantize: unsupported type %d", type); return -1;
    }
    return check_launch("dequantize");
}

extern "C" int leat_embedding(int type, const void* w, int rows, int cols, const int32_t* ids, int tokens, float* out,
                              void* stream) {
    LEAT_REQUIRE(w && ids && out && rows > 0, "embedding: null pointer or empty matrix");
    LEAT_REQUIRE(tokens >= 0 && tokens <= 65535, "embedding: %d tokens", tokens);
    if (check_cols(type, cols)) return -1;
    if (tokens == 0) return 0;
    const dim3 grid((cols / 32 + 255) / 256, tokens);
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* b = (const uint8_t*)w;
    switch (type) {
    case Q8_0: hipLaunchKernelGGL(embedding_kernel<Q8_0>, grid, dim3(256), 0, st, b, rows, cols, ids, out); break;
    case Q4_K: hipLaunchKernelGGL(embedding_kernel<Q4_K>, grid, dim3(256), 0, st, b, rows, cols, ids, out); break;
    default: hipLaunchKernelGGL(embedding_kernel<Q6_K>, grid, dim3(256), 0, st, b, rows, cols, ids, out); break;
    }
    return check_launch("embedding");
}

template <int TYPE>
static int f32x_t(const uint8_t* w, int rows, int cols, const float* x, int tokens, const float* res, float* out,
                  hipStream_t st) {
    const dim3 grid((rows + 3) / 4), block(256);
    switch (tokens) {
#define CASE(B) \
    case B: hipLaunchKernelGGL((matvec_f32x_kernel<TYPE, B>), grid, block, 0, st, w, rows, cols, x, res, out); break;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(16)
#undef CASE
    default: set_error("matvec_f32x: %d tokens (1..8 or 16 supported)", tokens); return -1;
    }
    return check_launch("matvec_f32x");
}

extern "C" int leat_matvec_f32x(int type, const void* w, int rows, int cols, const float* x, int tokens,
                                const float* residual, float* out, void* stream) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(w && x && out && rows > 0, "matvec_f32x: null pointer or empty matrix");
    LEAT_REQUIRE((uintptr_t)x % 16 == 0, "matvec_f32x: activations must start 16-byte aligned");
    const uint8_t* b = (const uint8_t*)w;
    hipStream_t st = (hipStream_t)stream;
    switch (type) {
    case Q8_0: return f32x_t<Q8_0>(b, rows, cols, x, tokens, residual, out, st);
    case Q4_K: return f32x_t<Q4_K>(b, rows, cols, x, tokens, residual, out, st);
    default: return f32x_t<Q6_K>(b, rows, cols, x, tokens, residual, out, st);
    }
}

extern "C" int leat_group_dots(int type, const void* w, int rows, int cols, const int32_t* xq, int tokens,
                               int32_t* out, void* stream) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(w && xq && out && rows > 0 && tokens > 0, "group_dots: null pointer or empty input");
    if (check_ptrs(type, w, xq)) return -1;
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* b = (const uint8_t*)w;
    const int task_w = type == Q8_0 ? 64 : 32;
    const int64_t n = (int64_t)tokens * rows * (cols / task_w);
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (type) {
    case Q8_0: hipLaunchKernelGGL(group_dots_kernel<Q8_0>, grid, block, 0, st, b, rows, cols, xq, tokens, out); break;
    case Q4_K: {
        const int64_t spans = (int64_t)tokens * rows * (cols / 32);
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((spans + 255) / 256)), dim3(256), 0, st, out, spans);
        hipLaunchKernelGGL(group_dots_kernel<Q4_K>, grid, block, 0, st, b, rows, cols, xq, tokens, out);
        break;
    }
    default: hipLaunchKernelGGL(group_dots_kernel<Q6_K>, grid, block, 0, st, b, rows, cols, xq, tokens, out); break;
    }
    return check_launch("group_dots");
}

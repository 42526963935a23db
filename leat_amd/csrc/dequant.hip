// Dequantization (leat/quant.py:117-119, 182-197, 213-223, in ggml's float operation order:
// Q8_0 d*q, Q4_K (d*sc)*q - (dmin*m), Q6_K (d*sc)*q, each product and difference rounded on its
// own, no fused multiply-add), the LEAT_KERNELS=ref linear layer on it (leat/ops.py:35-38: f32
// activations, not quantized), and the exact int32 span sums of the int8 path for parity tests.
#include "blocks.h"
#include "formats.h"

namespace leat {

template <int TYPE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ blocks, int64_t pieces,
                                                      float* __restrict__ out) {
    constexpr int PER = Format<TYPE>::WEIGHTS / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pieces) return;
    const int64_t b = i / PER;
    const int p = (int)(i % PER);
    float y[32];
    dequant_piece<TYPE>(blocks + b * Format<TYPE>::BYTES, p, y);
    float* o = out + i * 32;
#pragma unroll
    for (int l = 0; l < 32; l += 4) *(float4*)(o + l) = make_float4(y[l], y[l + 1], y[l + 2], y[l + 3]);
}

// out[t, :] = row ids[t] of W decoded (ids outside the matrix give zeros): a thread per 32 weights
template <int TYPE>
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t* __restrict__ w, int rows, int cols,
                                                        const int32_t* __restrict__ ids, float* __restrict__ out) {
    constexpr int PER = Format<TYPE>::WEIGHTS / 32;
    const int t = blockIdx.y, pieces = cols / 32;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= pieces) return;
    const int id = ids[t];
    float y[32];
    if (id >= 0 && id < rows) {
        const int64_t nb = cols / Format<TYPE>::WEIGHTS;
        dequant_piece<TYPE>(w + ((int64_t)id * nb + p / PER) * Format<TYPE>::BYTES, p % PER, y);
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
    constexpr int PER = Format<TYPE>::WEIGHTS / 32;
    const int lane = threadIdx.x & (WAVE - 1);
    const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE);
    if (row >= rows) return;
    const int nb = cols / Format<TYPE>::WEIGHTS, pieces = cols / 32;
    float acc[B];
#pragma unroll
    for (int t = 0; t < B; t++) acc[t] = 0.0f;
    for (int p = lane; p < pieces; p += WAVE) {
        float y[32];
        dequant_piece<TYPE>(w + ((int64_t)row * nb + p / PER) * Format<TYPE>::BYTES, p % PER, y);
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
    } else if (TYPE == Q4_K || TYPE == Q5_K) {  // two tasks (halves h) add up to a group: the h = 1 lane adds
        const int spans = cols / 32;
        int32_t* o = out + ((int64_t)t * rows + row) * spans;
        atomicAdd(o + g0, dd.a);
        atomicAdd(o + g1, dd.b);
    } else if (TYPE == IQ4_XS) {  // a task is one group, its two halves of 16
        out[((int64_t)t * rows + row) * (cols / 32) + g0] = dd.a + dd.b;
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

// a row length of whole blocks of `type` (any type the dequantizer decodes)
static int check_format_cols(int type, int cols, const char* what) {
    int weights = 0;
    switch (type) {
#define LEAT_WEIGHTS(T) \
    case T: weights = Format<T>::WEIGHTS; break;
        LEAT_FORMATS(LEAT_WEIGHTS)
#undef LEAT_WEIGHTS
    default: set_error("%s: unsupported type %d", what, type); return -1;
    }
    LEAT_REQUIRE(cols > 0 && cols % weights == 0, "%s: cols %d is not a whole number of %d-weight blocks", what, cols,
                 weights);
    return 0;
}

extern "C" int leat_dequantize(int type, const void* blocks, int64_t n_blocks, float* out, void* stream) {
    LEAT_REQUIRE(blocks && out && n_blocks >= 0, "dequantize: null pointer");
    if (n_blocks == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* b = (const uint8_t*)blocks;
    switch (type) {
#define LEAT_DEQUANT(T)                                                                                        \
    case T: {                                                                                                  \
        const int64_t pieces = n_blocks * (Format<T>::WEIGHTS / 32);                                           \
        hipLaunchKernelGGL(dequant_kernel<T>, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, st, b, pieces, out); \
        break;                                                                                                 \
    }
        LEAT_FORMATS(LEAT_DEQUANT)
#undef LEAT_DEQUANT
    default: set_error("dequantize: unsupported type %d", type); return -1;
    }
    return check_launch("dequantize");
}

extern "C" int leat_embedding(int type, const void* w, int rows, int cols, const int32_t* ids, int tokens, float* out,
                              void* stream) {
    LEAT_REQUIRE(w && ids && out && rows > 0, "embedding: null pointer or empty matrix");
    LEAT_REQUIRE(tokens >= 0 && tokens <= 65535, "embedding: %d tokens", tokens);
    if (check_format_cols(type, cols, "embedding")) return -1;
    if (tokens == 0) return 0;
    const dim3 grid((cols / 32 + 255) / 256, tokens);
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* b = (const uint8_t*)w;
    switch (type) {
#define LEAT_EMBED(T) \
    case T: hipLaunchKernelGGL(embedding_kernel<T>, grid, dim3(256), 0, st, b, rows, cols, ids, out); break;
        LEAT_FORMATS(LEAT_EMBED)
#undef LEAT_EMBED
    default: break;
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
    if (check_format_cols(type, cols, "matvec_f32x")) return -1;
    LEAT_REQUIRE(w && x && out && rows > 0, "matvec_f32x: null pointer or empty matrix");
    LEAT_REQUIRE((uintptr_t)x % 16 == 0, "matvec_f32x: activations must start 16-byte aligned");
    const uint8_t* b = (const uint8_t*)w;
    hipStream_t st = (hipStream_t)stream;
    switch (type) {
#define LEAT_F32X(T) \
    case T: return f32x_t<T>(b, rows, cols, x, tokens, residual, out, st);
        LEAT_FORMATS(LEAT_F32X)
#undef LEAT_F32X
    default: return -1;
    }
}

extern "C" int leat_group_dots(int type, const void* w, int rows, int cols, const int32_t* xq, int tokens,
                               int32_t* out, void* stream) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(w && xq && out && rows > 0 && tokens > 0, "group_dots: null pointer or empty input");
    if (check_ptrs(type, w, xq)) return -1;
    hipStream_t st = (hipStream_t)stream;
    const uint8_t* b = (const uint8_t*)w;
    const bool halves = type == Q4_K || type == Q5_K;  // two tasks add into each group: cleared first
    if (halves) {
        const int64_t spans = (int64_t)tokens * rows * (cols / 32);
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((spans + 255) / 256)), dim3(256), 0, st, out, spans);
    }
    switch (type) {
#define LEAT_DOTS(T)                                                                                                \
    case T: {                                                                                                       \
        const int64_t n = (int64_t)tokens * rows * (cols / Task<T>::TASK_W);                                        \
        hipLaunchKernelGGL(group_dots_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, b, rows, cols, \
                           xq, tokens, out);                                                                        \
        break;                                                                                                      \
    }
        LEAT_DOTS(Q4_0) LEAT_DOTS(Q4_1) LEAT_DOTS(Q5_0) LEAT_DOTS(Q5_1) LEAT_DOTS(Q8_0) LEAT_DOTS(Q4_K) LEAT_DOTS(Q5_K)
        LEAT_DOTS(Q6_K) LEAT_DOTS(IQ4_NL) LEAT_DOTS(IQ4_XS) LEAT_DOTS(MXFP4)
#undef LEAT_DOTS
    default: set_error("group_dots: unsupported type %d", type); return -1;
    }
    return check_launch("group_dots");
}

// Activations to int8 in groups of 32, as llama.cpp's q8_1 and leat's quantize_q8
// (leat/kernels/quantize.py:25-109; oracle tests/test_kernels.py:28-36): per group
// d = max|x| / 127, q = roundf(x / d) (both divisions IEEE, rounding half away from zero, q = 0
// where d = 0), s = d * sum(q); q packed four per int32 word, byte i of word w being value 4w+i.
// Optionally after RMSNorm with a weight: x * (1 / sqrt(mean(x^2) + eps)) * weight, in f32.
//
// A block of 256 threads per 1024 values of a row (a grid of rows x parts, so a decode step's
// few rows still spread over many CUs); each thread takes 4 consecutive values, so the 8 lanes
// of an aligned octet hold one group and reduce it with shuffles.
#include "common.h"

namespace leat {

template <bool NORM>
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x, int n,
                                                          const float* __restrict__ weight, float eps,
                                                          uint32_t* __restrict__ q, float* __restrict__ d,
                                                          float* __restrict__ s) {
    // block (row, part): 256 threads quantize values [1024 part, 1024 part + 1024) of the row
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)row * n;
    float inv = 1.0f;
    if (NORM) {  // every block of the row sums the whole row's squares, from L2 after the first
        __shared__ float partial[4];
        float ss = 0.0f;
        for (int at = tid * 4; at < n; at += 1024) {
            const float4 v = *(const float4*)(xr + at);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        if ((tid & (WAVE - 1)) == 0) partial[tid / WAVE] = ss;
        __syncthreads();
        const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
        inv = 1.0f / sqrtf(total / (float)n + eps);
    }
    const int at = blockIdx.y * 1024 + tid * 4;
    if (at >= n) return;  // n % 32 == 0: an aligned octet of lanes is all in or all out
    float4 v = *(const float4*)(xr + at);
    if (NORM) {
        const float4 wv = *(const float4*)(weight + at);
        v.x = v.x * inv * wv.x;
        v.y = v.y * inv * wv.y;
        v.z = v.z * inv * wv.z;
        v.w = v.w * inv * wv.w;
    }
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float scale = amax / 127.0f;
    int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
    if (scale > 0.0f) {
        q0 = (int)roundf(v.x / scale);
        q1 = (int)roundf(v.y / scale);
        q2 = (int)roundf(v.z / scale);
        q3 = (int)roundf(v.w / scale);
    }
    int total = q0 + q1 + q2 + q3;
    total += __shfl_xor(total, 1, 8);
    total += __shfl_xor(total, 2, 8);
    total += __shfl_xor(total, 4, 8);
    const int64_t word = ((int64_t)row * n + at) / 4;
    q[word] = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
              ((uint32_t)(q3 & 0xFF) << 24);
    if ((tid & 7) == 0) {
        const int64_t g = ((int64_t)row * n + at) / GROUP;
        d[g] = scale;
        s[g] = scale * (float)total;
    }
}

}  // namespace leat

using namespace leat;

extern "C" int leat_quantize_q8(const float* x, int rows, int n, const float* norm_weight, float eps, int32_t* q,
                                float* d, float* s, void* stream) {
    LEAT_REQUIRE(x && q && d && s, "quantize_q8: null pointer");
    LEAT_REQUIRE(rows >= 0 && n > 0 && n % GROUP == 0, "quantize_q8: rows of %d values are not whole groups of 32", n);
    if (rows == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(rows, (n + 1023) / 1024);
    if (norm_weight)
        hipLaunchKernelGGL(quantize_q8_kernel<true>, grid, dim3(256), 0, st, x, n, norm_weight, eps, (uint32_t*)q,
                           d, s);
    else
        hipLaunchKernelGGL(quantize_q8_kernel<false>, grid, dim3(256), 0, st, x, n, nullptr, 0.0f, (uint32_t*)q,
                           d, s);
    return check_launch("quantize_q8");
}

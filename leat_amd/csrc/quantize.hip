// Activations to int8 in groups of 32, as llama.cpp's q8_1 and leat's quantize_q8
// (leat/kernels/quantize.py:25-109; oracle tests/test_kernels.py:28-36): per group
// d = max|x| / 127, q = roundf(x / d) (both divisions IEEE, rounding half away from zero, q = 0
// where d = 0), s = d * sum(q); q packed four per int32 word, byte i of word w being value 4w+i.
// Optionally after RMSNorm with a weight: x * (1 / sqrt(mean(x^2) + eps)) * weight, in f32.
//
// A block of 256 threads per 1024 values of a row (a grid of rows x parts, so a decode step's
// few rows still spread over many CUs); each thread takes 4 consecutive values, so the 8 lanes
// of an aligned octet hold one group and reduce it with DPP moves (quantize4).
#include "q8.h"

namespace leat {

template <bool NORM>
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x, int n,
                                                          const float* __restrict__ weight, float eps,
                                                          uint32_t* __restrict__ q, float* __restrict__ d,
                                                          float* __restrict__ s) {
    // block (row, part): values [1024 part, 1024 part + 1024) of the row; with the norm, every
    // block of the row sums the whole row's squares (from L2 after the first)
    __shared__ float partial[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)row * n;
    const float inv = NORM ? block_inv_rms(xr, n, eps, partial) : 1.0f;
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
    float dv, sv;
    const uint32_t word = quantize4(v, &dv, &sv);
    const int64_t first = (int64_t)row * n + at;
    q[first / 4] = word;
    if ((tid & 7) == 0) {
        d[first / GROUP] = dv;
        s[first / GROUP] = sv;
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

// The next token of a greedy decode step (leat/kernels/argmax.py:14-45): the index of the
// largest value in each row of logits, the lowest index among equal values, NaN never chosen
// (a row of NaN and -inf gives 0). Two launches: ARGMAX_PARTS workgroups per row each reduce a
// slice (lanes striding through it, so loads coalesce) to one (value, index) in the workspace,
// then a wave per row reduces the parts.
#include "common.h"

namespace leat {

constexpr int ARGMAX_PARTS = 64;  // workgroups per row: a 128256-value row is 2004 values each

// keep the larger value, and on equal values the lower index
__device__ __forceinline__ void argmax_step(float& best, int& index, float value, int at) {
    if (value > best || (value == best && at < index)) best = value, index = at;
}

__device__ __forceinline__ void wave_argmax(float& best, int& index) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) argmax_step(best, index, __shfl_xor(best, m, WAVE), __shfl_xor(index, m, WAVE));
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ x, int n, float* __restrict__ values,
                                                             int* __restrict__ indices) {
    __shared__ float wb[4];
    __shared__ int wi[4];
    const int row = blockIdx.y, part = blockIdx.x;
    const int per = (n + ARGMAX_PARTS - 1) / ARGMAX_PARTS, first = part * per, last = min(n, first + per);
    const float* xr = x + (int64_t)row * n;
    float best = -INFINITY;
    int index = 0;
    for (int at = first + (int)threadIdx.x; at < last; at += 256) argmax_step(best, index, xr[at], at);
    wave_argmax(best, index);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) wb[w] = best, wi[w] = index;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int v = 1; v < 4; v++) argmax_step(best, index, wb[v], wi[v]);
        values[row * ARGMAX_PARTS + part] = best;
        indices[row * ARGMAX_PARTS + part] = index;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ values, const int* __restrict__ indices,
                                                          int32_t* __restrict__ out) {
    const int row = blockIdx.x, lane = threadIdx.x;
    float best = -INFINITY;
    int index = 0;
    for (int p = lane; p < ARGMAX_PARTS; p += WAVE)
        argmax_step(best, index, values[row * ARGMAX_PARTS + p], indices[row * ARGMAX_PARTS + p]);
    wave_argmax(best, index);
    if (lane == 0) out[row] = index;
}

}  // namespace leat

using namespace leat;

extern "C" int64_t leat_argmax_workspace(int rows) { return (int64_t)rows * ARGMAX_PARTS * 8; }

extern "C" int leat_argmax(const float* x, int rows, int n, void* workspace, int64_t workspace_bytes, int32_t* out,
                           void* stream) {
    LEAT_REQUIRE(x && workspace && out, "argmax: null pointer");
    LEAT_REQUIRE(rows >= 0 && rows <= 65535 && n > 0, "argmax: %d rows of %d values", rows, n);
    LEAT_REQUIRE(workspace_bytes >= leat_argmax_workspace(rows), "argmax: a workspace of %lld bytes (needs %lld)",
                 (long long)workspace_bytes, (long long)leat_argmax_workspace(rows));
    if (rows == 0) return 0;
    float* values = (float*)workspace;
    int* indices = (int*)(values + (int64_t)rows * ARGMAX_PARTS);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(ARGMAX_PARTS, rows), dim3(256), 0, st, x, n, values, indices);
    if (check_launch("argmax")) return -1;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, st, values, indices, out);
    return check_launch("argmax final");
}

// Router scores of a mixture of experts (leat/kernels/experts.py:44-124, `scores`): for each
// token t and expert e, (sum_i x[t,i] * weight[i] * router[e,i]) / sqrt(mean(x[t]^2) + eps), in
// f32, from an F32 router matrix (experts, dim). leat scores in f32 rather than through the
// quantized products because the top-k choice is sensitive to rounding.
//
// A workgroup of 4 waves per (token, 4 experts): the workgroup sums the token's squares once
// (the quantizer's block_inv_rms), then each wave streams one router row against x * weight with
// 16-byte loads and reduces by DPP. x and the weight stay in L2 across the grid; the router
// (1 MB for 128 x 2048) is read once per token.
#include "q8.h"

namespace leat {

constexpr int SCORES_WAVES = 4;

__global__ __launch_bounds__(SCORES_WAVES * 64) void scores_kernel(const float* __restrict__ x, int dim,
                                                                   const float* __restrict__ weight, float eps,
                                                                   const float* __restrict__ router, int experts,
                                                                   float* __restrict__ out) {
    __shared__ float partial[4];
    const int t = blockIdx.y;
    const float* xr = x + (int64_t)t * dim;
    const float inv = block_inv_rms(xr, dim, eps, partial);
    const int lane = threadIdx.x & (WAVE - 1);
    const int e = blockIdx.x * SCORES_WAVES + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (e >= experts) return;
    const float* rr = router + (int64_t)e * dim;
    float acc = 0.0f;
    for (int at = lane * 4; at < dim; at += 4 * WAVE) {
        const float4 xv = *(const float4*)(xr + at), wv = *(const float4*)(weight + at);
        const float4 rv = *(const float4*)(rr + at);
        acc += xv.x * wv.x * rv.x;
        acc += xv.y * wv.y * rv.y;
        acc += xv.z * wv.z * rv.z;
        acc += xv.w * wv.w * rv.w;
    }
    const float dot = wave_sum_dpp(acc);
    if (lane == 0) out[(int64_t)t * experts + e] = dot * inv;
}

}  // namespace leat

using namespace leat;

extern "C" int leat_scores(const float* x, int tokens, int dim, const float* norm_weight, float eps,
                           const float* router, int experts, float* out, void* stream) {
    LEAT_REQUIRE(x && norm_weight && router && out, "scores: null pointer");
    LEAT_REQUIRE(tokens >= 0 && tokens <= 65535, "scores: %d tokens (at most 65535)", tokens);
    LEAT_REQUIRE(dim > 0 && dim % 4 == 0, "scores: rows of %d values are not whole 16-byte loads", dim);
    LEAT_REQUIRE(experts > 0, "scores: %d experts", experts);
    LEAT_REQUIRE(((uintptr_t)x | (uintptr_t)norm_weight | (uintptr_t)router) % 16 == 0,
                 "scores: x, the norm weight and the router must be 16-byte aligned");
    if (tokens == 0) return 0;
    const dim3 grid((experts + SCORES_WAVES - 1) / SCORES_WAVES, tokens);
    hipLaunchKernelGGL(scores_kernel, grid, dim3(SCORES_WAVES * 64), 0, (hipStream_t)stream, x, dim, norm_weight, eps,
                       router, experts, out);
    return check_launch("scores");
}

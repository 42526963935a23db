// Mixtures of experts on the decode kernels' tasks (leat/kernels/experts.py:132-172, 209-270):
// routing, the chosen experts' gate and up products with the GLU, and the weighted sum of their
// down products.
//
// route: a wave per token, `used` rounds of wave argmax over the experts' scores (ties to the
//   lower id; -inf and NaN count as the least finite score, below which a taken winner drops),
//   then the softmax of the winners.
// experts_glu: a wave per (pair, row of the expert). Pairs routed to one expert are served by the
//   wave of the first of them, which reads the expert's row once for all of their tokens (at most
//   one pair a token per expert); the others' waves exit. So every chosen expert's rows are read
//   once per launch, whatever the number of tokens sharing it.
// experts_down: a wave per (token, row of the output). Its lanes take (slot, task) items across the
//   token's `used` experts and sum weight * (row . hidden of the pair) (+ the row's bias), so the
//   sum over slots stays inside one wave, in a fixed order, with no atomics.
#include <cfloat>

#include "blocks.h"

namespace leat {

constexpr float LOG2E = 1.4426950408889634f;

// ------------------------------------------------------------------------------------- route

// EPL experts per lane: experts <= 64 EPL
template <int EPL>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ scores, int tokens, int experts,
                                                    int used, int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (t >= tokens) return;
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + WAVE * i;
        const float s = e < experts ? scores[(int64_t)t * experts + e] : -INFINITY;
        // -inf and NaN as the least finite value; lanes past the experts below every score
        v[i] = e < experts ? (s > -FLT_MAX ? s : -FLT_MAX) : -INFINITY;
    }
    float my_top = -INFINITY;
    int my_id = 0;
    for (int round = 0; round < used; round++) {
        float best = v[0];
        int index = lane;
#pragma unroll
        for (int i = 1; i < EPL; i++)  // ascending ids: strictly greater keeps the lower on ties
            if (v[i] > best) best = v[i], index = lane + WAVE * i;
#pragma unroll
        for (int off = WAVE / 2; off > 0; off >>= 1) {
            const float ob = __shfl_xor(best, off);
            const int oi = __shfl_xor(index, off);
            if (ob > best || (ob == best && oi < index)) best = ob, index = oi;
        }
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (lane + WAVE * i == index) v[i] = -INFINITY;  // taken: below every remaining score
        if (lane == round) my_top = best, my_id = index;
    }
    // softmax of the winners, relative to the first (largest): exp2((top - top0) * log2 e), summed
    // in rounds' order (leat/kernels/experts.py:154-159)
    const float top0 = __shfl(my_top, 0);
    const float e = lane < used ? exp2f((my_top - top0) * LOG2E) : 0.0f;
    float total = __shfl(e, 0);
    for (int r = 1; r < used; r++) total += __shfl(e, r);
    if (lane < used) {
        ids[(int64_t)t * used + lane] = my_id;
        weights[(int64_t)t * used + lane] = e / total;
    }
}

// -------------------------------------------------------------------------------- experts_glu

struct ExpertsGluArgs {
    const uint8_t* gate;
    const uint8_t* up;
    int64_t stride;  // rows per expert in the gate (and up) storage: 2 rows when gate stacks both
    int up_first;    // the first up row within an expert's rows: rows when stacked, else 0
    int experts, rows, cols, used, pairs;
    const int32_t* xq;
    const float* xd;
    const float* xs;
    const int32_t* ids;
    const float* gate_bias;  // experts * rows, or null
    const float* up_bias;
    int kind;
    float* out;  // pairs * rows
};

__device__ __forceinline__ int expert_of(const int32_t* ids, int p, int experts) {
    return (int)min((unsigned)ids[p], (unsigned)(experts - 1));  // an id out of range reads the last
}

// C pairs at once (members m[0..n), the rest repeating m[0], computed and dropped)
template <int TYPE, int C>
__device__ __forceinline__ void glu_rows(const ExpertsGluArgs& a, int e, int row, const int (&m)[C], int n, int lane) {
    using T = Task<TYPE>;
    const int tasks = a.cols / T::TASK_W;
    const int64_t grow = (int64_t)e * a.stride + row, urow = grow + a.up_first;
    float ag[C], au[C];
#pragma unroll
    for (int j = 0; j < C; j++) ag[j] = au[j] = 0.0f;
    for (int task = lane; task < tasks; task += WAVE) {
        const typename T::Raw rg = T::load(a.gate, grow, a.cols, task);
        const typename T::Raw ru = T::load(a.up, urow, a.cols, task);
        const typename T::Dec dg = T::decode(rg, task), du = T::decode(ru, task);
#pragma unroll
        for (int j = 0; j < C; j++) {
            const ActQ x = load_act<TYPE>(a.xq, a.xd, a.xs, a.cols, m[j] / a.used, task);
            ag[j] += T::combine(dg, x, T::dots(dg, x));
            au[j] += T::combine(du, x, T::dots(du, x));
        }
    }
#pragma unroll
    for (int j = 0; j < C; j++) {
        ag[j] = wave_sum(ag[j]);
        au[j] = wave_sum(au[j]);
    }
    if (lane == 0) {
        const float gb = a.gate_bias ? a.gate_bias[(int64_t)e * a.rows + row] : 0.0f;
        const float ub = a.up_bias ? a.up_bias[(int64_t)e * a.rows + row] : 0.0f;
#pragma unroll
        for (int j = 0; j < C; j++)
            if (j < n) a.out[(int64_t)m[j] * a.rows + row] = glu(a.kind, ag[j] + gb, au[j] + ub);
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void experts_glu_kernel(ExpertsGluArgs a) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE;
    const int p = blockIdx.y;
    if (row >= a.rows) return;
    const int e = expert_of(a.ids, p, a.experts);
    // the first pair routed to e serves them all
    for (int base = 0; base < p; base += WAVE) {
        const int q = base + lane;
        if (__ballot(q < p && expert_of(a.ids, q, a.experts) == e)) return;
    }
    constexpr int C = 4;
    int m[C], n = 0;
    for (int base = p; base < a.pairs; base += WAVE) {
        const int q = base + lane;
        uint64_t mask = __ballot(q < a.pairs && expert_of(a.ids, q, a.experts) == e);
        while (mask) {
            const int q = base + (int)__builtin_ctzll(mask);
#pragma unroll
            for (int j = 0; j < C; j++)  // m[n] = q, without indexing registers at run time
                if (j == n) m[j] = q;
            n++;
            mask &= mask - 1;
            if (n == C) {
                glu_rows<TYPE, C>(a, e, row, m, n, lane);
                n = 0;
            }
        }
    }
    if (n == 1) {
        const int one[1] = {m[0]};
        glu_rows<TYPE, 1>(a, e, row, one, 1, lane);
    } else if (n > 1) {
#pragma unroll
        for (int j = 1; j < C; j++)
            if (j >= n) m[j] = m[0];
        glu_rows<TYPE, C>(a, e, row, m, n, lane);
    }
}

// ------------------------------------------------------------------------------- experts_down

struct ExpertsDownArgs {
    const uint8_t* w;
    int experts, rows, cols, used, tokens;
    const int32_t* hq;  // pairs' hidden activations, quantized: tokens * used rows of cols
    const float* hd;
    const float* hs;
    const int32_t* ids;
    const float* weights;
    const float* scales;    // experts, or null
    const float* bias;      // experts * rows, or null
    const float* residual;  // tokens * rows, or null
    float* out;             // tokens * rows
};

template <int TYPE>
__global__ __launch_bounds__(256) void experts_down_kernel(ExpertsDownArgs a) {
    using T = Task<TYPE>;
    const int lane = threadIdx.x & (WAVE - 1);
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE;
    const int t = blockIdx.y;
    if (row >= a.rows) return;
    const int tasks = a.cols / T::TASK_W, items = a.used * tasks;
    float acc = 0.0f;
    for (int it = lane; it < items; it += WAVE) {
        const int slot = it / tasks, task = it - slot * tasks;
        const int p = t * a.used + slot;
        const int e = expert_of(a.ids, p, a.experts);
        float weight = a.weights[p];
        if (a.scales) weight *= a.scales[e];
        const typename T::Dec d = T::decode(T::load(a.w, (int64_t)e * a.rows + row, a.cols, task), task);
        const ActQ x = load_act<TYPE>(a.hq, a.hd, a.hs, a.cols, p, task);
        float v = T::combine(d, x, T::dots(d, x));
        if (a.bias && task == 0) v += a.bias[(int64_t)e * a.rows + row];
        acc += weight * v;
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        const int64_t at = (int64_t)t * a.rows + row;
        a.out[at] = a.residual ? acc + a.residual[at] : acc;
    }
}

}  // namespace leat

using namespace leat;

extern "C" int leat_route(const float* scores, int tokens, int experts, int used, int32_t* ids, float* weights,
                          void* stream) {
    LEAT_REQUIRE(scores && ids && weights, "route: null pointer");
    LEAT_REQUIRE(experts > 0 && experts <= 4 * WAVE, "route: %d experts (1..256 supported)", experts);
    LEAT_REQUIRE(used > 0 && used <= experts && used <= WAVE, "route: %d of %d experts", used, experts);
    LEAT_REQUIRE(tokens >= 0, "route: %d tokens", tokens);
    if (tokens == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((tokens + 3) / 4);
    if (experts <= WAVE)
        hipLaunchKernelGGL(route_kernel<1>, grid, dim3(256), 0, st, scores, tokens, experts, used, ids, weights);
    else if (experts <= 2 * WAVE)
        hipLaunchKernelGGL(route_kernel<2>, grid, dim3(256), 0, st, scores, tokens, experts, used, ids, weights);
    else
        hipLaunchKernelGGL(route_kernel<4>, grid, dim3(256), 0, st, scores, tokens, experts, used, ids, weights);
    return check_launch("route");
}

extern "C" int leat_experts_glu(int type, const void* gate, const void* up, int experts, int rows, int cols,
                                const int32_t* xq, const float* xd, const float* xs, const int32_t* ids, int pairs,
                                int used, const float* gate_bias, const float* up_bias, int kind, float* out,
                                void* stream) {
    LEAT_REQUIRE(gate && xq && xd && xs && ids && out, "experts_glu: null pointer");
    LEAT_REQUIRE(experts > 0 && rows > 0 && used > 0, "experts_glu: empty experts");
    LEAT_REQUIRE(pairs >= 0 && pairs % used == 0 && pairs <= 65535, "experts_glu: %d pairs of %d", pairs, used);
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "experts_glu: unknown GLU kind %d", kind);
    if (check_cols(type, cols) || check_ptrs(type, gate, xq) || (up && check_ptrs(type, up, nullptr))) return -1;
    if (pairs == 0) return 0;
    ExpertsGluArgs a = {};
    a.gate = (const uint8_t*)gate;
    a.up = (const uint8_t*)(up ? up : gate);
    a.stride = up ? rows : 2 * (int64_t)rows;
    a.up_first = up ? 0 : rows;
    a.experts = experts, a.rows = rows, a.cols = cols, a.used = used, a.pairs = pairs;
    a.xq = xq, a.xd = xd, a.xs = xs, a.ids = ids;
    a.gate_bias = gate_bias, a.up_bias = up_bias;
    a.kind = kind, a.out = out;
    const dim3 grid((rows + 3) / 4, pairs);
    hipStream_t st = (hipStream_t)stream;
    switch (type) {
    case Q4_K: hipLaunchKernelGGL(experts_glu_kernel<Q4_K>, grid, dim3(256), 0, st, a); break;
    case Q6_K: hipLaunchKernelGGL(experts_glu_kernel<Q6_K>, grid, dim3(256), 0, st, a); break;
    case Q8_0: hipLaunchKernelGGL(experts_glu_kernel<Q8_0>, grid, dim3(256), 0, st, a); break;
    }
    return check_launch("experts_glu");
}

extern "C" int leat_experts_down(int type, const void* w, int experts, int rows, int cols, const int32_t* hq,
                                 const float* hd, const float* hs, const int32_t* ids, const float* weights,
                                 int tokens, int used, const float* scales, const float* bias, const float* residual,
                                 float* out, void* stream) {
    LEAT_REQUIRE(w && hq && hd && hs && ids && weights && out, "experts_down: null pointer");
    LEAT_REQUIRE(experts > 0 && rows > 0 && used > 0, "experts_down: empty experts");
    LEAT_REQUIRE(tokens >= 0 && tokens <= 65535, "experts_down: %d tokens", tokens);
    if (check_cols(type, cols) || check_ptrs(type, w, hq)) return -1;
    if (tokens == 0) return 0;
    ExpertsDownArgs a = {};
    a.w = (const uint8_t*)w;
    a.experts = experts, a.rows = rows, a.cols = cols, a.used = used, a.tokens = tokens;
    a.hq = hq, a.hd = hd, a.hs = hs, a.ids = ids, a.weights = weights;
    a.scales = scales, a.bias = bias, a.residual = residual, a.out = out;
    const dim3 grid((rows + 3) / 4, tokens);
    hipStream_t st = (hipStream_t)stream;
    switch (type) {
    case Q4_K: hipLaunchKernelGGL(experts_down_kernel<Q4_K>, grid, dim3(256), 0, st, a); break;
    case Q6_K: hipLaunchKernelGGL(experts_down_kernel<Q6_K>, grid, dim3(256), 0, st, a); break;
    case Q8_0: hipLaunchKernelGGL(experts_down_kernel<Q8_0>, grid, dim3(256), 0, st, a); break;
    }
    return check_launch("experts_down");
}

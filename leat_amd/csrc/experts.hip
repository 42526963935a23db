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
//   sum over slots stays inside one wave, in a fixed order, with no atomics. The slots' experts and
//   weights are read once a wave (lane s: slot s); for one or two tokens each lane has the loads of
//   4 items in flight together before it sums them.
#include <cfloat>

#include "blocks.h"
#include "q8.h"
#include "rowtask.h"

namespace leat {

constexpr float LOG2E = 1.4426950408889634f;

// ------------------------------------------------------------------------------------- route

// Routes one token's scores (experts <= 64 EPL, used <= 64) on one wave: `used` rounds of wave
// argmax (ties to the lower id; -inf and NaN count as the least finite score, below which a taken
// winner drops), then the softmax of the winners. Lane r < used gets round r's winner and weight.
template <int EPL>
__device__ __forceinline__ void route_token(const float* __restrict__ row, int experts, int used, int lane, int* id,
                                            float* weight) {
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + WAVE * i;
        const float s = e < experts ? row[e] : -INFINITY;
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
        // the wave's maximum, then the lowest id holding it: two DPP reductions (no LDS round
        // trips); a taken winner (-inf) never ties an untaken score (at least -FLT_MAX)
        const float top = wave_max_dpp(best);
        const int winner = wave_min_dpp(best == top ? index : 0x7FFFFFFF);
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (lane + WAVE * i == winner) v[i] = -INFINITY;  // taken: below every remaining score
        if (lane == round) my_top = top, my_id = winner;
    }
    // softmax of the winners, relative to the first (largest): exp2((top - top0) * log2 e), summed
    // in rounds' order (leat/kernels/experts.py:154-159)
    const float top0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_top), 0));
    const float e = lane < used ? exp2f((my_top - top0) * LOG2E) : 0.0f;
    float total = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), 0));
    for (int r = 1; r < used; r++) total += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), r));
    *id = my_id;
    *weight = e / total;
}

// a wave per token
template <int EPL>
__global__ __launch_bounds__(256) void route_kernel(const float* scores, int tokens, int experts, int used,
                                                    int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (t >= tokens) return;
    int id;
    float weight;
    route_token<EPL>(scores + (int64_t)t * experts, experts, used, lane, &id, &weight);
    if (lane < used) {
        ids[(int64_t)t * used + lane] = id;
        weights[(int64_t)t * used + lane] = weight;
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

// ------------------------------------------------------------------ fused decode GLU (1..8 tokens)

// The first steps of a decode mixture in one launch (leat/kernels/experts.py:341-377: route,
// quantize_q8 of rms_norm(x), experts_swiglu, quantize_q8 of the hidden rows). A workgroup owns
// 32 (or 64) rows of the expert of pair p = blockIdx.y (token p / used), so an expert chosen by k tokens
// is read k times: each pair's rows are streamed by workgroups of their own, which lets more
// of them run at once than sharing a pass between members does.
// 1. threads 0..255 load the token's x (and the norm weight) into registers before anything
//    else, so that its norm and quantization never wait behind the weight loads;
// 2. wave 0 routes the pair's token (route_token, the routing kernel's arithmetic) into LDS, and
//    the first row tile of each token's first pair publishes its ids and weights for the down
//    product (routing every token in every workgroup cost 5.7 us of a B=8 launch);
// 3. its waves issue the loads of their rows (lanes own the same tasks of every row, as in the
//    row-streaming matvec kernels, RowTask), then the workgroup normalizes and quantizes x into
//    LDS with the standalone quantizer's arithmetic (q8.h);
// 4. each wave streams 2 (or 8) rows of gate and up against the activations in registers;
// 5. every 32 rows are one group of 32, so the workgroup writes the hidden rows' q8 words, d and
//    s as well as (optionally) their f32 values.
// Workgroups of MOE_TILE rows in MOE_WAVES waves, 2 rows a wave; for launches of at least
// MOE_WIDE_PAIRS pairs, whose many workgroups then share out each one's routing and quantization
// over twice the weights, MOE_WIDE_TILE rows in MOE_WIDE_WAVES waves, 8 a wave. Measured at
// Qwen3-30B-A3B's shape: 16 waves took the B=1 launch from 10.5 to 10.2 us and the B=8 one from
// 24.0 to 25.9 us, hence the two widths.
constexpr int MOE_WAVES = 16, MOE_TILE = 32, MOE_MAX_TOKENS = 8, MOE_MAX_USED = 64;
constexpr int MOE_WIDE_TILE = 64, MOE_WIDE_WAVES = 8, MOE_WIDE_PAIRS = 32;

struct MoeGluArgs {
    const uint8_t* gate;
    const uint8_t* up;
    int64_t stride;  // rows per expert in the gate (and up) storage: 2 rows when gate stacks both
    int up_first;    // the first up row within an expert's rows: rows when stacked, else 0
    int experts, rows, cols, used, tokens;
    const float* x;  // tokens * cols
    const float* norm;
    float eps;
    const float* scores;  // tokens * experts
    const float* gate_bias;
    const float* up_bias;
    int kind;
    int32_t* ids;  // tokens * used, written
    float* weights;
    float* out;  // pairs * rows, or null
    uint32_t* hq;
    float* hd;
    float* hs;
};

template <int TYPE, int NT, int EPL, int TILE, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void moe_glu_kernel(MoeGluArgs a) {
    using RT = RowTask<TYPE>;
    constexpr int RPW = TILE / WAVES;
    // rows of loads in flight: all of a narrow tile's; one of a wide tile's, whose launches of many
    // pairs keep more waves resident instead (measured fastest at 8 tokens of top-8)
    constexpr int P = NT == 1 ? (TILE == MOE_TILE ? RPW : 1) : NT == 2 ? 2 : 1;
    extern __shared__ uint32_t moe_lds[];  // the token's q8 row: words, then d, then s
    __shared__ int route_id[MOE_MAX_USED];
    __shared__ float route_w[MOE_MAX_USED];
    __shared__ float partial[WAVES];
    __shared__ __align__(16) float glu_out[TILE];  // float4 reads by the q8 epilogue

    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int p = blockIdx.y, row_base = blockIdx.x * TILE;
    const int cols = a.cols, used = a.used;

    // 1. the token's x, first in every wave's queue of loads (up to 8192 values: longer rows
    // would spill the registers, and load theirs after the weights)
    constexpr int NX = NT * Task<TYPE>::TASK_W / 16;
    constexpr bool EARLY_X = NX <= 8;
    const float* xr = a.x + (int64_t)(p / used) * cols;
    RowsInRegs<1, EARLY_X ? NX : 1> xin;
    if (EARLY_X) xin.load(xr, a.norm, cols);

    // 2. routing of the pair's token
    const int token = p / used, slot = p - token * used;
    if (w == 0) {
        int id;
        float weight;
        route_token<EPL>(a.scores + (int64_t)token * a.experts, a.experts, used, lane, &id, &weight);
        if (lane < used) route_id[lane] = id, route_w[lane] = weight;
    }
    __syncthreads();
    if (blockIdx.x == 0 && slot == 0 && (int)threadIdx.x < used) {
        a.ids[(int64_t)token * used + threadIdx.x] = route_id[threadIdx.x];
        a.weights[(int64_t)token * used + threadIdx.x] = route_w[threadIdx.x];
    }
    const int e = route_id[slot];  // route_token ids are always below `experts`

    // 3. the rows' loads, then the token's activations
    const int row0 = row_base + w;  // the wave's rows: row0 + 8r
    const uint32_t row_bytes = (uint32_t)(cols / Task<TYPE>::WEIGHTS) * Task<TYPE>::BYTES;
    const typename RT::Off off = RT::at(lane);
    const int tasks = cols / Task<TYPE>::TASK_W;
    bool has[NT];  // the lane's task i lies in the row (a last partial turn leaves lanes idle)
#pragma unroll
    for (int i = 0; i < NT; i++) has[i] = lane + WAVE * i < tasks;
    const uint8_t* g_at = a.gate + (size_t)(e * a.stride) * row_bytes;
    const uint8_t* u_at = a.up + (size_t)(e * a.stride + a.up_first) * row_bytes;
    typename RT::Raw rg[P][NT], ru[P][NT];
    auto fetch = [&](int slot, int r) {
        const uint32_t at = (uint32_t)min(row0 + WAVES * r, a.rows - 1) * row_bytes;
#pragma unroll
        for (int i = 0; i < NT; i++)
            if (has[i]) {
                rg[slot][i] = RT::load(g_at + at + RT::STRIDE * i, off);
                ru[slot][i] = RT::load(u_at + at + RT::STRIDE * i, off);
            }
    };
#pragma unroll
    for (int r = 0; r < P; r++) fetch(r, r);
    float* lds_d = (float*)(moe_lds + cols / 4);
    if constexpr (EARLY_X) {
        xin.template quantize<WAVES * 64>(0, a.norm, a.eps, cols, partial, moe_lds, lds_d, lds_d + cols / GROUP);
    } else {
        const float inv = a.norm ? block_inv_rms<WAVES * 64>(xr, cols, a.eps, partial) : 1.0f;
        quantize_row<WAVES * 64>(xr, cols, a.norm, inv, moe_lds, lds_d, lds_d + cols / GROUP);
    }
    __syncthreads();
    ActQ act[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) act[i] = RT::act(load_act_lds<TYPE>(moe_lds, 1, cols, 0, has[i] ? lane + WAVE * i : 0), lane);

    // 4. the rows
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int row = row0 + WAVES * r;
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int i = 0; i < NT; i++)
            if (has[i]) {
                g += RT::dot(rg[r % P][i], off, act[i]);
                u += RT::dot(ru[r % P][i], off, act[i]);
            }
        if (r + P < RPW) fetch(r % P, r + P);
        const float gb = a.gate_bias && row < a.rows ? a.gate_bias[(int64_t)e * a.rows + row] : 0.0f;
        const float ub = a.up_bias && row < a.rows ? a.up_bias[(int64_t)e * a.rows + row] : 0.0f;
        const float y = glu(a.kind, wave_sum_dpp(g) + gb, wave_sum_dpp(u) + ub);
        if (lane == 0) {
            glu_out[w + WAVES * r] = y;
            if (a.out && row < a.rows) a.out[(int64_t)p * a.rows + row] = y;
        }
    }

    // 5. the outputs quantized in groups of 32 (rows a multiple of TILE): an aligned octet of
    // threads a group, a float4 a thread (quantize4: DPP moves only)
    if (!a.hq) return;
    __syncthreads();
    if ((int)threadIdx.x < TILE / 4) {
        const int i = threadIdx.x;
        float dv, sv;
        const uint32_t word = quantize4(((const float4*)glu_out)[i], &dv, &sv);
        const int64_t first = (int64_t)p * a.rows + row_base;  // the tile's first row: a group boundary
        a.hq[first / 4 + i] = word;
        if ((i & 7) == 0) {
            a.hd[first / GROUP + i / 8] = dv;
            a.hs[first / GROUP + i / 8] = sv;
        }
    }
}

template <int TYPE, int NT, int TILE, int WAVES>
static void moe_glu_tile(MoeGluArgs& a, hipStream_t st) {
    const dim3 grid(a.rows / TILE, a.tokens * a.used);
    const size_t lds = (size_t)a.cols + 2 * (size_t)(a.cols / GROUP) * 4;
    if (a.experts <= WAVE)
        hipLaunchKernelGGL((moe_glu_kernel<TYPE, NT, 1, TILE, WAVES>), grid, dim3(WAVES * 64), lds, st, a);
    else if (a.experts <= 2 * WAVE)
        hipLaunchKernelGGL((moe_glu_kernel<TYPE, NT, 2, TILE, WAVES>), grid, dim3(WAVES * 64), lds, st, a);
    else
        hipLaunchKernelGGL((moe_glu_kernel<TYPE, NT, 4, TILE, WAVES>), grid, dim3(WAVES * 64), lds, st, a);
}

template <int TYPE, int NT>
static void moe_glu_go(MoeGluArgs& a, hipStream_t st) {
    if (a.tokens * a.used >= MOE_WIDE_PAIRS && a.rows % MOE_WIDE_TILE == 0)
        return moe_glu_tile<TYPE, NT, MOE_WIDE_TILE, MOE_WIDE_WAVES>(a, st);
    moe_glu_tile<TYPE, NT, MOE_TILE, MOE_WAVES>(a, st);
}

template <int TYPE>
static void moe_glu_nt(MoeGluArgs& a, hipStream_t st) {
    // turns of a wave's 64 tasks, the last one possibly partial (has[] idles the lanes past it)
    const int turns = (a.cols / Task<TYPE>::TASK_W + WAVE - 1) / WAVE;
    if (turns <= 1) return moe_glu_go<TYPE, 1>(a, st);
    if (turns <= 2) return moe_glu_go<TYPE, 2>(a, st);
    return moe_glu_go<TYPE, 4>(a, st);
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

// U: items of a lane whose loads are in flight together (4 for 1-2 tokens, whose few waves leave
// registers to spare; 1 for more, whose waves fill the GPU at a higher occupancy)
template <int TYPE, int U>
__global__ __launch_bounds__(256) void experts_down_kernel(ExpertsDownArgs a) {
    using T = Task<TYPE>;
    const int lane = threadIdx.x & (WAVE - 1);
    const int row = blockIdx.x * 4 + threadIdx.x / WAVE;
    const int t = blockIdx.y;
    if (row >= a.rows) return;
    const int tasks = a.cols / T::TASK_W, items = a.used * tasks;
    // the token's experts and their weights, lane s holding slot s's (used <= 64), read once
    int slot_e = 0;
    float slot_w = 0.0f;
    if (lane < a.used) {
        const int p = t * a.used + lane;
        slot_e = expert_of(a.ids, p, a.experts);
        slot_w = a.weights[p];
        if (a.scales) slot_w *= a.scales[slot_e];
    }
    // items lane, lane + 64, ... in that order, U at a time: every load first, then the sums
    float acc = 0.0f;
    for (int base = lane; base < items; base += WAVE * U) {
        typename T::Raw raw[U];
        ActQ x[U];
        int task_of[U], e_of[U];
        float w_of[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int it = min(base + WAVE * u, items - 1);  // past the end: loads in range, sums dropped
            const int slot = it / tasks, task = it - slot * tasks;
            e_of[u] = __shfl(slot_e, slot);
            w_of[u] = __shfl(slot_w, slot);
            task_of[u] = task;
            raw[u] = T::load(a.w, (int64_t)e_of[u] * a.rows + row, a.cols, task);
            x[u] = load_act<TYPE>(a.hq, a.hd, a.hs, a.cols, t * a.used + slot, task);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (base + WAVE * u < items) {
                const typename T::Dec d = T::decode(raw[u], task_of[u]);
                float v = T::combine(d, x[u], T::dots(d, x[u]));
                if (a.bias && task_of[u] == 0) v += a.bias[(int64_t)e_of[u] * a.rows + row];
                acc += w_of[u] * v;
            }
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        const int64_t at = (int64_t)t * a.rows + row;
        a.out[at] = a.residual ? acc + a.residual[at] : acc;
    }
}

template <int TYPE>
static void experts_down_go(const dim3& grid, int tokens, hipStream_t st, const ExpertsDownArgs& a) {
    if (tokens <= 2)
        hipLaunchKernelGGL((experts_down_kernel<TYPE, 4>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((experts_down_kernel<TYPE, 1>), grid, dim3(256), 0, st, a);
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
    LEAT_REQUIRE(used <= WAVE, "experts_down: %d experts a token (1..%d)", used, WAVE);
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
    case Q4_K: experts_down_go<Q4_K>(grid, tokens, st, a); break;
    case Q6_K: experts_down_go<Q6_K>(grid, tokens, st, a); break;
    case Q8_0: experts_down_go<Q8_0>(grid, tokens, st, a); break;
    }
    return check_launch("experts_down");
}

extern "C" int leat_experts_glu_f32(int type, const void* gate, const void* up, int experts, int rows, int cols,
                                    const float* x, int tokens, const float* norm_weight, float eps,
                                    const float* scores, int used, const float* gate_bias, const float* up_bias,
                                    int kind, int32_t* ids, float* weights, float* out, int32_t* hq, float* hd,
                                    float* hs, void* stream) {
    LEAT_REQUIRE(gate && x && scores && ids && weights, "experts_glu_f32: null pointer");
    LEAT_REQUIRE(out || hq, "experts_glu_f32: neither f32 nor q8 output");
    LEAT_REQUIRE(tokens >= 1 && tokens <= MOE_MAX_TOKENS, "experts_glu_f32: %d tokens (1..%d)", tokens, MOE_MAX_TOKENS);
    LEAT_REQUIRE(experts > 0 && experts <= 4 * WAVE, "experts_glu_f32: %d experts (1..256 supported)", experts);
    LEAT_REQUIRE(used > 0 && used <= experts && used <= MOE_MAX_USED, "experts_glu_f32: %d of %d experts", used, experts);
    LEAT_REQUIRE(rows > 0 && rows % MOE_TILE == 0, "experts_glu_f32: rows %d not a multiple of %d", rows, MOE_TILE);
    LEAT_REQUIRE(!hq || (hd && hs), "experts_glu_f32: a q8 output needs d and s");
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "experts_glu_f32: unknown GLU kind %d", kind);
    // the row-streaming tasks: whole wave turns up to 4 (Q4_K rows of 256s, Q6_K of 512s: 4-byte
    // aligned rows), 16-byte aligned f32 rows
    const int tasks = type == Q8_0 ? cols / 64 : cols / 32;
    LEAT_REQUIRE((type == Q4_K && cols % 256 == 0) || (type == Q6_K && cols % 512 == 0) || (type == Q8_0 && cols % 64 == 0),
                 "experts_glu_f32: type %d, %d columns", type, cols);
    LEAT_REQUIRE(tasks <= 4 * WAVE, "experts_glu_f32: rows of %d weights (at most 4 turns of a wave's tasks)", cols);

    LEAT_REQUIRE((uintptr_t)x % 16 == 0 && (!norm_weight || (uintptr_t)norm_weight % 16 == 0),
                 "experts_glu_f32: f32 rows must be 16-byte aligned");
    if (check_ptrs(type, gate, nullptr) || (up && check_ptrs(type, up, nullptr))) return -1;
    MoeGluArgs a = {};
    a.gate = (const uint8_t*)gate;
    a.up = (const uint8_t*)(up ? up : gate);
    a.stride = up ? rows : 2 * (int64_t)rows;
    a.up_first = up ? 0 : rows;
    a.experts = experts, a.rows = rows, a.cols = cols, a.used = used, a.tokens = tokens;
    a.x = x, a.norm = norm_weight, a.eps = eps, a.scores = scores;
    a.gate_bias = gate_bias, a.up_bias = up_bias, a.kind = kind;
    a.ids = ids, a.weights = weights, a.out = out;
    a.hq = (uint32_t*)hq, a.hd = hd, a.hs = hs;
    hipStream_t st = (hipStream_t)stream;
    switch (type) {
    case Q4_K: moe_glu_nt<Q4_K>(a, st); break;
    case Q6_K: moe_glu_nt<Q6_K>(a, st); break;
    case Q8_0: moe_glu_nt<Q8_0>(a, st); break;
    }
    return check_launch("experts_glu_f32");
}

// Decode products for one or two tokens, streaming whole rows: y[t, row] = W[row] . x[t], the
// single-stream (and two-stream) case of leat's matvecs / swiglu (leat/kernels/matvec.py:306-395).
//
// Work split: lane l of a wave owns the same tasks of every row (tasks l, l + 64, ...; a task is
// 32 weights of Q4_K or Q6_K, 64 of Q8_0, as in blocks.h), so it loads its activation words and
// scales into registers once and reuses them for every row the wave streams. Rows of more than
// four turns of a wave's tasks (more than 8192 weights, up to 32768: 14336 has seven) are split by columns
// instead: each wave of a workgroup takes one turn of the same few rows (rows_split_kernel). A wave owns RPW
// consecutive rows (of each matrix of the launch: gate and up for the GLU) and walks them one at
// a time, the loads of the next rows (up to 4) in flight while the current row is computed. A row's sum
// is one wave-wide DPP reduction.
//
// Activations arrive either quantized (xq, xd, xs, as leat's quantize_q8 writes them) or as f32
// rows that each workgroup quantizes itself into LDS, with an optional RMSNorm, using the
// standalone quantizer's arithmetic (q8.h): bit for bit what quantize_q8 followed by the product
// gives, without the separate launch.
//
// The GLU can also quantize its own outputs for the down product that consumes them: a
// workgroup owns 32 consecutive rows (4 waves x 8), so each of its output groups of 32 is
// complete in the workgroup, and it writes their q8 words, d and s directly.
#include "blocks.h"
#include "q8.h"
#include "rows.h"
#include "rowtask.h"

namespace leat {

enum RowsMode : int { ROWS_PLAIN = 0, ROWS_RESIDUAL = 1, ROWS_GLU = 2 };

constexpr int ROWS_DEPTH = 1;  // rows of weight loads a wave has in flight, the one it computes next included

// FULL: the row's tasks fill exactly NT turns of the wave, so no lane needs a bounds check
// WPG waves per workgroup, RPW rows per wave: a workgroup owns a tile of WPG * RPW rows
template <int TYPE, int B, int NT, int RPW, int WPG, int MODE, bool XF32, bool FULL>
__global__ __launch_bounds__(WPG * 64) void rows_kernel(RowsArgs a) {
    using T = Task<TYPE>;
    using RT = RowTask<TYPE>;
    constexpr int NM = MODE == ROWS_GLU ? 2 : 1;
    extern __shared__ uint32_t rows_lds[];
    __shared__ float partial[WPG < 4 ? 4 : WPG];
    __shared__ __align__(16) float glu_out[B][32];  // float4 reads by the q8 epilogue

    const int cols = a.cols, tasks = cols / T::TASK_W;
    const int lane = threadIdx.x & (WAVE - 1);
    // the wave's number in the workgroup, known to the compiler as uniform so row addresses stay
    // scalar. A workgroup owns a tile of WPG * RPW consecutive rows of one matrix; its waves take
    // every WPG-th row (w, w + WPG, ...), so at each step the waves read adjacent rows
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int tile = blockIdx.x;
    int m = 0;
    if (MODE != ROWS_GLU)
        while (m + 1 < a.count && tile >= a.tile_start[m + 1]) m++;
    const int rows = a.rows[m];
    const int tile_row = (tile - a.tile_start[m]) * WPG * RPW;
    constexpr int STEP = WPG;
    const int row0 = tile_row + w;
    const uint32_t row_bytes = (uint32_t)(cols / T::WEIGHTS) * T::BYTES;
    const uint8_t* wm[NM];
    wm[0] = a.w[MODE == ROWS_GLU ? 0 : m];
    if (NM == 2) wm[NM - 1] = a.w[1];

    // the lane's tasks: lane + 64 i, each RT::STRIDE bytes past the previous in a row, so one set
    // of offsets (those of task `lane`) serves them all
    const typename RT::Off off = RT::at(lane);
    bool has[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) has[i] = FULL || lane + WAVE * i < tasks;

    // P rows' weights in flight at a time, the first P before the activations are ready
    constexpr int P = RPW < ROWS_DEPTH ? RPW : ROWS_DEPTH;
    typename RT::Raw buf[P][NM][NT];
    auto fetch = [&](typename RT::Raw(&dst)[NM][NT], int row) {
#pragma unroll
        for (int k = 0; k < NM; k++)
#pragma unroll
            for (int i = 0; i < NT; i++)
                if (has[i]) dst[k][i] = RT::load(wm[k] + (size_t)row * row_bytes + RT::STRIDE * i, off);
    };
    // f32 activations (and the norm weight) are asked for before the first rows, into registers.
    // The first rows' loads follow unconditionally (a wave past the last row reads the last row
    // again and uses nothing of it), so the compiler knows how many loads are still in flight
    // behind x's: the norm and quantization wait for x alone (vmcnt of the row loads, not zero)
    // and run while the rows arrive. Measured at B = 1 on the Llama-3-8B step: 1.33 ms against
    // 1.35 with the rows first or conditional fetches.
    constexpr bool EARLY_X = XF32;
    RowsInRegs<B, EARLY_X ? NT * T::TASK_W / 16 : 1> xin;
    if (EARLY_X) xin.load(a.x, a.norm, cols);
#pragma unroll
    for (int p = 0; p < P; p++) fetch(buf[p], min(row0 + STEP * p, rows - 1));

    // The activations, in registers
    if (XF32) {
        // the workgroup quantizes the tokens' rows into LDS: words, then d, then s
        const int words = B * (cols / 4), groups = B * (cols / GROUP);
        float* lds_d = (float*)(rows_lds + words);
#pragma unroll
        for (int t = 0; t < B; t++) {
            uint32_t* q = rows_lds + t * (cols / 4);
            float* d = lds_d + t * (cols / GROUP);
            float* s = lds_d + groups + t * (cols / GROUP);
            xin.template quantize<WPG * 64>(t, a.norm, a.eps, cols, partial, q, d, s);
        }
        __syncthreads();
    }
    auto fresh = [&](int i, int t, const uint32_t* lds) -> ActQ {
        const int task = has[i] ? lane + WAVE * i : 0;
        return XF32 ? load_act_lds<TYPE>(lds, B, cols, t, task)
                               : load_act<TYPE>(a.xq, a.xd, a.xs, cols, t, task);
    };
    ActQ act[NT][B];
#pragma unroll
    for (int i = 0; i < NT; i++)
#pragma unroll
        for (int t = 0; t < B; t++) act[i][t] = RT::act(fresh(i, t, rows_lds), lane);

    float keep[RPW][B];  // the GLU's outputs of the wave's rows, for the q8 epilogue
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int row = row0 + STEP * r;
        if (row >= rows) break;  // uniform across the wave
        float acc[NM][B];
#pragma unroll
        for (int k = 0; k < NM; k++)
#pragma unroll
            for (int t = 0; t < B; t++) acc[k][t] = 0.0f;
#pragma unroll
        for (int i = 0; i < NT; i++) {
            if (!has[i]) continue;
#pragma unroll
            for (int k = 0; k < NM; k++)
#pragma unroll
                for (int t = 0; t < B; t++) acc[k][t] += RT::dot(buf[r % P][k][i], off, act[i][t]);
        }
        // the slot is free again: the row P further on
        if (r + P < RPW && row + STEP * P < rows) fetch(buf[r % P], row + STEP * P);
#pragma unroll
        for (int t = 0; t < B; t++) {
            float y = wave_sum_dpp(acc[0][t]);
            if (MODE == ROWS_GLU) y = glu(a.kind, y, wave_sum_dpp(acc[NM - 1][t]));
            const int64_t at = (int64_t)t * rows + row;
            if (MODE == ROWS_RESIDUAL) y += a.residual[at];
            keep[r][t] = y;
            float* out = a.out[MODE == ROWS_GLU ? 0 : m];
            if (lane == 0 && out) out[at] = y;
        }
    }

    // q, k and v turned by RoPE and stored for attention (leat_qkv_rotate_f32): the workgroup's
    // 16 rows are 8 whole pairs of adjacent dimensions of one head (dim a multiple of 16), staged
    // in LDS and handed to a thread a (token, pair)
    if (MODE == ROWS_PLAIN && a.rope.q_out) {
        constexpr int TILE = WPG * RPW, PAIRS = TILE / 2;
        static_assert(TILE % 2 == 0 && TILE <= 32, "whole pairs in the staging rows");
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int t = 0; t < B; t++)
                if (lane == r) glu_out[t][row0 - tile_row + STEP * r] = keep[r][t];
        __syncthreads();
        if ((int)threadIdx.x < B * PAIRS) {
            const RopeStore& rp = a.rope;
            const int t = threadIdx.x / PAIRS, j = threadIdx.x % PAIRS;
            const int pos = rp.positions[t], slot = rp.slots[t];
            // a position or slot outside the cache stores nothing, as leat_rotate
            if (pos >= 0 && pos < rp.cache_positions && slot >= 0 && slot < rp.cache_slots) {
                const int rr = tile_row + 2 * j, head = rr / rp.dim, d0 = rr - head * rp.dim, i = d0 / 2;
                const int half = rp.rotated / 2;
                float x0 = glu_out[t][2 * j], x1 = glu_out[t][2 * j + 1];
                if (m < 2 && i < half) rope_pair(x0, x1, rp.cos[(int64_t)pos * half + i], rp.sin[(int64_t)pos * half + i]);
                if (m == 0) {
                    float* o = rp.q_out + ((int64_t)head * B + t) * rp.dim + d0;
                    o[0] = x0, o[1] = x1;
                } else {
                    const int64_t values = m == 2 ? (int64_t)rp.cache_slots * rp.kv_heads * rp.cache_positions * rp.dim : 0;
                    const int64_t at = values + (((int64_t)slot * rp.kv_heads + head) * rp.cache_positions + pos) * rp.dim + d0;
                    rp.cache[at] = (_Float16)x0;
                    rp.cache[at + 1] = (_Float16)x1;
                }
            }
        }
    }

    // the GLU's own outputs quantized: the workgroup's 32 rows are one group per token
    if (MODE == ROWS_GLU && WPG * RPW == 32 && a.hq) {
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int t = 0; t < B; t++)
                if (lane == r) glu_out[t][row0 - tile_row + STEP * r] = keep[r][t];
        __syncthreads();
        store_group_q8<B>(glu_out, a.rows[0], tile, a.hq, a.hd, a.hs);
    }
}

// Long rows (more than 4 turns of a wave's tasks, up to 16: Q6_K or Q4_K rows of more than 8192
// weights, up to 32768, such as 11008, 13824, 14336, 18944) split by columns: wave w of the KS waves of a
// workgroup takes turn w of every row, tasks 64w + lane (a last turn may be partial, and waves past
// the row's turns idle), so each lane holds one task's activations and streams the workgroup's R
// rows with P of them in flight; the waves' partial sums of a row meet in LDS and are added in
// wave order.
template <int TYPE, int B, int KS, int R, int P, int MODE, bool FULL>
__global__ __launch_bounds__(KS * 64) void rows_split_kernel(RowsArgs a) {
    using RT = RowTask<TYPE>;
    static_assert(P <= R, "rows in flight");
    __shared__ float part[KS][B][R];
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int cols = a.cols, rows = a.rows[0], row0 = blockIdx.x * R;
    const uint32_t row_bytes = (uint32_t)(cols / Task<TYPE>::WEIGHTS) * Task<TYPE>::BYTES;
    const int task = WAVE * w + lane;
    const bool has = FULL || task < cols / Task<TYPE>::TASK_W;  // the lane's task lies in the row (FULL: KS whole turns)
    const typename RT::Off off = RT::at(has ? task : 0);

    typename RT::Raw buf[P]{};  // lanes past the row's tasks keep zeros and add nothing
    auto fetch = [&](typename RT::Raw& dst, int row) {
        if (has) dst = RT::load(a.w[0] + (size_t)min(row, rows - 1) * row_bytes, off);  // rows past the end: never stored
    };
#pragma unroll
    for (int p = 0; p < P; p++) fetch(buf[p], row0 + p);
    ActQ act[B];
#pragma unroll
    for (int t = 0; t < B; t++) act[t] = RT::act(load_act<TYPE>(a.xq, a.xd, a.xs, cols, t, has ? task : 0), lane);

    float sum[B][R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float acc[B];
#pragma unroll
        for (int t = 0; t < B; t++) acc[t] = has ? RT::dot(buf[r % P], off, act[t]) : 0.0f;
        if (r + P < R) fetch(buf[r % P], row0 + r + P);
#pragma unroll
        for (int t = 0; t < B; t++) sum[t][r] = wave_sum_dpp(acc[t]);
    }
    if (lane == 0)
#pragma unroll
        for (int t = 0; t < B; t++)
#pragma unroll
            for (int r = 0; r < R; r++) part[w][t][r] = sum[t][r];
    __syncthreads();
    if ((int)threadIdx.x < B * R) {
        const int t = threadIdx.x / R, r = threadIdx.x % R, row = row0 + r;
        float y = 0.0f;
#pragma unroll
        for (int i = 0; i < KS; i++) y += part[i][t][r];
        const int64_t at = (int64_t)t * rows + row;
        if (row < rows) a.out[0][at] = MODE == ROWS_RESIDUAL ? y + a.residual[at] : y;
    }
}

// ------------------------------------------------------------------------------- launching

template <int TYPE, int B, int NT, int RPW, int WPG, int MODE, bool XF32>
static int rows_go(RowsArgs& a, hipStream_t st) {
    const bool full = a.cols / Task<TYPE>::TASK_W == NT * WAVE;
    int total = 0;  // workgroups: tiles of WPG * RPW rows, per matrix
    for (int i = 0; i < a.count; i++) {
        a.tile_start[i] = total;
        total += (a.rows[i] + WPG * RPW - 1) / (WPG * RPW);
    }
    a.tile_start[a.count] = total;
    const size_t lds = XF32 ? (size_t)B * a.cols + 2 * (size_t)B * (a.cols / GROUP) * 4 : 0;
    if (full)
        hipLaunchKernelGGL((rows_kernel<TYPE, B, NT, RPW, WPG, MODE, XF32, true>), dim3(total), dim3(WPG * 64), lds,
                           st, a);
    else
        hipLaunchKernelGGL((rows_kernel<TYPE, B, NT, RPW, WPG, MODE, XF32, false>), dim3(total), dim3(WPG * 64), lds,
                           st, a);
    return check_launch("rows");
}

constexpr int ROWS_RPW = 2;      // rows a wave streams in the plain and residual products
constexpr int ROWS_WPG = 8;      // waves per workgroup in the plain and residual products
constexpr int ROWS_GLU_WPG = 8;  // waves per workgroup of the GLU: tiles of 32 rows, 32 / WPG per wave

template <int TYPE, int B, int NT, int MODE>
static int rows_shape(RowsArgs& a, bool xf32, hipStream_t st) {
    constexpr int WPG = MODE == ROWS_GLU ? ROWS_GLU_WPG : ROWS_WPG;
    constexpr int RPW = MODE == ROWS_GLU ? 32 / WPG : ROWS_RPW;
    return xf32 ? rows_go<TYPE, B, NT, RPW, WPG, MODE, true>(a, st) : rows_go<TYPE, B, NT, RPW, WPG, MODE, false>(a, st);
}

// Rows a workgroup streams when long rows are split by columns, and of them the rows whose loads
// a wave has in flight. Each lane's activations serve R rows, so more rows cut the activation
// bytes read per weight byte (about 40 B of q8 words and scales a task against 18 B of Q4_K
// weights, 26 of Q6_K); measured on 4096x11008 to 4096x28672: Q4_K 4 rows (all 4 in flight at 1
// token, 2 at 2 tokens), Q6_K 4 rows with 2 in flight, except rows of exactly 7 whole turns
// (14336 weights) at 1 token, where 2 rows measured 4% faster. 8 rows were slower everywhere but
// one shape.
template <int TYPE, int B, bool FULL7>
constexpr int split_rows() {
    return TYPE == Q6_K && B == 1 && FULL7 ? 2 : 4;
}
template <int TYPE, int B>
constexpr int split_depth() {
    return TYPE == Q4_K && B == 1 ? 4 : 2;
}

template <int TYPE, int B, int KS, bool FULL, int MODE>
static int rows_split_at(RowsArgs& a, hipStream_t st) {
    constexpr int R = split_rows<TYPE, B, FULL && KS == 7>(), P = split_depth<TYPE, B>() < R ? split_depth<TYPE, B>() : R;
    RowsArgs one = a;
    for (int i = 0; i < a.count; i++) {  // a launch per matrix
        one.w[0] = a.w[i], one.out[0] = a.out[i], one.rows[0] = a.rows[i];
        hipLaunchKernelGGL((rows_split_kernel<TYPE, B, KS, R, P, MODE, FULL>), dim3((a.rows[i] + R - 1) / R),
                           dim3(KS * WAVE), 0, st, one);
        if (check_launch("rows")) return -1;
    }
    return 0;
}

template <int TYPE, int B, int KS, int MODE>
static int rows_split_go(RowsArgs& a, hipStream_t st) {
    return a.cols / Task<TYPE>::TASK_W == KS * WAVE ? rows_split_at<TYPE, B, KS, true, MODE>(a, st)
                                                    : rows_split_at<TYPE, B, KS, false, MODE>(a, st);
}

template <int TYPE, int B, int MODE>
static int rows_nt(RowsArgs& a, bool xf32, hipStream_t st) {
    const int tasks = a.cols / Task<TYPE>::TASK_W;
    if (tasks <= WAVE) return rows_shape<TYPE, B, 1, MODE>(a, xf32, st);
    if (tasks <= 2 * WAVE) return rows_shape<TYPE, B, 2, MODE>(a, xf32, st);
    if (tasks > 4 * WAVE) {  // long rows, split by columns: one matrix, q8 input, no GLU (rows_fits)
        if constexpr (MODE == ROWS_GLU || TYPE == Q8_0) {
            set_error("rows: rows of %d tasks", tasks);
            return -1;
        } else {
            if (xf32 || tasks > 16 * WAVE) {
                set_error("rows: long rows of %d tasks take quantized input, at most 16 turns", tasks);
                return -1;
            }
            // a wave a turn: the waves of the launch are the row's turns, rounded up
            const int turns = (tasks + WAVE - 1) / WAVE;
            if (turns <= 5) return rows_split_go<TYPE, B, 5, MODE>(a, st);
            if (turns <= 6) return rows_split_go<TYPE, B, 6, MODE>(a, st);
            if (turns <= 7) return rows_split_go<TYPE, B, 7, MODE>(a, st);
            if (turns <= 8) return rows_split_go<TYPE, B, 8, MODE>(a, st);
            if (turns <= 10) return rows_split_go<TYPE, B, 10, MODE>(a, st);
            if (turns <= 12) return rows_split_go<TYPE, B, 12, MODE>(a, st);
            return rows_split_go<TYPE, B, 16, MODE>(a, st);
        }
    }
    return rows_shape<TYPE, B, 4, MODE>(a, xf32, st);
}

template <int TYPE, int MODE>
static int rows_b(RowsArgs& a, int tokens, bool xf32, hipStream_t st) {
    return tokens == 1 ? rows_nt<TYPE, 1, MODE>(a, xf32, st) : rows_nt<TYPE, 2, MODE>(a, xf32, st);
}

bool rows_fits(int type, int cols, int tokens, bool glu) {
    if (tokens < 1 || tokens > ROWS_MAX_TOKENS) return false;
    // rows of 5..16 turns of a wave's 32-weight tasks (up to 32768 weights), split by columns: q8
    // input, no GLU
    const bool split = !glu && cols / 32 > 4 * WAVE && cols / 32 <= 16 * WAVE;
    if (type == Q4_K) return cols % 256 == 0 && (cols / 32 <= 4 * WAVE || split);
    if (type == Q8_0) return cols % 64 == 0 && cols / 64 <= 2 * WAVE;
    // Q6_K rows of whole 512s (block pairs: 4-byte aligned rows)
    if (type == Q6_K) return cols % 512 == 0 && (cols / 32 <= 4 * WAVE || split);
    return false;
}

int rows_launch(int type, int mode, RowsArgs& a, int tokens, bool xf32, hipStream_t st) {
#define LEAT_ROWS_MODES(T)                                                  \
    switch (mode) {                                                         \
    case ROWS_PLAIN: return rows_b<T, ROWS_PLAIN>(a, tokens, xf32, st);       \
    case ROWS_RESIDUAL: return rows_b<T, ROWS_RESIDUAL>(a, tokens, xf32, st); \
    default: return rows_b<T, ROWS_GLU>(a, tokens, xf32, st);                 \
    }
    switch (type) {
    case Q4_K: LEAT_ROWS_MODES(Q4_K)
    case Q6_K: LEAT_ROWS_MODES(Q6_K)
    case Q8_0: LEAT_ROWS_MODES(Q8_0)
    default: set_error("rows: unsupported type %d", type); return -1;
    }
#undef LEAT_ROWS_MODES
}

}  // namespace leat

// ------------------------------------------------------------------------------- the C ABI

using namespace leat;

static int rows_f32_check(int type, int cols, const float* x, int tokens, bool glu) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(x, "null activations");
    LEAT_REQUIRE(rows_fits(type, cols, tokens, glu) && cols <= 8192,
                 "type %d, %d columns, %d tokens: the kernels that quantize their own input take Q4_K and Q8_0 rows "
                 "of at most 8192 weights, Q6_K rows of whole 512s up to 8192, and 1..%d tokens",
                 type, cols, tokens, ROWS_MAX_TOKENS);
    LEAT_REQUIRE((uintptr_t)x % 16 == 0 && cols % 4 == 0, "f32 activations must start 16-byte aligned");
    return 0;
}

extern "C" int leat_matvecs_f32(int count, const int* types, const void* const* ws, const int* rows, int cols,
                                const float* x, int tokens, const float* norm_weight, float eps, float* const* outs,
                                void* stream) {
    LEAT_REQUIRE(count >= 1 && count <= ROWS_MATS, "matvecs_f32: 1..%d matrices", ROWS_MATS);
    RowsArgs a = {};
    for (int i = 0; i < count; i++) {
        LEAT_REQUIRE(types[i] == types[0], "matvecs_f32: the matrices of one call share a type");
        LEAT_REQUIRE(ws[i] && outs[i] && rows[i] > 0, "matvecs_f32: bad matrix %d", i);
        if (check_ptrs(types[i], ws[i], nullptr)) return -1;
        a.w[i] = (const uint8_t*)ws[i];
        a.out[i] = outs[i];
        a.rows[i] = rows[i];
    }
    if (rows_f32_check(types[0], cols, x, tokens, false)) return -1;
    LEAT_REQUIRE(!norm_weight || (uintptr_t)norm_weight % 16 == 0, "matvecs_f32: norm weight not 16-byte aligned");
    a.count = count, a.cols = cols;
    a.x = x, a.norm = norm_weight, a.eps = eps;
    return rows_launch(types[0], ROWS_PLAIN, a, tokens, true, (hipStream_t)stream);
}

extern "C" int leat_qkv_rotate_f32(int type, const void* wq, const void* wk, const void* wv, int heads, int kv_heads,
                                   int dim, int cols, const float* x, int tokens, const float* norm_weight, float eps,
                                   const float* cos, const float* sin, int rotated, const int32_t* slots,
                                   const int32_t* positions, float* q_out, void* cache, int cache_slots,
                                   int cache_positions, void* stream) {
    constexpr int TILE = ROWS_WPG * ROWS_RPW;
    LEAT_REQUIRE(wq && wk && wv && slots && positions && q_out && cache, "qkv_rotate_f32: null pointer");
    LEAT_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "qkv_rotate_f32: %d heads over %d kv heads",
                 heads, kv_heads);
    LEAT_REQUIRE(dim > 0 && dim % TILE == 0, "qkv_rotate_f32: heads of %d dimensions (a multiple of %d)", dim, TILE);
    LEAT_REQUIRE(rotated >= 0 && rotated <= dim && rotated % 2 == 0, "qkv_rotate_f32: %d rotated dimensions of %d",
                 rotated, dim);
    LEAT_REQUIRE(rotated == 0 || (cos && sin), "qkv_rotate_f32: RoPE tables missing");
    LEAT_REQUIRE(cache_slots > 0 && cache_positions > 0, "qkv_rotate_f32: an empty cache");
    if (check_ptrs(type, wq, nullptr) || check_ptrs(type, wk, nullptr) || check_ptrs(type, wv, nullptr) ||
        rows_f32_check(type, cols, x, tokens, false))
        return -1;
    LEAT_REQUIRE(!norm_weight || (uintptr_t)norm_weight % 16 == 0, "qkv_rotate_f32: norm weight not 16-byte aligned");
    RowsArgs a = {};
    const void* ws[3] = {wq, wk, wv};
    const int rows[3] = {heads * dim, kv_heads * dim, kv_heads * dim};
    for (int i = 0; i < 3; i++) {
        a.w[i] = (const uint8_t*)ws[i];
        a.out[i] = nullptr;  // the rows go to q_out and the cache only
        a.rows[i] = rows[i];
    }
    a.count = 3, a.cols = cols;
    a.x = x, a.norm = norm_weight, a.eps = eps;
    a.rope = {cos, sin, rotated, dim, kv_heads, slots, positions, q_out, (_Float16*)cache, cache_slots, cache_positions};
    return rows_launch(type, ROWS_PLAIN, a, tokens, true, (hipStream_t)stream);
}

extern "C" int leat_matvec_f32(int type, const void* w, int rows, int cols, const float* x, int tokens,
                               const float* norm_weight, float eps, const float* residual, float* out, void* stream) {
    LEAT_REQUIRE(w && out && rows > 0, "matvec_f32: null pointer or empty matrix");
    if (check_ptrs(type, w, nullptr) || rows_f32_check(type, cols, x, tokens, false)) return -1;
    LEAT_REQUIRE(!norm_weight || (uintptr_t)norm_weight % 16 == 0, "matvec_f32: norm weight not 16-byte aligned");
    RowsArgs a = {};
    a.w[0] = (const uint8_t*)w;
    a.out[0] = out;
    a.rows[0] = rows;
    a.count = 1, a.cols = cols;
    a.x = x, a.norm = norm_weight, a.eps = eps;
    a.residual = residual;
    return rows_launch(type, residual ? ROWS_RESIDUAL : ROWS_PLAIN, a, tokens, true, (hipStream_t)stream);
}

extern "C" int leat_glu_matvec_f32(int type, const void* gate, const void* up, int rows, int cols, const float* x,
                                   int tokens, const float* norm_weight, float eps, int kind, float* out, int32_t* hq,
                                   float* hd, float* hs, void* stream) {
    LEAT_REQUIRE(gate && up && rows > 0, "glu_matvec_f32: null pointer or empty matrix");
    LEAT_REQUIRE(out || hq, "glu_matvec_f32: neither f32 nor q8 output");
    LEAT_REQUIRE(!hq || (hd && hs && rows % 32 == 0), "glu_matvec_f32: a q8 output needs d, s and rows in 32s");
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matvec_f32: unknown GLU kind %d", kind);
    if (check_ptrs(type, gate, nullptr) || check_ptrs(type, up, nullptr) || rows_f32_check(type, cols, x, tokens, true))
        return -1;
    LEAT_REQUIRE(!norm_weight || (uintptr_t)norm_weight % 16 == 0, "glu_matvec_f32: norm weight not 16-byte aligned");
    RowsArgs a = {};
    a.w[0] = (const uint8_t*)gate;
    a.w[1] = (const uint8_t*)up;
    a.out[0] = out;
    a.rows[0] = rows;
    a.count = 1, a.cols = cols;
    a.x = x, a.norm = norm_weight, a.eps = eps;
    a.kind = kind;
    a.hq = (uint32_t*)hq, a.hd = hd, a.hs = hs;
    return rows_launch(type, ROWS_GLU, a, tokens, true, (hipStream_t)stream);
}

// Decode-path matrix-vector products on GGUF blocks as stored: y[t, row] = W[row] . x[t] for up
// to 16 tokens, every weight read once for all tokens (leat/kernels/matvec.py:1-4, 306-395).
//
// One wave64 owns R consecutive rows (of each of NM matrices: NM = 2 for gate and up). Its lanes
// take the rows' tasks in turn (a task is 32 weights of Q4_K/Q6_K, 64 of Q8_0, so rows of 4096
// and 14336 weights are whole turns), load each token's activation words once and use them for
// all R rows, take int32 dot products with v_dot4_i32_i8 and combine them in f32 per scale span;
// the wave then sums its lanes and lane 0 stores. Several matrices that share the activations
// (q, k and v) run in one launch: waves are numbered across them.
#include "blocks.h"
#include "leatmi.h"
#include "mmv.h"
#include "rows.h"
#include "tiles.h"

namespace leat {

constexpr int MAX_MATS = MMV_MATS;

struct MatvecArgs {
    const uint8_t* w[MAX_MATS];
    float* out[MAX_MATS];
    int rows[MAX_MATS];
    int wave_start[MAX_MATS + 1];  // first wave of each matrix; wave_start[count] = total
    int count;
    int cols;
    const int32_t* xq;
    const float* xd;
    const float* xs;
    const float* residual;  // MODE_RESIDUAL: tokens * rows[0]
    int kind;               // MODE_GLU: the GLU kind; w[0] gate, w[1] up, out[0]
    uint32_t* hq;           // MODE_GLU: q8 of the outputs, where the kernel writes it (glu_q8_inside)
    float* hd;
    float* hs;
};

enum Mode : int { MODE_PLAIN = 0, MODE_RESIDUAL = 1, MODE_GLU = 2 };





// U tasks of each row in flight per lane per iteration; LDS: the workgroup first stages the
// tokens' activations in LDS (xq words, then d, then s) and the lanes read them there.
template <int TYPE, int B, int R, int MODE, int U, bool LDS>
__global__ __launch_bounds__(256) void matvec_kernel(MatvecArgs args) {
    using T = Task<TYPE>;
    constexpr int NM = MODE == MODE_GLU ? 2 : 1;
    extern __shared__ uint32_t act_lds[];
    const int cols = args.cols, tasks = cols / T::TASK_W;
    if (LDS) {
        const int words = B * (cols / 4), scales = B * (cols / GROUP);
        const u32x4* q = (const u32x4*)args.xq;
        for (int i = threadIdx.x; i < words / 4; i += blockDim.x) ((u32x4*)act_lds)[i] = q[i];
        float* lds_d = (float*)(act_lds + words);
        for (int i = threadIdx.x; i < scales; i += blockDim.x) {
            lds_d[i] = args.xd[i];
            if (T::NEEDS_S) lds_d[scales + i] = args.xs[i];
        }
        __syncthreads();
    }
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) / WAVE);
    if (wave >= args.wave_start[args.count]) return;
    int m = 0;
    if (MODE != MODE_GLU) {
        while (m + 1 < args.count && wave >= args.wave_start[m + 1]) m++;
    }
    const int rows = args.rows[m];
    const int row0 = (wave - args.wave_start[m]) * R;

    float acc[NM][R][B];
#pragma unroll
    for (int i = 0; i < NM; i++)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int t = 0; t < B; t++) acc[i][r][t] = 0.0f;

    for (int first = lane; first < tasks; first += WAVE * U) {
        typename T::Raw raw[U][NM][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int task = first + u * WAVE;
            if (U > 1 && task >= tasks) break;
#pragma unroll
            for (int i = 0; i < NM; i++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = min(row0 + r, rows - 1);
                    raw[u][i][r] = T::load(MODE == MODE_GLU ? args.w[i] : args.w[m], row, cols, task);
                }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int task = first + u * WAVE;
            if (U > 1 && task >= tasks) break;
            ActQ act[B];
#pragma unroll
            for (int t = 0; t < B; t++)
                act[t] = LDS ? load_act_lds<TYPE>(act_lds, B, cols, t, task)
                             : load_act<TYPE>(args.xq, args.xd, args.xs, cols, t, task);
#pragma unroll
            for (int i = 0; i < NM; i++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const typename T::Dec dec = T::decode(raw[u][i][r], task);
#pragma unroll
                    for (int t = 0; t < B; t++) acc[i][r][t] += T::combine(dec, act[t], T::dots(dec, act[t]));
                }
        }
    }

#pragma unroll
    for (int i = 0; i < NM; i++)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int t = 0; t < B; t++) acc[i][r][t] = wave_sum(acc[i][r][t]);

    if (lane == 0) {
        float* out = args.out[MODE == MODE_GLU ? 0 : m];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
            if (row >= rows) break;
#pragma unroll
            for (int t = 0; t < B; t++) {
                const int64_t at = (int64_t)t * rows + row;
                float v = acc[0][r][t];
                if (MODE == MODE_GLU) v = glu(args.kind, acc[0][r][t], acc[NM - 1][r][t]);
                if (MODE == MODE_RESIDUAL) v += args.residual[at];
                out[at] = v;
            }
        }
    }
}

// rows per wave for B tokens: with more tokens the activation loads a wave shares across its
// rows cost more than the weights' (the reference's _per_warp, leat/kernels/matvec.py:340-347)
template <int B, int MODE>
constexpr int rows_per_wave() {
    return MODE == MODE_GLU ? 1 : (B <= 8 ? 2 : 1);
}

constexpr int MATVEC_UNROLL = 2;  // one token's rows: tasks a lane has in flight

template <int TYPE, int B, int MODE>
static int launch_b(MatvecArgs& a, hipStream_t stream) {
    constexpr int R = rows_per_wave<B, MODE>();
    int total = 0;
    for (int i = 0; i < a.count; i++) {
        a.wave_start[i] = total;
        total += (a.rows[i] + R - 1) / R;
    }
    a.wave_start[a.count] = total;
    const int blocks = (total + 3) / 4;
    // one or two tokens' activations fit LDS next to other workgroups on the CU; gate and up,
    // two rows a wave, measured faster reading them from L2
    const size_t lds = (size_t)B * (a.cols + a.cols / GROUP * 8);
    if (MODE != MODE_GLU && B <= 2 && lds <= 40960) {
        constexpr int U = B == 1 ? MATVEC_UNROLL : 1;
        hipLaunchKernelGGL((matvec_kernel<TYPE, B, R, MODE, U, true>), dim3(blocks), dim3(256), lds, stream, a);
    } else {
        hipLaunchKernelGGL((matvec_kernel<TYPE, B, R, MODE, 1, false>), dim3(blocks), dim3(256), 0, stream, a);
    }
    return check_launch("matvec");
}

template <int TYPE, int MODE>
static int launch_t(MatvecArgs& a, int tokens, hipStream_t s) {
    switch (tokens) {
    case 1: return launch_b<TYPE, 1, MODE>(a, s);
    case 2: return launch_b<TYPE, 2, MODE>(a, s);
    case 3: return launch_b<TYPE, 3, MODE>(a, s);
    case 4: return launch_b<TYPE, 4, MODE>(a, s);
    case 5: return launch_b<TYPE, 5, MODE>(a, s);
    case 6: return launch_b<TYPE, 6, MODE>(a, s);
    case 7: return launch_b<TYPE, 7, MODE>(a, s);
    case 8: return launch_b<TYPE, 8, MODE>(a, s);
    case 16: return launch_b<TYPE, 16, MODE>(a, s);
    default: set_error("matvec: %d tokens (1..8 or 16 supported)", tokens); return -1;
    }
}

// X(TYPE) for every type the decode tasks take (blocks.h, tasks.h)
#define LEAT_TASK_TYPES(X) X(Q4_0) X(Q4_1) X(Q5_0) X(Q5_1) X(Q8_0) X(Q4_K) X(Q5_K) X(Q6_K) X(IQ4_NL) X(IQ4_XS) X(MXFP4)

template <int MODE>
static int launch(int type, MatvecArgs& a, int tokens, hipStream_t s) {
    switch (type) {
#define LEAT_LAUNCH(T) \
    case T: return launch_t<T, MODE>(a, tokens, s);
        LEAT_TASK_TYPES(LEAT_LAUNCH)
#undef LEAT_LAUNCH
    default: set_error("matvec: unsupported type %d", type); return -1;
    }
}

constexpr int MMV_MIN_TOKENS = 3;  // the fewest tokens the matrix-core path takes

// one or two tokens: the row-streaming kernels; 3..8: the matrix-core tile kernels for the GLU,
// the staged matrix-core kernels (mmv) for the rest; more (16): the staged ones where they fit
// the shape; else the v_dot4 kernels
template <int MODE>
static int dispatch(int type, MatvecArgs& a, int tokens, hipStream_t s) {
    const int nw = MODE == MODE_GLU ? 2 : a.count;
    if (rows_fits(type, a.cols, tokens, MODE == MODE_GLU)) {
        RowsArgs r = {};
        for (int i = 0; i < MAX_MATS; i++) {
            r.w[i] = a.w[i];
            r.out[i] = a.out[i];
            r.rows[i] = a.rows[i];
        }
        r.count = a.count;
        r.cols = a.cols;
        r.xq = a.xq, r.xd = a.xd, r.xs = a.xs;
        r.residual = a.residual;
        r.kind = a.kind;
        r.hq = a.hq, r.hd = a.hd, r.hs = a.hs;
        return rows_launch(type, MODE, r, tokens, false, s);
    }
    // 3..16 tokens: the GLU on the tile kernels; the plain and residual products (where they fit)
    // on the staged ones, which measured faster for them
    if (tiles_fits(type, a.cols, tokens, (const void* const*)a.w, nw) &&
        (MODE == MODE_GLU || !mmv_fits(type, a.cols, tokens, (const void* const*)a.w, nw))) {
        TileArgs t = {};
        for (int i = 0; i < MAX_MATS; i++) {
            t.w[i] = a.w[i];
            t.out[i] = a.out[i];
            t.rows[i] = a.rows[i];
        }
        t.count = a.count;
        t.cols = a.cols;
        t.tokens = tokens;
        t.xq = a.xq, t.xd = a.xd, t.xs = a.xs;
        t.residual = a.residual;
        t.kind = a.kind;
        t.hq = a.hq, t.hd = a.hd, t.hs = a.hs;
        return tiles_launch(type, MODE, t, s);
    }
    if (tokens >= MMV_MIN_TOKENS && mmv_fits(type, a.cols, tokens, (const void* const*)a.w, nw)) {
        MmvArgs m = {};
        for (int i = 0; i < MAX_MATS; i++) {
            m.w[i] = a.w[i];
            m.out[i] = a.out[i];
            m.rows[i] = a.rows[i];
        }
        m.count = a.count;
        m.cols = a.cols;
        m.tokens = tokens;
        m.xq = a.xq, m.xd = a.xd, m.xs = a.xs;
        m.residual = a.residual;
        m.kind = a.kind;
        return mmv_launch(type, MODE, m, s);
    }
    return launch<MODE>(type, a, tokens, s);
}

// Q4_K blocks are read as 16-byte vectors: their matrices start 16-byte aligned; Q6_K and Q8_0
// blocks as aligned dwords from a 4-byte aligned start. Activation words are read 16 at a time.
int check_ptrs(int type, const void* w, const void* xq) {
    // Q4_K and Q5_K blocks are read in 16-byte pieces, IQ4_XS in 8-byte ones, the 32-weight types
    // other than Q8_0 in halfwords
    const uintptr_t need = type == Q4_K || type == Q5_K ? 16 : type == IQ4_XS ? 8 : type == Q8_0 || type == Q6_K ? 4 : 2;
    LEAT_REQUIRE((uintptr_t)w % need == 0, "weights of type %d must start %d-byte aligned", type, (int)need);
    LEAT_REQUIRE(xq == nullptr || (uintptr_t)xq % 16 == 0, "activation words must start 16-byte aligned");
    return 0;
}

int check_cols(int type, int cols) {
    if (type == Q4_K || type == Q5_K || type == Q6_K || type == IQ4_XS) {
        LEAT_REQUIRE(cols > 0 && cols % 256 == 0, "cols %d is not a whole number of 256-weight blocks", cols);
    } else if (type == Q8_0 || type == Q4_0 || type == Q4_1 || type == Q5_0 || type == Q5_1 || type == IQ4_NL ||
               type == MXFP4) {
        LEAT_REQUIRE(cols > 0 && cols % 64 == 0, "cols %d is not a whole number of block pairs", cols);
    } else {
        set_error("unsupported type %d", type);
        return -1;
    }
    return 0;
}

}  // namespace leat

using namespace leat;

extern "C" int leat_matvecs(int count, const int* types, const void* const* ws, const int* rows, int cols,
                            const int32_t* xq, const float* xd, const float* xs, int tokens,
                            float* const* outs, void* stream) {
    LEAT_REQUIRE(count >= 1, "matvecs: no matrices");
    LEAT_REQUIRE(xq && xd && xs, "matvecs: null activations");
    int done = 0;
    while (done < count) {
        // consecutive matrices of one type share a launch, up to MAX_MATS
        MatvecArgs a = {};
        const int type = types[done];
        if (check_cols(type, cols)) return -1;
        while (done < count && types[done] == type && a.count < MAX_MATS) {
            LEAT_REQUIRE(ws[done] && outs[done] && rows[done] > 0, "matvecs: bad matrix %d", done);
            if (check_ptrs(type, ws[done], xq)) return -1;
            a.w[a.count] = (const uint8_t*)ws[done];
            a.out[a.count] = outs[done];
            a.rows[a.count] = rows[done];
            a.count++;
            done++;
        }
        a.cols = cols;
        a.xq = xq, a.xd = xd, a.xs = xs;
        if (dispatch<MODE_PLAIN>(type, a, tokens, (hipStream_t)stream)) return -1;
    }
    return 0;
}

extern "C" int leat_matvec(int type, const void* w, int rows, int cols, const int32_t* xq, const float* xd,
                           const float* xs, int tokens, const float* residual, float* out, void* stream) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(w && out && xq && xd && xs && rows > 0, "matvec: null pointer or empty matrix");
    if (check_ptrs(type, w, xq)) return -1;
    MatvecArgs a = {};
    a.w[0] = (const uint8_t*)w;
    a.out[0] = out;
    a.rows[0] = rows;
    a.count = 1;
    a.cols = cols;
    a.xq = xq, a.xd = xd, a.xs = xs;
    a.residual = residual;
    return residual ? dispatch<MODE_RESIDUAL>(type, a, tokens, (hipStream_t)stream)
                    : dispatch<MODE_PLAIN>(type, a, tokens, (hipStream_t)stream);
}

// whether dispatch<MODE_GLU> takes a kernel that writes the q8 of its outputs itself (rows a
// multiple of 32): the row-streaming kernels (1..2 tokens) and the tile kernels (3..8 of Q4_K)
static bool glu_q8_inside(int type, int cols, int tokens, const void* gate, const void* up) {
    const void* ws[2] = {gate, up};
    return rows_fits(type, cols, tokens, true) || tiles_fits(type, cols, tokens, ws, 2);
}

extern "C" int leat_glu_matvec_q8(int type, const void* gate, const void* up, int rows, int cols, const int32_t* xq,
                                  const float* xd, const float* xs, int tokens, int kind, float* out, int32_t* hq,
                                  float* hd, float* hs, void* stream) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(gate && up && out && xq && xd && xs && hq && hd && hs && rows > 0,
                 "glu_matvec_q8: null pointer or empty matrix");
    LEAT_REQUIRE(rows % GROUP == 0, "glu_matvec_q8: rows %d not a multiple of 32", rows);
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matvec_q8: unknown GLU kind %d", kind);
    if (check_ptrs(type, gate, xq) || check_ptrs(type, up, xq)) return -1;
    MatvecArgs a = {};
    a.w[0] = (const uint8_t*)gate;
    a.w[1] = (const uint8_t*)up;
    a.out[0] = out;
    a.rows[0] = rows;
    a.count = 1;
    a.cols = cols;
    a.xq = xq, a.xd = xd, a.xs = xs;
    a.kind = kind;
    const bool inside = glu_q8_inside(type, cols, tokens, gate, up);
    if (inside) a.hq = (uint32_t*)hq, a.hd = hd, a.hs = hs;
    if (dispatch<MODE_GLU>(type, a, tokens, (hipStream_t)stream)) return -1;
    // other kernels: the outputs quantized by a second launch
    return inside ? 0 : leat_quantize_q8(out, tokens, rows, nullptr, 0.0f, hq, hd, hs, stream);
}

extern "C" int leat_glu_matvec(int type, const void* gate, const void* up, int rows, int cols, const int32_t* xq,
                               const float* xd, const float* xs, int tokens, int kind, float* out, void* stream) {
    if (check_cols(type, cols)) return -1;
    LEAT_REQUIRE(gate && up && out && xq && xd && xs && rows > 0, "glu_matvec: null pointer or empty matrix");
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matvec: unknown GLU kind %d", kind);
    if (check_ptrs(type, gate, xq) || check_ptrs(type, up, xq)) return -1;
    MatvecArgs a = {};
    a.w[0] = (const uint8_t*)gate;
    a.w[1] = (const uint8_t*)up;
    a.out[0] = out;
    a.rows[0] = rows;
    a.count = 1;
    a.cols = cols;
    a.xq = xq, a.xd = xd, a.xs = xs;
    a.kind = kind;
    return dispatch<MODE_GLU>(type, a, tokens, (hipStream_t)stream);
}

// Prefill products of Q6_K and Q8_0 weights on matrix cores (leat/kernels/matmul.py: llama.cpp's
// MMQ): out[t, r] = W[r] . x[t] for many tokens, the activations quantized to int8 per group of 32
// as for decode, int32 products per group on v_mfma_i32_32x32x32_i8, scaled into f32 per group
// exactly as leat's _Q6KTile / _Q80Tile.scaled (leat/kernels/matmul.py:379-387, 447-452). Q4_K
// takes prefill.hip's kernels and the plain and residual Q6_K products prefill6.hip's; the Q6_K
// gated product and Q8_0 stay here.
//
// A workgroup owns a tile of 128 tokens by MMQ_TILES row tiles of 32 (of one matrix, or half of
// gate and the same rows of up); each of its 4 waves owns one 32-token tile for all the row
// tiles, so the token scales it reads for a group serve MMQ_TILES products. The K loop takes 256
// weights a step: a Q6_K block, or 8 Q8_0 blocks per row. Each step the workgroup stages its
// rows' step bytes (coalesced 16-byte loads, as the decode kernels do) and the 128 tokens' 256
// int8 values (row stride padded against bank conflicts) and scales (group-major) in LDS, and
// loads the next step's bytes into registers while this one is multiplied.
//
// In each MFMA the rows are N (lane l holds row l % 32 and, per lane half h = l / 32, 16 of the
// group's 32 values), the tokens M (lane l holds token l % 32 of the token tile), and the result
// in lane l is row l % 32 for tokens 8(v/4) + 4h + v%4 of registers v = 0..15.
#include <algorithm>

#include "blocks.h"
#include "leatmi.h"
#include "mmv.h"
#include "prefill.h"
#include "tiles.h"

namespace leat {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int MMQ_TILES = 2;     // row tiles of 32 per workgroup
constexpr int MMQ_TOKENS = 128;  // tokens per workgroup: a tile of 32 per wave
constexpr int MMQ_K = 256;       // weights per row per step
constexpr int MMQ_XSTRIDE = 272; // bytes per token row of staged activations: 68 dwords

enum MmqMode : int { MMQ_PLAIN = 0, MMQ_RESIDUAL = 1, MMQ_GLU = 2 };

struct MmqArgs {
    const uint8_t* w[2];
    float* out;
    int rows, cols, tokens;
    const int32_t* xq;
    const float* xd;
    const float* xs;
    const float* residual;
    int kind;
};

extern __shared__ uint32_t mmq_lds[];

__device__ __forceinline__ v16i mmq_mfma(v4i a, u32x4 b) {
    const v16i zero = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, __builtin_bit_cast(v4i, b), zero, 0, 0, 0);
}

// the outer product a (x) b of the 32-vectors the lanes of half 0 hold (a: one entry per token,
// b: one per row), plus c, in the 32x32 result layout of mmq_mfma: the per-group scale matrix
// of the int32 products, built on the matrix cores rather than one multiply per element
__device__ __forceinline__ v16f outer(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 lds_u4(uint32_t at) { return *(const u32x4_a4*)((const char*)mmq_lds + at); }
__device__ __forceinline__ uint32_t lds_u1(uint32_t at) { return *(const uint32_t*)((const char*)mmq_lds + at); }

// 16 bytes at an even LDS address, 2 bytes off a 4-byte boundary when ODD
template <bool ODD>
__device__ __forceinline__ u32x4 lds_u4_even(uint32_t at) {
    if (!ODD) return lds_u4(at);
    const u32x4 a = lds_u4(at - 2);
    const uint32_t e = lds_u1(at + 14);
    u32x4 r;
    r[0] = align_bytes(a[1], a[0], 2);
    r[1] = align_bytes(a[2], a[1], 2);
    r[2] = align_bytes(a[3], a[2], 2);
    r[3] = align_bytes(e, a[3], 2);
    return r;
}

// A step's weight bytes per row: 256 weights from the step's first byte rounded down to 4 (rows
// start 4-byte aligned), as CPR chunks of 16 bytes, kept at a row stride of RS bytes.
template <int TYPE> struct QGeo;
template <> struct QGeo<Q6_K> { static constexpr int STEP_BYTES = 210, CPR = 14, RS = 240; };
template <> struct QGeo<Q8_0> { static constexpr int STEP_BYTES = 272, CPR = 17, RS = 304; };

// LDS: [xq: 128 x MMQ_XSTRIDE][d: 8 x 128 f32][s: 8 x 128 f32][weights: 32 MMQ_TILES x RS]
constexpr uint32_t MMQ_XQ = 0, MMQ_XD = MMQ_TOKENS * MMQ_XSTRIDE, MMQ_XS = MMQ_XD + 8 * MMQ_TOKENS * 4,
                   MMQ_W = MMQ_XS + 8 * MMQ_TOKENS * 4;

// the workgroup's 32 * MMQ_TILES staged rows: gated, the first half of gate, then the same of up
template <int TYPE>
struct WStage {
    static constexpr int CHUNKS = 32 * MMQ_TILES * QGeo<TYPE>::CPR;
    static constexpr int N = (CHUNKS + 255) / 256;
    u32x4 v[N];
};

// chunk `part` of a row's step starts `off` bytes into the row, `off` - s0 into its LDS row: a
// last chunk that would pass the row's end is read from 16 bytes before the end instead, and
// lands where those bytes belong
template <int TYPE>
__device__ __forceinline__ int64_t chunk_at(int64_t s0, int part, int64_t row_bytes) {
    return min(s0 + 16 * part, row_bytes - 16);
}

template <int TYPE, bool GATED>
__device__ __forceinline__ void wstage_load(WStage<TYPE>& st, const MmqArgs& a, int64_t row_bytes, int row0, int step,
                                            int tid) {
    using G = QGeo<TYPE>;
    const int64_t s0 = ((int64_t)step * G::STEP_BYTES) & ~(int64_t)3;
#pragma unroll
    for (int i = 0; i < WStage<TYPE>::N; i++) {
        const int c = tid + 256 * i;
        if (c < WStage<TYPE>::CHUNKS) {
            const int lr = c / G::CPR, part = c % G::CPR;
            constexpr int HALF = 16 * MMQ_TILES;  // gated: the first half of the rows are gate's
            const uint8_t* w = a.w[GATED ? lr / HALF : 0];
            const int64_t row = min(row0 + (GATED ? lr % HALF : lr), a.rows - 1);
            st.v[i] = stream_load((const u32x4_a4*)(w + row * row_bytes + chunk_at<TYPE>(s0, part, row_bytes)));
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void wstage_store(const WStage<TYPE>& st, int64_t row_bytes, int step, int tid) {
    using G = QGeo<TYPE>;
    const int64_t s0 = ((int64_t)step * G::STEP_BYTES) & ~(int64_t)3;
#pragma unroll
    for (int i = 0; i < WStage<TYPE>::N; i++) {
        const int c = tid + 256 * i;
        if (c < WStage<TYPE>::CHUNKS) {
            const int at = (int)(chunk_at<TYPE>(s0, c % G::CPR, row_bytes) - s0);
            *(u32x4_a4*)((char*)mmq_lds + MMQ_W + (c / G::CPR) * G::RS + at) = st.v[i];
        }
    }
}

// the workgroup's activations for one step: 128 tokens x 256 int8 values (8 chunks of 16 bytes
// per thread) and the step's 8 groups' d and s of each token (4 each per thread)
struct XStage {
    u32x4 q[8];
    float d[4], s[4];
};

__device__ __forceinline__ void xstage_load(XStage& x, const MmqArgs& a, int tok0, int step, int tid) {
    const int G = a.cols / GROUP;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int c = tid + 256 * i;  // chunk c: token c / 16, 16-byte part c % 16
        const int t = min(tok0 + c / 16, a.tokens - 1);
        x.q[i] = *(const u32x4*)((const uint8_t*)a.xq + (int64_t)t * a.cols + step * MMQ_K + 16 * (c % 16));
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = tid + 256 * i;  // entry e: group e / 128 of the step, token e % 128
        const int t = min(tok0 + e % MMQ_TOKENS, a.tokens - 1);
        const int64_t at = (int64_t)t * G + step * 8 + e / MMQ_TOKENS;
        x.d[i] = a.xd[at];
        x.s[i] = a.xs[at];
    }
}

__device__ __forceinline__ void xstage_store(const XStage& x, int tid) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int c = tid + 256 * i;
        *(u32x4*)((char*)mmq_lds + MMQ_XQ + (c / 16) * MMQ_XSTRIDE + 16 * (c % 16)) = x.q[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = tid + 256 * i;
        ((float*)((char*)mmq_lds + MMQ_XD))[e] = x.d[i];
        ((float*)((char*)mmq_lds + MMQ_XS))[e] = x.s[i];
    }
}

// the wave's token tile w: lane (t, h)'s 16 values of group g
__device__ __forceinline__ v4i x_operand(int w, int t, int h, int g) {
    return __builtin_bit_cast(v4i, lds_u4(MMQ_XQ + (32 * w + t) * MMQ_XSTRIDE + 32 * g + 16 * h));
}
// the scale (table at `off`) of group g for the lane's own token of the A operand (half 0's
// lanes; half 1's give 0, the second K slice of the outer product)
__device__ __forceinline__ float x_scale(uint32_t off, int w, int g, int r, int h) {
    const float v = ((const float*)((const char*)mmq_lds + off))[g * MMQ_TOKENS + 32 * w + r];
    return h == 0 ? v : 0.0f;
}

// one step: acc[q] += the share of the lane's row in row tile q for the wave's token tile
template <int TYPE> struct QCompute;

template <>
struct QCompute<Q6_K> {
    // ODD: the step's block is odd, so it starts 2 bytes off a 4-byte boundary (compile time: a
    // runtime flag keeps both variants of every load live)
    template <bool ODD>
    __device__ static void run(int step, int w, int r, int h, v16f (&acc)[MMQ_TILES]) {
        const uint32_t lead = ODD ? 2 : 0;  // (210 step) mod 4
        const v16f zero = {};
        float d[MMQ_TILES];
#pragma unroll
        for (int q = 0; q < MMQ_TILES; q++) {
            const uint32_t dat = MMQ_W + (32 * q + r) * QGeo<Q6_K>::RS + lead + 208;
            const uint32_t dw = lds_u1(dat & ~3u);
            d[q] = (dat & 2) ? f16_hi(dw) : f16_lo(dw);
        }
#pragma unroll
        for (int g = 0; g < 8; g++) {  // the row of 32 values 128n + 32k.., n = g / 4, k = g % 4
            const int n = g >> 2, k = g & 3;
            const v4i x = x_operand(w, r, h, g);
            const float xd = x_scale(MMQ_XD, w, g, r, h);
#pragma unroll
            for (int q = 0; q < MMQ_TILES; q++) {
                const uint32_t at = MMQ_W + (32 * q + r) * QGeo<Q6_K>::RS + lead;
                const u32x4 ql = lds_u4_even<ODD>(at + 64 * n + 32 * (k & 1) + 16 * h);
                const u32x4 qh = lds_u4_even<ODD>(at + 128 + 32 * n + 16 * h);
                u32x4 b;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t low = (ql[i] >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
                    const uint32_t high = (qh[i] >> (2 * k)) & 0x03030303u;
                    b[i] = minus_bytes(low | (high << 4), 32);
                }
                // scales 2g and 2g + 1 (8n + 2k and + 1: values 0..15 and 16..31 of the row)
                const uint32_t sat = at + 192 + 2 * g;
                const uint32_t sw = lds_u1(sat & ~3u) >> (8 * (sat & 2));
                const int sc0 = (int8_t)(sw & 0xFF), sc1 = (int8_t)((sw >> 8) & 0xFF);
                const u32x4 none = {};
                const v16i D0 = mmq_mfma(x, h == 0 ? b : none), D1 = mmq_mfma(x, h == 1 ? b : none);
                const v16f S = outer(xd, h == 0 ? d[q] : 0.0f, zero);  // d[row] * xd[token]
#pragma unroll
                for (int v = 0; v < 16; v++) acc[q][v] += (float)(__mul24(D0[v], sc0) + __mul24(D1[v], sc1)) * S[v];
                __builtin_amdgcn_sched_barrier(0);  // three 16-register results per product
            }
        }
    }
};

template <>
struct QCompute<Q8_0> {
    __device__ static void run(int w, int r, int h, v16f (&acc)[MMQ_TILES]) {
        const v16f zero = {};
#pragma unroll
        for (int e = 0; e < 8; e++) {  // 8 blocks of 34 bytes from a 4-aligned start
            const v4i x = x_operand(w, r, h, e);
            const float xd = x_scale(MMQ_XD, w, e, r, h);
#pragma unroll
            for (int q = 0; q < MMQ_TILES; q++) {
                const uint32_t blk = MMQ_W + (32 * q + r) * QGeo<Q8_0>::RS + 34 * e;
                const uint32_t dw = lds_u1(blk & ~3u);
                const float d = (e & 1) ? f16_hi(dw) : f16_lo(dw);
                const u32x4 qs = (e & 1) ? lds_u4_even<false>(blk + 2 + 16 * h) : lds_u4_even<true>(blk + 2 + 16 * h);
                const v16i D = mmq_mfma(x, qs);
                const v16f S = outer(xd, h == 0 ? d : 0.0f, zero);
#pragma unroll
                for (int v = 0; v < 16; v++) acc[q][v] += (float)D[v] * S[v];
            }
        }
    }
};

template <int TYPE, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mmq_kernel(MmqArgs args) {
    constexpr bool GATED = MODE == MMQ_GLU;
    constexpr int TILE_ROWS = GATED ? 16 * MMQ_TILES : 32 * MMQ_TILES;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, h = lane >> 5;
    const int row0 = blockIdx.x * TILE_ROWS;
    const int tok0 = blockIdx.y * MMQ_TOKENS;
    const int steps = args.cols / MMQ_K;
    const int nb = args.cols / (TYPE == Q8_0 ? 32 : 256);
    const int64_t row_bytes = (int64_t)nb * (TYPE == Q8_0 ? 34 : 210);

    WStage<TYPE> ws;
    XStage xs;
    wstage_load<TYPE, GATED>(ws, args, row_bytes, row0, 0, tid);
    xstage_load(xs, args, tok0, 0, tid);

    v16f acc[MMQ_TILES];
#pragma unroll
    for (int q = 0; q < MMQ_TILES; q++) acc[q] = v16f{};

    for (int step = 0; step < steps; step++) {
        __syncthreads();  // every wave is done with the previous step's LDS
        xstage_store(xs, tid);
        wstage_store<TYPE>(ws, row_bytes, step, tid);
        if (step + 1 < steps) {
            wstage_load<TYPE, GATED>(ws, args, row_bytes, row0, step + 1, tid);
            xstage_load(xs, args, tok0, step + 1, tid);
        }
        __syncthreads();
        if constexpr (TYPE == Q6_K) {
            if (step & 1)
                QCompute<Q6_K>::run<true>(step, wave, r, h, acc);
            else
                QCompute<Q6_K>::run<false>(step, wave, r, h, acc);
        } else {
            QCompute<Q8_0>::run(wave, r, h, acc);
        }
    }

    // row tile q holds rows row0 + 32q (gated: the first half gate's, the second up's same rows)
    constexpr int OUT_TILES = GATED ? MMQ_TILES / 2 : MMQ_TILES;
#pragma unroll
    for (int q = 0; q < OUT_TILES; q++) {
        const int row = row0 + 32 * q + r;
        if (row >= args.rows) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int t = tok0 + 32 * wave + 8 * (v >> 2) + 4 * h + (v & 3);
            if (t >= args.tokens) continue;
            const int64_t at = (int64_t)t * args.rows + row;
            float y = acc[q][v];
            if (GATED) y = glu(args.kind, acc[q][v], acc[q + OUT_TILES][v]);
            if (MODE == MMQ_RESIDUAL) y += args.residual[at];
            args.out[at] = y;
        }
    }
}

template <int TYPE, int MODE>
static int mmq_launch(MmqArgs& a, hipStream_t st) {
    const int tile_rows = MODE == MMQ_GLU ? 16 * MMQ_TILES : 32 * MMQ_TILES;
    const dim3 grid((a.rows + tile_rows - 1) / tile_rows, (a.tokens + MMQ_TOKENS - 1) / MMQ_TOKENS);
    const size_t lds = MMQ_W + (size_t)32 * MMQ_TILES * QGeo<TYPE>::RS;
    hipLaunchKernelGGL((mmq_kernel<TYPE, MODE>), grid, dim3(256), lds, st, a);
    return check_launch("matmul");
}

template <int MODE>
static int mmq_dispatch(int type, MmqArgs& a, hipStream_t st) {
    switch (type) {
    case Q6_K: return mmq_launch<Q6_K, MODE>(a, st);
    case Q8_0: return mmq_launch<Q8_0, MODE>(a, st);
    default: set_error("matmul: unsupported type %d", type); return -1;
    }
}

// shapes the tiles take (leat/kernels/matmul.py:1041-1048 matmul_fits: whole blocks of 256
// weights per step, here also rows whole 16-byte chunks and 16-byte aligned matrices)
static int mmq_check(int type, const void* w, int rows, int cols, const int32_t* xq, const float* xd, const float* xs,
                     int tokens, const float* out) {
    LEAT_REQUIRE(type == Q4_K || type == Q6_K || type == Q8_0, "matmul: unsupported type %d", type);
    LEAT_REQUIRE(w && xq && xd && xs && out, "matmul: null pointer");
    LEAT_REQUIRE(rows > 0 && tokens > 0, "matmul: empty product");
    LEAT_REQUIRE(cols > 0 && cols % MMQ_K == 0, "matmul: cols %d is not a whole number of 256-weight steps", cols);
    const int64_t row_bytes = type == Q8_0 ? (int64_t)cols / 32 * 34 : (int64_t)cols / 256 * (type == Q4_K ? 144 : 210);
    LEAT_REQUIRE(row_bytes % 4 == 0, "matmul: rows of %lld bytes do not keep blocks 4-byte aligned", (long long)row_bytes);
    LEAT_REQUIRE((uintptr_t)w % 4 == 0 && (uintptr_t)xq % 16 == 0, "matmul: weights must be 4-byte and words 16-byte aligned");
    // Q4_K's kernels load 16-byte chunks of its 144-byte blocks
    LEAT_REQUIRE(type != Q4_K || (uintptr_t)w % 16 == 0, "matmul: Q4_K weights must be 16-byte aligned");
    return 0;
}

// the split of a launch of `tiles` tiles (prefill.h): chunks double while the launch still fits the
// GPU's workgroup slots (two a CU) and every chunk keeps at least 4 of the `steps` K steps
Split split_schedule(int tiles, int steps, int64_t part_bytes) {
    const int slots = 2 * cu_count();
    int chunks = 1;
    while (chunks < 8 && (int64_t)tiles * chunks * 2 <= slots && steps >= 4 * chunks * 2) chunks *= 2;
    return Split{chunks, chunks > 1 ? (int64_t)tiles * chunks * part_bytes : 0};
}

// leat's tile height choice (leat/kernels/matmul.py:904-906, _tile_tokens): up to FEW_TOKENS
// tokens take the matrix-core decode kernels, whose tiles are 32 rows by 16 tokens
constexpr int FEW_TOKENS = 16;

static bool few_fits(int type, int cols, int tokens, const void* const* ws, int count) {
    return tokens <= FEW_TOKENS && mmv_fits(type, cols, tokens, ws, count);
}

static int few_launch(int type, int mode, const void* const* ws, int count, int rows, int cols, const int32_t* xq,
                      const float* xd, const float* xs, int tokens, const float* residual, int kind, float* out,
                      hipStream_t st) {
    MmvArgs m = {};
    for (int i = 0; i < count; i++) m.w[i] = (const uint8_t*)ws[i];
    m.out[0] = out;
    m.rows[0] = rows;
    m.count = 1;
    m.cols = cols;
    m.tokens = tokens;
    m.xq = xq, m.xd = xd, m.xs = xs;
    m.residual = residual;
    m.kind = kind;
    return mmv_launch(type, mode, m, st);
}

// the few-token gate+up GLU of Q4_K on the matrix-core tile kernels (3..16 tokens), which also
// write the outputs' q8 when hq is given: faster than the LDS-staged ones for the GLU
static bool few_tiles(int type, int cols, int tokens, const void* const* ws) {
    return type == Q4_K && tokens <= FEW_TOKENS && tiles_fits(type, cols, tokens, ws, 2);
}

static int few_tiles_glu(const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                         const float* xs, int tokens, int kind, float* out, int32_t* hq, float* hd, float* hs,
                         hipStream_t st) {
    constexpr int TILES_GLU_MODE = 2;
    TileArgs t = {};
    t.w[0] = (const uint8_t*)ws[0];
    t.w[1] = (const uint8_t*)ws[1];
    t.out[0] = out;
    t.rows[0] = rows;
    t.count = 1;
    t.cols = cols;
    t.tokens = tokens;
    t.xq = xq, t.xd = xd, t.xs = xs;
    t.kind = kind;
    t.hq = (uint32_t*)hq, t.hd = hd, t.hs = hs;
    return tiles_launch(Q4_K, TILES_GLU_MODE, t, st);
}

// the workspace a product would split into (0: it does not split)
static int64_t workspace_of(int type, int rows, int cols, int tokens, bool gated) {
    if (tokens <= FEW_TOKENS) return 0;  // the decode kernels (few_launch) take no workspace
    if (type == Q4_K) return prefill_split(gated ? PF_GLU : PF_PLAIN, rows, cols, tokens).bytes;
    if (type == Q6_K && !gated && prefill_q6k_fits(cols)) return prefill_q6k_split(rows, cols, tokens).bytes;
    return 0;
}

int64_t matmul_workspace(int type, int rows, int cols, int tokens, bool gated) {
    if (rows <= 0 || cols <= 0 || tokens <= 0 || cols % 256 != 0) return 0;
    return workspace_of(type, rows, cols, tokens, gated);
}

// the storage types without matrix-core tiles here (Q4_0, Q4_1, Q5_0, Q5_1, Q5_K, IQ4_NL, IQ4_XS,
// MXFP4): their products run on the decode kernels' v_dot4 tasks, 8 tokens a launch, so the int8
// arithmetic is the decode path's and the weights are read once per 8 tokens
static bool tileless(int type) { return type != Q4_K && type != Q6_K && type != Q8_0; }

static int chunked(int type, const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                   const float* xs, int tokens, const float* residual, int kind, float* out, hipStream_t st) {
    for (int t0 = 0; t0 < tokens; t0 += 8) {
        const int n = std::min(8, tokens - t0);
        const int32_t* q = xq + (int64_t)t0 * (cols / 4);
        const float *d = xd + (int64_t)t0 * (cols / GROUP), *s = xs + (int64_t)t0 * (cols / GROUP);
        float* o = out + (int64_t)t0 * rows;
        const int status = kind < 0 ? leat_matvec(type, ws[0], rows, cols, q, d, s, n, residual ? residual + (int64_t)t0 * rows : nullptr,
                                                  o, st)
                                    : leat_glu_matvec(type, ws[0], ws[1], rows, cols, q, d, s, n, kind, o, st);  // fmt: skip
        if (status) return -1;
    }
    return 0;
}

int matmul_go(int type, const void* w, int rows, int cols, const int32_t* xq, const float* xd, const float* xs,
              int tokens, const float* residual, float* out, void* workspace, int64_t workspace_bytes, hipStream_t st) {
    if (tileless(type)) {
        LEAT_REQUIRE(w && xq && xd && xs && out && rows > 0 && tokens > 0, "matmul: null pointer or empty product");
        return chunked(type, &w, rows, cols, xq, xd, xs, tokens, residual, -1, out, st);
    }
    if (mmq_check(type, w, rows, cols, xq, xd, xs, tokens, out)) return -1;
    if (few_fits(type, cols, tokens, &w, 1))
        return few_launch(type, residual ? MMV_RESIDUAL : MMV_PLAIN, &w, 1, rows, cols, xq, xd, xs, tokens, residual, 0,
                          out, st);
    if (type == Q4_K)
        return prefill_launch(residual ? PF_RESIDUAL : PF_PLAIN, &w, rows, cols, xq, xd, xs, tokens, residual, 0, out, st,
                              nullptr, nullptr, nullptr, workspace, workspace_bytes);
    if (type == Q6_K && prefill_q6k_fits(cols))
        return prefill_q6k_launch(w, rows, cols, xq, xd, tokens, residual, out, st, workspace, workspace_bytes);
    MmqArgs a = {};
    a.w[0] = a.w[1] = (const uint8_t*)w;
    a.out = out;
    a.rows = rows, a.cols = cols, a.tokens = tokens;
    a.xq = xq, a.xd = xd, a.xs = xs;
    a.residual = residual;
    return residual ? mmq_dispatch<MMQ_RESIDUAL>(type, a, st) : mmq_dispatch<MMQ_PLAIN>(type, a, st);
}

}  // namespace leat

using namespace leat;

extern "C" int64_t leat_matmul_workspace(int type, int rows, int cols, int tokens, int gated) {
    return matmul_workspace(type, rows, cols, tokens, gated != 0);
}

extern "C" int leat_matmul(int type, const void* w, int rows, int cols, const int32_t* xq, const float* xd,
                           const float* xs, int tokens, const float* residual, float* out, void* workspace,
                           int64_t workspace_bytes, void* stream) {
    return matmul_go(type, w, rows, cols, xq, xd, xs, tokens, residual, out, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int leat_glu_matmul(int type, const void* gate, const void* up, int rows, int cols, const int32_t* xq,
                               const float* xd, const float* xs, int tokens, int kind, float* out, void* workspace,
                               int64_t workspace_bytes, void* stream) {
    if (tileless(type)) {
        LEAT_REQUIRE(gate && up && xq && xd && xs && out && rows > 0 && tokens > 0, "glu_matmul: null pointer or empty product");
        LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matmul: unknown GLU kind %d", kind);
        const void* ws[2] = {gate, up};
        return chunked(type, ws, rows, cols, xq, xd, xs, tokens, nullptr, kind, out, (hipStream_t)stream);
    }
    if (mmq_check(type, gate, rows, cols, xq, xd, xs, tokens, out) || mmq_check(type, up, rows, cols, xq, xd, xs, tokens, out))
        return -1;
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matmul: unknown GLU kind %d", kind);
    const void* ws[2] = {gate, up};
    if (few_tiles(type, cols, tokens, ws))
        return few_tiles_glu(ws, rows, cols, xq, xd, xs, tokens, kind, out, nullptr, nullptr, nullptr, (hipStream_t)stream);
    if (few_fits(type, cols, tokens, ws, 2))
        return few_launch(type, MMV_GLU, ws, 2, rows, cols, xq, xd, xs, tokens, nullptr, kind, out, (hipStream_t)stream);
    if (type == Q4_K)
        return prefill_launch(PF_GLU, ws, rows, cols, xq, xd, xs, tokens, nullptr, kind, out, (hipStream_t)stream,
                              nullptr, nullptr, nullptr, workspace, workspace_bytes);
    MmqArgs a = {};
    a.w[0] = (const uint8_t*)gate;
    a.w[1] = (const uint8_t*)up;
    a.out = out;
    a.rows = rows, a.cols = cols, a.tokens = tokens;
    a.xq = xq, a.xd = xd, a.xs = xs;
    a.kind = kind;
    return mmq_dispatch<MMQ_GLU>(type, a, (hipStream_t)stream);
}

extern "C" int leat_glu_matmul_q8(int type, const void* gate, const void* up, int rows, int cols, const int32_t* xq,
                                  const float* xd, const float* xs, int tokens, int kind, float* out, int32_t* hq,
                                  float* hd, float* hs, void* workspace, int64_t workspace_bytes, void* stream) {
    LEAT_REQUIRE(hq && hd && hs && rows % GROUP == 0 && (uintptr_t)hq % 16 == 0,
                 "glu_matmul_q8: the q8 output needs d, s, rows in 32s and 16-byte aligned words");
    const void* ws[2] = {gate, up};
    // 3..16 tokens of Q4_K: the tile kernel writes the q8 itself
    if (few_tiles(type, cols, tokens, ws)) {
        if (mmq_check(type, gate, rows, cols, xq, xd, xs, tokens, hd) || mmq_check(type, up, rows, cols, xq, xd, xs, tokens, hd))
            return -1;
        LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matmul_q8: unknown GLU kind %d", kind);
        return few_tiles_glu(ws, rows, cols, xq, xd, xs, tokens, kind, out, hq, hd, hs, (hipStream_t)stream);
    }
    // few tokens (with the f32 output given), and types the Q4_K kernel does not take: the GLU,
    // then the quantizer on its f32 outputs
    if (type != Q4_K || (out && few_fits(type, cols, tokens, ws, 2))) {
        LEAT_REQUIRE(out, "glu_matmul_q8: type %d needs the f32 output", type);
        if (leat_glu_matmul(type, gate, up, rows, cols, xq, xd, xs, tokens, kind, out, workspace, workspace_bytes, stream))
            return -1;
        return leat_quantize_q8(out, tokens, rows, nullptr, 0.0f, hq, hd, hs, stream);
    }
    if (mmq_check(type, gate, rows, cols, xq, xd, xs, tokens, hd) || mmq_check(type, up, rows, cols, xq, xd, xs, tokens, hd))
        return -1;
    LEAT_REQUIRE(kind >= GLU_SILU && kind <= GLU_OAI, "glu_matmul_q8: unknown GLU kind %d", kind);
    return prefill_launch(PF_GLU, ws, rows, cols, xq, xd, xs, tokens, nullptr, kind, out, (hipStream_t)stream,
                          (uint32_t*)hq, hd, hs, workspace, workspace_bytes);
}

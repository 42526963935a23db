// Decode products for 3..16 tokens of Q4_K weights on matrix cores: y[t, row] = W[row] . x[t],
// every weight read once for all tokens (leat/kernels/matvec.py:1-4, 306-395 at batch sizes above
// two). Q6_K's 210-byte blocks, which do not split into aligned 16-byte runs, take the LDS-staged
// kernels of mmv.hip instead.
//
// Work split: a workgroup owns a tile of 32 consecutive rows (of gate and of up for the GLU); its
// S waves take every S-th block of the rows (wave w blocks w, w + S, ...), so at each step they
// read neighbouring blocks, whose shared 128-byte lines (a block is 144 bytes) are fetched once
// (contiguous runs a wave fetched 20% more than the weights); they add their sums through LDS at
// the end.
//
// Memory: every lane loads exactly the bytes its MFMA operand needs (row r = lane % 32, half
// h = lane / 32 of each group of 32 weights) straight into registers, the next block's loads in
// flight while the current one is computed; the tokens' q8 words are read from global memory (a
// few KB, hot in the caches) and their scales staged in LDS once per workgroup.
//
// Math: v_mfma_i32_32x32x32_i8 with the rows as N (operand B: lane l holds row l % 32) and the
// tokens as M (operand A: lane l holds token l % 32, zero past the last), K one group of 32. The
// int32 result in lane l is row l % 32 for tokens 8(v / 4) + 4h + v % 4 of its registers v; with
// at most 8 tokens (TOK = 8) the useful ones are v = 0..3, tokens 4h + v, with at most 16 v = 0..7,
// and they are scaled into f32 per group as
// leat's kernels combine each group's int32 dot (leat/kernels/matvec.py:107-181): lane h takes
// qs bytes [32j + 16h, +16) of pair j, whose low nibbles are group 2j's values 16h..16h+15 and
// high nibbles group 2j+1's; acc += d*sc*xd*D - dmin*m*xs.
// The GLU can also quantize its own outputs (the tile's 32 rows are one group of 32 per token)
// for the down product, as the one- and two-token kernels do.
#include "blocks.h"
#include "q8.h"
#include "tiles.h"

namespace leat {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

extern __shared__ uint32_t tiles_lds[];

constexpr size_t TILES_MAX_LDS = 160 * 1024;  // LDS a workgroup may have on gfx950

__device__ __forceinline__ v16i tiles_mfma(v4i a, u32x4 b) {
    const v16i zero = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, __builtin_bit_cast(v4i, b), zero, 0, 0, 0);
}

enum TilesMode : int { TILES_PLAIN = 0, TILES_RESIDUAL = 1, TILES_GLU = 2 };

// A block's bytes for the lane (row r, half h), loaded from the row's start.
template <int TYPE> struct TileBlock;

template <>
struct TileBlock<Q4_K> {
    static constexpr int BYTES = 144;
    struct Raw {
        u32x4 hdr;
        u32x4 qs[4];  // pair j: qs bytes [32j + 16h, +16)
    };
    __device__ static Raw load(const uint8_t* row, int b, int h) {
        const uint8_t* blk = row + 144u * (uint32_t)b;
        Raw r;
        r.hdr = stream_load((const u32x4*)blk);
#pragma unroll
        for (int j = 0; j < 4; j++) r.qs[j] = stream_load((const u32x4*)(blk + 16 + 32 * j + 16 * h));
        return r;
    }
};

// The tokens' activations: the q8 words of token t, group g at word t * cols / 4 + 8 g in global
// memory; the scale tables in LDS, group-major, TOK token slots a group (zero past the last
// token), d then s.
struct TileActs {
    const uint32_t* words;  // the lane's (token, half) words: token * cols / 4 + 4 h
    bool live;              // the lane's token is one of the tokens
    int d_off, s_off;       // the LDS tables' offsets in floats
    // operand A of block b's 8 groups: row l % 32 is token l % 32 (zero past the last token), read
    // from global memory (the few tokens' words stay in the caches). Issued before the next
    // block's weight loads, so that waiting for them (loads complete in order) does not wait for
    // those.
    __device__ void operands(int b, v4i (&xa)[8]) const {
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const v4i v = *(const v4i*)(words + 8 * (8 * b + s));
            const v4i zero = {};
            xa[s] = live ? v : zero;
        }
    }
    // tokens 8q + 4h .. 8q + 4h + 3 of group g, in a table of `tok` slots a group
    __device__ float4 scales(int off, int tok, int g, int q, int h) const {
        return *(const float4*)((const float*)tiles_lds + off + tok * g + 8 * q + 4 * h);
    }
};

// One block of NM matrices (gate and up for the GLU) for the lane: acc[k][v] += matrix k's share
// for the tokens 8(v / 4) + 4h + v % 4, v < TOK / 2. Each group's operand A and scale tables are
// read once for the matrices, whose products are issued back to back.
template <int TYPE> struct TileCompute;

template <>
struct TileCompute<Q4_K> {
    template <int NM, int TOK>
    __device__ static void run(const TileBlock<Q4_K>::Raw (&raw)[NM], int b, const v4i (&xa)[8], const TileActs& x,
                               int h, float (&acc)[NM][TOK / 2]) {
        float d[NM], dmin[NM];
#pragma unroll
        for (int k = 0; k < NM; k++) d[k] = f16_lo(raw[k].hdr[0]), dmin[k] = f16_hi(raw[k].hdr[0]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int s = 2 * j + e, g = 8 * b + s;
                const v4i a = xa[s];
                float4 xd[TOK / 8], xs[TOK / 8];
#pragma unroll
                for (int q = 0; q < TOK / 8; q++) xd[q] = x.scales(x.d_off, TOK, g, q, h), xs[q] = x.scales(x.s_off, TOK, g, q, h);
                v16i D[NM];
#pragma unroll
                for (int k = 0; k < NM; k++) {
                    const u32x4 w = e ? ((raw[k].qs[j] >> 4) & 0x0F0F0F0Fu) : (raw[k].qs[j] & 0x0F0F0F0Fu);
                    D[k] = tiles_mfma(a, w);
                }
#pragma unroll
                for (int k = 0; k < NM; k++) {
                    // get_scale_min_k4 (leat/quant.py:182-187), s known at compile time
                    const uint32_t sh = 8u * (uint32_t)(s & 3);
                    const uint32_t x0 = raw[k].hdr[1] >> sh, x1 = raw[k].hdr[2] >> sh, x2 = raw[k].hdr[3] >> sh;
                    const uint32_t scv = s < 4 ? (x0 & 63u) : ((x2 & 15u) | ((x0 >> 2) & 0x30u));
                    const uint32_t mv = s < 4 ? (x1 & 63u) : (((x2 >> 4) & 15u) | ((x1 >> 2) & 0x30u));
                    const float sc = d[k] * (float)scv, mn = dmin[k] * (float)mv;
#pragma unroll
                    for (int q = 0; q < TOK / 8; q++) {
                        acc[k][4 * q + 0] += sc * xd[q].x * (float)D[k][4 * q + 0] - mn * xs[q].x;
                        acc[k][4 * q + 1] += sc * xd[q].y * (float)D[k][4 * q + 1] - mn * xs[q].y;
                        acc[k][4 * q + 2] += sc * xd[q].z * (float)D[k][4 * q + 2] - mn * xs[q].z;
                        acc[k][4 * q + 3] += sc * xd[q].w * (float)D[k][4 * q + 3] - mn * xs[q].w;
                    }
                }
            }
        }
    }
};

template <int TYPE, int MODE, int S, int TOK>
__global__ __launch_bounds__(S * 64) void tiles_kernel(TileArgs a) {
    using TB = TileBlock<TYPE>;
    constexpr int NM = MODE == TILES_GLU ? 2 : 1;
    constexpr int TV = TOK / 2;  // result registers a lane keeps: tokens 8(v / 4) + 4h + v % 4
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int r = lane & 31, h = lane >> 5;
    const int cols = a.cols, tokens = a.tokens, G = cols / GROUP;
    const int nb = cols / 256;
    const uint32_t row_bytes = (uint32_t)nb * TB::BYTES;

    const int tile = blockIdx.x;
    int m = 0;
    if (MODE != TILES_GLU)
        while (m + 1 < a.count && tile >= a.tile_start[m + 1]) m++;
    const int rows = a.rows[m];
    const int row0 = (tile - a.tile_start[m]) * 32;
    const int row = min(row0 + r, rows - 1);  // rows past the end repeat the last (never stored)
    const uint8_t* wr[NM];
    wr[0] = (MODE == TILES_GLU ? a.w[0] : a.w[m]) + (size_t)row * row_bytes;
    if (NM == 2) wr[NM - 1] = a.w[1] + (size_t)row * row_bytes;

    // The tokens' scale tables go into LDS group-major, read in the source's order (token-major).
    // Their first TABLE_U entries a thread are asked for first, at clamped indices, then the
    // wave's first block of weights (blocks w, w + S, ...; a block index clamped into the row),
    // all unconditionally: the LDS writes then wait for the table alone (the compiler counts the
    // weight loads still in flight) and the barrier passes while the weights arrive.
    constexpr int TABLE_U = 4;
    const int entries = TOK * G, live_entries = tokens * G;
    float td[TABLE_U], ts[TABLE_U];
#pragma unroll
    for (int u = 0; u < TABLE_U; u++) {
        const int i = min((int)threadIdx.x + u * S * 64, live_entries - 1);
        td[u] = a.xd[i];
        ts[u] = a.xs[i];
    }
    __builtin_amdgcn_sched_barrier(0);  // the table's loads stay ahead of the weights'
    typename TB::Raw cur[NM];
#pragma unroll
    for (int k = 0; k < NM; k++) cur[k] = TB::load(wr[k], min(w, nb - 1), h);

    TileActs x;
    x.d_off = 0;
    x.s_off = TOK * G;
    {
        float* tab = (float*)tiles_lds;
#pragma unroll
        for (int u = 0; u < TABLE_U; u++) {
            const int i = (int)threadIdx.x + u * S * 64;
            if (i < entries) {
                const int t = i / G, g = i - t * G;
                const bool in = t < tokens;
                tab[TOK * g + t] = in ? td[u] : 0.0f;
                tab[TOK * G + TOK * g + t] = in ? ts[u] : 0.0f;
            }
        }
        // tables longer than TABLE_U entries a thread (rows of more than 4096 weights at 16 tokens)
        for (int i = threadIdx.x + TABLE_U * S * 64; i < entries; i += S * 64) {
            const int t = i / G, g = i - t * G;
            const bool in = t < tokens;
            tab[TOK * g + t] = in ? a.xd[i] : 0.0f;
            tab[TOK * G + TOK * g + t] = in ? a.xs[i] : 0.0f;
        }
        __syncthreads();
    }
    x.live = r < tokens;
    x.words = (const uint32_t*)a.xq + (int64_t)(x.live ? r : 0) * (cols / 4) + 4 * h;

    float acc[NM][TV];
#pragma unroll
    for (int k = 0; k < NM; k++)
#pragma unroll
        for (int v = 0; v < TV; v++) acc[k][v] = 0.0f;

    for (int b = w; b < nb; b += S) {
        v4i xa[8];
        x.operands(b, xa);
        typename TB::Raw nxt[NM];
        if (b + S < nb)
#pragma unroll
            for (int k = 0; k < NM; k++) nxt[k] = TB::load(wr[k], b + S, h);
        TileCompute<TYPE>::template run<NM, TOK>(cur, b, xa, x, h, acc);
        if (b + S < nb)
#pragma unroll
            for (int k = 0; k < NM; k++) cur[k] = nxt[k];
    }

    // the S waves' sums, through LDS (after the activations' last reads)
    __syncthreads();
    float* red = (float*)tiles_lds;
    if (S > 1) {
#pragma unroll
        for (int k = 0; k < NM; k++)
#pragma unroll
            for (int v = 0; v < TV; v++) red[((w * NM + k) * TV + v) * 64 + lane] = acc[k][v];
        __syncthreads();
        if (w != 0) return;
#pragma unroll
        for (int k = 0; k < NM; k++)
#pragma unroll
            for (int v = 0; v < TV; v++) {
                float sum = 0.0f;
                for (int i = 0; i < S; i++) sum += red[((i * NM + k) * TV + v) * 64 + lane];
                acc[k][v] = sum;
            }
    }
    // wave 0: lane (r, h) holds row row0 + r for tokens 8(v / 4) + 4h + v % 4
    const bool row_in = row0 + r < rows;
    float y[TV];
#pragma unroll
    for (int v = 0; v < TV; v++) {
        const int t = 8 * (v / 4) + 4 * h + v % 4;
        y[v] = acc[0][v];
        if (MODE == TILES_GLU) y[v] = glu(a.kind, acc[0][v], acc[NM - 1][v]);
        const int64_t at = (int64_t)t * rows + row0 + r;
        if (MODE == TILES_RESIDUAL && t < tokens && row_in) y[v] += a.residual[at];
        float* out = a.out[MODE == TILES_GLU ? 0 : m];
        if (out && t < tokens && row_in) out[at] = y[v];
    }
    // the GLU's outputs quantized: for each token the tile's 32 rows are one group of 32
    if (MODE == TILES_GLU && a.hq) {
#pragma unroll
        for (int v = 0; v < TV; v++) {
            const int t = 8 * (v / 4) + 4 * h + v % 4;
            float scale, sum;
            const uint32_t word = quantize_lane32(y[v], &scale, &sum);
            if (t < tokens) {
                if ((r & 3) == 0) a.hq[((int64_t)t * rows + row0 + r) / 4] = word;
                if (r == 0) {
                    const int64_t g = ((int64_t)t * rows + row0) / GROUP;
                    a.hd[g] = scale;
                    a.hs[g] = sum;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------- launching

constexpr int TILES_WAVES = 2048;  // waves a launch aims for

template <int TYPE, int MODE, int S, int TOK>
static int tiles_go(TileArgs& a, hipStream_t st) {
    const int tiles = a.tile_start[a.count];
    const int G = a.cols / GROUP;
    const size_t acts = (size_t)2 * TOK * G * 4;  // the scale tables
    const size_t red = (size_t)S * (MODE == TILES_GLU ? 2 : 1) * (TOK / 2) * 64 * 4;
    const size_t lds = acts > red ? acts : red;
    // a workgroup's LDS beyond 64 KB is allowed once per kernel
    static const hipError_t allowed = hipFuncSetAttribute((const void*)tiles_kernel<TYPE, MODE, S, TOK>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                                          (int)TILES_MAX_LDS);
    if (allowed != hipSuccess && lds > 64 * 1024) {
        set_error("tiles: %zu bytes of LDS refused", lds);
        return -1;
    }
    hipLaunchKernelGGL((tiles_kernel<TYPE, MODE, S, TOK>), dim3(tiles), dim3(S * 64), lds, st, a);
    return check_launch("tiles");
}

template <int TYPE, int MODE, int TOK>
static int tiles_s(TileArgs& a, hipStream_t st) {
    const int tiles = a.tile_start[a.count];
    const int blocks = a.cols / 256;
    // waves per tile: enough for the launch to fill the GPU, a few blocks each
    const int want = (TILES_WAVES + tiles - 1) / tiles;
    // (16 waves fit 1024 threads' 128 registers a lane only for the plain products of 8 tokens)
    if constexpr (MODE != TILES_GLU && TOK == 8)
        if (want >= 16 && blocks >= 32) return tiles_go<TYPE, MODE, 16, TOK>(a, st);
    if (want >= 8 && blocks >= 16) return tiles_go<TYPE, MODE, 8, TOK>(a, st);
    if (want >= 4 && blocks >= 8) return tiles_go<TYPE, MODE, 4, TOK>(a, st);
    if (want >= 2 && blocks >= 2) return tiles_go<TYPE, MODE, 2, TOK>(a, st);
    return tiles_go<TYPE, MODE, 1, TOK>(a, st);
}

// 3..8 tokens keep four result registers a lane, 9..16 eight
template <int TYPE, int MODE>
static int tiles_t(TileArgs& a, hipStream_t st) {
    return a.tokens <= 8 ? tiles_s<TYPE, MODE, 8>(a, st) : tiles_s<TYPE, MODE, 16>(a, st);
}

bool tiles_fits(int type, int cols, int tokens, const void* const* ws, int count) {
    // Q4_K only: Q6_K's 210-byte blocks load faster staged through LDS (the mmv kernels)
    if (tokens < 3 || tokens > 16 || type != Q4_K || cols % 256 != 0) return false;
    // the tokens' scale tables in LDS (160 KB a workgroup on gfx950)
    if ((size_t)2 * (tokens <= 8 ? 8 : 16) * (cols / GROUP) * 4 > TILES_MAX_LDS) return false;
    for (int i = 0; i < count; i++)
        if ((uintptr_t)ws[i] % 16 != 0) return false;
    return true;
}

int tiles_launch(int type, int mode, TileArgs& a, hipStream_t st) {
    int total = 0;
    for (int i = 0; i < a.count; i++) {
        a.tile_start[i] = total;
        total += (a.rows[i] + 31) / 32;
    }
    a.tile_start[a.count] = total;
#define LEAT_TILES_MODES(T)                                                 \
    switch (mode) {                                                         \
    case TILES_PLAIN: return tiles_t<T, TILES_PLAIN>(a, st);                \
    case TILES_RESIDUAL: return tiles_t<T, TILES_RESIDUAL>(a, st);          \
    default: return tiles_t<T, TILES_GLU>(a, st);                           \
    }
    switch (type) {
    case Q4_K: LEAT_TILES_MODES(Q4_K)
    default: set_error("tiles: unsupported type %d", type); return -1;
    }
#undef LEAT_TILES_MODES
}

}  // namespace leat

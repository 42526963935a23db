// Prefill products of Q4_K weights on matrix cores (leat/kernels/matmul.py: llama.cpp's MMQ),
// out[t, r] = W[r] . x[t] for many tokens, the activations quantized to int8 per group of 32 as
// for decode. Each group's int32 product comes from v_mfma_i32_32x32x32_i8 and is scaled into f32
// sums as leat's _Q4KTile.scaled (leat/kernels/matmul.py:285-291):
//   acc += (d * sc) * xd * D  -  (dmin * m) * xs
//
// Work split: a workgroup of 4 waves owns 64 tokens and 128 rows (the GLU: 64 rows of gate and
// the same 64 of up). Each wave owns one tile of 32 rows for both 32-token tiles, so every weight
// operand it decodes serves two products.
//
// Memory: the K loop takes one block (256 weights) of every row a step. The step's weight blocks,
// the tokens' 256 int8 values and their scale tables go straight from global memory into LDS
// (global_load_lds, no registers), double-buffered: the next step's loads are in flight while
// this step is computed, and one barrier a step hands the buffer over. LDS holds each kind
// chunk-major: the 16-byte chunk p of the 128 rows' blocks side by side, chunk c of the 64
// tokens' step values side by side, each group's scale of the 64 tokens side by side. An operand
// read of 32 rows or tokens is then 512 consecutive bytes (no bank conflicts), and every direct
// load is a uniform pointer plus a fixed per-lane offset.
// Workgroups that share a row tile are launched on one XCD (workgroup ids are dealt round-robin
// over the 8 XCDs), so its weights are fetched into that XCD's L2 once.
//
// Math, per group g of 32 and 32x32 tile: D = mfma_i8(x operand, w operand) with the tokens as M
// (operand A: lane l holds token l % 32, lane half h = l / 32 values 16h..16h+15 of the group)
// and the rows as N (operand B: lane l holds row l % 32, the same values); the int32 result in
// lane l is row l % 32 for tokens 8(v / 4) + 4h + v % 4 of registers v. The f32 scale matrices
// xd (x) (d * sc) of both token tiles come from one v_mfma_f32_32x32x1_2b_f32 (two outer
// products), in the layout of D, so acc[v] += D[v] * S[v] is two VALU ops an element. The mins
// take one more f32 product per pair of groups: K = 2 is the pair (lane half h supplies group
// 2j + h), added on the matrix cores straight into the sums at the end of a step.
#include "blocks.h"
#include "lds.h"
#include "prefill.h"
#include "q8.h"

namespace leat {

namespace {

using namespace pf;

constexpr int PF_WAVES = 4;
constexpr int PF_TOKENS = 64;              // tokens per workgroup: two tiles of 32
constexpr int PF_ROWS = 32 * PF_WAVES;     // rows staged per workgroup
constexpr int PF_BLOCK = 144;              // Q4_K block bytes
constexpr int PF_W_BYTES = PF_ROWS * PF_BLOCK;          // 18432: [9 chunks][128 rows][16 B]
constexpr int PF_X_BYTES = PF_TOKENS * 256;             // 16384: [16 chunks][64 tokens][16 B]
constexpr int PF_T_BYTES = 8 * PF_TOKENS * 4;           // one scale table: 2048, [8 groups][64 tokens]
constexpr int PF_BUF = PF_W_BYTES + PF_X_BYTES + 2 * PF_T_BYTES;  // 38912
constexpr int PF_LDS = 2 * PF_BUF;                      // 77824: two workgroups fit a CU

struct PrefillArgs {
    const uint8_t* w[2];  // the GLU: gate, up
    float* out;
    int rows, cols, tokens;
    const int32_t* xq;
    const float* xd;
    const float* xs;
    const float* residual;
    int kind;
    uint32_t* hq;  // the GLU: the q8 of its outputs (quantize_q8 of each token's row), or null
    float* hd;
    float* hs;
    int row_tiles, token_tiles;  // workgroup tiles of PF_ROWS (the GLU: PF_ROWS / 2) rows and PF_TOKENS tokens
    // split products (chunks > 1): each tile's steps are dealt over `chunks` workgroups, which
    // leave their sums in `parts` for prefill_fixup_q4k to add in chunk order
    int chunks;
    float* parts;  // [tile][chunk][wave][token tile q][register v][lane]
};

extern __shared__ __attribute__((aligned(16))) uint8_t pf_lds[];

// one group's operands (read from LDS) and products (matrix-core results) for the wave's two
// token tiles
struct GroupOps {
    v4i x[2];
    float xd;  // of token r of tile h (lane half h)
    u32x4 b;
    float wsc;
};
struct GroupRes {
    v16i D[2];
    v32f S;  // tile q's scales in registers 16q..16q+15
};

// The lanes' fixed parts of the direct loads. Every load reads consecutive bytes: one of weights
// brings 64 consecutive 16-byte chunks of one matrix's 64 rows' step blocks (576 chunks, 9 loads),
// which land row after row (row R's chunk p at byte 144 R + 16 p of the weights); one of
// activations 4 tokens' 256 values; one of scales 8 tokens' 8 groups.
struct StageOffsets {
    uint32_t w[5];    // weight loads i = w + 4u: chunk 64 (i % 9) + lane's byte past the step block of the load's first row
    uint32_t xt, xc;  // activations: token lane / 16 of a load's 4; its source chunk (lane % 16) ^ (token % 16), in bytes
    uint32_t tt;      // scales: token lane / 8 of a load's 8
    uint32_t tg[2];   // ... and its source group (lane % 8) ^ s, for the loads s = w and w + 4
};

// row R (of 64) and chunk p of weight load i's lane `lane`
__device__ __forceinline__ void chunk_of(int i, int lane, int& R, int& p) {
    const int c = 64 * (i % 9) + lane;
    R = c / 9;
    p = c - 9 * R;
}

// Issues the direct loads of step `step` into the buffer at LDS address `buf`. An instruction
// fills 64 consecutive 16-byte (or 4-byte) LDS slots, one per lane: the weights row after row
// (matrix half i / 9: the GLU's up, else rows 64..127), the activations token after token (chunk
// c of token t at chunk slot c ^ (t % 16)), the scales token after token (group s of token t at
// slot s ^ (t / 8 % 8); xd of the 64 tokens, then xs).
template <int MODE>
__device__ __forceinline__ void stage(const PrefillArgs& a, const StageOffsets& o, int row0, int tok0, bool full,
                                      uint32_t buf, int step, int w) {
    const uint32_t row_bytes = (uint32_t)(a.cols / 256) * PF_BLOCK;
#pragma unroll
    for (int u = 0; u < 5; u++) {
        const int i = w + PF_WAVES * u;
        if (i >= 18) break;
        const int half = i >= 9;
        const uint8_t* m = MODE == PF_GLU && half ? a.w[1] : a.w[0];
        const int first = row0 + (MODE == PF_GLU ? 0 : 64 * half);  // the load's first row
        const uint8_t* src = m + (size_t)first * row_bytes + (uint32_t)step * PF_BLOCK + o.w[u];
        if (!full) {  // a partial last tile: rows past the end read the last row
            int R, p;
            chunk_of(i, threadIdx.x & 63, R, p);
            src = m + (size_t)min(first + R, a.rows - 1) * row_bytes + (uint32_t)step * PF_BLOCK + 16u * (uint32_t)p;
        }
        to_lds16(src, buf + 1024 * i);
    }
    const uint32_t xbase = buf + PF_W_BYTES, tbase = xbase + PF_X_BYTES;
#pragma unroll
    for (int u = 0; u < 16 / PF_WAVES; u++) {  // activations: tokens 4i .. 4i + 3
        const int i = w + PF_WAVES * u;
        const size_t tok = (size_t)min(tok0 + 4 * i + (int)o.xt, a.tokens - 1);
        to_lds16((const uint8_t*)a.xq + tok * a.cols + 256u * step + o.xc, xbase + 1024 * i);
    }
    const int groups = a.cols / GROUP;
#pragma unroll
    for (int u = 0; u < 16 / PF_WAVES; u++) {  // scales: xd (i < 8), then xs, of tokens 8s .. 8s + 7
        const int i = w + PF_WAVES * u, s = i & 7;
        const float* tab = i < 8 ? a.xd : a.xs;
        const size_t tok = (size_t)min(tok0 + 8 * s + (int)o.tt, a.tokens - 1);
        to_lds4(tab + tok * groups + 8 * step + o.tg[u & 1], tbase + 256 * i);
    }
}

// the sums' slice of one (tile, chunk) in `parts`: 2 token tiles x 16 registers x 64 lanes a wave
constexpr int PF_PART = PF_WAVES * 2 * 16 * 64;

template <int MODE>
__device__ void pf_finish(const PrefillArgs& a, v16f (&acc)[2], int row0, int tok0, int w, int lane);

template <int MODE>
__global__ __launch_bounds__(64 * PF_WAVES, 2) void prefill_q4k(PrefillArgs a) {
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int r = lane & 31, h = lane >> 5;

    // workgroup id -> (chunk, tiles): ids on one XCD (id % 8) walk its row tiles' token tiles in
    // turn; a split product repeats that walk once per chunk
    const int per_chunk = (a.row_tiles + 7) / 8 * 8 * a.token_tiles;
    const int chunk = blockIdx.x / per_chunk, id = blockIdx.x - chunk * per_chunk;
    const int xcd = id & 7, local = id >> 3;
    const int tt = local % a.token_tiles, rt = (local / a.token_tiles) * 8 + xcd;
    if (rt >= a.row_tiles) return;
    constexpr int OUT_ROWS = MODE == PF_GLU ? PF_ROWS / 2 : PF_ROWS;
    const int row0 = rt * OUT_ROWS, tok0 = tt * PF_TOKENS;
    const int all_steps = a.cols / 256;
    // this chunk's steps [first, first + steps): all of them unless the product is split
    const int first = chunk * all_steps / a.chunks, steps = (chunk + 1) * all_steps / a.chunks - first;
    const uint32_t row_bytes = (uint32_t)all_steps * PF_BLOCK;
    const uint32_t lds0 = (uint32_t)(uintptr_t)pf_lds;

    StageOffsets so;
    {
#pragma unroll
        for (int u = 0; u < 5; u++) {
            int R, p;
            chunk_of(w + PF_WAVES * u, lane, R, p);
            so.w[u] = (uint32_t)R * row_bytes + 16u * (uint32_t)p;
        }
        so.xt = (uint32_t)lane >> 4;
        so.xc = 16u * (((uint32_t)lane & 15u) ^ ((4u * (uint32_t)w + ((uint32_t)lane >> 4)) & 15u));
        so.tt = (uint32_t)lane >> 3;
        so.tg[0] = ((uint32_t)lane & 7u) ^ (uint32_t)w;
        so.tg[1] = ((uint32_t)lane & 7u) ^ (uint32_t)(w + PF_WAVES);
    }
    const bool full = row0 + (MODE == PF_GLU ? 64 : 128) <= a.rows;
    stage<MODE>(a, so, row0, tok0, full, lds0, first, w);

    // the lane's LDS offsets within a buffer: its row's weights (of the 128: gate or the first 64
    // rows in waves 0, 1), token r's activations of tile q (chunk c = 2g + h at (xo ^ 32g) +
    // 8192 q), xd of token r of tile h (group g at td ^ 4g) and xs of token r of tile q (group
    // 2j + h at ts[q] ^ 8j)
    const uint32_t wo = PF_BLOCK * (32 * w + r);
    const uint32_t xo = PF_W_BYTES + 256u * r + ((16u * h) ^ (16u * (r & 15)));
    constexpr uint32_t TB = PF_W_BYTES + PF_X_BYTES;
    const uint32_t td = TB + 32u * (32 * h + r) + 4u * ((uint32_t)((32 * h + r) >> 3) & 7u);
    uint32_t ts[2];
#pragma unroll
    for (int q = 0; q < 2; q++)
        ts[q] = TB + PF_T_BYTES + 32u * (32 * q + r) + 4u * ((uint32_t)h ^ ((uint32_t)((32 * q + r) >> 3) & 7u));

    v16f acc[2] = {};

    for (int step = 0; step < steps; step++) {
        wait_loads();                        // this step's direct loads are in LDS
        __syncthreads();                     // ... everyone's; and the other buffer is free
        const uint32_t buf = lds0 + (uint32_t)(step & 1) * PF_BUF;
        if (step + 1 < steps)
            stage<MODE>(a, so, row0, tok0, full, lds0 + (uint32_t)((step + 1) & 1) * PF_BUF, first + step + 1, w);

        const uint32_t wl = buf + wo;

        // the step's mins, - dmin * m[row] * xs[token], on the matrix cores straight into the
        // sums: K = 2 is a pair of groups, 2j in lane half 0 and 2j + 1 in half 1. Issued first,
        // so that their chain of products runs while the groups' pipeline fills; the 8 xs reads
        // go out together, so their LDS latencies overlap instead of queueing one per product
        float xsv[4][2];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int q = 0; q < 2; q++) xsv[j][q] = lds_read<float>(buf + (ts[q] ^ (8u * j)));
        const u32x4 hdr = lds_read<u32x4>(wl);
        const float d = f16_lo(hdr[0]), dmin = f16_hi(hdr[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int g = 2 * j + h;
            const uint32_t sh = 8u * (uint32_t)(g & 3);
            const uint32_t x1 = hdr[2] >> sh, x2 = hdr[3] >> sh;
            const uint32_t mv = g < 4 ? (x1 & 63u) : (((x2 >> 4) & 15u) | ((x1 >> 2) & 0x30u));
            const float mn = -dmin * (float)mv;
#pragma unroll
            for (int q = 0; q < 2; q++) acc[q] = mfma_f32(xsv[j][q], mn, acc[q]);
        }

        // The step's 8 groups as a three-stage pipeline: the operands of group g + 2 are read from
        // LDS while the products of group g + 1 are issued and those of group g are scaled, so
        // neither LDS nor matrix-core latency stands between one group's VALU work and the next.
        GroupOps op[8];
        GroupRes rs[8];
        u32x4 qs = {};
        auto read = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            if constexpr (g % 2 == 0) qs = lds_read<u32x4>(wl + 16 * h + 16 * (1 + g));  // chunk 1 + 2j + h
            op[g].b = g % 2 ? ((qs >> 4) & 0x0F0F0F0Fu) : (qs & 0x0F0F0F0Fu);
            // get_scale_min_k4 (leat/quant.py:182-187): the group's 6-bit scale
            constexpr uint32_t sh = 8u * (g & 3);
            const uint32_t x0 = hdr[1] >> sh, x2 = hdr[3] >> sh;
            const uint32_t scv = g < 4 ? (x0 & 63u) : ((x2 & 15u) | ((x0 >> 2) & 0x30u));
            op[g].wsc = d * (float)scv;
#pragma unroll
            for (int q = 0; q < 2; q++) {
                op[g].x[q] = lds_read<v4i>(buf + (xo ^ (32u * g)) + 8192 * q);  // chunk 2g + h of token 32q + r
            }
            op[g].xd = lds_read<float>(buf + (td ^ (4u * g)));
        };
        auto issue = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
#pragma unroll
            for (int q = 0; q < 2; q++) rs[g].D[q] = mfma_i8(op[g].x[q], op[g].b);
            rs[g].S = mfma_outer2(op[g].xd, op[g].wsc);  // xd[token] * d * sc[row], both tiles
        };
        auto scale = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[q][v] += (float)rs[g].D[q][v] * rs[g].S[16 * q + v];
        };
        read(std::integral_constant<int, 0>{});
        read(std::integral_constant<int, 1>{});
        issue(std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, 8>([&](auto kc) __attribute__((always_inline)) {
            constexpr int k = decltype(kc)::value;
            if constexpr (k + 2 < 8) read(std::integral_constant<int, k + 2>{});
            if constexpr (k + 1 < 8) issue(std::integral_constant<int, k + 1>{});
            scale(kc);
            // the sums are due here: without this the compiler sinks every group's scaling below
            // the last group's products, keeping all their results live
            asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
            __builtin_amdgcn_sched_barrier(0);  // keeps the stages' registers bounded
        });
    }

    if (a.chunks > 1) {  // a chunk's sums, for the fixup to add (coalesced: register v of 64 lanes at a time)
        float* dst = a.parts + ((size_t)(rt * a.token_tiles + tt) * a.chunks + chunk) * PF_PART + w * (2 * 16 * 64) + lane;
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int v = 0; v < 16; v++) dst[(q * 16 + v) * 64] = acc[q][v];
        return;
    }
    pf_finish<MODE>(a, acc, row0, tok0, w, lane);
}

// The outputs of one workgroup's tile from its sums acc (lane (r, h) of wave w holding row 32w + r
// of the staged rows for tokens 32q + 8(v / 4) + 4h + v % 4): the GLU of gate and up, the q8 of
// those, the residual, the stores. Every wave of the workgroup calls it.
template <int MODE>
__device__ void pf_finish(const PrefillArgs& a, v16f (&acc)[2], int row0, int tok0, int w, int lane) {
    const int r = lane & 31, h = lane >> 5;
    int wave_row = 32 * w + r;
    if (MODE == PF_GLU) {
        // the up waves (2, 3) hand their sums to the gate waves (0, 1) through LDS
        __syncthreads();
        float* xchg = (float*)pf_lds;
        if (w >= 2) {
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int v = 0; v < 16; v++) xchg[(((w - 2) * 2 + q) * 16 + v) * 64 + lane] = acc[q][v];
        }
        __syncthreads();
        if (w >= 2) return;
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[q][v] = glu(a.kind, acc[q][v], xchg[((w * 2 + q) * 16 + v) * 64 + lane]);
    }
    const int row = row0 + wave_row;
    // the GLU's outputs quantized as quantize_q8 would (q8.h's arithmetic): the two gate waves
    // put their outputs in LDS token by token (64 rows a token, padded to 68 floats), then each of
    // their 128 threads quantizes one group of 32 rows of one token in its own registers
    if (MODE == PF_GLU && a.hq) {
        float* yt = (float*)pf_lds + 2 * 2 * 16 * 64;  // past the exchange area
        constexpr int YS = 68;
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int v = 0; v < 16; v++) yt[(32 * q + 8 * (v >> 2) + 4 * h + (v & 3)) * YS + wave_row] = acc[q][v];
        __syncthreads();  // the two gate waves (waves 2 and 3 have ended, and a barrier waits for none)
        const int tid = threadIdx.x, tl = tid >> 1, grp = tid & 1;  // token tl, rows 32 grp ..
        const int t = tok0 + tl, first = row0 + 32 * grp;
        if (t < a.tokens && first < a.rows) {
            float v[32];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 c = *(const float4*)(yt + tl * YS + 32 * grp + 4 * i);
                v[4 * i] = c.x, v[4 * i + 1] = c.y, v[4 * i + 2] = c.z, v[4 * i + 3] = c.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
            const float scale = amax / 127.0f;
            const float rs = __builtin_amdgcn_rcpf(scale);
            int total = 0;
            uint32_t word[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                uint32_t wv = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int qv = scale > 0.0f ? round_quotient(v[4 * i + k], scale, rs) : 0;
                    total += qv;
                    wv |= (uint32_t)(qv & 0xFF) << (8 * k);
                }
                word[i] = wv;
            }
            const size_t at = (size_t)t * a.rows + first;
            u32x4* dst = (u32x4*)(a.hq + at / 4);
            dst[0] = u32x4{word[0], word[1], word[2], word[3]};
            dst[1] = u32x4{word[4], word[5], word[6], word[7]};
            a.hd[at / GROUP] = scale;
            a.hs[at / GROUP] = scale * (float)total;
        }
    }
    if (row >= a.rows || !a.out) return;
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int t = tok0 + 32 * q + 8 * (v >> 2) + 4 * h + (v & 3);
            if (t >= a.tokens) continue;
            const size_t at = (size_t)t * a.rows + row;
            float y = acc[q][v];
            if (MODE == PF_RESIDUAL) y += a.residual[at];
            a.out[at] = y;
        }
}

// A split product's tiles: the chunks' sums added in chunk order (the same sums whichever
// workgroup ran first), then the tile's outputs as the main kernel would have written them.
template <int MODE>
__global__ __launch_bounds__(64 * PF_WAVES) void prefill_fixup_q4k(PrefillArgs a) {
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int tile = blockIdx.x, rt = tile / a.token_tiles, tt = tile - rt * a.token_tiles;
    constexpr int OUT_ROWS = MODE == PF_GLU ? PF_ROWS / 2 : PF_ROWS;
    const float* src = a.parts + (size_t)tile * a.chunks * PF_PART + w * (2 * 16 * 64) + lane;
    v16f acc[2] = {};
    for (int c = 0; c < a.chunks; c++, src += PF_PART)
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[q][v] += src[(q * 16 + v) * 64];
    pf_finish<MODE>(a, acc, rt * OUT_ROWS, tt * PF_TOKENS, w, lane);
}

// LDS the fixup's epilogue uses: the GLU's exchange of up sums, then 64 tokens' rows for the q8
constexpr int PF_FIXUP_LDS = 2 * 2 * 16 * 64 * 4 + 64 * 68 * 4;

template <int MODE>
int prefill_go(PrefillArgs& a, hipStream_t st) {
    // ids cover whole groups of 8 row tiles (one per XCD), once per chunk; ids past the last row
    // tile exit at once
    const int groups = (a.row_tiles + 7) / 8;
    const int grid = groups * 8 * a.token_tiles * a.chunks;
    static const hipError_t allowed = hipFuncSetAttribute((const void*)prefill_q4k<MODE>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS);
    if (allowed != hipSuccess) {
        set_error("prefill: %d bytes of LDS refused", PF_LDS);
        return -1;
    }
    hipLaunchKernelGGL((prefill_q4k<MODE>), dim3(grid), dim3(64 * PF_WAVES), PF_LDS, st, a);
    if (check_launch("prefill")) return -1;
    if (a.chunks > 1) {
        hipLaunchKernelGGL((prefill_fixup_q4k<MODE>), dim3(a.row_tiles * a.token_tiles), dim3(64 * PF_WAVES),
                           PF_FIXUP_LDS, st, a);
        return check_launch("prefill fixup");
    }
    return 0;
}

}  // namespace

Split prefill_split(int mode, int rows, int cols, int tokens) {
    const int out_rows = mode == PF_GLU ? PF_ROWS / 2 : PF_ROWS;
    const int tiles = (rows + out_rows - 1) / out_rows * ((tokens + PF_TOKENS - 1) / PF_TOKENS);
    return split_schedule(tiles, cols / 256, (int64_t)PF_PART * 4);
}

int prefill_launch(int mode, const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                   const float* xs, int tokens, const float* residual, int kind, float* out, hipStream_t st,
                   uint32_t* hq, float* hd, float* hs, void* workspace, int64_t workspace_bytes) {
    PrefillArgs a = {};
    const int out_rows = mode == PF_GLU ? PF_ROWS / 2 : PF_ROWS;
    a.row_tiles = (rows + out_rows - 1) / out_rows;
    a.token_tiles = (tokens + PF_TOKENS - 1) / PF_TOKENS;
    const Split sp = prefill_split(mode, rows, cols, tokens);
    a.chunks = 1;
    if (sp.chunks > 1 && workspace && workspace_bytes >= sp.bytes) a.chunks = sp.chunks, a.parts = (float*)workspace;
    a.hq = hq, a.hd = hd, a.hs = hs;
    a.w[0] = (const uint8_t*)ws[0];
    a.w[1] = (const uint8_t*)ws[mode == PF_GLU ? 1 : 0];
    a.out = out;
    a.rows = rows, a.cols = cols, a.tokens = tokens;
    a.xq = xq, a.xd = xd, a.xs = xs;
    a.residual = residual;
    a.kind = kind;
    switch (mode) {
    case PF_PLAIN: return prefill_go<PF_PLAIN>(a, st);
    case PF_RESIDUAL: return prefill_go<PF_RESIDUAL>(a, st);
    default: return prefill_go<PF_GLU>(a, st);
    }
}

}  // namespace leat

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
    int row_tiles, token_tiles;  // workgroup tiles of PF_ROWS (the GLU: PF_ROWS / 2) rows and PF_TOKENS tokens
};

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

// The lanes' fixed offsets of the direct loads: every load of a step is a uniform pointer (in
// scalar registers) plus one of these.
struct StageOffsets {
    uint32_t w[2];  // row (row0 + 64 half + lane)'s first byte in its matrix (the GLU: row0 + lane in both)
    uint32_t x;     // token (tok0 + lane)'s first q8 byte
    uint32_t t;     // token (tok0 + lane)'s first scale, in bytes
};

// Issues the direct loads of step `step` into the buffer at LDS address `buf`. An instruction
// fills 64 consecutive 16-byte (or 4-byte) LDS slots, one per lane: weights chunk p of 64 rows
// (slots [p][row]), activations chunk c of the 64 tokens (slots [c][token]), one group's scale of
// the 64 tokens (slots [g][token]).
template <int MODE>
__device__ __forceinline__ void stage(const PrefillArgs& a, const StageOffsets& o, uint32_t buf, int step, int w) {
    for (int i = w; i < 18; i += PF_WAVES) {  // weights: chunk p = i % 9 of the rows of half i / 9
        const int half = i >= 9, part = i - 9 * half;
        const uint8_t* m = MODE == PF_GLU && half ? a.w[1] : a.w[0];
        to_lds16(m + (uint32_t)step * PF_BLOCK + 16 * part + o.w[half], buf + 2048 * part + 1024 * half);
    }
    const uint32_t xbase = buf + PF_W_BYTES, tbase = xbase + PF_X_BYTES;
#pragma unroll
    for (int u = 0; u < 16 / PF_WAVES; u++) {  // activations: chunk c of every token
        const int c = w + PF_WAVES * u;
        to_lds16((const uint8_t*)a.xq + 256 * step + 16 * c + o.x, xbase + 1024 * c);
    }
#pragma unroll
    for (int u = 0; u < 16 / PF_WAVES; u++) {  // scales: group g of xd (i < 8), then of xs
        const int i = w + PF_WAVES * u, g = i & 7;
        const float* tab = i < 8 ? a.xd : a.xs;
        to_lds4((const uint8_t*)(tab + 8 * step + g) + o.t, tbase + 256 * i);
    }
}

template <int MODE>
__global__ __launch_bounds__(64 * PF_WAVES, 2) void prefill_q4k(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_lds[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int r = lane & 31, h = lane >> 5;

    // workgroup id -> tiles: ids on one XCD (id % 8) walk its row tiles' token tiles in turn
    const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
    const int tt = local % a.token_tiles, rt = (local / a.token_tiles) * 8 + xcd;
    if (rt >= a.row_tiles) return;
    constexpr int OUT_ROWS = MODE == PF_GLU ? PF_ROWS / 2 : PF_ROWS;
    const int row0 = rt * OUT_ROWS, tok0 = tt * PF_TOKENS;
    const int steps = a.cols / 256;
    const uint32_t row_bytes = (uint32_t)steps * PF_BLOCK;
    const uint32_t lds0 = (uint32_t)(uintptr_t)pf_lds;

    StageOffsets so;
    {
        const int half_rows = MODE == PF_GLU ? 0 : 64;
        so.w[0] = (uint32_t)min(row0 + lane, a.rows - 1) * row_bytes;
        so.w[1] = (uint32_t)min(row0 + half_rows + lane, a.rows - 1) * row_bytes;
        const int tok = min(tok0 + lane, a.tokens - 1);
        so.x = (uint32_t)tok * (uint32_t)a.cols;
        so.t = (uint32_t)tok * (uint32_t)(a.cols / GROUP) * 4u;
    }
    stage<MODE>(a, so, lds0, 0, w);

    v16f acc[2] = {};

    for (int step = 0; step < steps; step++) {
        wait_loads();                        // this step's direct loads are in LDS
        __syncthreads();                     // ... everyone's; and the other buffer is free
        const uint32_t buf = lds0 + (uint32_t)(step & 1) * PF_BUF;
        if (step + 1 < steps) stage<MODE>(a, so, lds0 + (uint32_t)((step + 1) & 1) * PF_BUF, step + 1, w);

        // lane (r, h)'s LDS bases: row 32w + r's chunks; token r's chunks of lane half h; token r's scales
        const uint32_t wl = buf + 16 * (32 * w + r);
        const uint32_t xl = buf + PF_W_BYTES + 1024 * h + 16 * r;
        const uint32_t tl = buf + PF_W_BYTES + PF_X_BYTES + 4 * r;
        const u32x4 hdr = lds_read<u32x4>(wl);
        const float d = f16_lo(hdr[0]), dmin = f16_hi(hdr[0]);

        // the step's mins, - dmin * m[row] * xs[token], on the matrix cores straight into the
        // sums: K = 2 is a pair of groups, 2j in lane half 0 and 2j + 1 in half 1. Issued first,
        // so that their chain of products runs while the groups' pipeline fills
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int g = 2 * j + h;
            const uint32_t sh = 8u * (uint32_t)(g & 3);
            const uint32_t x1 = hdr[2] >> sh, x2 = hdr[3] >> sh;
            const uint32_t mv = g < 4 ? (x1 & 63u) : (((x2 >> 4) & 15u) | ((x1 >> 2) & 0x30u));
            const float mn = -dmin * (float)mv;
#pragma unroll
            for (int q = 0; q < 2; q++) acc[q] = mfma_f32(lds_read<float>(tl + PF_T_BYTES + 256 * g + 128 * q), mn, acc[q]);
        }

        // The step's 8 groups as a three-stage pipeline: the operands of group g + 2 are read from
        // LDS while the products of group g + 1 are issued and those of group g are scaled, so
        // neither LDS nor matrix-core latency stands between one group's VALU work and the next.
        GroupOps op[8];
        GroupRes rs[8];
        u32x4 qs = {};
        auto read = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            if constexpr (g % 2 == 0) qs = lds_read<u32x4>(wl + 2048 * h + 2048 * (1 + g));  // chunk 1 + 2j + h
            op[g].b = g % 2 ? ((qs >> 4) & 0x0F0F0F0Fu) : (qs & 0x0F0F0F0Fu);
            // get_scale_min_k4 (leat/quant.py:182-187): the group's 6-bit scale
            constexpr uint32_t sh = 8u * (g & 3);
            const uint32_t x0 = hdr[1] >> sh, x2 = hdr[3] >> sh;
            const uint32_t scv = g < 4 ? (x0 & 63u) : ((x2 & 15u) | ((x0 >> 2) & 0x30u));
            op[g].wsc = d * (float)scv;
#pragma unroll
            for (int q = 0; q < 2; q++) {
                op[g].x[q] = lds_read<v4i>(xl + 512 * q + 2048 * g);  // chunk 2g + h of token t
            }
            op[g].xd = lds_read<float>(tl + 128 * h + 256 * g);
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

    // lane (r, h) holds row 32w + r of the staged rows for tokens 32q + 8(v / 4) + 4h + v % 4
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
    if (row >= a.rows) return;
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

template <int MODE>
int prefill_go(PrefillArgs& a, hipStream_t st) {
    const int out_rows = MODE == PF_GLU ? PF_ROWS / 2 : PF_ROWS;
    a.row_tiles = (a.rows + out_rows - 1) / out_rows;
    a.token_tiles = (a.tokens + PF_TOKENS - 1) / PF_TOKENS;
    // ids cover whole groups of 8 row tiles (one per XCD); ids past the last row tile exit at once
    const int groups = (a.row_tiles + 7) / 8;
    const int grid = groups * 8 * a.token_tiles;
    static const hipError_t allowed = hipFuncSetAttribute((const void*)prefill_q4k<MODE>,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS);
    if (allowed != hipSuccess) {
        set_error("prefill: %d bytes of LDS refused", PF_LDS);
        return -1;
    }
    hipLaunchKernelGGL((prefill_q4k<MODE>), dim3(grid), dim3(64 * PF_WAVES), PF_LDS, st, a);
    return check_launch("prefill");
}

}  // namespace

int prefill_launch(int mode, const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                   const float* xs, int tokens, const float* residual, int kind, float* out, hipStream_t st) {
    PrefillArgs a = {};
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

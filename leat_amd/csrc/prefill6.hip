// Prefill products of Q6_K weights on matrix cores (leat/kernels/matmul.py: llama.cpp's MMQ with
// _Q6KTile, :334-387), out[t, r] = W[r] . x[t] (+ residual) for many tokens, the activations
// quantized to int8 per group of 32 as for decode.
//
// Q6_K (leat/quant.py:213-223): a block of 256 weights holds ql[128], qh[64], 16 int8 scales and
// an f16 d. Weight 128n + 32k + l is (nibble k / 2 of ql[64n + 32(k % 2) + l] | bits 2k of
// qh[32n + l] << 4) - 32, scaled by d * scales[8n + 2k + l / 16]. Group g = 4n + k of 32 weights
// thus has one scale per half, and half h = l / 16 is exactly the K slice that lane half h
// supplies to v_mfma_i32_32x32x32_i8.
//
// Math, per group and 32x32 tile (tokens as M, rows as N): Df = the group's int8 product, Dh the
// product over half 1 only (the activation operand of lane half 0 read from a zeroed stretch of
// LDS). The group's int32 sum
// sc0 * (Df - Dh) + sc1 * Dh = sc0 * Df + (sc1 - sc0) * Dh is exact, and below 2^24 in magnitude,
// so its f32 conversion is exact too. It is scaled by xd[token] * d[row] (one
// v_mfma_f32_32x32x1_2b_f32 gives that matrix for a pair of groups) into the f32 sums, the
// arithmetic of _Q6KTile.scaled with the two halves' products summed in int32 first.
//
// Work split: a workgroup of 4 waves owns 64 rows and 64 tokens, each wave one 32x32 tile, so a
// 4096-row, 512-token product keeps two workgroups on every CU.
//
// Memory: the K loop takes one block of every row a step. The step's bytes go straight from
// global memory into LDS (global_load_lds), double-buffered, each load reading consecutive bytes:
// - weights: a block starts 2 bytes off a 4-byte boundary in odd blocks (rows are 4-byte
//   aligned, blocks 210 bytes), so a row loads the 53 dwords around its block (from the block
//   start rounded down to 4) with one dword load of 64 lanes into a 272-byte LDS slot. Reads of
//   one offset by 32 rows then hit distinct banks; odd blocks are shifted 2 bytes in registers.
// - activations: one 16-byte load brings 4 tokens' 256 values; chunk c of token t lands at
//   chunk slot c ^ (t % 16), so reads of one chunk by 32 tokens hit distinct banks.
// - xd: one dword load brings 8 tokens' 8 group scales; group s of token t at slot s ^ (t / 8 % 8).
// Workgroups that share a row tile run on one XCD (workgroup ids are dealt round-robin over the
// 8 XCDs), so its weights are fetched into that XCD's L2 once.
#include "blocks.h"
#include "lds.h"
#include "prefill.h"

namespace leat {

namespace {

using namespace pf;

constexpr int P6_WAVES = 4;
constexpr int P6_ROWS = 64;                                   // rows per workgroup: two tiles of 32
constexpr int P6_TOKENS = 64;                                 // tokens per workgroup: two tiles of 32
constexpr int P6_BLOCK = 210;                                 // Q6_K block bytes
constexpr int P6_WINDOW = 53;                                 // dwords loaded per row and block
constexpr int P6_SLOT = 272;                                  // LDS bytes per row slot
constexpr int P6_W_BYTES = P6_ROWS * P6_SLOT;                 // 17408
constexpr int P6_X_BYTES = P6_TOKENS * 256;                   // 16384: [token][16 chunks, swizzled]
constexpr int P6_T_BYTES = P6_TOKENS * 32;                    // 2048: [token][8 groups, swizzled]
constexpr int P6_BUF = P6_W_BYTES + P6_X_BYTES + P6_T_BYTES;  // 35840, a multiple of 256
constexpr int P6_ZERO = 2 * P6_BUF;                           // 256 zero bytes after the buffers
constexpr int P6_LDS = P6_ZERO + 256;                         // 71936: two workgroups fit a CU
static_assert(P6_W_BYTES % 256 == 0 && P6_BUF % 256 == 0, "swizzled slots need 256-byte aligned bases");

struct P6Args {
    const uint8_t* w;
    float* out;
    int rows, cols, tokens;
    const int32_t* xq;
    const float* xd;
    const float* residual;
    uint32_t row_bytes;
    int steps, row_tiles, token_tiles;
    int chunks;    // a split product (chunks > 1): the tile's steps dealt over that many workgroups
    float* parts;  // [tile][chunk][wave][register v][lane], added by prefill_fixup_q6k
};

// the sums' slice of one (tile, chunk) in `parts`: 16 registers x 64 lanes a wave
constexpr int P6_PART = P6_WAVES * 16 * 64;

// the lane's fixed parts of the direct loads
struct P6Lanes {
    uint32_t w;      // 4 * min(lane, 52): the lane's dword of a row's window
    uint32_t xt;     // activations: token lane / 16 of a load's 4
    uint32_t xc;     // ... and the byte offset of its source chunk (lane % 16) ^ (token % 16)
    uint32_t tt;     // xd: token lane / 8 of a load's 8
    uint32_t tg[2];  // ... and its source group (lane % 8) ^ s for the wave's loads s = w, w + 4
};

// Issues the direct loads of step `step` into the buffer at LDS address `buf`; wave w takes rows
// w + 4j, activation loads w + 4j (tokens 4(w + 4j)..) and xd loads w, w + 4.
__device__ __forceinline__ void p6_stage(const P6Args& a, const P6Lanes& o, int row0, int tok0, uint32_t buf, int step,
                                         int w) {
    const uint32_t window = (uint32_t)step * P6_BLOCK - 2u * (uint32_t)(step & 1);
#pragma unroll
    for (int j = 0; j < P6_ROWS / P6_WAVES; j++) {
        const int m = w + P6_WAVES * j;
        const size_t row = (size_t)min(row0 + m, a.rows - 1);
        to_lds4(a.w + row * a.row_bytes + window + o.w, buf + P6_SLOT * m);
    }
    const uint32_t xbase = buf + P6_W_BYTES, tbase = xbase + P6_X_BYTES;
#pragma unroll
    for (int j = 0; j < P6_TOKENS / 4 / P6_WAVES; j++) {
        const int m = w + P6_WAVES * j;
        const size_t tok = (size_t)min(tok0 + 4 * m + (int)o.xt, a.tokens - 1);
        to_lds16((const uint8_t*)a.xq + tok * a.cols + 256u * step + o.xc, xbase + 1024 * m);
    }
    const int groups = a.cols / GROUP;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int s = w + P6_WAVES * j;
        const size_t tok = (size_t)min(tok0 + 8 * s + (int)o.tt, a.tokens - 1);
        to_lds4(a.xd + tok * groups + 8 * step + o.tg[j], tbase + 256 * s);
    }
}

// byte h of Q6_UPPER is (h - 2) << 4 as a signed byte, h = 0..3 the two high bits of a 6-bit q:
// q - 32 is the low nibble of q with that upper nibble (a v_perm_b32 table lookup per byte)
constexpr uint32_t Q6_UPPER = 0x1000F0E0u;

// 16 bytes from `lead` (0 or 2) bytes into the 20 at c (4 words) and e (the next word)
__device__ __forceinline__ u32x4 shift_bytes(u32x4 c, uint32_t e, uint32_t lead) {
    u32x4 r;
    r[0] = align_bytes(c[1], c[0], lead);
    r[1] = align_bytes(c[2], c[1], lead);
    r[2] = align_bytes(c[3], c[2], lead);
    r[3] = align_bytes(e, c[3], lead);
    return r;
}

// one group's operands and products
struct P6Ops {
    v4i x;
    v4i xh;  // the activations of lane half 1 (half 0: zeros)
    u32x4 b;  // the weights
    int sc0, sdiff;
    float xd;  // even groups: xd of the lane's token for group g + lane half
};
struct P6Res {
    v16i Df, Dh;
};

// lane (r, h) of wave w holds row row0 + 32 (w % 2) + r for tokens tok0 + 32 (w / 2) + 8(v / 4) + 4h + v % 4
template <int MODE>
__device__ __forceinline__ void p6_finish(const P6Args& a, const v16f& acc, int row0, int tok0, int w, int lane) {
    const int r = lane & 31, h = lane >> 5;
    const int row = row0 + 32 * (w & 1) + r;
    if (row >= a.rows) return;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int tok = tok0 + 32 * (w >> 1) + 8 * (v >> 2) + 4 * h + (v & 3);
        if (tok >= a.tokens) continue;
        const size_t at = (size_t)tok * a.rows + row;
        float y = acc[v];
        if (MODE == PF_RESIDUAL) y += a.residual[at];
        a.out[at] = y;
    }
}

template <int MODE>
__global__ __launch_bounds__(64 * P6_WAVES, 2) void prefill_q6k(P6Args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t p6_lds[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int r = lane & 31, h = lane >> 5;
    const int rt = w & 1, tt = w >> 1;  // the wave's row tile and token tile

    // workgroup id -> (chunk, tiles): ids on one XCD (id % 8) walk its row tiles' token tiles in
    // turn; a split product repeats that walk once per chunk
    const int per_chunk = (a.row_tiles + 7) / 8 * 8 * a.token_tiles;
    const int chunk = blockIdx.x / per_chunk, id = blockIdx.x - chunk * per_chunk;
    const int xcd = id & 7, local = id >> 3;
    const int wt = local % a.token_tiles, wr = (local / a.token_tiles) * 8 + xcd;
    if (wr >= a.row_tiles) return;
    // this chunk's steps [first, first + steps)
    const int first = chunk * a.steps / a.chunks, steps = (chunk + 1) * a.steps / a.chunks - first;
    const int row0 = wr * P6_ROWS, tok0 = wt * P6_TOKENS;
    const uint32_t lds0 = (uint32_t)(uintptr_t)p6_lds;

    P6Lanes o;
    o.w = 4u * (uint32_t)min(lane, P6_WINDOW - 1);
    o.xt = (uint32_t)lane >> 4;
    o.xc = 16u * (((uint32_t)lane & 15u) ^ ((4u * (uint32_t)w + ((uint32_t)lane >> 4)) & 15u));
    o.tt = (uint32_t)lane >> 3;
    o.tg[0] = ((uint32_t)lane & 7u) ^ (uint32_t)w;
    o.tg[1] = ((uint32_t)lane & 7u) ^ (uint32_t)(w + P6_WAVES);
    p6_stage(a, o, row0, tok0, lds0, first, w);

    // the lane's LDS offsets within a buffer: its row's slot (and the lane half's 16 bytes of a
    // 32-byte run), its token's activations (chunk c at xo ^ 32 (c / 2) for c = 2g + h) and xd
    // (group g + h of an even g at to ^ 4g)
    const int m = 32 * rt + r, t = 32 * tt + r;
    const uint32_t wo = P6_SLOT * m;
    const uint32_t xo = P6_W_BYTES + 256u * t + ((16u * h) ^ (16u * (t & 15)));
    const uint32_t to = P6_W_BYTES + P6_X_BYTES + 32u * t + 4u * ((uint32_t)h ^ ((uint32_t)(t >> 3) & 7u));
    // lane half 0 reads its operand of the half-1 product from the zeros (at zo ^ 32g)
    const uint32_t xoh = h ? xo : 0u;
    if (threadIdx.x < 64) ((uint32_t*)(p6_lds + P6_ZERO))[threadIdx.x] = 0u;  // before the first barrier

    v16f acc = {};
    for (int i = 0; i < steps; i++) {
        const int step = first + i;
        wait_loads();     // this step's direct loads are in LDS
        __syncthreads();  // ... everyone's; and the other buffer is free
        const uint32_t buf = lds0 + (uint32_t)(i & 1) * P6_BUF;
        if (i + 1 < steps) p6_stage(a, o, row0, tok0, lds0 + (uint32_t)((i + 1) & 1) * P6_BUF, step + 1, w);

        const uint32_t hbuf = h ? buf : lds0 + P6_ZERO;
        const uint32_t lead = 2u * (uint32_t)(step & 1);  // the block's first byte in its window
        const uint32_t wl = buf + wo, wq = wl + 16u * h;
        // the row's 16 scales and d: window bytes lead + 192 .. lead + 209
        const u32x4 sc4 = shift_bytes(lds_read<u32x4>(wl + 192), lds_read<uint32_t>(wl + 208), lead);
        const uint32_t dword = lds_read<uint32_t>(wl + 208);
        const float d = lead ? f16_hi(dword) : f16_lo(dword);

        u32x4 ql[2], qh;
        P6Ops op[8];
        P6Res rs[8];
        v32f S[4];
        auto read = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value, n = g / 4, k = g % 4;
            if constexpr (k == 0) {  // half n's bytes of the lane's 16 weights: ql for k = 0, 2 and 1, 3; qh
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t at = wq + 64 * n + 32 * e;
                    ql[e] = shift_bytes(lds_read<u32x4>(at), lds_read<uint32_t>(at + 16), lead);
                }
                const uint32_t at = wq + 128 + 32 * n;
                qh = shift_bytes(lds_read<u32x4>(at), lds_read<uint32_t>(at + 16), lead);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // q - 32 = low | 16 (high - 2): the upper nibble (high - 2) << 4 by byte lookup
                const uint32_t high = (qh[i] >> (2 * k)) & 0x03030303u;
                const uint32_t upper = __builtin_amdgcn_perm(Q6_UPPER, Q6_UPPER, high);
                op[g].b[i] = ((ql[k & 1][i] >> (4 * (k >> 1))) & 0x0F0F0F0Fu) | upper;
            }
            // scales 8n + 2k and 8n + 2k + 1: bytes 2k % 4 and the next of word 2n + k / 2
            const uint32_t sw = sc4[2 * n + k / 2];
            op[g].sc0 = __builtin_amdgcn_sbfe(sw, 8 * ((2 * k) % 4), 8);
            op[g].sdiff = __builtin_amdgcn_sbfe(sw, 8 * ((2 * k) % 4) + 8, 8) - op[g].sc0;
            op[g].x = lds_read<v4i>(buf + (xo ^ (32u * g)));
            op[g].xh = lds_read<v4i>(hbuf + (xoh ^ (32u * g)));
            if constexpr (g % 2 == 0) op[g].xd = lds_read<float>(buf + (to ^ (4u * g)));
        };
        auto issue = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            rs[g].Df = mfma_i8(op[g].x, op[g].b);
            rs[g].Dh = mfma_i8(op[g].xh, op[g].b);
            if constexpr (g % 2 == 0) S[g / 2] = mfma_outer2(op[g].xd, d);  // xd[token] * d[row], groups g, g + 1
        };
        auto scale = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int dot = __mul24(rs[g].Df[v], op[g].sc0) + __mul24(rs[g].Dh[v], op[g].sdiff);
                acc[v] += (float)dot * S[g / 2][16 * (g % 2) + v];
            }
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
            // the sums are due here: the compiler would otherwise sink the groups' scaling below
            // the last group's products, keeping all their results live
            asm volatile("" : "+v"(acc));
            __builtin_amdgcn_sched_barrier(0);
        });
    }

    if (a.chunks > 1) {  // a chunk's sums, for the fixup to add
        float* dst = a.parts + ((size_t)(wr * a.token_tiles + wt) * a.chunks + chunk) * P6_PART + w * (16 * 64) + lane;
#pragma unroll
        for (int v = 0; v < 16; v++) dst[v * 64] = acc[v];
        return;
    }
    p6_finish<MODE>(a, acc, row0, tok0, w, lane);
}

// A split product's tiles: the chunks' sums added in chunk order, then the outputs
template <int MODE>
__global__ __launch_bounds__(64 * P6_WAVES) void prefill_fixup_q6k(P6Args a) {
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int tile = blockIdx.x, wr = tile / a.token_tiles, wt = tile - wr * a.token_tiles;
    const float* src = a.parts + (size_t)tile * a.chunks * P6_PART + w * (16 * 64) + lane;
    v16f acc = {};
    for (int c = 0; c < a.chunks; c++, src += P6_PART)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[v] += src[v * 64];
    p6_finish<MODE>(a, acc, wr * P6_ROWS, wt * P6_TOKENS, w, lane);
}

template <int MODE>
int p6_go(P6Args& a, hipStream_t st) {
    // ids cover whole groups of 8 row tiles (one per XCD), once per chunk; ids past the last row
    // tile exit at once
    const int grid = (a.row_tiles + 7) / 8 * 8 * a.token_tiles * a.chunks;
    static const hipError_t allowed =
        hipFuncSetAttribute((const void*)prefill_q6k<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, P6_LDS);
    if (allowed != hipSuccess) {
        set_error("prefill: %d bytes of LDS refused", P6_LDS);
        return -1;
    }
    hipLaunchKernelGGL((prefill_q6k<MODE>), dim3(grid), dim3(64 * P6_WAVES), P6_LDS, st, a);
    if (check_launch("prefill")) return -1;
    if (a.chunks > 1) {
        hipLaunchKernelGGL((prefill_fixup_q6k<MODE>), dim3(a.row_tiles * a.token_tiles), dim3(64 * P6_WAVES), 0, st, a);
        return check_launch("prefill fixup");
    }
    return 0;
}

}  // namespace

bool prefill_q6k_fits(int cols) { return cols > 0 && cols % 512 == 0; }

Split prefill_q6k_split(int rows, int cols, int tokens) {
    const int tiles = (rows + P6_ROWS - 1) / P6_ROWS * ((tokens + P6_TOKENS - 1) / P6_TOKENS);
    return split_schedule(tiles, cols / 256, (int64_t)P6_PART * 4);
}

int prefill_q6k_launch(const void* w, int rows, int cols, const int32_t* xq, const float* xd, int tokens,
                       const float* residual, float* out, hipStream_t st, void* workspace, int64_t workspace_bytes) {
    P6Args a = {};
    a.row_tiles = (rows + P6_ROWS - 1) / P6_ROWS;
    a.token_tiles = (tokens + P6_TOKENS - 1) / P6_TOKENS;
    const Split sp = prefill_q6k_split(rows, cols, tokens);
    a.chunks = 1;
    if (sp.chunks > 1 && workspace && workspace_bytes >= sp.bytes) a.chunks = sp.chunks, a.parts = (float*)workspace;
    a.w = (const uint8_t*)w;
    a.out = out;
    a.rows = rows, a.cols = cols, a.tokens = tokens;
    a.xq = xq, a.xd = xd;
    a.residual = residual;
    a.steps = cols / 256;
    a.row_bytes = (uint32_t)a.steps * P6_BLOCK;
    return residual ? p6_go<PF_RESIDUAL>(a, st) : p6_go<PF_PLAIN>(a, st);
}

}  // namespace leat

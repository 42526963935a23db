// Decode-path products on matrix cores: y[t, row] = W[row] . x[t] for 1..16 tokens, every
// weight read once for all tokens, with v_mfma_i32_32x32x32_i8 doing the int8 dot products.
//
// A wave owns a tile of 32 rows and a run of each row's blocks; a workgroup's S waves cover one
// tile's blocks between them and add their sums through LDS at the end.
//
// Memory: a wave streams its tile one stage (one block per row; a pair for Q8_0) at a time. Its
// lanes load the 32 rows' stage bytes as consecutive 16-byte chunks, every load instruction
// covering whole runs of a row, and write them to the wave's LDS region at a row stride padded
// so the later 16-byte reads of 8 consecutive rows hit distinct banks; the next stage's loads are
// in flight while the current one is computed from LDS.
//
// Math: in each MFMA the 32 rows are N (the B operand: lane l holds row l % 32), the tokens are
// M (the A operand: lane l holds token l % 32, zero past the last), K is one activation group of
// 32 (one scale), and lane half h = l / 32 supplies 16 of the group's 32 values. The int32
// result holds, in lane l, row l % 32 for tokens 8(v/4) + 4h + v%4 of its registers v; each
// group's result is scaled into f32 sums at once, as leat's kernels combine each group's int32
// dot in f32 (leat/kernels/matvec.py:107-181):
//   Q4_K  lane h takes qs bytes [32j + 16h, +16) of each pair j: low nibbles are group 2j's
//         values 16h.., high nibbles group 2j+1's. u += d*sc*xd*D - dmin*m*xs.
//   Q6_K  a scale covers 16 values, so a group takes two MFMAs, each with one half's lanes
//         zeroed: lane h supplies values 16h..16h+15 of each 32-value row of the block
//         (ql bytes [64n + 32(k%2) + 16h, +16), nibble k/2; qh bytes [128 + 32n + 16h, +16),
//         bits 2k), minus 32. u += d*sc*xd*D per half.
//   Q8_0  one block is one group: lane h takes bytes [2 + 16h, +16). u += d*xd*D.
#include <algorithm>
#include <atomic>

#include "blocks.h"
#include "lds.h"
#include "mmv.h"

namespace leat {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma_i8(v4i a, u32x4 b) {
    const v16i zero = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, __builtin_bit_cast(v4i, b), zero, 0, 0, 0);
}

extern __shared__ uint32_t mmv_lds[];

// 16 bytes of LDS at a byte address that is 4-byte aligned
__device__ __forceinline__ u32x4 lds16(uint32_t at) {
    return *(const u32x4_a4*)((const char*)mmv_lds + at);
}
__device__ __forceinline__ uint32_t lds4(uint32_t at) { return *(const uint32_t*)((const char*)mmv_lds + at); }

// 16 bytes of LDS at an even byte address, 2 bytes past a 4-byte boundary when `odd` (uniform)
__device__ __forceinline__ u32x4 lds16_even(uint32_t at, bool odd) {
    if (!odd) return lds16(at);
    const u32x4 a = lds16(at - 2);
    const uint32_t e = lds4(at + 14);
    u32x4 r;
    r[0] = align_bytes(a[1], a[0], 2);
    r[1] = align_bytes(a[2], a[1], 2);
    r[2] = align_bytes(a[3], a[2], 2);
    r[3] = align_bytes(e, a[3], 2);
    return r;
}

// Staging geometry per type: a stage is BPS blocks of each of the tile's 32 rows, read as CPR
// 16-byte chunks from the stage's first byte rounded down to 16 (a row starts 16-byte aligned),
// and kept in LDS at a row stride of RS bytes (RS/4 an odd multiple of 4 dwords, modulo 32 banks).
template <int TYPE> struct Geo;
template <> struct Geo<Q4_K> { static constexpr int BYTES = 144, BPS = 1, CPR = 9, RS = 176; };
template <> struct Geo<Q6_K> { static constexpr int BYTES = 210, BPS = 1, CPR = 15, RS = 240; };
template <> struct Geo<Q8_0> { static constexpr int BYTES = 34, BPS = 2, CPR = 6, RS = 112; };

template <int TYPE>
struct Stage {
    static constexpr int CHUNKS = 32 * Geo<TYPE>::CPR;
    static constexpr int N = (CHUNKS + 63) / 64;  // 16-byte loads per lane
    u32x4 v[N];
};

// lanes load the stage's chunks: chunk c is part c % CPR of row c / CPR
template <int TYPE>
__device__ __forceinline__ void stage_load(Stage<TYPE>& st, const uint8_t* w, int64_t row_bytes, int row0, int rows,
                                           int stage, int lane) {
    using G = Geo<TYPE>;
    const int64_t s0 = ((int64_t)stage * G::BPS * G::BYTES) & ~(int64_t)15;
#pragma unroll
    for (int i = 0; i < Stage<TYPE>::N; i++) {
        // lanes past the stage's chunks load its last one (never stored): no branch around the
        // load, so the wait for a stage's data counts exactly the loads issued after it
        const int c = min(lane + 64 * i, Stage<TYPE>::CHUNKS - 1);
        const int r = c / G::CPR, part = c % G::CPR;
        const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
        // chunks past the row's end (the last stage's spare ones) repeat its last chunk
        const uint32_t off = (uint32_t)min(s0 + 16 * part, row_bytes - 16);
        // a 32-bit offset from the matrix's (uniform) start: matrices are under 4 GiB
        st.v[i] = stream_load((const u32x4*)(w + (row * (uint32_t)row_bytes + off)));
    }
}

template <int TYPE>
__device__ __forceinline__ void stage_store(const Stage<TYPE>& st, uint32_t base, int lane) {
    using G = Geo<TYPE>;
#pragma unroll
    for (int i = 0; i < Stage<TYPE>::N; i++) {
        const int c = lane + 64 * i;
        if (c < Stage<TYPE>::CHUNKS) {
            const int r = c / G::CPR, part = c % G::CPR;
            *(u32x4*)__builtin_assume_aligned((char*)mmv_lds + base + r * G::RS + 16 * part, 16) = st.v[i];
        }
    }
}

// The tokens' activations as a lane reads them. The per-group scales d (and s = d * sum(q))
// are staged in the workgroup's LDS, group-major with TP token slots per group, so the tokens
// a lane's results hold (4h + v) are one vector read; the int8 words are staged too where they
// fit (XQ), else read from global memory (L2).
template <int NV>
constexpr int token_slots() {
    return NV <= 2 ? 2 : NV == 4 ? 8 : 16;
}

template <int NV, bool XQ, int SETS_>
struct Acts {
    static constexpr int SETS = SETS_;
    static constexpr int TP = token_slots<NV>();
    const uint32_t* q;  // global words, when not XQ
    int cols;
    int s_off;   // the s table's offset in mmv_lds, in floats (after d's G * TP)
    int xq_off;  // the words' offset in mmv_lds, in words
    // the lane's (token t, half h) words: group g's 16 values are 8 g words on, in global memory
    // (lq) or in LDS (lx); set once, so a group's address is a 32-bit offset from them
    const uint32_t* lq;
    uint32_t lx;
    __device__ void at_lane(int t, int h) {
        lq = q + (int64_t)t * (cols / 4) + 4 * h;
        lx = (uint32_t)(xq_off + t * (cols / 4) + 4 * h);
    }
    // the lane's 16 values of group g, the stage's group s. A lane past the last token reads
    // token 0's: its results (rows of tokens that are not there) are never stored, so no branch is
    // needed here. From global memory, the stage's operands are loaded together beforehand (load).
    static constexpr int GPS = 8;  // groups a stage
    // (from global memory: SETS = 2 stages' sets, the next one's in flight while one is used,
    // where the registers allow)
    v4i ops[SETS ? SETS : 1][XQ || !SETS ? 1 : GPS];
    __device__ __forceinline__ v4i operand(int g, int s, int set) const {
        if (XQ) return *(const v4i*)(mmv_lds + lx + g * 8);
        if (SETS == 0) return *(const v4i*)(lq + g * 8);  // one at a time (registers are short)
        return ops[set % (SETS ? SETS : 1)][s];
    }
    template <int N>  // into `set`: the stage's N groups from g0
    __device__ __forceinline__ void load(int set, int g0) {
        if (!XQ && SETS > 0)
#pragma unroll
            for (int s = 0; s < N; s++) ops[set % SETS][s] = *(const v4i*)(lq + (g0 + s) * 8);
    }
    // the scales of group g for the lane's result registers v = 0..NV-1
    __device__ void scales(int off, int g, int h, float (&out)[NV]) const {
        const float* tab = (const float*)mmv_lds + off + g * TP;
        if (NV == 1) {
            out[0] = tab[0];
        } else if (NV == 2) {
            const float2 x = *(const float2*)tab;
            out[0] = x.x, out[NV - 1] = x.y;
        } else {
#pragma unroll
            for (int i = 0; i < NV / 4; i++) {
                const float4 x = *(const float4*)(tab + 8 * i + 4 * h);
                out[4 * i] = x.x, out[4 * i + 1] = x.y, out[4 * i + 2] = x.z, out[4 * i + 3] = x.w;
            }
        }
    }
};

// One stage of one matrix for the lane (row r, half h), from the wave's LDS region `base`:
// acc[v] += its share for the lane's tokens. `b` is the stage's first block.
template <int TYPE> struct Compute;

template <>
struct Compute<Q4_K> {
    template <int NV, class A>
    __device__ __forceinline__ static void run(uint32_t base, int b, const A& a, int set, int r, int h, float (&acc)[NV]) {
        const uint32_t at = base + r * Geo<Q4_K>::RS;  // the block starts the chunk run
        const u32x4 hdr = lds16(at);
        const float d = f16_lo(hdr[0]), dmin = f16_hi(hdr[0]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const u32x4 qs = lds16(at + 16 + 32 * j + 16 * h);
            const u32x4 lo = qs & 0x0F0F0F0Fu;
            const u32x4 hi = (qs >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int s = 2 * j + e, g = 8 * b + s;
                // get_scale_min_k4 (leat/quant.py:182-187), s known at compile time
                const uint32_t sh = 8u * (uint32_t)(s & 3);
                const uint32_t x0 = hdr[1] >> sh, x1 = hdr[2] >> sh, x2 = hdr[3] >> sh;
                const uint32_t scv = s < 4 ? (x0 & 63u) : ((x2 & 15u) | ((x0 >> 2) & 0x30u));
                const uint32_t mv = s < 4 ? (x1 & 63u) : (((x2 >> 4) & 15u) | ((x1 >> 2) & 0x30u));
                const float sc = d * (float)scv, mn = dmin * (float)mv;
                const v16i D = mfma_i8(a.operand(g, s, set), e ? hi : lo);
                float xd[NV], xs[NV];
                a.scales(0, g, h, xd);
                a.scales(a.s_off, g, h, xs);
#pragma unroll
                for (int v = 0; v < NV; v++) acc[v] += sc * xd[v] * (float)D[v] - mn * xs[v];
                // consume each result before the next product: a result takes 16 registers
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
};

template <>
struct Compute<Q6_K> {
    template <int NV, class A>
    __device__ __forceinline__ static void run(uint32_t base, int b, const A& a, int set, int r, int h, float (&acc)[NV]) {
        // odd blocks as a compile-time case: a run-time flag keeps both forms of every read live
        if (b & 1)
            run_<NV, true>(base, b, a, set, r, h, acc);
        else
            run_<NV, false>(base, b, a, set, r, h, acc);
    }
    template <int NV, bool ODD, class A>
    __device__ __forceinline__ static void run_(uint32_t base, int b, const A& a, int set, int r, int h, float (&acc)[NV]) {
        // the block starts (210 b) mod 16 bytes into the row's chunk run: 2 bytes off a 4-byte
        // boundary for odd b
        const uint32_t at = base + r * Geo<Q6_K>::RS + ((210u * (uint32_t)b) & 15u);
        constexpr bool odd = ODD;
        const u32x4 scales = lds16_even(at + 192, odd);
        const uint32_t dword = lds4((at + 208) & ~3u);
        const float d = odd ? f16_hi(dword) : f16_lo(dword);
        if constexpr (A::SETS != 2) {  // 1-2 tokens and the GLU (fewer registers): a group at a time
#pragma unroll
            for (int n = 0; n < 2; n++) {
                const u32x4 qh = lds16_even(at + 128 + 32 * n + 16 * h, odd);
#pragma unroll
                for (int kk = 0; kk < 2; kk++) {
                    const u32x4 ql = lds16_even(at + 64 * n + 32 * kk + 16 * h, odd);
#pragma unroll
                    for (int k2 = 0; k2 < 2; k2++) {
                        const int k = kk + 2 * k2;  // rows kk (low nibbles) and kk + 2 (high)
                        const int g = 8 * b + 4 * n + k;
                        u32x4 q;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const uint32_t low = (ql[i] >> (4 * k2)) & 0x0F0F0F0Fu;
                            const uint32_t high = (qh[i] >> (2 * k)) & 0x03030303u;
                            q[i] = minus_bytes(low | (high << 4), 32);
                        }
                        const v4i x = a.operand(g, 4 * n + k, set);
                        const u32x4 zero = {};
                        const v16i D0 = mfma_i8(x, h == 0 ? q : zero);  // values 0..15 of the row
                        const v16i D1 = mfma_i8(x, h == 1 ? q : zero);  // values 16..31
                        const int si = 8 * n + 2 * k;                   // scales si, si + 1
                        const float s0 = d * (float)(int8_t)((scales[si >> 2] >> (8 * (si & 3))) & 0xFF);
                        const float s1 = d * (float)(int8_t)((scales[si >> 2] >> (8 * (si & 3) + 8)) & 0xFF);
                        float xd[NV];
                        a.scales(0, g, h, xd);
#pragma unroll
                        for (int v = 0; v < NV; v++) acc[v] += xd[v] * (s0 * (float)D0[v] + s1 * (float)D1[v]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
            return;
        }
        // else the 8 groups (n = g / 4, k = g % 4: the rows k of half n) as a pipeline: the operands
        // of group g + 2 are read and decoded while the products of g + 1 are issued and g is scaled
        struct Op {
            v4i x;
            u32x4 q;
            float s0, s1;
            float xd[NV];
        };
        struct Res {
            v16i D0, D1;
        };
        u32x4 qh[2], ql[2][2];
        Op op[8];
        Res rs[8];
        auto prep = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value, n = g / 4, k = g % 4, kk = k & 1, k2 = k >> 1;
            if constexpr (k == 0) {  // half n's bytes: qh, and ql of rows 0, 2 and 1, 3
                qh[n] = lds16_even(at + 128 + 32 * n + 16 * h, odd);
                ql[n][0] = lds16_even(at + 64 * n + 16 * h, odd);
                ql[n][1] = lds16_even(at + 64 * n + 32 + 16 * h, odd);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t low = (ql[n][kk][i] >> (4 * k2)) & 0x0F0F0F0Fu;
                const uint32_t high = (qh[n][i] >> (2 * k)) & 0x03030303u;
                op[g].q[i] = minus_bytes(low | (high << 4), 32);
            }
            op[g].x = a.operand(8 * b + g, g, set);
            constexpr int si = 8 * n + 2 * k;  // scales si, si + 1
            op[g].s0 = d * (float)(int8_t)((scales[si >> 2] >> (8 * (si & 3))) & 0xFF);
            op[g].s1 = d * (float)(int8_t)((scales[si >> 2] >> (8 * (si & 3) + 8)) & 0xFF);
            a.scales(0, 8 * b + g, h, op[g].xd);
        };
        auto issue = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            const u32x4 zero = {};
            rs[g].D0 = mfma_i8(op[g].x, h == 0 ? op[g].q : zero);  // values 0..15 of the row
            rs[g].D1 = mfma_i8(op[g].x, h == 1 ? op[g].q : zero);  // values 16..31
        };
        auto scale = [&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
#pragma unroll
            for (int v = 0; v < NV; v++)
                acc[v] += op[g].xd[v] * (op[g].s0 * (float)rs[g].D0[v] + op[g].s1 * (float)rs[g].D1[v]);
        };
        prep(std::integral_constant<int, 0>{});
        issue(std::integral_constant<int, 0>{});
        prep(std::integral_constant<int, 1>{});
        __builtin_amdgcn_sched_barrier(0);
        pf::static_for<0, 8>([&](auto gc) __attribute__((always_inline)) {
            constexpr int g = decltype(gc)::value;
            if constexpr (g + 1 < 8) issue(std::integral_constant<int, g + 1>{});
            if constexpr (g + 2 < 8) prep(std::integral_constant<int, g + 2>{});
            scale(gc);
            __builtin_amdgcn_sched_barrier(0);  // keeps two groups' results in registers, not eight
        });
    }
};

template <>
struct Compute<Q8_0> {
    template <int NV, class A>
    __device__ __forceinline__ static void run(uint32_t base, int b, const A& a, int set, int r, int h, float (&acc)[NV]) {
        // a stage is blocks b and b + 1 (68 bytes from a 4-byte aligned start, b even)
        const uint32_t at = base + r * Geo<Q8_0>::RS + ((34u * (uint32_t)b) & 15u);
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint32_t blk = at + 34 * e;
            const uint32_t dword = lds4(blk & ~3u);
            const float d = e ? f16_hi(dword) : f16_lo(dword);
            const u32x4 qs = lds16_even(blk + 2 + 16 * h, e == 0);
            const v16i D = mfma_i8(a.operand(b + e, e, set), qs);
            float xd[NV];
            a.scales(0, b + e, h, xd);
#pragma unroll
            for (int v = 0; v < NV; v++) acc[v] += d * xd[v] * (float)D[v];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

constexpr int MMV_DEPTH = 1;  // stages of loads a wave keeps in flight besides the one it computes

// waves per SIMD the register budget allows: 4 (128 registers) for one Q4_K or Q8_0 matrix and
// up to two tokens' results, 3 (168) for Q6_K's wider stages, else 2 (256). A wave keeps a stage
// of its tile in flight, so a few waves per SIMD cover HBM's latency.
constexpr int mmv_occupancy(int type, int mode, int nv) {
    return mode == MMV_GLU || nv > 2 ? 2 : type == Q6_K ? 3 : 4;
}

template <int TYPE>
constexpr int weights_per_block() {
    return TYPE == Q8_0 ? 32 : 256;
}

// the workgroup's LDS: scale tables, then staged words (XQ), then S * NM stage regions
template <int TYPE, int NV>
__host__ __device__ constexpr int table_bytes(int cols) {
    return (TYPE == Q4_K ? 2 : 1) * (cols / GROUP) * token_slots<NV>() * 4;
}

template <int TYPE, int MODE, int NV, int S, bool XQ>
__global__ __launch_bounds__(S * 64) __attribute__((amdgpu_waves_per_eu(mmv_occupancy(TYPE, MODE, NV))))
void mmv_kernel(MmvArgs args) {
    using G = Geo<TYPE>;
    constexpr int NM = MODE == MMV_GLU ? 2 : 1;
    const int cols = args.cols, tokens = args.tokens;
    const int nb = cols / weights_per_block<TYPE>(), G_ = cols / GROUP;
    const int64_t row_bytes = (int64_t)nb * G::BYTES;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 31, h = lane >> 5;

    // the workgroup's tile, and its part of the tile's blocks (parts > 1: the first or second half)
    const int part = (int)blockIdx.x / args.tile_start[args.count];
    const int tile = (int)blockIdx.x - part * args.tile_start[args.count];
    int m = 0;
    if (MODE != MMV_GLU)
        while (m + 1 < args.count && tile >= args.tile_start[m + 1]) m++;
    const int rows = args.rows[m];
    const int row0 = (tile - args.tile_start[m]) * 32;
    const uint8_t* wm[NM];
    wm[0] = MODE == MMV_GLU ? args.w[0] : args.w[m];
    if (NM == 2) wm[NM - 1] = args.w[1];

    // the wave's stages, and the first one's loads before anything else
    const int stages = nb / G::BPS;
    const int p0 = stages * part / args.parts, pn = stages * (part + 1) / args.parts - p0;
    // the wave's stages ka + ks j, j < nk: every S-th of the part's, so the S waves read
    // neighbouring blocks of the tile's rows at a time
    const int ka = p0 + wave, ks = S, nk = ka < p0 + pn ? (p0 + pn - ka + S - 1) / S : 0;
    // operand sets: 2 (prefetched) for Q6_K's 3+ tokens outside the GLU; none (loaded when used)
    // where the register budget is 128 (occupancy 4); else 1
    using A = Acts<NV, XQ,
                   TYPE == Q6_K && NV >= 4 && MODE != MMV_GLU ? 2 : mmv_occupancy(TYPE, MODE, NV) >= 4 ? 0 : 1>;
    constexpr int TP = A::TP;
    // The scales of the groups of the workgroup's blocks go into LDS, U loads in flight per thread.
    // The first U a thread are asked for before anything else, at clamped indices, then the first
    // MMV_DEPTH stages of weights (stage indices clamped into the row), all unconditionally: the
    // table's LDS writes then wait for the table alone, counting the weight loads still in flight.
    constexpr int GPS = TYPE == Q8_0 ? 2 : 8;  // groups a stage
    constexpr int U = NV >= 4 ? 8 : 2;
    const int gb0 = p0 * GPS, n = pn * GPS * TP;
    float vd[U], vs[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = (int)threadIdx.x + u * (int)blockDim.x;
        const int at = min(i % TP, tokens - 1) * G_ + min(gb0 + i / TP, G_ - 1);
        vd[u] = args.xd[at];
        vs[u] = TYPE == Q4_K ? args.xs[at] : 0.0f;
    }
    // staged words (XQ): their first V u32x4 a thread likewise
    constexpr int V = NV >= 4 ? 4 : 1;
    const int quads = XQ ? tokens * (cols / 4) / 4 : 1;
    u32x4 wq[XQ ? V : 1];
    if constexpr (XQ)
#pragma unroll
        for (int u = 0; u < V; u++) wq[u] = ((const u32x4*)args.xq)[min((int)threadIdx.x + u * (int)blockDim.x, quads - 1)];
    __builtin_amdgcn_sched_barrier(0);  // the table's (and words') loads stay ahead of the weights'
    // MMV_DEPTH stages in flight (a wave with fewer stages loads stages it never uses)
    Stage<TYPE> st[MMV_DEPTH][NM];
#pragma unroll
    for (int p = 0; p < MMV_DEPTH; p++)
#pragma unroll
        for (int i = 0; i < NM; i++)
            stage_load<TYPE>(st[p][i], wm[i], row_bytes, row0, rows, min(ka + ks * p, stages - 1), lane);

    A acts;
    acts.q = (const uint32_t*)args.xq;
    acts.cols = cols;
    acts.s_off = G_ * TP;
    acts.xq_off = table_bytes<TYPE, NV>(cols) / 4;
    {
        float* tab = (float*)mmv_lds;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = (int)threadIdx.x + u * (int)blockDim.x;
            if (i < n) {
                const bool in = i % TP < tokens;
                tab[gb0 * TP + i] = in ? vd[u] : 0.0f;
                if (TYPE == Q4_K) tab[(G_ + gb0) * TP + i] = in ? vs[u] : 0.0f;
            }
        }
        // tables longer than U entries a thread
        for (int base = threadIdx.x + U * blockDim.x; base < n; base += U * blockDim.x) {
            float rd[U], rs[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * (int)blockDim.x, g = gb0 + i / TP, tk = i % TP;
                const bool in = i < n && tk < tokens;
                rd[u] = in ? args.xd[tk * G_ + g] : 0.0f;
                rs[u] = TYPE == Q4_K && in ? args.xs[tk * G_ + g] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * (int)blockDim.x;
                if (i < n) {
                    tab[gb0 * TP + i] = rd[u];
                    if (TYPE == Q4_K) tab[(G_ + gb0) * TP + i] = rs[u];
                }
            }
        }
        if constexpr (XQ) {
            u32x4* staged = (u32x4*)(mmv_lds + acts.xq_off);
#pragma unroll
            for (int u = 0; u < V; u++) {
                const int i = (int)threadIdx.x + u * (int)blockDim.x;
                if (i < quads) staged[i] = wq[u];
            }
            for (int base = threadIdx.x + V * blockDim.x; base < quads; base += V * blockDim.x) {
                u32x4 v[V];
#pragma unroll
                for (int u = 0; u < V; u++) {
                    const int i = base + u * (int)blockDim.x;
                    if (i < quads) v[u] = ((const u32x4*)args.xq)[i];
                }
#pragma unroll
                for (int u = 0; u < V; u++) {
                    const int i = base + u * (int)blockDim.x;
                    if (i < quads) staged[i] = v[u];
                }
            }
        }
        __syncthreads();
    }
    const uint32_t regions = (uint32_t)table_bytes<TYPE, NV>(cols) + (XQ ? (uint32_t)tokens * cols : 0u);
    acts.at_lane(r < tokens ? r : 0, h);

    float acc[NM][NV];
#pragma unroll
    for (int i = 0; i < NM; i++)
#pragma unroll
        for (int v = 0; v < NV; v++) acc[i][v] = 0.0f;

    constexpr int GS = TYPE == Q8_0 ? 2 : 8;  // groups a stage
    if (A::SETS == 2 && nk > 0) acts.template load<GS>(0, ka * GS);
    constexpr int UNR = A::SETS == 2 ? 2 : MMV_DEPTH;  // stages a loop turn: the sets alternate
    for (int j0 = 0; j0 < nk; j0 += UNR) {
#pragma unroll
        for (int p = 0; p < UNR; p++) {
            // stage j: its registers go to the wave's LDS region and take the loads of stage
            // j + DEPTH; its activation operands are set p, the next stage's go to set 1 - p
            const int sp = p % MMV_DEPTH, j = j0 + p, k = ka + ks * j;
            if (j >= nk) break;
            // (the last stage loads its own set again: no branch around loads, as above)
            if (A::SETS == 1)
                acts.template load<GS>(0, k * GS);  // this stage's, all in flight at once
            else if (A::SETS == 2)
                acts.template load<GS>(1 - p, (ka + ks * min(j + 1, nk - 1)) * GS);
            // the previous stage's LDS reads are done before its region is overwritten
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < NM; i++) stage_store<TYPE>(st[sp][i], regions + (wave * NM + i) * 32 * G::RS, lane);
#pragma unroll
            for (int i = 0; i < NM; i++)  // (past the last stage: the last again, never stored)
                stage_load<TYPE>(st[sp][i], wm[i], row_bytes, row0, rows, ka + ks * min(j + MMV_DEPTH, nk - 1), lane);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < NM; i++)
                Compute<TYPE>::template run<NV>(regions + (wave * NM + i) * 32 * G::RS, k * G::BPS, acts, p, r, h,
                                                acc[i]);
        }
    }

    // the S waves' sums of the tile, through LDS
    if (S > 1) {
        __syncthreads();
        float* red = (float*)mmv_lds;
#pragma unroll
        for (int i = 0; i < NM; i++)
#pragma unroll
            for (int v = 0; v < NV; v++) red[((wave * NM + i) * NV + v) * 64 + lane] = acc[i][v];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int i = 0; i < NM; i++)
#pragma unroll
            for (int v = 0; v < NV; v++) {
                float sum = 0.0f;
                for (int w = 0; w < S; w++) sum += red[((w * NM + i) * NV + v) * 64 + lane];
                acc[i][v] = sum;
            }
    }
    const int row_out = row0 + r;
    if (row_out >= rows) return;
    float* out = args.out[MODE == MMV_GLU ? 0 : m];
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int tok = 8 * (v >> 2) + 4 * h + (v & 3);
        if (tok >= tokens) continue;
        const int64_t at = (int64_t)tok * rows + row_out;
        float y = acc[0][v];
        if (MODE == MMV_GLU) y = glu(args.kind, acc[0][v], acc[NM - 1][v]);
        if (MODE == MMV_RESIDUAL && part == 0) y += args.residual[at];
        if (MODE != MMV_GLU && args.parts > 1)
            atomicAdd(out + at, y);  // into zero: 0 + a + b is a + b in either order
        else
            out[at] = y;
    }
}

// zeroes the launch's outputs before a tile's two parts add into them
__global__ void mmv_zero(MmvArgs a) {
    const int m = blockIdx.y;
    const int64_t n = (int64_t)a.tokens * a.rows[m];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        a.out[m][i] = 0.0f;
}

constexpr int MMV_SPLIT_STAGES = 32;  // the fewest stages (blocks) a row needs to split it over two workgroups

// the current device's CU count, read once per device; callers on several threads may race to
// fill an entry, and all store the same value
int cu_count() {
    static std::atomic<int> counts[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int known = counts[dev].load(std::memory_order_relaxed);
    if (!known) {
        int n = 0;
        known = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
        counts[dev].store(known, std::memory_order_relaxed);
    }
    return known;
}
constexpr int MMV_WAVES = 4096;  // waves a launch aims for: 16 per CU

template <int TYPE, int MODE, int NV, int S>
static int mmv_launch_s(MmvArgs& a, hipStream_t st) {
    constexpr int NM = MODE == MMV_GLU ? 2 : 1;
    if (a.parts > 1) {
        hipLaunchKernelGGL(mmv_zero, dim3(64, a.count), dim3(256), 0, st, a);
        if (check_launch("mmv")) return -1;
    }
    const int tiles = a.tile_start[a.count] * a.parts;
    const size_t tables = table_bytes<TYPE, NV>(a.cols);
    const size_t words = (size_t)a.tokens * a.cols;
    const size_t stages = (size_t)S * NM * 32 * Geo<TYPE>::RS;
    const size_t red = (size_t)S * NM * NV * 64 * 4;
    if (words <= 16384) {
        const size_t lds = std::max(tables + words + stages, red);
        hipLaunchKernelGGL((mmv_kernel<TYPE, MODE, NV, S, true>), dim3(tiles), dim3(S * 64), lds, st, a);
    } else {
        const size_t lds = std::max(tables + stages, red);
        hipLaunchKernelGGL((mmv_kernel<TYPE, MODE, NV, S, false>), dim3(tiles), dim3(S * 64), lds, st, a);
    }
    return check_launch("mmv");
}

template <int TYPE, int MODE, int NV>
static int mmv_launch_nv(MmvArgs& a, hipStream_t st) {
    const int stages = a.cols / weights_per_block<TYPE>() / Geo<TYPE>::BPS;
    // fewer tiles than CUs (a 4096-row down product: 128): two workgroups a tile, each half the
    // blocks, so that every CU streams
    // (not when the output is the residual itself: zeroing it first would lose the residual)
    const size_t n = (size_t)a.tokens * a.rows[0];
    const bool in_place = MODE == MMV_RESIDUAL && a.residual < a.out[0] + n && a.out[0] < a.residual + n;
    a.parts = MODE != MMV_GLU && !in_place && a.tile_start[a.count] < cu_count() && stages >= MMV_SPLIT_STAGES
                  ? 2
                  : 1;
    const int tiles = a.tile_start[a.count] * a.parts;
    // waves per tile: enough for the launch to fill the GPU, at most one per stage of a row
    const int want = (MMV_WAVES + tiles - 1) / tiles;
    if constexpr (mmv_occupancy(TYPE, MODE, NV) > 1)
        if (want >= 8 && stages >= 8) return mmv_launch_s<TYPE, MODE, NV, 8>(a, st);
    if (want >= 4 && stages >= 4) return mmv_launch_s<TYPE, MODE, NV, 4>(a, st);
    if (want >= 2 && stages >= 2) return mmv_launch_s<TYPE, MODE, NV, 2>(a, st);
    return mmv_launch_s<TYPE, MODE, NV, 1>(a, st);
}

template <int TYPE, int MODE>
static int mmv_launch_t(MmvArgs& a, hipStream_t st) {
    const int B = a.tokens;
    if (B == 1) return mmv_launch_nv<TYPE, MODE, 1>(a, st);
    if (B == 2) return mmv_launch_nv<TYPE, MODE, 2>(a, st);
    if (B <= 8) return mmv_launch_nv<TYPE, MODE, 4>(a, st);
    return mmv_launch_nv<TYPE, MODE, 8>(a, st);
}

bool mmv_fits(int type, int cols, int tokens, const void* const* ws, int count) {
    if (tokens < 1 || tokens > 16) return false;
    int64_t row_bytes;
    if (type == Q4_K && cols % 256 == 0) row_bytes = (int64_t)cols / 256 * 144;
    else if (type == Q6_K && cols % 512 == 0) row_bytes = (int64_t)cols / 256 * 210;
    else if (type == Q8_0 && cols % 64 == 0) row_bytes = (int64_t)cols / 32 * 34;
    else return false;
    // stages are read as 16-byte chunks of rows that start 16-byte aligned
    if (row_bytes % 16 != 0) return false;
    for (int i = 0; i < count; i++)
        if ((uintptr_t)ws[i] % 16 != 0) return false;
    return true;
}

int mmv_launch(int type, int mode, MmvArgs& a, hipStream_t st) {
    int total = 0;
    for (int i = 0; i < a.count; i++) {
        a.tile_start[i] = total;
        total += (a.rows[i] + 31) / 32;
    }
    a.tile_start[a.count] = total;
#define LEAT_MMV_MODES(T)                                           \
    switch (mode) {                                                 \
    case MMV_PLAIN: return mmv_launch_t<T, MMV_PLAIN>(a, st);       \
    case MMV_RESIDUAL: return mmv_launch_t<T, MMV_RESIDUAL>(a, st); \
    default: return mmv_launch_t<T, MMV_GLU>(a, st);                \
    }
    switch (type) {
    case Q4_K: LEAT_MMV_MODES(Q4_K)
    case Q6_K: LEAT_MMV_MODES(Q6_K)
    case Q8_0: LEAT_MMV_MODES(Q8_0)
    default: set_error("mmv: unsupported type %d", type); return -1;
    }
#undef LEAT_MMV_MODES
}

}  // namespace leat

// The decode step's attention around the quantized products (leat/kernels/attention.py): each
// token's queries and keys rotated by RoPE with its keys and values stored in an f16 cache
// (`rotate`, :656-782), and FlashDecoding of one query token per row over its slot of the cache
// (`attention`, :226-279: partial softmax sums per chunk of keys, then a combine launch).
//
// Cache layout (as leat's): f16 (2, slots, kv_heads, positions, dim), keys then values, a head's
// positions one after another, each position's dim values contiguous. Rotated queries are f32
// (heads, tokens, dim). Positions and lengths are device arrays, so one captured graph serves
// every step of a decode.
#include <algorithm>

#include "common.h"
#include "q8.h"

namespace leat {

// ------------------------------------------------------------------------------------ rotate

struct RotateArgs {
    const float* q;  // (tokens, heads, dim)
    const float* k;  // (tokens, kv_heads, dim)
    const float* v;
    int tokens, heads, kv_heads, dim;
    const float* cos;  // (table positions, rotated / 2)
    const float* sin;
    int rotated, halves;
    const int32_t* slots;      // tokens
    const int32_t* positions;  // tokens
    float* q_out;              // (heads, tokens, dim)
    _Float16* cache;           // (2, cache_slots, kv_heads, cache_positions, dim)
    int cache_slots, cache_positions;
};

// A wave per (token, head of q, then of k with its v); lane i takes pairs i, i + 64, ...: the
// dimensions that turn together (adjacent, or i and i + rotated / 2 with `halves`), by the
// angle of pair i at the token's position; pairs past the rotated ones stay as they are.
__global__ __launch_bounds__(64) void rotate_kernel(RotateArgs a) {
    const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const bool is_q = head < a.heads;
    const int kv = head - a.heads;
    const int pos = a.positions[t], slot = a.slots[t];
    // a position or slot outside the cache (the tables cover its positions) stores nothing
    if (pos < 0 || pos >= a.cache_positions || slot < 0 || slot >= a.cache_slots) return;
    const int half = a.rotated / 2;
    const float* src = is_q ? a.q + ((int64_t)t * a.heads + head) * a.dim : a.k + ((int64_t)t * a.kv_heads + kv) * a.dim;
    const int64_t cache_row = (((int64_t)slot * a.kv_heads + kv) * a.cache_positions + pos) * a.dim;
    const int64_t values = (int64_t)a.cache_slots * a.kv_heads * a.cache_positions * a.dim;  // the values' half
    for (int i = lane; i < a.dim / 2; i += WAVE) {
        const bool turns = i < half;
        const int d0 = a.halves && turns ? i : 2 * i;
        const int d1 = a.halves && turns ? i + half : 2 * i + 1;
        float x0 = src[d0], x1 = src[d1];
        if (turns) {
            rope_pair(x0, x1, a.cos[(int64_t)pos * half + i], a.sin[(int64_t)pos * half + i]);
        }
        if (is_q) {
            float* o = a.q_out + ((int64_t)head * a.tokens + t) * a.dim;
            o[d0] = x0, o[d1] = x1;
        } else {
            a.cache[cache_row + d0] = (_Float16)x0;
            a.cache[cache_row + d1] = (_Float16)x1;
            const float* vs = a.v + ((int64_t)t * a.kv_heads + kv) * a.dim;
            a.cache[values + cache_row + d0] = (_Float16)vs[d0];
            a.cache[values + cache_row + d1] = (_Float16)vs[d1];
        }
    }
}

// --------------------------------------------------------------------------------- attention

constexpr int ATT_WAVES = 8;                       // waves a workgroup
constexpr int ATT_CHUNKS = 64;                     // most workgroups per (row, kv head): longer rows loop
// Keys a wave takes per round: 16, or 8 for launches whose rows run past one 128-key chunk but at
// most ATT_EIGHT_KEYS_UP_TO keys, where twice the workgroups (each with half the serial math a
// round) finish sooner; longer rows keep 16, whose 32 or fewer chunks a row the combine gathers
// in fewer loads a lane.
constexpr int ATT_EIGHT_KEYS_UP_TO = 2048;
constexpr int ATT_DIM = 128;                       // head dimension: a pair of dimensions a lane
constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG = -1e30f;  // a finite floor: a fully masked wave never computes -inf - -inf

struct AttentionArgs {
    const float* q;  // (heads, rows, dim)
    const _Float16* cache;
    int cache_slots, kv_heads, cache_positions;
    int rows, heads, group;   // group = heads / kv_heads
    const int32_t* slots;     // rows
    const int32_t* lengths;   // rows: keys 0 .. length - 1 of the row's slot
    int chunks;               // workgroups per (row, kv head)
    int key_bits;             // log2 of the keys a workgroup takes per round (ATT_WAVES times a wave's)
    float scale;
    float* partial;  // (rows * heads, chunks, dim + 2): unnormalized output, then max (log2 units) and sum
    float* out;      // (rows, heads * dim)
    // or null; else the q8 of out as leat_quantize_q8 writes a row of heads * dim values: words,
    // then each group's d and s
    uint32_t* hq;
    float* hd;
    float* hs;
};

// The q8 of 4 consecutive output values v at column `col` (a multiple of 4) of row `row`, by the
// aligned octet of lanes that holds one group of 32 (the standalone quantizer's arithmetic,
// quantize4): every lane of the octet takes part; `store` says whether this lane's word is kept.
__device__ __forceinline__ void attention_q8(const AttentionArgs& a, float4 v, int row, int col, bool store) {
    float dv, sv;
    const uint32_t word = quantize4(v, &dv, &sv);
    const int64_t at = (int64_t)row * a.heads * ATT_DIM + col;
    if (!store) return;
    a.hq[at / 4] = word;
    if (col % GROUP == 0) {
        a.hd[at / GROUP] = dv;
        a.hs[at / GROUP] = sv;
    }
}

// 16 values of each lane summed over the wave's 64 lanes, transposed: lane l ends with the sum of
// value ((l >> 2) & 15). Each step keeps half the values and adds the partner lane's other half,
// so 16 sums over 64 lanes take 8 + 4 + 2 + 1 exchanges and 2 more within each quad of lanes.
// The exchanges stay in registers: across lane halves and rows of 16 by gfx950's permlane swaps
// (one instruction trades a pair of registers' halves, leaving each lane its own value and its
// partner's), within rows by DPP moves. The sums are the same additions in the same order as a
// shuffle through LDS would make. The register indices are compile-time constants: a run-time
// index into v would compile to a compare-and-select chain over the whole array.
__device__ __forceinline__ float f32_of(uint32_t u) { return __uint_as_float(u); }

// lanes of bit `MASK` (32 or 16) clear keep v[i] and add the partner's v[i]; lanes of it set keep
// v[HALF + i] and add the partner's. permlane32_swap trades lanes 32..63 of its first operand
// with lanes 0..31 of its second, permlane16_swap the odd rows of 16 of the first with the even
// rows of the second: either way each lane ends with its kept value in one register and the
// partner's in the other. (Each half of the returned pair is copied into a scalar before its
// bits are read as a float.)
template <int HALF, int MASK>
__device__ __forceinline__ void swap_step(float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < HALF; i++) {
        uint32_t lo, hi;
        if constexpr (MASK == 32) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[HALF + i]), false, false);
            lo = r[0], hi = r[1];
        } else {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[HALF + i]), false, false);
            lo = r[0], hi = r[1];
        }
        // lanes of bit MASK clear: lo = their v[i], hi = the partner's; set: lo = the partner's
        // v[HALF + i], hi = their own. keep + give in either case (addition commutes exactly)
        v[i] = f32_of(lo) + f32_of(hi);
    }
}

// DPP within rows of 16: row_ror:8 reads lane l ^ 8; row_shl:4 reads lane l + 4, row_shr:4 lane
// l - 4, so the lanes of bit 2 clear take the first and those of it set the second (lane l ^ 4)
constexpr int DPP_ROW_SHL4 = 0x104, DPP_ROW_SHR4 = 0x114, DPP_ROW_ROR8 = 0x128;

template <int HALF, int MASK>
__device__ __forceinline__ void dpp_step(float (&v)[16], int lane) {
    const bool upper = lane & MASK;
#pragma unroll
    for (int i = 0; i < HALF; i++) {
        const float keep = upper ? v[HALF + i] : v[i], give = upper ? v[i] : v[HALF + i];
        const int g = __float_as_int(give);
        float other;
        if constexpr (MASK == 8) {
            other = __int_as_float(__builtin_amdgcn_mov_dpp(g, DPP_ROW_ROR8, 0xF, 0xF, false));
        } else {
            const float up = __int_as_float(__builtin_amdgcn_mov_dpp(g, DPP_ROW_SHL4, 0xF, 0xF, false));
            const float down = __int_as_float(__builtin_amdgcn_mov_dpp(g, DPP_ROW_SHR4, 0xF, 0xF, false));
            other = upper ? down : up;
        }
        v[i] = keep + other;
    }
}

__device__ __forceinline__ float transpose_sum16(float (&v)[16], int lane) {
    swap_step<8, 32>(v);
    swap_step<4, 16>(v);
    dpp_step<2, 8>(v, lane);
    dpp_step<1, 4>(v, lane);
    float s = v[0];
    s += LEAT_DPP(s, 0xB1, 0xF, 0xF);  // quad_perm [1,0,3,2]: lane ^ 1
    s += LEAT_DPP(s, 0x4E, 0xF, 0xF);  // quad_perm [2,3,0,1]: lane ^ 2
    return s;
}

// A workgroup per (row, kv head, chunk): its waves take WK keys each a round, from key
// chunk * KEYS + WK w (KEYS = ATT_WAVES WK), then every chunks * KEYS keys on. Lane l holds dimensions 2l, 2l + 1
// of the group's queries (scaled by scale * log2 e, so scores are in log2 units) and reads the
// same two of each key: every key is one coalesced 256-byte read. The keys' partial dot
// products of each lane are summed across the wave by transpose_sum16, the scores go through LDS
// to lanes a key each for the online softmax, and the weighted values are summed with lanes
// again a pair of dimensions (a key's values one coalesced 256-byte read). The waves merge
// through LDS into the workgroup's partial.
template <int G, int WK>
__global__ __launch_bounds__(ATT_WAVES * 64) void attention_partial_kernel(AttentionArgs a) {
    constexpr int KEYS = ATT_WAVES * WK;
    __shared__ float scores[ATT_WAVES][G][WK];
    __shared__ float merge[ATT_WAVES][G][ATT_DIM + 2];
    __shared__ float4 alone_out[G][ATT_DIM / 4];  // a single-chunk row's outputs, for their q8
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = blockIdx.z, kvh = blockIdx.y, chunk = blockIdx.x;
    // the row's slot and length, both asked for at once; a slot outside the cache holds no keys,
    // and lengths past its positions stop at them
    const int slot = a.slots[row], asked = a.lengths[row];
    const int length = slot >= 0 && slot < a.cache_slots ? min(asked, a.cache_positions) : 0;
    const int h0 = kvh * G;
    const float qscale = a.scale * LOG2E;
    float qa[G], qb[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float2 v = *(const float2*)(a.q + ((int64_t)(h0 + h) * a.rows + row) * ATT_DIM + 2 * lane);
        qa[h] = v.x * qscale, qb[h] = v.y * qscale;
    }
    const int64_t head_base = ((int64_t)slot * a.kv_heads + kvh) * a.cache_positions;  // position 0 of the head
    const uint32_t* keys = (const uint32_t*)(a.cache + head_base * ATT_DIM) + lane;
    const uint32_t* vals = (const uint32_t*)(a.cache + ((int64_t)a.cache_slots * a.kv_heads * a.cache_positions + head_base) * ATT_DIM) + lane;
    const int last = a.cache_positions - 1;
    float m[G], l[G], acc[G][2];
#pragma unroll
    for (int h = 0; h < G; h++) m[h] = NEG, l[h] = 0.0f, acc[h][0] = acc[h][1] = 0.0f;

    for (int base = chunk * KEYS + w * WK; base < length; base += a.chunks * KEYS) {
        // the round's keys and values are all read at once (2 WK reads in flight a wave)
        uint32_t kv[WK], vv[WK];
#pragma unroll
        for (int j = 0; j < WK; j++) kv[j] = keys[(int64_t)min(base + j, last) * (ATT_DIM / 2)];
#pragma unroll
        for (int j = 0; j < WK; j++) vv[j] = vals[(int64_t)min(base + j, last) * (ATT_DIM / 2)];
        // scores of keys base .. base + WK - 1, lane l's share of each dot product summed over the
        // wave 16 values at a time: 8 keys of two heads (value i: head 2 hp + i / 8, key i % 8; a
        // missing odd head adds zeros), or 16 keys of one
        if constexpr (WK == 8) {
#pragma unroll
            for (int hp = 0; hp < (G + 1) / 2; hp++) {
                const int odd = 2 * hp + 1 < G ? 2 * hp + 1 : 2 * hp;
                float part[16];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t kj = kv[j];
                    const float k0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(kj & 0xFFFFu));
                    const float k1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(kj >> 16));
                    part[j] = qa[2 * hp] * k0 + qb[2 * hp] * k1;
                    part[8 + j] = 2 * hp + 1 < G ? qa[odd] * k0 + qb[odd] * k1 : 0.0f;
                }
                const float s = transpose_sum16(part, lane);
                const int i = (lane >> 2) & 15;
                if ((lane & 3) == 0 && 2 * hp + i / 8 < G) scores[w][i < 8 ? 2 * hp : odd][i & 7] = s;
            }
        }
#pragma unroll
        for (int sb = 0; sb < WK / 16; sb++) {
#pragma unroll
            for (int h = 0; h < G; h++) {
                float part[16];
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const uint32_t kj = kv[16 * sb + j];
                    const float k0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(kj & 0xFFFFu));
                    const float k1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(kj >> 16));
                    part[j] = qa[h] * k0 + qb[h] * k1;
                }
                const float s = transpose_sum16(part, lane);
                if ((lane & 3) == 0) scores[w][h][16 * sb + (lane >> 2)] = s;
            }
        }
        // the online softmax, a key a lane (lanes WK.. idle): rescale by the new maximum's step
        const int keys_here = min(WK, length - base);
        const bool valid = lane < keys_here;
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float sc = valid ? scores[w][h][lane & (WK - 1)] : NEG;
            const float top = fmaxf(m[h], wave_max_dpp(sc));
            const float p = valid ? exp2f(sc - top) : 0.0f;
            const float shrink = exp2f(m[h] - top);
            m[h] = top;
            l[h] = l[h] * shrink + wave_sum_dpp(p);
            acc[h][0] *= shrink, acc[h][1] *= shrink;
            if (lane < WK) scores[w][h][lane] = p;
        }
        // weighted values: lane = dimensions 2 lane, 2 lane + 1; keys past the row weigh nothing
#pragma unroll
        for (int j = 0; j < WK; j++) {
            // a position past the row's keys may hold anything, NaN included: it adds nothing
            const bool in = j < keys_here;
            const float v0 = in ? (float)__builtin_bit_cast(_Float16, (uint16_t)(vv[j] & 0xFFFFu)) : 0.0f;
            const float v1 = in ? (float)__builtin_bit_cast(_Float16, (uint16_t)(vv[j] >> 16)) : 0.0f;
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float p = scores[w][h][j];  // 0 past the row's keys
                acc[h][0] += p * v0, acc[h][1] += p * v1;
            }
        }
    }
    // merge the waves: each leaves its (sums, max, total) in LDS; the workgroup's partial is
    // the waves' sums rescaled to their common maximum. A row whose keys fit one chunk is done
    // here: chunk 0 writes its sums over their total, the combine's arithmetic for one chunk
    // (a weight of exactly 1), and the combine skips the row.
#pragma unroll
    for (int h = 0; h < G; h++) {
        merge[w][h][2 * lane] = acc[h][0];
        merge[w][h][2 * lane + 1] = acc[h][1];
        if (lane == 0) merge[w][h][ATT_DIM] = m[h], merge[w][h][ATT_DIM + 1] = l[h];
    }
    __syncthreads();
    const bool alone = (length + KEYS - 1) / KEYS <= 1;  // no keys, or all in chunk 0
    if (alone && chunk != 0) return;
    for (int i = threadIdx.x; i < G * (ATT_DIM + 2); i += ATT_WAVES * 64) {
        const int h = i / (ATT_DIM + 2), d = i % (ATT_DIM + 2);
        float top = NEG;
#pragma unroll
        for (int v = 0; v < ATT_WAVES; v++) top = fmaxf(top, merge[v][h][ATT_DIM]);
        float y = 0.0f;
        if (d == ATT_DIM) {
            y = top;
        } else {
#pragma unroll
            for (int v = 0; v < ATT_WAVES; v++) y += exp2f(merge[v][h][ATT_DIM] - top) * merge[v][h][d];
        }
        if (!alone) {
            a.partial[(((int64_t)row * a.heads + h0 + h) * a.chunks + chunk) * (ATT_DIM + 2) + d] = y;
        } else if (d < ATT_DIM) {
            float total = 0.0f;
#pragma unroll
            for (int v = 0; v < ATT_WAVES; v++) total += exp2f(merge[v][h][ATT_DIM] - top) * merge[v][h][ATT_DIM + 1];
            const float inv = total > 0.0f ? 1.0f / total : 0.0f;
            a.out[((int64_t)row * a.heads + h0 + h) * ATT_DIM + d] = y * inv;
            if (a.hq) ((float*)alone_out[h])[d] = y * inv;
        }
    }
    // the q8 of a single-chunk row's G heads: a thread a float4, an octet of threads a group
    if (alone && a.hq) {
        __syncthreads();
        const int t = threadIdx.x, h = t / (ATT_DIM / 4), c = t % (ATT_DIM / 4);
        if (t < G * (ATT_DIM / 4)) attention_q8(a, alone_out[h][c], row, (h0 + h) * ATT_DIM + 4 * c, true);
    }
}

// A workgroup of ATT_COMBINE_WAVES waves per (row, query head). Every load goes out at once (the
// row's slot and length too), so the kernel waits for one round trip: lane c of every wave takes chunk c's max and sum (up to 64
// chunks), and with lane = dimensions 2 lane, 2 lane + 1 wave w takes the partial sums of chunks
// w, w + ATT_COMBINE_WAVES, .... The wave then finds the common maximum and the total weight by
// DPP, rescales its chunks' sums, and the waves' sums meet in LDS.
constexpr int ATT_COMBINE_WAVES = 4;
static_assert(ATT_CHUNKS <= WAVE && ATT_CHUNKS % ATT_COMBINE_WAVES == 0, "a lane per chunk, whole spans");

// SPAN: chunks a wave sums, at least chunks / ATT_COMBINE_WAVES
template <int SPAN>
__global__ __launch_bounds__(ATT_COMBINE_WAVES * 64) void attention_combine_kernel(AttentionArgs a) {
    __shared__ float2 sums[ATT_COMBINE_WAVES - 1][64];
    const int rh = blockIdx.x, row = rh / a.heads, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // the partials of every chunk the workgroup may take, asked for before the row's slot and
    // length (their addresses need neither), at indices clamped into the row's a.chunks entries
    // so that no load waits on a branch; chunks past the live ones are masked below, so whatever
    // an earlier call left there adds nothing
    const float* p = a.partial + (int64_t)rh * a.chunks * (ATT_DIM + 2);
    const int top_chunk = a.chunks - 1;
    // (max, sum) of chunk `lane`: adjacent floats at an 8-byte boundary (rows of 130 floats)
    float2 mine = *(const float2*)(p + min(lane, top_chunk) * (ATT_DIM + 2) + ATT_DIM);
    float2 v[SPAN];
#pragma unroll
    for (int i = 0; i < SPAN; i++) v[i] = *(const float2*)(p + min(w + ATT_COMBINE_WAVES * i, top_chunk) * (ATT_DIM + 2) + 2 * lane);
    const int slot = a.slots[row], asked = a.lengths[row];
    const int length = slot >= 0 && slot < a.cache_slots ? min(asked, a.cache_positions) : 0;
    // a row of one live chunk was written by the partial kernel's chunk 0: the workgroup runs
    // through (no branch for the loads above to sink below) and stores nothing
    const int live = min(a.chunks, (length + (1 << a.key_bits) - 1) >> a.key_bits);
    if (lane >= live) mine = make_float2(NEG, 0.0f);
#pragma unroll
    for (int i = 0; i < SPAN; i++)
        if (w + ATT_COMBINE_WAVES * i >= live) v[i] = make_float2(0.0f, 0.0f);
    const float top = wave_max_dpp(mine.x);
    const float f = lane < live ? exp2f(mine.x - top) : 0.0f;  // chunk lane's weight, 0 past the live chunks
    float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
    for (int i = 0; i < SPAN; i++) {
        // chunk w + ATT_COMBINE_WAVES i's weight, from its lane: a wave-uniform lane index (readlane)
        const float fc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), w + ATT_COMBINE_WAVES * i));
        y0 += fc * v[i].x, y1 += fc * v[i].y;
    }
    if (w > 0) sums[w - 1][lane] = make_float2(y0, y1);
    __syncthreads();
    if (w > 0) return;
    const float total = wave_sum_dpp(f * mine.y);
#pragma unroll
    for (int i = 0; i < ATT_COMBINE_WAVES - 1; i++) y0 += sums[i][lane].x, y1 += sums[i][lane].y;
    const float inv = total > 0.0f ? 1.0f / total : 0.0f;
    float* o = a.out + (int64_t)row * a.heads * ATT_DIM + (int64_t)(rh % a.heads) * ATT_DIM;
    const float2 y = make_float2(y0 * inv, y1 * inv);
    if (live > 1) *(float2*)(o + 2 * lane) = y;
    if (a.hq) {
        // the head's q8: lanes 0..31 gather dimensions 4 lane .. 4 lane + 3 (held by lanes 2 lane
        // and 2 lane + 1), and each octet of them quantizes one group; lanes 32.. take part in the
        // octet reductions of their own rows and store nothing
        const float2 lo = make_float2(__shfl(y.x, 2 * lane, WAVE), __shfl(y.y, 2 * lane, WAVE));
        const float2 hi = make_float2(__shfl(y.x, 2 * lane + 1, WAVE), __shfl(y.y, 2 * lane + 1, WAVE));
        attention_q8(a, make_float4(lo.x, lo.y, hi.x, hi.y), row, (rh % a.heads) * ATT_DIM + 4 * lane,
                     live > 1 && lane < ATT_DIM / 4);
    }
}

template <int G>
static int attention_go(AttentionArgs& a, hipStream_t st) {
    const dim3 chunks(a.chunks, a.kv_heads, a.rows), waves(ATT_WAVES * 64);
    if (a.key_bits == 6)
        hipLaunchKernelGGL((attention_partial_kernel<G, 8>), chunks, waves, 0, st, a);
    else
        hipLaunchKernelGGL((attention_partial_kernel<G, 16>), chunks, waves, 0, st, a);
    if (check_launch("attention")) return -1;
    // one chunk a row (every length at most a round's keys): the partial kernel wrote every row
    if (a.chunks == 1) return 0;
    const dim3 grid(a.rows * a.heads), block(ATT_COMBINE_WAVES * 64);
    const int span = (a.chunks + ATT_COMBINE_WAVES - 1) / ATT_COMBINE_WAVES;
    if (span <= 2)
        hipLaunchKernelGGL(attention_combine_kernel<2>, grid, block, 0, st, a);
    else if (span <= 4)
        hipLaunchKernelGGL(attention_combine_kernel<4>, grid, block, 0, st, a);
    else if (span <= 8)
        hipLaunchKernelGGL(attention_combine_kernel<8>, grid, block, 0, st, a);
    else
        hipLaunchKernelGGL(attention_combine_kernel<ATT_CHUNKS / ATT_COMBINE_WAVES>, grid, block, 0, st, a);
    return check_launch("attention combine");
}

// log2 of the keys a workgroup takes per round for rows of up to max_length keys
static int attention_key_bits(int max_length) {
    static_assert(ATT_WAVES == 8, "8 waves of 8 or 16 keys");
    return max_length > ATT_WAVES * 16 && max_length <= ATT_EIGHT_KEYS_UP_TO ? 6 : 7;
}

static int attention_chunks(int max_length) {
    const int keys = 1 << attention_key_bits(max_length);
    return std::max(1, std::min(ATT_CHUNKS, (max_length + keys - 1) / keys));
}

}  // namespace leat

using namespace leat;

extern "C" int leat_rotate(const float* q, const float* k, const float* v, int tokens, int heads, int kv_heads, int dim,
                           const float* cos, const float* sin, int rotated, int halves, const int32_t* slots,
                           const int32_t* positions, float* q_out, void* cache, int cache_slots, int cache_positions,
                           void* stream) {
    LEAT_REQUIRE(q && k && v && slots && positions && q_out && cache, "rotate: null pointer");
    LEAT_REQUIRE(tokens >= 0 && tokens <= 65535 && heads > 0 && kv_heads > 0 && heads + kv_heads <= 65535,
                 "rotate: %d tokens of %d + %d heads", tokens, heads, kv_heads);
    LEAT_REQUIRE(dim > 0 && dim % 2 == 0, "rotate: heads of %d dimensions (pairs needed)", dim);
    LEAT_REQUIRE(rotated >= 0 && rotated <= dim && rotated % 2 == 0, "rotate: %d rotated dimensions of %d", rotated, dim);
    LEAT_REQUIRE(rotated == 0 || (cos && sin), "rotate: RoPE tables missing");
    LEAT_REQUIRE(cache_slots > 0 && cache_positions > 0, "rotate: an empty cache");
    if (tokens == 0) return 0;
    RotateArgs a = {q, k, v, tokens, heads, kv_heads, dim, cos, sin, rotated, halves != 0, slots, positions, q_out,
                    (_Float16*)cache, cache_slots, cache_positions};
    hipLaunchKernelGGL(rotate_kernel, dim3(heads + kv_heads, tokens), dim3(64), 0, (hipStream_t)stream, a);
    return check_launch("rotate");
}

// Chunks a workspace for rows of at most max_length keys holds: the most that any launch of up to
// max_length keys takes, since launches of 8-key rounds take more chunks than some longer ones
// (2048 keys 32, 2049 keys 17), and a workspace serves every shorter launch.
static int attention_workspace_chunks(int max_length) {
    return max_length > ATT_EIGHT_KEYS_UP_TO
               ? std::max(attention_chunks(max_length), attention_chunks(ATT_EIGHT_KEYS_UP_TO))
               : attention_chunks(max_length);
}

extern "C" int64_t leat_attention_workspace(int rows, int heads, int max_length) {
    return (int64_t)rows * heads * attention_workspace_chunks(max_length) * (ATT_DIM + 2) * 4;
}

static int attention_launch(const float* q, const void* cache, int cache_slots, int kv_heads, int cache_positions,
                            int dim, int rows, int heads, const int32_t* slots, const int32_t* lengths, int max_length,
                            float scale, float* workspace, int64_t workspace_bytes, float* out, uint32_t* hq,
                            float* hd, float* hs, void* stream) {
    LEAT_REQUIRE(q && cache && slots && lengths && workspace && out, "attention: null pointer");
    LEAT_REQUIRE(dim == ATT_DIM, "attention: heads of %d dimensions (this kernel takes %d)", dim, ATT_DIM);
    LEAT_REQUIRE(kv_heads > 0 && heads % kv_heads == 0, "attention: %d query heads over %d kv heads", heads, kv_heads);
    const int group = heads / kv_heads;
    LEAT_REQUIRE(group == 1 || group == 2 || group == 4 || group == 8, "attention: %d query heads a kv head (1, 2, 4 or 8)",
                 group);
    LEAT_REQUIRE(rows >= 0 && rows <= 65535 && kv_heads <= 65535, "attention: %d rows", rows);
    LEAT_REQUIRE(max_length >= 0 && max_length <= cache_positions,
                 "attention: rows of up to %d keys in a cache of %d positions", max_length, cache_positions);
    LEAT_REQUIRE(workspace_bytes >= leat_attention_workspace(rows, heads, max_length),
                 "attention: a workspace of %lld bytes (needs %lld)", (long long)workspace_bytes,
                 (long long)leat_attention_workspace(rows, heads, max_length));
    if (rows == 0) return 0;
    AttentionArgs a = {q, (const _Float16*)cache, cache_slots, kv_heads, cache_positions, rows, heads, group, slots,
                       lengths, attention_chunks(max_length), attention_key_bits(max_length), scale, workspace,
                       out, hq, hd, hs};
    hipStream_t st = (hipStream_t)stream;
    switch (group) {
    case 1: return attention_go<1>(a, st);
    case 2: return attention_go<2>(a, st);
    case 4: return attention_go<4>(a, st);
    default: return attention_go<8>(a, st);
    }
}

extern "C" int leat_attention(const float* q, const void* cache, int cache_slots, int kv_heads, int cache_positions,
                              int dim, int rows, int heads, const int32_t* slots, const int32_t* lengths,
                              int max_length, float scale, float* workspace, int64_t workspace_bytes, float* out,
                              void* stream) {
    return attention_launch(q, cache, cache_slots, kv_heads, cache_positions, dim, rows, heads, slots, lengths,
                            max_length, scale, workspace, workspace_bytes, out, nullptr, nullptr, nullptr, stream);
}

extern "C" int leat_attention_q8(const float* q, const void* cache, int cache_slots, int kv_heads, int cache_positions,
                                 int dim, int rows, int heads, const int32_t* slots, const int32_t* lengths,
                                 int max_length, float scale, float* workspace, int64_t workspace_bytes, float* out,
                                 int32_t* hq, float* hd, float* hs, void* stream) {
    LEAT_REQUIRE(hq && hd && hs, "attention_q8: null q8 output");
    LEAT_REQUIRE((uintptr_t)hq % 4 == 0, "attention_q8: q8 words 4-byte aligned");
    return attention_launch(q, cache, cache_slots, kv_heads, cache_positions, dim, rows, heads, slots, lengths,
                            max_length, scale, workspace, workspace_bytes, out, (uint32_t*)hq, hd, hs, stream);
}

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
            const float c = a.cos[(int64_t)pos * half + i], s = a.sin[(int64_t)pos * half + i];
            const float r0 = x0 * c - x1 * s, r1 = x0 * s + x1 * c;
            x0 = r0, x1 = r1;
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

constexpr int ATT_WAVES = 2;                 // waves a workgroup: 64 keys each
constexpr int ATT_KEYS = ATT_WAVES * WAVE;   // keys a workgroup takes per round
constexpr int ATT_CHUNKS = 64;               // most workgroups per (row, kv head): longer rows loop
constexpr int ATT_GROUP = 8;                 // most query heads sharing a kv head
constexpr int ATT_DIM = 128;                 // head dimension
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
    float scale;
    float* partial;  // (rows * heads, chunks, dim + 2): unnormalized output, then max and sum
    float* out;      // (rows, heads * dim)
};

// A workgroup per (row, kv head, chunk): the group's query heads over keys chunk * ATT_KEYS + 64w +
// lane, then every chunks-th round after. Lane = key while scoring (the key's 128 values from
// 16-byte loads), lane = a pair of dimensions while the weighted values are summed (a key's
// values one coalesced 256-byte read), an online softmax across rounds; the waves' sums merge
// through LDS into the workgroup's partial.
template <int G>
__global__ __launch_bounds__(ATT_WAVES * 64) void attention_partial_kernel(AttentionArgs a) {
    __shared__ float qs[G][ATT_DIM];
    __shared__ float probs[ATT_WAVES][G][WAVE];
    __shared__ float merge[ATT_WAVES][G][ATT_DIM + 2];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = blockIdx.z, kvh = blockIdx.y, chunk = blockIdx.x;
    const int slot = a.slots[row];
    // a slot outside the cache holds no keys; lengths past its positions stop at them
    const int length = slot >= 0 && slot < a.cache_slots ? min(a.lengths[row], a.cache_positions) : 0;
    const int h0 = kvh * G;
    for (int i = threadIdx.x; i < G * ATT_DIM; i += ATT_WAVES * 64)
        qs[i / ATT_DIM][i % ATT_DIM] = a.q[((int64_t)(h0 + i / ATT_DIM) * a.rows + row) * ATT_DIM + i % ATT_DIM];
    __syncthreads();

    const int64_t head_base = ((int64_t)slot * a.kv_heads + kvh) * a.cache_positions;  // position 0 of the head
    const _Float16* keys = a.cache + head_base * ATT_DIM;
    const _Float16* vals = a.cache + ((int64_t)a.cache_slots * a.kv_heads * a.cache_positions + head_base) * ATT_DIM;
    float m[G], l[G], acc[G][2];
#pragma unroll
    for (int h = 0; h < G; h++) m[h] = NEG, l[h] = 0.0f, acc[h][0] = acc[h][1] = 0.0f;

    for (int base = chunk * ATT_KEYS + w * WAVE; base < length; base += a.chunks * ATT_KEYS) {
        // scores: lane = key
        const int key = base + lane;
        const bool valid = key < length;
        const uint4* kp = (const uint4*)(keys + (int64_t)min(key, a.cache_positions - 1) * ATT_DIM);
        float s[G];
#pragma unroll
        for (int h = 0; h < G; h++) s[h] = 0.0f;
#pragma unroll 4
        for (int c = 0; c < ATT_DIM / 8; c++) {
            const uint4 raw = kp[c];
            const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float k0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[e] & 0xFFFFu));
                const float k1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(words[e] >> 16));
#pragma unroll
                for (int h = 0; h < G; h++) s[h] += qs[h][8 * c + 2 * e] * k0 + qs[h][8 * c + 2 * e + 1] * k1;
            }
        }
        // the online softmax: rescale the sums by the new maximum's step
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float sc = valid ? s[h] * a.scale : NEG;
            const float top = fmaxf(m[h], wave_max_dpp(sc));
            const float p = valid ? exp2f((sc - top) * LOG2E) : 0.0f;
            const float shrink = exp2f((m[h] - top) * LOG2E);
            m[h] = top;
            l[h] = l[h] * shrink + wave_sum_dpp(p);
            acc[h][0] *= shrink, acc[h][1] *= shrink;
            probs[w][h][lane] = p;
        }
        // weighted values: lane = dimensions 2 lane, 2 lane + 1; keys past the row weigh 0
        const int keys_here = min(WAVE, length - base);
        for (int j = 0; j < keys_here; j++) {
            const uint32_t pair = *(const uint32_t*)(vals + (int64_t)(base + j) * ATT_DIM + 2 * lane);
            const float v0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(pair & 0xFFFFu));
            const float v1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(pair >> 16));
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float p = probs[w][h][j];
                acc[h][0] += p * v0, acc[h][1] += p * v1;
            }
        }
    }
    // merge the waves: each leaves its (sums, max, total) in LDS; the workgroup's partial is
    // the waves' sums rescaled to their common maximum
#pragma unroll
    for (int h = 0; h < G; h++) {
        merge[w][h][2 * lane] = acc[h][0];
        merge[w][h][2 * lane + 1] = acc[h][1];
        if (lane == 0) merge[w][h][ATT_DIM] = m[h], merge[w][h][ATT_DIM + 1] = l[h];
    }
    __syncthreads();
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
            for (int v = 0; v < ATT_WAVES; v++) y += exp2f((merge[v][h][ATT_DIM] - top) * LOG2E) * merge[v][h][d];
        }
        a.partial[(((int64_t)row * a.heads + h0 + h) * a.chunks + chunk) * (ATT_DIM + 2) + d] = y;
    }
}

// A wave per (row, query head): the chunks' partials rescaled to their common maximum and
// summed, over the sum of their weights; lane = dimensions 2 lane, 2 lane + 1
__global__ __launch_bounds__(64) void attention_combine_kernel(AttentionArgs a) {
    const int rh = blockIdx.x, row = rh / a.heads, lane = threadIdx.x;
    const int slot = a.slots[row];
    const int length = slot >= 0 && slot < a.cache_slots ? min(a.lengths[row], a.cache_positions) : 0;
    const int live = min(a.chunks, (length + ATT_KEYS - 1) / ATT_KEYS);
    const float* p = a.partial + (int64_t)rh * a.chunks * (ATT_DIM + 2);
    float top = NEG;
    for (int c = 0; c < live; c++) top = fmaxf(top, p[c * (ATT_DIM + 2) + ATT_DIM]);
    float y0 = 0.0f, y1 = 0.0f, total = 0.0f;
    for (int c = 0; c < live; c++) {
        const float* q = p + c * (ATT_DIM + 2);
        const float f = exp2f((q[ATT_DIM] - top) * LOG2E);
        total += f * q[ATT_DIM + 1];
        y0 += f * q[2 * lane], y1 += f * q[2 * lane + 1];
    }
    const float inv = total > 0.0f ? 1.0f / total : 0.0f;
    float* o = a.out + (int64_t)row * a.heads * ATT_DIM + (int64_t)(rh % a.heads) * ATT_DIM;
    o[2 * lane] = y0 * inv;
    o[2 * lane + 1] = y1 * inv;
}

template <int G>
static int attention_go(AttentionArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((attention_partial_kernel<G>), dim3(a.chunks, a.kv_heads, a.rows), dim3(ATT_WAVES * 64), 0, st, a);
    if (check_launch("attention")) return -1;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(a.rows * a.heads), dim3(64), 0, st, a);
    return check_launch("attention combine");
}

static int attention_chunks(int max_length) {
    return std::max(1, std::min(ATT_CHUNKS, (max_length + ATT_KEYS - 1) / ATT_KEYS));
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

extern "C" int64_t leat_attention_workspace(int rows, int heads, int max_length) {
    return (int64_t)rows * heads * attention_chunks(max_length) * (ATT_DIM + 2) * 4;
}

extern "C" int leat_attention(const float* q, const void* cache, int cache_slots, int kv_heads, int cache_positions,
                              int dim, int rows, int heads, const int32_t* slots, const int32_t* lengths,
                              int max_length, float scale, float* workspace, int64_t workspace_bytes, float* out,
                              void* stream) {
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
                       lengths, attention_chunks(max_length), scale, workspace, out};
    hipStream_t st = (hipStream_t)stream;
    switch (group) {
    case 1: return attention_go<1>(a, st);
    case 2: return attention_go<2>(a, st);
    case 4: return attention_go<4>(a, st);
    default: return attention_go<8>(a, st);
    }
}

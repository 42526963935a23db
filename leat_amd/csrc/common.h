// Shared device helpers for the gfx950 (CDNA4, wave64) kernels of the quantized-weight path.
//
// GGUF blocks are consumed exactly as stored (no repacking):
//   Q8_0  34 B / 32 weights:  f16 d, int8 qs[32]                       (leat/quant.py:117-119)
//   Q4_K 144 B / 256 weights: f16 d, f16 dmin, u8 scales[12], u8 qs[128] (leat/quant.py:190-197)
//   Q6_K 210 B / 256 weights: u8 ql[128], u8 qh[64], i8 scales[16], f16 d (leat/quant.py:213-223)
// Activations are q8 as leat's quantize_q8 writes them (leat/kernels/quantize.py:25-49): int8
// values packed four per int32 word, per row, and f32 d and s = d * sum(q) per group of 32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace leat {

enum GgmlType : int {
    Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14,
    IQ4_NL = 20, IQ4_XS = 23, MXFP4 = 39
};

constexpr int WAVE = 64;
constexpr int GROUP = 32;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// a 16-byte vector whose address is only known to be 4-byte aligned: global_load_dwordx4 needs
// dword alignment only
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef u32x2 u32x2_a4 __attribute__((aligned(4)));

__device__ __forceinline__ float f16_lo(uint32_t word) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(word & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(uint32_t word) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(word >> 16));
}

// acc + the dot product of the four signed bytes of a and b (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int acc) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, acc, false);
}

// 32 bits from byte `shift` (0..3) of the 64-bit (hi:lo)
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// each byte b (< 2 * offset) of a word as the signed byte b - offset: b + 128 - offset stays in
// its byte, and flipping the top bit makes it b - offset in two's complement
__device__ __forceinline__ uint32_t minus_bytes(uint32_t q, uint32_t offset) {
    return (q + (128u - offset) * 0x01010101u) ^ 0x80808080u;
}

// a weight load: a plain one. Marking them nontemporal (streamed once) measured slower on gfx950:
// a block's bytes straddle 128-byte lines that neighbouring loads read again, and the hint evicts
// them first.
template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
    return *p;
}

// RoPE of one pair of dimensions by its angle's cosine c and sine s: (x0 c - x1 s, x0 s + x1 c),
// each as one fused multiply-add of a product, so every kernel that turns pairs rounds them alike
__device__ __forceinline__ void rope_pair(float& x0, float& x1, float c, float s) {
    const float r0 = fmaf(x0, c, -(x1 * s)), r1 = fmaf(x0, s, x1 * c);
    x0 = r0, x1 = r1;
}

// 16 bytes at a byte offset that is even but maybe not 4-aligned: 5 aligned dwords, realigned
__device__ __forceinline__ void load16_even(const uint8_t* base, uint64_t off, uint32_t out[4]) {
    const uint32_t* p = (const uint32_t*)(base + (off & ~(uint64_t)3));
    uint32_t shift = (uint32_t)(off & 3);
    u32x4 a = stream_load((const u32x4_a4*)p);
    uint32_t e = stream_load(p + 4);
    out[0] = align_bytes(a[1], a[0], shift);
    out[1] = align_bytes(a[2], a[1], shift);
    out[2] = align_bytes(a[3], a[2], shift);
    out[3] = align_bytes(e, a[3], shift);
}

// The xor butterfly over the wave's 64 lanes (partners 32, 16, 8, 4, 2, 1 lanes apart, in that
// order), every lane ending with the sum, by gfx950's permlane32 / permlane16 swaps and DPP moves
// instead of shuffles (no LDS traffic). Each step adds the partner's value to the lane's own, the
// shuffle butterfly's arithmetic, so sums are bit for bit the same; all 64 lanes must be active.
// T: a 32-bit type.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    static_assert(sizeof(T) == 4, "32-bit values");
    auto bits = [](T x) { return __builtin_bit_cast(uint32_t, x); };
    auto val = [](uint32_t x) { return __builtin_bit_cast(T, x); };
    {
        // lanes with the step's bit clear get (own, partner), those with it set (partner, own)
        const auto r = __builtin_amdgcn_permlane32_swap(bits(v), bits(v), false, false);
        const uint32_t lo = r[0], hi = r[1];
        v = val(lo) + val(hi);
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(bits(v), bits(v), false, false);
        const uint32_t lo = r[0], hi = r[1];
        v = val(lo) + val(hi);
    }
    v += val((uint32_t)__builtin_amdgcn_update_dpp(0, (int)bits(v), 0x128, 0xF, 0xF, false));  // row_ror:8 (lane ^ 8)
    {
        // lane ^ 4: row_shl:4 into banks 0 and 2, row_shr:4 into banks 1 and 3
        int other = __builtin_amdgcn_update_dpp((int)bits(v), (int)bits(v), 0x104, 0xF, 0x5, false);
        other = __builtin_amdgcn_update_dpp(other, (int)bits(v), 0x114, 0xF, 0xA, false);
        v += val((uint32_t)other);
    }
    v += val((uint32_t)__builtin_amdgcn_update_dpp(0, (int)bits(v), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    v += val((uint32_t)__builtin_amdgcn_update_dpp(0, (int)bits(v), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    return v;
}

// the sum over the wave's 64 lanes, in every lane, by DPP moves (quad permutes, row shifts and
// row broadcasts): no LDS traffic, unlike a shuffle's ds_bpermute
#define LEAT_DPP(v, ctrl, rm, bm) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rm, bm, false))

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += LEAT_DPP(v, 0xB1, 0xF, 0xF);   // quad_perm [1,0,3,2]
    v += LEAT_DPP(v, 0x4E, 0xF, 0xF);   // quad_perm [2,3,0,1]: each lane holds its quad's sum
    v += LEAT_DPP(v, 0x114, 0xF, 0xE);  // row_shr:4 into banks 1..3
    v += LEAT_DPP(v, 0x118, 0xF, 0xC);  // row_shr:8 into banks 2..3: lane 15 of a row holds its sum
    v += LEAT_DPP(v, 0x142, 0xA, 0xF);  // row_bcast:15 into rows 1 and 3
    v += LEAT_DPP(v, 0x143, 0xC, 0xF);  // row_bcast:31 into rows 2 and 3: lane 63 holds the total
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// the same reduction for max (floats) and min (ints): lanes a move leaves out keep the operation's
// identity (-inf, INT_MAX) as their moved value
#define LEAT_DPP_ID(id, v, ctrl, rm, bm) __builtin_amdgcn_update_dpp(id, v, ctrl, rm, bm, false)
__device__ __forceinline__ float wave_max_dpp(float v) {
    const int ninf = __builtin_bit_cast(int, -INFINITY);
#define LEAT_MAX_STEP(ctrl, rm, bm) \
    v = fmaxf(v, __builtin_bit_cast(float, LEAT_DPP_ID(ninf, __builtin_bit_cast(int, v), ctrl, rm, bm)))
    LEAT_MAX_STEP(0xB1, 0xF, 0xF);
    LEAT_MAX_STEP(0x4E, 0xF, 0xF);
    LEAT_MAX_STEP(0x114, 0xF, 0xE);
    LEAT_MAX_STEP(0x118, 0xF, 0xC);
    LEAT_MAX_STEP(0x142, 0xA, 0xF);
    LEAT_MAX_STEP(0x143, 0xC, 0xF);
#undef LEAT_MAX_STEP
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ int wave_min_dpp(int v) {
#define LEAT_MIN_STEP(ctrl, rm, bm) v = min(v, LEAT_DPP_ID(0x7FFFFFFF, v, ctrl, rm, bm))
    LEAT_MIN_STEP(0xB1, 0xF, 0xF);
    LEAT_MIN_STEP(0x4E, 0xF, 0xF);
    LEAT_MIN_STEP(0x114, 0xF, 0xE);
    LEAT_MIN_STEP(0x118, 0xF, 0xC);
    LEAT_MIN_STEP(0x142, 0xA, 0xF);
    LEAT_MIN_STEP(0x143, 0xC, 0xF);
#undef LEAT_MIN_STEP
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, WAVE));
    return v;
}

// The GLU activations of leat/kernels/common.py:299-321: silu(g)*u, gelu(g)*u (tanh
// approximation) and gpt-oss's clamped "oai" SwiGLU.
enum GluKind : int { GLU_SILU = 0, GLU_GELU = 1, GLU_OAI = 2 };

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

__device__ __forceinline__ float glu(int kind, float g, float u) {
    if (kind == GLU_OAI) {
        g = fminf(g, 7.0f);
        u = fminf(fmaxf(u, -7.0f), 7.0f);
        return g * sigmoid(1.702f * g) * (u + 1.0f);
    }
    if (kind == GLU_GELU) {
        const float c = 1.5957691216057308f;  // 2 * sqrt(2 / pi)
        return g * sigmoid(c * (g + 0.044715f * g * g * g)) * u;
    }
    return g * sigmoid(g) * u;
}

}  // namespace leat

// ---------------------------------------------------------------- host-side error plumbing
namespace leat {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
// weights and activation words aligned as the kernels read them (matvec.hip)
int check_ptrs(int type, const void* w, const void* xq);
// a row length of whole decode tasks of `type` (matvec.hip)
int check_cols(int type, int cols);
}  // namespace leat

#define LEAT_REQUIRE(cond, ...)          \
    do {                                 \
        if (!(cond)) {                   \
            ::leat::set_error(__VA_ARGS__); \
            return -1;                   \
        }                                \
    } while (0)

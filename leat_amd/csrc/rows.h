// The row-streaming decode kernels' arguments and launcher (rows.hip), shared with matvec.hip.
#pragma once

#include "common.h"

namespace leat {

constexpr int ROWS_MATS = 4;
constexpr int ROWS_MAX_TOKENS = 2;

// The q, k and v products' rows turned by RoPE and stored for attention in the launch's epilogue
// (leat_qkv_rotate_f32): pairs of adjacent dimensions, the first `rotated` of each head's `dim`
struct RopeStore {
    const float* cos;  // (cache positions, rotated / 2)
    const float* sin;
    int rotated, dim, kv_heads;
    const int32_t* slots;      // tokens
    const int32_t* positions;  // tokens
    float* q_out;              // (heads, tokens, dim) f32; null: no epilogue
    _Float16* cache;           // (2, cache_slots, kv_heads, cache_positions, dim)
    int cache_slots, cache_positions;
};

struct RowsArgs {
    const uint8_t* w[ROWS_MATS];  // the GLU: gate, up
    float* out[ROWS_MATS];        // the GLU: out[0], or null when only its q8 is wanted
    int rows[ROWS_MATS];
    int tile_start[ROWS_MATS + 1];  // first workgroup of each matrix; tile_start[count] = total
    int count;
    int cols;
    // activations: quantized (xq, xd, xs), or f32 rows x quantized by the kernel after an RMSNorm
    // with `norm` (null: none) and `eps`
    const int32_t* xq;
    const float* xd;
    const float* xs;
    const float* x;
    const float* norm;
    float eps;
    const float* residual;  // ROWS_RESIDUAL: tokens * rows[0]
    int kind;               // ROWS_GLU: the GLU kind
    uint32_t* hq;           // ROWS_GLU: q8 of the outputs (rows a multiple of 32), or null
    float* hd;
    float* hs;
    RopeStore rope;         // ROWS_PLAIN over q, k, v: their RoPE and KV store (rope.q_out set)
};

// whether the row-streaming kernels take this type, row length and token count (glu: for the
// gate+up GLU, which takes shorter rows)
bool rows_fits(int type, int cols, int tokens, bool glu);
// mode: 0 plain (up to ROWS_MATS matrices), 1 residual, 2 gate+up GLU; xf32: quantize a.x
int rows_launch(int type, int mode, RowsArgs& a, int tokens, bool xf32, hipStream_t st);

}  // namespace leat

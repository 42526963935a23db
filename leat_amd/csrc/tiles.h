// The matrix-core decode kernels for 3..16 tokens of Q4_K (tiles.hip), shared with matvec.hip.
#pragma once

#include "common.h"

namespace leat {

constexpr int TILES_MATS = 4;

struct TileArgs {
    const uint8_t* w[TILES_MATS];  // the GLU: gate, up
    float* out[TILES_MATS];        // the GLU: out[0], or null when only its q8 is wanted
    int rows[TILES_MATS];
    int tile_start[TILES_MATS + 1];  // first 32-row tile of each matrix; tile_start[count] = total
    int count;
    int cols;
    int tokens;
    const int32_t* xq;  // the tokens' q8 words, scales d and sums s
    const float* xd;
    const float* xs;
    const float* residual;  // mode 1: tokens * rows[0]
    int kind;               // mode 2: the GLU kind
    uint32_t* hq;           // mode 2: q8 of the outputs (rows a multiple of 32), or null
    float* hd;
    float* hs;
};

// whether the tile kernels take this type, row length, token count and weight alignment
bool tiles_fits(int type, int cols, int tokens, const void* const* ws, int count);
// mode: 0 plain (up to TILES_MATS matrices), 1 residual, 2 gate+up GLU
int tiles_launch(int type, int mode, TileArgs& a, hipStream_t st);

}  // namespace leat

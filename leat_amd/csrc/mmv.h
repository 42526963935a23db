// The matrix-core decode kernels' arguments and launcher (mmv.hip), shared with matvec.hip.
#pragma once

#include "common.h"

namespace leat {

constexpr int MMV_MATS = 4;

struct MmvArgs {
    const uint8_t* w[MMV_MATS];
    float* out[MMV_MATS];
    int rows[MMV_MATS];
    int tile_start[MMV_MATS + 1];  // first 32-row tile of each matrix
    int count;
    int cols;
    int tokens;
    const int32_t* xq;
    const float* xd;
    const float* xs;
    const float* residual;  // MMV_RESIDUAL: tokens * rows[0]
    int kind;               // MMV_GLU: w[0] gate, w[1] up, out[0]
    int parts;              // set by mmv_launch: workgroups a tile's blocks are split over (1, or 2:
                            // the two sums are added atomically into zeroed outputs)
};

enum MmvMode : int { MMV_PLAIN = 0, MMV_RESIDUAL = 1, MMV_GLU = 2 };

// whether the matrix-core path takes this shape: 1..16 tokens, whole blocks per row (pairs of
// blocks for Q6_K and Q8_0), rows a whole number of 16-byte chunks, matrices 16-byte aligned
bool mmv_fits(int type, int cols, int tokens, const void* const* ws, int count);
int mmv_launch(int type, int mode, MmvArgs& a, hipStream_t st);

}  // namespace leat

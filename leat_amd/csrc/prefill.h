// The Q4_K prefill kernels (prefill.hip), shared with mmq.hip's entry points.
#pragma once

#include "common.h"

namespace leat {

// Q4_K weights, 16-byte aligned, cols a multiple of 256, xq 16-byte aligned (checked by the caller).
// mode: 0 plain, 1 residual, 2 GLU (ws[0] gate, ws[1] up)
int prefill_launch(int mode, const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                   const float* xs, int tokens, const float* residual, int kind, float* out, hipStream_t st);

}  // namespace leat

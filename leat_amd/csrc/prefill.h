// The prefill kernels of Q4_K (prefill.hip) and Q6_K (prefill6.hip) weights, behind mmq.hip's
// entry points.
#pragma once

#include "common.h"

namespace leat {

enum PrefillMode : int { PF_PLAIN = 0, PF_RESIDUAL = 1, PF_GLU = 2 };

// Q4_K weights, 16-byte aligned, cols a multiple of 256, xq 16-byte aligned (checked by the caller).
// mode: 0 plain, 1 residual, 2 GLU (ws[0] gate, ws[1] up; out may be null when hq is given). hq,
// hd, hs (the GLU, rows a multiple of 32): also the q8 of the outputs, as quantize_q8 gives it.
int prefill_launch(int mode, const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                   const float* xs, int tokens, const float* residual, int kind, float* out, hipStream_t st,
                   uint32_t* hq = nullptr, float* hd = nullptr, float* hs = nullptr);

// Q6_K weights of 4-byte aligned rows (cols a multiple of 512), xq 16-byte aligned: out = W x (+ residual)
bool prefill_q6k_fits(int cols);
int prefill_q6k_launch(const void* w, int rows, int cols, const int32_t* xq, const float* xd, int tokens,
                       const float* residual, float* out, hipStream_t st);

}  // namespace leat

// The prefill kernels of Q4_K (prefill.hip) and Q6_K (prefill6.hip) weights, behind mmq.hip's
// entry points.
#pragma once

#include "common.h"

namespace leat {

enum PrefillMode : int { PF_PLAIN = 0, PF_RESIDUAL = 1, PF_GLU = 2 };

// A split product (leat/kernels/matmul.py:926-964, _schedule): when a launch has fewer tiles than
// the GPU runs at once, each tile's K steps are dealt over `chunks` workgroups whose f32 sums land
// in a workspace of `bytes`, and a fixup launch adds them in chunk order and writes the outputs.
struct Split {
    int chunks;     // 1: no split
    int64_t bytes;  // the workspace it needs
};
// the split for `tiles` workgroup tiles of `steps` K steps, each chunk's sums taking part_bytes:
// chunks double while the launch still fits the GPU's workgroup slots (two a CU) and each chunk
// keeps at least 4 steps, up to 8
Split split_schedule(int tiles, int steps, int64_t part_bytes);
// the current device's compute units
int cu_count();

// leat_matmul (mmq.hip) with an explicit workspace, and the workspace its split takes
int64_t matmul_workspace(int type, int rows, int cols, int tokens, bool gated);
int matmul_go(int type, const void* w, int rows, int cols, const int32_t* xq, const float* xd, const float* xs,
              int tokens, const float* residual, float* out, void* workspace, int64_t workspace_bytes, hipStream_t st);

// Q4_K weights, 16-byte aligned, cols a multiple of 256, xq 16-byte aligned (checked by the caller).
// mode: 0 plain, 1 residual, 2 GLU (ws[0] gate, ws[1] up; out may be null when hq is given). hq,
// hd, hs (the GLU, rows a multiple of 32): also the q8 of the outputs, as quantize_q8 gives it.
// A workspace of at least prefill_split(...).bytes lets a launch of few tiles split (else it runs
// unsplit).
Split prefill_split(int mode, int rows, int cols, int tokens);
int prefill_launch(int mode, const void* const* ws, int rows, int cols, const int32_t* xq, const float* xd,
                   const float* xs, int tokens, const float* residual, int kind, float* out, hipStream_t st,
                   uint32_t* hq = nullptr, float* hd = nullptr, float* hs = nullptr, void* workspace = nullptr,
                   int64_t workspace_bytes = 0);

// Q6_K weights of 4-byte aligned rows (cols a multiple of 512), xq 16-byte aligned: out = W x (+ residual)
bool prefill_q6k_fits(int cols);
Split prefill_q6k_split(int rows, int cols, int tokens);
int prefill_q6k_launch(const void* w, int rows, int cols, const int32_t* xq, const float* xd, int tokens,
                       const float* residual, float* out, hipStream_t st, void* workspace = nullptr,
                       int64_t workspace_bytes = 0);

}  // namespace leat

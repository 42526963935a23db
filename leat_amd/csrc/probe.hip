// Measurement probes: the rates this GPU reaches on a plain streaming read and on back-to-back
// int8 matrix-core products, reported beside the published peaks (8 TB/s HBM, 5.0 POPS dense
// int8) that the benchmark's rooflines divide by. Neither has a counterpart in leat; both return
// values a test can check exactly, so a probe that skipped work would show.
#include "common.h"

namespace leat {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int PROBE_THREADS = 256;
constexpr int PROBE_UNROLL = 4;  // 16-byte loads a thread has in flight

// Every 32-bit word of `words` x 4 (16-byte chunks), summed modulo 2^32: workgroup g leaves its
// sum in sink[g]. Thread loads are 16 bytes, PROBE_UNROLL of them in flight, the workgroups'
// chunks interleaved so that each pass of the grid reads one contiguous span.
__global__ __launch_bounds__(PROBE_THREADS) void probe_read_kernel(const uint4* data, int64_t chunks, uint32_t* sink) {
    __shared__ uint32_t part[PROBE_THREADS / WAVE];
    const int64_t threads = (int64_t)gridDim.x * PROBE_THREADS;
    uint32_t sum = 0;
    for (int64_t base = (int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x; base < chunks; base += threads * PROBE_UNROLL) {
        uint4 v[PROBE_UNROLL];
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; u++) {
            const int64_t at = base + threads * u;
            v[u] = at < chunks ? data[at] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; u++) sum += v[u].x + v[u].y + v[u].z + v[u].w;
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & (WAVE - 1)) == 0) part[threadIdx.x / WAVE] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t total = 0;
#pragma unroll
        for (int w = 0; w < PROBE_THREADS / WAVE; w++) total += part[w];
        sink[blockIdx.x] = total;
    }
}

// Each wave runs `iters` rounds of 4 v_mfma_i32_32x32x32_i8 on 4 independent accumulators, every
// operand byte 1: each product adds 32 to every accumulator element, so after the loop every
// element of each accumulator is 32 * iters. Wave w of workgroup g leaves the sum of its lane 0's
// first elements, 4 * 32 * iters, in sink[4 g + w].
__global__ __launch_bounds__(PROBE_THREADS) void probe_mfma_kernel(int iters, int32_t* sink) {
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    v16i acc[4] = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ones, ones, acc[c], 0, 0, 0);
    }
    if ((threadIdx.x & (WAVE - 1)) == 0) sink[blockIdx.x * (PROBE_THREADS / WAVE) + threadIdx.x / WAVE] = acc[0][0] + acc[1][0] + acc[2][0] + acc[3][0];
}

}  // namespace

}  // namespace leat

using namespace leat;

extern "C" int leat_probe_read(const void* data, int64_t bytes, uint32_t* sink, int workgroups, void* stream) {
    LEAT_REQUIRE(data && sink, "probe_read: null pointer");
    LEAT_REQUIRE(bytes > 0 && bytes % 16 == 0 && (uintptr_t)data % 16 == 0, "probe_read: %lld bytes: whole 16-byte chunks, 16-byte aligned", (long long)bytes);
    LEAT_REQUIRE(workgroups > 0 && workgroups <= 65536, "probe_read: %d workgroups", workgroups);
    hipLaunchKernelGGL(probe_read_kernel, dim3(workgroups), dim3(PROBE_THREADS), 0, (hipStream_t)stream,
                       (const uint4*)data, bytes / 16, sink);
    return check_launch("probe_read");
}

extern "C" int leat_probe_mfma_i8(int iters, int workgroups, int32_t* sink, void* stream) {
    LEAT_REQUIRE(sink, "probe_mfma_i8: null pointer");
    LEAT_REQUIRE(iters > 0 && iters <= (1 << 22), "probe_mfma_i8: %d rounds (1..4194304)", iters);
    LEAT_REQUIRE(workgroups > 0 && workgroups <= 65536, "probe_mfma_i8: %d workgroups", workgroups);
    hipLaunchKernelGGL(probe_mfma_kernel, dim3(workgroups), dim3(PROBE_THREADS), 0, (hipStream_t)stream, iters, sink);
    return check_launch("probe_mfma_i8");
}

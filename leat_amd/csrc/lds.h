// Building blocks of the prefill kernels (prefill.hip, prefill6.hip): direct global->LDS loads,
// LDS reads at raw addresses, the matrix-core products they use, and a compile-time loop.
#pragma once

#include <type_traits>

#include "common.h"

namespace leat {
namespace pf {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void global_void;

// global_load_lds: every lane's 16 (or 4) bytes from its own address land at LDS address
// lds_at + 16 * lane (4 * lane); lds_at is uniform. The loads count in vmcnt.
__device__ __forceinline__ void to_lds16(const void* src, uint32_t lds_at) {
    __builtin_amdgcn_global_load_lds((global_void*)src, (lds_void*)(uintptr_t)lds_at, 16, 0, 0);
}
__device__ __forceinline__ void to_lds4(const void* src, uint32_t lds_at) {
    __builtin_amdgcn_global_load_lds((global_void*)src, (lds_void*)(uintptr_t)lds_at, 4, 0, 0);
}

// s_waitcnt vmcnt(0): every direct load this wave issued has landed in LDS
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <typename T>
__device__ __forceinline__ T lds_read(uint32_t at) {
    return *(const __attribute__((address_space(3))) T*)(uintptr_t)at;
}

// v_mfma_i32_32x32x32_i8: lane l supplies row l % 32 of A (M) and of B (N) with the 16 values
// 16h..16h+15 of K (h = l / 32); the int32 result in lane l is N = l % 32 for
// M = 8(v / 4) + 4h + v % 4 in registers v
__device__ __forceinline__ v16i mfma_i8(v4i a, u32x4 b) {
    const v16i zero = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, __builtin_bit_cast(v4i, b), zero, 0, 0, 0);
}
// v_mfma_f32_32x32x2f32: c + the K = 2 product, lane half h supplying k = h
__device__ __forceinline__ v16f mfma_f32(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
// two outer products at once (v_mfma_f32_32x32x1_2b_f32): block k = lane half, its a[i] from
// lane i + 32k, b[j] from lane j + 32k; block k's result in registers 16k.. in the 32x32 layout
__device__ __forceinline__ v32f mfma_outer2(float a, float b) {
    const v32f zero = {};
    return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, zero, 0, 0, 0);
}

template <int K, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (K < N) {
        f(std::integral_constant<int, K>{});
        static_for<K + 1, N>(f);
    }
}

}  // namespace pf
}  // namespace leat

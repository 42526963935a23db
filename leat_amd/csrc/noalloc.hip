// leat_matmul for callers that cannot allocate device memory (code under HIP graph capture,
// serving loops that forbid hipMalloc): a split product's partial sums go to a file-scope device
// array instead of a caller's workspace. The array is SCRATCH_BYTES on every GPU the library
// runs on, held until the process ends. Every call on one GPU shares that GPU's array, so calls
// that overlap on one GPU (on different streams) race; calls in one stream order are safe. The
// array keeps the last call's partial sums: nothing in it needs to start at zero, since every
// chunk's slice is written before the fixup reads it.
#include <mutex>

#include "prefill.h"

namespace leat {

constexpr int64_t SCRATCH_BYTES = int64_t(8) << 20;
constexpr int SCRATCH_DEVICES = 64;

static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

// the array's address on each device, looked up once with that device current: a host-side
// `scratch` is only a stand-in symbol, never a device address
static void* scratch_at[SCRATCH_DEVICES];
static hipError_t scratch_status[SCRATCH_DEVICES];
static std::once_flag scratch_once[SCRATCH_DEVICES];

static void* scratch_on(int device) {
    std::call_once(scratch_once[device], [device] {
        void* at = nullptr;
        scratch_status[device] = hipGetSymbolAddress(&at, HIP_SYMBOL(scratch));
        scratch_at[device] = at;
    });
    return scratch_status[device] == hipSuccess ? scratch_at[device] : nullptr;
}

}  // namespace leat

using namespace leat;

extern "C" int leat_matmul_noalloc(int type, const void* w, int rows, int cols, const int32_t* xq, const float* xd,
                                   const float* xs, int tokens, const float* residual, float* out, void* stream) {
    int device = 0;
    LEAT_REQUIRE(hipGetDevice(&device) == hipSuccess && device >= 0 && device < SCRATCH_DEVICES,
                 "matmul_noalloc: no current device below %d", SCRATCH_DEVICES);
    const int64_t need = matmul_workspace(type, rows, cols, tokens, false);
    LEAT_REQUIRE(need <= SCRATCH_BYTES,
                 "matmul_noalloc: this product splits into %lld bytes of partial sums; the no-allocation entry "
                 "holds %lld (call leat_matmul with a workspace)",
                 (long long)need, (long long)SCRATCH_BYTES);
    void* at = need > 0 ? scratch_on(device) : nullptr;
    LEAT_REQUIRE(need == 0 || at, "matmul_noalloc: the scratch array's address: %s",
                 hipGetErrorString(scratch_status[device]));
    return matmul_go(type, w, rows, cols, xq, xd, xs, tokens, residual, out, at, need > 0 ? SCRATCH_BYTES : 0,
                     (hipStream_t)stream);
}

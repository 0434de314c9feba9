// noalloc.hip -- cm_matmul_noalloc: cm_matmul_ex for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  Its split-K partial sums live in a
// file-scope device array instead of a caller's workspace.
//
// The array is `scratch`, kScratchBytes large; every GPU the library runs on
// holds its own copy from module load until the process ends.  Host code never
// passes the array's name to a kernel or a copy (on the host that name is a
// stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, taken once per device with that device current, at the
// first call on it, and is kept per device.
//
// Every call on one GPU shares that GPU's array and it keeps the last call's
// contents.  Nothing in it needs clearing: each split block writes every
// partial it owns before the reduce pass reads it.  Calls that overlap in time
// on one GPU (different streams, a replayed graph beside eager work) race on it.
#include <mutex>

#include "cm_internal.h"

namespace {

constexpr size_t kScratchBytes = 16u << 20;   // 16 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mutex;
void* g_ptr[kMaxDevices] = {};   // device address of `scratch` on each device

// The device address of this device's `scratch`, looked up on first use.
int scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return cm_set_error(CM_ERR_HIP, "matmul_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return cm_set_error(CM_ERR_RANGE, "matmul_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return cm_set_error(CM_ERR_HIP, "matmul_noalloc: hipGetSymbolAddress(scratch): %s",
                                hipGetErrorString(e));
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return CM_OK;
}

}  // namespace

extern "C" int cm_matmul_noalloc(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n,
                                 uint32_t k, uint32_t m, uint32_t batch, uint32_t a_stride,
                                 uint32_t b_stride, uint32_t c_stride, const cm_epilogue_t* epi,
                                 hipStream_t stream) {
    if (batch == 0 || n == 0 || m == 0) return CM_OK;
    size_t need = 0;
    {
        const LaunchCtx dry{nullptr, nullptr, 0u, &need};
        const int rc = cm_matmul_launch(a, b, c, n, k, m, batch, a_stride, b_stride, c_stride,
                                        nullptr, dry);
        if (rc) return rc;
    }
    if (need > kScratchBytes)
        return cm_set_error(CM_ERR_RANGE,
                            "matmul_noalloc: this shape's split-K partials need %zu bytes, above the "
                            "%zu-byte static scratch; use cm_matmul_ex with a workspace",
                            need, kScratchBytes);
    void* ws = nullptr;
    if (need) {
        const int rc = scratch_ptr(&ws);
        if (rc) return rc;
    }
    return cm_matmul_ex(a, b, c, n, k, m, batch, a_stride, b_stride, c_stride, epi, ws,
                        need ? kScratchBytes : 0u, stream);
}

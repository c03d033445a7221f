// nq_linear_static: nq_linear for callers that cannot allocate device memory
// (code under HIP graph capture that may not call hipMalloc, tight serving
// loops, harnesses that forbid allocation). The workspace nq_linear takes as
// an argument is instead a file-scope device array of NQ_STATIC_SCRATCH_BYTES
// bytes: every GPU the library runs on holds its own copy until the process
// ends. Nothing in it needs to start at zero (every kernel writes the
// workspace bytes it later reads), so no call clears it. Calls share the
// array: two calls that overlap in time on one GPU (different streams without
// ordering) race on it and must not be issued.
#include <mutex>

#include "nq_common.h"

namespace {

static __device__ __align__(256) uint8_t scratch[NQ_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch` on each device

// Device address of this device's copy of `scratch`, looked up once per
// device with that device current (the host-side name of the array is not a
// device address and must never reach a kernel).
int scratch_address(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return NQ_ERR_DEVICE;
    }
    std::lock_guard<std::mutex> hold(g_lock);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return NQ_ERR_DEVICE;
        }
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return NQ_OK;
}

}  // namespace

extern "C" int nq_linear_static(const nq_linear_desc* desc, const void* x, int32_t x_dtype, int64_t tokens,
                                void* y, int32_t y_dtype, void* stream) {
    const int64_t need = nq_linear_workspace_bytes(desc, tokens);
    if (need < 0) {
        // The same validation nq_linear runs, for its status code.
        return nq_linear(desc, x, x_dtype, tokens, y, y_dtype, nullptr, 0, stream);
    }
    if (need > NQ_STATIC_SCRATCH_BYTES) return NQ_ERR_SCRATCH;
    void* ws = nullptr;
    const int st = scratch_address(&ws);
    if (st != NQ_OK) return st;
    return nq_linear(desc, x, x_dtype, tokens, y, y_dtype, ws, NQ_STATIC_SCRATCH_BYTES, stream);
}

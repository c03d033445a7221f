// Library-level entry points: ABI version, status text and device query.
#include <string.h>

#include "nq_common.h"

extern "C" int nq_abi_version(void) { return NQ_ABI_VERSION; }

extern "C" const char* nq_status_string(int status) {
    switch (status) {
        case NQ_OK: return "ok";
        case NQ_ERR_ARGUMENT: return "invalid argument (null pointer or inconsistent sizes)";
        case NQ_ERR_DTYPE: return "dtype not accepted for this operand";
        case NQ_ERR_SHAPE: return "dimension outside the supported range";
        case NQ_ERR_ALIGNMENT: return "pointer alignment required by the kernel is missing";
        case NQ_ERR_WORKSPACE: return "workspace smaller than nq_linear_workspace_bytes";
        case NQ_ERR_LAUNCH: return "kernel launch failed";
        case NQ_ERR_DEVICE: return "no usable HIP device";
        case NQ_ERR_UNSUPPORTED: return "request not implemented by this library";
        case NQ_ERR_SCRATCH: return "request needs more workspace than the static scratch array (NQ_STATIC_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

extern "C" int nq_query_device(int device, nq_device_caps* out) {
    if (!out) return NQ_ERR_ARGUMENT;
    memset(out, 0, sizeof(*out));
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        (void)hipGetLastError();
        return NQ_ERR_DEVICE;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return NQ_ERR_DEVICE;
    strncpy(out->arch, prop.gcnArchName, sizeof(out->arch) - 1);
    out->compute_units = prop.multiProcessorCount;
    out->wavefront_size = prop.warpSize;
    out->lds_bytes_per_block = static_cast<int64_t>(prop.sharedMemPerBlock);
    out->global_mem_bytes = static_cast<int64_t>(prop.totalGlobalMem);
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width_bits = prop.memoryBusWidth;
    out->is_gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
    return NQ_OK;
}

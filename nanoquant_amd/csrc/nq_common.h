// Shared device helpers for the gfx950 packed-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nqamd.h"

namespace nq {

// Scalar load of element `i` of a typed buffer as fp32. The dtype is uniform
// across a launch, so the switch is a uniform branch.
__device__ __forceinline__ float load_f32(const void* __restrict__ p, int dtype, int64_t i) {
    switch (dtype) {
        case NQ_DTYPE_F32:
            return static_cast<const float*>(p)[i];
        case NQ_DTYPE_F16:
            return static_cast<float>(static_cast<const _Float16*>(p)[i]);
        case NQ_DTYPE_BF16:
            return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
        case NQ_DTYPE_I8:
            return static_cast<float>(static_cast<const int8_t*>(p)[i]);
        default:
            return 0.0f;
    }
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ void store_f32_as(void* __restrict__ p, int dtype, int64_t i, float v) {
    switch (dtype) {
        case NQ_DTYPE_F32:
            static_cast<float*>(p)[i] = v;
            break;
        case NQ_DTYPE_F16:
            static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
            break;
        case NQ_DTYPE_BF16:
            static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
            break;
        default:
            break;
    }
}

__host__ __device__ constexpr int64_t words_for(int64_t cols) { return (cols + 31) / 32; }

// Cache rows per block of the one-token decode attention's pass 1: the grain of
// its partial (max, sum, acc) results, which the merge and the O projection's
// attention input kind read.
constexpr int kAttnBlockRows = 64;

// e^x for the weights that merge attention blocks (x = a block's max minus the
// running max, <= 0 or -inf): the hardware base-2 exponential of x * log2(e).
// Every merge of block partials uses this one form, so they agree bit for bit.
__device__ __forceinline__ float merge_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

inline bool is_float_dtype(int d) {
    return d == NQ_DTYPE_F32 || d == NQ_DTYPE_F16 || d == NQ_DTYPE_BF16;
}

inline int dtype_bytes(int d) {
    switch (d) {
        case NQ_DTYPE_F32:
        case NQ_DTYPE_I32:
            return 4;
        case NQ_DTYPE_F16:
        case NQ_DTYPE_BF16:
            return 2;
        case NQ_DTYPE_I8:
            return 1;
        default:
            return 0;
    }
}

inline int launch_status() {
    return hipGetLastError() == hipSuccess ? NQ_OK : NQ_ERR_LAUNCH;
}

}  // namespace nq

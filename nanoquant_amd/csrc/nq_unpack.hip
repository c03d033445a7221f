// Bit-exact device unpack of llama.cpp-i32-lsb-v1 sign words and the device
// padding check (src/nanoquant/runtime/packed.py:189-218).
//
// One thread per output element keeps the dense stores coalesced; the word a
// thread reads is shared by 32 neighbours and comes from L2/L1.
#include "nq_common.h"

namespace {

template <typename OutT>
__device__ __forceinline__ OutT sign_value(uint32_t bit);

template <>
__device__ __forceinline__ float sign_value<float>(uint32_t bit) {
    return bit ? -1.0f : 1.0f;
}
template <>
__device__ __forceinline__ _Float16 sign_value<_Float16>(uint32_t bit) {
    return bit ? static_cast<_Float16>(-1.0f) : static_cast<_Float16>(1.0f);
}
// bf16 ±1 bit patterns: 0x3F80 / 0xBF80.
template <>
__device__ __forceinline__ uint16_t sign_value<uint16_t>(uint32_t bit) {
    return static_cast<uint16_t>(0x3F80u | (bit << 15));
}

template <typename OutT>
__global__ __launch_bounds__(256) void k_unpack_signs(const uint32_t* __restrict__ words,
                                                      int64_t rows, int64_t cols,
                                                      int64_t stride_words,
                                                      OutT* __restrict__ out) {
    const int64_t total = rows * cols;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = e / cols;
        const int64_t c = e - r * cols;
        const uint32_t w = words[r * stride_words + (c >> 5)];
        out[e] = sign_value<OutT>((w >> (c & 31)) & 1u);
    }
}

__global__ __launch_bounds__(256) void k_count_bad_padding(const uint32_t* __restrict__ words,
                                                           int64_t rows, int64_t last_word,
                                                           int64_t stride_words,
                                                           uint32_t pad_mask,
                                                           int32_t* __restrict__ bad_rows) {
    int count = 0;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; r < rows;
         r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        count += (words[r * stride_words + last_word] & pad_mask) != 0u;
    }
    // Wave-level sum, then one atomic per wave.
    for (int off = 32; off >= 1; off >>= 1) count += __shfl_xor(count, off);
    if ((threadIdx.x & 63) == 0 && count) atomicAdd(bad_rows, count);
}

__global__ void k_zero_i32(int32_t* p) { *p = 0; }

int grid_for(int64_t n) {
    const int64_t blocks = (n + 255) / 256;
    return static_cast<int>(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

}  // namespace

extern "C" int nq_unpack_signs(const int32_t* words, int64_t rows, int64_t cols,
                               int64_t row_stride_words, int32_t out_dtype, void* out,
                               void* stream) {
    if (!words || !out) return NQ_ERR_ARGUMENT;
    if (rows <= 0 || cols <= 0 || row_stride_words < nq::words_for(cols)) return NQ_ERR_SHAPE;
    const auto* w = reinterpret_cast<const uint32_t*>(words);
    auto s = static_cast<hipStream_t>(stream);
    const int grid = grid_for(rows * cols);
    switch (out_dtype) {
        case NQ_DTYPE_F32:
            hipLaunchKernelGGL(k_unpack_signs<float>, dim3(grid), dim3(256), 0, s, w, rows, cols,
                               row_stride_words, static_cast<float*>(out));
            break;
        case NQ_DTYPE_F16:
            hipLaunchKernelGGL(k_unpack_signs<_Float16>, dim3(grid), dim3(256), 0, s, w, rows,
                               cols, row_stride_words, static_cast<_Float16*>(out));
            break;
        case NQ_DTYPE_BF16:
            hipLaunchKernelGGL(k_unpack_signs<uint16_t>, dim3(grid), dim3(256), 0, s, w, rows,
                               cols, row_stride_words, static_cast<uint16_t*>(out));
            break;
        default:
            return NQ_ERR_DTYPE;
    }
    return nq::launch_status();
}

extern "C" int nq_count_bad_padding(const int32_t* words, int64_t rows, int64_t cols,
                                    int64_t row_stride_words, int32_t* bad_rows,
                                    void* stream) {
    if (!words || !bad_rows) return NQ_ERR_ARGUMENT;
    if (rows <= 0 || cols <= 0 || row_stride_words < nq::words_for(cols)) return NQ_ERR_SHAPE;
    auto s = static_cast<hipStream_t>(stream);
    // Zero with a kernel rather than a memset node so the call is capture-safe.
    hipLaunchKernelGGL(k_zero_i32, dim3(1), dim3(1), 0, s, bad_rows);
    const int tail = static_cast<int>(cols & 31);
    if (tail == 0) return nq::launch_status();
    const uint32_t pad_mask = ~((1u << tail) - 1u);
    hipLaunchKernelGGL(k_count_bad_padding, dim3(grid_for(rows)), dim3(256), 0, s,
                       reinterpret_cast<const uint32_t*>(words), rows, nq::words_for(cols) - 1,
                       row_stride_words, pad_mask, bad_rows);
    return nq::launch_status();
}

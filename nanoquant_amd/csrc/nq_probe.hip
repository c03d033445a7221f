// nq_read_stream: the HBM read ceiling the decode kernels are held against.
// It reads a buffer with the decode kernels' access pattern (16-byte
// nontemporal vector loads, four in flight per lane before any is used) and
// writes one XOR of the read words per workgroup, so the loads cannot be
// elided; nothing else is stored and nothing is atomic.
#include "nq_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void k_read_stream(const v4u* __restrict__ src, int64_t vectors,
                                                          uint32_t* __restrict__ sink) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    v4u acc = v4u{0u, 0u, 0u, 0u};
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; base < vectors;
         base += stride * kUnroll) {
        v4u v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + u * stride;
            v[u] = __builtin_nontemporal_load(src + (i < vectors ? i : vectors - 1));
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            if (base + u * stride < vectors) acc ^= v[u];
    }
    uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int off = 32; off >= 1; off >>= 1) x ^= __shfl_xor(x, off);
    __shared__ uint32_t waves[kThreads / 64];
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = waves[0] ^ waves[1] ^ waves[2] ^ waves[3];
}

}  // namespace

extern "C" int nq_read_stream(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_count, void* stream) {
    if (!src || !sink || bytes <= 0 || sink_count <= 0) return NQ_ERR_ARGUMENT;
    if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) & 15) != 0) return NQ_ERR_ALIGNMENT;
    const int64_t vectors = bytes / 16;
    // One round of kUnroll vectors per lane when the buffer allows, at most sink_count workgroups.
    int64_t blocks = (vectors + kThreads * kUnroll - 1) / (kThreads * kUnroll);
    blocks = blocks < sink_count ? blocks : sink_count;
    blocks = blocks < 65535 ? blocks : 65535;
    hipLaunchKernelGGL(k_read_stream, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const v4u*>(src), vectors, sink);
    return nq::launch_status();
}

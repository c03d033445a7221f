// Launcher of the fused (single-kernel) decode launch (instantiations of
// k_decode_fused; the kernels are documented in nq_decode_kernels.h).
#include "nq_decode_kernels.h"

namespace nqdec {
namespace {

template <int TPB, int TB, int KC1, int KC2>
int go(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    constexpr int kThreads = TPB == 1 ? threads_for(1, KC1 > KC2 ? KC1 : KC2) : 512;  // see plan_shapes
    if (64 * s.nw > kThreads) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL((k_decode_fused<TPB, TB, KC1, KC2, kThreads>), s.grid, dim3(64 * s.nw), s.lds, stream,
                       batch);
    return nq::launch_status();
}

template <int TPB>
int by_chunks(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.kc == 1) return s.kc2 == 1 ? go<TPB, 1, 1, 1>(batch, s, stream) : go<TPB, 1, 1, 2>(batch, s, stream);
    return s.kc2 == 1 ? go<TPB, 1, 2, 1>(batch, s, stream) : go<TPB, 1, 2, 2>(batch, s, stream);
}

}  // namespace

int enqueue_fused(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tpb == 1) return by_chunks<1>(batch, s, stream);
    if (s.tb == 1) return by_chunks<4>(batch, s, stream);
    return go<4, 4, 1, 1>(batch, s, stream);
}

}  // namespace nqdec

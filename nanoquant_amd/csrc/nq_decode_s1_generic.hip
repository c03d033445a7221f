// Launcher of the split decode stage-1 kernel for any float x and scales (instantiations of
// k_decode_stage1<kActGeneric, ...>; the kernels are documented in
// nq_decode_kernels.h). One translation unit per activation kind keeps the
// library build parallel.
#include "nq_decode_kernels.h"

namespace nqdec {
namespace {

template <int TPB, int TB, int TW, int KC>
int go(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    constexpr int kThreads = threads_for(TPB, KC);
    if (64 * s.nw > kThreads) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL((k_decode_stage1<kActGeneric, TPB, TB, TW, KC, kThreads>), s.grid, dim3(64 * s.nw), s.lds, stream,
                       batch);
    return nq::launch_status();
}

template <int TPB>
int by_tiles(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tw == 4) return s.kc == 2 ? go<TPB, 1, 4, 2>(batch, s, stream) : go<TPB, 1, 4, 1>(batch, s, stream);
    if (s.tw == 2) return s.kc == 2 ? go<TPB, 1, 2, 2>(batch, s, stream) : go<TPB, 1, 2, 1>(batch, s, stream);
    if (s.tw == 3) return s.kc == 2 ? go<TPB, 1, 3, 2>(batch, s, stream) : go<TPB, 1, 3, 1>(batch, s, stream);
    return s.kc == 2 ? go<TPB, 1, 1, 2>(batch, s, stream) : go<TPB, 1, 1, 1>(batch, s, stream);
}

}  // namespace

int enqueue_stage1_generic(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tpb == 1) return by_tiles<1>(batch, s, stream);
    // Two to four tokens stage in the kernel; more take stage 0 + k_decode_stage1m (nq_decode_multi.hip).
    if (s.tb == 1) return by_tiles<4>(batch, s, stream);
    return NQ_ERR_UNSUPPORTED;
}

}  // namespace nqdec

// Launcher of the split decode stage-2 kernel (instantiations of
// k_decode_stage2; the kernels are documented in nq_decode_kernels.h).
#include "nq_decode_kernels.h"

namespace nqdec {
namespace {

template <int TPB, int TB, int TW, int KC>
int go(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    constexpr int kThreads = threads_for(TPB, KC, TB);
    if (64 * s.nw > kThreads) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL((k_decode_stage2<TPB, TB, TW, KC, kThreads>), s.grid, dim3(64 * s.nw), s.lds, stream, batch);
    return nq::launch_status();
}

template <int TPB>
int by_tiles(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tw == 4) return s.kc == 2 ? go<TPB, 1, 4, 2>(batch, s, stream) : go<TPB, 1, 4, 1>(batch, s, stream);
    if (s.tw == 2) return s.kc == 2 ? go<TPB, 1, 2, 2>(batch, s, stream) : go<TPB, 1, 2, 1>(batch, s, stream);
    if (s.tw == 3) return s.kc == 2 ? go<TPB, 1, 3, 2>(batch, s, stream) : go<TPB, 1, 3, 1>(batch, s, stream);
    return s.kc == 2 ? go<TPB, 1, 1, 2>(batch, s, stream) : go<TPB, 1, 1, 1>(batch, s, stream);
}

// Several token blocks (five tokens or more): one chunk per wave per pass.
template <int TB>
int by_tiles_blocks(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.kc != 1) return NQ_ERR_LAUNCH;
    if (s.tw == 4) return go<4, TB, 4, 1>(batch, s, stream);
    if (s.tw == 2) return go<4, TB, 2, 1>(batch, s, stream);
    return go<4, TB, 1, 1>(batch, s, stream);
}

template <int TW, int KC>
int go_pair(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    constexpr int kThreads = threads_for(1, KC);
    if (64 * s.nw > kThreads) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL((k_decode_stage2_pair<TW, KC, kThreads>), s.grid, dim3(64 * s.nw), s.lds, stream, batch);
    return nq::launch_status();
}

}  // namespace

int enqueue_stage2_pair(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tw == 4) return s.kc == 2 ? go_pair<4, 2>(batch, s, stream) : go_pair<4, 1>(batch, s, stream);
    if (s.tw == 3) return s.kc == 2 ? go_pair<3, 2>(batch, s, stream) : go_pair<3, 1>(batch, s, stream);
    if (s.tw == 2) return s.kc == 2 ? go_pair<2, 2>(batch, s, stream) : go_pair<2, 1>(batch, s, stream);
    return s.kc == 2 ? go_pair<1, 2>(batch, s, stream) : go_pair<1, 1>(batch, s, stream);
}

int enqueue_stage2(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tpb == 1) return by_tiles<1>(batch, s, stream);
    if (s.tb == 1) return by_tiles<4>(batch, s, stream);
    if (s.tb == 2) return by_tiles_blocks<2>(batch, s, stream);
    return by_tiles_blocks<4>(batch, s, stream);
}

}  // namespace nqdec

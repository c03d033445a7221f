// Launchers of the several-token decode path (split launch, 2-16 tokens):
// k_decode_stage0 and k_decode_stage1m, documented in nq_decode_kernels.h.
#include "nq_decode_kernels.h"

namespace nqdec {
namespace {

template <int AK>
int go0(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    hipLaunchKernelGGL((k_decode_stage0<AK>), s.grid, dim3(256), 0, stream, batch);
    return nq::launch_status();
}

template <int TB, int TW, int KC>
int go1(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    constexpr int kThreads = 512;
    if (64 * s.nw > kThreads) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL((k_decode_stage1m<TB, TW, KC, kThreads>), s.grid, dim3(64 * s.nw), s.lds, stream, batch);
    return nq::launch_status();
}

template <int TB, int KC>
int by_tiles(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    switch (s.tw) {
        case 1: return go1<TB, 1, KC>(batch, s, stream);
        case 2: return go1<TB, 2, KC>(batch, s, stream);
        case 4: return go1<TB, 4, KC>(batch, s, stream);
        default: return NQ_ERR_LAUNCH;
    }
}

}  // namespace

int enqueue_stage0(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    switch (s.ak) {
        case kActBf16: return go0<kActBf16>(batch, s, stream);
        case kActF16: return go0<kActF16>(batch, s, stream);
        case kActF32: return go0<kActF32>(batch, s, stream);
        case kActGeneric: return go0<kActGeneric>(batch, s, stream);
        default: return NQ_ERR_UNSUPPORTED;
    }
}

int enqueue_stage1m(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tpb != 4) return NQ_ERR_LAUNCH;
    if (s.tb == 1) return s.kc == 2 ? by_tiles<1, 2>(batch, s, stream) : by_tiles<1, 1>(batch, s, stream);
    if (s.kc != 1) return NQ_ERR_LAUNCH;  // two token blocks per wave: one chunk per pass
    if (s.tb == 2) return by_tiles<2, 1>(batch, s, stream);
    if (s.tb == 4) return by_tiles<4, 1>(batch, s, stream);
    return NQ_ERR_LAUNCH;
}

}  // namespace nqdec

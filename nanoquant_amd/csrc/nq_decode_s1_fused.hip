// Launcher of the split decode stage-1 kernel for the decoder's fused inputs
// (one token): the RMSNorm-folded fp32 residual (k_decode_stage1<kActNormF32,
// ...>) and the SiLU-gated fp32 gate/up pair (k_decode_stage1<kActGatedF32,
// ...>). The kernels are documented in nq_decode_kernels.h.
#include "nq_decode_kernels.h"

namespace nqdec {
namespace {

template <int AK, int TW, int KC>
int go(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    constexpr int kThreads = threads_for(1, KC);
    if (64 * s.nw > kThreads) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL((k_decode_stage1<AK, 1, 1, TW, KC, kThreads>), s.grid, dim3(64 * s.nw), s.lds, stream, batch);
    return nq::launch_status();
}

template <int AK>
int by_tiles(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tw == 4) return s.kc == 2 ? go<AK, 4, 2>(batch, s, stream) : go<AK, 4, 1>(batch, s, stream);
    if (s.tw == 3) return s.kc == 2 ? go<AK, 3, 2>(batch, s, stream) : go<AK, 3, 1>(batch, s, stream);
    if (s.tw == 2) return s.kc == 2 ? go<AK, 2, 2>(batch, s, stream) : go<AK, 2, 1>(batch, s, stream);
    return s.kc == 2 ? go<AK, 1, 2>(batch, s, stream) : go<AK, 1, 1>(batch, s, stream);
}

}  // namespace

int enqueue_stage1_fused(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tpb != 1 || s.tb != 1) return NQ_ERR_UNSUPPORTED;
    return s.ak == kActNormF32 ? by_tiles<kActNormF32>(batch, s, stream) : by_tiles<kActGatedF32>(batch, s, stream);
}

}  // namespace nqdec

// Launcher of the split decode stage-1 kernel for the decoder's fused inputs
// (one token): the RMSNorm-folded fp32 residual (k_decode_stage1<kActNormF32,
// ...>), the SiLU-gated fp32 gate/up pair (k_decode_stage1<kActGatedF32,
// ...>) and the attention output merged from pass-1 partials
// (k_decode_stage1<kActAttn8 ... kActAttn16E, ...>). The kernels are documented
// in nq_decode_kernels.h.
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

// Attention kinds: one chunk per wave and at most eight waves, so the launch
// bound of 512 threads leaves room for every block's partials in registers.
template <int AK, int TW>
int go_attn(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.kc != 1 || 64 * s.nw > 512) return NQ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((k_decode_stage1<AK, 1, 1, TW, 1, 512>), s.grid, dim3(64 * s.nw), s.lds, stream, batch);
    return nq::launch_status();
}

template <int AK>
int attn_by_tiles(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tw == 1) return go_attn<AK, 1>(batch, s, stream);
    if (s.tw == 2) return go_attn<AK, 2>(batch, s, stream);
    return NQ_ERR_UNSUPPORTED;
}

}  // namespace

int enqueue_stage1_fused(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    if (s.tpb != 1 || s.tb != 1) return NQ_ERR_UNSUPPORTED;
    switch (s.ak) {
        case kActNormF32: return by_tiles<kActNormF32>(batch, s, stream);
        case kActGatedF32: return by_tiles<kActGatedF32>(batch, s, stream);
        case kActAttn8: return attn_by_tiles<kActAttn8>(batch, s, stream);
        case kActAttn12: return attn_by_tiles<kActAttn12>(batch, s, stream);
        case kActAttn8E: return attn_by_tiles<kActAttn8E>(batch, s, stream);
        case kActAttn12E: return attn_by_tiles<kActAttn12E>(batch, s, stream);
        case kActAttn16E: return attn_by_tiles<kActAttn16E>(batch, s, stream);
        case kActAttn16: return attn_by_tiles<kActAttn16>(batch, s, stream);
        default: return NQ_ERR_UNSUPPORTED;
    }
}

}  // namespace nqdec

// Tiled-layout decode path. Placeholder until the MFMA decode kernel lands:
// no tiled layout is produced, so nq_linear always takes the general path.
#include "nq_decode.h"

namespace nq {

int64_t decode_scratch_bytes(const nq_linear_desc*, int64_t) { return 0; }

bool decode_path_applies(const nq_linear_desc*, int64_t) { return false; }

int launch_decode(const nq_linear_desc*, const void*, int, int64_t, void*, int, void*, hipStream_t) {
    return NQ_ERR_UNSUPPORTED;
}

}  // namespace nq

extern "C" int64_t nq_tiles_bytes(int64_t, int64_t, int64_t) { return 0; }

extern "C" int nq_prepare_tiles(const nq_linear_desc*, void*, int64_t, void*) {
    return NQ_ERR_UNSUPPORTED;
}

// Tiled-layout decode path (token counts the fused MFMA kernel covers).
#pragma once

#include "nq_common.h"

namespace nq {

// Words of the sync header in front of the V tiles in a tiles buffer.
int64_t tiles_header_words();

// Word index, within that header, of max|s_mid| (fp32 bits, written by nq_prepare_tiles).
int64_t tiles_max_mid_word();

// Extra workspace bytes the tiled decode path needs for `tokens` slots.
int64_t decode_scratch_bytes(const nq_linear_desc* d, int64_t tokens);

// True when desc->tiles is set and the tiled decode kernel handles `tokens`.
bool decode_path_applies(const nq_linear_desc* d, int64_t tokens);

// Launch the tiled decode path; scratch is decode_scratch_bytes(d, tokens) bytes.
int launch_decode(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y,
                  int y_dtype, void* scratch, hipStream_t stream);

// One launch for `count` (1..8) linears sharing the token count and dtypes.
// `fusion` (NULL for none) adds the decoder fusions of nq_linear_batch_fused.
int launch_decode_batch(const nq_linear_desc* const* descs, int count, const void* const* xs, int x_dtype,
                        int64_t tokens, void* const* ys, int y_dtype, void* const* scratch,
                        hipStream_t stream, const nq_decode_fusion* fusion = nullptr);

}  // namespace nq

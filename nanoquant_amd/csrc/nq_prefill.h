// Prefill path (token counts above the decode kernel's 16) on the tile layout.
#pragma once

#include "nq_common.h"
#include "nq_decode.h"

namespace nq {

// Workspace bytes the prefill path needs for `tokens` slots.
int64_t prefill_scratch_bytes(const nq_linear_desc* d, int64_t tokens);

// True when desc->tiles is set and tokens exceed the decode kernel's range.
bool prefill_path_applies(const nq_linear_desc* d, int64_t tokens);

// Launch prep -> GEMM(V) -> GEMM(U); scratch is prefill_scratch_bytes bytes.
int launch_prefill(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y, int y_dtype,
                   void* scratch, hipStream_t stream);

}  // namespace nq

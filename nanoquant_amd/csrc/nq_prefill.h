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

// The same for 1..8 linears with one token count: one launch per phase (row
// passes, GEMM 1, its reductions, GEMM 2, its reductions) for all members;
// scratch[i] is prefill_scratch_bytes(descs[i], tokens) bytes.
int launch_prefill_batch(const nq_linear_desc* const* descs, int count, const void* const* xs, int x_dtype,
                         int64_t tokens, void* const* ys, int y_dtype, void* const* scratch, hipStream_t stream);

}  // namespace nq

// Packed binary low-rank linear: the general (any token count, canonical word
// layout) HIP path and the nq_linear entry point.
//
// Math (src/nanoquant/runtime/reference.py:208-235; the two-stage split of
// src/nanoquant/runtime/cuda_kernels.py:65-162):
//   stage 1: lm[t, r]  = s_mid[r] * Σ_i sgn(V[r, i]) * x[t, i] * s_in[i]
//   stage 2: y[t, o]   = s_out[o] * Σ_r sgn(U[o, r]) * lm[t, r]
//                        + Σ_k x[t, idx_k] * W_sal[o, k] (* scale_k) + bias[o]
//   then     y        += patch_left · (patch_right · x)      (float patch)
//            y[:, ri] += row_scale_i * (Q_i · x)             (int8 output rows)
//
// Both stages are the same "binary rows" product: each output row is a sign
// row of the packed matrix dotted with an fp32 activation vector. A 256-thread
// block owns 16 sign rows (four 16-lane groups per wave); the activation is
// staged in LDS 512 columns at a time as [token][bit][word-slot] so the 16
// lanes of a group read 16 consecutive floats (no bank conflicts) and the
// four groups of a wave read the same addresses (broadcast).
#include "nq_common.h"
#include "nq_decode.h"
#include "nq_prefill.h"

namespace {

constexpr int kBlock = 256;
constexpr int kChunkWords = 16;
constexpr int kChunkCols = kChunkWords * 32;
constexpr int kRowsPerBlock = 16;

// Activation a(t, k) = a0[t * ld + k] * (a1 ? a1[k] : 1).
struct ActSource {
    const void* a0;
    int a0_dtype;
    const void* a1;
    int a1_dtype;
    int64_t ld;
    int64_t cols;
};

__device__ __forceinline__ float act_value(const ActSource& a, int64_t t, int64_t k) {
    float v = nq::load_f32(a.a0, a.a0_dtype, t * a.ld + k);
    if (a.a1) v *= nq::load_f32(a.a1, a.a1_dtype, k);
    return v;
}

// Stage-2 extras applied by the lane that owns (t, row).
struct Epilogue {
    const void* x;             // raw input for the salient gather
    int x_dtype;
    int64_t in_features;
    int64_t salient_count;
    const int32_t* salient_indices;
    const void* salient_values;  // [rows, k]
    int salient_dtype;
    const void* salient_scales;  // [k] or null
    int scale_dtype;
    const void* bias;
    int bias_dtype;
};

struct BinaryRowsArgs {
    const uint32_t* words;  // [rows, wpr]
    int64_t rows;
    int64_t wpr;
    ActSource act;
    int64_t tokens;
    const void* row_scale;
    int row_scale_dtype;
    void* out;  // [tokens, rows]
    int out_dtype;
    Epilogue ep;
};

template <int MT>
__global__ __launch_bounds__(kBlock) void k_binary_rows(const BinaryRowsArgs args) {
    __shared__ float act[MT][32][kChunkWords];

    const int lane = threadIdx.x & 63;
    const int group = lane >> 4;
    const int slot = lane & 15;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock +
                        (threadIdx.x >> 6) * 4 + group;
    const int64_t t0 = static_cast<int64_t>(blockIdx.y) * MT;
    const bool row_ok = row < args.rows;

    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;

    for (int64_t w0 = 0; w0 < args.wpr; w0 += kChunkWords) {
        __syncthreads();
        for (int e = threadIdx.x; e < MT * kChunkCols; e += kBlock) {
            const int t = e / kChunkCols;
            const int c = e - t * kChunkCols;
            const int64_t k = w0 * 32 + c;
            float v = 0.0f;
            if (t0 + t < args.tokens && k < args.act.cols) v = act_value(args.act, t0 + t, k);
            act[t][c & 31][c >> 5] = v;
        }
        __syncthreads();
        const int64_t w = w0 + slot;
        if (row_ok && w < args.wpr) {
            const uint32_t bits = args.words[row * args.wpr + w];
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const uint32_t sign = (bits << (31 - j)) & 0x80000000u;
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    acc[t] += __uint_as_float(__float_as_uint(act[t][j][slot]) ^ sign);
                }
            }
        }
    }

#pragma unroll
    for (int t = 0; t < MT; ++t) {
        for (int off = 8; off >= 1; off >>= 1) acc[t] += __shfl_xor(acc[t], off, 16);
    }

    // Salient columns: lanes of the group split the k columns, then reduce.
    float sal[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) sal[t] = 0.0f;
    const Epilogue& ep = args.ep;
    if (ep.salient_count > 0 && row_ok) {
        for (int64_t s = slot; s < ep.salient_count; s += 16) {
            float wv = nq::load_f32(ep.salient_values, ep.salient_dtype, row * ep.salient_count + s);
            if (ep.salient_scales) wv *= nq::load_f32(ep.salient_scales, ep.scale_dtype, s);
            const int64_t col = ep.salient_indices[s];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (t0 + t < args.tokens) {
                    sal[t] += wv * nq::load_f32(ep.x, ep.x_dtype, (t0 + t) * ep.in_features + col);
                }
            }
        }
    }
    if (ep.salient_count > 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            for (int off = 8; off >= 1; off >>= 1) sal[t] += __shfl_xor(sal[t], off, 16);
        }
    }

    if (!row_ok || slot >= MT || t0 + slot >= args.tokens) return;
    float total = 0.0f;
    float extra = 0.0f;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        if (t == slot) {
            total = acc[t];
            extra = sal[t];
        }
    }
    float value = total * nq::load_f32(args.row_scale, args.row_scale_dtype, row) + extra;
    if (ep.bias) value += nq::load_f32(ep.bias, ep.bias_dtype, row);
    nq::store_f32_as(args.out, args.out_dtype, (t0 + slot) * args.rows + row, value);
}

// Dense rows: out[t, dst(r)] (+)= rscale(r) * Σ_k W[r, k] * act(t, k); one wave per row.
struct DenseRowsArgs {
    const void* w;
    int w_dtype;
    int64_t rows;
    ActSource act;  // act.cols = K
    int64_t tokens;
    const void* row_scale;  // optional
    int row_scale_dtype;
    const int32_t* dst_rows;  // optional scatter
    float* out;
    int64_t out_ld;
    int accumulate;
};

template <int MT>
__global__ __launch_bounds__(kBlock) void k_dense_rows(const DenseRowsArgs args) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
    const int64_t t0 = static_cast<int64_t>(blockIdx.y) * MT;
    if (row >= args.rows) return;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (int64_t k = lane; k < args.act.cols; k += 64) {
        const float wv = nq::load_f32(args.w, args.w_dtype, row * args.act.cols + k);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t0 + t < args.tokens) acc[t] += wv * act_value(args.act, t0 + t, k);
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        for (int off = 32; off >= 1; off >>= 1) acc[t] += __shfl_xor(acc[t], off);
    }
    if (lane >= MT || t0 + lane >= args.tokens) return;
    float v = 0.0f;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        if (t == lane) v = acc[t];
    }
    if (args.row_scale) v *= nq::load_f32(args.row_scale, args.row_scale_dtype, row);
    const int64_t dst = args.dst_rows ? args.dst_rows[row] : row;
    float* cell = args.out + (t0 + lane) * args.out_ld + dst;
    *cell = args.accumulate ? *cell + v : v;
}

// Output-row sidecar, vector form: out[t, dst[r]] += scale[r] * Σ_k Q[r, k] * x[t, k]
// for int8 rows Q [rows, K] with K % 16 == 0 and 16-byte aligned Q and x rows.
// One workgroup per (row, token group); each thread takes 16 consecutive
// columns per step (one 16-byte load of Q, one or more of x per token), all
// loads of a step issued before use; the four waves' sums are added in wave
// order, so the result does not depend on timing.
constexpr int kRowSteps = 4;  // 16-byte Q loads in flight per thread

template <int MT, int XDT>
__global__ __launch_bounds__(kBlock) void k_row_sidecar(const int8_t* __restrict__ q, int64_t cols,
                                                         const void* __restrict__ x, int64_t tokens,
                                                         const void* __restrict__ scale, int scale_dtype,
                                                         const int32_t* __restrict__ dst, float* __restrict__ out,
                                                         int64_t out_ld) {
    __shared__ float part[kBlock / 64][MT];
    const int64_t row = blockIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.y) * MT;
    const int64_t vecs = cols / 16;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (int64_t v0 = threadIdx.x; v0 < vecs; v0 += kBlock * kRowSteps) {
        int4 qv[kRowSteps];
#pragma unroll
        for (int s = 0; s < kRowSteps; ++s) {
            const int64_t v = v0 + s * kBlock;
            qv[s] = reinterpret_cast<const int4*>(q + row * cols)[v < vecs ? v : vecs - 1];
        }
#pragma unroll
        for (int s = 0; s < kRowSteps; ++s) {
            const int64_t v = v0 + s * kBlock;
            if (v >= vecs) break;
            float w[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t d = static_cast<uint32_t>(reinterpret_cast<const int*>(&qv[s])[i]);
#pragma unroll
                for (int b = 0; b < 4; ++b) w[4 * i + b] = static_cast<float>(static_cast<int8_t>(d >> (8 * b)));
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int64_t tt = t0 + t < tokens ? t0 + t : tokens - 1;
                float xv[16];
                if constexpr (XDT == NQ_DTYPE_F32) {
                    const float4* xp = reinterpret_cast<const float4*>(static_cast<const float*>(x) + tt * cols) + 4 * v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float4 f = xp[i];
                        xv[4 * i] = f.x; xv[4 * i + 1] = f.y; xv[4 * i + 2] = f.z; xv[4 * i + 3] = f.w;
                    }
                } else {
                    const uint4* xp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + tt * cols) + 2 * v;
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint4 h = xp[i];
                        const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            if constexpr (XDT == NQ_DTYPE_BF16) {
                                xv[8 * i + 2 * j] = __uint_as_float(hw[j] << 16);
                                xv[8 * i + 2 * j + 1] = __uint_as_float(hw[j] & 0xffff0000u);
                            } else {
                                xv[8 * i + 2 * j] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hw[j])));
                                xv[8 * i + 2 * j + 1] =
                                    static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hw[j] >> 16)));
                            }
                        }
                    }
                }
                float sum = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) sum += w[i] * xv[i];
                acc[t] += sum;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
        for (int off = 32; off >= 1; off >>= 1) acc[t] += __shfl_xor(acc[t], off);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) part[threadIdx.x >> 6][t] = acc[t];
    }
    __syncthreads();
    if (threadIdx.x < MT && t0 + threadIdx.x < tokens) {
        const int t = threadIdx.x;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) v += part[w][t];
        v *= nq::load_f32(scale, scale_dtype, row);
        float* cell = out + (t0 + t) * out_ld + dst[row];
        *cell += v;
    }
}

template <int XDT>
int launch_row_sidecar_x(int mt, dim3 grid, hipStream_t s, const int8_t* q, int64_t cols, const void* x,
                         int64_t tokens, const void* scale, int scale_dtype, const int32_t* dst, float* out,
                         int64_t out_ld) {
    switch (mt) {
        case 1: hipLaunchKernelGGL((k_row_sidecar<1, XDT>), grid, dim3(kBlock), 0, s, q, cols, x, tokens, scale, scale_dtype, dst, out, out_ld); break;
        case 2: hipLaunchKernelGGL((k_row_sidecar<2, XDT>), grid, dim3(kBlock), 0, s, q, cols, x, tokens, scale, scale_dtype, dst, out, out_ld); break;
        case 4: hipLaunchKernelGGL((k_row_sidecar<4, XDT>), grid, dim3(kBlock), 0, s, q, cols, x, tokens, scale, scale_dtype, dst, out, out_ld); break;
        default: hipLaunchKernelGGL((k_row_sidecar<8, XDT>), grid, dim3(kBlock), 0, s, q, cols, x, tokens, scale, scale_dtype, dst, out, out_ld); break;
    }
    return nq::launch_status();
}

// The vector row-sidecar kernel when the shapes allow it, else -1.
int launch_row_sidecar(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, float* y, hipStream_t s) {
    const int64_t cols = d->in_features;
    const bool ok = cols % 16 == 0 && (reinterpret_cast<uintptr_t>(d->row_values) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(x) & 15) == 0 && nq::is_float_dtype(x_dtype);
    if (!ok) return -1;
    const int mt = tokens <= 1 ? 1 : (tokens <= 2 ? 2 : (tokens <= 4 ? 4 : 8));
    const dim3 grid(static_cast<unsigned>(d->row_count), static_cast<unsigned>((tokens + mt - 1) / mt));
    switch (x_dtype) {
        case NQ_DTYPE_F32:
            return launch_row_sidecar_x<NQ_DTYPE_F32>(mt, grid, s, d->row_values, cols, x, tokens, d->row_scales,
                                                      d->scale_dtype, d->row_indices, y, d->out_features);
        case NQ_DTYPE_F16:
            return launch_row_sidecar_x<NQ_DTYPE_F16>(mt, grid, s, d->row_values, cols, x, tokens, d->row_scales,
                                                      d->scale_dtype, d->row_indices, y, d->out_features);
        default:
            return launch_row_sidecar_x<NQ_DTYPE_BF16>(mt, grid, s, d->row_values, cols, x, tokens, d->row_scales,
                                                       d->scale_dtype, d->row_indices, y, d->out_features);
    }
}

int tokens_tile(int64_t tokens) {
    if (tokens <= 1) return 1;
    if (tokens <= 2) return 2;
    if (tokens <= 4) return 4;
    if (tokens <= 8) return 8;
    return 16;
}

int launch_binary_rows(const BinaryRowsArgs& a, hipStream_t s) {
    const int mt = tokens_tile(a.tokens);
    const dim3 grid(static_cast<unsigned>((a.rows + kRowsPerBlock - 1) / kRowsPerBlock),
                    static_cast<unsigned>((a.tokens + mt - 1) / mt));
    switch (mt) {
        case 1: hipLaunchKernelGGL(k_binary_rows<1>, grid, dim3(kBlock), 0, s, a); break;
        case 2: hipLaunchKernelGGL(k_binary_rows<2>, grid, dim3(kBlock), 0, s, a); break;
        case 4: hipLaunchKernelGGL(k_binary_rows<4>, grid, dim3(kBlock), 0, s, a); break;
        case 8: hipLaunchKernelGGL(k_binary_rows<8>, grid, dim3(kBlock), 0, s, a); break;
        default: hipLaunchKernelGGL(k_binary_rows<16>, grid, dim3(kBlock), 0, s, a); break;
    }
    return nq::launch_status();
}

int launch_dense_rows(const DenseRowsArgs& a, hipStream_t s) {
    const int mt = tokens_tile(a.tokens);
    const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4),
                    static_cast<unsigned>((a.tokens + mt - 1) / mt));
    switch (mt) {
        case 1: hipLaunchKernelGGL(k_dense_rows<1>, grid, dim3(kBlock), 0, s, a); break;
        case 2: hipLaunchKernelGGL(k_dense_rows<2>, grid, dim3(kBlock), 0, s, a); break;
        case 4: hipLaunchKernelGGL(k_dense_rows<4>, grid, dim3(kBlock), 0, s, a); break;
        case 8: hipLaunchKernelGGL(k_dense_rows<8>, grid, dim3(kBlock), 0, s, a); break;
        default: hipLaunchKernelGGL(k_dense_rows<16>, grid, dim3(kBlock), 0, s, a); break;
    }
    return nq::launch_status();
}

int64_t align256(int64_t n) { return (n + 255) & ~static_cast<int64_t>(255); }

int validate(const nq_linear_desc* d) {
    if (!d) return NQ_ERR_ARGUMENT;
    if (d->in_features <= 0 || d->out_features <= 0 || d->rank <= 0) return NQ_ERR_SHAPE;
    if (!d->right_words || !d->left_words || !d->scale_pre || !d->scale_mid || !d->scale_post)
        return NQ_ERR_ARGUMENT;
    if (!nq::is_float_dtype(d->scale_dtype)) return NQ_ERR_DTYPE;
    if (d->bias && !nq::is_float_dtype(d->bias_dtype)) return NQ_ERR_DTYPE;
    if (d->salient_count < 0 || d->salient_count > d->in_features) return NQ_ERR_SHAPE;
    if (d->salient_count > 0) {
        if (!d->salient_indices || !d->salient_values) return NQ_ERR_ARGUMENT;
        if (!nq::is_float_dtype(d->salient_dtype) && d->salient_dtype != NQ_DTYPE_I8)
            return NQ_ERR_DTYPE;
        if ((d->salient_dtype == NQ_DTYPE_I8) != (d->salient_scales != nullptr))
            return NQ_ERR_ARGUMENT;
    }
    if (d->patch_rank < 0) return NQ_ERR_SHAPE;
    if (d->patch_rank > 0) {
        if (!d->patch_left || !d->patch_right) return NQ_ERR_ARGUMENT;
        if (!nq::is_float_dtype(d->patch_dtype)) return NQ_ERR_DTYPE;
    }
    if (d->row_count < 0 || d->row_count > d->out_features) return NQ_ERR_SHAPE;
    if (d->row_count > 0 && (!d->row_indices || !d->row_values || !d->row_scales))
        return NQ_ERR_ARGUMENT;
    if (d->decode_launch != NQ_DECODE_SPLIT && d->decode_launch != NQ_DECODE_FUSED) return NQ_ERR_ARGUMENT;
    if (d->prefill_operands != NQ_PREFILL_FP16 && d->prefill_operands != NQ_PREFILL_FP16_SPLIT) return NQ_ERR_ARGUMENT;
    return NQ_OK;
}

// Workspace carve-up: [lm: tokens*rank f32][patch tmp: tokens*p f32][decode scratch].
struct WorkspaceLayout {
    int64_t lm_offset, patch_offset, decode_offset, total;
};

WorkspaceLayout workspace_layout(const nq_linear_desc* d, int64_t tokens) {
    WorkspaceLayout w{};
    w.lm_offset = 0;
    w.patch_offset = align256(tokens * d->rank * 4);
    w.decode_offset = w.patch_offset + align256(tokens * d->patch_rank * 4);
    const int64_t tiled = nq::decode_path_applies(d, tokens) ? nq::decode_scratch_bytes(d, tokens)
                                                             : nq::prefill_scratch_bytes(d, tokens);
    w.total = w.decode_offset + tiled;
    return w;
}

// Float patch and output-row sidecar, accumulated into fp32 y after stage 2.
int apply_extras(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y, char* patch_ws,
                 hipStream_t s) {
    int st = NQ_OK;
    if (d->patch_rank > 0) {
        float* tmp = reinterpret_cast<float*>(patch_ws);
        DenseRowsArgs p1{};
        p1.w = d->patch_right;
        p1.w_dtype = d->patch_dtype;
        p1.rows = d->patch_rank;
        p1.act = ActSource{x, x_dtype, nullptr, 0, d->in_features, d->in_features};
        p1.tokens = tokens;
        p1.out = tmp;
        p1.out_ld = d->patch_rank;
        st = launch_dense_rows(p1, s);
        if (st != NQ_OK) return st;
        DenseRowsArgs p2{};
        p2.w = d->patch_left;
        p2.w_dtype = d->patch_dtype;
        p2.rows = d->out_features;
        p2.act = ActSource{tmp, NQ_DTYPE_F32, nullptr, 0, d->patch_rank, d->patch_rank};
        p2.tokens = tokens;
        p2.out = static_cast<float*>(y);
        p2.out_ld = d->out_features;
        p2.accumulate = 1;
        st = launch_dense_rows(p2, s);
        if (st != NQ_OK) return st;
    }
    if (d->row_count > 0) {
        st = launch_row_sidecar(d, x, x_dtype, tokens, static_cast<float*>(y), s);
        if (st >= 0) return st;
        DenseRowsArgs r{};
        r.w = d->row_values;
        r.w_dtype = NQ_DTYPE_I8;
        r.rows = d->row_count;
        r.act = ActSource{x, x_dtype, nullptr, 0, d->in_features, d->in_features};
        r.tokens = tokens;
        r.row_scale = d->row_scales;
        r.row_scale_dtype = d->scale_dtype;
        r.dst_rows = d->row_indices;
        r.out = static_cast<float*>(y);
        r.out_ld = d->out_features;
        r.accumulate = 1;
        st = launch_dense_rows(r, s);
        if (st != NQ_OK) return st;
    }
    return NQ_OK;
}

}  // namespace

extern "C" int64_t nq_linear_workspace_bytes(const nq_linear_desc* desc, int64_t tokens) {
    if (validate(desc) != NQ_OK || tokens <= 0) return -1;
    return workspace_layout(desc, tokens).total;
}

extern "C" int nq_linear(const nq_linear_desc* d, const void* x, int32_t x_dtype, int64_t tokens,
                         void* y, int32_t y_dtype, void* workspace, int64_t workspace_bytes,
                         void* stream) {
    int st = validate(d);
    if (st != NQ_OK) return st;
    if (!x || !y) return NQ_ERR_ARGUMENT;
    if (tokens <= 0) return NQ_ERR_SHAPE;
    if (!nq::is_float_dtype(x_dtype) || !nq::is_float_dtype(y_dtype)) return NQ_ERR_DTYPE;
    // Patch and row sidecar accumulate into y after stage 2; keep that in fp32.
    if (y_dtype != NQ_DTYPE_F32 && (d->patch_rank > 0 || d->row_count > 0)) return NQ_ERR_UNSUPPORTED;
    const WorkspaceLayout wl = workspace_layout(d, tokens);
    if (!workspace || workspace_bytes < wl.total) return NQ_ERR_WORKSPACE;
    auto s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);

    if (d->tiles && nq::decode_path_applies(d, tokens)) {
        st = nq::launch_decode(d, x, x_dtype, tokens, y, y_dtype, ws + wl.decode_offset, s);
        if (st != NQ_OK) return st;
    } else if (nq::prefill_path_applies(d, tokens)) {
        st = nq::launch_prefill(d, x, x_dtype, tokens, y, y_dtype, ws + wl.decode_offset, s);
        if (st != NQ_OK) return st;
    } else {
        float* lm = reinterpret_cast<float*>(ws + wl.lm_offset);
        BinaryRowsArgs s1{};
        s1.words = reinterpret_cast<const uint32_t*>(d->right_words);
        s1.rows = d->rank;
        s1.wpr = nq::words_for(d->in_features);
        s1.act = ActSource{x, x_dtype, d->scale_pre, d->scale_dtype, d->in_features, d->in_features};
        s1.tokens = tokens;
        s1.row_scale = d->scale_mid;
        s1.row_scale_dtype = d->scale_dtype;
        s1.out = lm;
        s1.out_dtype = NQ_DTYPE_F32;
        st = launch_binary_rows(s1, s);
        if (st != NQ_OK) return st;

        BinaryRowsArgs s2{};
        s2.words = reinterpret_cast<const uint32_t*>(d->left_words);
        s2.rows = d->out_features;
        s2.wpr = nq::words_for(d->rank);
        s2.act = ActSource{lm, NQ_DTYPE_F32, nullptr, 0, d->rank, d->rank};
        s2.tokens = tokens;
        s2.row_scale = d->scale_post;
        s2.row_scale_dtype = d->scale_dtype;
        s2.out = y;
        s2.out_dtype = y_dtype;
        s2.ep = Epilogue{x,
                         x_dtype,
                         d->in_features,
                         d->salient_count,
                         d->salient_indices,
                         d->salient_values,
                         d->salient_dtype,
                         d->salient_scales,
                         d->scale_dtype,
                         d->bias,
                         d->bias_dtype};
        st = launch_binary_rows(s2, s);
        if (st != NQ_OK) return st;
    }

    return apply_extras(d, x, x_dtype, tokens, y, ws + wl.patch_offset, s);
}

extern "C" int nq_linear_batch(const nq_linear_desc* const* descs, int32_t count, const void* const* xs,
                               int32_t x_dtype, int64_t tokens, void* const* ys, int32_t y_dtype,
                               void* const* workspaces, const int64_t* workspace_bytes, void* stream) {
    if (!descs || !xs || !ys || !workspaces || !workspace_bytes) return NQ_ERR_ARGUMENT;
    if (count < 1 || count > 8) return NQ_ERR_SHAPE;
    if (tokens < 1) return NQ_ERR_SHAPE;
    if (!nq::is_float_dtype(x_dtype) || !nq::is_float_dtype(y_dtype)) return NQ_ERR_DTYPE;
    const bool decode = tokens <= 16;
    void* scratch[8];
    for (int i = 0; i < count; ++i) {
        const nq_linear_desc* d = descs[i];
        int st = validate(d);
        if (st != NQ_OK) return st;
        if (!d->tiles || !xs[i] || !ys[i]) return NQ_ERR_ARGUMENT;
        if (y_dtype != NQ_DTYPE_F32 && (d->patch_rank > 0 || d->row_count > 0)) return NQ_ERR_UNSUPPORTED;
        if (decode) {
            for (int j = 0; j < i; ++j) {
                if (descs[j]->tiles == d->tiles) return NQ_ERR_ARGUMENT;  // one sync header per launch
            }
        } else if (!nq::prefill_path_applies(d, tokens)) {
            return NQ_ERR_SHAPE;
        }
        const WorkspaceLayout wl = workspace_layout(d, tokens);
        if (!workspaces[i] || workspace_bytes[i] < wl.total) return NQ_ERR_WORKSPACE;
        scratch[i] = static_cast<char*>(workspaces[i]) + wl.decode_offset;
    }
    auto s = static_cast<hipStream_t>(stream);
    int st = decode ? nq::launch_decode_batch(descs, count, xs, x_dtype, tokens, ys, y_dtype, scratch, s)
                    : nq::launch_prefill_batch(descs, count, xs, x_dtype, tokens, ys, y_dtype, scratch, s);
    if (st != NQ_OK) return st;
    for (int i = 0; i < count; ++i) {
        const WorkspaceLayout wl = workspace_layout(descs[i], tokens);
        st = apply_extras(descs[i], xs[i], x_dtype, tokens, ys[i],
                          static_cast<char*>(workspaces[i]) + wl.patch_offset, s);
        if (st != NQ_OK) return st;
    }
    return NQ_OK;
}

extern "C" int nq_linear_batch_fused(const nq_linear_desc* const* descs, int32_t count, const void* const* xs,
                                     int32_t x_dtype, void* const* ys, int32_t y_dtype, void* const* workspaces,
                                     const int64_t* workspace_bytes, const nq_decode_fusion* fusion, void* stream) {
    if (!descs || !xs || !ys || !workspaces || !workspace_bytes || !fusion) return NQ_ERR_ARGUMENT;
    if (count < 1 || count > 8) return NQ_ERR_SHAPE;
    if (!nq::is_float_dtype(x_dtype) || !nq::is_float_dtype(y_dtype)) return NQ_ERR_DTYPE;
    if (fusion->input_kind != NQ_INPUT_PLAIN && x_dtype != NQ_DTYPE_F32) return NQ_ERR_DTYPE;
    constexpr int64_t tokens = 1;
    void* scratch[8];
    for (int i = 0; i < count; ++i) {
        const nq_linear_desc* d = descs[i];
        int st = validate(d);
        if (st != NQ_OK) return st;
        if (!d->tiles || !xs[i]) return NQ_ERR_ARGUMENT;
        const bool silu_second = fusion->output_kind == NQ_OUTPUT_SILU_PRODUCT && i == 1;  // writes nothing
        if (!fusion->residuals && !ys[i] && !silu_second) return NQ_ERR_ARGUMENT;
        if (d->patch_rank > 0 || d->row_count > 0) return NQ_ERR_UNSUPPORTED;  // they add to y afterwards
        if (d->scale_dtype != NQ_DTYPE_F16) return NQ_ERR_DTYPE;
        for (int j = 0; j < i; ++j) {
            if (descs[j]->tiles == d->tiles) return NQ_ERR_ARGUMENT;  // one sync header per launch
        }
        const WorkspaceLayout wl = workspace_layout(d, tokens);
        if (!workspaces[i] || workspace_bytes[i] < wl.total) return NQ_ERR_WORKSPACE;
        scratch[i] = static_cast<char*>(workspaces[i]) + wl.decode_offset;
    }
    return nq::launch_decode_batch(descs, count, xs, x_dtype, tokens, ys, y_dtype, scratch,
                                   static_cast<hipStream_t>(stream), fusion);
}

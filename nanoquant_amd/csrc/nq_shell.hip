// Decoder-shell kernels for batch-1 autoregressive decode around the packed
// linears on gfx950 (Qwen3 geometry): embedding gather, residual add +
// RMSNorm, per-head q/k RMSNorm + rotate-half RoPE + KV-cache append,
// split-sequence grouped-query attention, SiLU-gated product, bf16 output
// projection with per-workgroup argmax partials, and greedy selection.
//
// All kernels read the token position from device memory, so one captured
// decode step replays for every position. Every reduction runs in a fixed
// order (wave butterflies, then waves in index order, then sequence blocks in
// index order), so results are identical from run to run.
#include <math.h>

#include "nq_common.h"
#include "../../include/nqamd_shell.h"

namespace {

using nq::f32_to_bf16_bits;

constexpr int kWave = 64;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSeqBlock = nq::kAttnBlockRows;  // cache rows per attention block
constexpr int kRowThreads = 256;        // per-row kernels
constexpr int kProjWaves = 4;           // output projection: waves per workgroup (2 or 8: 13% slower)
constexpr int kProjLoads = 32;          // 16-byte weight loads per lane in flight

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Wave reductions with DPP row operations and four lane reads (no LDS round
// trips); every lane gets the result, combined in a fixed order.
// Lane value CTRL-permuted within rows; `identity` where a source lane is off.
template <int CTRL>
__device__ __forceinline__ float dpp_src(float x, float identity) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float row_lane(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_src<0xB1>(v, 0.0f);   // quad_perm [1,0,3,2]
    v += dpp_src<0x4E>(v, 0.0f);   // quad_perm [2,3,0,1]
    v += dpp_src<0x141>(v, 0.0f);  // row_half_mirror
    v += dpp_src<0x140>(v, 0.0f);  // row_mirror
    return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}

// Max / sum over each row of 16 lanes (every lane of the row gets it).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_src<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_src<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_src<0x141>(v, -INFINITY));
    return fmaxf(v, dpp_src<0x140>(v, -INFINITY));
}

__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_src<0xB1>(v, 0.0f);
    v += dpp_src<0x4E>(v, 0.0f);
    v += dpp_src<0x141>(v, 0.0f);
    return v + dpp_src<0x140>(v, 0.0f);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_src<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_src<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_src<0x141>(v, -INFINITY));
    v = fmaxf(v, dpp_src<0x140>(v, -INFINITY));
    return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}

// Elements [i, i + 8) of a typed buffer as fp32; i % 8 == 0 and the buffer is
// 16-byte aligned (checked on the host).
__device__ __forceinline__ void load8(const void* __restrict__ p, int dtype, int64_t i, float (&v)[8]) {
    if (dtype == NQ_DTYPE_F32) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 a = q[0], b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        return;
    }
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    if (dtype == NQ_DTYPE_BF16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = bf16_lo(w[j]);
            v[2 * j + 1] = bf16_hi(w[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[j] & 0xffffu)));
            v[2 * j + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[j] >> 16)));
        }
    }
}

__device__ __forceinline__ uint32_t pack2(int dtype, float a, float b) {
    if (dtype == NQ_DTYPE_BF16) return f32_to_bf16_bits(a) | (static_cast<uint32_t>(f32_to_bf16_bits(b)) << 16);
    const uint16_t ha = __builtin_bit_cast(uint16_t, static_cast<_Float16>(a));
    const uint16_t hb = __builtin_bit_cast(uint16_t, static_cast<_Float16>(b));
    return ha | (static_cast<uint32_t>(hb) << 16);
}

__device__ __forceinline__ void store8(void* __restrict__ p, int dtype, int64_t i, const float (&v)[8]) {
    if (dtype == NQ_DTYPE_F32) {
        float4* q = reinterpret_cast<float4*>(static_cast<float*>(p) + i);
        q[0] = make_float4(v[0], v[1], v[2], v[3]);
        q[1] = make_float4(v[4], v[5], v[6], v[7]);
        return;
    }
    uint4 u;
    u.x = pack2(dtype, v[0], v[1]);
    u.y = pack2(dtype, v[2], v[3]);
    u.z = pack2(dtype, v[4], v[5]);
    u.w = pack2(dtype, v[6], v[7]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = u;
}

// ---------------------------------------------------------------------------
// Embedding gather.

__global__ __launch_bounds__(kRowThreads) void k_embedding(const int64_t* __restrict__ ids, const void* __restrict__ table,
                                                           int dtype, int64_t vocab, int64_t hidden,
                                                           const float* __restrict__ scale, float* __restrict__ out,
                                                           float* __restrict__ slots) {
    const int64_t t = blockIdx.x;
    const int64_t id = ids[t];
    const bool ok = id >= 0 && id < vocab;
    const float s = scale ? scale[0] : 1.0f;
    for (int64_t i = threadIdx.x * 8; i < hidden; i += kRowThreads * 8) {
        float v[8];
        if (ok) {
            load8(table, dtype, id * hidden + i, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = __fmul_rn(v[j], s);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = __builtin_nanf("");
        }
        store8(out, NQ_DTYPE_F32, t * hidden + i, v);
        if (slots) {  // uniform. hidden % 16 == 0: threads 2k and 2k + 1 hold the 16 columns of one slot
            float sq = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) sq = fmaf(v[j], v[j], sq);
            const float pair = sq + __shfl_xor(sq, 1, kWave);
            if ((threadIdx.x & 1) == 0) slots[t * (hidden / 16) + i / 16] = pair;
        }
    }
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm, one workgroup of kNormThreads per token row. Thread
// i holds elements [8 (i + kNormThreads j), +8) for j < NV in registers, so
// residual, delta and weight are loaded in one round trip; the sum of squares
// goes through wave butterflies and then the wave sums in wave order.

constexpr int kNormThreads = 512;

template <int NV>
__global__ __launch_bounds__(kNormThreads) void k_add_rmsnorm(float* __restrict__ residual, const void* __restrict__ delta,
                                                              int ddt, const void* __restrict__ weight, int wdt,
                                                              float eps, int64_t hidden, void* __restrict__ out, int odt) {
    __shared__ float red[kNormThreads / kWave];
    const int64_t row = static_cast<int64_t>(blockIdx.x) * hidden;
    float v[NV][8], w[NV][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t i = (threadIdx.x + static_cast<int64_t>(kNormThreads) * j) * 8;
        if (i < hidden) {
            load8(residual, NQ_DTYPE_F32, row + i, v[j]);
            load8(weight, wdt, i, w[j]);
            if (delta) {
                float d[8];
                load8(delta, ddt, row + i, d);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = __fadd_rn(v[j][e], d[e]);
                store8(residual, NQ_DTYPE_F32, row + i, v[j]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = w[j][e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / kWave; ++i) total += red[i];
    const float inv = 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(hidden), eps));  // no fma contraction
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t i = (threadIdx.x + static_cast<int64_t>(kNormThreads) * j) * 8;
        if (i < hidden) {
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __fmul_rn(w[j][e], __fmul_rn(v[j][e], inv));
            store8(out, odt, row + i, o);
        }
    }
}

// ---------------------------------------------------------------------------
// q/k per-head RMSNorm + rotate-half RoPE + KV-cache append. One wave per
// (token, head); grid.y = q_heads + kv_heads. Lane l holds elements
// d = l + 64 j, so for head_dim >= 128 the rotate-half partner d +- D/2 is
// element j +- E/2 of the same lane; for head_dim 64 it is lane l ^ 32.

// Element i of an F32 / F16 / BF16 buffer from one unconditional 32-bit load
// (the fp32 itself, or the pair of 16-bit elements 2 (i / 2) and 2 (i / 2) + 1,
// counted from the buffer's start: the callers' buffers hold head_dim
// elements, an even count): no branch surrounds the load and nothing is
// derived from it before use, so a wave issues all of them before waiting on
// any.
struct RawHalves {
    uint32_t word, shift;
};

__device__ __forceinline__ RawHalves load_raw(const void* __restrict__ p, int dtype, int64_t i) {
    const bool wide = dtype == NQ_DTYPE_F32;
    RawHalves r;
    r.word = static_cast<const uint32_t*>(p)[wide ? i : i >> 1];
    r.shift = wide ? 0u : static_cast<uint32_t>(i & 1) << 4;
    return r;
}

__device__ __forceinline__ float raw_value(const RawHalves& r, int dtype) {
    const uint32_t half = r.word >> r.shift;
    const float f32 = __uint_as_float(r.word);
    const float bf16 = __uint_as_float(half << 16);
    const float f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(half)));
    return dtype == NQ_DTYPE_F32 ? f32 : (dtype == NQ_DTYPE_BF16 ? bf16 : f16);
}

// The operands of norm_rope_regs for one lane: the head vector's elements
// d = lane + 64 j and the norm weights (loaded from the head vector itself,
// and ignored, when there is no weight).
template <int D>
struct NormRopeIn {
    float x[D / kWave];
    RawHalves w[D / kWave];
};

template <int D>
__device__ __forceinline__ void load_norm_rope_in(NormRopeIn<D>& in, const float* __restrict__ src,
                                                  const void* __restrict__ nw, int ndt, int lane) {
    const void* wp = nw ? nw : static_cast<const void*>(src);
    const int wdt = nw ? ndt : NQ_DTYPE_F32;
#pragma unroll
    for (int j = 0; j < D / kWave; ++j) {
        in.x[j] = src[lane + kWave * j];
        in.w[j] = load_raw(wp, wdt, lane + kWave * j);
    }
}

// norm_rope on loaded operands: cs / sn are the lane's RoPE table entries
// (index d mod D/2 of the position's row).
template <int D>
__device__ __forceinline__ void norm_rope_regs(const NormRopeIn<D>& in, bool has_w, int ndt, float eps,
                                               const float (&cs)[D / kWave], const float (&sn)[D / kWave], int lane,
                                               float (&y)[D / kWave]) {
    constexpr int E = D / kWave;
    constexpr int kHalf = D / 2;
    float x[E];
#pragma unroll
    for (int j = 0; j < E; ++j) x[j] = in.x[j];
    // Branch-free (a branch here would sink the weight loads into it).
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) ss = fmaf(x[j], x[j], ss);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(__fadd_rn(ss / static_cast<float>(D), eps));  // no fma contraction
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const float normed = __fmul_rn(raw_value(in.w[j], ndt), __fmul_rn(x[j], inv));
        x[j] = has_w ? normed : x[j];
    }
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        const bool first = d < kHalf;
        float partner;
        if constexpr (E == 1) {
            partner = __shfl_xor(x[0], 32, kWave);
        } else {
            partner = first ? x[j + E / 2] : x[j - E / 2];
        }
        const float rot = first ? -partner : partner;
        y[j] = __fadd_rn(__fmul_rn(x[j], cs[j]), __fmul_rn(rot, sn[j]));
    }
}

// Lane's E = D / 64 elements d = lane + 64 j of one head vector: RMSNorm with
// weight nw (when not NULL), then rotate-half RoPE with the table rows cr/sr
// (the same arithmetic as the fused decode attention, norm_rope_regs).
template <int D>
__device__ __forceinline__ void norm_rope(const float* __restrict__ src, const void* __restrict__ nw, int ndt, float eps,
                                          const float* __restrict__ cr, const float* __restrict__ sr, int lane,
                                          float (&y)[D / kWave]) {
    constexpr int E = D / kWave;
    NormRopeIn<D> in;
    load_norm_rope_in<D>(in, src, nw, ndt, lane);
    float cs[E], sn[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        const int fi = d < D / 2 ? d : d - D / 2;
        cs[j] = cr[fi];
        sn[j] = sr[fi];
    }
    norm_rope_regs<D>(in, nw != nullptr, ndt, eps, cs, sn, lane, y);
}

template <int D>
__global__ __launch_bounds__(kWave) void k_qk_norm_rope_cache(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, int q_heads,
    int kv_heads, const void* __restrict__ q_norm, const void* __restrict__ k_norm, int ndt, float eps,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table, const int32_t* __restrict__ position,
    int64_t max_positions, float* __restrict__ q_out, void* __restrict__ k_cache, void* __restrict__ v_cache, int cdt) {
    constexpr int E = D / kWave;
    const int64_t t = blockIdx.x;
    const int h = blockIdx.y;
    const int lane = threadIdx.x;
    const int64_t pos = static_cast<int64_t>(position[0]) + t;
    if (pos < 0 || pos >= max_positions) return;
    const bool is_q = h < q_heads;
    const int g = is_q ? h : h - q_heads;
    const float* src = is_q ? q + (t * q_heads + h) * D : k + (t * kv_heads + g) * D;
    float y[E];
    norm_rope<D>(src, is_q ? q_norm : k_norm, ndt, eps, cos_table + pos * (D / 2), sin_table + pos * (D / 2), lane, y);
    if (is_q) {
        float* dst = q_out + (t * q_heads + h) * D;
#pragma unroll
        for (int j = 0; j < E; ++j) dst[lane + kWave * j] = y[j];
        return;
    }
    const int64_t crow = (static_cast<int64_t>(g) * max_positions + pos) * D;
    const float* vs = v + (t * kv_heads + g) * D;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        nq::store_f32_as(k_cache, cdt, crow + d, y[j]);
        nq::store_f32_as(v_cache, cdt, crow + d, vs[d]);
    }
}

// ---------------------------------------------------------------------------
// Attention, pass 1: one workgroup per (kv head, block of QT queries,
// 64-row cache block s); wave w serves q head kv_head * G + w. The K rows of
// the block are copied to LDS as stored (16-byte copies, padded rows); lane j
// scores cache row 64 s + j against the query (fp32, in LDS), the wave forms
// its softmax partial (max m, sum l) and lane pairs of dimensions accumulate
// P.V straight from the V rows (all waves of the workgroup read the same rows,
// so they come from cache). The partial goes to the workspace.

template <int CT>
constexpr int cache_bytes() { return CT == NQ_DTYPE_F32 ? 4 : 2; }

template <int D, int CT>
constexpr int k_row_bytes() { return D * cache_bytes<CT>() + 16; }

// k_attention_blocks stages the block's V rows in LDS too when a row is at
// most 256 bytes (the K and V blocks then fit 64 KB with the per-wave rows).
template <int D, int CT>
constexpr bool attention_stages_v() { return D * cache_bytes<CT>() <= 256; }

template <int D, int CT>
constexpr size_t attention_lds(int waves) {
    return static_cast<size_t>(kSeqBlock) * k_row_bytes<D, CT>() +
           (attention_stages_v<D, CT>() ? static_cast<size_t>(kSeqBlock) * D * cache_bytes<CT>() : 0) +
           static_cast<size_t>(waves) * (D + kSeqBlock) * 4;
}

template <int CT>
__device__ __forceinline__ float cache_value(uint32_t bits16) {
    if constexpr (CT == NQ_DTYPE_BF16) return __uint_as_float(bits16 << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// Dot product of one staged K row with the query (both D long).
template <int D, int CT>
__device__ __forceinline__ float k_row_dot(const char* __restrict__ kr, const float* __restrict__ qw) {
    // Four accumulators (dimensions d mod 4), combined at the end: four short
    // dependency chains instead of one of length D.
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    if constexpr (CT == NQ_DTYPE_F32) {
#pragma unroll 8
        for (int d = 0; d < D; d += 4) {
            const float4 kk = *reinterpret_cast<const float4*>(kr + 4 * d);
            const float4 qq = *reinterpret_cast<const float4*>(qw + d);
            a0 = fmaf(kk.x, qq.x, a0);
            a1 = fmaf(kk.y, qq.y, a1);
            a2 = fmaf(kk.z, qq.z, a2);
            a3 = fmaf(kk.w, qq.w, a3);
        }
    } else {
#pragma unroll 4
        for (int d = 0; d < D; d += 8) {
            const uint4 u = *reinterpret_cast<const uint4*>(kr + 2 * d);
            const float4 qa = *reinterpret_cast<const float4*>(qw + d);
            const float4 qb = *reinterpret_cast<const float4*>(qw + d + 4);
            a0 = fmaf(cache_value<CT>(u.x & 0xffffu), qa.x, a0);
            a1 = fmaf(cache_value<CT>(u.x >> 16), qa.y, a1);
            a2 = fmaf(cache_value<CT>(u.y & 0xffffu), qa.z, a2);
            a3 = fmaf(cache_value<CT>(u.y >> 16), qa.w, a3);
            a0 = fmaf(cache_value<CT>(u.z & 0xffffu), qb.x, a0);
            a1 = fmaf(cache_value<CT>(u.z >> 16), qb.y, a1);
            a2 = fmaf(cache_value<CT>(u.w & 0xffffu), qb.z, a2);
            a3 = fmaf(cache_value<CT>(u.w >> 16), qb.w, a3);
        }
    }
    return (a0 + a1) + (a2 + a3);
}

// E consecutive cache elements (E = D / 64, lane's dimensions) as fp32.
template <int E, int CT>
__device__ __forceinline__ void load_v(const char* __restrict__ p, float (&v)[E]) {
    if constexpr (CT == NQ_DTYPE_F32) {
#pragma unroll
        for (int j = 0; j < E; ++j) v[j] = reinterpret_cast<const float*>(p)[j];
    } else if constexpr (E == 1) {
        v[0] = cache_value<CT>(*reinterpret_cast<const uint16_t*>(p));
    } else {
#pragma unroll
        for (int j = 0; j < E; j += 2) {
            const uint32_t u = reinterpret_cast<const uint32_t*>(p)[j / 2];
            v[j] = cache_value<CT>(u & 0xffffu);
            v[j + 1] = cache_value<CT>(u >> 16);
        }
    }
}

constexpr int kMergeRound = 16;  // partial blocks merged per round of loads

__device__ __forceinline__ int64_t attn_part_index(int64_t t, int h, int s, int q_heads, int blocks) {
    return (t * q_heads + h) * blocks + s;
}

template <int D, int CT>
__global__ __launch_bounds__(1024) void k_attention_blocks(const float* __restrict__ q, const char* __restrict__ k_cache,
                                                           const char* __restrict__ v_cache, int64_t tokens,
                                                           int q_heads, int kv_heads, int qt,
                                                           const int32_t* __restrict__ position, int64_t max_positions,
                                                           float scaling, float* __restrict__ part_ml,
                                                           float* __restrict__ part_acc) {
    constexpr int E = D / kWave;
    constexpr int EB = cache_bytes<CT>();
    constexpr int RB = k_row_bytes<D, CT>();
    constexpr int PIECES = D * EB / 16;  // 16-byte pieces per row
    constexpr int U = 8;                 // V rows per unrolled step
    constexpr bool SV = attention_stages_v<D, CT>();
    constexpr int VRB = D * EB;          // V row in LDS
    extern __shared__ float lds_raw[];
    char* klds = reinterpret_cast<char*>(lds_raw);
    char* vlds = klds + kSeqBlock * RB;                                         // [64][D] when SV
    float* qv = reinterpret_cast<float*>(vlds + (SV ? kSeqBlock * VRB : 0));  // [waves][D]
    float* pv = qv + (blockDim.x / kWave) * D;                                  // [waves][64]

    const int group = q_heads / kv_heads;
    const int g = blockIdx.x % kv_heads;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x / kv_heads) * qt;
    const int s = blockIdx.y;
    const int blocks = gridDim.y;
    const int64_t p0 = position[0];
    const int64_t row0 = static_cast<int64_t>(s) * kSeqBlock;
    const int64_t t_end = t0 + qt < tokens ? t0 + qt : tokens;
    // Highest cache row any query of this workgroup may see.
    int64_t last = p0 + t_end - 1;
    if (last >= max_positions) last = max_positions - 1;
    if (p0 < 0 || row0 > last) return;  // uniform: no query of this workgroup reaches row0
    const int rows = static_cast<int>((last - row0 + 1) < kSeqBlock ? (last - row0 + 1) : kSeqBlock);

    // Copy K rows [row0, row0 + rows) of kv head g to LDS as stored, and the
    // V rows too when they fit (every query of the workgroup reads them).
    const int64_t head_row0 = static_cast<int64_t>(g) * max_positions + row0;
    const char* kbase = k_cache + head_row0 * D * EB;
    const char* vbase = v_cache + head_row0 * D * EB;
    for (int i = threadIdx.x; i < rows * PIECES; i += blockDim.x) {
        const int r = i / PIECES, c = i % PIECES;
        const uint4 kq = *reinterpret_cast<const uint4*>(kbase + (static_cast<int64_t>(r) * D) * EB + 16 * c);
        if constexpr (SV) {
            const uint4 vq = *reinterpret_cast<const uint4*>(vbase + (static_cast<int64_t>(r) * D) * EB + 16 * c);
            *reinterpret_cast<uint4*>(vlds + r * VRB + 16 * c) = vq;
        }
        *reinterpret_cast<uint4*>(klds + r * RB + 16 * c) = kq;
    }
    const int w = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int h = g * group + w;
    float* qw = qv + w * D;
    float* pw = pv + w * kSeqBlock;
    const char* vlane = SV ? vlds + lane * E * EB : v_cache + (head_row0 * D + lane * E) * EB;
    __syncthreads();

    for (int64_t t = t0; t < t_end; ++t) {
        const int64_t pt = p0 + t;
        if (pt < row0 || pt >= max_positions) continue;  // uniform per workgroup
        const float* qs = q + (t * q_heads + h) * D;
#pragma unroll
        for (int j = 0; j < E; ++j) qw[lane + kWave * j] = qs[lane + kWave * j];
        __builtin_amdgcn_wave_barrier();
        const int nvalid = static_cast<int>((pt - row0 + 1) < kSeqBlock ? (pt - row0 + 1) : kSeqBlock);
        const bool valid = lane < nvalid;
        // Lanes past the staged rows score row 0 (always staged) and are masked.
        const float dot = k_row_dot<D, CT>(klds + (lane < rows ? lane : 0) * RB, qw);
        const float score = valid ? dot * scaling : -INFINITY;
        const float m = wave_max(score);
        const float p = valid ? expf(score - m) : 0.0f;
        const float l = wave_sum(p);
        pw[lane] = p;
        __builtin_amdgcn_wave_barrier();
        float acc[E];
#pragma unroll
        for (int j = 0; j < E; ++j) acc[j] = 0.0f;
        for (int r0 = 0; r0 < nvalid; r0 += U) {
            float vv[U][E];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = r0 + u < nvalid ? r0 + u : nvalid - 1;  // p is 0 past nvalid
                load_v<E, CT>(vlane + static_cast<int64_t>(r) * D * EB, vv[u]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float pr = pw[(r0 + u) & (kSeqBlock - 1)];
#pragma unroll
                for (int j = 0; j < E; ++j) acc[j] = fmaf(pr, vv[u][j], acc[j]);
            }
        }
        const int64_t pi = attn_part_index(t, h, s, q_heads, blocks);
        if (lane == 0) {
            part_ml[2 * pi] = m;
            part_ml[2 * pi + 1] = l;
        }
        float* pa = part_acc + pi * D + lane * E;
#pragma unroll
        for (int j = 0; j < E; ++j) pa[j] = acc[j];
        __builtin_amdgcn_wave_barrier();  // qw / pw are rewritten for the next query
    }
}

// Attention, pass 2: merge the blocks (of block_rows cache rows each) of one
// (token, q head) in block order.
template <int D>
__global__ __launch_bounds__(D) void k_attention_merge(const float* __restrict__ part_ml, const float* __restrict__ part_acc,
                                                       int q_heads, int blocks, int block_rows,
                                                       const int32_t* __restrict__ position, int64_t max_positions,
                                                       void* __restrict__ out, int odt) {
    const int h = blockIdx.x;
    const int64_t t = blockIdx.y;
    const int d = threadIdx.x;
    const int64_t o = (t * q_heads + h) * D + d;
    const int64_t p0 = attn_part_index(t, h, 0, q_heads, blocks);
    // Rounds of kMergeRound blocks: every load of a round is issued before any
    // use, the first round before the position is read (block indices clamped
    // to the grid's blocks; blocks past the position weigh 0), and rounds
    // combine with a running max.
    float mb[kMergeRound], lb[kMergeRound], ab[kMergeRound];
    const auto load_round = [&](const int b0, const int last) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kMergeRound; ++i) {
            const int64_t pb = p0 + (b0 + i < last ? b0 + i : last);
            mb[i] = part_ml[2 * pb];
            lb[i] = part_ml[2 * pb + 1];
            ab[i] = part_acc[pb * D + d];
        }
    };
    load_round(0, blocks - 1);
    const int64_t pt = static_cast<int64_t>(position[0]) + t;
    const bool in_range = pt >= 0 && pt < max_positions;  // uniform
    const int nb = in_range ? static_cast<int>(pt / block_rows) + 1 : 1;
    float mrun = -INFINITY, lsum = 0.0f, acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += kMergeRound) {
        if (b0 > 0) load_round(b0, nb - 1);
        float mnew = mrun;
#pragma unroll
        for (int i = 0; i < kMergeRound; ++i) mnew = b0 + i < nb ? fmaxf(mnew, mb[i]) : mnew;
        const float keep = nq::merge_exp(mrun - mnew);  // 0 in the first round
        lsum *= keep;
        acc *= keep;
#pragma unroll
        for (int i = 0; i < kMergeRound; ++i) {
            if (b0 + i < nb) {  // a select: slots past the position may hold anything
                const float f = nq::merge_exp(mb[i] - mnew);
                lsum = fmaf(lb[i], f, lsum);
                acc = fmaf(ab[i], f, acc);
            }
        }
        mrun = mnew;
    }
    if (!in_range) acc = 0.0f, lsum = 1.0f;
    nq::store_f32_as(out, odt, o, acc / lsum);
}

// ---------------------------------------------------------------------------
// One-token decode attention on MFMA (head_dim 128, four q heads per kv head,
// 16-bit cache): the same workgroup grid, loads, staging, RoPE / KV append and
// partial output as k_decode_attention below, with the two products on
// v_mfma_f32_16x16x32 (bf16 or f16, the cache's type). The query and the
// softmax weights are fp32; each is split into three 16-bit parts (the
// rounding of the value, of its remainder and of the remainder's remainder),
// which occupy A rows 4h, 4h + 1, 4h + 2 for q head h of the group (row
// 4h + 3 is zero), so the products carry about 24 bits of the fp32 operand
// and K / V (stored 16-bit) are exact. Output rows 4h .. 4h + 3 then sit in
// the four accumulator registers of lane group h.
//   Scores: wave w takes cache rows 16w + n (B columns n; B = K rows from LDS,
//   eight dimensions per lane per step), four steps of 32 dimensions.
//   P.V: wave w takes dimensions 32w + 16u + n (u = 0, 1), two steps of 32
//   cache rows; A = the weights from LDS, B = V rows from LDS.
// The softmax max and sum cross the four waves through LDS; rows past the
// token's position weigh zero (their LDS rows are zero-filled, so 0 * V stays
// 0). Results differ from k_decode_attention only by rounding.
constexpr int kMfmaHeads = 4;

template <int CT>
struct Mfma16 {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
};
template <>
struct Mfma16<NQ_DTYPE_F16> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
};

typedef float v4f_t __attribute__((ext_vector_type(4)));

template <int CT>
__device__ __forceinline__ v4f_t mfma16(const typename Mfma16<CT>::v8& a, const typename Mfma16<CT>::v8& b,
                                        const v4f_t& c) {
    if constexpr (CT == NQ_DTYPE_BF16) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The 16-bit rounding (nearest-even) of x, and a 16-bit value as fp32.
template <int CT>
__device__ __forceinline__ uint16_t to16(float x) {
    if constexpr (CT == NQ_DTYPE_BF16) return f32_to_bf16_bits(x);
    else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

template <int CT>
__device__ __forceinline__ float from16(uint16_t h) {
    if constexpr (CT == NQ_DTYPE_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
    else return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// The three 16-bit parts of x: the rounding of x, of its remainder and of the
// remainder's remainder (each subtraction is exact in fp32).
template <int CT>
__device__ __forceinline__ void split3(float x, uint16_t (&h)[3]) {
    h[0] = to16<CT>(x);
    const float r1 = x - from16<CT>(h[0]);
    h[1] = to16<CT>(r1);
    h[2] = to16<CT>(r1 - from16<CT>(h[1]));
}

template <int CT>
constexpr size_t decode_attention_mfma_lds() {
    // K and V blocks (plus a scratch row each), the 16-bit parts of q [4][4][128]
    // and of P [4][4][64], maxima and sums [2][4][4].
    return static_cast<size_t>(kSeqBlock + 1) * k_row_bytes<128, CT>() * 2 + kMfmaHeads * 4 * 128 * 2 +
           kMfmaHeads * 4 * kSeqBlock * 2 + 2 * kMfmaHeads * kMfmaHeads * 4;
}

template <int CT, bool HALF>
__global__ __launch_bounds__(kMfmaHeads * kWave) void k_decode_attention_mfma(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, int kv_heads,
    const void* __restrict__ q_norm, const void* __restrict__ k_norm, int ndt, float eps,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table, const int32_t* __restrict__ position,
    int64_t max_positions, char* __restrict__ k_cache, char* __restrict__ v_cache, float scaling,
    float* __restrict__ part_ml, float* __restrict__ part_acc) {
    constexpr int D = 128;
    constexpr int G = kMfmaHeads;
    constexpr int E = D / kWave;
    constexpr int RB = k_row_bytes<D, CT>();  // padded row in LDS (K and V alike)
    constexpr int VRB = D * 2;                // row in the cache
    constexpr int PIECES = VRB / 16;
    constexpr int PER_THREAD = kSeqBlock * PIECES / (G * kWave);
    typedef typename Mfma16<CT>::v8 v8;
    extern __shared__ float lds_raw[];
    char* klds = reinterpret_cast<char*>(lds_raw);
    char* vlds = klds + (kSeqBlock + 1) * RB;
    uint16_t* qs = reinterpret_cast<uint16_t*>(vlds + (kSeqBlock + 1) * RB);  // [G][4 parts][D]
    uint16_t* ps = qs + G * 4 * D;                                             // [G][4 parts][64]
    float* mx = reinterpret_cast<float*>(ps + G * 4 * kSeqBlock);             // [G][4 waves]
    float* ls = mx + G * G;                                                    // [G][4 waves]

    const int g = blockIdx.x;
    const int s = blockIdx.y;
    // gridDim.y, from an argument: gridDim is read from the hidden kernel
    // arguments, one more scalar-cache line before the first load.
    const int blocks = static_cast<int>((max_positions + kSeqBlock - 1) / kSeqBlock);
    const int q_heads = kv_heads * G;
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int lane = threadIdx.x & (kWave - 1);

    NormRopeIn<D> qin, kin;
    load_norm_rope_in<D>(qin, q + static_cast<int64_t>(g * G + w) * D, q_norm, ndt, lane);
    load_norm_rope_in<D>(kin, k + static_cast<int64_t>(g) * D, k_norm, ndt, lane);
    float vraw[E];
#pragma unroll
    for (int j = 0; j < E; ++j) vraw[j] = v[static_cast<int64_t>(g) * D + lane + kWave * j];

    const int64_t row0 = static_cast<int64_t>(s) * kSeqBlock;
    const int64_t head_row0 = static_cast<int64_t>(g) * max_positions;
    u32x4 kp[PER_THREAD], vp[PER_THREAD];
    const int last_row = static_cast<int>(max_positions - 1 - row0);
    const char* kbase = k_cache + (head_row0 + row0) * VRB;
    const char* vbase = v_cache + (head_row0 + row0) * VRB;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = threadIdx.x + i * G * kWave;
        const int r = idx / PIECES, c = idx % PIECES;
        const int rr = r < last_row ? r : last_row;
        kp[i] = *reinterpret_cast<const u32x4*>(kbase + rr * VRB + 16 * c);
        vp[i] = *reinterpret_cast<const u32x4*>(vbase + rr * VRB + 16 * c);
    }
    __builtin_amdgcn_sched_barrier(0);

    const int64_t pos = position[0];
    const bool live = pos >= 0 && pos < max_positions && row0 <= pos;  // uniform
    const int64_t p = live ? pos : row0;
    const bool owns_p = live && p < row0 + kSeqBlock;
    const int rows = live ? static_cast<int>(owns_p ? p - row0 + 1 : kSeqBlock) : 1;
    const int cached = live ? (owns_p ? rows - 1 : rows) : 0;

    float cs[E], sn[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        const int fi = d < D / 2 ? d : d - D / 2;
        cs[j] = cos_table[p * (D / 2) + fi];
        sn[j] = sin_table[p * (D / 2) + fi];
    }
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) asm volatile("" : "+v"(kp[i]), "+v"(vp[i]));
    float qy[E];
    norm_rope_regs<D>(qin, q_norm != nullptr, ndt, eps, cs, sn, lane, qy);
    // Cached rows go to their LDS rows; rows past the token's row are zero
    // (their weights are zero, and 0 * V must stay 0); the token's own row is
    // written below, so its staging piece goes to the scratch row.
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = threadIdx.x + i * G * kWave;
        const int r = idx / PIECES, c = idx % PIECES;
        const bool keep = r < cached;
        const int lr = keep || r >= rows ? r : kSeqBlock;
        const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(klds + lr * RB + 16 * c) = keep ? kp[i] : zero;
        *reinterpret_cast<u32x4*>(vlds + lr * RB + 16 * c) = keep ? vp[i] : zero;
    }
#pragma unroll
    for (int j = 0; j < E; ++j) {  // wave w: the parts of q head w (part 3 zero)
        uint16_t h[3];
        split3<CT>(qy[j], h);
        const int d = lane + kWave * j;
#pragma unroll
        for (int part = 0; part < 3; ++part) qs[(w * 4 + part) * D + d] = h[part];
        qs[(w * 4 + 3) * D + d] = 0;
    }
    float ky[E];
    norm_rope_regs<D>(kin, k_norm != nullptr, ndt, eps, cs, sn, lane, ky);
    const int nr = owns_p ? rows - 1 : kSeqBlock;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        nq::store_f32_as(klds + nr * RB, CT, d, ky[j]);
        nq::store_f32_as(vlds + nr * RB, CT, d, vraw[j]);
    }
    if (owns_p) {
        const int64_t crow = (head_row0 + p) * D;
        if (w == 0) {
#pragma unroll
            for (int j = 0; j < E; ++j) nq::store_f32_as(k_cache, CT, crow + lane + kWave * j, ky[j]);
        }
        if (w == G - 1) {
#pragma unroll
            for (int j = 0; j < E; ++j) nq::store_f32_as(v_cache, CT, crow + lane + kWave * j, vraw[j]);
        }
    }
    __syncthreads();

    // Lane (kg, n): column n of the B operands, q head kg of the A rows
    // (row 4 kg + part, part = n & 3) and of the accumulator rows 4 kg + j.
    const int n = lane & 15, kg = lane >> 4;
    const int arow = lane & 15;  // A row: head arow / 4, part arow % 4 (parts are stored in that order)
    // Scores of cache rows 16w + n.
    v4f_t sc = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < D / 32; ++st) {
        const int d0 = 32 * st + 8 * kg;
        const v8 a = *reinterpret_cast<const v8*>(qs + arow * D + d0);
        const v8 b = *reinterpret_cast<const v8*>(klds + (16 * w + n) * RB + 2 * d0);
        sc = mfma16<CT>(a, b, sc);
    }
    const int r = 16 * w + n;
    const bool valid = r < rows;
    const float score = valid ? ((sc[0] + sc[1]) + (sc[2] + sc[3])) * scaling : -INFINITY;  // head kg
    const float mw = row16_max(score);
    if (n == 0) mx[kg * G + w] = mw;
    __syncthreads();
    float M = mx[kg * G];
#pragma unroll
    for (int i = 1; i < G; ++i) M = fmaxf(M, mx[kg * G + i]);
    const float pr = valid ? expf(score - M) : 0.0f;
    const float lw = row16_sum(pr);
    {
        uint16_t h[3];
        split3<CT>(pr, h);
#pragma unroll
        for (int part = 0; part < 3; ++part) ps[(kg * 4 + part) * kSeqBlock + r] = h[part];
        ps[(kg * 4 + 3) * kSeqBlock + r] = 0;
    }
    if (n == 0) ls[kg * G + w] = lw;
    __syncthreads();

    // P.V for dimensions 32w + 16u + n.
    v4f_t o[2] = {v4f_t{0.0f, 0.0f, 0.0f, 0.0f}, v4f_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int t = 0; t < kSeqBlock / 32; ++t) {
        const int r0 = 32 * t + 8 * kg;
        const v8 a = *reinterpret_cast<const v8*>(ps + arow * kSeqBlock + r0);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            union {
                uint16_t h[8];
                v8 v;
            } b;
            const int d = 32 * w + 16 * u + n;
#pragma unroll
            for (int i = 0; i < 8; ++i) b.h[i] = *reinterpret_cast<const uint16_t*>(vlds + (r0 + i) * RB + 2 * d);
            o[u] = mfma16<CT>(a, b.v, o[u]);
        }
    }
    // A block past the token's row stores the neutral partial (max -inf, sum
    // 0, accumulators 0), which adds nothing to a merge over every block.
    // HALF: the block's output acc / sum as fp16 in place of the accumulators.
    const int64_t pi = attn_part_index(0, g * G + kg, s, q_heads, blocks);
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < G; ++i) l += ls[kg * G + i];
    const float inv = HALF && live ? 1.0f / l : 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float a = (o[u][0] + o[u][1]) + (o[u][2] + o[u][3]);
        if constexpr (HALF)
            reinterpret_cast<_Float16*>(part_acc)[pi * D + 32 * w + 16 * u + n] =
                static_cast<_Float16>(live ? a * inv : 0.0f);
        else
            part_acc[pi * D + 32 * w + 16 * u + n] = live ? a : 0.0f;
    }
    if (w == 0 && n == 0) {
        part_ml[2 * pi] = live ? M : -INFINITY;
        part_ml[2 * pi + 1] = live ? l : 0.0f;
    }
}

// ---------------------------------------------------------------------------
// Prompt attention, pass 1 on MFMA (head_dim 128, four q heads per kv head,
// 16-bit cache): workgroup (kv head g, tile of kPromptTile tokens, 64-row
// cache block s); wave w computes q head 4g + w for the tile's tokens, the
// same partial (m, l, acc) per (token, q head, block) as k_attention_blocks,
// so k_attention_merge combines them unchanged.
//   Scores S = Q K^T on v_mfma_f32_16x16x32 (bf16 / f16, the cache's type):
//   A = the query rows (token i of the tile = row i), read from global memory
//   and split into three 16-bit parts in registers (the rounding of q, of its
//   remainder and of the remainder's remainder), all three accumulated into
//   the same tile, so the product carries about 24 bits of the fp32 query; B =
//   the block's K rows from LDS (exact). Four column tiles of 16 cache rows.
//   Causal softmax per query row over the block (rows past the token's
//   position weigh zero); the weights, split into three parts the same way,
//   go through LDS into the A layout; O = P V with B = V staged transposed in
//   LDS (one 16-byte read per lane), eight tiles of 16 dimensions.
// Results differ from k_attention_blocks only by rounding.
constexpr int kPromptTile = 16;                  // tokens per workgroup (A rows)
constexpr int kPromptVStride = kSeqBlock + 8;    // halfs per transposed V row and per P row

template <int CT>
constexpr size_t prompt_attention_mfma_lds() {
    // K block [64][row], V transposed [128][64 + 8], weight parts [3][4 waves][16][64 + 8].
    return static_cast<size_t>(kSeqBlock) * k_row_bytes<128, CT>() + 128 * kPromptVStride * 2 +
           3 * kMfmaHeads * kPromptTile * kPromptVStride * 2;
}

template <int CT>
__global__ __launch_bounds__(kMfmaHeads * kWave) void k_prompt_attention_mfma(
    const float* __restrict__ q, const char* __restrict__ k_cache, const char* __restrict__ v_cache, int64_t tokens,
    int kv_heads, const int32_t* __restrict__ position, int64_t max_positions, float scaling,
    float* __restrict__ part_ml, float* __restrict__ part_acc) {
    constexpr int D = 128;
    constexpr int G = kMfmaHeads;
    constexpr int T = kPromptTile;
    constexpr int RB = k_row_bytes<D, CT>();  // padded K row in LDS
    constexpr int VRB = D * 2;                // row in the cache
    constexpr int PIECES = VRB / 16;
    constexpr int VS = kPromptVStride;
    typedef typename Mfma16<CT>::v8 v8;
    extern __shared__ float lds_raw[];
    char* klds = reinterpret_cast<char*>(lds_raw);
    uint16_t* vt = reinterpret_cast<uint16_t*>(klds + kSeqBlock * RB);  // [D][VS]
    uint16_t* ps = vt + D * VS;                                         // [3][G][T][VS]

    const int q_heads = kv_heads * G;
    const int g = static_cast<int>(blockIdx.x) % kv_heads;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x / kv_heads) * T;
    const int s = blockIdx.y;
    const int blocks = gridDim.y;
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t p0 = position[0];
    const int64_t row0 = static_cast<int64_t>(s) * kSeqBlock;
    const int64_t t_end = t0 + T < tokens ? t0 + T : tokens;
    // Highest cache row any query of this workgroup may see.
    int64_t last = p0 + t_end - 1;
    if (last >= max_positions) last = max_positions - 1;
    if (p0 < 0 || row0 > last) return;  // uniform: no query of this workgroup reaches row0
    const int rows = static_cast<int>((last - row0 + 1) < kSeqBlock ? (last - row0 + 1) : kSeqBlock);

    // Query operands: lane (kg, n) holds token row n, dimensions 32 st + 8 kg + [0, 8).
    const int n = lane & 15, kg = lane >> 4;
    const int h = g * G + w;
    const int64_t tq = t0 + n < tokens ? t0 + n : tokens - 1;  // rows past the last token reuse it (not stored)
    float qf[4][8];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        const float4* src = reinterpret_cast<const float4*>(q + (tq * q_heads + h) * D + 32 * st + 8 * kg);
        const float4 x0 = src[0], x1 = src[1];
        qf[st][0] = x0.x; qf[st][1] = x0.y; qf[st][2] = x0.z; qf[st][3] = x0.w;
        qf[st][4] = x1.x; qf[st][5] = x1.y; qf[st][6] = x1.z; qf[st][7] = x1.w;
    }
    // K rows [row0, row0 + rows) to LDS as stored, V transposed; rows past
    // `rows` are zero (their weights are zero, and 0 * V must stay 0).
    const int64_t head_row0 = static_cast<int64_t>(g) * max_positions + row0;
    const char* kbase = k_cache + head_row0 * VRB;
    const char* vbase = v_cache + head_row0 * VRB;
    constexpr int PER_THREAD = kSeqBlock * PIECES / (G * kWave);
    u32x4 kp[PER_THREAD], vp[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = static_cast<int>(threadIdx.x) + i * G * kWave;
        const int r = idx % kSeqBlock, c = idx / kSeqBlock;
        const int rr = r < rows ? r : rows - 1;
        kp[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(rr) * VRB + 16 * c);
        vp[i] = *reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(rr) * VRB + 16 * c);
    }
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = static_cast<int>(threadIdx.x) + i * G * kWave;
        const int r = idx % kSeqBlock, c = idx / kSeqBlock;
        const bool keep = r < rows;
        const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(klds + r * RB + 16 * c) = keep ? kp[i] : zero;
        const u32x4 vv = keep ? vp[i] : zero;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            vt[(8 * c + e) * VS + r] = static_cast<uint16_t>((vv[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    }
    v8 qa[3][4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        union {
            uint16_t h[8];
            v8 v;
        } part[3];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint16_t hh[3];
            split3<CT>(qf[st][e], hh);
#pragma unroll
            for (int pp = 0; pp < 3; ++pp) part[pp].h[e] = hh[pp];
        }
#pragma unroll
        for (int pp = 0; pp < 3; ++pp) qa[pp][st] = part[pp].v;
    }
    __syncthreads();

    // Scores: sc[ct][j] = S[token row 4 kg + j][cache row 16 ct + n].
    v4f_t sc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
        sc[ct] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const v8 b = *reinterpret_cast<const v8*>(klds + (16 * ct + n) * RB + 2 * (32 * st + 8 * kg));
#pragma unroll
            for (int pp = 0; pp < 3; ++pp) sc[ct] = mfma16<CT>(qa[pp][st], b, sc[ct]);
        }
    }
    // Causal softmax per token row over this block.
    float mrow[4], lrow[4];
    uint16_t* pw = ps + w * T * VS;  // this wave's [T][VS] for part 0; parts are G * T * VS apart
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = 4 * kg + j;  // token row of the tile
        const int64_t pt = p0 + t0 + i;
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int cr = 16 * ct + n;
            const bool valid = cr < rows && row0 + cr <= pt;
            sv[ct] = valid ? sc[ct][j] * scaling : -INFINITY;
            mx = fmaxf(mx, sv[ct]);
        }
        const float m = row16_max(mx);
        const float msafe = m == -INFINITY ? 0.0f : m;
        float lsum = 0.0f;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const float pv = sv[ct] == -INFINITY ? 0.0f : expf(sv[ct] - msafe);
            lsum += pv;
            uint16_t hh[3];
            split3<CT>(pv, hh);
#pragma unroll
            for (int pp = 0; pp < 3; ++pp) pw[pp * G * T * VS + i * VS + 16 * ct + n] = hh[pp];
        }
        mrow[j] = m;
        lrow[j] = row16_sum(lsum);
    }
    __syncthreads();

    // O = P V: o[dt][j] = O[token row 4 kg + j][dimension 16 dt + n].
    v4f_t o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kst = 0; kst < kSeqBlock / 32; ++kst) {
        v8 pa[3];
#pragma unroll
        for (int pp = 0; pp < 3; ++pp)
            pa[pp] = *reinterpret_cast<const v8*>(pw + pp * G * T * VS + n * VS + 32 * kst + 8 * kg);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const v8 b = *reinterpret_cast<const v8*>(vt + (16 * dt + n) * VS + 32 * kst + 8 * kg);
#pragma unroll
            for (int pp = 0; pp < 3; ++pp) o[dt] = mfma16<CT>(pa[pp], b, o[dt]);
        }
    }
    // Partials of the tokens that reach this block (the merge reads block s of
    // token t only when row0 <= position + t).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t t = t0 + 4 * kg + j;
        const int64_t pt = p0 + t;
        if (t >= tokens || pt < row0 || pt >= max_positions) continue;
        const int64_t pi = attn_part_index(t, h, s, q_heads, blocks);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) part_acc[pi * D + 16 * dt + n] = o[dt][j];
        if (n == 0) {
            part_ml[2 * pi] = mrow[j];
            part_ml[2 * pi + 1] = lrow[j];
        }
    }
}

// ---------------------------------------------------------------------------
// One-token decode attention with the q/k RMSNorm + RoPE + KV append fused in
// (pass 1; k_attention_merge is pass 2). Workgroup (kv head g, 64-row cache
// block s), one wave per q head of the group:
//   - every load is issued first: the block's K and V rows below the token's
//     row p (coalesced 16-byte pieces), each wave's raw q head, and, in the
//     block that holds p, the raw k and v of head g;
//   - K and V rows go to LDS as stored; wave w normalises and rotates q head
//     g * G + w into LDS; in p's block wave 0 rotates k and wave G - 1 (wave 0
//     when G == 1) copies v into LDS row p - 64 s and into cache row p;
//   - after one barrier lane j scores row 64 s + j (K row from LDS, q
//     broadcast), the wave forms its softmax partial and lanes over
//     dimensions accumulate P.V from LDS; the partial goes to the workspace.
// Used when head_dim * element bytes <= 256 (the staged block fits LDS
// twice) and G is 1, 2, 4 or 8.

template <int D, int CT, int G>
constexpr size_t decode_attention_lds() {
    return static_cast<size_t>(kSeqBlock + 1) * k_row_bytes<D, CT>() +
           static_cast<size_t>(kSeqBlock + 1) * D * cache_bytes<CT>() + static_cast<size_t>(G) * (D + kSeqBlock) * sizeof(float);
}

template <int D, int CT, int G, bool HALF>
__global__ __launch_bounds__(G * kWave) void k_decode_attention(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, int kv_heads,
    const void* __restrict__ q_norm, const void* __restrict__ k_norm, int ndt, float eps,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table, const int32_t* __restrict__ position,
    int64_t max_positions, char* __restrict__ k_cache, char* __restrict__ v_cache, float scaling,
    float* __restrict__ part_ml, float* __restrict__ part_acc) {
    constexpr int E = D / kWave;
    constexpr int EB = cache_bytes<CT>();
    constexpr int RB = k_row_bytes<D, CT>();   // padded K row in LDS
    constexpr int VRB = D * EB;                // V row in LDS
    constexpr int PIECES = D * EB / 16;        // 16-byte pieces per row
    constexpr int PER_THREAD = kSeqBlock * PIECES / (G * kWave);
    extern __shared__ float lds_raw[];
    char* klds = reinterpret_cast<char*>(lds_raw);   // kSeqBlock rows + one scratch row
    char* vlds = klds + (kSeqBlock + 1) * RB;
    float* qs = reinterpret_cast<float*>(vlds + (kSeqBlock + 1) * VRB);  // [G][D]
    float* ps = qs + G * D;                                             // [G][64]

    const int g = blockIdx.x;
    const int s = blockIdx.y;
    // gridDim.y, from an argument: gridDim is read from the hidden kernel
    // arguments, one more scalar-cache line before the first load.
    const int blocks = static_cast<int>((max_positions + kSeqBlock - 1) / kSeqBlock);
    const int q_heads = kv_heads * G;
    const int w = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);

    // Loads that do not need the position go first: this wave's q head and
    // the k and v of head g, with their norm weights (no branch on the dtype).
    NormRopeIn<D> qin, kin;
    load_norm_rope_in<D>(qin, q + static_cast<int64_t>(g * G + w) * D, q_norm, ndt, lane);
    load_norm_rope_in<D>(kin, k + static_cast<int64_t>(g) * D, k_norm, ndt, lane);
    float vraw[E];
#pragma unroll
    for (int j = 0; j < E; ++j) vraw[j] = v[static_cast<int64_t>(g) * D + lane + kWave * j];

    // The block's K and V rows, loaded whatever the position (rows past the
    // cache's end reload its last row); rows at or past `cached` go to the
    // scratch row. The position and its RoPE entries follow the barrier;
    // nothing is used before all are issued.
    const int64_t row0 = static_cast<int64_t>(s) * kSeqBlock;
    const int64_t head_row0 = static_cast<int64_t>(g) * max_positions;
    u32x4 kp[PER_THREAD], vp[PER_THREAD];
    const int last_row = static_cast<int>(max_positions - 1 - row0);  // >= 0: the block starts in the cache
    const char* kbase = k_cache + (head_row0 + row0) * VRB;
    const char* vbase = v_cache + (head_row0 + row0) * VRB;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = threadIdx.x + i * G * kWave;
        const int r = idx / PIECES, c = idx % PIECES;
        const int rr = r < last_row ? r : last_row;
        kp[i] = *reinterpret_cast<const u32x4*>(kbase + rr * VRB + 16 * c);
        vp[i] = *reinterpret_cast<const u32x4*>(vbase + rr * VRB + 16 * c);
    }
    __builtin_amdgcn_sched_barrier(0);

    // No early exit (it would sink the loads above below the wait for the
    // position): a block past the position runs the arithmetic of a one-row
    // block at row0 and stores nothing; the merge ignores it. The position is
    // read after the scheduling barrier, so every load above is issued before
    // its (scalar) wait.
    const int64_t pos = position[0];
    const bool live = pos >= 0 && pos < max_positions && row0 <= pos;  // uniform
    const int64_t p = live ? pos : row0;
    const bool owns_p = live && p < row0 + kSeqBlock;
    const int rows = live ? static_cast<int>(owns_p ? p - row0 + 1 : kSeqBlock) : 1;  // rows scored
    const int cached = live ? (owns_p ? rows - 1 : rows) : 0;                         // rows read from the cache

    float cs[E], sn[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        const int fi = d < D / 2 ? d : d - D / 2;
        cs[j] = cos_table[p * (D / 2) + fi];
        sn[j] = sin_table[p * (D / 2) + fi];
    }
    // Pin the block loads here: all of them are issued before the first wait.
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) asm volatile("" : "+v"(kp[i]), "+v"(vp[i]));
    float qy[E];
    norm_rope_regs<D>(qin, q_norm != nullptr, ndt, eps, cs, sn, lane, qy);
    // Stage K and V rows below p (the others to the scratch row).
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = threadIdx.x + i * G * kWave;
        const int r = idx / PIECES, c = idx % PIECES;
        const int lr = r < cached ? r : kSeqBlock;
        *reinterpret_cast<u32x4*>(klds + lr * RB + 16 * c) = kp[i];
        *reinterpret_cast<u32x4*>(vlds + lr * VRB + 16 * c) = vp[i];
    }
#pragma unroll
    for (int j = 0; j < E; ++j) qs[w * D + lane + kWave * j] = qy[j];
    // Row p's k and v: every wave forms them (identical values) and writes
    // them to LDS row rows - 1 when this block holds p, else to the scratch
    // row (no branch, so their loads stay ahead of the position wait); wave 0
    // appends k and wave G - 1 appends v to the cache.
    float ky[E];
    norm_rope_regs<D>(kin, k_norm != nullptr, ndt, eps, cs, sn, lane, ky);
    const int nr = owns_p ? rows - 1 : kSeqBlock;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int d = lane + kWave * j;
        nq::store_f32_as(klds + nr * RB, CT, d, ky[j]);
        nq::store_f32_as(vlds + nr * VRB, CT, d, vraw[j]);
    }
    if (owns_p) {
        const int64_t crow = (head_row0 + p) * D;
        if (w == 0) {
#pragma unroll
            for (int j = 0; j < E; ++j) nq::store_f32_as(k_cache, CT, crow + lane + kWave * j, ky[j]);
        }
        if (w == G - 1) {
#pragma unroll
            for (int j = 0; j < E; ++j) nq::store_f32_as(v_cache, CT, crow + lane + kWave * j, vraw[j]);
        }
    }
    __syncthreads();

    // Scores, softmax partial, P.V for q head g * G + w.
    const bool valid = lane < rows;
    const float dot = k_row_dot<D, CT>(klds + (valid ? lane : 0) * RB, qs + w * D);
    const float score = valid ? dot * scaling : -INFINITY;
    const float m = wave_max(score);
    const float pj = valid ? expf(score - m) : 0.0f;
    const float l = wave_sum(pj);
    float* pw = ps + w * kSeqBlock;
    pw[lane] = pj;
    __builtin_amdgcn_wave_barrier();
    // P.V over the scored rows in groups of four, one accumulator per row of
    // the group (four short dependency chains), combined at the end; rows past
    // `rows` read row 0 with weight 0.
    float acc4[4][E];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < E; ++e) acc4[u][e] = 0.0f;
    for (int r0 = 0; r0 < rows; r0 += 4) {
        float pr[4], vv[4][E];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = r0 + u < rows ? r0 + u : 0;
            pr[u] = r0 + u < rows ? pw[r] : 0.0f;
            load_v<E, CT>(vlds + r * VRB + lane * E * EB, vv[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < E; ++e) acc4[u][e] = fmaf(pr[u], vv[u][e], acc4[u][e]);
    }
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = (acc4[0][e] + acc4[1][e]) + (acc4[2][e] + acc4[3][e]);
    // A block past the token's row stores the neutral partial (max -inf, sum
    // 0, accumulators 0), which adds nothing to a merge over every block.
    // HALF: the block's output acc / sum as fp16 in place of the accumulators.
    const int h = g * G + w;
    const int64_t pi = attn_part_index(0, h, s, q_heads, blocks);
    if (lane == 0) {
        part_ml[2 * pi] = live ? m : -INFINITY;
        part_ml[2 * pi + 1] = live ? l : 0.0f;
    }
    const float inv = HALF && live ? 1.0f / l : 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if constexpr (HALF)
            reinterpret_cast<_Float16*>(part_acc)[pi * D + lane * E + e] =
                static_cast<_Float16>(live ? acc[e] * inv : 0.0f);
        else
            part_acc[pi * D + lane * E + e] = live ? acc[e] : 0.0f;
    }
}

// ---------------------------------------------------------------------------
// SiLU-gated product.

__global__ __launch_bounds__(kRowThreads) void k_silu_mul(const float* __restrict__ gate, const float* __restrict__ up,
                                                          int64_t n, void* __restrict__ out, int odt) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * kRowThreads + threadIdx.x) * 8;
    if (i >= n) return;
    float gv[8], uv[8];
    load8(gate, NQ_DTYPE_F32, i, gv);
    load8(up, NQ_DTYPE_F32, i, uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) gv[j] = __fmul_rn(gv[j] / (1.0f + expf(-gv[j])), uv[j]);
    store8(out, odt, i, gv);
}

// ---------------------------------------------------------------------------
// Output projection: logits = W x for one token, W bf16 [vocab, hidden].
// Wave w of workgroup b owns RW = kProjLoads / NCH consecutive rows; lane l
// reads 8-element chunk k * 64 + l of each row for k < NCH, so all of a
// wave's RW * NCH 16-byte loads are issued before the first is used. x is
// staged in LDS as fp32. Each workgroup also writes its best (logit, index)
// as one orderable 64-bit key.

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<uint64_t>(u) << 32) | static_cast<uint64_t>(0xffffffffu - idx);
}

template <int NCH>
__global__ __launch_bounds__(kProjWaves * kWave) void k_output_projection(const void* __restrict__ x, int xdt,
                                                                          const uint16_t* __restrict__ weight,
                                                                          int64_t vocab, int64_t hidden,
                                                                          float* __restrict__ logits,
                                                                          uint64_t* __restrict__ partial) {
    constexpr int RW = kProjLoads / NCH;
    __shared__ float xs[NCH * kWave * 8];
    __shared__ uint64_t best[kProjWaves];
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x / kWave;
    const int64_t chunks = hidden / 8;
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kProjWaves + w) * RW;

    // Weight loads first (clamped rows and chunks; masked in the arithmetic),
    // nontemporal: the matrix streams through once per token. Measured on
    // MI355X at 151936 x 4096: 193 us (6.4 TB/s) against 215 us with plain
    // loads, the same logits bit for bit.
    uint4 wv[RW][NCH];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int64_t row = row0 + r < vocab ? row0 + r : vocab - 1;
#pragma unroll
        for (int kk = 0; kk < NCH; ++kk) {
            const int64_t c = kk * kWave + lane;
            const int64_t cc = c < chunks ? c : chunks - 1;
            const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(weight + row * hidden + cc * 8));
            wv[r][kk] = make_uint4(t.x, t.y, t.z, t.w);
        }
    }
    for (int64_t i = threadIdx.x * 8; i < static_cast<int64_t>(NCH) * kWave * 8; i += kProjWaves * kWave * 8) {
        float v[8];
        if (i < hidden) {
            load8(x, xdt, i, v);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = 0.0f;
        }
        float4* d = reinterpret_cast<float4*>(&xs[i]);
        d[0] = make_float4(v[0], v[1], v[2], v[3]);
        d[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();

    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < NCH; ++kk) {
        const int64_t c = kk * kWave + lane;
        const float4 xa = *reinterpret_cast<const float4*>(&xs[c * 8]);
        const float4 xb = *reinterpret_cast<const float4*>(&xs[c * 8 + 4]);
        const bool live = c < chunks;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const uint4 u = wv[r][kk];
            float a = acc[r];
            a = fmaf(bf16_lo(u.x), xa.x, a);
            a = fmaf(bf16_hi(u.x), xa.y, a);
            a = fmaf(bf16_lo(u.y), xa.z, a);
            a = fmaf(bf16_hi(u.y), xa.w, a);
            a = fmaf(bf16_lo(u.z), xb.x, a);
            a = fmaf(bf16_hi(u.z), xb.y, a);
            a = fmaf(bf16_lo(u.w), xb.z, a);
            a = fmaf(bf16_hi(u.w), xb.w, a);
            acc[r] = live ? a : acc[r];
        }
    }
    uint64_t key = 0;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const float sum = wave_sum(acc[r]);
        const int64_t row = row0 + r;
        if (row < vocab) {
            if (lane == r) logits[row] = sum;
            const uint64_t kr = argmax_key(sum, static_cast<uint32_t>(row));
            key = kr > key ? kr : key;
        }
    }
    if (lane == 0) best[w] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = best[0];
#pragma unroll
        for (int i = 1; i < kProjWaves; ++i) b = best[i] > b ? best[i] : b;
        partial[blockIdx.x] = b;
    }
}

__global__ __launch_bounds__(1024) void k_greedy_select(const uint64_t* __restrict__ partial, int64_t count,
                                                        int64_t* __restrict__ token_out, int64_t* __restrict__ history,
                                                        int64_t history_capacity, int32_t* __restrict__ step,
                                                        int32_t* __restrict__ position) {
    constexpr int kThreads = 1024;  // the launch's block size
    constexpr int kRound = 16;      // loads in flight per thread
    __shared__ uint64_t red[kThreads / kWave];
    // Rounds of kRound independent loads per thread (indices clamped to the
    // last partial, whose repeats do not change the maximum), so a round
    // costs one memory round trip: 9496 partials for a 151936-row vocabulary
    // are one round instead of ten dependent loads.
    uint64_t key = 0;
    for (int64_t base = threadIdx.x; base < count; base += static_cast<int64_t>(kThreads) * kRound) {
        uint64_t v[kRound];
#pragma unroll
        for (int j = 0; j < kRound; ++j) {
            const int64_t i = base + static_cast<int64_t>(j) * kThreads;
            v[j] = partial[i < count ? i : count - 1];
        }
#pragma unroll
        for (int j = 0; j < kRound; ++j) key = v[j] > key ? v[j] : key;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(key), o, kWave);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(key >> 32), o, kWave);
        const uint64_t other = (static_cast<uint64_t>(hi) << 32) | lo;
        key = other > key ? other : key;
    }
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = red[0];
        for (int i = 1; i < kThreads / kWave; ++i) b = red[i] > b ? red[i] : b;
        const int64_t token = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(b & 0xffffffffu));
        token_out[0] = token;
        if (history && step) {
            const int32_t k = step[0];
            if (k >= 0 && k < history_capacity) history[k] = token;
            step[0] = k + 1;
        }
        if (position) position[0] += 1;
    }
}

// ---------------------------------------------------------------------------
// Host helpers.

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool float_code(int d) { return nq::is_float_dtype(d); }
hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int proj_chunks_per_lane(int64_t hidden) {
    for (int n : {1, 2, 4, 8, 16})
        if (static_cast<int64_t>(n) * kWave * 8 >= hidden) return n;
    return 0;
}

int64_t proj_workgroups(int64_t vocab, int64_t hidden) {
    const int nch = proj_chunks_per_lane(hidden);
    if (nch == 0) return -1;
    const int64_t rows = static_cast<int64_t>(kProjWaves) * (kProjLoads / nch);
    return (vocab + rows - 1) / rows;
}

int attention_blocks(int64_t max_positions) { return static_cast<int>((max_positions + kSeqBlock - 1) / kSeqBlock); }

template <int D, int CT>
int launch_attention(const float* q, const void* kc, const void* vc, int64_t tokens, int q_heads, int kv_heads,
                     const int32_t* position, int64_t max_positions, float scaling, void* out, int odt, float* ml,
                     float* acc, hipStream_t st) {
    const int group = q_heads / kv_heads;
    const int blocks = attention_blocks(max_positions);
    if constexpr (D == 128 && CT != NQ_DTYPE_F32) {
        if (group == kMfmaHeads && tokens > 1) {
            const int64_t qblocks = (tokens + kPromptTile - 1) / kPromptTile;
            if (qblocks * kv_heads > 0x7fffffff) return NQ_ERR_SHAPE;
            dim3 grid(static_cast<unsigned>(qblocks * kv_heads), static_cast<unsigned>(blocks));
            hipLaunchKernelGGL((k_prompt_attention_mfma<CT>), grid, dim3(kMfmaHeads * kWave),
                               prompt_attention_mfma_lds<CT>(), st, q, static_cast<const char*>(kc),
                               static_cast<const char*>(vc), tokens, kv_heads, position, max_positions, scaling, ml,
                               acc);
            if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
            hipLaunchKernelGGL(k_attention_merge<D>, dim3(q_heads, static_cast<unsigned>(tokens)), dim3(D), 0, st, ml,
                               acc, q_heads, blocks, kSeqBlock, position, max_positions, out, odt);
            return nq::launch_status();
        }
    }
    const int qt = tokens == 1 ? 1 : 16;
    const int64_t qblocks = (tokens + qt - 1) / qt;
    const size_t lds = attention_lds<D, CT>(group);
    if (lds > 64 * 1024) return NQ_ERR_UNSUPPORTED;
    if (qblocks * kv_heads > 0x7fffffff) return NQ_ERR_SHAPE;
    dim3 grid(static_cast<unsigned>(qblocks * kv_heads), static_cast<unsigned>(blocks));
    hipLaunchKernelGGL((k_attention_blocks<D, CT>), grid, dim3(group * kWave), lds, st, q,
                       static_cast<const char*>(kc), static_cast<const char*>(vc), tokens, q_heads, kv_heads, qt,
                       position, max_positions, scaling, ml, acc);
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL(k_attention_merge<D>, dim3(q_heads, static_cast<unsigned>(tokens)), dim3(D), 0, st, ml, acc,
                       q_heads, blocks, kSeqBlock, position, max_positions, out, odt);
    return nq::launch_status();
}

template <int D>
int launch_attention_for(int cdt, const float* q, const void* kc, const void* vc, int64_t tokens, int q_heads,
                         int kv_heads, const int32_t* position, int64_t max_positions, float scaling, void* out,
                         int odt, float* ml, float* acc, hipStream_t st) {
    switch (cdt) {
        case NQ_DTYPE_F32:
            return launch_attention<D, NQ_DTYPE_F32>(q, kc, vc, tokens, q_heads, kv_heads, position, max_positions,
                                                     scaling, out, odt, ml, acc, st);
        case NQ_DTYPE_F16:
            return launch_attention<D, NQ_DTYPE_F16>(q, kc, vc, tokens, q_heads, kv_heads, position, max_positions,
                                                     scaling, out, odt, ml, acc, st);
        case NQ_DTYPE_BF16:
            return launch_attention<D, NQ_DTYPE_BF16>(q, kc, vc, tokens, q_heads, kv_heads, position, max_positions,
                                                      scaling, out, odt, ml, acc, st);
        default:
            return NQ_ERR_DTYPE;
    }
}

bool decode_fast_path(int head_dim, int cdt, int group) {
    const int eb = cdt == NQ_DTYPE_F32 ? 4 : 2;
    return head_dim * eb <= 256 && (group == 1 || group == 2 || group == 4 || group == 8);
}

int64_t round16(int64_t bytes) { return (bytes + 15) / 16 * 16; }

template <int D, int CT, int G>
int launch_decode_attention_g(const float* q, const float* k, const float* v, int kv_heads, const void* qn,
                              const void* kn, int ndt, float eps, const float* cs, const float* sn,
                              const int32_t* position, int64_t max_positions, void* kc, void* vc, float scaling,
                              void* out, int odt, float* ml, float* acc, bool merge, hipStream_t st) {
    const int blocks = attention_blocks(max_positions);
    // The partials form (no merge here) stores each block's output in fp16 for
    // the projection input that merges them; the merge below reads fp32 sums.
    if constexpr (D == 128 && G == kMfmaHeads && CT != NQ_DTYPE_F32) {
        if (merge)
            hipLaunchKernelGGL((k_decode_attention_mfma<CT, false>), dim3(kv_heads, blocks), dim3(G * kWave),
                               decode_attention_mfma_lds<CT>(), st, q, k, v, kv_heads, qn, kn, ndt, eps, cs, sn,
                               position, max_positions, static_cast<char*>(kc), static_cast<char*>(vc), scaling, ml,
                               acc);
        else
            hipLaunchKernelGGL((k_decode_attention_mfma<CT, true>), dim3(kv_heads, blocks), dim3(G * kWave),
                               decode_attention_mfma_lds<CT>(), st, q, k, v, kv_heads, qn, kn, ndt, eps, cs, sn,
                               position, max_positions, static_cast<char*>(kc), static_cast<char*>(vc), scaling, ml,
                               acc);
    } else {
        const size_t lds = decode_attention_lds<D, CT, G>();
        if (lds > 64 * 1024) return NQ_ERR_UNSUPPORTED;
        if (merge)
            hipLaunchKernelGGL((k_decode_attention<D, CT, G, false>), dim3(kv_heads, blocks), dim3(G * kWave), lds,
                               st, q, k, v, kv_heads, qn, kn, ndt, eps, cs, sn, position, max_positions,
                               static_cast<char*>(kc), static_cast<char*>(vc), scaling, ml, acc);
        else
            hipLaunchKernelGGL((k_decode_attention<D, CT, G, true>), dim3(kv_heads, blocks), dim3(G * kWave), lds,
                               st, q, k, v, kv_heads, qn, kn, ndt, eps, cs, sn, position, max_positions,
                               static_cast<char*>(kc), static_cast<char*>(vc), scaling, ml, acc);
    }
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    if (!merge) return NQ_OK;  // the partials stay in the workspace
    hipLaunchKernelGGL(k_attention_merge<D>, dim3(kv_heads * G, 1), dim3(D), 0, st, ml, acc, kv_heads * G, blocks,
                       kSeqBlock, position, max_positions, out, odt);
    return nq::launch_status();
}

template <int D, int CT>
int launch_decode_attention_ct(int group, const float* q, const float* k, const float* v, int kv_heads, const void* qn,
                               const void* kn, int ndt, float eps, const float* cs, const float* sn,
                               const int32_t* position, int64_t max_positions, void* kc, void* vc, float scaling,
                               void* out, int odt, float* ml, float* acc, bool merge, hipStream_t st) {
#define NQ_DA(G)                                                                                                   \
    return launch_decode_attention_g<D, CT, G>(q, k, v, kv_heads, qn, kn, ndt, eps, cs, sn, position, max_positions, \
                                               kc, vc, scaling, out, odt, ml, acc, merge, st)
    switch (group) {
        case 1: NQ_DA(1);
        case 2: NQ_DA(2);
        case 4: NQ_DA(4);
        case 8: NQ_DA(8);
        default: return NQ_ERR_UNSUPPORTED;
    }
#undef NQ_DA
}

}  // namespace

extern "C" int nq_embedding(const int64_t* ids, int64_t tokens, const void* table, int32_t table_dtype, int64_t vocab,
                            int64_t hidden, const float* scale, float* out, void* stream) {
    if (!ids || !table || !out) return NQ_ERR_ARGUMENT;
    if (!float_code(table_dtype)) return NQ_ERR_DTYPE;
    if (tokens <= 0 || tokens > 0x7fffffff || vocab <= 0 || hidden <= 0 || hidden % 8) return NQ_ERR_SHAPE;
    if (!aligned16(table) || !aligned16(out)) return NQ_ERR_ALIGNMENT;
    hipLaunchKernelGGL(k_embedding, dim3(static_cast<unsigned>(tokens)), dim3(kRowThreads), 0, as_stream(stream), ids,
                       table, table_dtype, vocab, hidden, scale, out, nullptr);
    return nq::launch_status();
}

extern "C" int nq_embedding_slots(const int64_t* ids, int64_t tokens, const void* table, int32_t table_dtype,
                                  int64_t vocab, int64_t hidden, const float* scale, float* out, float* slots,
                                  void* stream) {
    if (!ids || !table || !out || !slots) return NQ_ERR_ARGUMENT;
    if (!float_code(table_dtype)) return NQ_ERR_DTYPE;
    if (tokens <= 0 || tokens > 0x7fffffff || vocab <= 0 || hidden <= 0 || hidden % 16) return NQ_ERR_SHAPE;
    if (!aligned16(table) || !aligned16(out)) return NQ_ERR_ALIGNMENT;
    hipLaunchKernelGGL(k_embedding, dim3(static_cast<unsigned>(tokens)), dim3(kRowThreads), 0, as_stream(stream), ids,
                       table, table_dtype, vocab, hidden, scale, out, slots);
    return nq::launch_status();
}

extern "C" int nq_add_rmsnorm(float* residual, const void* delta, int32_t delta_dtype, const void* weight,
                              int32_t weight_dtype, float eps, int64_t tokens, int64_t hidden, void* out,
                              int32_t out_dtype, void* stream) {
    if (!residual || !weight || !out) return NQ_ERR_ARGUMENT;
    if ((delta && !float_code(delta_dtype)) || !float_code(weight_dtype) || !float_code(out_dtype)) return NQ_ERR_DTYPE;
    if (tokens <= 0 || tokens > 0x7fffffff || hidden <= 0 || hidden % 8 || hidden > kNormThreads * 32)
        return NQ_ERR_SHAPE;
    if (!(eps >= 0.0f)) return NQ_ERR_ARGUMENT;
    if (!aligned16(residual) || (delta && !aligned16(delta)) || !aligned16(weight) || !aligned16(out))
        return NQ_ERR_ALIGNMENT;
    const dim3 grid(static_cast<unsigned>(tokens)), block(kNormThreads);
    hipStream_t st = as_stream(stream);
    if (hidden <= kNormThreads * 8) {
        hipLaunchKernelGGL(k_add_rmsnorm<1>, grid, block, 0, st, residual, delta, delta_dtype, weight, weight_dtype,
                           eps, hidden, out, out_dtype);
    } else if (hidden <= kNormThreads * 16) {
        hipLaunchKernelGGL(k_add_rmsnorm<2>, grid, block, 0, st, residual, delta, delta_dtype, weight, weight_dtype,
                           eps, hidden, out, out_dtype);
    } else {
        hipLaunchKernelGGL(k_add_rmsnorm<4>, grid, block, 0, st, residual, delta, delta_dtype, weight, weight_dtype,
                           eps, hidden, out, out_dtype);
    }
    return nq::launch_status();
}

extern "C" int nq_qk_norm_rope_cache(const float* q, const float* k, const float* v, int64_t tokens, int32_t q_heads,
                                     int32_t kv_heads, int32_t head_dim, const void* q_norm, const void* k_norm,
                                     int32_t norm_dtype, float eps, const float* cos_table, const float* sin_table,
                                     const int32_t* position, int64_t max_positions, float* q_out, void* k_cache,
                                     void* v_cache, int32_t cache_dtype, void* stream) {
    if (!q || !k || !v || !cos_table || !sin_table || !position || !q_out || !k_cache || !v_cache)
        return NQ_ERR_ARGUMENT;
    if (((q_norm || k_norm) && !float_code(norm_dtype)) || !float_code(cache_dtype)) return NQ_ERR_DTYPE;
    if (tokens <= 0 || tokens > 0x7fffffff || q_heads <= 0 || kv_heads <= 0 || q_heads + kv_heads > 65535 ||
        max_positions <= 0)
        return NQ_ERR_SHAPE;
    if (!(eps >= 0.0f)) return NQ_ERR_ARGUMENT;
    dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(q_heads + kv_heads));
    hipStream_t st = as_stream(stream);
#define NQ_QKR(D)                                                                                                     \
    hipLaunchKernelGGL(k_qk_norm_rope_cache<D>, grid, dim3(kWave), 0, st, q, k, v, q_heads, kv_heads, q_norm, k_norm, \
                       norm_dtype, eps, cos_table, sin_table, position, max_positions, q_out, k_cache, v_cache,        \
                       cache_dtype)
    switch (head_dim) {
        case 64: NQ_QKR(64); break;
        case 128: NQ_QKR(128); break;
        case 256: NQ_QKR(256); break;
        default: return NQ_ERR_SHAPE;
    }
#undef NQ_QKR
    return nq::launch_status();
}

extern "C" int64_t nq_attention_workspace_bytes(int64_t tokens, int32_t q_heads, int32_t head_dim,
                                                int64_t max_positions) {
    if (tokens <= 0 || q_heads <= 0 || head_dim <= 0 || max_positions <= 0) return -1;
    const int64_t parts = tokens * q_heads * attention_blocks(max_positions);
    return parts * (2 + head_dim) * static_cast<int64_t>(sizeof(float));
}

extern "C" int nq_attention(const float* q, const void* k_cache, const void* v_cache, int32_t cache_dtype,
                            int64_t tokens, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                            const int32_t* position, int64_t max_positions, float scaling, void* out, int32_t out_dtype,
                            void* workspace, int64_t workspace_bytes, void* stream) {
    if (!q || !k_cache || !v_cache || !position || !out || !workspace) return NQ_ERR_ARGUMENT;
    if (!float_code(cache_dtype) || !float_code(out_dtype)) return NQ_ERR_DTYPE;
    if (tokens <= 0 || tokens > 65535 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads ||
        q_heads / kv_heads > 16 || max_positions <= 0 || attention_blocks(max_positions) > 65535)
        return NQ_ERR_SHAPE;
    if (!(scaling > 0.0f)) return NQ_ERR_ARGUMENT;
    if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(workspace)) return NQ_ERR_ALIGNMENT;
    const int64_t need = nq_attention_workspace_bytes(tokens, q_heads, head_dim, max_positions);
    if (need < 0) return NQ_ERR_SHAPE;
    if (workspace_bytes < need) return NQ_ERR_WORKSPACE;
    const int64_t parts = tokens * q_heads * attention_blocks(max_positions);
    float* ml = static_cast<float*>(workspace);
    float* acc = ml + 2 * parts;
    hipStream_t st = as_stream(stream);
    switch (head_dim) {
        case 64:
            return launch_attention_for<64>(cache_dtype, q, k_cache, v_cache, tokens, q_heads, kv_heads, position,
                                            max_positions, scaling, out, out_dtype, ml, acc, st);
        case 128:
            return launch_attention_for<128>(cache_dtype, q, k_cache, v_cache, tokens, q_heads, kv_heads, position,
                                             max_positions, scaling, out, out_dtype, ml, acc, st);
        case 256:
            return launch_attention_for<256>(cache_dtype, q, k_cache, v_cache, tokens, q_heads, kv_heads, position,
                                             max_positions, scaling, out, out_dtype, ml, acc, st);
        default:
            return NQ_ERR_SHAPE;
    }
}

extern "C" int nq_silu_mul(const float* gate, const float* up, int64_t n, void* out, int32_t out_dtype, void* stream) {
    if (!gate || !up || !out) return NQ_ERR_ARGUMENT;
    if (!float_code(out_dtype)) return NQ_ERR_DTYPE;
    if (n <= 0 || n % 8) return NQ_ERR_SHAPE;
    if (!aligned16(gate) || !aligned16(up) || !aligned16(out)) return NQ_ERR_ALIGNMENT;
    const int64_t groups = (n / 8 + kRowThreads - 1) / kRowThreads;
    if (groups > 0x7fffffff) return NQ_ERR_SHAPE;
    hipLaunchKernelGGL(k_silu_mul, dim3(static_cast<unsigned>(groups)), dim3(kRowThreads), 0, as_stream(stream), gate,
                       up, n, out, out_dtype);
    return nq::launch_status();
}

extern "C" int64_t nq_output_projection_workspace_bytes(int64_t vocab, int64_t hidden) {
    if (vocab <= 0 || hidden <= 0 || hidden % 8) return -1;
    const int64_t wgs = proj_workgroups(vocab, hidden);
    return wgs < 0 ? -1 : wgs * static_cast<int64_t>(sizeof(uint64_t));
}

extern "C" int nq_output_projection(const void* x, int32_t x_dtype, const void* weight, int64_t vocab, int64_t hidden,
                                    float* logits, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!x || !weight || !logits || !workspace) return NQ_ERR_ARGUMENT;
    if (x_dtype != NQ_DTYPE_F32 && x_dtype != NQ_DTYPE_BF16) return NQ_ERR_DTYPE;
    if (vocab <= 0 || vocab > 0x7fffffffLL || hidden <= 0 || hidden % 8 || hidden > 16 * kWave * 8)
        return NQ_ERR_SHAPE;
    if (!aligned16(x) || !aligned16(weight) || !aligned16(workspace)) return NQ_ERR_ALIGNMENT;
    const int64_t need = nq_output_projection_workspace_bytes(vocab, hidden);
    if (need < 0) return NQ_ERR_SHAPE;
    if (workspace_bytes < need) return NQ_ERR_WORKSPACE;
    const int64_t wgs = proj_workgroups(vocab, hidden);
    hipStream_t st = as_stream(stream);
    const uint16_t* w = static_cast<const uint16_t*>(weight);
    uint64_t* part = static_cast<uint64_t*>(workspace);
    const dim3 grid(static_cast<unsigned>(wgs)), block(kProjWaves * kWave);
    switch (proj_chunks_per_lane(hidden)) {
        case 1: hipLaunchKernelGGL(k_output_projection<1>, grid, block, 0, st, x, x_dtype, w, vocab, hidden, logits, part); break;
        case 2: hipLaunchKernelGGL(k_output_projection<2>, grid, block, 0, st, x, x_dtype, w, vocab, hidden, logits, part); break;
        case 4: hipLaunchKernelGGL(k_output_projection<4>, grid, block, 0, st, x, x_dtype, w, vocab, hidden, logits, part); break;
        case 8: hipLaunchKernelGGL(k_output_projection<8>, grid, block, 0, st, x, x_dtype, w, vocab, hidden, logits, part); break;
        case 16: hipLaunchKernelGGL(k_output_projection<16>, grid, block, 0, st, x, x_dtype, w, vocab, hidden, logits, part); break;
        default: return NQ_ERR_SHAPE;
    }
    return nq::launch_status();
}

extern "C" int nq_greedy_select(const void* workspace, int64_t vocab, int64_t hidden, int64_t* token_out,
                                int64_t* history, int64_t history_capacity, int32_t* step, int32_t* position,
                                void* stream) {
    if (!workspace || !token_out) return NQ_ERR_ARGUMENT;
    if ((history != nullptr) != (step != nullptr) || history_capacity < 0) return NQ_ERR_ARGUMENT;
    const int64_t wgs = vocab > 0 && vocab <= 0x7fffffffLL && hidden > 0 && hidden % 8 == 0 ? proj_workgroups(vocab, hidden) : -1;
    if (wgs <= 0) return NQ_ERR_SHAPE;
    hipLaunchKernelGGL(k_greedy_select, dim3(1), dim3(1024), 0, as_stream(stream),
                       static_cast<const uint64_t*>(workspace), wgs, token_out, history, history_capacity, step,
                       position);
    return nq::launch_status();
}

extern "C" int64_t nq_decode_attention_workspace_bytes(int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                                       int32_t cache_dtype, int64_t max_positions) {
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || head_dim <= 0 || max_positions <= 0) return -1;
    if (decode_fast_path(head_dim, cache_dtype, q_heads / kv_heads))
        return nq_attention_workspace_bytes(1, q_heads, head_dim, max_positions);
    const int64_t attn = nq_attention_workspace_bytes(1, q_heads, head_dim, max_positions);
    return attn < 0 ? -1 : round16(static_cast<int64_t>(q_heads) * head_dim * 4) + attn;
}

namespace {

// nq_decode_attention (merge) and nq_decode_attention_partials (!merge: pass 1
// only, out unused).
int decode_attention(const float* q, const float* k, const float* v, int32_t q_heads, int32_t kv_heads,
                     int32_t head_dim, const void* q_norm, const void* k_norm, int32_t norm_dtype, float eps,
                     const float* cos_table, const float* sin_table, const int32_t* position, int64_t max_positions,
                     void* k_cache, void* v_cache, int32_t cache_dtype, float scaling, void* out, int32_t out_dtype,
                     bool merge, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !cos_table || !sin_table || !position || !k_cache || !v_cache || (merge && !out) || !workspace)
        return NQ_ERR_ARGUMENT;
    if (((q_norm || k_norm) && !float_code(norm_dtype)) || !float_code(cache_dtype) || (merge && !float_code(out_dtype)))
        return NQ_ERR_DTYPE;
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || max_positions <= 0 ||
        attention_blocks(max_positions) > 65535)
        return NQ_ERR_SHAPE;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return NQ_ERR_SHAPE;
    if (!(eps >= 0.0f) || !(scaling > 0.0f)) return NQ_ERR_ARGUMENT;
    if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(workspace)) return NQ_ERR_ALIGNMENT;
    const int64_t need = nq_decode_attention_workspace_bytes(q_heads, kv_heads, head_dim, cache_dtype, max_positions);
    if (need < 0) return NQ_ERR_SHAPE;
    if (workspace_bytes < need) return NQ_ERR_WORKSPACE;
    hipStream_t st = as_stream(stream);
    const int group = q_heads / kv_heads;
    if (!decode_fast_path(head_dim, cache_dtype, group)) {
        if (!merge) return NQ_ERR_UNSUPPORTED;  // the partials exist only in the one-pass form
        // Unfused: rotate q into the workspace and append k/v, then attend.
        float* q_rot = static_cast<float*>(workspace);
        char* attn_ws = static_cast<char*>(workspace) + round16(static_cast<int64_t>(q_heads) * head_dim * 4);
        int rc = nq_qk_norm_rope_cache(q, k, v, 1, q_heads, kv_heads, head_dim, q_norm, k_norm, norm_dtype, eps,
                                       cos_table, sin_table, position, max_positions, q_rot, k_cache, v_cache,
                                       cache_dtype, stream);
        if (rc != NQ_OK) return rc;
        return nq_attention(q_rot, k_cache, v_cache, cache_dtype, 1, q_heads, kv_heads, head_dim, position,
                            max_positions, scaling, out, out_dtype, attn_ws,
                            workspace_bytes - round16(static_cast<int64_t>(q_heads) * head_dim * 4), stream);
    }
    float* ml = static_cast<float*>(workspace);
    float* acc = ml + 2 * static_cast<int64_t>(q_heads) * attention_blocks(max_positions);
#define NQ_DAC(D, CT)                                                                                             \
    return launch_decode_attention_ct<D, CT>(group, q, k, v, kv_heads, q_norm, k_norm, norm_dtype, eps, cos_table, \
                                             sin_table, position, max_positions, k_cache, v_cache, scaling, out,   \
                                             out_dtype, ml, acc, merge, st)
    if (head_dim == 64) {
        if (cache_dtype == NQ_DTYPE_F32) NQ_DAC(64, NQ_DTYPE_F32);
        if (cache_dtype == NQ_DTYPE_F16) NQ_DAC(64, NQ_DTYPE_F16);
        NQ_DAC(64, NQ_DTYPE_BF16);
    }
    if (cache_dtype == NQ_DTYPE_F16) NQ_DAC(128, NQ_DTYPE_F16);
    NQ_DAC(128, NQ_DTYPE_BF16);
#undef NQ_DAC
}

}  // namespace

extern "C" int nq_decode_attention(const float* q, const float* k, const float* v, int32_t q_heads, int32_t kv_heads,
                                   int32_t head_dim, const void* q_norm, const void* k_norm, int32_t norm_dtype,
                                   float eps, const float* cos_table, const float* sin_table, const int32_t* position,
                                   int64_t max_positions, void* k_cache, void* v_cache, int32_t cache_dtype,
                                   float scaling, void* out, int32_t out_dtype, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
    return decode_attention(q, k, v, q_heads, kv_heads, head_dim, q_norm, k_norm, norm_dtype, eps, cos_table,
                            sin_table, position, max_positions, k_cache, v_cache, cache_dtype, scaling, out, out_dtype,
                            true, workspace, workspace_bytes, stream);
}

extern "C" int nq_decode_attention_partials(const float* q, const float* k, const float* v, int32_t q_heads,
                                            int32_t kv_heads, int32_t head_dim, const void* q_norm,
                                            const void* k_norm, int32_t norm_dtype, float eps,
                                            const float* cos_table, const float* sin_table,
                                            const int32_t* position, int64_t max_positions, void* k_cache,
                                            void* v_cache, int32_t cache_dtype, float scaling, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
    return decode_attention(q, k, v, q_heads, kv_heads, head_dim, q_norm, k_norm, norm_dtype, eps, cos_table,
                            sin_table, position, max_positions, k_cache, v_cache, cache_dtype, scaling, nullptr,
                            NQ_DTYPE_F32, false, workspace, workspace_bytes, stream);
}

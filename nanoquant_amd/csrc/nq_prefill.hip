// Prefill path (tokens > 16) for the packed binary low-rank linear on gfx950:
// two dense sign GEMMs on v_mfma_f32_32x32x16_f16.
//
//   k_prep_rows:  xs16[t, :] = fp16(x[t, :] * s_in * 2^e_t)       (exact power of
//                 two per row from max |x * s_in|, so fp16 cannot overflow),
//                 and 2^f_t from the bound |lm[t, r]| <= max|s_mid| * Σ_i |x s_in|
//   GEMM 1:       lm16[t, r] = fp16(2^f_t * s_mid[r] * (xs16 · V±1ᵀ)[t, r] / 2^e_t)
//   GEMM 2:       y[t, o]    = s_out[o] * (lm16 · U±1ᵀ)[t, o] / 2^f_t
//                              + Σ_k x[t, idx_k] W_sal[o, k] (* scale_k) + bias[o]
//
// The bound puts every lm16 value at or below 2^14, inside the fp16 range,
// and values far below the bound keep fp16's relative precision down to
// 2^-14 (they lie within a few binades of it for any real row), so the
// rank intermediate never takes a pass of its own.
//
// The sign operand comes straight from the decode tile layout (16-row tiles;
// in 128-column block kb = 4c + d a lane's word d of chunk c holds, at bit
// 8b + m, column 128kb + 16m + 4g + b for lane group g). A 32 x 32 x 16 MFMA
// over 16-column slice m takes, in lane 32h + r, the 8 k slots of B column r
// (sign row r of a 32-row pair of tiles) for columns 16m + 8h + [0, 8): the
// words of lane groups 2h and 2h + 1 of row r hold exactly those columns, so
// each lane loads two words per tile pair and 128-column block and expands
// them in registers (one shift and one and_or per fp16 pair). k_prep_rows
// stores activation rows with columns 1 and 2 of every group of four swapped,
// which puts the A operand's 8 k slots in the same order: one 16-byte LDS
// read per A fragment. Each expanded B fragment serves two A fragments and
// each A fragment two B fragments.
//
// Block tile 128 (tokens) x 128 (sign rows), 4 waves in a 2 x 2 grid, each
// wave 64 x 64 = 2 x 2 MFMA tiles of 32 x 32 accumulated in fp32 (or 128 x
// 256, waves side by side, for large GEMMs). The activation tile (128 x 128
// fp16, 16-byte chunks XOR-swizzled by row) is double-buffered in LDS and
// moved there by global_load_lds_dwordx4, so the next 128-column block is in
// flight during the current block's MFMAs without holding registers; one
// barrier per block orders the buffer swap. Within a block the eight
// 16-column slices are software-pipelined: slice m's MFMAs issue while slice
// m + 1's A fragments are read and its signs expanded.
//
// Split operands (nq_linear_desc.prefill_operands = NQ_PREFILL_FP16_SPLIT):
// every prepared row and the rank intermediate carry, per 128-column block,
// the fp16 values hi = fp16(v) and then the fp16 remainders lo = fp16(v - hi)
// (v - hi is exact in fp32), so a row of K columns is 2K fp16 wide. Each K
// step then moves both 128-column planes into LDS and issues every MFMA
// twice, hi then lo into the same accumulator: about 22 bits per operand
// instead of 11, against twice the MFMA and activation work (the signs are
// expanded once).
//
// Split K: when a GEMM has too few (token, sign-row) tiles to fill the GPU,
// its K blocks are split into slices of at least two, each workgroup writes
// its raw fp32 accumulators to partial[slice][t][n], and k_reduce_splits, one
// thread per output element, sums them in slice order (deterministic) and
// applies the epilogue. A batched call runs up to eight GEMMs of one phase in
// one launch, their (column block, slice) ranges concatenated along grid x.
#include "nq_prefill.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBlock = 256;
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 128;                 // one superchunk per K step
constexpr int kTileRows = 16;
constexpr int kPrefillBatch = 8;         // members of one batched call
// s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15): wait for this wave's vector
// memory operations only (gfx9 encoding), as a builtin the compiler's own
// wait tracking takes into account.
constexpr int kWaitVmcnt0 = 0x0F70;

__device__ __forceinline__ float exp2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

__device__ __forceinline__ float range_scale(float bound) {
    if (!(bound > 0.0f)) return 1.0f;
    int e = static_cast<int>((__float_as_uint(bound) >> 23) & 0xff) - 127;
    e = 13 - (e < -126 ? -126 : e);
    e = e > 100 ? 100 : (e < -100 ? -100 : e);
    return exp2i(e);
}

// Scale of a prepared row from its max |a s| and its sum of |a s|. The sum
// is NaN or +Inf exactly when the row holds a NaN or an infinity (fmaxf
// drops NaN, a sum does not); such a row is scaled by NaN, so every output of
// the token is NaN, as the reference's fp32 forward yields (a non-finite
// activation reaches every rank value with both signs; reference.py:208-217).
__device__ __forceinline__ float prep_scale(float max_abs, float sum_abs) {
    return sum_abs <= 3.402823466e38f ? range_scale(max_abs) : __builtin_nanf("");
}

// Position of column c in a prepared row: columns 1 and 2 of every group of
// four are swapped (the order the sign operand's fp16 pairs come in).
__device__ __forceinline__ int64_t swizzle4(int64_t c) { return (c & ~int64_t(3)) | ((c & 1) << 1) | ((c >> 1) & 1); }

// fp32 values of elements [c, c + 8) of a row (c % 8 == 0): one 16-byte (or
// two, for fp32) vector load when `vec` (the host checked alignment and
// cols % 8 == 0), bounds-checked element loads otherwise.
__device__ __forceinline__ void load8(const void* __restrict__ p, int dtype, bool vec, int64_t base, int64_t c,
                                      int64_t cols, float (&v)[8]) {
    if (vec) {
        if (dtype == NQ_DTYPE_F32) {
            const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + base + c);
            const float4 a = q[0], b = q[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + base + c);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (dtype == NQ_DTYPE_BF16) {
                    v[2 * i] = __uint_as_float(w[i] << 16);
                    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                } else {
                    union {
                        uint32_t u;
                        _Float16 h[2];
                    } h;
                    h.u = w[i];
                    v[2 * i] = static_cast<float>(h.h[0]);
                    v[2 * i + 1] = static_cast<float>(h.h[1]);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = c + i < cols ? nq::load_f32(p, dtype, base + c + i) : 0.0f;
    }
}

// Row pass of one member of a batched call (grid y = member, x = token).
struct PrepArgs {
    const void* act;                 // [tokens, ld] activations
    int64_t ld;
    const void* colscale;            // [cols] s_in, or null
    int colscale_dtype;
    int vec;                         // 16-byte loads allowed (generic kernel)
    int64_t cols, cols_pad;
    _Float16* out16;                 // [tokens, cols_pad], or [tokens, 2 cols_pad] with split
    int split;                       // split operands: hi and lo planes per 128-column block
    float* scale_out;                // [tokens]
    const uint32_t* max_mid_bits;    // fp32 bits of max|s_mid|, or null
    float* bound_scale_out;          // [tokens]
};

struct PrepBatch {
    PrepArgs p[kPrefillBatch];
};

// Stores columns [c, c + 8) (c % 8 == 0) of prepared row t, v times `scale`,
// into a buffer of rows of cols_pad columns: fp16 with columns 1 and 2 of
// every group of four exchanged (swizzle4), one 16-byte store; with `split`
// the rows are 2 cols_pad wide, block c / 128 holding its 128 high parts and
// then their remainders: two stores.
__device__ __forceinline__ void store_prepped(_Float16* __restrict__ out, int64_t t, int64_t cols_pad, int64_t c,
                                              const float (&v)[8], float scale, bool split) {
    union {
        _Float16 h[8];
        uint4 u;
    } hi, lo;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = v[4 * g + (i == 1 ? 2 : (i == 2 ? 1 : i))] * scale;
            hi.h[4 * g + i] = static_cast<_Float16>(x);
            lo.h[4 * g + i] = static_cast<_Float16>(x - static_cast<float>(hi.h[4 * g + i]));
        }
    }
    if (!split) {
        *reinterpret_cast<uint4*>(out + t * cols_pad + c) = hi.u;
        return;
    }
    _Float16* const row = out + t * 2 * cols_pad + (c >> 7) * 256 + (c & 127);
    *reinterpret_cast<uint4*>(row) = hi.u;
    *reinterpret_cast<uint4*>(row + 128) = lo.u;
}

// One workgroup per row: out16[t, swizzle4(c)] = fp16(a[t, c] * s[c] * scale_t)
// for c < cols, zero for cols <= c < cols_pad; scale_out[t] = scale_t. Each
// thread takes 8 consecutive columns per step (one 16-byte store of fp16).
// With `max_mid_bits` (fp32 bits of max|s_mid|) it also writes
// bound_scale_out[t], the power of two that puts max|s_mid| * Σ_c |a s| at
// or below 2^14: the scale of the row's rank intermediate.
__global__ __launch_bounds__(kBlock) void k_prep_rows(const PrepBatch batch, int act_dtype) {
    const PrepArgs& pa = batch.p[blockIdx.y];
    const void* __restrict__ act = pa.act;
    const int64_t ld = pa.ld;
    const void* __restrict__ colscale = pa.colscale;
    const int colscale_dtype = pa.colscale_dtype;
    const int64_t cols = pa.cols, cols_pad = pa.cols_pad;
    const int vec = pa.vec;
    _Float16* __restrict__ out16 = pa.out16;
    float* __restrict__ scale_out = pa.scale_out;
    const uint32_t* __restrict__ max_mid_bits = pa.max_mid_bits;
    float* __restrict__ bound_scale_out = pa.bound_scale_out;
    __shared__ float wmax[kBlock / 64];
    __shared__ float wsum[kBlock / 64];
    const int64_t t = blockIdx.x;
    auto values = [&](int64_t c, float (&v)[8]) {
        load8(act, act_dtype, vec != 0, t * ld, c, cols, v);
        if (colscale) {
            float s8[8];
            load8(colscale, colscale_dtype, vec != 0, 0, c, cols, s8);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] *= s8[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = c + i < cols ? v[i] : 0.0f;
    };
    float m = 0.0f, l1 = 0.0f;
    for (int64_t c = 8 * threadIdx.x; c < cols; c += 8 * kBlock) {
        float v[8];
        values(c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i])), l1 += fabsf(v[i]);
    }
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off)), l1 += __shfl_xor(l1, off);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m, wsum[threadIdx.x >> 6] = l1;
    __syncthreads();
    const float l1t = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const float scale = prep_scale(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])), l1t);
    if (max_mid_bits && threadIdx.x == 0) bound_scale_out[t] = range_scale(__uint_as_float(*max_mid_bits) * l1t);
    for (int64_t c = 8 * threadIdx.x; c < cols_pad; c += 8 * kBlock) {
        float v[8];
        if (c < cols) values(c, v);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        store_prepped(out16, t, cols_pad, c, v, scale, pa.split != 0);
    }
    if (threadIdx.x == 0) scale_out[t] = scale;
}

// Elements [i, i + 8) of a buffer of dtype DT as fp32: one 16-byte load
// (two for fp32), no branch.
template <int DT>
__device__ __forceinline__ void load8_as(const void* __restrict__ p, int64_t i, float (&v)[8]) {
    if constexpr (DT == NQ_DTYPE_F32) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 a = q[0], b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (DT == NQ_DTYPE_BF16) {
                v[2 * j] = __uint_as_float(w[j] << 16);
                v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            } else {
                v[2 * j] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[j])));
                v[2 * j + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[j] >> 16)));
            }
        }
    }
}

// k_prep_rows for rows of at most NCH * 8 * kBlock padded columns whose
// activations and column scales allow 16-byte loads (cols % 8 == 0, aligned):
// each thread keeps its NCH chunks of eight columns in registers, so the row
// is read once, and every load is issued before the first use. Same
// arithmetic and summation order as k_prep_rows, so both give identical
// results. NCH = 2 (rows up to 4096 columns) keeps the registers low enough
// for eight workgroups per CU.
constexpr int kPrepChunksMax = 8;

template <int ADT, int SDT, int NCH>
__global__ __launch_bounds__(kBlock) void k_prep_rows_vec(const PrepBatch batch) {
    const PrepArgs& pa = batch.p[blockIdx.y];
    const void* __restrict__ act = pa.act;
    const int64_t ld = pa.ld;
    const void* __restrict__ colscale = pa.colscale;
    const int64_t cols = pa.cols, cols_pad = pa.cols_pad;
    _Float16* __restrict__ out16 = pa.out16;
    float* __restrict__ scale_out = pa.scale_out;
    const uint32_t* __restrict__ max_mid_bits = pa.max_mid_bits;
    float* __restrict__ bound_scale_out = pa.bound_scale_out;
    __shared__ float wmax[kBlock / 64];
    __shared__ float wsum[kBlock / 64];
    const int64_t t = blockIdx.x;
    float v[NCH][8];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int64_t c = 8 * threadIdx.x + 8 * kBlock * k;
        const int64_t cc = c < cols ? c : 0;  // chunks past the row reload its first
        float s8[8];
        load8_as<ADT>(act, t * ld + cc, v[k]);
        load8_as<SDT>(colscale, cc, s8);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[k][i] *= s8[i];
    }
    float m = 0.0f, l1 = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const bool live = 8 * threadIdx.x + 8 * kBlock * k < cols;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[k][i] = live ? v[k][i] : 0.0f;
            if (live) m = fmaxf(m, fabsf(v[k][i])), l1 += fabsf(v[k][i]);
        }
    }
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off)), l1 += __shfl_xor(l1, off);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m, wsum[threadIdx.x >> 6] = l1;
    __syncthreads();
    const float l1t = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const float scale = prep_scale(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])), l1t);
    if (max_mid_bits && threadIdx.x == 0) bound_scale_out[t] = range_scale(__uint_as_float(*max_mid_bits) * l1t);
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        const int64_t c = 8 * threadIdx.x + 8 * kBlock * k;
        if (c >= cols_pad) continue;
        store_prepped(out16, t, cols_pad, c, v[k], scale, pa.split != 0);
    }
    if (threadIdx.x == 0) scale_out[t] = scale;
}

// B operand of the 32 x 32 x 16 MFMA of 16-column slice m from the words of
// lane groups 2h and 2h + 1 (w0, w1): at bit 8b + m they hold columns
// 16m + 8h + b and 16m + 8h + 4 + b. The A rows are stored with columns 1 and
// 2 of every group of four swapped, so the eight k slots of a lane are columns
// 8h + {0, 2, 1, 3, 4, 6, 5, 7}: dword e pairs bits (m, m + 16) or
// (m + 8, m + 24) of one word, which one shift moves to the fp16 sign
// positions 15 and 31.
__device__ __forceinline__ uint32_t sign_pair(uint32_t w, int shift, uint32_t mask, uint32_t one) {
    // ((w << shift) & mask) | one as two instructions: the masks are kept in
    // registers because a VOP3 instruction cannot take two literal constants.
    return ((w << shift) & mask) | one;
}

// 64-bit left shift as one instruction (a shift by a constant is otherwise
// split into a 32-bit shift and an alignbit); the amount comes from an SGPR.
__device__ __forceinline__ uint64_t shl64(uint64_t w, int s) {
    uint64_t r;
    asm("v_lshlrev_b64 %0, %1, %2" : "=v"(r) : "s"(s), "v"(w));
    return r;
}

// The two words take the same shifts, so each shift moves both as one 64-bit
// value (w1:w0): a shift s <= 15 carries bits of w0 only into bits below s of
// the high half, never into its sign positions 15 and 31.
__device__ __forceinline__ v8h expand_signs32(uint32_t w0, uint32_t w1, int m, uint32_t mask, uint32_t one) {
    union {
        uint32_t u[4];
        v8h v;
    } x;
    const uint64_t w = (static_cast<uint64_t>(w1) << 32) | w0;
    const uint64_t hi = shl64(w, 15 - m), lo = shl64(w, 7 - m);
    x.u[0] = (static_cast<uint32_t>(hi) & mask) | one;
    x.u[1] = (static_cast<uint32_t>(lo) & mask) | one;
    x.u[2] = (static_cast<uint32_t>(hi >> 32) & mask) | one;
    x.u[3] = (static_cast<uint32_t>(lo >> 32) & mask) | one;
    return x.v;
}

struct GemmArgs {
    const _Float16* a;        // [M, kpad] fp16 activations (row-scaled); [M, 2 kpad] with split
    int64_t m;                // tokens
    int64_t kpad;             // nb * 128
    const uint32_t* tiles;    // sign tiles [rt][nb * 64] (chunked, see above)
    int64_t n;                // sign rows (rank or out)
    int64_t nb;               // 128-column blocks
    const float* row_scale;   // [M]: divide accumulators by this
    const void* col_scale;    // [n] s_mid or s_out
    int col_scale_dtype;
    // epilogue (GEMM 2 only; salient_count == 0 and bias == null for GEMM 1)
    const void* x;
    int x_dtype;
    int64_t in;
    int64_t salient_count;
    const int32_t* salient_indices;
    const void* salient_values;
    int salient_dtype;
    const void* salient_scales;
    int scale_dtype;
    const void* bias;
    int bias_dtype;
    void* out;                // [M, n], or fp16 [M, out_ld] with out_scale
    int out_dtype;
    const float* out_scale;   // [M] or null: write fp16(v * out_scale[t]) at column
                              // swizzle4(c) of an out_ld-wide row, zero for n <= c < out_ld
                              // (split: rows 2 out_ld wide, the prepared-row layout)
    int64_t out_ld;
    int split;                // split operands (A, and the rank intermediate written)
    int64_t k_per_split;      // K blocks per K slice
    int64_t splits;           // K slices (1: no split)
    int64_t col_blocks;       // column blocks at the launch's block width
    float* partial;           // [splits][M][n] raw accumulators, or null (direct epilogue)
};

// Up to kPrefillBatch GEMMs of one phase (the members of a batched call share
// the token count) in one launch. Grid x concatenates the members' ranges:
// member i owns [begin[i], begin[i + 1]) (k_sign_gemm: col_blocks * splits
// workgroups, slice-major; k_reduce_splits: its column blocks, none for a
// member without a split); begin[i] = INT32_MAX past the last member.
struct GemmBatch {
    int32_t begin[kPrefillBatch];
    GemmArgs p[kPrefillBatch];
};

// The member whose range holds grid-x index x: the last one beginning at or
// before it (a member with an empty range shares its begin with the next).
__device__ __forceinline__ int batch_member(const GemmBatch& b, int x) {
    int m = 0;
#pragma unroll
    for (int i = 1; i < kPrefillBatch; ++i) m = x >= b.begin[i] ? i : m;
    return m;
}

// Block shapes, as (WR wave rows, II 32-row A fragments and JJ 32-column B
// fragments per wave): (2, 2, 2): the four waves form a 2 x 2 grid of 64 x 64
// tiles (block tile 128 x 128). (1, 4, 2): they sit side by side, each
// 128 x 64 (block tile 128 x 256): every expanded sign fragment then serves
// four A fragments instead of two, for GEMMs with enough blocks to fill the
// GPU at that size. (1, 2, 1): side by side, each 64 x 32 (block tile
// 64 x 128), for at most 64 tokens: no MFMA or A read is spent on rows past
// the last token.
template <int WR, int II, int JJ, bool SPLIT>
__global__ __launch_bounds__(kBlock, JJ == 1 ? 4 : 2) void k_sign_gemm(const GemmBatch batch) {
    constexpr int BM = WR * 32 * II;      // token rows per block
    constexpr int BN = (4 / WR) * 32 * JJ;  // sign rows per block
    constexpr int NJ = BM / 16;           // 1-KB LDS transfers per wave per K step and plane
    constexpr int kABytes = BM * kBK * 2;   // one activation plane, rows of 256 bytes
    constexpr int kPlanes = SPLIT ? 2 : 1;  // split operands: the hi plane, then the lo plane
    constexpr int kBufBytes = kPlanes * kABytes;
    constexpr int kParkStride = 32 * JJ + 1;  // floats per parked accumulator row
    constexpr int kParkBytes = 4 * 64 * kParkStride * 4;
    constexpr int kLds = 2 * kBufBytes > kParkBytes ? 2 * kBufBytes : kParkBytes;  // double-buffered A
    const int member = batch_member(batch, static_cast<int>(blockIdx.x));
    const GemmArgs& g = batch.p[member];
    const int local = static_cast<int>(blockIdx.x) - batch.begin[member];
    const int col_blocks = static_cast<int>(g.col_blocks);
    const int slice = local / col_blocks;
    const int col_block = local - slice * col_blocks;
    __shared__ __attribute__((aligned(16))) char lds[kLds];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int wm = WR == 2 ? wave >> 1 : 0;  // wave row
    const int wn = WR == 2 ? wave & 1 : wave;  // wave column
    const int h = lane >> 5;   // K half of the 32 x 32 x 16 operands
    const int r = lane & 31;   // A row / B column within a 32-wide fragment
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
    const int64_t n0 = static_cast<int64_t>(col_block) * BN;
    const int64_t rt_count = (g.n + kTileRows - 1) / kTileRows;
    // B fragment jj covers sign rows n0 + 32 JJ wn + 32 jj + [0, 32): lane r
    // reads row r of tile (r >> 4) of that pair, from the words of lane groups
    // 2h and 2h + 1, which hold columns 16m + 8h + [0, 8) of each 16-column slice.
    const int64_t rt0 = n0 / kTileRows + 2 * JJ * wn + (r >> 4);
    const int wl0 = 16 * (2 * h) + (r & 15), wl1 = wl0 + 16;

    v16f acc[II][JJ];
#pragma unroll
    for (int i = 0; i < II; ++i)
#pragma unroll
        for (int j = 0; j < JJ; ++j) acc[i][j] = v16f{};

    uint32_t words[JJ][2], next_words[JJ][2];
    // Activation tile: BM rows of 128 fp16 (256 bytes) per buffer, moved
    // from global memory straight into LDS (global_load_lds_dwordx4: lane l
    // of an instruction writes 16 bytes at the wave's LDS address + 16 l), so
    // the next K step's tile costs no registers while it is in flight. Wave w's
    // instruction j fills LDS rows 4 (NJ w + j) + [0, 4); lane l writes chunk
    // position p = l & 15 of row r, which holds the row's 16-byte column chunk
    // p ^ (r & 15): the A-fragment reads (32 rows at one chunk per
    // instruction) then fall on distinct banks. Every load is unconditional
    // (no branch in the K loop): rows past M read the last valid row and sign
    // tiles past N a valid tile; they only feed accumulators whose outputs are
    // never stored.
    const int64_t nsc = g.nb, lda = kPlanes * g.kpad;  // fp16 per activation row
    const int64_t a_rows = g.m - m0;  // valid rows of this block (>= 1)
    // Byte offsets from the block's first row (below 2^31: at most 128 rows
    // of a padded K that the host limits), added to a wave-uniform base.
    const char* const a_blk = reinterpret_cast<const char*>(g.a + m0 * lda);
    uint32_t a_src[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int row = 4 * (NJ * wave + j) + (lane >> 4);
        const int chunk = (lane & 15) ^ (row & 15);
        const int64_t rr = row < a_rows ? row : a_rows - 1;
        a_src[j] = static_cast<uint32_t>((rr * lda + 8 * chunk) * 2);
    }
    const uint32_t* bt[JJ];
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj) {
        const int64_t rt = rt0 + 2 * jj < rt_count ? rt0 + 2 * jj : rt_count - 1;
        bt[jj] = g.tiles + rt * nsc * 64;
    }
    const int64_t k_begin = static_cast<int64_t>(slice) * g.k_per_split;
    const int64_t k_end = k_begin + g.k_per_split < nsc ? k_begin + g.k_per_split : nsc;
    // The transfer is issued as inline asm with its LDS address in M0: the
    // compiler then does not track it, so the A-fragment reads of the current
    // buffer wait only on themselves (lgkmcnt(4)) instead of lgkmcnt(0) while
    // the next tile is in flight. Completion is this kernel's own business: a
    // transfer only targets the buffer no wave reads in that step, and every
    // step ends with vmcnt(0) and a barrier before that buffer is read.
    typedef __attribute__((address_space(3))) void lds_void_t;
    const auto load_a = [&](int64_t sc, int buf) __attribute__((always_inline)) {
        // wave-uniform: a scalar base, per-lane 32-bit offsets; plane q of
        // block sc starts 256 q bytes after the hi plane.
        const char* base = a_blk + sc * (2 * kBK * kPlanes);
#pragma unroll
        for (int q = 0; q < kPlanes; ++q)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                lds_void_t* dst = (lds_void_t*)(lds + buf * kBufBytes + q * kABytes + (NJ * wave + j) * 1024);
                const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
                // s_nop: one wait state between the M0 write and the LDS transfer.
                asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(a_src[j]), "s"(base + 2 * kBK * q),
                             "{m0}"(lds_addr)
                             : "memory");
            }
    };
    const auto load_words = [&](int64_t sc) __attribute__((always_inline)) {
        const int64_t c_ = sc >> 2;
        const int64_t rem_ = nsc - 4 * c_;
        const int dw_ = static_cast<int>(rem_ < 4 ? rem_ : 4);
        const int64_t off_ = c_ * 256 + (sc & 3);
#pragma unroll
        for (int jj = 0; jj < JJ; ++jj) {
            next_words[jj][0] = bt[jj][off_ + wl0 * dw_];
            next_words[jj][1] = bt[jj][off_ + wl1 * dw_];
        }
    };
    // Byte offset, within a buffer, of the A fragment of 16-column slice m
    // for fragment row 0 (fragment ii adds 32 rows = 8192 bytes).
    int a_off[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) a_off[m] = (32 * II * wm + r) * 256 + 16 * ((2 * m + h) ^ (r & 15));
    // Step s computes on buffer s & 1 while the tile of step s + 1 moves into
    // the other; a wait for this wave's transfers and one barrier per step
    // make every wave's part of the next tile visible before it is read.
    load_a(k_begin, 0);
    load_words(k_begin);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj) words[jj][0] = next_words[jj][0], words[jj][1] = next_words[jj][1];
    int buf = 0;
    uint32_t sign_mask = 0x80008000u, fp16_one = 0x3C003C00u;
    asm volatile("" : "+v"(sign_mask), "+v"(fp16_one));  // keep them in VGPRs
    for (int64_t sc = k_begin; sc < k_end; ++sc) {
        const int64_t nxt = sc + 1 < k_end ? sc + 1 : sc;  // the last step reloads its tile into the idle buffer
        load_a(nxt, buf ^ 1);
        load_words(nxt);
        // The sign words of the next step are issued here, ahead of the
        // MFMAs; left to itself the scheduler sinks them to the step's end,
        // where the wait before the barrier would take their whole latency.
        __builtin_amdgcn_sched_barrier(0);
        const char* a_lds = lds + buf * kBufBytes;
        // Software pipeline over the eight 16-column slices: slice m's MFMAs
        // issue while slice m + 1's A fragments are read from LDS and its
        // sign fragments expanded, so no MFMA waits on a read issued just
        // before it. Each slice is one scheduling region (sched_barrier) laid
        // out as the reads, then MFMAs alternating with the expansion. With
        // split operands fragment II + ii is the lo plane of fragment ii.
        constexpr int NA = kPlanes * II;
        v8h a_cur[NA], b_cur[JJ];
#pragma unroll
        for (int ai = 0; ai < NA; ++ai)
            a_cur[ai] = *reinterpret_cast<const v8h*>(a_lds + (ai / II) * kABytes + a_off[0] + 8192 * (ai % II));
#pragma unroll
        for (int jj = 0; jj < JJ; ++jj) b_cur[jj] = expand_signs32(words[jj][0], words[jj][1], 0, sign_mask, fp16_one);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            __builtin_amdgcn_sched_barrier(0);
            v8h a_nxt[NA], b_nxt[JJ];
            if (m < 7) {
#pragma unroll
                for (int ai = 0; ai < NA; ++ai)
                    a_nxt[ai] = *reinterpret_cast<const v8h*>(a_lds + (ai / II) * kABytes + a_off[m + 1] +
                                                              8192 * (ai % II));
#pragma unroll
                for (int jj = 0; jj < JJ; ++jj)
                    b_nxt[jj] = expand_signs32(words[jj][0], words[jj][1], m + 1, sign_mask, fp16_one);
            }
#pragma unroll
            for (int ai = 0; ai < NA; ++ai)
#pragma unroll
                for (int jj = 0; jj < JJ; ++jj)
                    acc[ai % II][jj] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(a_cur[ai], b_cur[jj], acc[ai % II][jj], 0, 0, 0);
            if (m < 7) {
                __builtin_amdgcn_sched_group_barrier(0x100, NA, 0);  // LDS reads of slice m + 1
#pragma unroll
                for (int q = 0; q < NA * JJ; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA of slice m
                    __builtin_amdgcn_sched_group_barrier(0x002, 8 / NA, 0);  // expansion of m + 1
                }
#pragma unroll
                for (int ai = 0; ai < NA; ++ai) a_cur[ai] = a_nxt[ai];
#pragma unroll
                for (int jj = 0; jj < JJ; ++jj) b_cur[jj] = b_nxt[jj];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jj = 0; jj < JJ; ++jj) words[jj][0] = next_words[jj][0], words[jj][1] = next_words[jj][1];
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        buf ^= 1;
    }


    // Epilogue through LDS: each wave parks its 64 x 64 fp32 tile (lane holds
    // D[8 (q / 4) + 4 (lane / 32) + q % 4][lane % 32] of each 32 x 32 MFMA
    // tile), then walks it row by row with lane = column, so every output row
    // segment is one coalesced 64-wide store and the salient sum joins before
    // the single rounding to the output dtype.
    float* park = reinterpret_cast<float*>(lds) + wave * (64 * kParkStride);
    // One 64-row half of the wave's tile (rows row0 + [0, 64)); `return`
    // leaves only this lambda.
    const auto emit = [&](const int64_t row0) __attribute__((always_inline)) {
        const int64_t col = n0 + 32 * JJ * wn + lane;
        const bool lane_ok = lane < 32 * JJ;  // lanes past the wave's columns store nothing
        const int p_lane = lane_ok ? lane : 0;  // and read a parked column of their own row
        const int rows = __builtin_amdgcn_readfirstlane(static_cast<int>(g.m - row0 < 64 ? g.m - row0 : 64));
        if (rows <= 0) return;  // the whole wave is past the last token
        const bool col_ok = lane_ok && col < g.n;
        if (g.partial) {
            if (!col_ok) return;
            float* dst = g.partial + static_cast<int64_t>(slice) * g.m * g.n;
            for (int e = 0; e < rows; ++e) dst[(row0 + e) * g.n + col] = park[e * kParkStride + p_lane];
            return;
        }
        // Every lane stays active up to the stores: lane e holds values of row
        // row0 + e that other lanes read with readlane. 1 / row_scale is exact
        // (row_scale is a normal power of two; exponent field 254 - E), so the
        // row loop multiplies by it and waits on no memory.
        const int64_t col_c = col_ok ? col : g.n - 1;
        const int lane_row = lane < rows ? lane : rows - 1;
        const float inv_lane =
            __uint_as_float((254u << 23) - (__float_as_uint(g.row_scale[row0 + lane_row]) & 0x7f800000u));
        const float cs = nq::load_f32(g.col_scale, g.col_scale_dtype, col_c);
        const float bias = g.bias ? nq::load_f32(g.bias, g.bias_dtype, col_c) : 0.0f;
        auto inv_of = [&](int e) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_lane), e)); };
        const int64_t salient = g.salient_count;
        float v[64];
#pragma unroll
        for (int e = 0; e < 64; ++e) v[e] = park[e * kParkStride + p_lane] * inv_of(e) * cs + bias;
        // Salient columns (none for most layers): v[e] for the wave's 64 rows
        // stays in registers while the columns are added in index order, eight at
        // a time. Lane e loads x[row0 + e, idx_k] and the row loop takes it with
        // readlane, so a batch of eight columns costs one round of loads.
        for (int64_t k0 = 0; k0 < salient; k0 += 8) {
            float xk[8], wk[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t k = k0 + j < salient ? k0 + j : salient - 1;
                const int64_t idx = g.salient_indices[k];
                xk[j] = nq::load_f32(g.x, g.x_dtype, (row0 + lane_row) * g.in + idx);
                float w = nq::load_f32(g.salient_values, g.salient_dtype, col_c * salient + k);
                if (g.salient_scales) w *= nq::load_f32(g.salient_scales, g.scale_dtype, k);
                wk[j] = k0 + j < salient ? w : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (k0 + j < salient) {
#pragma unroll
                    for (int e = 0; e < 64; ++e)
                        v[e] += wk[j] * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xk[j]), e));
                }
            }
        }
        if (g.out_scale) {
            // The rank intermediate for GEMM 2: fp16, row-scaled, swizzled, with
            // the padding columns up to out_ld written as zeros (a 256-wide
            // block can reach past out_ld: those lanes store nothing); split:
            // the prepared-row layout, high parts and remainders.
            const float os_lane = g.out_scale[row0 + lane_row];
            const bool in_row = lane_ok && col < g.out_ld;
            const int64_t cc = in_row ? col : 0;
            const int64_t stride = kPlanes * g.out_ld;
            _Float16* o = static_cast<_Float16*>(g.out) + row0 * stride + (cc >> 7) * (128 * kPlanes) +
                          swizzle4(cc & 127);
#pragma unroll
            for (int e = 0; e < 64; ++e) {
                const float os = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(os_lane), e));
                if (e < rows && in_row) {
                    const float x = col_ok ? v[e] * os : 0.0f;
                    const _Float16 hi = static_cast<_Float16>(x);
                    o[e * stride] = hi;
                    if constexpr (SPLIT) o[e * stride + 128] = static_cast<_Float16>(x - static_cast<float>(hi));
                }
            }
            return;
        }
        if (!col_ok) return;
        // One switch on the output dtype, then 64 predicated stores with
        // constant register indices.
        const int64_t out0 = row0 * g.n + col;
        switch (g.out_dtype) {
            case NQ_DTYPE_F32: {
                float* o = static_cast<float*>(g.out) + out0;
#pragma unroll
                for (int e = 0; e < 64; ++e)
                    if (e < rows) o[e * g.n] = v[e];
                break;
            }
            case NQ_DTYPE_F16: {
                _Float16* o = static_cast<_Float16*>(g.out) + out0;
#pragma unroll
                for (int e = 0; e < 64; ++e)
                    if (e < rows) o[e * g.n] = static_cast<_Float16>(v[e]);
                break;
            }
            case NQ_DTYPE_BF16: {
                uint16_t* o = static_cast<uint16_t*>(g.out) + out0;
#pragma unroll
                for (int e = 0; e < 64; ++e)
                    if (e < rows) o[e * g.n] = nq::f32_to_bf16_bits(v[e]);
                break;
            }
            default:
                break;
        }
    };
    // Park fragments ii0 and ii0 + 1 (a 64-row half), then emit it. Written
    // out per half rather than as a loop: the accumulators must keep constant
    // register indices, and the compiler does not always unroll a loop around
    // two copies of emit.
    const auto park_half = [&](const v16f (&a0)[JJ], const v16f (&a1)[JJ]) __attribute__((always_inline)) {
#pragma unroll
        for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                park[(8 * (q >> 2) + 4 * h + (q & 3)) * kParkStride + 32 * jj + r] = a0[jj][q];
                park[(32 + 8 * (q >> 2) + 4 * h + (q & 3)) * kParkStride + 32 * jj + r] = a1[jj][q];
            }
    };
    park_half(acc[0], acc[1]);
    __syncthreads();
    emit(m0 + 32 * II * wm);
    if constexpr (II == 4) {
        __syncthreads();  // the first half is read out of the park area
        park_half(acc[2], acc[3]);
        __syncthreads();
        emit(m0 + 32 * II * wm + 64);
    }
}

// Element i of an F32 / F16 / BF16 buffer from two unconditional 16-bit
// loads (the halves of an fp32, or the same half twice), decoded by a
// uniform select: no branch surrounds the loads, so they issue together.
struct Raw2 {
    uint32_t lo, hi;
};

__device__ __forceinline__ Raw2 load_raw2(const void* __restrict__ p, int dtype, int64_t i) {
    const uint16_t* h = static_cast<const uint16_t*>(p);
    const bool wide = dtype == NQ_DTYPE_F32;
    return Raw2{h[wide ? 2 * i : i], h[wide ? 2 * i + 1 : i]};
}

__device__ __forceinline__ float raw2_value(const Raw2& r, int dtype) {
    const float f32 = __uint_as_float((r.hi << 16) | (r.lo & 0xffffu));
    const float bf16 = __uint_as_float(r.lo << 16);
    const float f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.lo)));
    return dtype == NQ_DTYPE_F32 ? f32 : (dtype == NQ_DTYPE_BF16 ? bf16 : f16);
}

// Split-K epilogue, one thread per output element (t, c), grid (the members'
// column blocks, token rows; t = blockIdx.y + kRowsPerGridZ * blockIdx.z): out[t, c] =
// (Σ_z partial[z][t][c]) / row_scale[t] * col_scale[c] (+ bias + salient
// columns for GEMM 2), the slices summed in z order. The column's scale and
// bias and the first eight partials are loaded before any is used. With
// out_scale the threads cover out_ld columns and write the fp16 rank
// intermediate as the direct epilogue does (zeros past column n).
constexpr int64_t kRowsPerGridZ = 65535;

__global__ __launch_bounds__(kBlock) void k_reduce_splits(const GemmBatch batch) {
    const int member = batch_member(batch, static_cast<int>(blockIdx.x));
    const GemmArgs& ga = batch.p[member];
    const int splits = static_cast<int>(ga.splits);
    // Every argument the kernel reads is loaded in one batch: the empty asm
    // needs them all at one point, instead of one round trip per branch.
    GemmArgs g;
    g.m = ga.m;
    g.n = ga.n;
    g.out_ld = ga.out_ld;
    g.out_scale = ga.out_scale;
    g.out = ga.out;
    g.out_dtype = ga.out_dtype;
    g.partial = ga.partial;
    g.row_scale = ga.row_scale;
    g.col_scale = ga.col_scale;
    g.col_scale_dtype = ga.col_scale_dtype;
    g.bias = ga.bias;
    g.bias_dtype = ga.bias_dtype;
    g.salient_count = ga.salient_count;
    g.split = ga.split;
    asm volatile("" ::"s"(g.m), "s"(g.n), "s"(g.out_ld), "s"(g.out_scale), "s"(g.out), "s"(g.out_dtype),
                 "s"(g.partial), "s"(g.row_scale), "s"(g.col_scale), "s"(g.col_scale_dtype), "s"(g.bias),
                 "s"(g.bias_dtype), "s"(g.salient_count), "s"(splits));
    g.salient_values = ga.salient_values;
    g.salient_dtype = ga.salient_dtype;
    g.salient_scales = ga.salient_scales;
    g.scale_dtype = ga.scale_dtype;
    g.salient_indices = ga.salient_indices;
    g.x = ga.x;
    g.x_dtype = ga.x_dtype;
    g.in = ga.in;
    const int64_t c = static_cast<int64_t>(static_cast<int>(blockIdx.x) - batch.begin[member]) * kBlock + threadIdx.x;
    const int64_t t = static_cast<int64_t>(blockIdx.z) * kRowsPerGridZ + blockIdx.y;
    const int64_t width = g.out_scale ? g.out_ld : g.n;
    if (splits <= 1 || c >= width || t >= g.m) return;  // members without a split have no partials
    // With out_scale: the rank intermediate's position of column c (split
    // operands: the high part, its remainder 128 further).
    const int64_t planes = g.split ? 2 : 1;
    _Float16* const lm = g.out_scale ? static_cast<_Float16*>(g.out) + t * planes * g.out_ld +
                                           (c >> 7) * (128 * planes) + swizzle4(c & 127)
                                     : nullptr;
    if (c >= g.n) {  // only with out_scale: a padding column of the rank intermediate
        lm[0] = static_cast<_Float16>(0.0f);
        if (g.split) lm[128] = static_cast<_Float16>(0.0f);
        return;
    }
    const int64_t plane = g.m * g.n;
    const int64_t pi = t * g.n + c;
    const Raw2 cs_raw = load_raw2(g.col_scale, g.col_scale_dtype, c);
    const Raw2 bias_raw = load_raw2(g.bias ? g.bias : g.col_scale, g.bias ? g.bias_dtype : g.col_scale_dtype, c);
    float part[8];
    float v = 0.0f;
    for (int z0 = 0; z0 < splits; z0 += 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) part[j] = z0 + j < splits ? g.partial[(z0 + j) * plane + pi] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) v += part[j];
    }
    v = v / g.row_scale[t] * raw2_value(cs_raw, g.col_scale_dtype);
    if (g.bias) v += raw2_value(bias_raw, g.bias_dtype);
    for (int64_t k = 0; k < g.salient_count; ++k) {
        float w = nq::load_f32(g.salient_values, g.salient_dtype, c * g.salient_count + k);
        if (g.salient_scales) w *= nq::load_f32(g.salient_scales, g.scale_dtype, k);
        v += w * nq::load_f32(g.x, g.x_dtype, t * g.in + g.salient_indices[k]);
    }
    if (g.out_scale) {
        const float x = v * g.out_scale[t];
        const _Float16 hi = static_cast<_Float16>(x);
        lm[0] = hi;
        if (g.split) lm[128] = static_cast<_Float16>(x - static_cast<float>(hi));
    } else {
        nq::store_f32_as(g.out, g.out_dtype, pi, v);
    }
}

// Tile counts and 128-column block counts of V [rank, in] and U [out, rank]
// (the same geometry as the decode tiles).
struct Geometry {
    int64_t rt1, nsc1, rt2, nsc2, v_words, u_words;
};

Geometry geometry(const nq_linear_desc* d) {
    Geometry g{};
    g.rt1 = (d->rank + kTileRows - 1) / kTileRows;
    g.nsc1 = (d->in_features + kBK - 1) / kBK;
    g.rt2 = (d->out_features + kTileRows - 1) / kTileRows;
    g.nsc2 = (d->rank + kBK - 1) / kBK;
    g.v_words = g.rt1 * g.nsc1 * 64;
    g.u_words = g.rt2 * g.nsc2 * 64;
    return g;
}

int64_t a256(int64_t n) { return (n + 255) & ~int64_t(255); }

// Split of a GEMM with `tiles` (token, sign-row) tiles over K blocks, from a
// latency model of the K loop (fitted to layer timings on MI355X): a K step
// costs kStepNs (the next step's tile is in flight during the current one,
// so a step is about one compute pass, not a memory round trip), while the GPU holds every
// workgroup at once (kResident: two per CU, bound by LDS); workgroups beyond
// that run in further rounds; a split adds the reduce launch and the
// partials' write and read (M x N x 4 bytes per slice, mostly served by the
// last-level cache). Slices hold at least kMinSliceBlocks K blocks.
constexpr int64_t kResident = 512;
constexpr int64_t kResidentSmall = 1024;  // the 64 x 128 block: four per CU
constexpr double kStepNsSmall = 500.0;    // half the MFMA and A work of a 128-row step
constexpr int64_t kMinSliceBlocks = 2;
constexpr double kStepNs = 1000.0;
constexpr double kReduceNsSmall = 3000.0;  // the reduce launch after 64 x 128 blocks
constexpr double kReduceNs = 6000.0;       // and after 128-row blocks (measured: 2.5% faster at
                                           // 256 tokens than 3000, the same above)
constexpr double kPartialBytesPerNs = 8000.0;

struct Split {
    int64_t slices, k_per_split;
};

// Resident workgroups, K-step cost and reduce cost of the block tile used for `tokens`.
int64_t resident_for(int64_t tokens) { return tokens <= kBM / 2 ? kResidentSmall : kResident; }
double step_ns_for(int64_t tokens) { return tokens <= kBM / 2 ? kStepNsSmall : kStepNs; }
double reduce_ns_for(int64_t tokens) { return tokens <= kBM / 2 ? kReduceNsSmall : kReduceNs; }

Split split_for(int64_t tiles, int64_t k_blocks, int64_t tokens, int64_t n) {
    const int64_t resident = resident_for(tokens);
    const double step_ns = step_ns_for(tokens);
    Split best{1, k_blocks};
    double best_ns = -1.0;
    const int64_t most = k_blocks / kMinSliceBlocks > 1 ? k_blocks / kMinSliceBlocks : 1;
    for (int64_t want = 1; want <= most; ++want) {
        Split s;
        s.k_per_split = (k_blocks + want - 1) / want;
        s.slices = (k_blocks + s.k_per_split - 1) / s.k_per_split;
        const int64_t rounds = (tiles * s.slices + resident - 1) / resident;
        double ns = static_cast<double>(rounds * (s.k_per_split + 1)) * step_ns;
        if (s.slices > 1)
            ns += reduce_ns_for(tokens) + 2.0 * static_cast<double>(s.slices * tokens * n * 4) / kPartialBytesPerNs;
        if (best_ns < 0.0 || ns < best_ns) best = s, best_ns = ns;
    }
    return best;
}

// Splits of the members of one batched GEMM launch: each member's slices
// come from one bound kmax on K blocks per workgroup, chosen by the same
// latency model over the whole launch (its workgroups share the GPU), and
// stay within what the member's partial buffer holds (cap[i] elements) and
// kMinSliceBlocks. A batch of one takes split_for's choice, which the
// member's workspace is sized for.
void batch_splits(int count, const int64_t* tiles, const int64_t* k_blocks, const int64_t* n, const int64_t* cap,
                  const Split* solo, int64_t tokens, Split* out) {
    if (count == 1) {
        out[0] = solo[0];
        return;
    }
    int64_t kb_max = 1;
    for (int i = 0; i < count; ++i) kb_max = k_blocks[i] > kb_max ? k_blocks[i] : kb_max;
    double best_ns = -1.0;
    for (int64_t kmax = kb_max; kmax >= 1; --kmax) {
        Split cand[kPrefillBatch];
        int64_t wgs = 0, steps = 0, partial_elems = 0;
        for (int i = 0; i < count; ++i) {
            const int64_t most_k = k_blocks[i] / kMinSliceBlocks > 1 ? k_blocks[i] / kMinSliceBlocks : 1;
            const int64_t most_cap = cap[i] / (tokens * n[i]) > 1 ? cap[i] / (tokens * n[i]) : 1;
            int64_t sl = (k_blocks[i] + kmax - 1) / kmax;
            sl = sl < most_k ? sl : most_k;
            sl = sl < most_cap ? sl : most_cap;
            cand[i].k_per_split = (k_blocks[i] + sl - 1) / sl;
            cand[i].slices = (k_blocks[i] + cand[i].k_per_split - 1) / cand[i].k_per_split;
            wgs += tiles[i] * cand[i].slices;
            steps = cand[i].k_per_split > steps ? cand[i].k_per_split : steps;
            if (cand[i].slices > 1) partial_elems += cand[i].slices * tokens * n[i];
        }
        const int64_t rounds = (wgs + resident_for(tokens) - 1) / resident_for(tokens);
        double ns = static_cast<double>(rounds * (steps + 1)) * step_ns_for(tokens);
        if (partial_elems > 0)
            ns += reduce_ns_for(tokens) + 2.0 * static_cast<double>(partial_elems * 4) / kPartialBytesPerNs;
        if (best_ns < 0.0 || ns < best_ns) {
            best_ns = ns;
            for (int i = 0; i < count; ++i) out[i] = cand[i];
        }
    }
}

// One launch of a phase's GEMMs (p[i].splits, k_per_split and partial set)
// and, when any member's K is split, one launch of the reductions. Up to 64
// tokens take the 64 x 128 block tile; otherwise the 128 x 256 block tile is
// used when it is the cheaper of the two by the round model below (K slices
// count as blocks of their own), and 128 x 128 when not.
constexpr double kWideStepCost = 1.65;
void launch_phase(GemmArgs* p, int count, int64_t tokens, hipStream_t stream) {
    const int64_t mt = (tokens + kBM - 1) / kBM;
    const bool small = tokens <= kBM / 2;  // one 64-row block holds every token
    bool wide = !small;
    int64_t wide_blocks = 0, narrow_blocks = 0, steps = 0;
    for (int i = 0; i < count; ++i) {
        wide_blocks += mt * ((p[i].n + 2 * kBN - 1) / (2 * kBN)) * p[i].splits;
        narrow_blocks += mt * ((p[i].n + kBN - 1) / kBN) * p[i].splits;
        steps = p[i].k_per_split > steps ? p[i].k_per_split : steps;
    }
    // Rounds of resident workgroups times K steps, a 128 x 256 step costing
    // kWideStepCost 128 x 128 steps (measured: twice the MFMAs at 1.65x the time).
    const double narrow_cost = static_cast<double>(((narrow_blocks + kResident - 1) / kResident) * (steps + 1));
    const double wide_cost =
        kWideStepCost * static_cast<double>(((wide_blocks + kResident - 1) / kResident) * (steps + 1));
    wide = wide && wide_cost < narrow_cost;
    const int64_t bn = wide ? 2 * kBN : kBN;
    GemmBatch gb;
    GemmBatch rb;
    int64_t x = 0, rx = 0;
    for (int i = 0; i < kPrefillBatch; ++i) {
        if (i >= count) {
            gb.begin[i] = rb.begin[i] = INT32_MAX;
            gb.p[i] = rb.p[i] = GemmArgs{};
            continue;
        }
        p[i].col_blocks = (p[i].n + bn - 1) / bn;
        gb.begin[i] = static_cast<int32_t>(x);
        rb.begin[i] = static_cast<int32_t>(rx);
        gb.p[i] = rb.p[i] = p[i];
        x += p[i].col_blocks * p[i].splits;
        if (p[i].splits > 1) {
            const int64_t width = p[i].out_scale ? p[i].out_ld : p[i].n;
            rx += (width + kBlock - 1) / kBlock;
        }
    }
    const dim3 grid(static_cast<unsigned>(x), static_cast<unsigned>(mt));
    const bool split = p[0].split != 0;  // every member of a batch agrees (launch_prefill_batch)
    if (small && split)
        hipLaunchKernelGGL((k_sign_gemm<1, 2, 1, true>), grid, dim3(kBlock), 0, stream, gb);
    else if (small)
        hipLaunchKernelGGL((k_sign_gemm<1, 2, 1, false>), grid, dim3(kBlock), 0, stream, gb);
    else if (wide && split)
        hipLaunchKernelGGL((k_sign_gemm<1, 4, 2, true>), grid, dim3(kBlock), 0, stream, gb);
    else if (wide)
        hipLaunchKernelGGL((k_sign_gemm<1, 4, 2, false>), grid, dim3(kBlock), 0, stream, gb);
    else if (split)
        hipLaunchKernelGGL((k_sign_gemm<2, 2, 2, true>), grid, dim3(kBlock), 0, stream, gb);
    else
        hipLaunchKernelGGL((k_sign_gemm<2, 2, 2, false>), grid, dim3(kBlock), 0, stream, gb);
    if (rx > 0) {
        const dim3 rgrid(static_cast<unsigned>(rx), static_cast<unsigned>(tokens < kRowsPerGridZ ? tokens : kRowsPerGridZ),
                         static_cast<unsigned>((tokens + kRowsPerGridZ - 1) / kRowsPerGridZ));
        hipLaunchKernelGGL(k_reduce_splits, rgrid, dim3(kBlock), 0, stream, rb);
    }
}

struct Scratch {
    int64_t xs16, scale1, lm16, scale2, partial, total;
    int64_t partial_elems;  // fp32 elements of the partial buffer
    Split s1, s2;
};

Scratch scratch_layout(const nq_linear_desc* d, int64_t tokens) {
    const Geometry g = geometry(d);
    const int64_t mt = (tokens + kBM - 1) / kBM;
    Scratch s{};
    s.s1 = split_for(mt * ((d->rank + kBN - 1) / kBN), g.nsc1, tokens, d->rank);
    s.s2 = split_for(mt * ((d->out_features + kBN - 1) / kBN), g.nsc2, tokens, d->out_features);
    const int64_t planes = d->prefill_operands == NQ_PREFILL_FP16_SPLIT ? 2 : 1;
    s.xs16 = 0;
    s.scale1 = s.xs16 + a256(tokens * g.nsc1 * kBK * 2 * planes);
    s.lm16 = s.scale1 + a256(tokens * 4);
    s.scale2 = s.lm16 + a256(tokens * g.nsc2 * kBK * 2 * planes);
    s.partial = s.scale2 + a256(tokens * 4);
    const int64_t p1 = s.s1.slices > 1 ? s.s1.slices * tokens * d->rank : 0;
    const int64_t p2 = s.s2.slices > 1 ? s.s2.slices * tokens * d->out_features : 0;
    s.partial_elems = p1 > p2 ? p1 : p2;
    s.total = s.partial + a256(4 * s.partial_elems);
    return s;
}

}  // namespace

namespace nq {

int64_t prefill_scratch_bytes(const nq_linear_desc* d, int64_t tokens) {
    if (!d->tiles) return 0;
    return scratch_layout(d, tokens).total;
}

bool prefill_path_applies(const nq_linear_desc* d, int64_t tokens) {
    return d->tiles != nullptr && tokens > 16 && tokens <= 65535 * int64_t(kBM);
}

int launch_prefill_batch(const nq_linear_desc* const* descs, int count, const void* const* xs, int x_dtype,
                         int64_t tokens, void* const* ys, int y_dtype, void* const* scratch, hipStream_t stream) {
    if (count < 1 || count > kPrefillBatch) return NQ_ERR_SHAPE;
    const int64_t header_words = tiles_header_words();
    auto aligned = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
    Geometry geo[kPrefillBatch];
    Scratch sl[kPrefillBatch];
    PrepBatch pb{};
    bool all_vec = true;
    int64_t pad_max = 0;
    const int split = descs[0]->prefill_operands == NQ_PREFILL_FP16_SPLIT ? 1 : 0;
    for (int i = 0; i < count; ++i) {
        const nq_linear_desc* d = descs[i];
        geo[i] = geometry(d);
        if (d->tiles_bytes < (header_words + geo[i].v_words + geo[i].u_words) * 4) return NQ_ERR_ARGUMENT;
        if (d->prefill_operands != descs[0]->prefill_operands) return NQ_ERR_ARGUMENT;
        // The GEMMs read the fp16 staging buffers with 16-byte vector loads.
        if (!aligned(scratch[i], 16)) return NQ_ERR_ALIGNMENT;
        sl[i] = scratch_layout(d, tokens);
        char* ws = static_cast<char*>(scratch[i]);
        PrepArgs& pa = pb.p[i];
        pa.act = xs[i];
        pa.ld = d->in_features;
        pa.colscale = d->scale_pre;
        pa.colscale_dtype = d->scale_dtype;
        // Vector row loads: 8 elements per load, 16-byte aligned rows.
        pa.vec = (d->in_features % 8 == 0 && aligned(xs[i], 16) && aligned(d->scale_pre, 16)) ? 1 : 0;
        pa.cols = d->in_features;
        pa.cols_pad = geo[i].nsc1 * kBK;
        pa.out16 = reinterpret_cast<_Float16*>(ws + sl[i].xs16);
        pa.split = split;
        pa.scale_out = reinterpret_cast<float*>(ws + sl[i].scale1);
        pa.max_mid_bits = static_cast<const uint32_t*>(d->tiles) + tiles_max_mid_word();
        pa.bound_scale_out = reinterpret_cast<float*>(ws + sl[i].scale2);
        all_vec = all_vec && pa.vec && d->scale_dtype == descs[0]->scale_dtype;
        pad_max = pa.cols_pad > pad_max ? pa.cols_pad : pad_max;
    }

    // Row passes: one launch, grid (tokens, members).
    const dim3 rows(static_cast<unsigned>(tokens), static_cast<unsigned>(count));
    bool prepped = false;
    if (all_vec && pad_max <= int64_t(kPrepChunksMax) * 8 * kBlock) {
        const bool short_rows = pad_max <= 2 * 8 * kBlock;
        const int sdt = descs[0]->scale_dtype;
#define NQ_PREP(ADT, SDT)                                                                                      \
    if (x_dtype == ADT && sdt == SDT) {                                                                        \
        if (short_rows)                                                                                        \
            hipLaunchKernelGGL((k_prep_rows_vec<ADT, SDT, 2>), rows, dim3(kBlock), 0, stream, pb);              \
        else                                                                                                   \
            hipLaunchKernelGGL((k_prep_rows_vec<ADT, SDT, kPrepChunksMax>), rows, dim3(kBlock), 0, stream, pb); \
        prepped = true;                                                                                        \
    }
#define NQ_PREP_S(ADT) NQ_PREP(ADT, NQ_DTYPE_F16) NQ_PREP(ADT, NQ_DTYPE_BF16) NQ_PREP(ADT, NQ_DTYPE_F32)
        NQ_PREP_S(NQ_DTYPE_BF16) NQ_PREP_S(NQ_DTYPE_F16) NQ_PREP_S(NQ_DTYPE_F32)
#undef NQ_PREP_S
#undef NQ_PREP
    }
    if (!prepped) hipLaunchKernelGGL(k_prep_rows, rows, dim3(kBlock), 0, stream, pb, x_dtype);

    const int64_t mt = (tokens + kBM - 1) / kBM;
    int64_t tiles[kPrefillBatch], kb[kPrefillBatch], n[kPrefillBatch], cap[kPrefillBatch];
    Split solo[kPrefillBatch], sp[kPrefillBatch];
    GemmArgs g[kPrefillBatch];

    // GEMM 1: lm16 = fp16 rank intermediate, scaled per row by scale2.
    for (int i = 0; i < count; ++i) {
        tiles[i] = mt * ((descs[i]->rank + kBN - 1) / kBN);
        kb[i] = geo[i].nsc1;
        n[i] = descs[i]->rank;
        cap[i] = sl[i].partial_elems;
        solo[i] = sl[i].s1;
    }
    batch_splits(count, tiles, kb, n, cap, solo, tokens, sp);
    for (int i = 0; i < count; ++i) {
        const nq_linear_desc* d = descs[i];
        char* ws = static_cast<char*>(scratch[i]);
        GemmArgs& a = g[i];
        a = GemmArgs{};
        a.a = pb.p[i].out16;
        a.m = tokens;
        a.kpad = geo[i].nsc1 * kBK;
        a.tiles = static_cast<const uint32_t*>(d->tiles) + header_words;
        a.n = d->rank;
        a.nb = geo[i].nsc1;
        a.row_scale = pb.p[i].scale_out;
        a.col_scale = d->scale_mid;
        a.col_scale_dtype = d->scale_dtype;
        a.out = ws + sl[i].lm16;
        a.out_dtype = NQ_DTYPE_F16;
        a.out_scale = pb.p[i].bound_scale_out;
        a.out_ld = geo[i].nsc2 * kBK;  // GEMM 1's column blocks cover exactly this width
        a.split = split;
        a.k_per_split = sp[i].k_per_split;
        a.splits = sp[i].slices;
        a.partial = sp[i].slices > 1 ? reinterpret_cast<float*>(ws + sl[i].partial) : nullptr;
    }
    launch_phase(g, count, tokens, stream);

    // GEMM 2: y = s_out * (lm16 · U±1ᵀ) / scale2 + salient columns + bias.
    for (int i = 0; i < count; ++i) {
        tiles[i] = mt * ((descs[i]->out_features + kBN - 1) / kBN);
        kb[i] = geo[i].nsc2;
        n[i] = descs[i]->out_features;
        solo[i] = sl[i].s2;
    }
    batch_splits(count, tiles, kb, n, cap, solo, tokens, sp);
    for (int i = 0; i < count; ++i) {
        const nq_linear_desc* d = descs[i];
        char* ws = static_cast<char*>(scratch[i]);
        GemmArgs& a = g[i];
        a = GemmArgs{};
        a.a = reinterpret_cast<const _Float16*>(ws + sl[i].lm16);
        a.m = tokens;
        a.kpad = geo[i].nsc2 * kBK;
        a.tiles = static_cast<const uint32_t*>(d->tiles) + header_words + geo[i].v_words;
        a.n = d->out_features;
        a.nb = geo[i].nsc2;
        a.row_scale = pb.p[i].bound_scale_out;
        a.col_scale = d->scale_post;
        a.col_scale_dtype = d->scale_dtype;
        a.x = xs[i];
        a.x_dtype = x_dtype;
        a.in = d->in_features;
        a.salient_count = d->salient_count;
        a.salient_indices = d->salient_indices;
        a.salient_values = d->salient_values;
        a.salient_dtype = d->salient_dtype;
        a.salient_scales = d->salient_scales;
        a.scale_dtype = d->scale_dtype;
        a.bias = d->bias;
        a.bias_dtype = d->bias_dtype;
        a.out = ys[i];
        a.out_dtype = y_dtype;
        a.split = split;
        a.k_per_split = sp[i].k_per_split;
        a.splits = sp[i].slices;
        a.partial = sp[i].slices > 1 ? reinterpret_cast<float*>(ws + sl[i].partial) : nullptr;
    }
    launch_phase(g, count, tokens, stream);
    return launch_status();
}

int launch_prefill(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y, int y_dtype,
                   void* scratch, hipStream_t stream) {
    return launch_prefill_batch(&d, 1, &x, x_dtype, tokens, &y, y_dtype, &scratch, stream);
}

}  // namespace nq

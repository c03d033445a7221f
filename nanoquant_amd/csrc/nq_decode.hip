// Fused single-launch decode path (tokens <= 16) for the packed binary
// low-rank linear on gfx950, for one linear or a batch of up to 8 linears in
// one launch.
//
//   lm[t, r] = s_mid[r] * Σ_i sgn(V[r, i]) * x[t, i] * s_in[i]     (stage 1)
//   y[t, o]  = s_out[o] * Σ_r sgn(U[o, r]) * lm[t, r] + salient + bias (stage 2)
//
// Weight layout ("tiles", built once by nq_prepare_tiles): a sign matrix
// [R rows, K cols] is cut into 16-row tiles and 128-column superchunks; word
// (tile, superchunk, lane) holds the 32 signs lane `l` feeds to four
// v_mfma_f32_16x16x32_f16 instructions, in the order their B operand needs
// them: lane l = 16*g + n carries row n and, for MFMA chunk m (32 columns),
// columns 32*m + 8*g + j (j < 8). Inside the word, the pair of signs for
// operand dword (m, d) sits at bits 15-s and 31-s with s = 4*m + d, so
//   dword = ((word << s) & 0x80008000) | 0x3C003C00
// is two fp16 ±1 values in one shift + one and_or. A wave reads one word per
// lane per superchunk: 256 contiguous bytes, fully coalesced.
//
// Launch structure (nq_linear_desc.decode_launch):
//   split (default): kernel 1 runs the stage-1 tiles (16 ranks each, the four
//     waves split the columns) of every linear in the batch and stores lm;
//     kernel 2 runs the stage-2 tiles (16 output rows each). The kernel
//     boundary is the grid-wide barrier.
//   fused: one kernel whose first workgroups are the stage-1 tiles and the
//     rest the stage-2 tiles. Stage-1 workgroups store lm write-through at
//     agent scope and then signal; stage-2 workgroups issue the loads of
//     their U tile first, then wait for their linear's signal (bounded spin),
//     so the U stream overlaps stage 1. Workgroups are dispatched in index
//     order, so every stage-1 workgroup is resident or finished before a
//     stage-2 workgroup can take its slot, and stage-1 workgroups never wait.
// On gfx950 the eight XCDs have separate L2s, so the fused signal and its
// polls travel through the fabric (agent-scope atomics); measured, that costs
// more than a graph-launched kernel boundary, hence split is the default.
//
// Activations enter the fp16 MFMA scaled by an exact per-token power of two
// (from the exact max |x * s_in| for one token, else max|x| * max|s_in|, and
// from the |lm| maximum), so the fp16 range cannot overflow; products are
// accumulated in fp32.
#include "nq_decode.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr int kWaves = 4;
constexpr int kTileRows = 16;
constexpr int kSuperCols = 128;
constexpr int kMaxTokens = 16;
constexpr int kMaxBatch = 8;
constexpr uint32_t kTilesMagic = 0x4e515432u;  // "NQT2"
constexpr uint32_t kSpinLimit = 1u << 22;

// Sync header at the start of each linear's tiles buffer. Every word lives on
// its own 256-byte line. All counters only ever increase, so nothing is reset
// between launches (graph replays included):
//   Counters are 64-bit (first two words of their line); flags are 32-bit and
//   compared wrap-safely.
//   ready slots: stage-1 workgroup b adds 1 to slot b % kReadySlots; with
//     c = that slot's participant count, the value it saw, v, gives the
//     launch index k = v / c, and v % c == c - 1 marks the slot complete.
//   ready root: each slot completer adds 1; the root completer of launch k
//     (old value == (k + 1) * used_slots - 1) writes k + 1 into every ready
//     flag.
//   arrive slots: stage-2 workgroup i adds 1 to slot i % kArriveSlots at its
//     start, which yields its own launch index k the same way; it then waits
//     until ready flag i % kReplicas reaches k + 1 (wrap-safe compare).
constexpr int kLine = 64;  // words per line
constexpr int kReadySlots = 16;
constexpr int kArriveSlots = 32;
constexpr int kReplicas = 64;
constexpr int kReadySlot0 = 0;
constexpr int kReadyRoot = kReadySlots;
constexpr int kArriveSlot0 = kReadyRoot + 1;
constexpr int kReplica0 = kArriveSlot0 + kArriveSlots;
constexpr int kMiscLine = kReplica0 + kReplicas;
constexpr int kHeaderLines = kMiscLine + 1;
constexpr int kHeaderWords = kHeaderLines * kLine;
// Words on the misc line.
enum : int { kMiscError = 0, kMiscMagic = 1, kMiscPreMax = 2 };

__host__ __device__ constexpr int line_word(int line) { return line * kLine; }

// Optional phase tracing (build with -DNQ_DECODE_TRACE): thread 0 of every
// workgroup stamps the 100 MHz real-time counter at each phase boundary into
// g_nq_trace[block * 8 + phase]. Compiled out of the shipped library.
#ifdef NQ_DECODE_TRACE
__device__ uint64_t* g_nq_trace;
#define NQ_TRACE(phase)                                                              \
    do {                                                                             \
        if (threadIdx.x == 0 && g_nq_trace)                                          \
            g_nq_trace[blockIdx.x * 8 + (phase)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define NQ_TRACE(phase) \
    do {                \
    } while (0)
#endif

__host__ __device__ inline int64_t tiles_of(int64_t rows) { return (rows + kTileRows - 1) / kTileRows; }
__host__ __device__ inline int64_t supers_of(int64_t cols) { return (cols + kSuperCols - 1) / kSuperCols; }

// ---------------------------------------------------------------------------
// Prepare: canonical words -> tile words.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void k_build_tiles(const uint32_t* __restrict__ canon,
                                                        int64_t rows, int64_t cols,
                                                        uint32_t* __restrict__ tiles) {
    const int64_t wpr = (cols + 31) / 32;
    const int64_t nsc = supers_of(cols);
    const int64_t total = tiles_of(rows) * nsc * 64;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(e & 63);
        const int64_t sc = (e >> 6) % nsc;
        const int64_t rt = (e >> 6) / nsc;
        const int64_t row = rt * kTileRows + (lane & 15);
        const int g = lane >> 4;
        uint32_t word = 0;
        if (row < rows) {
            for (int p = 0; p < 32; ++p) {
                const int h = p >> 4;
                const int s = 15 - (p & 15);
                const int m = s >> 2;
                const int d = s & 3;
                const int64_t col = sc * kSuperCols + 32 * m + 8 * g + 2 * d + h;
                if (col < cols) {
                    const uint32_t bit = (canon[row * wpr + (col >> 5)] >> (col & 31)) & 1u;
                    word |= bit << p;
                }
            }
        }
        tiles[e] = word;
    }
}

__global__ void k_init_header(uint32_t* header, const void* s_in, int scale_dtype, int64_t in) {
    // One block: zero the sync header, record max|s_in| (bounds x * s_in).
    __shared__ float red[kBlock];
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < in; i += kBlock) m = fmaxf(m, fabsf(nq::load_f32(s_in, scale_dtype, i)));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = kBlock / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    for (int i = threadIdx.x; i < kHeaderWords; i += kBlock) header[i] = 0;
    __syncthreads();
    if (threadIdx.x == 0) {
        header[line_word(kMiscLine) + kMiscMagic] = kTilesMagic;
        header[line_word(kMiscLine) + kMiscPreMax] = __float_as_uint(red[0]);
    }
}

// ---------------------------------------------------------------------------
// Fused kernel.
// ---------------------------------------------------------------------------

struct FusedArgs {
    int64_t in, rank, out;
    int64_t n1, n2;          // stage-1 / stage-2 workgroups (= row tiles of V / U)
    int64_t nsc1, nsc2;      // superchunks of in / rank
    const uint32_t* v_tiles;
    const uint32_t* u_tiles;
    uint32_t* header;
    const void* x;
    int x_dtype;
    int tokens;
    const void* s_in;
    const void* s_mid;
    const void* s_out;
    int scale_dtype;
    int64_t salient_count;
    const int32_t* salient_indices;
    const void* salient_values;
    int salient_dtype;
    const void* salient_scales;
    const void* bias;
    int bias_dtype;
    void* y;
    int y_dtype;
    float* lm;      // [16][n1*16]
    float* wgmax;   // [n1][16]
    int x_vec;      // x rows and s_in are 16-byte aligned with in % 8 == 0
};

struct FusedBatch {
    int count;
    int64_t first1[kMaxBatch + 1];  // stage-1 workgroup prefix per linear
    int64_t first2[kMaxBatch + 1];  // stage-2 workgroup prefix (after all stage-1)
    FusedArgs p[kMaxBatch];
};

// 2^e for an integer e in the fp32 normal range.
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

// Exponent e with 2^e <= v < 2^(e+1) for finite v > 0 (normals only; tiny values clamp).
__device__ __forceinline__ int exponent_of(float v) {
    const int e = static_cast<int>((__float_as_uint(v) >> 23) & 0xff) - 127;
    return e < -126 ? -126 : e;
}

// Exact power of two mapping values bounded by `bound` below 2^14 (fp16-safe).
__device__ __forceinline__ float range_scale(float bound) {
    if (!(bound > 0.0f)) return 1.0f;
    int e = 13 - exponent_of(bound);
    e = e > 100 ? 100 : (e < -100 ? -100 : e);
    return exp2i(e);
}

__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void hdr_store(uint32_t* header, int word, uint32_t v) {
    __hip_atomic_store(header + word, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 64-bit monotonic counter at the start of a header line (never wraps in practice).
__device__ __forceinline__ uint64_t hdr_add(uint32_t* header, int word) {
    return __hip_atomic_fetch_add(reinterpret_cast<uint64_t*>(header + word), uint64_t{1}, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
}

// Participants of slot `slot` when `count` participants are spread over `slots`.
__device__ __forceinline__ uint64_t slot_count(int slot, int slots, int64_t count) {
    return static_cast<uint64_t>(count / slots + (slot < count % slots ? 1 : 0));
}

// LDS of one workgroup for MT token rows and a column window of 4 * SC
// superchunks (SC per wave).
template <int MT, int SC>
struct alignas(16) Lds {
    static constexpr int kMT = MT;
    // Activation staging: MT rows of fp16, row stride padded by 8 halfs so the
    // 16 token rows of a ds_read_b128 land in different banks.
    static constexpr int kStageCols = 4 * SC * kSuperCols;
    static constexpr int kStride = kStageCols + 8;
    _Float16 act[MT * kStride];
    float red[kWaves][kMaxTokens][kTileRows];
    float tokscale[kMaxTokens];
    float wmax[kWaves];
};

__device__ __forceinline__ v8h expand_signs(uint32_t word, int m) {
    union {
        uint32_t u[4];
        v8h v;
    } r;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int s = 4 * m + d;
        r.u[d] = ((word << s) & 0x80008000u) | 0x3C003C00u;
    }
    return r.v;
}

// Eight consecutive elements [i, i + 8) of a typed buffer as fp32. The caller
// guarantees 16-byte alignment of element i (rows of length % 8 == 0 on
// 256-byte aligned allocations).
__device__ __forceinline__ void load8(const void* __restrict__ p, int dtype, int64_t i, float (&v)[8]) {
    if (dtype == NQ_DTYPE_F32) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 lo = q[0], hi = q[1];
        v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
        v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    } else {
        const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        if (dtype == NQ_DTYPE_BF16) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[2 * k] = __uint_as_float(w[k] << 16);
                v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                union { uint32_t u; _Float16 h[2]; } c;
                c.u = w[k];
                v[2 * k] = static_cast<float>(c.h[0]);
                v[2 * k + 1] = static_cast<float>(c.h[1]);
            }
        }
    }
}

// Elements [i, i + 8) of a row of length `limit`, zero past the end.
__device__ __forceinline__ void load8_tail(const void* __restrict__ p, int dtype, int64_t row_base,
                                           int64_t i, int64_t limit, float (&v)[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = i + k < limit ? nq::load_f32(p, dtype, row_base + i + k) : 0.0f;
}

__device__ __forceinline__ uint4 pack8_f16(const float (&v)[8]) {
    union { _Float16 h[8]; uint4 u; } r;
#pragma unroll
    for (int k = 0; k < 8; ++k) r.h[k] = static_cast<_Float16>(v[k]);
    return r.u;
}

// Stage columns [c0, c0 + ncols) of the activation rows into LDS as
// fp16(a * s * tokscale[t]); `s` (a per-column scale) may be null.
// act[t][c - c0]; rows t >= tokens are zero.
template <typename L>
__device__ __forceinline__ void stage_rows(L& lds, const void* __restrict__ act, int act_dtype,
                                           int64_t row_len, const void* __restrict__ colscale,
                                           int colscale_dtype, int tokens, int64_t c0, int ncols,
                                           bool vec) {
    const int nv = ncols >> 3;
    for (int t = 0; t < L::kMT; ++t) {
        uint4* dst = reinterpret_cast<uint4*>(&lds.act[t * L::kStride]);
        if (t >= tokens) {
            for (int j = threadIdx.x; j < nv; j += kBlock) dst[j] = make_uint4(0, 0, 0, 0);
            continue;
        }
        const float scale = lds.tokscale[t];
#pragma unroll 4
        for (int j = threadIdx.x; j < nv; j += kBlock) {
            const int64_t col = c0 + 8 * j;
            float v[8], w[8];
            if (vec && col + 8 <= row_len) {
                load8(act, act_dtype, t * row_len + col, v);
                if (colscale) load8(colscale, colscale_dtype, col, w);
            } else {
                load8_tail(act, act_dtype, t * row_len, col, row_len, v);
                if (colscale) load8_tail(colscale, colscale_dtype, 0, col, row_len, w);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] *= (colscale ? w[k] : 1.0f) * scale;
            dst[j] = pack8_f16(v);
        }
    }
}

// max |a[t, :]| for each token t < tokens, accumulated into lds.tokscale[t]
// (non-negative floats compare like their bit patterns).
template <typename L>
__device__ __forceinline__ void row_absmax(L& lds, const void* __restrict__ act, int act_dtype,
                                           int64_t row_len, int64_t row_stride, int tokens, bool vec) {
    const int64_t nv = (row_len + 7) >> 3;
    for (int t = 0; t < L::kMT && t < tokens; ++t) {
        float m = 0.0f;
#pragma unroll 4
        for (int64_t j = threadIdx.x; j < nv; j += kBlock) {
            float v[8];
            if (vec) load8(act, act_dtype, t * row_stride + 8 * j, v);
            else load8_tail(act, act_dtype, t * row_stride, 8 * j, row_len, v);
#pragma unroll
            for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(v[k]));
        }
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if ((threadIdx.x & 63) == 0 && m > 0.0f) {
            atomicMax(reinterpret_cast<unsigned int*>(&lds.tokscale[t]), __float_as_uint(m));
        }
    }
}

// One-token staging in a single memory round trip, split in two so the caller
// can issue other loads (the weight words) after the activation loads:
//   row_single_load:   every thread loads its NV vectors of a[col] * s[col];
//   row_single_stage:  the block reduces max |value| into a range scale
//                      (lds.tokscale[0]) and writes the scaled fp16 values to
//                      LDS row 0. Columns [n, ncols_pad) are zero.
// Requires ncols_pad <= 2048 * NV.
template <int NV>
struct RowRegs {
    float v[NV][8];
};

template <typename L>
__device__ __forceinline__ RowRegs<L::kStageCols / (8 * kBlock)> row_single_load(
    const void* __restrict__ act, int act_dtype, const void* __restrict__ colscale, int colscale_dtype,
    int64_t n, int ncols_pad, bool vec) {
    constexpr int NV = L::kStageCols / (8 * kBlock);
    RowRegs<NV> r;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int64_t col = 8 * (static_cast<int64_t>(threadIdx.x) + i * kBlock);
        float w[8];
        if (col < ncols_pad) {
            if (vec && col + 8 <= n) {
                load8(act, act_dtype, col, r.v[i]);
                if (colscale) load8(colscale, colscale_dtype, col, w);
            } else {
                load8_tail(act, act_dtype, 0, col, n, r.v[i]);
                if (colscale) load8_tail(colscale, colscale_dtype, 0, col, n, w);
            }
            if (colscale) {
#pragma unroll
                for (int k = 0; k < 8; ++k) r.v[i][k] *= w[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) r.v[i][k] = 0.0f;
        }
    }
    return r;
}

template <typename L, int NV>
__device__ __forceinline__ void row_single_stage(L& lds, RowRegs<NV>& r, int ncols_pad) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
        for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(r.v[i][k]));
    }
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) lds.wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    const float scale = range_scale(fmaxf(fmaxf(lds.wmax[0], lds.wmax[1]), fmaxf(lds.wmax[2], lds.wmax[3])));
    if (threadIdx.x == 0) lds.tokscale[0] = scale;
    uint4* dst = reinterpret_cast<uint4*>(&lds.act[0]);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = threadIdx.x + i * kBlock;
        if (8 * j < ncols_pad) {
#pragma unroll
            for (int k = 0; k < 8; ++k) r.v[i][k] *= scale;
            dst[j] = pack8_f16(r.v[i]);
        }
    }
}

// One wave's share of a 16-row tile: superchunks sc = w, w + 4, ... of the
// current stage window. Returns the partial D (token rows x 16 tile rows).
template <int MT, int SCMAX>
__device__ __forceinline__ v4f tile_mfma(const Lds<MT, SCMAX>& lds, const uint32_t (&words)[SCMAX],
                                         int64_t sc_first, int64_t nsc, int64_t window_sc0, v4f acc) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int i = 0; i < SCMAX; ++i) {
        const int64_t sc = sc_first + 4 * i + wave;
        if (sc < nsc) {
            const int base = static_cast<int>(sc - window_sc0) * kSuperCols + 8 * g;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                v8h a = {};
                if (t < MT) a = *reinterpret_cast<const v8h*>(&lds.act[t * Lds<MT, SCMAX>::kStride + base + 32 * m]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, expand_signs(words[i], m), acc, 0, 0, 0);
            }
        }
    }
    return acc;
}

template <int SCMAX>
__device__ __forceinline__ void load_words(uint32_t (&words)[SCMAX], const uint32_t* __restrict__ tile,
                                           int64_t sc_first, int64_t nsc) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < SCMAX; ++i) {
        const int64_t sc = sc_first + 4 * i + wave;
        words[i] = sc < nsc ? __builtin_nontemporal_load(tile + sc * 64 + lane) : 0u;
    }
}

// Sum the four waves' partial tiles (fixed order: deterministic). Returns the
// value for (t = tid / 16, n = tid % 16).
template <typename L>
__device__ __forceinline__ float reduce_waves(L& lds, v4f acc) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 4; ++i) lds.red[wave][4 * (lane >> 4) + i][lane & 15] = acc[i];
    __syncthreads();
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    return ((lds.red[0][t][n] + lds.red[1][t][n]) + lds.red[2][t][n]) + lds.red[3][t][n];
}

template <int MT, int SCMAX, bool FUSED>
__device__ __forceinline__ void stage1_tile(const FusedArgs& a, Lds<MT, SCMAX>& lds, int64_t rt) {
    NQ_TRACE(0);
    const uint32_t* tile = a.v_tiles + rt * a.nsc1 * 64;
    constexpr int kWindowSc = 4 * SCMAX;
    uint32_t words[SCMAX];

    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (MT == 1 && a.nsc1 <= kWindowSc) {
        // One token, one window: x * s_in loaded once (issued before the weight
        // words, so the in-order load counter lets staging start early), exact
        // range scale.
        const int ncols = static_cast<int>(a.nsc1 * kSuperCols);
        auto xr = row_single_load<Lds<MT, SCMAX>>(a.x, a.x_dtype, a.s_in, a.scale_dtype, a.in, ncols,
                                                  a.x_vec != 0);
        load_words<SCMAX>(words, tile, 0, a.nsc1);
        row_single_stage(lds, xr, ncols);
        __syncthreads();
        NQ_TRACE(1);
        acc = tile_mfma<MT, SCMAX>(lds, words, 0, a.nsc1, 0, acc);
    } else {
        load_words<SCMAX>(words, tile, 0, a.nsc1);
        // Per-token range scale: bound |x * s_in| by max|x| * max|s_in|.
        if (threadIdx.x < kMaxTokens) lds.tokscale[threadIdx.x] = 0.0f;
        __syncthreads();
        row_absmax(lds, a.x, a.x_dtype, a.in, a.in, a.tokens, a.x_vec != 0);
        __syncthreads();
        const float premax = __uint_as_float(a.header[line_word(kMiscLine) + kMiscPreMax]);
        if (threadIdx.x < kMaxTokens) lds.tokscale[threadIdx.x] = range_scale(lds.tokscale[threadIdx.x] * premax);
        __syncthreads();
        NQ_TRACE(1);
        for (int64_t w0 = 0; w0 < a.nsc1; w0 += kWindowSc) {
            if (w0 > 0) load_words<SCMAX>(words, tile, w0, a.nsc1);
            const int64_t c0 = w0 * kSuperCols;
            const int64_t cend = (w0 + kWindowSc < a.nsc1 ? w0 + kWindowSc : a.nsc1) * kSuperCols;
            stage_rows(lds, a.x, a.x_dtype, a.in, a.s_in, a.scale_dtype, a.tokens, c0,
                       static_cast<int>(cend - c0), a.x_vec != 0);
            __syncthreads();
            acc = tile_mfma<MT, SCMAX>(lds, words, w0, a.nsc1, w0, acc);
            __syncthreads();
        }
    }

    NQ_TRACE(2);
    const float sum = reduce_waves(lds, acc);
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    const int64_t r = rt * kTileRows + n;
    // Pad ranks [rank, 16 * n1) are written as zero: stage 2 stages whole rows and
    // its pad sign bits decode to +1.
    float lmv = 0.0f;
    if (t < a.tokens && r < a.rank) lmv = sum / lds.tokscale[t] * nq::load_f32(a.s_mid, a.scale_dtype, r);
    float am = fabsf(lmv);
    for (int off = 8; off >= 1; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 16));
    if (!FUSED) {
        // Split launch: the kernel boundary publishes lm to the stage-2 kernel.
        if (t < a.tokens) a.lm[t * (a.n1 * kTileRows) + r] = lmv;
        if (n == 0) a.wgmax[rt * kMaxTokens + t] = am;
        NQ_TRACE(3);
        NQ_TRACE(4);
        return;
    }
    // lm and the maxima are stored write-through at agent scope (no L2
    // writeback needed); the wait makes them complete before the signal.
    if (t < a.tokens) store_agent(&a.lm[t * (a.n1 * kTileRows) + r], lmv);
    if (n == 0) store_agent(&a.wgmax[rt * kMaxTokens + t], am);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    NQ_TRACE(3);
    if (threadIdx.x == 0) {
        const int slot = static_cast<int>(rt % kReadySlots);
        const uint64_t c = slot_count(slot, kReadySlots, a.n1);
        const uint64_t v = hdr_add(a.header, line_word(kReadySlot0 + slot));
        if (v % c == c - 1) {
            const uint64_t used = static_cast<uint64_t>(a.n1 < kReadySlots ? a.n1 : kReadySlots);
            const uint64_t k = v / c;
            const uint64_t w = hdr_add(a.header, line_word(kReadyRoot));
            if (w + 1 == (k + 1) * used) {
                const uint32_t flag = static_cast<uint32_t>(k + 1);
                for (int i = 0; i < kReplicas; ++i) hdr_store(a.header, line_word(kReplica0 + i), flag);
            }
        }
    }
    NQ_TRACE(4);
}

template <int MT, int SCMAX, bool FUSED>
__device__ __forceinline__ void stage2_tile(const FusedArgs& a, Lds<MT, SCMAX>& lds, int64_t rt) {
    NQ_TRACE(0);
    const uint32_t* tile = a.u_tiles + rt * a.nsc2 * 64;
    constexpr int kWindowSc = 4 * SCMAX;
    uint32_t words[SCMAX];
    load_words<SCMAX>(words, tile, 0, a.nsc2);  // prefetch before waiting

    // Fused launch: launch index from this workgroup's arrival, then poll its
    // ready flag with relaxed agent-scope loads; one acquire fence (L2
    // invalidate) at the end. Split launch: stage 1 finished in the previous
    // kernel.
    if (FUSED && threadIdx.x == 0) {
        const int slot = static_cast<int>(rt % kArriveSlots);
        const uint64_t c = slot_count(slot, kArriveSlots, a.n2);
        const uint32_t target = static_cast<uint32_t>(hdr_add(a.header, line_word(kArriveSlot0 + slot)) / c + 1);
        const uint32_t* flag = a.header + line_word(kReplica0 + static_cast<int>(rt % kReplicas));
        uint32_t spins = 0;
        while (static_cast<int32_t>(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
            if (++spins > kSpinLimit) {
                hdr_store(a.header, line_word(kMiscLine) + kMiscError, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    if (FUSED) __syncthreads();
    NQ_TRACE(1);

    const int64_t lm_ld = a.n1 * kTileRows;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (MT == 1 && a.nsc2 <= kWindowSc) {
        // One token, one window: lm loaded once, range scale from its own max.
        const int ncols = static_cast<int>(a.nsc2 * kSuperCols);
        auto lr = row_single_load<Lds<MT, SCMAX>>(a.lm, NQ_DTYPE_F32, nullptr, 0, lm_ld, ncols, true);
        row_single_stage(lds, lr, ncols);
        __syncthreads();
        acc = tile_mfma<MT, SCMAX>(lds, words, 0, a.nsc2, 0, acc);
    } else {
        // Per-token |lm| maximum over all stage-1 workgroups -> range scale.
        if (threadIdx.x < kMaxTokens) lds.tokscale[threadIdx.x] = 0.0f;
        __syncthreads();
        {
            const int t = threadIdx.x % MT;
            const int part = threadIdx.x / MT;
            float m = 0.0f;
            if (t < a.tokens) {
                for (int64_t b = part; b < a.n1; b += kBlock / MT) m = fmaxf(m, a.wgmax[b * kMaxTokens + t]);
            }
            if (m > 0.0f) atomicMax(reinterpret_cast<unsigned int*>(&lds.tokscale[t]), __float_as_uint(m));
        }
        __syncthreads();
        if (threadIdx.x < kMaxTokens) lds.tokscale[threadIdx.x] = range_scale(lds.tokscale[threadIdx.x]);
        __syncthreads();
        for (int64_t w0 = 0; w0 < a.nsc2; w0 += kWindowSc) {
            if (w0 > 0) load_words<SCMAX>(words, tile, w0, a.nsc2);
            const int64_t c0 = w0 * kSuperCols;
            const int64_t cend = (w0 + kWindowSc < a.nsc2 ? w0 + kWindowSc : a.nsc2) * kSuperCols;
            // lm rows have stride lm_ld (a multiple of 16, zeros past `rank`).
            stage_rows(lds, a.lm, NQ_DTYPE_F32, lm_ld, nullptr, 0, a.tokens, c0, static_cast<int>(cend - c0),
                       true);
            __syncthreads();
            acc = tile_mfma<MT, SCMAX>(lds, words, w0, a.nsc2, w0, acc);
            __syncthreads();
        }
    }

    NQ_TRACE(2);
    const float sum = reduce_waves(lds, acc);
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    const int64_t o = rt * kTileRows + n;
    if (t < a.tokens && o < a.out) {
        float v = sum / lds.tokscale[t] * nq::load_f32(a.s_out, a.scale_dtype, o);
        for (int64_t k = 0; k < a.salient_count; ++k) {
            float wv = nq::load_f32(a.salient_values, a.salient_dtype, o * a.salient_count + k);
            if (a.salient_scales) wv *= nq::load_f32(a.salient_scales, a.scale_dtype, k);
            v += wv * nq::load_f32(a.x, a.x_dtype, t * a.in + a.salient_indices[k]);
        }
        if (a.bias) v += nq::load_f32(a.bias, a.bias_dtype, o);
        nq::store_f32_as(a.y, a.y_dtype, t * a.out + o, v);
    }
    NQ_TRACE(3);
}

template <int MT, int SCMAX>
__global__ __launch_bounds__(kBlock) void k_decode_fused(const FusedBatch batch) {
    __shared__ Lds<MT, SCMAX> lds;
    const int64_t b = blockIdx.x;
    if (b < batch.first1[batch.count]) {
        int p = 0;
        while (p + 1 < batch.count && b >= batch.first1[p + 1]) ++p;
        stage1_tile<MT, SCMAX, true>(batch.p[p], lds, b - batch.first1[p]);
    } else {
        int p = 0;
        while (p + 1 < batch.count && b >= batch.first2[p + 1]) ++p;
        stage2_tile<MT, SCMAX, true>(batch.p[p], lds, b - batch.first2[p]);
    }
}

// Split launch, kernel 1: the stage-1 tiles of every linear in the batch.
template <int MT, int SCMAX>
__global__ __launch_bounds__(kBlock) void k_decode_stage1(const FusedBatch batch) {
    __shared__ Lds<MT, SCMAX> lds;
    const int64_t b = blockIdx.x;
    int p = 0;
    while (p + 1 < batch.count && b >= batch.first1[p + 1]) ++p;
    stage1_tile<MT, SCMAX, false>(batch.p[p], lds, b - batch.first1[p]);
}

// Split launch, kernel 2: the stage-2 tiles (block index offset by the
// stage-1 count so first2[] is shared with the fused grid).
template <int MT, int SCMAX>
__global__ __launch_bounds__(kBlock) void k_decode_stage2(const FusedBatch batch) {
    __shared__ Lds<MT, SCMAX> lds;
    const int64_t b = blockIdx.x + batch.first1[batch.count];
    int p = 0;
    while (p + 1 < batch.count && b >= batch.first2[p + 1]) ++p;
    stage2_tile<MT, SCMAX, false>(batch.p[p], lds, b - batch.first2[p]);
}

struct TilesGeometry {
    int64_t rt1, nsc1, rt2, nsc2;
    int64_t v_words, u_words;
};

TilesGeometry geometry(int64_t in, int64_t out, int64_t rank) {
    TilesGeometry g{};
    g.rt1 = tiles_of(rank);
    g.nsc1 = supers_of(in);
    g.rt2 = tiles_of(out);
    g.nsc2 = supers_of(rank);
    g.v_words = g.rt1 * g.nsc1 * 64;
    g.u_words = g.rt2 * g.nsc2 * 64;
    return g;
}

int64_t scratch_lm_bytes(const TilesGeometry& g) {
    return (kMaxTokens * g.rt1 * kTileRows * 4 + 255) & ~int64_t(255);
}

int64_t scratch_bytes(const TilesGeometry& g) {
    return scratch_lm_bytes(g) + ((g.rt1 * kMaxTokens * 4 + 255) & ~int64_t(255));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Fill one problem of a batch; NQ_OK or an error status.
int describe(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y, int y_dtype,
             void* scratch, FusedArgs& a, TilesGeometry& g) {
    g = geometry(d->in_features, d->out_features, d->rank);
    if (!d->tiles) return NQ_ERR_ARGUMENT;
    if (d->tiles_bytes < (kHeaderWords + g.v_words + g.u_words) * 4) return NQ_ERR_ARGUMENT;
    a = FusedArgs{};
    a.in = d->in_features;
    a.rank = d->rank;
    a.out = d->out_features;
    a.n1 = g.rt1;
    a.n2 = g.rt2;
    a.nsc1 = g.nsc1;
    a.nsc2 = g.nsc2;
    uint32_t* base = static_cast<uint32_t*>(const_cast<void*>(d->tiles));
    a.header = base;
    a.v_tiles = base + kHeaderWords;
    a.u_tiles = base + kHeaderWords + g.v_words;
    a.x = x;
    a.x_dtype = x_dtype;
    a.tokens = static_cast<int>(tokens);
    a.s_in = d->scale_pre;
    a.s_mid = d->scale_mid;
    a.s_out = d->scale_post;
    a.scale_dtype = d->scale_dtype;
    a.salient_count = d->salient_count;
    a.salient_indices = d->salient_indices;
    a.salient_values = d->salient_values;
    a.salient_dtype = d->salient_dtype;
    a.salient_scales = d->salient_scales;
    a.bias = d->bias;
    a.bias_dtype = d->bias_dtype;
    a.y = y;
    a.y_dtype = y_dtype;
    char* ws = static_cast<char*>(scratch);
    a.lm = reinterpret_cast<float*>(ws);
    a.wgmax = reinterpret_cast<float*>(ws + scratch_lm_bytes(g));
    a.x_vec = (d->in_features % 8 == 0 && aligned16(x) && aligned16(d->scale_pre)) ? 1 : 0;
    return NQ_OK;
}

template <int MT, int SCMAX>
void enqueue(const FusedBatch& batch, bool fused, hipStream_t stream) {
    const int64_t n1 = batch.first1[batch.count];
    const int64_t n = batch.first2[batch.count];
    if (fused) {
        hipLaunchKernelGGL((k_decode_fused<MT, SCMAX>), dim3(static_cast<unsigned>(n)), dim3(kBlock), 0, stream,
                           batch);
    } else {
        hipLaunchKernelGGL((k_decode_stage1<MT, SCMAX>), dim3(static_cast<unsigned>(n1)), dim3(kBlock), 0, stream,
                           batch);
        hipLaunchKernelGGL((k_decode_stage2<MT, SCMAX>), dim3(static_cast<unsigned>(n - n1)), dim3(kBlock), 0,
                           stream, batch);
    }
}

int launch_batch(FusedBatch& batch, int64_t tokens, int64_t max_nsc, bool fused, hipStream_t stream) {
    const int64_t n = batch.first2[batch.count];
    if (n <= 0 || n > 0x7fffffff) return NQ_ERR_SHAPE;
    if (tokens == 1 && max_nsc <= 32) {
        // in, rank <= 4096: one 4096-column window per stage, small register file.
        enqueue<1, 8>(batch, fused, stream);
    } else if (tokens == 1) {
        enqueue<1, 24>(batch, fused, stream);
    } else if (tokens <= 4) {
        enqueue<4, 6>(batch, fused, stream);
    } else {
        enqueue<16, 4>(batch, fused, stream);
    }
    return nq::launch_status();
}

}  // namespace

namespace nq {

int64_t tiles_header_words() { return kHeaderWords; }

int64_t decode_scratch_bytes(const nq_linear_desc* d, int64_t tokens) {
    (void)tokens;
    if (!d->tiles) return 0;
    return scratch_bytes(geometry(d->in_features, d->out_features, d->rank));
}

bool decode_path_applies(const nq_linear_desc* d, int64_t tokens) {
    return d->tiles != nullptr && tokens >= 1 && tokens <= kMaxTokens;
}

int launch_decode(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y,
                  int y_dtype, void* scratch, hipStream_t stream) {
    return launch_decode_batch(&d, 1, &x, x_dtype, tokens, &y, y_dtype, &scratch, stream);
}

int launch_decode_batch(const nq_linear_desc* const* descs, int count, const void* const* xs, int x_dtype,
                        int64_t tokens, void* const* ys, int y_dtype, void* const* scratch,
                        hipStream_t stream) {
    if (count < 1 || count > kMaxBatch) return NQ_ERR_SHAPE;
    if (tokens < 1 || tokens > kMaxTokens) return NQ_ERR_SHAPE;
    FusedBatch batch{};
    batch.count = count;
    int64_t max_nsc = 0;
    int64_t stage1 = 0;
    for (int i = 0; i < count; ++i) {
        if (descs[i]->decode_launch != descs[0]->decode_launch) return NQ_ERR_ARGUMENT;
        TilesGeometry g{};
        const int st = describe(descs[i], xs[i], x_dtype, tokens, ys[i], y_dtype, scratch[i], batch.p[i], g);
        if (st != NQ_OK) return st;
        batch.first1[i] = stage1;
        stage1 += g.rt1;
        max_nsc = g.nsc1 > max_nsc ? g.nsc1 : max_nsc;
        max_nsc = g.nsc2 > max_nsc ? g.nsc2 : max_nsc;
    }
    batch.first1[count] = stage1;
    int64_t stage2 = stage1;
    for (int i = 0; i < count; ++i) {
        batch.first2[i] = stage2;
        stage2 += batch.p[i].n2;
    }
    batch.first2[count] = stage2;
    return launch_batch(batch, tokens, max_nsc, descs[0]->decode_launch == NQ_DECODE_FUSED, stream);
}

}  // namespace nq

#ifdef NQ_DECODE_TRACE
extern "C" int nq_debug_set_trace(uint64_t* buffer) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_nq_trace), &buffer, sizeof(buffer)) == hipSuccess ? NQ_OK
                                                                                             : NQ_ERR_LAUNCH;
}
#endif

extern "C" int64_t nq_tiles_header_bytes(void) { return static_cast<int64_t>(kHeaderWords) * 4; }

extern "C" int64_t nq_tiles_bytes(int64_t in_features, int64_t out_features, int64_t rank) {
    if (in_features <= 0 || out_features <= 0 || rank <= 0) return -1;
    const TilesGeometry g = geometry(in_features, out_features, rank);
    return (kHeaderWords + g.v_words + g.u_words) * 4;
}

extern "C" int nq_prepare_tiles(const nq_linear_desc* d, void* tiles, int64_t tiles_bytes, void* stream) {
    if (!d || !tiles || !d->right_words || !d->left_words || !d->scale_pre) return NQ_ERR_ARGUMENT;
    if (d->in_features <= 0 || d->out_features <= 0 || d->rank <= 0) return NQ_ERR_SHAPE;
    if (!nq::is_float_dtype(d->scale_dtype)) return NQ_ERR_DTYPE;
    const TilesGeometry g = geometry(d->in_features, d->out_features, d->rank);
    if (tiles_bytes < (kHeaderWords + g.v_words + g.u_words) * 4) return NQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(tiles) % 256 != 0) return NQ_ERR_ALIGNMENT;
    auto s = static_cast<hipStream_t>(stream);
    uint32_t* base = static_cast<uint32_t*>(tiles);
    hipLaunchKernelGGL(k_init_header, dim3(1), dim3(kBlock), 0, s, base, d->scale_pre, d->scale_dtype,
                       d->in_features);
    auto grid_for = [](int64_t n) {
        const int64_t b = (n + kBlock - 1) / kBlock;
        return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
    };
    hipLaunchKernelGGL(k_build_tiles, dim3(grid_for(g.v_words)), dim3(kBlock), 0, s,
                       reinterpret_cast<const uint32_t*>(d->right_words), d->rank, d->in_features,
                       base + kHeaderWords);
    hipLaunchKernelGGL(k_build_tiles, dim3(grid_for(g.u_words)), dim3(kBlock), 0, s,
                       reinterpret_cast<const uint32_t*>(d->left_words), d->out_features, d->rank,
                       base + kHeaderWords + g.v_words);
    return nq::launch_status();
}

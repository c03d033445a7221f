// Tiled decode path (tokens <= 16) for the packed binary low-rank linear on
// gfx950, for one linear or a batch of up to 8 linears per launch.
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
// One workgroup computes one 16-row tile (16 ranks in stage 1, 16 output rows
// in stage 2). Its four waves split the K superchunks into contiguous ranges
// and work independently until the final cross-wave sum:
//   - a wave issues the loads of its activation window (x and s_in, or lm)
//     first and its sign words second, so the activations arrive first;
//   - it scales the window into fp16 with an exact per-token power of two
//     taken from the window's own max |value| (no block-wide reduction), parks
//     it in its private LDS rows and runs the MFMAs on it;
//   - the window result is divided by that power of two (exact) and added to
//     an fp32 total; the four wave totals are summed in a fixed order.
// Epilogue operands (s_mid, s_out, bias) are loaded at kernel start.
//
// Launch structure (nq_linear_desc.decode_launch):
//   split (default): kernel 1 runs the stage-1 tiles of every linear in the
//     batch and stores lm; kernel 2 runs the stage-2 tiles. The kernel
//     boundary is the grid-wide barrier.
//   fused: one kernel whose first workgroups are the stage-1 tiles and the
//     rest the stage-2 tiles. Stage-1 workgroups store lm write-through at
//     agent scope and then signal; stage-2 workgroups touch their first U
//     words, then wait for their linear's signal (bounded spin) and only then
//     load lm. Workgroups are dispatched in index order, so every stage-1
//     workgroup is resident or finished before a stage-2 workgroup can take
//     its slot, and stage-1 workgroups never wait.
// On gfx950 the eight XCDs have separate L2s, so the fused signal and its
// polls travel through the fabric (agent-scope atomics); measured, that costs
// more than a graph-launched kernel boundary, hence split is the default. Both
// run the same tile arithmetic in the same order: their outputs are identical.
#include "nq_decode.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr int kWaves = 4;
constexpr int kTileRows = 16;
constexpr int kSuperCols = 128;
constexpr int kMaxTokens = 16;
constexpr int kMaxBatch = 8;
constexpr uint32_t kTilesMagic = 0x4e515432u;  // "NQT2"
constexpr uint32_t kSpinLimit = 1u << 22;
constexpr int kAny = -1;  // dtype template tag: runtime dtype, element loads

// Sync header at the start of each linear's tiles buffer (used by the fused
// launch only). Every word lives on its own 256-byte line. All counters only
// ever increase, so nothing is reset between launches (graph replays included):
//   Counters are 64-bit (first two words of their line); flags are 32-bit and
//   compared wrap-safely.
//   ready slots: stage-1 workgroup b adds 1 to slot b % kReadySlots; with
//     c = that slot's participant count, the value it saw, v, gives the
//     launch index k = v / c, and v % c == c - 1 marks the slot complete.
//   ready root: each slot completer adds 1; the root completer of launch k
//     (old value == (k + 1) * used_slots - 1) writes k + 1 into every ready
//     flag.
//   arrive slots: each output tile i of a stage-2 workgroup adds 1 to slot
//     i % kArriveSlots at the workgroup's start, which yields the launch index
//     k the same way; the workgroup then waits until its ready flag (any of
//     the kReplicas copies) reaches k + 1 (wrap-safe compare).
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
enum : int { kMiscError = 0, kMiscMagic = 1 };

__host__ __device__ constexpr int line_word(int line) { return line * kLine; }

// Optional phase tracing (build with -DNQ_DECODE_TRACE): thread 0 of every
// workgroup stamps the 100 MHz real-time counter at each phase boundary into
// g_nq_trace[gblock * 8 + phase], gblock = the workgroup's index in the fused
// grid numbering. Compiled out of the shipped library.
#ifdef NQ_DECODE_TRACE
__device__ uint64_t* g_nq_trace;
#define NQ_TRACE(phase)                                                          \
    do {                                                                         \
        if (threadIdx.x == 0 && g_nq_trace)                                      \
            g_nq_trace[gblock * 8 + (phase)] = __builtin_amdgcn_s_memrealtime(); \
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

__global__ void k_init_header(uint32_t* header) {
    for (int i = threadIdx.x; i < kHeaderWords; i += kBlock) header[i] = 0;
    __syncthreads();
    if (threadIdx.x == 0) header[line_word(kMiscLine) + kMiscMagic] = kTilesMagic;
}

// ---------------------------------------------------------------------------
// Decode kernels.
// ---------------------------------------------------------------------------

struct FusedArgs {
    int64_t in, rank, out;
    int64_t n1, n2;          // row tiles of V / U (stage-1 workgroups = n1)
    int64_t g2;              // stage-2 workgroups (n2 tiles in groups of the launch's T)
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
    float* lm;      // [16][n1 * 16], ranks >= rank hold zero
};

struct FusedBatch {
    int count;
    int64_t first1[kMaxBatch + 1];  // stage-1 workgroup prefix per linear
    int64_t first2[kMaxBatch + 1];  // stage-2 workgroup prefix (after all stage-1)
    FusedArgs p[kMaxBatch];
};

// 2^e for an integer e in the fp32 normal range.
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

// Exponent e of a power of two mapping values bounded by `bound` below 2^14
// (fp16-safe); 0 when the bound is zero or not finite-positive.
__device__ __forceinline__ int range_exponent(float bound) {
    if (!(bound > 0.0f)) return 0;
    int e = static_cast<int>((__float_as_uint(bound) >> 23) & 0xff) - 127;
    e = 13 - (e < -126 ? -126 : e);
    return e > 100 ? 100 : (e < -100 ? -100 : e);
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

// --- activation vectors: 8 consecutive elements -------------------------------

// Raw bits of 8 elements of dtype D (kAny: already fp32, loaded element-wise).
template <int D>
struct Raw8 {
    v4u u[D == NQ_DTYPE_F32 ? 2 : 1];
};
template <>
struct Raw8<kAny> {
    float f[8];
};

// Elements [i, i + 8) of a row whose valid part ends at `limit`. Typed D: the
// caller guarantees i + 8 <= limit and 16-byte alignment (rows of length % 8 ==
// 0 on 16-byte aligned buffers). kAny: bounds-checked element loads.
template <int D>
__device__ __forceinline__ void raw_load(Raw8<D>& r, const void* __restrict__ p, int64_t row_base, int64_t i,
                                         int64_t limit, int rt_dtype) {
    if constexpr (D == kAny) {
#pragma unroll
        for (int k = 0; k < 8; ++k) r.f[k] = i + k < limit ? nq::load_f32(p, rt_dtype, row_base + i + k) : 0.0f;
    } else if constexpr (D == NQ_DTYPE_F32) {
        const v4u* q = reinterpret_cast<const v4u*>(static_cast<const float*>(p) + row_base + i);
        r.u[0] = q[0];
        r.u[1] = q[1];
    } else {
        r.u[0] = *reinterpret_cast<const v4u*>(static_cast<const uint16_t*>(p) + row_base + i);
    }
}

template <int D>
__device__ __forceinline__ void raw_zero(Raw8<D>& r) {
    if constexpr (D == kAny) {
#pragma unroll
        for (int k = 0; k < 8; ++k) r.f[k] = 0.0f;
    } else {
#pragma unroll
        for (int k = 0; k < (D == NQ_DTYPE_F32 ? 2 : 1); ++k) r.u[k] = v4u{0u, 0u, 0u, 0u};
    }
}

template <int D>
__device__ __forceinline__ void raw_unpack(const Raw8<D>& r, float (&v)[8]) {
    if constexpr (D == kAny) {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = r.f[k];
    } else if constexpr (D == NQ_DTYPE_F32) {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = __uint_as_float(r.u[k >> 2][k & 3]);
    } else if constexpr (D == NQ_DTYPE_BF16) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = __uint_as_float(r.u[0][k] << 16);
            v[2 * k + 1] = __uint_as_float(r.u[0][k] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            union {
                uint32_t u;
                _Float16 h[2];
            } c;
            c.u = r.u[0][k];
            v[2 * k] = static_cast<float>(c.h[0]);
            v[2 * k + 1] = static_cast<float>(c.h[1]);
        }
    }
}

// One element of a typed buffer as fp32 (kAny: runtime dtype switch).
template <int D>
__device__ __forceinline__ float load_one(const void* __restrict__ p, int64_t i, int rt_dtype) {
    if constexpr (D == kAny) {
        return nq::load_f32(p, rt_dtype, i);
    } else if constexpr (D == NQ_DTYPE_F32) {
        return static_cast<const float*>(p)[i];
    } else if constexpr (D == NQ_DTYPE_BF16) {
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
    } else {
        return static_cast<float>(static_cast<const _Float16*>(p)[i]);
    }
}

// --- one wave's window ----------------------------------------------------------

// A window is KW superchunks (128 * KW columns) of MT token rows. Vector e =
// lane + 64 * j (j < NV) covers token t = e / CV and columns 8 * (e % CV) of
// the window; vectors e >= MT * CV (a partial last j) are dead. When
// 64 % CV == 0 the column (and so its column scale) is the same for every j
// of a lane.
template <int MT, int KW>
struct Win {
    static constexpr int CW = KW * kSuperCols;          // columns per window
    static constexpr int CV = CW / 8;                   // 8-column vectors per token row
    static constexpr int NE = MT * CV;                  // vectors per window
    static constexpr int NV = (NE + 63) / 64;           // vectors per lane
    static constexpr bool kSameCol = (CV <= 64) && (64 % CV == 0);
    static constexpr int NS = kSameCol ? 1 : NV;        // column-scale vectors per lane
    static constexpr int kStride = CW + 8;              // LDS row stride (halfs)
};

// Registers of one wave's window: the activation vectors and the sign words
// of T tiles that share them.
template <int MT, int KW, int XD, int SD, int T>
struct WinRegs {
    Raw8<XD> x[Win<MT, KW>::NV];
    Raw8<SD> s[Win<MT, KW>::NS];
    bool live[Win<MT, KW>::NV];
    uint32_t w[T][KW];
};

// Where the activations of a window come from.
struct ActRef {
    const void* p;        // [tokens][ld]
    int dtype;            // runtime dtype (kAny loads)
    int64_t ld;           // row stride (elements)
    int64_t limit;        // valid columns (typed dtypes: a multiple of 8, >= 8)
    const void* colscale; // [limit] or null
    int colscale_dtype;
    int tokens;
};

// Issue the activation loads of a window. Typed dtypes load unconditionally
// from clamped addresses (no branches, so the compiler can count outstanding
// loads exactly) and record which vectors are live; dead vectors are zeroed
// when unpacked. Columns past the wave's range are dead, so their MFMAs add 0.
template <int MT, int KW, int XD, int SD, int T>
__device__ __forceinline__ void load_acts(WinRegs<MT, KW, XD, SD, T>& r, const ActRef& a, int64_t sc0,
                                          int64_t sc_end, int lane) {
    using W = Win<MT, KW>;
#pragma unroll
    for (int j = 0; j < W::NV; ++j) {
        const int e = lane + 64 * j;
        const int t = e / W::CV;
        const int64_t col = sc0 * kSuperCols + 8 * (e % W::CV);
        r.live[j] = e < W::NE && t < a.tokens && col < a.limit && sc0 + (8 * (e % W::CV)) / kSuperCols < sc_end;
        if constexpr (XD == kAny) {
            if (r.live[j]) raw_load<XD>(r.x[j], a.p, t * a.ld, col, a.limit, a.dtype);
            else raw_zero<XD>(r.x[j]);
        } else {
            const int64_t tc = t < a.tokens ? t : a.tokens - 1;
            const int64_t cc = col < a.limit - 8 ? col : a.limit - 8;
            raw_load<XD>(r.x[j], a.p, tc * a.ld, cc, a.limit, a.dtype);
        }
    }
    if (a.colscale) {
#pragma unroll
        for (int j = 0; j < W::NS; ++j) {
            const int e = lane + 64 * j;
            const int64_t col = sc0 * kSuperCols + 8 * (e % W::CV);
            if constexpr (SD == kAny) {
                if (col < a.limit) raw_load<SD>(r.s[j], a.colscale, 0, col, a.limit, a.colscale_dtype);
                else raw_zero<SD>(r.s[j]);
            } else {
                const int64_t cc = col < a.limit - 8 ? col : a.limit - 8;
                raw_load<SD>(r.s[j], a.colscale, 0, cc, a.limit, a.colscale_dtype);
            }
        }
    }
}

// Sign words of a window; superchunks past the tile's last load a valid word
// (their activations are zero).
template <int MT, int KW, int XD, int SD, int T>
__device__ __forceinline__ void load_words(WinRegs<MT, KW, XD, SD, T>& r, const uint32_t* const (&tiles)[T],
                                           int64_t sc0, int64_t nsc, int lane) {
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const int64_t sc = sc0 + i < nsc ? sc0 + i : nsc - 1;
            r.w[tt][i] = __builtin_nontemporal_load(tiles[tt] + sc * 64 + lane);
        }
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false);
    return fmaxf(x, __int_as_float(y));
}

// Max over the 16 lanes of each row of the wave (every lane gets its row's max).
__device__ __forceinline__ float row16_max(float v) {
    v = dpp_max<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_max<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_max<0x141>(v);  // row_half_mirror
    v = dpp_max<0x140>(v);  // row_mirror
    return v;
}

// Scale the window into fp16 (per-token exact power of two from the window's
// max |value|), write it to this wave's LDS rows act[t][c], and return the
// per-token exponents (uniform; tokens >= MT unused).
template <int MT, int KW, int XD, int SD, int T>
__device__ __forceinline__ void stage_window(const WinRegs<MT, KW, XD, SD, T>& r, bool has_colscale,
                                             _Float16* __restrict__ act, int lane, int (&expo)[MT]) {
    using W = Win<MT, KW>;
    // Two passes over the raw registers (max, then scale + pack) keep only one
    // vector unpacked at a time.
    auto values = [&](int j, float (&v)[8]) {
        raw_unpack<XD>(r.x[j], v);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = r.live[j] ? v[k] : 0.0f;
        if (has_colscale) {
            float s[8];
            raw_unpack<SD>(r.s[W::kSameCol ? 0 : j], s);
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] *= s[k];
        }
    };
    float m[W::NV];
#pragma unroll
    for (int j = 0; j < W::NV; ++j) {
        float v[8];
        values(j, v);
        m[j] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) m[j] = fmaxf(m[j], fabsf(v[k]));
    }
    // Per-token maxima: reduce each j over 16-lane rows, then combine rows.
    float tmax[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) tmax[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < W::NV; ++j) {
        const float rm = row16_max(m[j]);
#pragma unroll
        for (int row = 0; row < 4; ++row) {
            const int t = (16 * row + 64 * j) / W::CV;
            if (t < MT) {  // compile time: rows of a dead tail hold zeros
                const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 16 * row));
                tmax[t] = fmaxf(tmax[t], rv);
            }
        }
    }
    float scale[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        expo[t] = range_exponent(tmax[t]);
        scale[t] = exp2i(expo[t]);
    }
#pragma unroll
    for (int j = 0; j < W::NV; ++j) {
        const int e = lane + 64 * j;
        // Token of this vector; uniform per j unless a token row spans less than a wave.
        float sc;
        if constexpr (W::CV >= 64) {
            sc = scale[(64 * j) / W::CV < MT ? (64 * j) / W::CV : MT - 1];
        } else {
            sc = scale[0];
#pragma unroll
            for (int t = 1; t < MT; ++t) sc = (e / W::CV == t) ? scale[t] : sc;
        }
        float v[8];
        values(j, v);
        union {
            _Float16 h[8];
            v4u u;
        } pk;
#pragma unroll
        for (int k = 0; k < 8; ++k) pk.h[k] = static_cast<_Float16>(v[k] * sc);
        if (W::NE % 64 == 0 || e < W::NE) *reinterpret_cast<v4u*>(act + (e / W::CV) * W::kStride + 8 * (e % W::CV)) = pk.u;
    }
}

// MFMAs of one window (KW superchunks, of which the first nact are live) for
// each of the T tiles. Every lane reads an A row: lanes of token rows >= MT
// read row t % MT, which only feeds D rows that are never used. One accumulator per tile and 32-column chunk
// keeps the MFMA chains short; they are summed in a fixed order.
template <int MT, int KW, int XD, int SD, int T, bool SKIP>
__device__ __forceinline__ void window_mfma(const WinRegs<MT, KW, XD, SD, T>& r, const _Float16* __restrict__ act,
                                            int nact, int lane, v4f (&out)[T]) {
    using W = Win<MT, KW>;
    const int g = lane >> 4;
    const _Float16* row = act + ((lane & 15) % MT) * W::kStride + 8 * g;
    v4f acc[T][4];
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[tt][m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < KW; ++i) {
        // Superchunks past the wave's range hold zero activations; SKIP
        // branches over them (uniform), otherwise they add exact zeros.
        if (!SKIP || i < nact) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const v8h a = *reinterpret_cast<const v8h*>(row + i * kSuperCols + 32 * m);
#pragma unroll
                for (int tt = 0; tt < T; ++tt)
                    acc[tt][m] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(a, expand_signs(r.w[tt][i], m), acc[tt][m], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < T; ++tt) out[tt] = (acc[tt][0] + acc[tt][1]) + (acc[tt][2] + acc[tt][3]);
}

// Order this wave's LDS writes before its own reads (waves never share rows).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

// D row of MFMA register q in this lane is token 4 * (lane / 16) + q.
template <int MT>
__device__ __forceinline__ void add_scaled(v4f& tot, const v4f& acc, const int (&expo)[MT], int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        int e;
        if constexpr (MT <= 4) {
            e = expo[q < MT ? q : 0];
        } else {
            const int grp = lane >> 4;
            e = expo[q];
#pragma unroll
            for (int gg = 1; gg < 4; ++gg) e = (grp == gg && 4 * gg + q < MT) ? expo[4 * gg + q] : e;
        }
        tot[q] += acc[q] * exp2i(-e);
    }
}

// Shared memory of one workgroup.
template <int MT, int KW, int T>
struct alignas(16) TileLds {
    _Float16 act[kWaves][MT * Win<MT, KW>::kStride];
    float red[T][kWaves][kMaxTokens][kTileRows];
};

// One wave's share of T 16-row tiles: superchunks [s_begin, s_end) in windows
// of KW. Writes the wave's fp32 partial D (tokens x 16 rows) of each tile.
template <int MT, int KW, int XD, int SD, int T, bool WORDS_FIRST, bool SKIP>
__device__ __forceinline__ void wave_tile(const ActRef& act_ref, const uint32_t* const (&tiles)[T], int64_t nsc,
                                          int64_t s_begin, int64_t s_end, _Float16* __restrict__ act, int lane,
                                          v4f (&tot)[T]) {
#pragma unroll
    for (int tt = 0; tt < T; ++tt) tot[tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t sc0 = s_begin; sc0 < s_end; sc0 += KW) {
        WinRegs<MT, KW, XD, SD, T> r;
        if (WORDS_FIRST) {
            load_words(r, tiles, sc0, nsc, lane);
            __builtin_amdgcn_sched_barrier(0);
            load_acts(r, act_ref, sc0, s_end, lane);
        } else {
            load_acts(r, act_ref, sc0, s_end, lane);
            __builtin_amdgcn_sched_barrier(0);
            load_words(r, tiles, sc0, nsc, lane);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load is issued before any use
        int expo[MT];
        stage_window(r, act_ref.colscale != nullptr, act, lane, expo);
        wave_lds_sync();
        v4f acc[T];
        window_mfma<MT, KW, XD, SD, T, SKIP>(r, act, static_cast<int>(s_end - sc0 < KW ? s_end - sc0 : KW), lane, acc);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) add_scaled<MT>(tot[tt], acc[tt], expo, lane);
        wave_lds_sync();  // the next window rewrites the rows this one read
    }
}

// Contiguous superchunk range of wave `w` out of nsc.
__device__ __forceinline__ void wave_range(int64_t nsc, int w, int64_t& b, int64_t& e) {
    const int64_t q = (nsc + kWaves - 1) / kWaves;
    b = q * w < nsc ? q * w : nsc;
    e = b + q < nsc ? b + q : nsc;
}

// Sum the four waves' partial tiles (fixed order: deterministic). Returns,
// per tile, the value for (t = tid / 16, n = tid % 16).
template <int MT, int KW, int T>
__device__ __forceinline__ void reduce_waves(TileLds<MT, KW, T>& lds, const v4f (&tot)[T], float (&sum)[T]) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) lds.red[tt][wave][4 * (lane >> 4) + i][lane & 15] = tot[tt][i];
    __syncthreads();
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
        sum[tt] = ((lds.red[tt][0][t][n] + lds.red[tt][1][t][n]) + lds.red[tt][2][t][n]) + lds.red[tt][3][t][n];
}

template <int MT, int KW, int XD, int SD, bool FUSED>
__device__ __forceinline__ void stage1_tile(const FusedArgs& a, TileLds<MT, KW, 1>& lds, int64_t rt,
                                            [[maybe_unused]] int64_t gblock) {
    NQ_TRACE(0);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    const int64_t r = rt * kTileRows + n;
    // Epilogue operand first (typed, unconditional): its latency hides under
    // the main loads.
    const float smid = load_one<SD>(a.s_mid, r < a.rank ? r : a.rank - 1, a.scale_dtype);

    int64_t sb, se;
    wave_range(a.nsc1, wave, sb, se);
    const ActRef xr{a.x, a.x_dtype, a.in, a.in, a.s_in, a.scale_dtype, a.tokens};
    const uint32_t* const tiles[1] = {a.v_tiles + rt * a.nsc1 * 64};
    v4f tot[1];
    wave_tile<MT, KW, XD, SD, 1, false, FUSED>(xr, tiles, a.nsc1, sb, se, lds.act[wave], lane, tot);
    NQ_TRACE(1);
    float sums[1];
    reduce_waves(lds, tot, sums);
    const float sum = sums[0];
    NQ_TRACE(2);
    // Pad ranks [rank, 16 * n1) are written as zero: stage 2 reads whole rows
    // and their sign bits decode to +1.
    const float lmv = (t < a.tokens && r < a.rank) ? sum * smid : 0.0f;
    float* dst = &a.lm[t * (a.n1 * kTileRows) + r];
    if (!FUSED) {
        // Split launch: the kernel boundary publishes lm to the stage-2 kernel.
        if (t < a.tokens) *dst = lmv;
        NQ_TRACE(3);
        return;
    }
    // lm is stored write-through at agent scope (no L2 writeback needed); the
    // wait makes it complete before the signal.
    if (t < a.tokens) store_agent(dst, lmv);
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
}

// Fused launch: wait until every stage-1 workgroup of this launch has signalled.
// Arrivals are counted per output tile (each of the group's tiles adds 1 to
// slot tile % kArriveSlots), so the per-slot count of a launch depends only on
// the layer, not on how many tiles a workgroup takes: launches of one layer
// with different grouping keep consistent launch indices.
template <int T>
__device__ __forceinline__ void wait_ready(const FusedArgs& a, int64_t grp) {
    if (threadIdx.x == 0) {
        uint32_t target = 0;
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const int64_t tile = grp * T + tt;
            if (tile < a.n2) {
                const int slot = static_cast<int>(tile % kArriveSlots);
                const uint64_t v = hdr_add(a.header, line_word(kArriveSlot0 + slot));
                if (tt == 0) target = static_cast<uint32_t>(v / slot_count(slot, kArriveSlots, a.n2) + 1);
            }
        }
        const uint32_t* flag = a.header + line_word(kReplica0 + static_cast<int>(grp % kReplicas));
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
    __syncthreads();
}

// Stage-2 workgroup `grp`: output tiles grp * T + tt (tt < T) share each lm window.
template <int MT, int KW, int SD, int T, bool FUSED>
__device__ __forceinline__ void stage2_tile(const FusedArgs& a, TileLds<MT, KW, T>& lds, int64_t grp,
                                            [[maybe_unused]] int64_t gblock) {
    NQ_TRACE(0);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    int64_t o[T];
    float sout[T];
    const uint32_t* tiles[T];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
        const int64_t rt = grp * T + tt;
        o[tt] = rt * kTileRows + n;
        sout[tt] = load_one<SD>(a.s_out, o[tt] < a.out ? o[tt] : a.out - 1, a.scale_dtype);
        // A tile past the last one (partial group) reuses the last tile's words; it is never stored.
        tiles[tt] = a.u_tiles + (rt < a.n2 ? rt : a.n2 - 1) * a.nsc2 * 64;
    }

    int64_t sb, se;
    wave_range(a.nsc2, wave, sb, se);
    const int64_t lm_ld = a.n1 * kTileRows;
    // lm rows have stride lm_ld (a multiple of 16, zeros past `rank`), so whole
    // 8-element vectors up to lm_ld are valid.
    const ActRef lr{a.lm, NQ_DTYPE_F32, lm_ld, lm_ld, nullptr, 0, a.tokens};
    v4f tot[T];
    if (FUSED) {
        // Touch the first window's words before waiting, so the U stream
        // overlaps stage 1; the loop below then hits in cache.
        if (sb < se) {
#pragma unroll
            for (int tt = 0; tt < T; ++tt) (void)__builtin_nontemporal_load(tiles[tt] + sb * 64 + lane);
        }
        wait_ready<T>(a, grp);
        NQ_TRACE(1);
        wave_tile<MT, KW, NQ_DTYPE_F32, NQ_DTYPE_F32, T, true, true>(lr, tiles, a.nsc2, sb, se, lds.act[wave], lane,
                                                                     tot);
    } else {
        NQ_TRACE(1);
        wave_tile<MT, KW, NQ_DTYPE_F32, NQ_DTYPE_F32, T, false, false>(lr, tiles, a.nsc2, sb, se, lds.act[wave], lane,
                                                                       tot);
    }
    NQ_TRACE(2);
    float sum[T];
    reduce_waves(lds, tot, sum);
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
        if (t < a.tokens && o[tt] < a.out) {
            float v = sum[tt] * sout[tt];
            for (int64_t k = 0; k < a.salient_count; ++k) {
                float wv = nq::load_f32(a.salient_values, a.salient_dtype, o[tt] * a.salient_count + k);
                if (a.salient_scales) wv *= nq::load_f32(a.salient_scales, a.scale_dtype, k);
                v += wv * nq::load_f32(a.x, a.x_dtype, t * a.in + a.salient_indices[k]);
            }
            if (a.bias) v += nq::load_f32(a.bias, a.bias_dtype, o[tt]);
            nq::store_f32_as(a.y, a.y_dtype, t * a.out + o[tt], v);
        }
    }
    NQ_TRACE(3);
}

// Linear of block b: the number of prefix entries first[1..count-1] <= b
// (independent scalar loads, no dependent chain).
__device__ __forceinline__ int member_of(const int64_t (&first)[kMaxBatch + 1], int count, int64_t b) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatch; ++i) p += (i < count && b >= first[i]) ? 1 : 0;
    return p;
}

// Kernel configurations: MT token rows, KW1 / KW2 superchunks per wave window
// in stage 1 / stage 2, XD / SD the dtypes of x and s_in (kAny: runtime), T2
// the output tiles per stage-2 workgroup.
template <int MT, int KW1, int KW2, int XD, int SD, int T2>
__global__ __launch_bounds__(kBlock) void k_decode_fused(const FusedBatch batch) {
    const int64_t b = blockIdx.x;
    if (b < batch.first1[batch.count]) {
        __shared__ TileLds<MT, KW1, 1> lds1;
        const int p = member_of(batch.first1, batch.count, b);
        stage1_tile<MT, KW1, XD, SD, true>(batch.p[p], lds1, b - batch.first1[p], b);
    } else {
        __shared__ TileLds<MT, KW2, T2> lds2;
        const int p = member_of(batch.first2, batch.count, b);
        stage2_tile<MT, KW2, SD, T2, true>(batch.p[p], lds2, b - batch.first2[p], b);
    }
}

// Split launch, kernel 1: the stage-1 tiles of every linear in the batch.
template <int MT, int KW, int XD, int SD>
__global__ __launch_bounds__(kBlock) void k_decode_stage1(const FusedBatch batch) {
    __shared__ TileLds<MT, KW, 1> lds;
    const int64_t b = blockIdx.x;
    const int p = member_of(batch.first1, batch.count, b);
    stage1_tile<MT, KW, XD, SD, false>(batch.p[p], lds, b - batch.first1[p], b);
}

// Split launch, kernel 2: the stage-2 tiles (block index offset by the
// stage-1 count so first2[] is shared with the fused grid).
template <int MT, int KW, int SD, int T>
__global__ __launch_bounds__(kBlock) void k_decode_stage2(const FusedBatch batch) {
    __shared__ TileLds<MT, KW, T> lds;
    const int64_t b = blockIdx.x + batch.first1[batch.count];
    const int p = member_of(batch.first2, batch.count, b);
    stage2_tile<MT, KW, SD, T, false>(batch.p[p], lds, b - batch.first2[p], b);
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

int64_t scratch_bytes(const TilesGeometry& g) {
    return (kMaxTokens * g.rt1 * kTileRows * 4 + 255) & ~int64_t(255);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Fill one problem of a batch; NQ_OK or an error status.
int describe(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y, int y_dtype,
             void* scratch, FusedArgs& a, TilesGeometry& g) {
    g = geometry(d->in_features, d->out_features, d->rank);
    if (!d->tiles) return NQ_ERR_ARGUMENT;
    if (d->tiles_bytes < (kHeaderWords + g.v_words + g.u_words) * 4) return NQ_ERR_ARGUMENT;
    if (!aligned16(scratch)) return NQ_ERR_ALIGNMENT;
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
    a.lm = static_cast<float*>(scratch);
    return NQ_OK;
}

// Typed vector loads of x and s_in need rows of length % 8 == 0 and 16-byte
// aligned bases; anything else takes the element-wise kAny configuration.
bool typed_ok(const FusedArgs& a) {
    return a.in % 8 == 0 && aligned16(a.x) && aligned16(a.s_in);
}

// Split launch: stage-1 configuration (KW1 superchunks per window, typed bf16 /
// f16 / f32 x with fp16 scales, element-wise kAny otherwise).
template <int MT, int KW1>
void enqueue_stage1(const FusedBatch& batch, bool typed, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(batch.first1[batch.count]));
    const int xd = batch.p[0].x_dtype;
    const int sd = batch.p[0].scale_dtype;
    if (typed && sd == NQ_DTYPE_F16 && xd == NQ_DTYPE_BF16) {
        hipLaunchKernelGGL((k_decode_stage1<MT, KW1, NQ_DTYPE_BF16, NQ_DTYPE_F16>), grid, dim3(kBlock), 0, stream,
                           batch);
    } else if (typed && sd == NQ_DTYPE_F16 && xd == NQ_DTYPE_F16) {
        hipLaunchKernelGGL((k_decode_stage1<MT, KW1, NQ_DTYPE_F16, NQ_DTYPE_F16>), grid, dim3(kBlock), 0, stream,
                           batch);
    } else if (typed && sd == NQ_DTYPE_F16 && xd == NQ_DTYPE_F32) {
        hipLaunchKernelGGL((k_decode_stage1<MT, KW1, NQ_DTYPE_F32, NQ_DTYPE_F16>), grid, dim3(kBlock), 0, stream,
                           batch);
    } else {
        hipLaunchKernelGGL((k_decode_stage1<MT, KW1, kAny, kAny>), grid, dim3(kBlock), 0, stream, batch);
    }
}

template <int MT, int KW2, int T2>
void enqueue_stage2(const FusedBatch& batch, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(batch.first2[batch.count] - batch.first1[batch.count]));
    if (batch.p[0].scale_dtype == NQ_DTYPE_F16) {
        hipLaunchKernelGGL((k_decode_stage2<MT, KW2, NQ_DTYPE_F16, T2>), grid, dim3(kBlock), 0, stream, batch);
    } else {
        hipLaunchKernelGGL((k_decode_stage2<MT, KW2, kAny, T2>), grid, dim3(kBlock), 0, stream, batch);
    }
}

// Fused launch: element-wise activation loads and a window of 8 or 24
// superchunks (dead superchunks skipped), so its few configurations cover
// every shape; a single-window wave computes the same values for any window
// size, so fused and split outputs are identical.
template <int MT, int KW1, int KW2, int T2>
void enqueue_fused(const FusedBatch& batch, hipStream_t stream) {
    hipLaunchKernelGGL((k_decode_fused<MT, KW1, KW2, kAny, kAny, T2>),
                       dim3(static_cast<unsigned>(batch.first2[batch.count])), dim3(kBlock), 0, stream, batch);
}

// Output tiles per stage-2 workgroup: two when the batch has enough tiles to
// fill the GPU twice over (each lm window then feeds two tiles' MFMAs).
constexpr int64_t kPairTilesFrom = 512;

// Superchunks per wave of a K of nsc superchunks.
int64_t per_wave(int64_t nsc) { return (nsc + kWaves - 1) / kWaves; }

int launch_batch(FusedBatch& batch, int64_t tokens, int64_t max_nsc1, int64_t max_nsc2, bool typed, bool fused,
                 hipStream_t stream) {
    int64_t tiles2 = 0;
    for (int i = 0; i < batch.count; ++i) tiles2 += batch.p[i].n2;
    const int t2 = (tokens == 1 && tiles2 >= kPairTilesFrom) ? 2 : 1;
    int64_t stage2 = batch.first1[batch.count];
    for (int i = 0; i < batch.count; ++i) {
        batch.p[i].g2 = (batch.p[i].n2 + t2 - 1) / t2;
        batch.first2[i] = stage2;
        stage2 += batch.p[i].g2;
    }
    batch.first2[batch.count] = stage2;
    const int64_t n = batch.first2[batch.count];
    if (n <= 0 || n > 0x7fffffff) return NQ_ERR_SHAPE;
    const int64_t q1 = per_wave(max_nsc1), q2 = per_wave(max_nsc2);
    if (fused) {
        if (tokens == 1) {
            const bool w1 = q1 > 8, w2 = q2 > 8;
            if (t2 == 2) {
                if (!w1 && !w2) enqueue_fused<1, 8, 8, 2>(batch, stream);
                else if (w1 && !w2) enqueue_fused<1, 24, 8, 2>(batch, stream);
                else if (!w1 && w2) enqueue_fused<1, 8, 24, 2>(batch, stream);
                else enqueue_fused<1, 24, 24, 2>(batch, stream);
            } else {
                if (!w1 && !w2) enqueue_fused<1, 8, 8, 1>(batch, stream);
                else if (w1 && !w2) enqueue_fused<1, 24, 8, 1>(batch, stream);
                else if (!w1 && w2) enqueue_fused<1, 8, 24, 1>(batch, stream);
                else enqueue_fused<1, 24, 24, 1>(batch, stream);
            }
        } else if (tokens <= 4) {
            enqueue_fused<4, 4, 4, 1>(batch, stream);
        } else {
            enqueue_fused<16, 2, 2, 1>(batch, stream);
        }
        return nq::launch_status();
    }
    if (tokens == 1) {
        // One token: the window covers a wave's whole K range when it fits,
        // sized to that range so no MFMA runs on dead superchunks.
        if (q1 <= 4) enqueue_stage1<1, 4>(batch, typed, stream);
        else if (q1 <= 8) enqueue_stage1<1, 8>(batch, typed, stream);
        else enqueue_stage1<1, 24>(batch, typed, stream);
        if (t2 == 2) {
            if (q2 <= 2) enqueue_stage2<1, 2, 2>(batch, stream);
            else if (q2 <= 4) enqueue_stage2<1, 4, 2>(batch, stream);
            else if (q2 <= 6) enqueue_stage2<1, 6, 2>(batch, stream);
            else if (q2 <= 8) enqueue_stage2<1, 8, 2>(batch, stream);
            else enqueue_stage2<1, 24, 2>(batch, stream);
        } else {
            if (q2 <= 2) enqueue_stage2<1, 2, 1>(batch, stream);
            else if (q2 <= 4) enqueue_stage2<1, 4, 1>(batch, stream);
            else if (q2 <= 6) enqueue_stage2<1, 6, 1>(batch, stream);
            else if (q2 <= 8) enqueue_stage2<1, 8, 1>(batch, stream);
            else enqueue_stage2<1, 24, 1>(batch, stream);
        }
    } else if (tokens <= 4) {
        enqueue_stage1<4, 4>(batch, typed, stream);
        enqueue_stage2<4, 4, 1>(batch, stream);
    } else {
        enqueue_stage1<16, 2>(batch, typed, stream);
        enqueue_stage2<16, 2, 1>(batch, stream);
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
    int64_t max_nsc1 = 0, max_nsc2 = 0;
    int64_t stage1 = 0;
    bool typed = true;
    for (int i = 0; i < count; ++i) {
        if (descs[i]->decode_launch != descs[0]->decode_launch) return NQ_ERR_ARGUMENT;
        if (descs[i]->scale_dtype != descs[0]->scale_dtype) return NQ_ERR_DTYPE;
        TilesGeometry g{};
        const int st = describe(descs[i], xs[i], x_dtype, tokens, ys[i], y_dtype, scratch[i], batch.p[i], g);
        if (st != NQ_OK) return st;
        typed = typed && typed_ok(batch.p[i]);
        batch.first1[i] = stage1;
        stage1 += g.rt1;
        max_nsc1 = g.nsc1 > max_nsc1 ? g.nsc1 : max_nsc1;
        max_nsc2 = g.nsc2 > max_nsc2 ? g.nsc2 : max_nsc2;
    }
    batch.first1[count] = stage1;
    return launch_batch(batch, tokens, max_nsc1, max_nsc2, typed, descs[0]->decode_launch == NQ_DECODE_FUSED,
                        stream);
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
    hipLaunchKernelGGL(k_init_header, dim3(1), dim3(kBlock), 0, s, base);
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

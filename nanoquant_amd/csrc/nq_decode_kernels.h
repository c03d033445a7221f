// Decode path (tokens <= 16) for the packed binary low-rank linear on gfx950,
// for one linear or a batch of up to 8 linears per launch.
//
//   lm[t, r] = s_mid[r] * Σ_i sgn(V[r, i]) * x[t, i] * s_in[i]           (stage 1)
//   y[t, o]  = s_out[o] * Σ_r sgn(U[o, r]) * lm[t, r] + salient + bias    (stage 2)
//
// Both stages are the same contraction: rows R of a sign matrix [R, K] against
// an activation a[t, k]. They run on v_mfma_i32_16x16x64_i8 with exact integer
// arithmetic from the bits to the per-chunk fp32 partial.
//
// Weight layout ("tiles", built once by nq_prepare_tiles). A sign matrix
// [R, K] is cut into 16-row tiles and 512-column chunks (the last chunk may be
// 128, 256 or 384 columns wide: the matrix is padded to 128 columns only).
// Lane l = 16*g + n of a wave owns row n of a tile and, in chunk c, `dw` words
// (dw = 4 for a full chunk) stored contiguously:
//     word d, bit 8*b + m  =  sign bit of column 512*c + 128*d + 16*m + 4*g + b
// (bit set = -1; bits past K or past R are 0). The 64 lanes' words of one
// (tile, chunk) are 256*dw contiguous bytes: one 16-byte load per lane.
//
// Sign expansion is one v_and_b32 per four signs: word_d & (0x01010101 << m)
// is four int8 values in {0, 2^m} (m = 7 gives {0, -128}), the B operand dword
// d of MFMA m. The bits are used as b in {0, 1} with sgn = 1 - 2b, so
//     Σ_k sgn_k a_k = Σ_k a_k - 2 Σ_k b_k a_k .
// Activations (per chunk, per token) are rounded to x_q = rint(a * 2^E) with
// the chunk's own exact power of two E (max |x_q| <= 2^15), then the value fed
// to MFMA m is w = x_q * 2^(7-m) (w = -x_q for m = 7), written as three signed
// int8 digits w = d0 + 256*d1 + 65536*d2 in A rows 4*t + {0, 1, 2}. Every
// product is then 2^7 * b * x_q whatever m is, so the eight MFMAs of a chunk
// accumulate into one int32 accumulator and
//     Σ_k b_k x_q,k = (D0 + 256*D1 + 65536*D2) / 2^7    (D = digit rows of D)
//     chunk partial = 2^-E * (Σ_k x_q,k - (D0 + 256*D1 + 65536*D2) / 64).
// The only rounding before fp32 is x_q itself (|x_q| <= 2^15). Chunk partials
// are summed in chunk order, so the result is the same for every launch shape
// (waves per workgroup, tiles per workgroup, split or fused launch).
//
// Staging (per wave, per chunk, per block of up to 4 tokens): lane L loads
// the 8 activations of (m, g, dp) = (L >> 3, (L >> 1) & 3, L & 1), namely the
// runs 512c + 256dp + 16m + 4g + {0..3} and the same + 128, scales them, takes
// the wave max and sum, and writes its 8 digit bytes per digit row into the
// wave's LDS operand area A[m][row][g][16 bytes] with one 8-byte store; each
// lane then reads its eight A operands (one 16-byte LDS read per MFMA).
//
// Workgroup: NW waves; wave w takes chunks w, w + NW, ... of TW consecutive
// tiles, so one staged chunk feeds TW tiles. Per (chunk, tile) the wave stores
// its fp32 partial in LDS; after one barrier each output sums its partials in
// chunk order and the epilogue applies s_mid (stage 1, writes lm) or s_out +
// salient + bias (stage 2).
//
// Latency: every load of a pass (activations, then sign words; in the fused
// stage 2 the words before the wait) is issued from straight-line code before
// any of it is used: no branch surrounds a load (addresses are clamped, dead
// chunks reload a valid chunk and skip only the arithmetic, the wave index is
// made uniform with readfirstlane), so the compiler never waits on one load to
// issue the next. The activation dtype pair is a template parameter
// (bf16 / f16 / f32 x with fp16 scales as vector loads); any other
// combination, and unaligned buffers, take a generic variant whose element
// loads are two unconditional 16-bit loads decoded by a uniform select.
//
// Launch structure (nq_linear_desc.decode_launch):
//   split (default): kernel 1 runs the stage-1 tiles of every linear in the
//     batch and stores lm; kernel 2 runs the stage-2 tiles. The kernel
//     boundary is the grid-wide barrier.
//   fused: one kernel whose first workgroups are the stage-1 tiles and the
//     rest the stage-2 tiles. Stage-1 workgroups store lm at agent scope and
//     then signal; stage-2 workgroups issue their U loads, wait for their
//     linear's signal (bounded spin) and only then load lm. Workgroups are
//     dispatched in index order, so every stage-1 workgroup is resident or
//     finished before a stage-2 workgroup can take its slot, and stage-1
//     workgroups never wait.
// Measured on MI355X, a graph-launched kernel boundary (about 1.5 us) is
// cheaper than any grid-wide handoff inside a kernel (3 us or more across the
// eight XCDs), hence split is the default.
#pragma once

#include "nq_decode.h"

namespace nqdec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

constexpr int kTileRows = 16;
constexpr int kBlockCols = 128;   // one word per lane
constexpr int kChunkBlocks = 4;   // words per lane in a full chunk
constexpr int kChunkCols = kBlockCols * kChunkBlocks;
constexpr int kMaxTokens = 16;
constexpr int kMaxBatch = 8;
constexpr uint32_t kTilesMagic = 0x4e515433u;  // "NQT3"
constexpr uint32_t kSpinLimit = 1u << 22;

// Sync header at the start of each linear's tiles buffer (used by the fused
// launch only). Every word lives on its own 256-byte line. All counters only
// ever increase, so nothing is reset between launches (graph replays included):
//   Counters are 64-bit (first two words of their line); flags are 32-bit and
//   compared wrap-safely.
//   ready slots: each stage-1 tile b adds 1 to slot b % kReadySlots; with
//     c = that slot's participant count, the value it saw, v, gives the launch
//     index k = v / c, and v % c == c - 1 marks the slot complete.
//   ready root: each slot completer adds 1; the root completer of launch k
//     (old value == (k + 1) * used_slots - 1) writes k + 1 into every ready
//     flag.
//   arrive slots: each output tile i of a stage-2 workgroup adds 1 to slot
//     i % kArriveSlots at the workgroup's start, which yields the launch index
//     k the same way; the workgroup then waits until its ready flag (one of
//     the kReplicas copies) reaches k + 1 (wrap-safe compare).
// Counting per tile (not per workgroup) keeps the launch index consistent when
// the tiles-per-workgroup choice changes between launches of one layer.
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

// Geometry of one sign matrix [rows, cols] in the tile layout.
struct MatGeo {
    int64_t nt;  // 16-row tiles
    int64_t nb;  // 128-column blocks (words per lane per tile)
    int64_t nc;  // 512-column chunks
};

__host__ __device__ inline MatGeo mat_geo(int64_t rows, int64_t cols) {
    MatGeo g;
    g.nt = (rows + kTileRows - 1) / kTileRows;
    g.nb = (cols + kBlockCols - 1) / kBlockCols;
    g.nc = (g.nb + kChunkBlocks - 1) / kChunkBlocks;
    return g;
}

__host__ __device__ inline int64_t mat_words(const MatGeo& g) { return g.nt * g.nb * 64; }

// Words per lane in chunk c.
__host__ __device__ inline int chunk_words(const MatGeo& g, int64_t c) {
    const int64_t r = g.nb - kChunkBlocks * c;
    return static_cast<int>(r < kChunkBlocks ? r : kChunkBlocks);
}

// ---------------------------------------------------------------------------
// Decode kernels.
// ---------------------------------------------------------------------------

struct LinArgs {
    int64_t in, rank, out;
    MatGeo g1, g2;           // V [rank, in], U [out, rank]
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
    float* lm;               // [tokens][lm_ld]; entries past `rank` are never read
    int64_t lm_ld;           // 128 * g2.nb
};

struct Batch {
    int count;
    int tw1, tw2;                    // tiles per workgroup of each stage
    int64_t first1[kMaxBatch + 1];   // stage-1 workgroup prefix per linear
    int64_t first2[kMaxBatch + 1];   // stage-2 workgroup prefix (after all stage-1)
    LinArgs p[kMaxBatch];
};

// Activation kinds (template parameter AK): how a stage reads a[t, k].
enum : int {
    kActBf16 = 0,     // stage 1: bf16 x, fp16 s_in, vector loads
    kActF16 = 1,      // stage 1: fp16 x, fp16 s_in, vector loads
    kActF32 = 2,      // stage 1: fp32 x, fp16 s_in, vector loads
    kActGeneric = 3,  // stage 1: any float x and s_in, element loads
    kActLm = 4,       // stage 2: fp32 lm, no column scale, vector loads
};

// 2^e for an integer e in the fp32 normal range.
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

// Exponent E with bound * 2^E < 2^15 (so |rint(a * 2^E)| <= 2^15 for |a| <=
// bound); 0 when the bound is zero or not finite-positive.
__device__ __forceinline__ int chunk_exponent(float bound) {
    if (!(bound > 0.0f)) return 0;
    int e = static_cast<int>((__float_as_uint(bound) >> 23) & 0xff) - 127;
    e = 14 - (e < -126 ? -126 : e);
    return e > 120 ? 120 : (e < -113 ? -113 : e);
}

template <int CTRL>
__device__ __forceinline__ float dpp_maxf(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false);
    return fmaxf(x, __int_as_float(y));
}

template <int CTRL>
__device__ __forceinline__ int dpp_addi(int x) {
    return x + __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}

// Max / sum over the whole wave (every lane gets the result, as a uniform value).
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_maxf<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_maxf<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_maxf<0x141>(v);  // row_half_mirror
    v = dpp_maxf<0x140>(v);  // row_mirror
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ int wave_sum(int v) {
    v = dpp_addi<0xB1>(v);
    v = dpp_addi<0x4E>(v);
    v = dpp_addi<0x141>(v);
    v = dpp_addi<0x140>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
           __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

// --- branch-free element loads of a runtime float dtype ------------------------

// Raw bits of element i of an F32 / F16 / BF16 buffer: two unconditional
// 16-bit loads (the two halves of an fp32, or the same half twice).
struct RawElem {
    uint32_t lo, hi;
};

__device__ __forceinline__ RawElem load_elem(const void* __restrict__ p, int dtype, int64_t i) {
    const uint16_t* h = static_cast<const uint16_t*>(p);
    const bool wide = dtype == NQ_DTYPE_F32;
    RawElem r;
    r.lo = h[wide ? 2 * i : i];
    r.hi = h[wide ? 2 * i + 1 : i];
    return r;
}

__device__ __forceinline__ float elem_value(const RawElem& r, int dtype) {
    union {
        uint16_t u;
        _Float16 h;
    } c;
    c.u = static_cast<uint16_t>(r.lo);
    const float f32 = __uint_as_float((r.hi << 16) | (r.lo & 0xffffu));
    const float bf16 = __uint_as_float(r.lo << 16);
    const float f16 = static_cast<float>(c.h);
    return dtype == NQ_DTYPE_F32 ? f32 : (dtype == NQ_DTYPE_BF16 ? bf16 : f16);
}

// --- activation runs: 4 consecutive columns -------------------------------------

// Raw registers of one run for kind AK: fp16/bf16 pairs in two dwords, fp32 in
// four, generic as four raw elements.
template <int AK>
struct Run {
    static constexpr int kDwords = (AK == kActBf16 || AK == kActF16) ? 2 : 4;
    uint32_t u[AK == kActGeneric ? 1 : kDwords];
    RawElem e[AK == kActGeneric ? 4 : 1];
};

// Columns [k, k + 4) of row `row` of a buffer with leading dimension ld,
// loaded from an address clamped to rows_valid rows and `clamp` columns
// (vector kinds: k % 4 == 0, clamp % 4 == 0, clamp >= 4, ld % 4 == 0 and an
// aligned base, checked by the host; generic: each element clamped to
// cols_valid). Values past the valid range are zeroed when staged.
template <int AK, int DT>
__device__ __forceinline__ Run<AK> load_run(const void* __restrict__ p, int rt_dtype, int64_t row,
                                            int64_t rows_valid, int64_t ld, int64_t k, int64_t cols_valid,
                                            int64_t clamp) {
    Run<AK> r;
    const int64_t rr = row < rows_valid ? row : rows_valid - 1;
    if constexpr (AK == kActGeneric) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t kk = k + i < cols_valid ? k + i : cols_valid - 1;
            r.e[i] = load_elem(p, rt_dtype, rr * ld + kk);
        }
    } else {
        const int64_t kk = k < clamp ? k : clamp - 4;
        if constexpr (DT == NQ_DTYPE_F32) {
            const v4u q = *reinterpret_cast<const v4u*>(static_cast<const float*>(p) + rr * ld + kk);
#pragma unroll
            for (int i = 0; i < 4; ++i) r.u[i] = q[i];
        } else {
            const v2u q = *reinterpret_cast<const v2u*>(static_cast<const uint16_t*>(p) + rr * ld + kk);
            r.u[0] = q.x;
            r.u[1] = q.y;
        }
    }
    return r;
}

// The four values of a run stored as dtype DT (generic: runtime rt_dtype).
template <int AK, int DT>
__device__ __forceinline__ void run_values(const Run<AK>& r, int rt_dtype, float (&v)[4]) {
    if constexpr (AK == kActGeneric) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = elem_value(r.e[i], rt_dtype);
    } else if constexpr (DT == NQ_DTYPE_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(r.u[i]);
    } else if constexpr (DT == NQ_DTYPE_BF16) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            v[2 * i] = __uint_as_float(r.u[i] << 16);
            v[2 * i + 1] = __uint_as_float(r.u[i] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            union {
                uint32_t u;
                _Float16 h[2];
            } c;
            c.u = r.u[i];
            v[2 * i] = static_cast<float>(c.h[0]);
            v[2 * i + 1] = static_cast<float>(c.h[1]);
        }
    }
}

// Storage dtype of the activation and of the column scale for each kind.
template <int AK>
constexpr int act_dtype() {
    return AK == kActBf16 ? NQ_DTYPE_BF16 : (AK == kActF16 ? NQ_DTYPE_F16 : NQ_DTYPE_F32);
}
constexpr int kScaleDtype = NQ_DTYPE_F16;  // column scale of the vector kinds

// What one stage reads and writes.
struct StageView {
    int64_t rows, cols;
    MatGeo g;
    const uint32_t* tiles;
    const void* act;      // [tokens][act_ld]
    int act_dtype;        // runtime dtype (generic kind)
    int64_t act_ld;
    int64_t act_clamp;    // vector loads stay below this column
    const void* colscale; // s_in (stage 1) or null
    int colscale_dtype;
    const void* rowscale; // s_mid / s_out
};

template <int STAGE>
__device__ __forceinline__ StageView stage_view(const LinArgs& a) {
    StageView v;
    if (STAGE == 1) {
        v.rows = a.rank;
        v.cols = a.in;
        v.g = a.g1;
        v.tiles = a.v_tiles;
        v.act = a.x;
        v.act_dtype = a.x_dtype;
        v.act_ld = a.in;
        v.act_clamp = a.in;
        v.colscale = a.s_in;
        v.colscale_dtype = a.scale_dtype;
        v.rowscale = a.s_mid;
    } else {
        v.rows = a.out;
        v.cols = a.rank;
        v.g = a.g2;
        v.tiles = a.u_tiles;
        v.act = a.lm;
        v.act_dtype = NQ_DTYPE_F32;
        v.act_ld = a.lm_ld;
        v.act_clamp = a.lm_ld;  // the last chunk's runs may reach past lm_ld: clamped, then masked
        v.colscale = nullptr;
        v.colscale_dtype = 0;
        v.rowscale = a.s_out;
    }
    return v;
}

// Rows of the LDS operand area per token block: 4 digit rows per token.
template <int TPB>
struct Ops {
    static constexpr int kRows = 4 * TPB;
    static constexpr int kWaveBytes = 8 * kRows * 4 * 16;  // A[m][row][g][16 B]
};

// Registers one wave holds for one chunk: activation runs of every token and
// the column-scale runs, plus the sign words of its TW tiles.
template <int AK, int TOK, int TW>
struct ChunkRegs {
    Run<AK> x[TOK][2];
    Run<AK> s[AK == kActLm ? 1 : 2];
    v4u w[TW];
};

// Staging lane roles: lane L stages (m, g, dp) = (L >> 3, (L >> 1) & 3, L & 1),
// i.e. columns k0 + {0..3} and k0 + 128 + {0..3} of the chunk.
__device__ __forceinline__ int64_t stage_col0(int64_t c, int lane) {
    return kChunkCols * c + 2 * kBlockCols * (lane & 1) + 16 * (lane >> 3) + 4 * ((lane >> 1) & 3);
}

// Issue the activation loads of chunk c (tokens [0, TOK)).
template <int AK, int TOK, int TW>
__device__ __forceinline__ void load_chunk_acts(ChunkRegs<AK, TOK, TW>& r, const StageView& v, int tokens,
                                                int64_t c, int lane) {
    constexpr int DT = act_dtype<AK>();
    const int64_t k0 = stage_col0(c, lane);
#pragma unroll
    for (int t = 0; t < TOK; ++t)
#pragma unroll
        for (int run = 0; run < 2; ++run)
            r.x[t][run] = load_run<AK, DT>(v.act, v.act_dtype, t, tokens, v.act_ld, k0 + kBlockCols * run, v.cols,
                                           v.act_clamp);
    if constexpr (AK != kActLm) {
#pragma unroll
        for (int run = 0; run < 2; ++run)
            r.s[run] = load_run<AK, kScaleDtype>(v.colscale, v.colscale_dtype, 0, 1, 0, k0 + kBlockCols * run,
                                                 v.cols, v.act_clamp);
    }
}

// Issue the sign-word loads of chunk c for tiles t0 .. t0 + TW - 1 (tiles past
// the last one load the last tile; their results are never stored). A partial
// last chunk (dw < 4 words per lane) loads its dw words and repeats the last
// one; tile_partial masks the repeats out.
template <int AK, int TOK, int TW>
__device__ __forceinline__ void load_chunk_words(ChunkRegs<AK, TOK, TW>& r, const StageView& v, int64_t t0,
                                                 int64_t c, int lane) {
    const int dw = chunk_words(v.g, c);
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
        const int64_t tile = t0 + tt < v.g.nt ? t0 + tt : v.g.nt - 1;
        const uint32_t* base = v.tiles + tile * v.g.nb * 64 + c * 256;
        if (dw == kChunkBlocks) {  // uniform
            r.w[tt] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(base) + lane);
        } else {
            v4u w;
#pragma unroll
            for (int d = 0; d < kChunkBlocks; ++d) {
                const int dd = d < dw ? d : dw - 1;
                w[d] = __builtin_nontemporal_load(base + lane * dw + dd);
            }
            r.w[tt] = w;
        }
    }
}

// Order this wave's LDS writes before its own reads (waves never share areas).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int sext8(int v) { return (v << 24) >> 24; }

// Stage tokens [t_base, t_base + TPB) of chunk c into this wave's operand area
// and return each token's exponent E and integer sum S (uniform values).
template <int AK, int TOK, int TW, int TPB>
__device__ __forceinline__ void stage_block(const ChunkRegs<AK, TOK, TW>& r, const StageView& v, int tokens,
                                            int64_t c, int t_base, char* __restrict__ ops, int lane, int (&expo)[TPB],
                                            int (&qsum)[TPB]) {
    constexpr int DT = act_dtype<AK>();
    const int m = lane >> 3, grp = (lane >> 1) & 3, dp = lane & 1;
    const int64_t k0 = stage_col0(c, lane);
    float sc[2][4];
    if constexpr (AK != kActLm) {
        run_values<AK, kScaleDtype>(r.s[0], v.colscale_dtype, sc[0]);
        run_values<AK, kScaleDtype>(r.s[1], v.colscale_dtype, sc[1]);
    }
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
        const int t = t_base + u;
        float a[2][4];
        float mx = 0.0f;
#pragma unroll
        for (int run = 0; run < 2; ++run) {
            run_values<AK, DT>(r.x[t][run], v.act_dtype, a[run]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float val = a[run][i];
                if constexpr (AK != kActLm) val *= sc[run][i];
                const bool ok = t < tokens && k0 + kBlockCols * run + i < v.cols;
                val = ok ? val : 0.0f;
                a[run][i] = val;
                mx = fmaxf(mx, fabsf(val));
            }
        }
        const int e = chunk_exponent(wave_max(mx));
        const float scale = exp2i(e);
        int q[2][4];
        int s = 0;
#pragma unroll
        for (int run = 0; run < 2; ++run)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q[run][i] = static_cast<int>(__builtin_rintf(a[run][i] * scale));
                s += q[run][i];
            }
        expo[u] = e;
        qsum[u] = wave_sum(s);
        // Digits of w = x_q * 2^(7 - m) (m < 7) or -x_q (m = 7); byte 4*run + i
        // of each digit row is column k0 + 128*run + i.
        uint32_t dig[3][2];
#pragma unroll
        for (int run = 0; run < 2; ++run) {
            uint32_t b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int w = m < 7 ? (q[run][i] << (7 - m)) : -q[run][i];
                const int d0 = sext8(w);
                const int w1 = (w - d0) >> 8;
                const int d1 = sext8(w1);
                const int d2 = (w1 - d1) >> 8;
                b0 |= (static_cast<uint32_t>(d0) & 0xffu) << (8 * i);
                b1 |= (static_cast<uint32_t>(d1) & 0xffu) << (8 * i);
                b2 |= (static_cast<uint32_t>(d2) & 0xffu) << (8 * i);
            }
            dig[0][run] = b0;
            dig[1][run] = b1;
            dig[2][run] = b2;
        }
#pragma unroll
        for (int digit = 0; digit < 3; ++digit) {
            const int row = 4 * u + digit;
            *reinterpret_cast<v2u*>(ops + ((m * Ops<TPB>::kRows + row) * 4 + grp) * 16 + 8 * dp) =
                v2u{dig[digit][0], dig[digit][1]};
        }
    }
}

// The eight MFMAs of one (chunk, tile, token block) and the exact conversion to
// the chunk's fp32 partial; words d >= dw (a partial chunk) count as zero.
// Lane 16*t' + n returns token t' (of the block), row n.
template <int TPB>
__device__ __forceinline__ float tile_partial(const v4i (&A)[8], const v4u& w, int dw, int lane,
                                              const int (&expo)[TPB], const int (&qsum)[TPB]) {
    v4i acc = v4i{0, 0, 0, 0};
    const uint32_t keep1 = dw > 1 ? ~0u : 0u, keep2 = dw > 2 ? ~0u : 0u, keep3 = dw > 3 ? ~0u : 0u;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const uint32_t mask = 0x01010101u << m;
        const v4i b = v4i{static_cast<int>(w[0] & mask), static_cast<int>(w[1] & (mask & keep1)),
                          static_cast<int>(w[2] & (mask & keep2)), static_cast<int>(w[3] & (mask & keep3))};
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], b, acc, 0, 0, 0);
    }
    int e = expo[0];
    int s = qsum[0];
    if (TPB > 1) {
        const int tl = lane >> 4;
#pragma unroll
        for (int u = 1; u < TPB; ++u) {
            e = tl == u ? expo[u] : e;
            s = tl == u ? qsum[u] : s;
        }
    }
    const float tsum = static_cast<float>(acc[0]) + 256.0f * static_cast<float>(acc[1]) +
                       65536.0f * static_cast<float>(acc[2]);
    return (static_cast<float>(s) - tsum * 0.015625f) * exp2i(-e);
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

// Fused launch, stage 1: thread 0 signals each of the workgroup's tiles once
// the workgroup's lm stores are complete (the caller waits and barriers first).
__device__ __forceinline__ void signal_ready(const LinArgs& a, int64_t t0, int tw) {
    if (threadIdx.x != 0) return;
    const int64_t n1 = a.g1.nt;
    for (int tt = 0; tt < tw; ++tt) {
        const int64_t tile = t0 + tt;
        if (tile >= n1) break;
        const int slot = static_cast<int>(tile % kReadySlots);
        const uint64_t c = slot_count(slot, kReadySlots, n1);
        const uint64_t v = hdr_add(a.header, line_word(kReadySlot0 + slot));
        if (v % c == c - 1) {
            const uint64_t used = static_cast<uint64_t>(n1 < kReadySlots ? n1 : kReadySlots);
            const uint64_t k = v / c;
            const uint64_t w = hdr_add(a.header, line_word(kReadyRoot));
            if (w + 1 == (k + 1) * used) {
                const uint32_t flag = static_cast<uint32_t>(k + 1);
                for (int i = 0; i < kReplicas; ++i) hdr_store(a.header, line_word(kReplica0 + i), flag);
            }
        }
    }
}

// Fused launch, stage 2: register the workgroup's tiles, then wait until every
// stage-1 tile of this launch has signalled.
__device__ __forceinline__ void wait_ready(const LinArgs& a, int64_t t0, int tw, int64_t wg) {
    if (threadIdx.x == 0) {
        const int64_t n2 = a.g2.nt;
        uint32_t target = 0;
        for (int tt = 0; tt < tw; ++tt) {
            const int64_t tile = t0 + tt;
            if (tile >= n2) break;
            const int slot = static_cast<int>(tile % kArriveSlots);
            const uint64_t v = hdr_add(a.header, line_word(kArriveSlot0 + slot));
            if (tt == 0) target = static_cast<uint32_t>(v / slot_count(slot, kArriveSlots, n2) + 1);
        }
        const uint32_t* flag = a.header + line_word(kReplica0 + static_cast<int>(wg % kReplicas));
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

// Chunks of one pass: chunk c_j = base + wave + j * nw; a dead chunk (past nc)
// loads chunk nc - 1 and skips its arithmetic.
template <int KC>
struct PassChunks {
    int64_t c[KC];
    bool live[KC];
};

template <int KC>
__device__ __forceinline__ PassChunks<KC> pass_chunks(int64_t base, int wave, int nw, int64_t nc) {
    PassChunks<KC> p;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        const int64_t c = base + wave + static_cast<int64_t>(j) * nw;
        p.live[j] = c < nc;
        p.c[j] = c < nc ? c : nc - 1;
    }
    return p;
}

// One workgroup of one stage: tiles [t0, t0 + TW) of linear `a`. TPB tokens per
// block and TB blocks cover the launch's tokens; KC chunks per wave per pass.
template <int STAGE, int AK, int TPB, int TB, int TW, int KC, bool FUSED>
__device__ __forceinline__ void stage_wg(const LinArgs& a, int64_t wg, char* __restrict__ lds) {
    constexpr int TOK = TPB * TB;
    const StageView v = stage_view<STAGE>(a);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int nw = static_cast<int>(blockDim.x >> 6);
    const int tokens = a.tokens;
    const int64_t t0 = wg * TW;
    const int64_t nc = v.g.nc;
    char* const ops = lds + wave * Ops<TPB>::kWaveBytes;
    float* const red = reinterpret_cast<float*>(lds + nw * Ops<TPB>::kWaveBytes);

    // Epilogue operands of this thread's first output (see the epilogue loop),
    // issued first so their latency hides under the main loads.
    const int outs = TW * tokens * kTileRows;
    const int first = threadIdx.x;
    const int64_t first_tile = t0 + (first < outs ? first : 0) / (tokens * kTileRows);
    const int64_t fr = first_tile * kTileRows + (first & 15);
    const int64_t first_row = fr < v.rows ? fr : v.rows - 1;
    const RawElem rs0 = load_elem(v.rowscale, a.scale_dtype, first_row);
    RawElem bias0{0u, 0u};
    if (STAGE == 2 && a.bias) bias0 = load_elem(a.bias, a.bias_dtype, first_row);

    for (int64_t base = 0; base < nc; base += static_cast<int64_t>(nw) * KC) {
        const PassChunks<KC> pc = pass_chunks<KC>(base, wave, nw, nc);
        ChunkRegs<AK, TOK, TW> r[KC];
        if (FUSED && STAGE == 2) {
            // The U words do not depend on stage 1: issue them, wait for the
            // signal (first pass only), then load lm.
#pragma unroll
            for (int j = 0; j < KC; ++j) load_chunk_words(r[j], v, t0, pc.c[j], lane);
            if (base == 0) wait_ready(a, t0, TW, wg);
#pragma unroll
            for (int j = 0; j < KC; ++j) load_chunk_acts(r[j], v, tokens, pc.c[j], lane);
        } else {
            // Activations first, sign words second: the staging math waits only
            // for the activations, the MFMAs for the words.
#pragma unroll
            for (int j = 0; j < KC; ++j) load_chunk_acts(r[j], v, tokens, pc.c[j], lane);
#pragma unroll
            for (int j = 0; j < KC; ++j) load_chunk_words(r[j], v, t0, pc.c[j], lane);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the pass is issued before any use
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            if (!pc.live[j]) continue;  // uniform
            const int64_t c = pc.c[j];
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                if (tb * TPB >= tokens) break;
                int expo[TPB], qsum[TPB];
                stage_block<AK, TOK, TW, TPB>(r[j], v, tokens, c, tb * TPB, ops, lane, expo, qsum);
                wave_lds_sync();
                v4i A[8];
                const int row = TPB == 1 ? (lane & 3) : (lane & 15);
#pragma unroll
                for (int m = 0; m < 8; ++m)
                    A[m] = *reinterpret_cast<const v4i*>(ops + ((m * Ops<TPB>::kRows + row) * 4 + (lane >> 4)) * 16);
                const int dw = chunk_words(v.g, c);
#pragma unroll
                for (int tt = 0; tt < TW; ++tt)
                    red[((c * TW + tt) * TB + tb) * 64 + lane] = tile_partial<TPB>(A, r[j].w[tt], dw, lane, expo, qsum);
                wave_lds_sync();  // the next block rewrites this wave's operand area
            }
        }
    }
    __syncthreads();

    // Epilogue: output idx = (tt, t, n); partials summed in chunk order.
    for (int idx = threadIdx.x; idx < outs; idx += blockDim.x) {
        const int tt = idx / (tokens * kTileRows);
        const int t = (idx / kTileRows) % tokens;
        const int n = idx & 15;
        const int64_t row = (t0 + tt) * kTileRows + n;
        if (t0 + tt >= v.g.nt || row >= v.rows) continue;
        const int tb = TPB == 1 ? 0 : t / TPB;
        const int rl = TPB == 1 ? n : 16 * (t % TPB) + n;
        float sum = 0.0f;
        for (int64_t c = 0; c < nc; ++c) sum += red[((c * TW + tt) * TB + tb) * 64 + rl];
        const float rs = elem_value(idx == first ? rs0 : load_elem(v.rowscale, a.scale_dtype, row), a.scale_dtype);
        if (STAGE == 1) {
            const float val = sum * rs;
            float* dst = a.lm + t * a.lm_ld + row;
            if (FUSED) store_agent(dst, val);
            else *dst = val;
        } else {
            float val = sum * rs;
            for (int64_t k = 0; k < a.salient_count; ++k) {
                float wv = nq::load_f32(a.salient_values, a.salient_dtype, row * a.salient_count + k);
                if (a.salient_scales) wv *= nq::load_f32(a.salient_scales, a.scale_dtype, k);
                val += wv * nq::load_f32(a.x, a.x_dtype, t * a.in + a.salient_indices[k]);
            }
            if (a.bias) val += elem_value(idx == first ? bias0 : load_elem(a.bias, a.bias_dtype, row), a.bias_dtype);
            nq::store_f32_as(a.y, a.y_dtype, t * a.out + row, val);
        }
    }
    if (FUSED && STAGE == 1) {
        // lm went out at agent scope; the wait makes it complete before the signal.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        signal_ready(a, t0, TW);
    }
}

// Linear of block b: the number of prefix entries first[1..count-1] <= b
// (independent scalar loads, no dependent chain).
__device__ __forceinline__ int member_of(const int64_t (&first)[kMaxBatch + 1], int count, int64_t b) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatch; ++i) p += (i < count && b >= first[i]) ? 1 : 0;
    return p;
}

// Split launch: one kernel per stage; block b of the stage-2 kernel is block
// b + first1[count] of the combined numbering. THREADS is the launch bound:
// 1024 for one token per block, 768 when a wave takes two chunks per pass
// (168 VGPRs), 512 for four tokens per block (256 VGPRs).
template <int STAGE, int AK, int TPB, int TB, int TW, int KC, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_stage(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    if (STAGE == 1) {
        const int64_t b = blockIdx.x;
        const int p = member_of(batch.first1, batch.count, b);
        stage_wg<1, AK, TPB, TB, TW, KC, false>(batch.p[p], b - batch.first1[p], lds);
    } else {
        const int64_t b = blockIdx.x + batch.first1[batch.count];
        const int p = member_of(batch.first2, batch.count, b);
        stage_wg<2, AK, TPB, TB, TW, KC, false>(batch.p[p], b - batch.first2[p], lds);
    }
}

// Fused launch (one tile per workgroup, generic stage-1 loads): stage-1 blocks
// first, then stage-2.
template <int TPB, int TB, int KC1, int KC2, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_fused(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int64_t b = blockIdx.x;
    if (b < batch.first1[batch.count]) {
        const int p = member_of(batch.first1, batch.count, b);
        stage_wg<1, kActGeneric, TPB, TB, 1, KC1, true>(batch.p[p], b - batch.first1[p], lds);
    } else {
        const int p = member_of(batch.first2, batch.count, b);
        stage_wg<2, kActLm, TPB, TB, 1, KC2, true>(batch.p[p], b - batch.first2[p], lds);
    }
}

// Launch bound of a configuration (see k_decode_stage).
constexpr int threads_for(int tpb, int kc) { return tpb == 1 ? (kc == 1 ? 1024 : 768) : 512; }

// Shape of one decode launch, chosen on the host (nq_decode.hip).
struct LaunchShape {
    int ak;          // activation kind of stage 1
    int tpb, tb;     // tokens per block, blocks
    int tw;          // tiles per workgroup
    int nw;          // waves per workgroup
    int kc, kc2;     // chunks per wave per pass (stage kernels: kc; fused: stage 1 kc, stage 2 kc2)
    size_t lds;      // dynamic LDS bytes
    unsigned grid;   // workgroups
};

// Launchers, one translation unit each (they instantiate disjoint kernels).
int enqueue_stage1_bf16(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_f16(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_f32(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_generic(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage2(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_fused(const Batch& batch, const LaunchShape& s, hipStream_t stream);

}  // namespace nqdec

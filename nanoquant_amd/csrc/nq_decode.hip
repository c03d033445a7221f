// Fused single-launch decode path (tokens <= 16) for the packed binary
// low-rank linear on gfx950.
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
// Grid: one launch. Workgroups [0, n1) are stage-1 tiles (16 ranks each, the
// four waves split the columns); workgroups [n1, n1 + n2) are stage-2 tiles
// (16 output rows each). Stage-1 workgroups write lm (fp32) and a per-token
// |lm| maximum to the workspace, then release a counter (agent scope).
// Stage-2 workgroups first issue the loads of their U tile, then acquire the
// counter (bounded spin), so the U stream overlaps stage 1. Workgroups are
// dispatched in index order, so every stage-1 workgroup is resident or done
// before any stage-2 workgroup can occupy its slot; stage-1 workgroups never
// wait. The last stage-2 workgroup resets the counters for the next launch.
//
// Activations enter the fp16 MFMA scaled by an exact per-token power of two
// (from the maximum |x| exponent times max|s_in|, and from the stage-1 |lm|
// maximum), so the fp16 range cannot overflow; products are accumulated in
// fp32.
#include "nq_decode.h"

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr int kWaves = 4;
constexpr int kTileRows = 16;
constexpr int kSuperCols = 128;
constexpr int kMaxTokens = 16;
constexpr int kHeaderWords = 64;  // 256-byte sync header at the start of the tiles buffer
constexpr uint32_t kTilesMagic = 0x4e515431u;  // "NQT1"
constexpr uint32_t kSpinLimit = 1u << 20;

// Sync header words.
enum : int { kHdrCounter = 0, kHdrDone = 1, kHdrError = 2, kHdrMagic = 3, kHdrPreMax = 4 };

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
    // One block: header words plus max|s_in| (used to bound x * s_in).
    __shared__ float red[kBlock];
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < in; i += kBlock) m = fmaxf(m, fabsf(nq::load_f32(s_in, scale_dtype, i)));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = kBlock / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x < kHeaderWords) header[threadIdx.x] = 0;
    __syncthreads();
    if (threadIdx.x == 0) {
        header[kHdrMagic] = kTilesMagic;
        header[kHdrPreMax] = __float_as_uint(red[0]);
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
};

// 2^e for an integer e in the fp32 normal range.
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

// Exponent e with 2^e <= v < 2^(e+1) for finite v > 0 (normals only; tiny values clamp).
__device__ __forceinline__ int exponent_of(float v) {
    const int e = static_cast<int>((__float_as_uint(v) >> 23) & 0xff) - 127;
    return e < -126 ? -126 : e;
}

// Scale that maps values bounded by `bound` below 2^14 (fp16-safe with headroom
// for the sum of 32 terms the MFMA never rounds to fp16 anyway).
__device__ __forceinline__ float range_scale(float bound) {
    if (!(bound > 0.0f)) return 1.0f;
    int e = 13 - exponent_of(bound);
    e = e > 100 ? 100 : (e < -100 ? -100 : e);
    return exp2i(e);
}

template <int MT>
struct alignas(16) Lds {
    // Activation staging: MT rows of fp16, row stride padded by 8 halfs so the
    // 16 token rows of a ds_read_b128 land in different banks.
    static constexpr int kStageCols = MT == 1 ? 12288 : (MT <= 4 ? 3072 : 2048);
    static constexpr int kStride = kStageCols + 8;
    _Float16 act[MT * kStride];
    float red[kWaves][kMaxTokens][kTileRows];
    float tokscale[kMaxTokens];
    uint32_t flag;
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

// Stage activation columns [c0, c0 + ncols) into LDS: act[t][c - c0] = fp16(a(t, c) * scale[t]).
template <int MT, typename Fn>
__device__ __forceinline__ void stage_columns(Lds<MT>& lds, int64_t c0, int ncols, int64_t col_limit,
                                              int tokens, Fn value) {
    for (int e = threadIdx.x; e < MT * ncols; e += kBlock) {
        const int t = e / ncols;
        const int c = e - t * ncols;
        const int64_t col = c0 + c;
        float v = 0.0f;
        if (t < tokens && col < col_limit) v = value(t, col) * lds.tokscale[t];
        lds.act[t * Lds<MT>::kStride + c] = static_cast<_Float16>(v);
    }
}

// One wave's share of a 16-row tile: superchunks sc = w, w + 4, ... of the
// current stage window. Returns the partial D (token rows x 16 tile rows).
template <int MT, int SCMAX>
__device__ __forceinline__ v4f tile_mfma(const Lds<MT>& lds, const uint32_t (&words)[SCMAX],
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
                if (t < MT) a = *reinterpret_cast<const v8h*>(&lds.act[t * Lds<MT>::kStride + base + 32 * m]);
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
template <int MT>
__device__ __forceinline__ float reduce_waves(Lds<MT>& lds, v4f acc) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 4; ++i) lds.red[wave][4 * (lane >> 4) + i][lane & 15] = acc[i];
    __syncthreads();
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    return ((lds.red[0][t][n] + lds.red[1][t][n]) + lds.red[2][t][n]) + lds.red[3][t][n];
}

template <int MT, int SCMAX>
__device__ void stage1_tile(const FusedArgs& a, Lds<MT>& lds, int64_t rt) {
    const uint32_t* tile = a.v_tiles + rt * a.nsc1 * 64;
    constexpr int kWindowSc = 4 * SCMAX;
    uint32_t words[SCMAX];
    load_words<SCMAX>(words, tile, 0, a.nsc1);

    // Per-token range scale: bound |x * s_in| by max|x| * max|s_in|.
    if (threadIdx.x < kMaxTokens) lds.tokscale[threadIdx.x] = 0.0f;
    __syncthreads();
    {
        const int t = threadIdx.x % MT;     // kBlock / MT threads cooperate per token
        const int part = threadIdx.x / MT;
        float m = 0.0f;
        if (t < a.tokens) {
            for (int64_t i = part; i < a.in; i += kBlock / MT) {
                m = fmaxf(m, fabsf(nq::load_f32(a.x, a.x_dtype, t * a.in + i)));
            }
        }
        // Non-negative floats order like their bit patterns.
        if (m > 0.0f) atomicMax(reinterpret_cast<unsigned int*>(&lds.tokscale[t]), __float_as_uint(m));
    }
    __syncthreads();
    const float premax = __uint_as_float(a.header[kHdrPreMax]);
    if (threadIdx.x < kMaxTokens) lds.tokscale[threadIdx.x] = range_scale(lds.tokscale[threadIdx.x] * premax);
    __syncthreads();

    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t w0 = 0; w0 < a.nsc1; w0 += kWindowSc) {
        if (w0 > 0) load_words<SCMAX>(words, tile, w0, a.nsc1);
        const int64_t c0 = w0 * kSuperCols;
        const int64_t cend = (w0 + kWindowSc < a.nsc1 ? w0 + kWindowSc : a.nsc1) * kSuperCols;
        stage_columns<MT>(lds, c0, static_cast<int>(cend - c0), a.in, a.tokens,
                          [&](int t, int64_t col) {
                              return nq::load_f32(a.x, a.x_dtype, t * a.in + col) *
                                     nq::load_f32(a.s_in, a.scale_dtype, col);
                          });
        __syncthreads();
        acc = tile_mfma<MT, SCMAX>(lds, words, w0, a.nsc1, w0, acc);
        __syncthreads();
    }

    const float sum = reduce_waves<MT>(lds, acc);
    const int t = threadIdx.x >> 4;
    const int n = threadIdx.x & 15;
    const int64_t r = rt * kTileRows + n;
    float lmv = 0.0f;
    if (t < a.tokens && r < a.rank) {
        lmv = sum / lds.tokscale[t] * nq::load_f32(a.s_mid, a.scale_dtype, r);
        a.lm[t * (a.n1 * kTileRows) + r] = lmv;
    }
    // Per-token max over the 16 tile rows (lanes n = 0..15 of this group).
    float am = fabsf(lmv);
    for (int off = 8; off >= 1; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 16));
    if (n == 0) a.wgmax[rt * kMaxTokens + t] = am;

    // Publish: every wave makes its stores visible at agent scope, then one
    // release increment.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(a.header + kHdrCounter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int MT, int SCMAX>
__device__ void stage2_tile(const FusedArgs& a, Lds<MT>& lds, int64_t rt) {
    const uint32_t* tile = a.u_tiles + rt * a.nsc2 * 64;
    constexpr int kWindowSc = 4 * SCMAX;
    uint32_t words[SCMAX];
    load_words<SCMAX>(words, tile, 0, a.nsc2);  // prefetch before waiting

    if (threadIdx.x == 0) {
        uint32_t spins = 0;
        while (__hip_atomic_load(a.header + kHdrCounter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) <
               static_cast<uint32_t>(a.n1)) {
            if (++spins > kSpinLimit) {
                __hip_atomic_store(a.header + kHdrError, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

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

    const int64_t lm_ld = a.n1 * kTileRows;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t w0 = 0; w0 < a.nsc2; w0 += kWindowSc) {
        if (w0 > 0) load_words<SCMAX>(words, tile, w0, a.nsc2);
        const int64_t c0 = w0 * kSuperCols;
        const int64_t cend = (w0 + kWindowSc < a.nsc2 ? w0 + kWindowSc : a.nsc2) * kSuperCols;
        stage_columns<MT>(lds, c0, static_cast<int>(cend - c0), a.rank, a.tokens,
                          [&](int t, int64_t col) { return a.lm[t * lm_ld + col]; });
        __syncthreads();
        acc = tile_mfma<MT, SCMAX>(lds, words, w0, a.nsc2, w0, acc);
        __syncthreads();
    }

    const float sum = reduce_waves<MT>(lds, acc);
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

    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done =
            __hip_atomic_fetch_add(a.header + kHdrDone, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (done + 1 == static_cast<uint32_t>(a.n2)) {
            __hip_atomic_store(a.header + kHdrCounter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.header + kHdrDone, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int MT, int SCMAX>
__global__ __launch_bounds__(kBlock) void k_decode_fused(const FusedArgs a) {
    __shared__ Lds<MT> lds;
    const int64_t b = blockIdx.x;
    if (b < a.n1) {
        stage1_tile<MT, SCMAX>(a, lds, b);
    } else {
        stage2_tile<MT, SCMAX>(a, lds, b - a.n1);
    }
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

}  // namespace

namespace nq {

int64_t decode_scratch_bytes(const nq_linear_desc* d, int64_t tokens) {
    (void)tokens;
    if (!d->tiles) return 0;
    const TilesGeometry g = geometry(d->in_features, d->out_features, d->rank);
    const int64_t lm = kMaxTokens * g.rt1 * kTileRows * 4;
    const int64_t wgmax = g.rt1 * kMaxTokens * 4;
    return ((lm + 255) & ~int64_t(255)) + ((wgmax + 255) & ~int64_t(255));
}

bool decode_path_applies(const nq_linear_desc* d, int64_t tokens) {
    return d->tiles != nullptr && tokens >= 1 && tokens <= kMaxTokens;
}

int launch_decode(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y,
                  int y_dtype, void* scratch, hipStream_t stream) {
    const TilesGeometry g = geometry(d->in_features, d->out_features, d->rank);
    if (d->tiles_bytes < static_cast<int64_t>(kHeaderWords + g.v_words + g.u_words) * 4) return NQ_ERR_ARGUMENT;
    FusedArgs a{};
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
    const int64_t lm_bytes = kMaxTokens * g.rt1 * kTileRows * 4;
    a.lm = reinterpret_cast<float*>(ws);
    a.wgmax = reinterpret_cast<float*>(ws + ((lm_bytes + 255) & ~int64_t(255)));
    const dim3 grid(static_cast<unsigned>(g.rt1 + g.rt2));
    if (tokens == 1) {
        hipLaunchKernelGGL((k_decode_fused<1, 24>), grid, dim3(kBlock), 0, stream, a);
    } else if (tokens <= 4) {
        hipLaunchKernelGGL((k_decode_fused<4, 6>), grid, dim3(kBlock), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_decode_fused<16, 4>), grid, dim3(kBlock), 0, stream, a);
    }
    return launch_status();
}

}  // namespace nq

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

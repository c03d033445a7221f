// Decode path (tokens <= 16) for the packed binary low-rank linear on gfx950,
// for one linear or a batch of up to 8 linears per launch.
//
//   lm[t, r] = s_mid[r] * Σ_i sgn(V[r, i]) * x[t, i] * s_in[i]           (stage 1)
//   y[t, o]  = s_out[o] * Σ_r sgn(U[o, r]) * lm[t, r] + salient + bias    (stage 2)
//
// Both stages are the same contraction: rows R of a sign matrix [R, K] against
// an activation a[t, k], on v_mfma_i32_16x16x64_i8 with exact integer
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
// d of MFMA m; the bits are b in {0, 1} with sgn = 1 - 2b.
//
// Activation operands. With a power of two E shared by a chunk, MFMA m
// receives an integer w_m ~ a * 2^(E+7-m) (w_7 ~ -a * 2^E) as signed int8
// digits w = Σ_j 256^j d_j in A rows 4*t + j. Every product with B is then b
// times a multiple of 2^-(E+7) whatever m is, so the eight MFMAs of a chunk
// share one int32 accumulator T (per digit row), and eight more MFMAs against
// B = 0x01010101 << m give S, the same sum with every b = 1. Then
//     Σ_k sgn_k a_k ~ (S - 2T) / 2^(E+7),   combined over digit rows as
//     Σ_j 256^j (S_j - 2 T_j)   (each S_j - 2 T_j exact in int32),
//     chunk partial = 2^-E * 2^-7 * Σ_j 256^j (S_j - 2 T_j).
// The only rounding before fp32 is that of the w's.
//   Stage 1 stages x * s_in per (wave, chunk, block of up to 4 tokens): lane L
//     takes the 8 consecutive columns 512c + 128d + 16m + 8h + {0..7} of
//     (m, d, h) = (L >> 3, (L >> 1) & 3, L & 1) (one 16-byte load of x and one
//     of s_in for 16-bit x), the wave max gives E (|a 2^E| < 2^23, so
//     w_m = rint(a 2^(E+7-m)) has four digits), and each lane writes its
//     digit bytes into the wave's LDS area A[m][row][g][16 B] (g = 2h, 2h + 1,
//     byte 4d + b); each lane then reads its eight A operands (one 16-byte LDS
//     read per MFMA).
//   Stage 2 does no staging: stage 1's epilogue writes lm straight into the
//     stage-2 operand layout in global memory as x_q = rint(lm 2^E) times
//     2^(7-m) (four digits, |x_q| <= 2^22) with one exponent per token from a
//     bound every stage-1 workgroup computes identically, |lm| <= max|s_mid| *
//     Σ_i |x_i s_in_i| (summed per chunk by the staging waves, then in chunk
//     order); stage 2 loads a chunk's operands (one
//     token: 2 KB, spread through LDS; more tokens: one 16-byte load each).
// Chunk partials are summed in chunk order, so the result is the same for
// every launch shape (waves or tiles per workgroup, split or fused launch).
//
// Workgroup: NW waves; wave w takes chunks w, w + NW, ... of TW consecutive
// tiles, so one staged chunk feeds TW tiles. Per (chunk, tile) the wave stores
// its fp32 partial in LDS; after one barrier each output sums its partials in
// chunk order and the epilogue applies s_mid (stage 1) or s_out + salient +
// bias (stage 2). The grid is two-dimensional (blockIdx.y = batch member), so
// a workgroup needs one round trip to its kernel arguments.
//
// Latency: every load of a pass (activations, then sign words; in the fused
// stage 2 the words before the wait) is issued from straight-line code before
// any of it is used: no branch surrounds a load (addresses are clamped, dead
// chunks reload a valid chunk and skip only the arithmetic, the wave index is
// made uniform with readfirstlane), so the compiler never waits on one load to
// issue the next. The stage-1 activation dtype pair is a template parameter
// (bf16 / f16 / f32 x with fp16 scales as vector loads); any other
// combination, and unaligned buffers, take a generic variant whose element
// loads are two unconditional 16-bit loads decoded by a uniform select.
//
// Launch structure (nq_linear_desc.decode_launch):
//   split (default): kernel 1 runs the stage-1 tiles of every linear in the
//     batch and writes the stage-2 operands; kernel 2 runs the stage-2 tiles. The kernel
//     boundary is the grid-wide barrier. From five tokens a kernel 0 first
//     stages x * s_in once per (chunk, token block) and kernel 1 loads those
//     operands instead of staging them in every workgroup (k_decode_stage0,
//     k_decode_stage1m below).
//   fused: one kernel whose first grid rows are the stage-1 workgroups and
//     the rest the stage-2 workgroups. Stage-1 workgroups store the operands
//     at agent scope and then signal; stage-2 workgroups issue their U loads,
//     wait for their linear's signal (bounded spin) and only then load the
//     operands. Workgroups are dispatched in linear index order, so every
//     stage-1 workgroup is resident or finished before a stage-2 workgroup
//     can take its slot, and stage-1 workgroups never wait.
// Measured on MI355X, a graph-launched kernel boundary (about 1.5 us) is
// cheaper than any grid-wide handoff inside a kernel (3 us or more across the
// eight XCDs), hence split is the default.
#pragma once

#include "nq_decode.h"

namespace nqdec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

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
// Words on the misc line. kMiscSpin is the fused launch's spin limit
// (kSpinLimit from prepare; a host may lower it, e.g. to exercise the timeout).
enum : int { kMiscError = 0, kMiscMagic = 1, kMiscMaxMid = 2, kMiscSpin = 3 };

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

// Kernel-side indices are 32-bit: the host rejects a launch whose word,
// operand or element offsets could reach 2^31 (check_offsets in nq_decode.hip).
__device__ __forceinline__ int chunk_words32(int nb, int c) {
    const int r = nb - kChunkBlocks * c;
    return r < kChunkBlocks ? r : kChunkBlocks;
}

// ---------------------------------------------------------------------------
// Decode kernels.
// ---------------------------------------------------------------------------

// One linear of a decode launch as the kernels and the host planning use it.
struct Lin {
    int64_t in, rank, out;
    MatGeo g1, g2;           // V [rank, in], U [out, rank]
    int64_t nwg1, nwg2;      // workgroups of each stage (tiles / tiles per workgroup)
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
    uint8_t* lmq;            // stage-2 A operands, see lmq_offset
    int* lme;                // [tokens] exponent of lmq per token
    int nw1, nw2;            // waves per workgroup of each stage (the fused launch: both equal)
    // Decoder fusions (nq_linear_batch_fused, one token; null / zero otherwise).
    const void* x2;          // gated input: up [in] (fp32); x is the gate
    const float* col_scale;  // normed input: fp32 column scale replacing s_in
    const float* slots_in;   // normed input: sums of squares of x per 16-row tile of its producer
    float* residual;         // stage 2: residual[o] += y (y is not written)
    float* slots_out;        // stage 2: sum of residual^2 per 16-row output tile
    int nslots;              // entries of slots_in
    float eps;               // normed input: RMSNorm epsilon
    // Attention input (one token): x is the fp16 block outputs (acc / sum) of
    // the decode attention's pass 1, [heads][attn_blocks][head_dim] with heads =
    // in / head_dim, and attn_ml their fp32 (max, sum) pairs [heads][attn_blocks][2].
    const float* attn_ml;
    const int32_t* attn_pos;    // the token's cache position
    int attn_blocks;            // cache blocks of kAttnBlockRows rows
    int attn_hd_log2;           // log2(head_dim)
    int64_t attn_max_positions;
};

// The kernel arguments of one linear: four 64-byte lines, each holding what
// one use reads first, so a workgroup waits on one line before its first
// vector load (stage 0, stage 1, stage 2) or two (the fused input kinds of
// stage 1; the fused launch). load_args rebuilds the rest of a Lin: the
// geometry from in / rank / out, the tiles header from the V tile pointer,
// the exponent line from the operand pointer. Every scalar-cache line a
// launch waits on before its first vector load lengthens it: measured on
// MI355X, twelve scalar loads over five lines instead of six over three put
// the end-to-end Qwen3-8B decode at 522.9 instead of 537.2 tok/s.
struct alignas(64) LinArgs {
    // line 0: stage 1 and stage 0
    const uint32_t* v_tiles;
    const void* x;
    const void* s_in;
    const void* s_mid;
    uint8_t* lmq;
    int32_t in, rank, nwg1;
    uint32_t kinds1;         // x_dtype | scale_dtype << 8 | nw1 << 16 | tokens << 24
    int32_t pad0_[2];
    // line 1: stage 2
    const uint32_t* u_tiles;
    uint8_t* lmq2;           // lmq again
    const void* s_out;
    const void* bias;
    void* y;
    int32_t out, rank2, nwg2, salient_count;
    uint32_t kinds2;         // tokens | scale_dtype << 8 | bias_dtype << 16 | nw2 << 24
    uint32_t kinds3;         // y_dtype | salient_dtype << 8 | x_dtype << 16
    // line 2: the fused input kinds of stage 1
    const void* x2;
    const float* col_scale;
    const float* slots_in;
    const float* attn_ml;
    const int32_t* attn_pos;
    int32_t nslots;
    float eps;
    int32_t attn_blocks, attn_hd_log2;
    int64_t attn_max_positions;
    // line 3: stage 2's epilogue (residual, salient columns)
    float* residual;
    float* slots_out;
    const int32_t* salient_indices;
    const void* salient_values;
    const void* salient_scales;
    const void* x_s2;        // x again
    int32_t in2;             // in again
    int32_t pad1_[3];
};
static_assert(sizeof(LinArgs) == 256 && offsetof(LinArgs, u_tiles) == 64 && offsetof(LinArgs, x2) == 128 &&
                  offsetof(LinArgs, residual) == 192 && offsetof(LinArgs, kinds1) + 4 <= 64 &&
                  offsetof(LinArgs, kinds3) + 4 == 128 && offsetof(LinArgs, attn_max_positions) + 8 == 192,
              "one use per 64-byte line");

// Stage-2 operand bytes of a [out, rank] U for `tokens` tokens (1: one block of
// one token; 2-4: one block of four; 5-16: four blocks of four). A multiple of 256.
__host__ __device__ inline int64_t lmq_bytes_for(const MatGeo& g2, int64_t tokens) {
    return g2.nc * (tokens == 1 ? 2048 : (tokens <= 4 ? 8192 : 32768));
}

// The kernel arguments of a Lin (host side). The narrow fields were range
// checked by the host (offsets below 2^31, at most 16 tokens and waves).
inline LinArgs pack_args(const Lin& a) {
    LinArgs p{};
    p.v_tiles = a.v_tiles;
    p.x = a.x;
    p.s_in = a.s_in;
    p.s_mid = a.s_mid;
    p.lmq = a.lmq;
    p.in = static_cast<int32_t>(a.in);
    p.rank = static_cast<int32_t>(a.rank);
    p.nwg1 = static_cast<int32_t>(a.nwg1);
    p.kinds1 = static_cast<uint32_t>(a.x_dtype) | static_cast<uint32_t>(a.scale_dtype) << 8 |
               static_cast<uint32_t>(a.nw1) << 16 | static_cast<uint32_t>(a.tokens) << 24;
    p.u_tiles = a.u_tiles;
    p.lmq2 = a.lmq;
    p.s_out = a.s_out;
    p.bias = a.bias;
    p.y = a.y;
    p.out = static_cast<int32_t>(a.out);
    p.rank2 = p.rank;
    p.nwg2 = static_cast<int32_t>(a.nwg2);
    p.salient_count = static_cast<int32_t>(a.salient_count);
    p.kinds2 = static_cast<uint32_t>(a.tokens) | static_cast<uint32_t>(a.scale_dtype) << 8 |
               static_cast<uint32_t>(a.bias_dtype) << 16 | static_cast<uint32_t>(a.nw2) << 24;
    p.kinds3 = static_cast<uint32_t>(a.y_dtype) | static_cast<uint32_t>(a.salient_dtype) << 8 |
               static_cast<uint32_t>(a.x_dtype) << 16;
    p.x2 = a.x2;
    p.col_scale = a.col_scale;
    p.slots_in = a.slots_in;
    p.attn_ml = a.attn_ml;
    p.attn_pos = a.attn_pos;
    p.nslots = a.nslots;
    p.eps = a.eps;
    p.attn_blocks = a.attn_blocks;
    p.attn_hd_log2 = a.attn_hd_log2;
    p.attn_max_positions = a.attn_max_positions;
    p.residual = a.residual;
    p.slots_out = a.slots_out;
    p.salient_indices = a.salient_indices;
    p.salient_values = a.salient_values;
    p.salient_scales = a.salient_scales;
    p.x_s2 = a.x;
    p.in2 = p.in;
    return p;
}

// ---------------------------------------------------------------------------
// XCD-contiguous workgroup order.
//
// MI355X dispatches the workgroups of a launch to its eight XCDs round-robin
// in linear order, so with a grid row whose x extent is a multiple of 8,
// workgroup x runs on XCD x % 8. The split-launch kernels give the workgroups
// of each XCD one contiguous range of blocks: with B live workgroups in a row
// and q = B / 8, r = B % 8, those on XCD c take blocks [c q + min(c, r),
// (c + 1) q + min(c + 1, r)) (xcd_block). Each XCD (one L2) then reads one
// contiguous range of every sign matrix and writes one contiguous range of
// the outputs. Measured on MI355X against blocks in launch order: the
// Qwen3-8B gate/up call 9.40 instead of 9.77 us, end-to-end decode 534 instead
// of 514 tokens/s.
// ---------------------------------------------------------------------------

// Block of workgroup x (x < nblocks; XCD x % 8) in the XCD-contiguous order.
__host__ __device__ inline int xcd_block(int x, int nblocks) {
    const int q = nblocks >> 3, r = nblocks & 7, c = x & 7;
    return c * q + (c < r ? c : r) + (x >> 3);
}

// Kernel arguments of a launch: the members' lines first, so member i starts
// at byte 256 i of the segment.
struct Batch {
    LinArgs p[kMaxBatch];
    int32_t count;           // members (the fused launch)
};

// A launch as the host plans it: its members as Lins and the tiles per
// workgroup of each stage (the kernels take those as template arguments).
struct HostBatch {
    int count;
    int tw1, tw2;
    Lin p[kMaxBatch];
};

inline void pack_batch(const HostBatch& h, Batch& b) {
    for (int i = 0; i < kMaxBatch; ++i) b.p[i] = i < h.count ? pack_args(h.p[i]) : LinArgs{};
    b.count = h.count;
}

// A member's arguments as a Lin (load_args): the fields of the line a use
// reads first are copied from the kernel-argument segment and passed through
// one empty asm (pin_line*), so all their scalar loads are issued together and
// complete at one point instead of lazily (one dependent round trip per
// uniform branch that needs a field); the derived fields are computed from
// them after that point. Fields of the other lines are copied too and load
// where a kernel first uses them. The copies stay typed loads, so the
// pointers are still known to be global. The fused input kinds add the
// fields of line 2 they read first (kArgsNorm: the column scale and the
// producer's row sums; kArgsGated: the up input; kArgsAttn: the attention
// partials and position) to the same wait: left to the compiler, those
// loads were issued only after it, a second round trip before the kernel's
// first vector load.
enum : int { kArgsPlain = 0, kArgsNorm = 1, kArgsGated = 2, kArgsAttn = 3 };
enum : int { kPinStage1 = 1, kPinStage2 = 2, kPinStages = 3 };

// Device-side geometry from 32-bit sizes (shifts only).
__device__ __forceinline__ MatGeo mat_geo32(uint32_t rows, uint32_t cols) {
    static_assert(kTileRows == 16 && kBlockCols == 128 && kChunkBlocks == 4, "shift forms below");
    const uint32_t nb = (cols + kBlockCols - 1) >> 7;
    MatGeo g;
    g.nt = (rows + kTileRows - 1) >> 4;
    g.nb = nb;
    g.nc = (nb + kChunkBlocks - 1) >> 2;
    return g;
}

// Line 0 (stage 1) and line 1 (stage 2), as loaded.
struct Line0 {
    const uint32_t* v_tiles;
    const void* x;
    const void* s_in;
    const void* s_mid;
    uint8_t* lmq;
    uint32_t in, rank, nwg1, kinds1;
};
struct Line1 {
    const uint32_t* u_tiles;
    uint8_t* lmq;
    const void* s_out;
    const void* bias;
    void* y;
    uint32_t out, rank, nwg2, salient_count, kinds2, kinds3;
};

__device__ __forceinline__ Line0 copy_line0(const LinArgs& s) {
    return Line0{s.v_tiles, s.x, s.s_in, s.s_mid, s.lmq, static_cast<uint32_t>(s.in), static_cast<uint32_t>(s.rank),
                 static_cast<uint32_t>(s.nwg1), s.kinds1};
}
__device__ __forceinline__ Line1 copy_line1(const LinArgs& s) {
    return Line1{s.u_tiles, s.lmq2, s.s_out, s.bias, s.y, static_cast<uint32_t>(s.out),
                 static_cast<uint32_t>(s.rank2), static_cast<uint32_t>(s.nwg2),
                 static_cast<uint32_t>(s.salient_count), s.kinds2, s.kinds3};
}

#define NQ_PIN0_OUT(l) "+s"(l.in), "+s"(l.rank), "+s"(l.nwg1), "+s"(l.kinds1)
#define NQ_PIN0_IN(l) "s"(l.v_tiles), "s"(l.x), "s"(l.s_in), "s"(l.s_mid), "s"(l.lmq)
#define NQ_PIN1_OUT(l) "+s"(l.out), "+s"(l.rank), "+s"(l.nwg2), "+s"(l.salient_count), "+s"(l.kinds2)
#define NQ_PIN1_IN(l) "s"(l.u_tiles), "s"(l.lmq), "s"(l.s_out), "s"(l.bias)

// Line 0, with the line-2 fields the input kind reads first.
template <int EXTRA>
__device__ __forceinline__ void pin_line0(Line0& l, const void*& x2, const float*& col_scale, const float*& slots_in,
                                          const float*& attn_ml, const int32_t*& attn_pos, int& nslots, float& eps,
                                          int& attn_blocks, int& attn_hd_log2, int64_t& attn_max_positions) {
    if constexpr (EXTRA == kArgsNorm) {
        asm volatile("" : NQ_PIN0_OUT(l), "+s"(nslots), "+s"(eps) : NQ_PIN0_IN(l), "s"(col_scale), "s"(slots_in));
    } else if constexpr (EXTRA == kArgsGated) {
        asm volatile("" : NQ_PIN0_OUT(l) : NQ_PIN0_IN(l), "s"(x2));
    } else if constexpr (EXTRA == kArgsAttn) {
        asm volatile(""
                     : NQ_PIN0_OUT(l), "+s"(attn_blocks), "+s"(attn_hd_log2), "+s"(attn_max_positions)
                     : NQ_PIN0_IN(l), "s"(attn_ml), "s"(attn_pos));
    } else {
        asm volatile("" : NQ_PIN0_OUT(l) : NQ_PIN0_IN(l));
    }
}
__device__ __forceinline__ void pin_line1(Line1& l) { asm volatile("" : NQ_PIN1_OUT(l) : NQ_PIN1_IN(l)); }
// Both lines (the fused launch), or line 1 of two members (the paired stage 2):
// one wait.
__device__ __forceinline__ void pin_lines(Line0& l0, Line1& l1) {
    asm volatile("" : NQ_PIN0_OUT(l0), NQ_PIN1_OUT(l1) : NQ_PIN0_IN(l0), NQ_PIN1_IN(l1));
}
__device__ __forceinline__ void pin_line1_pair(Line1& a, Line1& b) {
    asm volatile("" : NQ_PIN1_OUT(a), NQ_PIN1_OUT(b) : NQ_PIN1_IN(a), NQ_PIN1_IN(b));
}
#undef NQ_PIN0_OUT
#undef NQ_PIN0_IN
#undef NQ_PIN1_OUT
#undef NQ_PIN1_IN

// The Lin of member s, from its (pinned) line 0 and line 1 and the lazily
// loaded lines 2 and 3. FROM1: the fields both lines hold (rank, tokens, the
// scale dtype, the operand pointer) are taken from line 1 (stage 2), else
// from line 0.
template <bool FROM1>
__device__ __forceinline__ Lin build_lin(const LinArgs& s, const Line0& l0, const Line1& l1, const void* x2,
                                         const float* col_scale, const float* slots_in, const float* attn_ml,
                                         const int32_t* attn_pos, int nslots, float eps, int attn_blocks,
                                         int attn_hd_log2, int64_t attn_max_positions) {
    Lin a;
    const uint32_t rank = FROM1 ? l1.rank : l0.rank;
    const uint32_t in = FROM1 ? static_cast<uint32_t>(s.in2) : l0.in;
    const int tokens = FROM1 ? static_cast<int>(l1.kinds2 & 0xff) : static_cast<int>(l0.kinds1 >> 24);
    a.in = in;
    a.rank = rank;
    a.out = l1.out;
    a.g1 = mat_geo32(rank, in);
    a.g2 = mat_geo32(l1.out, rank);
    a.nwg1 = l0.nwg1;
    a.nwg2 = l1.nwg2;
    a.v_tiles = l0.v_tiles;
    a.u_tiles = l1.u_tiles;
    a.header = const_cast<uint32_t*>(l0.v_tiles) - kHeaderWords;
    a.x = FROM1 ? s.x_s2 : l0.x;
    a.x_dtype = FROM1 ? static_cast<int>((l1.kinds3 >> 16) & 0xff) : static_cast<int>(l0.kinds1 & 0xff);
    a.tokens = tokens;
    a.s_in = l0.s_in;
    a.s_mid = l0.s_mid;
    a.s_out = l1.s_out;
    a.scale_dtype = FROM1 ? static_cast<int>((l1.kinds2 >> 8) & 0xff) : static_cast<int>((l0.kinds1 >> 8) & 0xff);
    a.salient_count = l1.salient_count;
    a.salient_indices = s.salient_indices;
    a.salient_values = s.salient_values;
    a.salient_dtype = static_cast<int>((l1.kinds3 >> 8) & 0xff);
    a.salient_scales = s.salient_scales;
    a.bias = l1.bias;
    a.bias_dtype = static_cast<int>((l1.kinds2 >> 16) & 0xff);
    a.y = l1.y;
    a.y_dtype = static_cast<int>(l1.kinds3 & 0xff);
    a.lmq = FROM1 ? l1.lmq : l0.lmq;
    a.lme = reinterpret_cast<int*>(a.lmq + lmq_bytes_for(a.g2, tokens));
    a.nw1 = static_cast<int>((l0.kinds1 >> 16) & 0xff);
    a.nw2 = static_cast<int>(l1.kinds2 >> 24);
    a.x2 = x2;
    a.col_scale = col_scale;
    a.slots_in = slots_in;
    a.residual = s.residual;
    a.slots_out = s.slots_out;
    a.nslots = nslots;
    a.eps = eps;
    a.attn_ml = attn_ml;
    a.attn_pos = attn_pos;
    a.attn_blocks = attn_blocks;
    a.attn_hd_log2 = attn_hd_log2;
    a.attn_max_positions = attn_max_positions;
    return a;
}

template <int STAGE, int EXTRA = kArgsPlain>
__device__ __forceinline__ Lin load_args(const Batch& batch, int member) {
    const LinArgs& s = batch.p[member];
    Line0 l0 = copy_line0(s);
    Line1 l1 = copy_line1(s);
    const void* x2 = s.x2;
    const float* col_scale = s.col_scale;
    const float* slots_in = s.slots_in;
    const float* attn_ml = s.attn_ml;
    const int32_t* attn_pos = s.attn_pos;
    int nslots = s.nslots;
    float eps = s.eps;
    int attn_blocks = s.attn_blocks, attn_hd_log2 = s.attn_hd_log2;
    int64_t attn_max_positions = s.attn_max_positions;
    if constexpr (STAGE == kPinStage2) {
        pin_line1(l1);
    } else if constexpr (STAGE == kPinStages) {
        pin_lines(l0, l1);
    } else {
        pin_line0<EXTRA>(l0, x2, col_scale, slots_in, attn_ml, attn_pos, nslots, eps, attn_blocks, attn_hd_log2,
                         attn_max_positions);
    }
    return build_lin<STAGE == kPinStage2>(s, l0, l1, x2, col_scale, slots_in, attn_ml, attn_pos, nslots, eps,
                                          attn_blocks, attn_hd_log2, attn_max_positions);
}

// Stage 2 of members 0 and 1 (the paired stage 2): one wait for both lines.
__device__ __forceinline__ void load_args_pair(const Batch& batch, Lin& a, Lin& b) {
    const LinArgs& s = batch.p[0];
    const LinArgs& t = batch.p[1];
    Line0 s0 = copy_line0(s), t0 = copy_line0(t);
    Line1 s1 = copy_line1(s), t1 = copy_line1(t);
    pin_line1_pair(s1, t1);
    a = build_lin<true>(s, s0, s1, s.x2, s.col_scale, s.slots_in, s.attn_ml, s.attn_pos, s.nslots, s.eps,
                        s.attn_blocks, s.attn_hd_log2, s.attn_max_positions);
    b = build_lin<true>(t, t0, t1, t.x2, t.col_scale, t.slots_in, t.attn_ml, t.attn_pos, t.nslots, t.eps,
                        t.attn_blocks, t.attn_hd_log2, t.attn_max_positions);
}
// Activation kinds (template parameter AK): how stage 1 reads a[t, k].
enum : int {
    kActBf16 = 0,      // bf16 x, fp16 s_in, vector loads
    kActF16 = 1,       // fp16 x, fp16 s_in, vector loads
    kActF32 = 2,       // fp32 x, fp16 s_in, vector loads
    kActGeneric = 3,   // any float x and s_in, element loads
    kActNormF32 = 4,   // fp32 x (a residual), fp32 col_scale (norm weight * s_in), RMS factor from slots_in
    kActGatedF32 = 5,  // silu(x) * x2 from fp32 gate x and up x2, fp16 s_in
    kActAttn8 = 6,     // attention output merged from pass-1 partials of up to 8 cache blocks, fp16 s_in
    kActAttn16 = 7,    // the same for up to 16 cache blocks
    kActAttn12 = 8,    // the same for up to 12 cache blocks (fewer partial registers than kActAttn16)
    kActAttn8E = 9,    // kActAttn8 for an even block count: two blocks' (max, sum) pairs per load
    kActAttn12E = 10,  // kActAttn12 for an even block count
    kActAttn16E = 11,  // kActAttn16 for an even block count
};

template <int AK>
constexpr bool attn_kind() { return AK >= kActAttn8 && AK <= kActAttn16E; }

// Attention kinds that load two blocks' (max, sum) pairs at once (even block counts).
template <int AK>
constexpr bool attn_paired() { return AK == kActAttn8E || AK == kActAttn12E || AK == kActAttn16E; }

// Cache blocks whose partials one lane loads (the attention kinds).
template <int AK>
constexpr int attn_parts() {
    return AK == kActAttn16 || AK == kActAttn16E ? 16 : (AK == kActAttn12 || AK == kActAttn12E ? 12 : 8);
}

using nq::kAttnBlockRows;

// Column-scale dtype of a vector kind.
template <int AK>
constexpr int col_scale_dtype() { return AK == kActNormF32 ? NQ_DTYPE_F32 : NQ_DTYPE_F16; }

// Rows of an A operand block: 4 digit rows for each of TPB tokens.
template <int TPB>
struct Ops {
    static constexpr int kRows = 4 * TPB;
    static constexpr int kBytes = 8 * kRows * 4 * 16;  // A[m][row][g][16 B]
};

// Byte offset of (chunk c, token block tb, MFMA m, row, lane group g) in the
// stage-2 operand buffer; byte j of the 16 is column 512c + 128*(j/4) + 16m +
// 4g + j%4.
template <int TPB, int TB>
__host__ __device__ inline int lmq_offset(int c, int tb, int m, int row, int g) {
    return ((((c * TB + tb) * 8 + m) * Ops<TPB>::kRows + row) * 4 + g) * 16;
}

template <int TPB, int TB>
__host__ __device__ inline int64_t lmq_bytes(const MatGeo& g2) { return g2.nc * TB * Ops<TPB>::kBytes; }

// Several tokens (split launch from five tokens): stage 0 writes the stage-1 A
// operands of x * s_in in the lmq layout (xq, one token block up to four
// tokens, four above), with the exponent (xe) and Σ |x s_in| (xm) of every
// (chunk, token) at [chunk * kMaxTokens + token]. They follow the 256-byte
// exponent line lme in the workspace, each 256-byte aligned, so the kernels
// derive their addresses from lme and the geometry. Measured on MI355X: the
// three pointers as kernel arguments, loaded by every launch's load_args,
// cost the one-token stack 1.0 us per Qwen3 layer (35.0 against 36.0) and
// end-to-end decode 2.3% (523.3 against 511.5 tok/s).
__host__ __device__ inline int64_t round256(int64_t n) { return (n + 255) & ~int64_t(255); }
__host__ __device__ inline int64_t xq_bytes_for(const MatGeo& g1, int64_t tokens) {
    return tokens == 1 ? 0 : g1.nc * (tokens <= 4 ? 1 : 4) * Ops<4>::kBytes;
}
__host__ __device__ inline int64_t xe_bytes_for(const MatGeo& g1, int64_t tokens) {
    return tokens == 1 ? 0 : round256(g1.nc * kMaxTokens * 4);
}
struct MultiWs {
    uint8_t* xq;
    int* xe;
    float* xm;
};
__host__ __device__ inline MultiWs multi_ws(int* lme, const MatGeo& g1, int64_t tokens) {
    char* const xq = reinterpret_cast<char*>(lme) + 256;
    char* const xe = xq + round256(xq_bytes_for(g1, tokens));
    return MultiWs{reinterpret_cast<uint8_t*>(xq), reinterpret_cast<int*>(xe),
                   reinterpret_cast<float*>(xe + xe_bytes_for(g1, tokens))};
}

// Nearest integer of x (halves round up), |x| < 2^31: one instruction
// (v_cvt_rpi_i32_f32 computes floor(x + 0.5)) where rintf and a conversion
// take two.
__device__ __forceinline__ int round_to_int(float x) {
    int r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

// 2^e for an integer e in the fp32 normal range.
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float(static_cast<uint32_t>(e + 127) << 23); }

// Exponent E with bound * 2^E < 2^(top + 1), clamped to [-113, 119] (so 2^-E-7
// stays a normal fp32); 0 when the bound is zero or not finite-positive.
__device__ __forceinline__ int range_exponent(float bound, int top) {
    if (!(bound > 0.0f)) return 0;
    int e = static_cast<int>((__float_as_uint(bound) >> 23) & 0xff) - 127;
    e = top - (e < -126 ? -126 : e);
    return e > 119 ? 119 : (e < -113 ? -113 : e);
}

template <int CTRL>
__device__ __forceinline__ float dpp_maxf(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false);
    return fmaxf(x, __int_as_float(y));
}

// Max over the whole wave (every lane gets the result, as a uniform value).
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

template <int CTRL>
__device__ __forceinline__ float dpp_addf(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false);
    return x + __int_as_float(y);
}

// Sum over each row of 16 lanes (every lane of the row gets it); the whole
// wave must be active.
__device__ __forceinline__ float row16_sum(float v) {
    v = dpp_addf<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_addf<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_addf<0x141>(v);  // row_half_mirror
    return dpp_addf<0x140>(v);  // row_mirror
}

// Sum over the whole wave (a uniform value); the whole wave must be active.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
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

// A word at a uniform address, read through the scalar data cache (s_load).
__device__ __forceinline__ uint32_t scalar_load(const uint32_t* p) {
    typedef const __attribute__((address_space(4))) uint32_t* ConstWord;
    return *(ConstWord)(p);
}

// Element i of a 16-bit buffer in the RawElem form (both halves the same).
__device__ __forceinline__ RawElem load_half(const void* __restrict__ p, int64_t i) {
    RawElem r;
    r.lo = r.hi = static_cast<const uint16_t*>(p)[i];
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

// --- stage-1 activation runs: 4 consecutive columns -----------------------------

// Raw registers of one run for kind AK: fp16/bf16 pairs in two dwords, fp32 in
// four, generic as four raw elements.
template <int AK>
struct Run {
    static constexpr int kDwords = (AK == kActBf16 || AK == kActF16) ? 2 : 4;
    uint32_t u[AK == kActGeneric ? 1 : kDwords];
    RawElem e[AK == kActGeneric ? 4 : 1];
};

// Columns [k, k + 4) of row `row` of a buffer with leading dimension ld,
// loaded from an address clamped to rows_valid rows and `cols` columns
// (vector kinds: k % 4 == 0, cols % 4 == 0, cols >= 4, ld % 4 == 0 and an
// aligned base, checked by the host; generic: each element clamped). Values
// past the valid range are zeroed when staged.
template <int AK, int DT>
__device__ __forceinline__ Run<AK> load_run(const void* __restrict__ p, int rt_dtype, int row, int rows_valid,
                                            int ld, int k, int cols) {
    Run<AK> r;
    const int rr = row < rows_valid ? row : rows_valid - 1;
    if constexpr (AK == kActGeneric) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kk = k + i < cols ? k + i : cols - 1;
            r.e[i] = load_elem(p, rt_dtype, rr * ld + kk);
        }
    } else {
        const int kk = k < cols ? k : cols - 4;
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

template <int AK>
constexpr int act_dtype() {
    return AK == kActBf16 ? NQ_DTYPE_BF16 : (AK == kActF16 ? NQ_DTYPE_F16 : NQ_DTYPE_F32);
}

// Staging lane roles: lane L stages (m, d, h) = (L >> 3, (L >> 1) & 3, L & 1),
// the eight consecutive columns k0 + {0..7}, k0 = 512c + 128d + 16m + 8h: run 0
// is lane group g = 2h, run 1 is g = 2h + 1 (byte 4d + b of each group's 16).
__device__ __forceinline__ int stage_col0(int c, int lane) {
    return kChunkCols * c + kBlockCols * ((lane >> 1) & 3) + 16 * (lane >> 3) + 8 * (lane & 1);
}

// Registers one stage-1 wave holds for one chunk: the activation runs of every
// token, the s_in runs and the sign words of its TW tiles.
// Attention kinds: a lane's partials for its eight columns (one head, eight
// dimensions): acc of every cache block (two runs of four), the block's
// (max, sum) pair, and the token's position.
template <int NB>
struct AttnParts {
    v4u out[NB];       // the block outputs of the lane's eight columns, fp16
    v2u ml[NB];        // (max, sum) of each block (single loads)
    v4u mlp[NB / 2];   // (max, sum) of blocks 2j, 2j + 1 (paired loads)
    int pos;
};
template <int AK>
struct AttnRegsOf {
    struct type {};
};
template <>
struct AttnRegsOf<kActAttn8> {
    using type = AttnParts<8>;
};
template <>
struct AttnRegsOf<kActAttn12> {
    using type = AttnParts<12>;
};
template <>
struct AttnRegsOf<kActAttn16> {
    using type = AttnParts<16>;
};
template <>
struct AttnRegsOf<kActAttn8E> {
    using type = AttnParts<8>;
};
template <>
struct AttnRegsOf<kActAttn12E> {
    using type = AttnParts<12>;
};
template <>
struct AttnRegsOf<kActAttn16E> {
    using type = AttnParts<16>;
};

template <int AK, int TOK, int TW>
struct S1Regs {
    Run<AK> x[TOK][2];
    Run<AK> x2[AK == kActGatedF32 ? TOK : 1][2];  // gated kind: up
    Run<AK> s[2];
    v4u w[TW];
    typename AttnRegsOf<AK>::type at;
};

// Registers one stage-2 wave holds for one chunk: its A operands (8 per token
// block) and the sign words of its TW tiles.
template <int TB, int TW>
struct S2Regs {
    v4i a[TB][8];
    v4u w[TW];
};

// The two runs of a lane's eight columns: one 16-byte load for 16-bit kinds
// (vector kinds need in % 8 == 0 and 16-byte aligned rows, checked by the
// host), a load per run otherwise.
template <int AK, int DT>
__device__ __forceinline__ void load_runs(Run<AK> (&r)[2], const void* __restrict__ p, int rt_dtype, int row,
                                          int rows_valid, int ld, int k, int cols) {
    if constexpr (AK != kActGeneric && DT != NQ_DTYPE_F32) {
        const int rr = row < rows_valid ? row : rows_valid - 1;
        const int kk = k < cols ? k : cols - 8;
        const v4u q = *reinterpret_cast<const v4u*>(static_cast<const uint16_t*>(p) + rr * ld + kk);
        r[0].u[0] = q.x;
        r[0].u[1] = q.y;
        r[1].u[0] = q.z;
        r[1].u[1] = q.w;
    } else {
        r[0] = load_run<AK, DT>(p, rt_dtype, row, rows_valid, ld, k, cols);
        r[1] = load_run<AK, DT>(p, rt_dtype, row, rows_valid, ld, k + 4, cols);
    }
}

template <int AK, int TOK, int TW>
__device__ __forceinline__ void load_s1_acts(S1Regs<AK, TOK, TW>& r, const Lin& a, int c, int lane) {
    constexpr int DT = act_dtype<AK>();
    const int k0 = stage_col0(c, lane);
    const int in = static_cast<int>(a.in);
    if constexpr (attn_kind<AK>()) {
        // Every block's partials, issued before the position is known (pass 1
        // stores a neutral partial for the blocks past the position); slots
        // past the cache's blocks hold the neutral partial without a load. in
        // is a multiple of 8 and of the head dimension. A block's output is
        // fp16 (acc / sum; one 16-byte load for the lane's eight columns).
        constexpr int NB = attn_parts<AK>();
        const int kk = k0 < in ? k0 : in - 8;
        const int hd = a.attn_hd_log2;
        const int blocks = a.attn_blocks;
        const int64_t head = kk >> hd;
        const _Float16* outs =
            static_cast<const _Float16*>(a.x) + ((head * blocks) << hd) + (kk & ((1 << hd) - 1));
        const float* ml = a.attn_ml + head * blocks * 2;
        if constexpr (attn_paired<AK>()) {
            // An even block count (the host's choice of kind): each head's (max,
            // sum) pairs start 16-byte aligned, and one load takes two blocks'
            // pairs (measured on MI355X, Qwen3-8B decode at 10 blocks: 571.9
            // against 567.1 tok/s).
#pragma unroll
            for (int s = 0; s < NB; s += 2) {
                if (s < blocks) {  // uniform; s + 1 < blocks too
                    r.at.out[s] = *reinterpret_cast<const v4u*>(outs + (static_cast<int64_t>(s) << hd));
                    r.at.out[s + 1] = *reinterpret_cast<const v4u*>(outs + (static_cast<int64_t>(s + 1) << hd));
                    r.at.mlp[s / 2] = *reinterpret_cast<const v4u*>(ml + 2 * s);
                } else {
                    r.at.out[s] = r.at.out[s + 1] = v4u{0u, 0u, 0u, 0u};
                    r.at.mlp[s / 2] = v4u{0xff800000u, 0u, 0xff800000u, 0u};  // (-inf, 0) twice
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < NB; ++s) {
                if (s < blocks) {  // uniform
                    r.at.out[s] = *reinterpret_cast<const v4u*>(outs + (static_cast<int64_t>(s) << hd));
                    r.at.ml[s] = *reinterpret_cast<const v2u*>(ml + 2 * s);
                } else {
                    r.at.out[s] = v4u{0u, 0u, 0u, 0u};
                    r.at.ml[s] = v2u{0xff800000u, 0u};  // (-inf, 0)
                }
            }
        }
        r.at.pos = a.attn_pos[0];
        load_runs<AK, NQ_DTYPE_F16>(r.s, a.s_in, a.scale_dtype, 0, 1, 0, k0, in);
        return;
    }
#pragma unroll
    for (int t = 0; t < TOK; ++t) load_runs<AK, DT>(r.x[t], a.x, a.x_dtype, t, a.tokens, in, k0, in);
    if constexpr (AK == kActGatedF32) {
#pragma unroll
        for (int t = 0; t < TOK; ++t) load_runs<AK, DT>(r.x2[t], a.x2, a.x_dtype, t, a.tokens, in, k0, in);
    }
    load_runs<AK, col_scale_dtype<AK>()>(r.s, AK == kActNormF32 ? static_cast<const void*>(a.col_scale) : a.s_in,
                                         a.scale_dtype, 0, 1, 0, k0, in);
}

// Sign words of chunk c for tiles t0 .. t0 + TW - 1 (tiles past the last one
// load the last tile; their results are never stored): one 16-byte load per
// lane at word lane * dw. In a partial last chunk (dw < 4) the words past dw
// belong to the next lane (or, for the last lane of the matrix, to the
// buffer's tail padding) and the MFMA step masks them out.
template <int TW>
__device__ __forceinline__ void load_words(v4u (&w)[TW], const uint32_t* tiles, int nt, int nb, int t0, int c,
                                           int lane) {
    const int dw = chunk_words32(nb, c);
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
        const int tile = t0 + tt < nt ? t0 + tt : nt - 1;
        const uint32_t* base = tiles + (tile * nb * 64 + c * 256 + static_cast<int>(__umul24(lane, dw)));
        w[tt] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(base));
    }
}

// Order this wave's LDS writes before its own reads (waves never share areas).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

// Stage-2 A operands of chunk c. The eight operands of a one-token block
// repeat four digit rows over the sixteen MFMA rows, so loading them directly
// would fetch every byte four times: one token loads the chunk's 2 KB once
// (two 16-byte loads per lane) and spread_s2_ops distributes it through the
// wave's LDS area.
constexpr int kS2SpreadBytes = 8 * 4 * 4 * 16;

// (One token; several tokens load each MFMA's operand directly, in stage2_wg.)
template <int TPB, int TB, int TW>
__device__ __forceinline__ void load_s2_ops(S2Regs<TB, TW>& r, const Lin& a, int c, int lane) {
    static_assert(TPB == 1 && TB == 1, "one token per launch");
    const uint8_t* src = a.lmq + lmq_offset<1, TB>(c, 0, 0, 0, 0);
    r.a[0][0] = *reinterpret_cast<const v4i*>(src + 16 * lane);
    r.a[0][1] = *reinterpret_cast<const v4i*>(src + kS2SpreadBytes / 2 + 16 * lane);
}

// One token: the two loaded vectors through this wave's LDS area (kS2SpreadBytes)
// into the eight A operands (MFMA m: digit row lane & 3, lane group lane >> 4).
template <int TPB, int TB, int TW>
__device__ __forceinline__ void spread_s2_ops(S2Regs<TB, TW>& r, char* __restrict__ area, int lane) {
    if constexpr (TPB == 1) {
        *reinterpret_cast<v4i*>(area + 16 * lane) = r.a[0][0];
        *reinterpret_cast<v4i*>(area + kS2SpreadBytes / 2 + 16 * lane) = r.a[0][1];
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < 8; ++m)
            r.a[0][m] = *reinterpret_cast<const v4i*>(area + lmq_offset<1, 1>(0, 0, m, lane & 3, lane >> 4));
    }
}

// Low byte of each of four ints, packed.
__device__ __forceinline__ uint32_t pack_bytes(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
           ((static_cast<uint32_t>(c) & 0xffu) << 16) | (static_cast<uint32_t>(d) << 24);
}

// Byte j of a, b, c, d packed into out[j] (a in byte 0): a 4 x 4 byte
// transpose in eight v_perm_b32 (result byte k = byte sel_k of {src0:src1},
// bytes 0-3 from src1, 4-7 from src0).
__device__ __forceinline__ void transpose_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&out)[4]) {
    const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
    const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
    const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
    const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
    out[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);        // a0 b0 c0 d0
    out[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);        // a1 b1 c1 d1
    out[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);        // a2 b2 c2 d2
    out[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);        // a3 b3 c3 d3
}

// Signed base-256 digits of w: w = d0 + 256 d1 + 65536 d2 + ..., each digit in
// [-128, 127]. The byte of d_j is the low byte of w_j with w_0 = w and
// w_{j+1} = (w_j + 128) >> 8.
__device__ __forceinline__ int next_digit_word(int w) { return (w + 128) >> 8; }

// Byte B of each of four words, packed (v_perm on the device).
template <int B>
__device__ __forceinline__ uint32_t bytes_at(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return ((a >> (8 * B)) & 0xffu) | (((b >> (8 * B)) & 0xffu) << 8) | (((c >> (8 * B)) & 0xffu) << 16) |
           (((d >> (8 * B)) & 0xffu) << 24);
}

// Normed kind: lane l's share of the producer's tile sums, vectors i * 64 + l
// (zero past nslots; nslots % 4 == 0 and nslots <= 256 * kSlotVecs, checked
// by the host).
constexpr int kSlotVecs = 4;

__device__ __forceinline__ void load_slots(v4f (&sl)[kSlotVecs], const float* __restrict__ slots, int nslots,
                                           int lane) {
    const int nv = nslots >> 2;
#pragma unroll
    for (int i = 0; i < kSlotVecs; ++i) {
        sl[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (i * 64 < nv) {  // uniform
            const int vi = i * 64 + lane;
            const v4f q = *reinterpret_cast<const v4f*>(slots + 4 * (vi < nv ? vi : nv - 1));
            sl[i] = vi < nv ? q : sl[i];
        }
    }
}

// Gated kind: v = silu(v) * up = v * up / (1 + e^-v), with the hardware
// exponential and reciprocal (a few ulp; the staging then rounds to 15 bits
// per chunk); other kinds leave v unchanged.
template <int AK, int TOK, int TW>
__device__ __forceinline__ void gate_values(const S1Regs<AK, TOK, TW>& r, int t, int run, float (&v)[4]) {
    if constexpr (AK == kActGatedF32) {
        float up[4];
        run_values<AK, NQ_DTYPE_F32>(r.x2[t][run], NQ_DTYPE_F32, up);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            v[i] = v[i] * up[i] * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v[i] * -1.4426950408889634f));
    }
}

// Attention kinds: the lane's eight columns of the attention output, merged
// from the partials of the cache blocks up to the token's position, the order
// of k_attention_merge's one round: M = max m_s, then sum_s acc_s e^(m_s - M)
// over sum_s l_s e^(m_s - M). Blocks past the position are selected out (their
// slots may hold anything); a position outside the cache gives zeros.
template <int AK, int TOK, int TW>
__device__ __forceinline__ void attn_merge(const S1Regs<AK, TOK, TW>& r, const Lin& a, float (&mv)[2][4]) {
    constexpr int NB = attn_parts<AK>();
    const int64_t pos = r.at.pos;
    const bool in_range = pos >= 0 && pos < a.attn_max_positions;  // uniform
    // Every slot in block order, block s weighted by sum_s * exp(m_s - m): the
    // slots past the position hold the neutral partial, whose weight is
    // 0 * exp(-inf - m) = 0, so they add nothing.
    const auto mx = [&](int s) __attribute__((always_inline)) {
        if constexpr (attn_paired<AK>()) return __uint_as_float(s & 1 ? r.at.mlp[s / 2].z : r.at.mlp[s / 2].x);
        else return __uint_as_float(r.at.ml[s].x);
    };
    const auto sm = [&](int s) __attribute__((always_inline)) {
        if constexpr (attn_paired<AK>()) return __uint_as_float(s & 1 ? r.at.mlp[s / 2].w : r.at.mlp[s / 2].y);
        else return __uint_as_float(r.at.ml[s].y);
    };
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NB; ++s) m = fmaxf(m, mx(s));
    float l = 0.0f, acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int s = 0; s < NB; ++s) {
        const float wgt = sm(s) * nq::merge_exp(mx(s) - m);
        l += wgt;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t pair = r.at.out[s][j];
            const float lo = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(pair & 0xffffu)));
            const float hi = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(pair >> 16)));
            acc[2 * j] = fmaf(lo, wgt, acc[2 * j]);
            acc[2 * j + 1] = fmaf(hi, wgt, acc[2 * j + 1]);
        }
    }
    // One reciprocal for the lane's eight columns (eight divisions are about
    // ten instructions each).
    const float inv = 1.0f / l;
#pragma unroll
    for (int i = 0; i < 8; ++i) mv[i >> 2][i & 3] = in_range ? acc[i] * inv : 0.0f;
}

// One run's values of token t: the activations as read (with the gated kind's
// product), or the attention kinds' merged values.
template <int AK, int TOK, int TW>
__device__ __forceinline__ void act_run(const S1Regs<AK, TOK, TW>& r, const Lin& a, int t, int run,
                                        const float (&mv)[2][4], float (&v)[4]) {
    if constexpr (attn_kind<AK>()) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = mv[run][i];
    } else {
        run_values<AK, act_dtype<AK>()>(r.x[t][run], a.x_dtype, v);
        gate_values<AK, TOK, TW>(r, t, run, v);
    }
}

// Exponent a stage-1 epilogue writes for a token whose activations hold a
// NaN or an infinity: stage 2 then stores NaN for every output of that token,
// as the reference's fp32 forward yields (a non-finite activation reaches
// every rank value with both signs; reference.py:208-217).
constexpr int kPoisonExp = 0x7fffffff;

// Stage tokens [t_base, t_base + TPB) of chunk c into this wave's operand area
// (four digit rows per token) and return each token's exponent E and the
// chunk's Σ |a| (uniform values; not finite when a staged value is not).
//
// MFMA m receives w = rint(a * 2^(E + 7 - m)) (m = 7: w = -rint(a * 2^E)), so
// every product with its B bytes {0, 2^m} (m = 7: {0, -128}) is b times a
// multiple of 2^-(E+7) and the eight MFMAs of a chunk share one accumulator.
// |a * 2^E| < 2^23 gives |w| < 2^30, rounded once (halves up) from the
// exact product, as four signed base-256 digits: digit j is the low byte of
// w_j with w_0 = w, w_{j+1} = (w_j + 128) >> 8, i.e. byte j of w, w + 0x80,
// w + 0x8080 and w + 0x808080. Byte j of w + 0x808080 is digit j with its top
// bit flipped for j < 3 (the +0x80 at byte j carries into byte j + 1 exactly
// as digit j + 1 needs), so the bytes of (w + 0x808080) ^ 0x808080 are the
// four digits: one add and one xor per value, then a byte transpose of four
// values. Every value keeps 24 bits relative to the chunk's largest.
template <int AK, int TOK, int TW, int TPB>
__device__ __forceinline__ void stage_block(const S1Regs<AK, TOK, TW>& r, const Lin& a, int c, int t_base,
                                            char* __restrict__ ops, int lane, int (&expo)[TPB], float (&csum)[TPB]) {
    const int m = lane >> 3, d = (lane >> 1) & 3, h = lane & 1;
    const int k0 = stage_col0(c, lane);
    const int in = static_cast<int>(a.in);
    // Column k0 + 4 * run + i is inside the row when 4 * run + i is below lim.
    const int left = in - k0;
    const int lim = left > 8 ? 8 : (left < 0 ? 0 : left);
    const bool full_chunk = (c + 1) * kChunkCols <= in;  // uniform
    float sc[2][4];
    run_values<AK, col_scale_dtype<AK>()>(r.s[0], a.scale_dtype, sc[0]);
    run_values<AK, col_scale_dtype<AK>()>(r.s[1], a.scale_dtype, sc[1]);
    float mv[2][4];  // attention kinds: the merged values (one token)
    if constexpr (attn_kind<AK>()) attn_merge<AK, TOK, TW>(r, a, mv);
    // A block whose token slots are all in the call stages them in one
    // straight-line loop; one with slots past the call's tokens (uniform)
    // stages only those in it: the other slots' digit rows keep what the
    // operand area held, and every result of those rows is discarded (the
    // epilogues store tokens < a.tokens only).
    const auto stage_tokens = [&](auto skip) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < TPB; ++u) {
            const int t = t_base + u;
            if (decltype(skip)::value && t >= a.tokens) {
                expo[u] = 0;
                csum[u] = 0.0f;
                continue;
            }
            float v[2][4];
            float mx = 0.0f, sa = 0.0f;
            if (full_chunk) {  // uniform: every value is inside
#pragma unroll
                for (int run = 0; run < 2; ++run) {
                    act_run<AK, TOK, TW>(r, a, t, run, mv, v[run]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[run][i] *= sc[run][i];
                        mx = fmaxf(mx, fabsf(v[run][i]));
                        sa += fabsf(v[run][i]);
                    }
                }
            } else {
#pragma unroll
                for (int run = 0; run < 2; ++run) {
                    act_run<AK, TOK, TW>(r, a, t, run, mv, v[run]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool ok = 4 * run + i < lim;
                        v[run][i] = ok ? v[run][i] * sc[run][i] : 0.0f;
                        mx = fmaxf(mx, fabsf(v[run][i]));
                        sa += fabsf(v[run][i]);
                    }
                }
            }
            // fmaxf drops NaN, the sum does not: a NaN or an infinity makes the
            // chunk sum, and so the token's bound in the epilogue, not finite.
            const float wmx = wave_max(mx);
            csum[u] = wave_sum(sa);
            const int e = range_exponent(wmx, 22);
            const float sm = m < 7 ? exp2i(e + 7 - m) : -exp2i(e);
            uint32_t dig[4][2];
#pragma unroll
            for (int run = 0; run < 2; ++run) {
                uint32_t u[4], t[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    u[i] = (static_cast<uint32_t>(round_to_int(v[run][i] * sm)) + 0x808080u) ^ 0x808080u;
                transpose_bytes(u[0], u[1], u[2], u[3], t);
#pragma unroll
                for (int j = 0; j < 4; ++j) dig[j][run] = t[j];
            }
            expo[u] = e;
#pragma unroll
            for (int digit = 0; digit < 4; ++digit) {
                const int row = 4 * u + digit;
#pragma unroll
                for (int run = 0; run < 2; ++run)
                    *reinterpret_cast<uint32_t*>(ops + ((m * Ops<TPB>::kRows + row) * 4 + 2 * h + run) * 16 + 4 * d) =
                        dig[digit][run];
            }
        }
    };
    if (TPB == 1 || t_base + TPB <= a.tokens) stage_tokens(std::false_type{});
    else stage_tokens(std::true_type{});
}

// S = 2^7 Σ x_q of one chunk and operand block: eight MFMAs against 0x01 << m.
__device__ __forceinline__ v4i ones_mfma(const v4i (&A)[8]) {
    v4i s0 = v4i{0, 0, 0, 0}, s1 = v4i{0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 8; m += 2) {
        const int o0 = static_cast<int>(0x01010101u << m), o1 = static_cast<int>(0x01010101u << (m + 1));
        s0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], v4i{o0, o0, o0, o0}, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m + 1], v4i{o1, o1, o1, o1}, s1, 0, 0, 0);
    }
    return s0 + s1;
}

// The eight sign MFMAs of one (chunk, tile, operand block) and the exact
// conversion to the chunk's fp32 partial; words d >= dw (a partial chunk)
// count as zero. NDIG digit rows per token; lane 16*t' + n returns token t' of
// the block, row n; scale is 2^(-e-7) for that token's exponent e.
template <int NDIG>
__device__ __forceinline__ float tile_partial(const v4i (&A)[8], const v4i& S, v4u w, int dw, float scale) {
    // A partial last chunk: words past dw belong to other lanes (uniform masks).
    w[1] &= dw > 1 ? ~0u : 0u;
    w[2] &= dw > 2 ? ~0u : 0u;
    w[3] &= dw > 3 ? ~0u : 0u;
    v4i t0 = v4i{0, 0, 0, 0}, t1 = v4i{0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 8; m += 2) {
        const uint32_t k0 = 0x01010101u << m, k1 = 0x01010101u << (m + 1);
        const v4i b0 = v4i{static_cast<int>(w[0] & k0), static_cast<int>(w[1] & k0), static_cast<int>(w[2] & k0),
                           static_cast<int>(w[3] & k0)};
        const v4i b1 = v4i{static_cast<int>(w[0] & k1), static_cast<int>(w[1] & k1), static_cast<int>(w[2] & k1),
                           static_cast<int>(w[3] & k1)};
        t0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], b0, t0, 0, 0, 0);
        t1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m + 1], b1, t1, 0, 0, 0);
    }
    const v4i diff = S - 2 * (t0 + t1);
    float v = static_cast<float>(diff[0]) + 256.0f * static_cast<float>(diff[1]) +
              65536.0f * static_cast<float>(diff[2]);
    if (NDIG == 4) v += 16777216.0f * static_cast<float>(diff[3]);
    return v * scale;
}

// tile_partial for TB operand blocks (four tokens each) against one tile's
// words: each sign-expansion AND feeds the blocks' MFMAs, so a block costs
// eight MFMAs and its conversion. Every block is computed (a uniform guard
// per block costs the compiler's register copies more than an unused
// block's MFMAs); the caller stores the live ones. Integer results, and so
// the partials, equal tile_partial's.
template <int NDIG, int TB>
__device__ __forceinline__ void tile_partials(const v4i (&A)[TB][8], const v4i (&S)[TB], v4u w, int dw,
                                              const float (&scale)[TB], float (&out)[TB]) {
    w[1] &= dw > 1 ? ~0u : 0u;
    w[2] &= dw > 2 ? ~0u : 0u;
    w[3] &= dw > 3 ? ~0u : 0u;
    v4i t0[TB], t1[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) t0[tb] = t1[tb] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < 8; m += 2) {
        const uint32_t k0 = 0x01010101u << m, k1 = 0x01010101u << (m + 1);
        const v4i b0 = v4i{static_cast<int>(w[0] & k0), static_cast<int>(w[1] & k0), static_cast<int>(w[2] & k0),
                           static_cast<int>(w[3] & k0)};
        const v4i b1 = v4i{static_cast<int>(w[0] & k1), static_cast<int>(w[1] & k1), static_cast<int>(w[2] & k1),
                           static_cast<int>(w[3] & k1)};
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            t0[tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[tb][m], b0, t0[tb], 0, 0, 0);
            t1[tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[tb][m + 1], b1, t1[tb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const v4i diff = S[tb] - 2 * (t0[tb] + t1[tb]);
        float v = static_cast<float>(diff[0]) + 256.0f * static_cast<float>(diff[1]) +
                  65536.0f * static_cast<float>(diff[2]);
        if (NDIG == 4) v += 16777216.0f * static_cast<float>(diff[3]);
        out[tb] = v * scale[tb];
    }
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
// the workgroup's operand stores are complete (the caller waits and barriers first).
__device__ __forceinline__ void signal_ready(const Lin& a, int64_t t0, int tw) {
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
// stage-1 tile of this launch has signalled. Returns true (in every thread)
// when the bounded wait gave up: the stage-1 operands may then be stale, so
// the caller stores NaN for the workgroup's outputs, and the sticky error
// flag in the header records the event for the host.
__device__ __forceinline__ bool wait_ready(const Lin& a, int64_t t0, int tw, int64_t wg, bool dead) {
    __shared__ int gave_up;
    if (threadIdx.x == 0) gave_up = 0;
    if (threadIdx.x == 0 && !dead) {
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
        const uint32_t limit = a.header[line_word(kMiscLine) + kMiscSpin];
        uint32_t spins = 0;
        while (static_cast<int32_t>(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
            if (++spins > limit) {
                hdr_store(a.header, line_word(kMiscLine) + kMiscError, 1u);
                gave_up = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    return gave_up != 0;
}

// Chunks of one pass: chunk c_j = base + wave + j * nw; a dead chunk (past nc)
// loads chunk nc - 1 and skips its arithmetic.
template <int KC>
struct PassChunks {
    int c[KC];
    bool live[KC];
};

template <int KC>
__device__ __forceinline__ PassChunks<KC> pass_chunks(int base, int wave, int nw, int nc) {
    PassChunks<KC> p;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        const int c = base + wave + j * nw;
        p.live[j] = c < nc;
        p.c[j] = c < nc ? c : nc - 1;
    }
    return p;
}

// Output index idx of a workgroup: (tile tt, token t, row n).
struct OutIdx {
    int tt, t, n;
};

// One token per block (TPB = 1) means one token per launch: no division.
template <int TPB>
__device__ __forceinline__ OutIdx out_index(int idx, int tokens) {
    OutIdx o;
    o.tt = TPB == 1 ? idx >> 4 : idx / (tokens * kTileRows);
    o.t = TPB == 1 ? 0 : (idx / kTileRows) % tokens;
    o.n = idx & 15;
    return o;
}

// Partial-sum slot of (chunk c, tile tt, token t, row n) in the LDS array red.
template <int TPB, int TB, int TW>
__device__ __forceinline__ int red_index(int c, int tt, int t, int n) {
    const int tb = TPB == 1 ? 0 : t / TPB;
    const int rl = TPB == 1 ? n : 16 * (t % TPB) + n;
    return ((c * TW + tt) * TB + tb) * 64 + rl;
}

// Stage-1 epilogue store of one rank value: x_q = rint(v * 2^e) as four digits
// of w = x_q * mult into the stage-2 operand buffer (agent scope when fused).
template <int TPB, int TB, bool FUSED>
__device__ __forceinline__ void store_lmq(uint8_t* lmq, int r, int t, float v, int e) {
    const int c = r >> 9;
    const int col = r & 511;
    const int d = col >> 7, m = (col >> 4) & 7, g = (col >> 2) & 3, b = col & 3;
    const int tb = TPB == 1 ? 0 : t / TPB, u = TPB == 1 ? 0 : t % TPB;
    const int q = static_cast<int>(__builtin_rintf(v * exp2i(e)));
    int w = q * (m < 7 ? (1 << (7 - m)) : -1);
#pragma unroll
    for (int digit = 0; digit < 4; ++digit) {
        uint8_t* p = lmq + lmq_offset<TPB, TB>(c, tb, m, 4 * u + digit, g) + 4 * d + b;
        const uint8_t byte = static_cast<uint8_t>(w & 0xff);
        if (FUSED) __hip_atomic_store(p, byte, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else *p = byte;
        w = next_digit_word(w);
    }
}

// One stage-1 workgroup: tiles [t0, t0 + TW) of linear `a`. TPB tokens per
// block and TB blocks cover the launch's tokens; KC chunks per wave per pass.
template <int AK, int TPB, int TB, int TW, int KC, bool FUSED>
__device__ __forceinline__ void stage1_wg(const Lin& a, int wg_in, char* __restrict__ lds) {
    constexpr int TOK = TPB * TB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int nw = a.nw1;
    const int nthreads = nw * 64;  // the workgroup size (blockDim.x is a vector load of a hidden argument)
    const int tokens = a.tokens;
    // Workgroups past this member's count compute the last workgroup's tiles
    // and store nothing.
    const int nwg = static_cast<int>(a.nwg1);
    const bool dead = wg_in >= nwg;
    const int wg = dead ? nwg - 1 : wg_in;
    const int t0 = wg * TW;
    const int nt = static_cast<int>(a.g1.nt), nb = static_cast<int>(a.g1.nb), nc = static_cast<int>(a.g1.nc);
    const int rank = static_cast<int>(a.rank);
    char* const ops = lds + wave * Ops<TPB>::kBytes;
    float* const red = reinterpret_cast<float*>(lds + nw * Ops<TPB>::kBytes);
    float* const cmx = red + nc * TW * TB * 64;  // [nc][TOK] chunk Σ |x s_in|

    const int outs = TW * tokens * kTileRows;
    const OutIdx f = out_index<TPB>(threadIdx.x < outs ? threadIdx.x : 0, tokens);
    const int fr = (t0 + f.tt) * kTileRows + f.n;
    RawElem rs0;
    float maxsm;
    // Normed kind: the producer's per-tile sums of squares of x (up to
    // kSlotVecs * 256 of them), loaded ahead of the first pass's loads.
    v4f slots[kSlotVecs];
    float rs = 1.0f;  // 1 / RMS(x)

    // One pass: KC chunks per wave. The first pass is a separate copy ahead of
    // the loop (so its loads are not held behind waits for registers a
    // previous iteration could still be loading) and issues the epilogue
    // operands right after its own loads.
    const auto pass = [&](const int base, const bool first) __attribute__((always_inline)) {
        const PassChunks<KC> pc = pass_chunks<KC>(base, wave, nw, nc);
        S1Regs<AK, TOK, TW> r[KC];
        if constexpr (AK == kActNormF32) {
            if (first) load_slots(slots, a.slots_in, a.nslots, lane);
        }
        // Activations first, sign words second: the staging math waits only
        // for the activations, the MFMAs for the words.
#pragma unroll
        for (int j = 0; j < KC; ++j) load_s1_acts(r[j], a, pc.c[j], lane);
#pragma unroll
        for (int j = 0; j < KC; ++j) load_words(r[j].w, a.v_tiles, nt, nb, t0, pc.c[j], lane);
        if constexpr (AK == kActNormF32) {
            if (first) {
                // Issued before the activations, so waiting for them here costs
                // nothing the staging would not wait for anyway.
#pragma unroll
                for (int i = 0; i < kSlotVecs; ++i) asm volatile("" : "+v"(slots[i]));
                float part = 0.0f;
#pragma unroll
                for (int i = 0; i < kSlotVecs; ++i) part += (slots[i].x + slots[i].y) + (slots[i].z + slots[i].w);
                const float total = wave_sum(part);
                rs = 1.0f / sqrtf(__fadd_rn(total / static_cast<float>(a.in), a.eps));  // no fma contraction
            }
        }
        if (first) {
            // Vector kinds have fp16 scales: one 16-bit load (the generic kind
            // loads both halves); the bound sits at a uniform address.
            const int frc = fr < rank ? fr : rank - 1;
            rs0 = AK == kActGeneric ? load_elem(a.s_mid, a.scale_dtype, frc) : load_half(a.s_mid, frc);
            maxsm = __uint_as_float(scalar_load(a.header + line_word(kMiscLine) + kMiscMaxMid));
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the pass is issued before any use
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            if (!pc.live[j]) continue;  // uniform
            const int c = pc.c[j];
            const int dw = chunk_words32(nb, c);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                if (tb * TPB >= tokens) break;
                int expo[TPB];
                float cm[TPB];
                stage_block<AK, TOK, TW, TPB>(r[j], a, c, tb * TPB, ops, lane, expo, cm);
                wave_lds_sync();
                // The staging waits only for the activations: the sign words
                // are redefined here, so no use of them moves into it.
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) asm volatile("" : "+v"(r[j].w[tt]));
                v4i A[8];
                const int row = TPB == 1 ? (lane & 3) : (lane & 15);
#pragma unroll
                for (int m = 0; m < 8; ++m)
                    A[m] = *reinterpret_cast<const v4i*>(ops + ((m * Ops<TPB>::kRows + row) * 4 + (lane >> 4)) * 16);
                const v4i S = ones_mfma(A);
                int e = expo[0];
#pragma unroll
                for (int u = 1; u < TPB; ++u) e = (lane >> 4) == u ? expo[u] : e;
                const float sc = exp2i(-e - 7);
#pragma unroll
                for (int tt = 0; tt < TW; ++tt)
                    red[((c * TW + tt) * TB + tb) * 64 + lane] = tile_partial<4>(A, S, r[j].w[tt], dw, sc);
                if (lane == 0) {
#pragma unroll
                    for (int u = 0; u < TPB; ++u) cmx[c * TOK + tb * TPB + u] = cm[u];
                }
                wave_lds_sync();  // the next block rewrites this wave's operand area
            }
        }
    };
    const int step = nw * KC;
    pass(0, true);
    for (int base = step; base < nc; base += step) pass(base, false);
    __syncthreads();

    if (dead) return;  // uniform, after the workgroup's only barrier

    // Epilogue: lm = s_mid * Σ_chunks partial, written as stage-2 operands with
    // the per-token exponent of the bound |lm| <= max|s_mid| * Σ_i |x_i s_in_i|
    // (times 1/RMS for the normed kind).
    for (int idx = threadIdx.x; idx < outs; idx += nthreads) {
        const OutIdx o = out_index<TPB>(idx, tokens);
        const int row = (t0 + o.tt) * kTileRows + o.n;
        if (t0 + o.tt >= nt) continue;
        float sum = 0.0f, bound = 0.0f;
        for (int c = 0; c < nc; ++c) {
            sum += red[red_index<TPB, TB, TW>(c, o.tt, o.t, o.n)];
            bound += cmx[c * TOK + o.t];
        }
        // Every workgroup sums the same chunk sums in the same order, so all
        // agree on the exponent and on a poisoned (non-finite) token.
        const bool poison = !(bound <= 3.402823466e38f);
        const int e = poison ? 0 : range_exponent(bound * rs * maxsm, 21);
        float v = 0.0f;
        if (row < rank && !poison)
            v = sum * elem_value(idx == threadIdx.x ? rs0 : load_elem(a.s_mid, a.scale_dtype, row), a.scale_dtype) * rs;
        store_lmq<TPB, TB, FUSED>(a.lmq, row, o.t, v, e);
        if (wg == 0 && o.tt == 0 && o.n == 0) {
            const int le = poison ? kPoisonExp : e;
            if (FUSED) __hip_atomic_store(a.lme + o.t, le, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else a.lme[o.t] = le;
        }
    }
    // The last workgroup zeroes the operand columns past its last tile up to
    // the end of the last chunk (every stage-2 ones-MFMA reads them).
    if (t0 + TW >= nt) {
        const int from = nt * kTileRows, to = static_cast<int>(a.g2.nc) * kChunkCols;
        const int n = (to - from) * tokens;
        for (int i = threadIdx.x; i < n; i += nthreads)
            store_lmq<TPB, TB, FUSED>(a.lmq, from + i / tokens, i % tokens, 0.0f, 0);
    }
    if (FUSED) {
        // The operands went out at agent scope; the wait makes them complete
        // before the signal.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        signal_ready(a, t0, TW);
    }
}

// ---------------------------------------------------------------------------
// Several tokens (2-16), split launch: stage 0 + stage 1 from operands.
//
// With several tokens the staging of x * s_in (about 110 VALU instructions per
// token, chunk and wave) is repeated by every stage-1 workgroup, one per tile
// group, and a stage-1 wave's A operands grow to 8 KB per block of four
// tokens per chunk against 1 KB of sign words per tile. Stage 0 therefore
// stages every (chunk, token block) once per call, with stage_block's
// arithmetic, into xq (the lmq layout with TB blocks) and records every
// (chunk, token)'s exponent (xe) and Σ |x s_in| (xm). Stage 1 then loads its
// A operands like stage 2 and takes TW
// tiles per wave, one sign expansion feeding every token block
// (tile_partials). The digits, exponents, integer partials and their
// chunk-order sums are those of stage1_wg, so the results are bit-identical.
// ---------------------------------------------------------------------------

// Element size of x for kind AK (the generic kind: its runtime dtype).
template <int AK>
__device__ __forceinline__ int act_elem_bytes(int x_dtype) {
    if constexpr (AK == kActGeneric) return x_dtype == NQ_DTYPE_F32 ? 4 : 2;
    else return act_dtype<AK>() == NQ_DTYPE_F32 ? 4 : 2;
}

// Stage 0 of (chunk c, token block tb) in a layout of tbl blocks: one wave.
template <int AK>
__device__ __forceinline__ void stage0_wave(const Lin& a, int c, int tb, int tbl, int lane) {
    constexpr int TPB = 4;
    Lin b = a;
    b.x = static_cast<const char*>(a.x) +
          static_cast<int64_t>(tb) * TPB * a.in * act_elem_bytes<AK>(a.x_dtype);
    b.tokens = a.tokens - TPB * tb < TPB ? a.tokens - TPB * tb : TPB;
    S1Regs<AK, TPB, 1> r;
    load_s1_acts<AK, TPB, 1>(r, b, c, lane);
    const MultiWs ws = multi_ws(a.lme, a.g1, a.tokens);
    char* const ops = reinterpret_cast<char*>(ws.xq) + (c * tbl + tb) * Ops<TPB>::kBytes;
    int expo[TPB];
    float cm[TPB];
    stage_block<AK, TPB, 1, TPB>(r, b, c, 0, ops, lane, expo, cm);
    int e = expo[0];
    float mx = cm[0];
#pragma unroll
    for (int u = 1; u < TPB; ++u) {
        e = lane == u ? expo[u] : e;
        mx = lane == u ? cm[u] : mx;
    }
    if (lane < TPB) {
        ws.xe[c * kMaxTokens + TPB * tb + lane] = e;
        ws.xm[c * kMaxTokens + TPB * tb + lane] = mx;
    }
}

// Token blocks per wave and wave groups per chunk of the several-token
// kernels: a wave holds the A operands of at most two token blocks (64
// VGPRs per chunk), so with four blocks two waves share each chunk, wave w
// taking blocks 2 (w % 2) and 2 (w % 2) + 1 of chunk slot w / 2.
template <int TB>
constexpr int blocks_per_wave() { return TB > 2 ? 2 : TB; }
template <int TB>
constexpr int wave_groups() { return TB / blocks_per_wave<TB>(); }

// One stage-1 workgroup of the several-token path: tiles [t0, t0 + TW) of
// linear `a`, operands from xq; TB blocks of four tokens in the layout.
template <int TB, int TW, int KC>
__device__ __forceinline__ void stage1m_wg(const Lin& a, int wg_in, char* __restrict__ lds) {
    constexpr int TPB = 4;
    constexpr int TBW = blocks_per_wave<TB>(), NG = wave_groups<TB>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int grp = wave % NG, slot = wave / NG;
    const int nw = a.nw1;
    const int nslots = nw / NG;
    const int nthreads = nw * 64;
    const int tokens = a.tokens;
    const int nblk = (tokens + TPB - 1) / TPB;
    const int nwg = static_cast<int>(a.nwg1);
    const bool dead = wg_in >= nwg;  // computes the last workgroup's tiles, stores nothing
    const int wg = dead ? nwg - 1 : wg_in;
    const int t0 = wg * TW;
    const int nt = static_cast<int>(a.g1.nt), nb = static_cast<int>(a.g1.nb), nc = static_cast<int>(a.g1.nc);
    const int rank = static_cast<int>(a.rank);
    float* const red = reinterpret_cast<float*>(lds);
    float* const cmx = red + nc * TW * TB * 64;  // [nc][kMaxTokens] Σ |x s_in|
    const int nxm = nc * kMaxTokens;
    const MultiWs ws = multi_ws(a.lme, a.g1, tokens);

    const int outs = TW * tokens * kTileRows;
    const OutIdx f = out_index<TPB>(threadIdx.x < outs ? threadIdx.x : 0, tokens);
    const int fr = (t0 + f.tt) * kTileRows + f.n;
    RawElem rs0;
    float maxsm = 0.0f, xmv = 0.0f;

    // This wave's token blocks are grp * TBW + i, i < gblk.
    const int gblk0 = nblk - grp * TBW;
    const int gblk = gblk0 < 0 ? 0 : (gblk0 > TBW ? TBW : gblk0);
    const auto pass = [&](const int base, const bool first) __attribute__((always_inline)) {
        const PassChunks<KC> pc = pass_chunks<KC>(base, slot, nslots, nc);
        S2Regs<TBW, TW> r[KC];
        int e[KC][TBW];
#pragma unroll
        for (int j = 0; j < KC; ++j) load_words(r[j].w, a.v_tiles, nt, nb, t0, pc.c[j], lane);
        // Every block of the wave's group is loaded (xq holds TB blocks per
        // chunk); blocks past the last token are computed and not stored.
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
            for (int i = 0; i < TBW; ++i) {
                const int tb = grp * TBW + i;
#pragma unroll
                for (int m = 0; m < 8; ++m)
                    r[j].a[i][m] = *reinterpret_cast<const v4i*>(
                        ws.xq + lmq_offset<TPB, TB>(pc.c[j], tb, m, lane & 15, lane >> 4));
                e[j][i] = ws.xe[pc.c[j] * kMaxTokens + TPB * tb + (lane >> 4)];
            }
        if (first) {
            const int frc = fr < rank ? fr : rank - 1;
            rs0 = load_elem(a.s_mid, a.scale_dtype, frc);
            maxsm = __uint_as_float(scalar_load(a.header + line_word(kMiscLine) + kMiscMaxMid));
            xmv = ws.xm[static_cast<int>(threadIdx.x) < nxm ? static_cast<int>(threadIdx.x) : 0];
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the pass is issued before any use
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            if (!pc.live[j]) continue;  // uniform
            const int c = pc.c[j];
            const int dw = chunk_words32(nb, c);
            v4i S[TBW];
            float sc[TBW];
#pragma unroll
            for (int i = 0; i < TBW; ++i) {
                S[i] = ones_mfma(r[j].a[i]);
                sc[i] = exp2i(-e[j][i] - 7);
            }
#pragma unroll
            for (int tt = 0; tt < TW; ++tt) {
                float part[TBW];
                tile_partials<4, TBW>(r[j].a, S, r[j].w[tt], dw, sc, part);
#pragma unroll
                for (int i = 0; i < TBW; ++i)
                    if (i < gblk) red[((c * TW + tt) * TB + grp * TBW + i) * 64 + lane] = part[i];
            }
        }
    };
    const int step = nslots * KC;
    pass(0, true);
    for (int base = step; base < nc; base += step) pass(base, false);
    if (static_cast<int>(threadIdx.x) < nxm) cmx[threadIdx.x] = xmv;
    for (int i = static_cast<int>(threadIdx.x) + nthreads; i < nxm; i += nthreads) cmx[i] = ws.xm[i];
    __syncthreads();

    if (dead) return;  // uniform, after the workgroup's only barrier

    // Epilogue of stage1_wg (no input norm): lm = s_mid * Σ_chunks partial as
    // stage-2 operands with the per-token exponent of max|s_mid| * Σ |x s_in|.
    for (int idx = threadIdx.x; idx < outs; idx += nthreads) {
        const OutIdx o = out_index<TPB>(idx, tokens);
        const int row = (t0 + o.tt) * kTileRows + o.n;
        if (t0 + o.tt >= nt) continue;
        float sum = 0.0f, bound = 0.0f;
        for (int c = 0; c < nc; ++c) {
            sum += red[red_index<TPB, TB, TW>(c, o.tt, o.t, o.n)];
            bound += cmx[c * kMaxTokens + o.t];
        }
        const bool poison = !(bound <= 3.402823466e38f);
        const int e = poison ? 0 : range_exponent(bound * maxsm, 21);
        float v = 0.0f;
        if (row < rank && !poison)
            v = sum * elem_value(idx == static_cast<int>(threadIdx.x) ? rs0 : load_elem(a.s_mid, a.scale_dtype, row),
                                 a.scale_dtype);
        store_lmq<TPB, TB, false>(a.lmq, row, o.t, v, e);
        if (wg == 0 && o.tt == 0 && o.n == 0) a.lme[o.t] = poison ? kPoisonExp : e;
    }
    if (t0 + TW >= nt) {
        const int from = nt * kTileRows, to = static_cast<int>(a.g2.nc) * kChunkCols;
        const int n = (to - from) * tokens;
        for (int i = threadIdx.x; i < n; i += nthreads)
            store_lmq<TPB, TB, false>(a.lmq, from + i / tokens, i % tokens, 0.0f, 0);
    }
}

// Salient columns in the stage-2 epilogue. Up to kSalMax columns, the
// workgroup's rows of W_sal (16 TW rows x k) and the gathered x[t, idx_k] *
// scale_k of every token are loaded in the first pass, with the other
// epilogue operands, and parked in LDS after the partial sums; each output
// then adds Σ_k W_sal[row, k] * xs[t, k] from LDS. More columns take a loop of
// element loads. Each thread loads at most kSalLoads weights in the first pass.
constexpr int kSalMax = 96;
constexpr int kSalLoads = 4;

// LDS bytes of the staged salient operands (0 when the loop is used).
__host__ __device__ constexpr int sal_lds_bytes(int64_t ks, int tw, int tokens) {
    return ks > 0 && ks <= kSalMax ? static_cast<int>((16 * tw + tokens) * ks * 4) : 0;
}

// Raw bits of element i of an F32 / F16 / BF16 / I8 buffer (one load of the
// element's size) and their value.
__device__ __forceinline__ uint32_t load_bits(const void* __restrict__ p, int dtype, int i) {
    if (dtype == NQ_DTYPE_F32) return static_cast<const uint32_t*>(p)[i];
    if (dtype == NQ_DTYPE_I8) return static_cast<const uint8_t*>(p)[i];
    return static_cast<const uint16_t*>(p)[i];
}

__device__ __forceinline__ float bits_value(uint32_t b, int dtype) {
    if (dtype == NQ_DTYPE_F32) return __uint_as_float(b);
    if (dtype == NQ_DTYPE_I8) return static_cast<float>(static_cast<int8_t>(b & 0xffu));
    if (dtype == NQ_DTYPE_BF16) return __uint_as_float(b << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}

// One stage-2 workgroup: output tiles [t0, t0 + TW) of linear `a`. PAIR: the
// same tiles of `a` (gate) and `b` (up, same geometry, no sidecars or bias),
// one token, and the output silu(y_a) * y_b stored to a.y (the decoder's
// SiLU-gated MLP product), so the down projection reads one plain input.
template <int TPB, int TB, int TW, int KC, bool FUSED, bool PAIR = false>
__device__ __forceinline__ void stage2_wg(const Lin& a, int wg_in, char* __restrict__ lds,
                                          const Lin* pair = nullptr) {
    // Split launch with four token blocks: two waves per chunk slot
    // (blocks_per_wave); one token or the fused launch: one wave per slot.
    constexpr int NG = (TPB == 4 && !FUSED) ? wave_groups<TB>() : 1;
    constexpr int TBW = TB / NG;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int grp = wave % NG, slot = wave / NG;
    const int nw = a.nw2;
    const int nslots = nw / NG;
    const int nthreads = nw * 64;  // the workgroup size (blockDim.x is a vector load of a hidden argument)
    const int tokens = a.tokens;
    const int nblk = (tokens + TPB - 1) / TPB;
    // This wave's token blocks are grp * TBW + i, i < gblk.
    const int gblk0 = nblk - grp * TBW;
    const int gblk = gblk0 < 0 ? 0 : (gblk0 > TBW ? TBW : gblk0);
    const int nwg = static_cast<int>(a.nwg2);
    const bool dead = wg_in >= nwg;  // computes the last workgroup's tiles, stores nothing
    const int wg = dead ? nwg - 1 : wg_in;
    const int t0 = wg * TW;
    const int nt = static_cast<int>(a.g2.nt), nb = static_cast<int>(a.g2.nb), nc = static_cast<int>(a.g2.nc);
    const int out = static_cast<int>(a.out), in = static_cast<int>(a.in);
    float* const red = reinterpret_cast<float*>(lds);
    // PAIR: the second member's partial sums follow the first's.
    float* const red_b = red + nc * TW * TB * 64;
    char* const after_red = lds + (PAIR ? 2 : 1) * nc * TW * TB * 64 * 4;
    // One token: this wave's operand spread areas (KC of them) after the partial sums.
    char* const spread = after_red + wave * KC * kS2SpreadBytes;
    // Staged salient operands after the spread areas: W rows [16 TW][ks], then xs [tokens][ks].
    const int ks = static_cast<int>(a.salient_count);
    const bool sal_lds = ks > 0 && ks <= kSalMax;  // uniform
    float* const salw = reinterpret_cast<float*>(after_red + (TPB == 1 ? nw * KC * kS2SpreadBytes : 0));
    float* const salx = salw + 16 * TW * ks;

    const int outs = TW * tokens * kTileRows;
    const OutIdx f = out_index<TPB>(threadIdx.x < outs ? threadIdx.x : 0, tokens);
    const int fr0 = (t0 + f.tt) * kTileRows + f.n;
    const int fr = fr0 < out ? fr0 : out - 1;
    RawElem rs0, bias0, rs1;
    float res0 = 0.0f;   // residual epilogue: residual[fr], loaded with the first pass
    bool stale = false;  // fused launch: the wait for stage 1 gave up
    // First-pass salient loads: weights i = threadIdx.x + n * nthreads of the
    // workgroup's block, and for threadIdx.x < tokens * ks one gathered x and scale.
    uint32_t wbits[kSalLoads];
    RawElem sx, ssc;
    const int wtotal = 16 * TW * ks;           // weights parked per workgroup
    const int wlimit = out * ks - 1;           // last weight element of the buffer
    const int wbase = t0 * kTileRows * ks;     // first weight element of the workgroup

    // One pass; the first is peeled off the loop and issues the epilogue
    // operands after its own loads (see stage1_wg).
    // A pass is split into its loads and its arithmetic so that a paired
    // workgroup issues both members' loads before either waits.
    struct PassRegs {
        PassChunks<KC> pc;
        S2Regs<TBW, TW> r[KC];
        int e[TBW];
    };
    const auto load_pass = [&](const Lin& m, PassRegs& ps, const int base, const bool first)
                               __attribute__((always_inline)) {
        ps.pc = pass_chunks<KC>(base, slot, nslots, nc);
#pragma unroll
        for (int j = 0; j < KC; ++j) load_words(ps.r[j].w, m.u_tiles, nt, nb, t0, ps.pc.c[j], lane);
        // The U words do not depend on stage 1; the fused launch waits for its
        // signal only now.
        if (FUSED && first) stale = wait_ready(m, t0, TW, wg, dead);
        if constexpr (TPB == 1) {
#pragma unroll
            for (int j = 0; j < KC; ++j) load_s2_ops<TPB, TB, TW>(ps.r[j], m, ps.pc.c[j], lane);
            ps.e[0] = m.lme[0];
        } else {
            // Every block of the wave's group is loaded (the operand buffer
            // holds TB blocks per chunk); blocks past the last token are
            // computed and not stored.
#pragma unroll
            for (int j = 0; j < KC; ++j)
#pragma unroll
                for (int i = 0; i < TBW; ++i)
#pragma unroll
                    for (int mm = 0; mm < 8; ++mm)
                        ps.r[j].a[i][mm] = *reinterpret_cast<const v4i*>(
                            m.lmq + lmq_offset<TPB, TB>(ps.pc.c[j], grp * TBW + i, mm, lane & 15, lane >> 4));
#pragma unroll
            for (int i = 0; i < TBW; ++i) {
                const int t = (grp * TBW + i) * TPB + (lane >> 4);
                ps.e[i] = m.lme[t < tokens ? t : tokens - 1];
            }
        }
        if (PAIR && first && &m != &a) rs1 = load_elem(m.s_out, m.scale_dtype, fr);
        if (first && &m == &a) {
            rs0 = load_elem(a.s_out, a.scale_dtype, fr);
            // No branch on the optional bias: without one, s_out is loaded instead and ignored.
            bias0 = load_elem(a.bias ? a.bias : a.s_out, a.bias ? a.bias_dtype : a.scale_dtype, fr);
            // Only this workgroup writes these rows, so the value read now is the
            // one the epilogue adds to (in the fused launch, read after the wait).
            if (TPB == 1 && a.residual != nullptr) res0 = a.residual[fr];
            if (sal_lds) {  // uniform
#pragma unroll
                for (int n = 0; n < kSalLoads; ++n) {
                    const int i = wbase + static_cast<int>(threadIdx.x) + n * nthreads;
                    wbits[n] = load_bits(a.salient_values, a.salient_dtype, i < wlimit ? i : wlimit);
                }
                const int j = static_cast<int>(threadIdx.x) < tokens * ks ? static_cast<int>(threadIdx.x) : 0;
                const int t = j / ks, k = j - (j / ks) * ks;
                sx = load_elem(a.x, a.x_dtype, t * in + a.salient_indices[k]);
                ssc = load_elem(a.salient_scales ? a.salient_scales : a.s_in, a.scale_dtype, k);  // s_in: ks <= in
            }
        }
    };
    const auto compute_pass = [&](PassRegs& ps, float* const redm) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            if (!ps.pc.live[j]) continue;  // uniform
            const int c = ps.pc.c[j];
            const int dw = chunk_words32(nb, c);
            // A poisoned token (non-finite activations) yields NaN partials.
            if constexpr (TPB == 1) {
                spread_s2_ops<TPB, TB, TW>(ps.r[j], spread + j * kS2SpreadBytes, lane);
                const v4i S = ones_mfma(ps.r[j].a[0]);
                const float sc = ps.e[0] == kPoisonExp ? __builtin_nanf("") : exp2i(-ps.e[0] - 7);
#pragma unroll
                for (int tt = 0; tt < TW; ++tt)
                    redm[(c * TW + tt) * 64 + lane] = tile_partial<4>(ps.r[j].a[0], S, ps.r[j].w[tt], dw, sc);
            } else {
                v4i S[TBW];
                float sc[TBW];
#pragma unroll
                for (int i = 0; i < TBW; ++i) {
                    S[i] = ones_mfma(ps.r[j].a[i]);
                    sc[i] = ps.e[i] == kPoisonExp ? __builtin_nanf("") : exp2i(-ps.e[i] - 7);
                }
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) {
                    float part[TBW];
                    tile_partials<4, TBW>(ps.r[j].a, S, ps.r[j].w[tt], dw, sc, part);
#pragma unroll
                    for (int i = 0; i < TBW; ++i)
                        if (i < gblk) redm[((c * TW + tt) * TB + grp * TBW + i) * 64 + lane] = part[i];
                }
            }
        }
    };
    const int step = nslots * KC;
    {
        PassRegs pa;
        load_pass(a, pa, 0, true);
        if constexpr (PAIR) {
            PassRegs pb;
            load_pass(*pair, pb, 0, true);
            __builtin_amdgcn_sched_barrier(0);  // both members' loads are issued before any use
            compute_pass(pa, red);
            compute_pass(pb, red_b);
        } else {
            __builtin_amdgcn_sched_barrier(0);  // every load of the pass is issued before any use
            compute_pass(pa, red);
        }
    }
    for (int base = step; base < nc; base += step) {
        PassRegs ps;
        load_pass(a, ps, base, false);
        __builtin_amdgcn_sched_barrier(0);
        compute_pass(ps, red);
    }
    if constexpr (PAIR) {
        for (int base = step; base < nc; base += step) {
            PassRegs ps;
            load_pass(*pair, ps, base, false);
            __builtin_amdgcn_sched_barrier(0);
            compute_pass(ps, red_b);
        }
    }
    if (sal_lds) {  // uniform: park the salient operands beside the partial sums
#pragma unroll
        for (int n = 0; n < kSalLoads; ++n) {
            const int i = static_cast<int>(threadIdx.x) + n * nthreads;
            if (i < wtotal) salw[i] = bits_value(wbits[n], a.salient_dtype);
        }
        for (int i = static_cast<int>(threadIdx.x) + kSalLoads * nthreads; i < wtotal;
             i += nthreads)  // blocks wider than the first-pass loads
            salw[i] = bits_value(load_bits(a.salient_values, a.salient_dtype, wbase + i < wlimit ? wbase + i : wlimit),
                                 a.salient_dtype);
        const auto gathered = [&](const RawElem& xv, const RawElem& sv) __attribute__((always_inline)) {
            return elem_value(xv, a.x_dtype) * (a.salient_scales ? elem_value(sv, a.scale_dtype) : 1.0f);
        };
        if (static_cast<int>(threadIdx.x) < tokens * ks) salx[threadIdx.x] = gathered(sx, ssc);
        for (int j = static_cast<int>(threadIdx.x + nthreads); j < tokens * ks; j += nthreads) {
            const int t = j / ks, k = j - t * ks;  // more gathered values than threads
            salx[j] = gathered(load_elem(a.x, a.x_dtype, t * in + a.salient_indices[k]),
                               load_elem(a.salient_scales ? a.salient_scales : a.s_in, a.scale_dtype, k));
        }
    }
    __syncthreads();
    if (dead) return;  // uniform, after the workgroup's only barrier

    // Output value of index idx (row < out and its tile < nt).
    const auto value = [&](const int idx, const OutIdx& o, const int row) __attribute__((always_inline)) {
        float sum = 0.0f;
        for (int c = 0; c < nc; ++c) sum += red[red_index<TPB, TB, TW>(c, o.tt, o.t, o.n)];
        float val = sum * elem_value(idx == threadIdx.x ? rs0 : load_elem(a.s_out, a.scale_dtype, row), a.scale_dtype);
        if (sal_lds) {
            const float* w = salw + (row - t0 * kTileRows) * ks;
            const float* xs = salx + o.t * ks;
            for (int k = 0; k < ks; ++k) val += w[k] * xs[k];
        } else {
            for (int k = 0; k < ks; ++k) {
                float wv = nq::load_f32(a.salient_values, a.salient_dtype, row * ks + k);
                if (a.salient_scales) wv *= nq::load_f32(a.salient_scales, a.scale_dtype, k);
                val += wv * nq::load_f32(a.x, a.x_dtype, o.t * in + a.salient_indices[k]);
            }
        }
        if (a.bias) val += elem_value(idx == threadIdx.x ? bias0 : load_elem(a.bias, a.bias_dtype, row), a.bias_dtype);
        return stale ? __builtin_nanf("") : val;
    };
    if constexpr (PAIR) {
        // One token: outputs idx = 16 tt + n; silu(gate) * up in a.y's dtype.
        for (int idx = threadIdx.x; idx < outs; idx += nthreads) {
            const OutIdx o = out_index<TPB>(idx, tokens);
            const int row = (t0 + o.tt) * kTileRows + o.n;
            if (t0 + o.tt >= nt || row >= out) continue;
            float sg = 0.0f, su = 0.0f;
            for (int c = 0; c < nc; ++c) {
                sg += red[red_index<TPB, TB, TW>(c, o.tt, o.t, o.n)];
                su += red_b[red_index<TPB, TB, TW>(c, o.tt, o.t, o.n)];
            }
            const bool own = idx == static_cast<int>(threadIdx.x);
            const float g = sg * elem_value(own ? rs0 : load_elem(a.s_out, a.scale_dtype, row), a.scale_dtype);
            const float u = su * elem_value(own ? rs1 : load_elem(pair->s_out, pair->scale_dtype, row),
                                            pair->scale_dtype);
            nq::store_f32_as(a.y, a.y_dtype, row, g / (1.0f + expf(-g)) * u);
        }
        return;
    }
    if (TPB == 1 && a.residual) {
        // Residual epilogue (one token, outs <= 64: wave 0, lanes 16 tt + n):
        // residual[row] += value, and lane 16 tt writes the tile's sum of the
        // new residual's squares (added in a fixed order).
        if (threadIdx.x < 64) {
            const int idx = threadIdx.x;
            const OutIdx o = out_index<TPB>(idx, tokens);
            const int row = (t0 + o.tt) * kTileRows + o.n;
            const bool ok = idx < outs && t0 + o.tt < nt && row < out;
            float sq = 0.0f;
            if (ok) {
                const float h = res0 + value(idx, o, row);  // row == fr here
                a.residual[row] = h;
                sq = h * h;
            }
            sq = row16_sum(sq);
            if (o.n == 0 && idx < outs && t0 + o.tt < nt) a.slots_out[t0 + o.tt] = sq;
        }
        return;
    }
    for (int idx = threadIdx.x; idx < outs; idx += nthreads) {
        const OutIdx o = out_index<TPB>(idx, tokens);
        const int row = (t0 + o.tt) * kTileRows + o.n;
        if (t0 + o.tt >= nt || row >= out) continue;
        nq::store_f32_as(a.y, a.y_dtype, o.t * out + row, value(idx, o, row));
    }
}

// Split launch: one kernel per stage, grid (workgroups, members). THREADS is
// the launch bound: 1024 for one token per block, 768 when a wave takes two
// chunks per pass (168 VGPRs), 512 for four tokens per block (256 VGPRs).
// Grid: (workgroups of the widest member, members). A workgroup reads its
// member's arguments in one batch (load_args), and nothing branches on them
// before the main loads are issued except the grid-padding exit (optional
// operands load from a valid address and are selected later, partial chunks
// use the same 16-byte word loads as full ones).
//
// The grid's x extent is a multiple of 8 and workgroup x takes block
// xcd_block(x, workgroups) (the XCD-contiguous order above).
template <int AK, int TPB, int TB, int TW, int KC, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_stage1(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    constexpr int kExtra = AK == kActNormF32    ? kArgsNorm
                           : AK == kActGatedF32 ? kArgsGated
                           : attn_kind<AK>()    ? kArgsAttn
                                                : kArgsPlain;
    const Lin a = load_args<kPinStage1, kExtra>(batch, blockIdx.y);
    const int nwg = static_cast<int>(a.nwg1);
    if (static_cast<int>(blockIdx.x) >= nwg) return;  // grid padding: the arguments are already loaded
    stage1_wg<AK, TPB, TB, TW, KC, false>(a, xcd_block(blockIdx.x, nwg), lds);
}

// Stage 0 of the several-token path: grid (ceil(chunks * token blocks / 4),
// members), four waves per workgroup, one (chunk, token block) per wave.
template <int AK>
__global__ __launch_bounds__(256) void k_decode_stage0(const Batch batch) {
    const Lin a = load_args<kPinStage1>(batch, blockIdx.y);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int nblk = (a.tokens + 3) >> 2;
    const int item = static_cast<int>(blockIdx.x) * 4 + wave;
    if (item >= static_cast<int>(a.g1.nc) * nblk) return;  // uniform per wave
    const int c = item / nblk;
    stage0_wave<AK>(a, c, item - c * nblk, nblk > 2 ? 4 : nblk, lane);
}

// Stage 1 of the several-token path (split launch, grid as k_decode_stage1).
template <int TB, int TW, int KC, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_stage1m(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const Lin a = load_args<kPinStage1>(batch, blockIdx.y);
    const int nwg = static_cast<int>(a.nwg1);
    if (static_cast<int>(blockIdx.x) >= nwg) return;
    stage1m_wg<TB, TW, KC>(a, xcd_block(blockIdx.x, nwg), lds);
}

template <int TPB, int TB, int TW, int KC, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_stage2(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const Lin a = load_args<kPinStage2>(batch, blockIdx.y);
    const int nwg = static_cast<int>(a.nwg2);
    if (static_cast<int>(blockIdx.x) >= nwg) return;  // grid padding: the arguments are already loaded
    stage2_wg<TPB, TB, TW, KC, false>(a, xcd_block(blockIdx.x, nwg), lds);
}

// Paired stage 2 (one token): members 0 and 1 of the batch, one grid row.
template <int TW, int KC, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_stage2_pair(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    Lin a, b;
    load_args_pair(batch, a, b);
    const int nwg = static_cast<int>(a.nwg2);
    if (static_cast<int>(blockIdx.x) >= nwg) return;
    stage2_wg<1, 1, TW, KC, false, true>(a, xcd_block(blockIdx.x, nwg), lds, &b);
}

// Fused launch (one tile per workgroup, generic stage-1 loads): grid rows
// [0, count) are stage 1, rows [count, 2 count) stage 2.
template <int TPB, int TB, int KC1, int KC2, int THREADS>
__global__ __launch_bounds__(THREADS) void k_decode_fused(const Batch batch) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int y = static_cast<int>(blockIdx.y);
    const int count = batch.count;
    const Lin a = load_args<kPinStages>(batch, y < count ? y : y - count);
    if (y < count) {
        if (blockIdx.x >= a.nwg1) return;
        stage1_wg<kActGeneric, TPB, TB, 1, KC1, true>(a, blockIdx.x, lds);
    } else {
        if (blockIdx.x >= a.nwg2) return;
        stage2_wg<TPB, TB, 1, KC2, true>(a, blockIdx.x, lds);
    }
}

// Launch bound of a configuration (see k_decode_stage1): blocks of up to four
// tokens take up to 16 waves of one chunk or 12 of two; several token blocks
// take at most 8 waves (their operand registers for two or four blocks would
// spill under a bound of 16 waves).
constexpr int threads_for(int tpb, int kc, int tb = 1) { return tb > 1 ? 512 : (kc == 1 ? 1024 : 768); }

// Shape of one decode launch, chosen on the host (nq_decode.hip).
struct LaunchShape {
    int ak;          // activation kind of stage 1
    int tpb, tb;     // tokens per block, blocks
    int tw;          // tiles per workgroup
    int nw;          // waves per workgroup
    int kc, kc2;     // chunks per wave per pass (stage kernels: kc; fused: stage 1 kc, stage 2 kc2)
    size_t lds;      // dynamic LDS bytes
    dim3 grid;
};

// Launchers, one translation unit each (they instantiate disjoint kernels).
int enqueue_stage1_bf16(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_f16(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_f32(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_generic(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1_fused(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage2(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage2_pair(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage0(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_stage1m(const Batch& batch, const LaunchShape& s, hipStream_t stream);
int enqueue_fused(const Batch& batch, const LaunchShape& s, hipStream_t stream);

}  // namespace nqdec

// Decode path (tokens <= 16): prepare-time tile builder and host-side launch
// logic. The kernels and the tile layout are documented in
// nq_decode_kernels.h.
#include "nq_decode_kernels.h"

namespace nqdec {
namespace {

// ---------------------------------------------------------------------------
// Prepare: canonical words -> tile words.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_build_tiles(const uint32_t* __restrict__ canon, int64_t rows,
                                                     int64_t cols, uint32_t* __restrict__ tiles) {
    const int64_t wpr = (cols + 31) / 32;
    const MatGeo g = mat_geo(rows, cols);
    const int64_t per_tile = g.nb * 64;
    const int64_t total = g.nt * per_tile;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t t = e / per_tile;
        const int64_t rem = e - t * per_tile;
        const int64_t c = rem >> 8;
        const int within = static_cast<int>(rem - (c << 8));
        const int dw = chunk_words(g, c);
        const int lane = within / dw;
        const int d = within - lane * dw;
        const int64_t row = t * kTileRows + (lane & 15);
        const int grp = lane >> 4;
        uint32_t word = 0;
        if (row < rows) {
            const uint32_t* src = canon + row * wpr;
            for (int b = 0; b < 4; ++b) {
                for (int m = 0; m < 8; ++m) {
                    const int64_t col = kChunkCols * c + kBlockCols * d + 16 * m + 4 * grp + b;
                    if (col < cols) word |= ((src[col >> 5] >> (col & 31)) & 1u) << (8 * b + m);
                }
            }
        }
        tiles[e] = word;
    }
}

// Zero the header, write the magic, the fused launch's spin limit and
// max|s_mid| (the stage-1 epilogue's bound on the rank intermediate). One
// workgroup of 256 threads.
__global__ __launch_bounds__(256) void k_init_header(uint32_t* header, const void* s_mid, int scale_dtype,
                                                     int64_t rank) {
    __shared__ float wmax[4];
    for (int i = threadIdx.x; i < kHeaderWords; i += blockDim.x) header[i] = 0;
    float m = 0.0f;
    for (int64_t r = threadIdx.x; r < rank; r += blockDim.x) m = fmaxf(m, fabsf(nq::load_f32(s_mid, scale_dtype, r)));
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        header[line_word(kMiscLine) + kMiscMagic] = kTilesMagic;
        header[line_word(kMiscLine) + kMiscSpin] = kSpinLimit;
        header[line_word(kMiscLine) + kMiscMaxMid] =
            __float_as_uint(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
    }
}

struct TilesGeometry {
    MatGeo g1, g2;
    int64_t v_words, u_words;
};

// Tail padding after the U tiles: a partial chunk's 16-byte word load reads up
// to three words past its lane's own (see load_words).
constexpr int64_t kTailBytes = 256;

int64_t tiles_bytes_of(const TilesGeometry& g) { return (kHeaderWords + g.v_words + g.u_words) * 4 + kTailBytes; }

TilesGeometry geometry(int64_t in, int64_t out, int64_t rank) {
    TilesGeometry g{};
    g.g1 = mat_geo(rank, in);
    g.g2 = mat_geo(out, rank);
    g.v_words = mat_words(g.g1);
    g.u_words = mat_words(g.g2);
    return g;
}

static_assert(Ops<1>::kBytes == 2048 && Ops<4>::kBytes == 8192, "lmq_bytes_for's operand block sizes");

// Workspace: [lmq][lme: 256 B][xq][xe][xm] (the last three for several
// tokens, at the addresses multi_ws derives from lme).
int64_t scratch_bytes(const TilesGeometry& g, int64_t tokens) {
    return round256(lmq_bytes_for(g.g2, tokens)) + 256 + round256(xq_bytes_for(g.g1, tokens)) +
           2 * xe_bytes_for(g.g1, tokens);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// The kernels index with 32-bit offsets: every word, operand byte and element
// offset of a launch stays below 2^31 (sign words up to 8 GiB per factor).
bool offsets_fit(const TilesGeometry& g, int64_t in, int64_t out, int64_t tokens, int64_t salient) {
    constexpr int64_t kMax = int64_t(1) << 31;
    return g.v_words < kMax && g.u_words < kMax && scratch_bytes(g, tokens) < kMax && tokens * in < kMax &&
           tokens * out < kMax && out * (salient > 0 ? salient : 1) < kMax;
}

// Fill one linear of a batch; NQ_OK or an error status. `vector_ok` is cleared
// when this member's x or s_in cannot take the vector-load kinds.
int describe(const nq_linear_desc* d, const void* x, int x_dtype, int64_t tokens, void* y, int y_dtype,
             void* scratch, Lin& a, bool& vector_ok) {
    const TilesGeometry g = geometry(d->in_features, d->out_features, d->rank);
    if (!d->tiles) return NQ_ERR_ARGUMENT;
    if (d->tiles_bytes < tiles_bytes_of(g)) return NQ_ERR_ARGUMENT;
    if (!offsets_fit(g, d->in_features, d->out_features, tokens, d->salient_count)) return NQ_ERR_SHAPE;
    if (!aligned(d->tiles, 16) || !aligned(scratch, 16)) return NQ_ERR_ALIGNMENT;
    a = Lin{};
    a.in = d->in_features;
    a.rank = d->rank;
    a.out = d->out_features;
    a.g1 = g.g1;
    a.g2 = g.g2;
    uint32_t* base = static_cast<uint32_t*>(const_cast<void*>(d->tiles));
    a.header = base;
    a.v_tiles = base + kHeaderWords;
    a.u_tiles = base + kHeaderWords + g.v_words;
    a.x = x;
    a.x_dtype = x_dtype;
    // Vector loads of x and s_in: rows of length % 8 == 0, fp16 scales and
    // 16-byte aligned bases (eight 16-bit or four fp32 elements per load).
    if (!(d->in_features % 8 == 0 && d->scale_dtype == NQ_DTYPE_F16 && aligned(x, 16) && aligned(d->scale_pre, 16)))
        vector_ok = false;
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
    char* const ws = static_cast<char*>(scratch);
    a.lmq = reinterpret_cast<uint8_t*>(ws);
    a.lme = reinterpret_cast<int*>(ws + round256(lmq_bytes_for(g.g2, tokens)));
    return NQ_OK;
}

// Waves per workgroup and chunks per wave per pass for a stage whose widest
// member has nc chunks. One block of up to four tokens: one chunk per wave up
// to 16 waves, otherwise two chunks per wave on at most 12 waves (the 24
// chunks of a 12288-wide input in one pass; measured on MI355X over the
// Qwen3-8B stack at 2-4 tokens: 49.2 against 50.6 us per layer with at most
// 8 waves and two passes). Several blocks (the fused launch from five tokens):
// at most 8 waves of one chunk (their activation registers would not fit
// twice) and the pass loop covers the rest.
void pick_waves(int64_t nc, int tpb, int tb, int& nw, int& kc) {
    if (tpb == 1 || tb == 1) {
        if (nc <= 16) {
            nw = static_cast<int>(nc);
            kc = 1;
        } else {
            const int64_t half = (nc + 1) / 2;
            nw = static_cast<int>(half < 12 ? half : 12);
            kc = 2;
        }
    } else {
        nw = static_cast<int>(nc < 8 ? nc : 8);
        kc = (tb == 1 && nc > 8) ? 2 : 1;
    }
}

// The same for the several-token stages of the split launch: at most eight
// waves, two per chunk slot with four token blocks (blocks_per_wave); with one
// token block two chunks per wave per pass when the slots would not cover the
// chunks (a wave holding two blocks has no registers for a second chunk).
void pick_waves_multi(int64_t nc, int tb, int& nw, int& kc) {
    const int ng = tb > 2 ? 2 : 1;
    const int64_t max_slots = 8 / ng;
    kc = nc > max_slots && tb == 1 ? 2 : 1;
    int64_t slots = (nc + kc - 1) / kc;
    if (slots > max_slots) slots = max_slots;
    nw = static_cast<int>(slots) * ng;
}

// Dynamic LDS of a stage: per-wave operand areas (stage 1), the partial sums
// [nc][tw][tb][64], the chunk maxima [nc][tpb * tb] (stage 1) and, for one
// token, kc operand spread areas per wave (stage 2), then the staged salient
// operands of the member with the most salient columns (stage 2).
size_t lds_bytes(int stage, int tpb, int tb, int tw, int nw, int kc, int64_t nc, int64_t ks = 0, int tokens = 1) {
    const size_t red = static_cast<size_t>(nc) * tw * tb * 64 * 4;
    if (stage == 2)
        return red + (tpb == 1 ? static_cast<size_t>(nw) * kc * kS2SpreadBytes : 0) + sal_lds_bytes(ks, tw, tokens);
    return static_cast<size_t>(nw) * (8 * 4 * tpb * 4 * 16) + red + static_cast<size_t>(nc) * tpb * tb * 4;
}

// Tiles per workgroup (measured on MI355X over the Qwen3-8B decode calls).
// A wave's fixed work (arguments, addresses, the chunk's ones-MFMAs and, in
// stage 1, the staging) is shared by its TW tiles, against fewer waves to
// hide latency:
//   stage 1: two tiles when one chunk per wave and one tile per workgroup
//     would launch more than 1536 waves (the staging is then the larger
//     cost), else one;
//   stage 2: the fewest tiles that keep the stage within three waves per SIMD
//     (3072 waves), at most four.
// Blocks of several token groups (registers) and the fused launch (its
// stage-2 wait is per workgroup) take one.
constexpr int64_t kStage1Waves = 1536;
constexpr int64_t kStage2Waves = 3 * 4 * 256;

int pick_tiles(int stage, int64_t tiles, int nw, int kc, int tb, bool fused) {
    if (fused || tb > 1) return 1;
    const int64_t waves = tiles * nw;
    if (stage == 1) return kc == 1 && waves > kStage1Waves ? 2 : 1;
    for (int tw = 1; tw < 4; ++tw)
        if (waves <= kStage2Waves * tw) return tw;
    return 4;
}

// Tokens from which the split launch stages x * s_in in a kernel of its own
// (stage 0) instead of in every stage-1 workgroup. Measured on MI355X over the
// Qwen3-8B decode stack (us per layer, in-kernel staging against stage 0):
// 2 tokens 50.8 / 59.0, 4 tokens 50.1 / 59.3, 8 tokens 93.8 / 76.3,
// 16 tokens 132.2 / 105.1: below two token blocks the extra launch costs more
// than the staging it saves.
constexpr int64_t kStage0Tokens = 5;
bool stage0_path(int64_t tokens) { return tokens >= kStage0Tokens; }

// Tiles per workgroup of the several-token stages: a wave's A operands (8 KB
// per block of four tokens per chunk) are shared by its TW tiles, against
// fewer waves. One token block (stage 2 after the in-kernel staging): four
// tiles from 4096 waves, two from 2048. Two or four blocks (stage 0 path):
// two tiles in both stages (measured best against one and four, per stage,
// at 8 and 16 tokens).
int pick_tiles_multi(int64_t tiles, int nw, int tb) {
    if (tb > 1) return 2;
    const int64_t waves = tiles * nw;
    return waves >= 4 * 1024 ? 4 : (waves >= 2 * 1024 ? 2 : 1);
}

int enqueue_stage1(const Batch& batch, const LaunchShape& s, hipStream_t stream) {
    switch (s.ak) {
        case kActBf16: return enqueue_stage1_bf16(batch, s, stream);
        case kActF16: return enqueue_stage1_f16(batch, s, stream);
        case kActF32: return enqueue_stage1_f32(batch, s, stream);
        case kActNormF32:
        case kActGatedF32:
        case kActAttn8:
        case kActAttn12:
        case kActAttn16:
        case kActAttn8E:
        case kActAttn12E:
        case kActAttn16E: return enqueue_stage1_fused(batch, s, stream);
        default: return enqueue_stage1_generic(batch, s, stream);
    }
}

// Cache blocks of the decode attention's pass 1 for a cache of max_positions rows.
int64_t attn_blocks_of(int64_t max_positions) { return (max_positions + kAttnBlockRows - 1) / kAttnBlockRows; }

// Fill member i's fusion fields; NQ_OK or an error status.
int describe_fusion(const nq_decode_fusion& f, int i, const nq_linear_desc* d, Lin& a) {
    const int64_t in = d->in_features;
    if (f.input_kind == NQ_INPUT_RMSNORM) {
        if (!f.col_scales || !f.col_scales[i] || !f.norm_slots) return NQ_ERR_ARGUMENT;
        if (f.norm_slot_count != (in + kTileRows - 1) / kTileRows || f.norm_slot_count % 4 != 0 ||
            f.norm_slot_count > 256 * kSlotVecs)
            return NQ_ERR_SHAPE;
        if (!aligned(f.col_scales[i], 16) || !aligned(f.norm_slots, 16)) return NQ_ERR_ALIGNMENT;
        if (!(f.eps > 0.0f)) return NQ_ERR_ARGUMENT;
        a.col_scale = f.col_scales[i];
        a.slots_in = f.norm_slots;
        a.nslots = static_cast<int>(f.norm_slot_count);
        a.eps = f.eps;
    } else if (f.input_kind == NQ_INPUT_SILU_GATE) {
        if (!f.ups || !f.ups[i]) return NQ_ERR_ARGUMENT;
        if (!aligned(f.ups[i], 16)) return NQ_ERR_ALIGNMENT;
        a.x2 = f.ups[i];
    } else if (f.input_kind == NQ_INPUT_ATTENTION) {
        // x (already in a.x) is the pass-1 workspace: fp32 (max, sum) pairs
        // [heads][blocks][2], then the fp16 block outputs [heads][blocks][head_dim].
        const int hd = f.attn_head_dim;
        if (!f.attn_position || (hd != 64 && hd != 128 && hd != 256)) return NQ_ERR_ARGUMENT;
        if (in % hd != 0 || f.attn_max_positions <= 0 || f.attn_max_positions > 0x7fffffff) return NQ_ERR_SHAPE;
        const int64_t blocks = attn_blocks_of(f.attn_max_positions);
        // One chunk per wave and at most eight waves; every block's partials in registers.
        if (in > 8 * kChunkCols || blocks > attn_parts<kActAttn16>()) return NQ_ERR_UNSUPPORTED;
        const int64_t heads = in / hd;
        if ((heads * blocks) % 2 != 0 || !aligned(a.x, 16)) return NQ_ERR_ALIGNMENT;  // 16-byte accumulator rows
        a.attn_ml = static_cast<const float*>(a.x);
        a.x = static_cast<const float*>(a.x) + 2 * heads * blocks;
        a.attn_pos = f.attn_position;
        a.attn_blocks = static_cast<int>(blocks);
        a.attn_hd_log2 = hd == 64 ? 6 : (hd == 128 ? 7 : 8);
        a.attn_max_positions = f.attn_max_positions;
    } else if (f.input_kind != NQ_INPUT_PLAIN) {
        return NQ_ERR_ARGUMENT;
    }
    if (f.input_kind != NQ_INPUT_PLAIN && d->salient_count > 0) return NQ_ERR_UNSUPPORTED;
    if (f.residuals) {
        if (!f.residuals[i] || !f.out_slots || !f.out_slots[i]) return NQ_ERR_ARGUMENT;
        a.residual = f.residuals[i];
        a.slots_out = f.out_slots[i];
    }
    return NQ_OK;
}

// Launch shapes of a batch: tiles and waves per workgroup of each stage,
// written into the batch (tw1, tw2, and every member's nw / nwg).
struct Shapes {
    LaunchShape s1, s2;
    int64_t nc1, nc2, ks, max1, max2;
};

// The stage-1 chunk count that most of a batch's stage-1 tiles have (ties:
// the larger). A one-token batch plans its stage-1 waves for it; members with
// more chunks run more passes. Measured on MI355X with the seven linears of a
// Qwen3-8B layer in one batch (six of 8 chunks, down_proj of 24): 18.4 us per
// layer against 23.5 us when planned for the widest member (12 waves of two
// chunks, one 768-thread workgroup per CU).
int64_t typical_chunks1(const HostBatch& batch) {
    int64_t best = 0, best_tiles = -1;
    for (int i = 0; i < batch.count; ++i) {
        const int64_t nc = batch.p[i].g1.nc;
        int64_t tiles = 0;
        for (int j = 0; j < batch.count; ++j) tiles += batch.p[j].g1.nc == nc ? batch.p[j].g1.nt : 0;
        if (tiles > best_tiles || (tiles == best_tiles && nc > best)) best = nc, best_tiles = tiles;
    }
    return best;
}

int plan_shapes(HostBatch& batch, int64_t tokens, int ak, bool fused, Shapes& sh) {
    int64_t tiles1 = 0, tiles2 = 0, nc1 = 0, nc2 = 0, ks = 0;
    for (int i = 0; i < batch.count; ++i) {
        ks = batch.p[i].salient_count <= kSalMax && batch.p[i].salient_count > ks ? batch.p[i].salient_count : ks;
        tiles1 += batch.p[i].g1.nt;
        tiles2 += batch.p[i].g2.nt;
        nc1 = batch.p[i].g1.nc > nc1 ? batch.p[i].g1.nc : nc1;
        nc2 = batch.p[i].g2.nc > nc2 ? batch.p[i].g2.nc : nc2;
    }
    LaunchShape s1{}, s2{};
    s1.tpb = s2.tpb = tokens == 1 ? 1 : 4;
    // Blocks of four tokens: 1, 2 or 4 in the split launch, 1 or 4 fused.
    s1.tb = s2.tb = tokens <= 4 ? 1 : (tokens <= 8 && !fused && stage0_path(tokens) ? 2 : 4);
    s1.ak = s2.ak = ak;
    if (fused) {
        // The fused kernel keeps both stages' registers live: blocks of four
        // tokens stay within 8 waves (512 threads) there.
        int kc_unused = 0;
        const int64_t ncf = nc1 > nc2 ? nc1 : nc2;
        pick_waves(ncf, s1.tpb, s1.tb, s1.nw, kc_unused);
        if (s1.tpb > 1 && s1.nw > 8) s1.nw = 8;
        s1.kc = (s1.tb == 1 && nc1 > s1.nw) ? 2 : 1;
        s1.kc2 = (s1.tb == 1 && nc2 > s1.nw) ? 2 : 1;
        s1.tw = 1;
    } else {
        if (!stage0_path(tokens)) {
            pick_waves(tokens == 1 ? typical_chunks1(batch) : nc1, s1.tpb, s1.tb, s1.nw, s1.kc);
            pick_waves(nc2, s2.tpb, s2.tb, s2.nw, s2.kc);
            s1.tw = pick_tiles(1, tiles1, s1.nw, s1.kc, s1.tb, false);
            s2.tw = tokens == 1 ? pick_tiles(2, tiles2, s2.nw, s2.kc, s2.tb, false)
                                : pick_tiles_multi(tiles2, s2.nw, s2.tb);
        } else {
            pick_waves_multi(nc1, s1.tb, s1.nw, s1.kc);
            pick_waves_multi(nc2, s2.tb, s2.nw, s2.kc);
            s1.tw = pick_tiles_multi(tiles1, s1.nw, s1.tb);
            s2.tw = pick_tiles_multi(tiles2, s2.nw, s2.tb);
            // Partial sums within 64 KB of LDS.
            while (s1.tw > 1 && nc1 * s1.tw * s1.tb * 256 + nc1 * kMaxTokens * 4 > 65536) s1.tw >>= 1;
            while (s2.tw > 1 && static_cast<int64_t>(lds_bytes(2, s2.tpb, s2.tb, s2.tw, s2.nw, s2.kc, nc2, ks,
                                                               static_cast<int>(tokens))) > 65536)
                s2.tw >>= 1;
        }
    }
    batch.tw1 = s1.tw;
    batch.tw2 = fused ? 1 : s2.tw;
    int64_t max1 = 0, max2 = 0;
    for (int i = 0; i < batch.count; ++i) {
        Lin& a = batch.p[i];
        a.nw1 = s1.nw;
        a.nw2 = fused ? s1.nw : s2.nw;
        a.nwg1 = (a.g1.nt + batch.tw1 - 1) / batch.tw1;
        a.nwg2 = (a.g2.nt + batch.tw2 - 1) / batch.tw2;
        max1 = a.nwg1 > max1 ? a.nwg1 : max1;
        max2 = a.nwg2 > max2 ? a.nwg2 : max2;
    }
    if (max1 > 0x7ffffff0 || max2 > 0x7ffffff0) return NQ_ERR_SHAPE;
    sh = Shapes{s1, s2, nc1, nc2, ks, max1, max2};
    return NQ_OK;
}

// Grid x extent of a split-launch stage: a multiple of 8, so workgroup x of
// every grid row runs on XCD x % 8 (workgroups are dispatched to the eight
// XCDs round-robin in linear order).
unsigned xcd_grid(int64_t workgroups) { return static_cast<unsigned>((workgroups + 7) & ~int64_t(7)); }

int launch_batch(HostBatch& plan, int64_t tokens, int ak, bool fused, hipStream_t stream, bool pair = false) {
    Shapes sh{};
    int st = plan_shapes(plan, tokens, ak, fused, sh);
    if (st != NQ_OK) return st;
    Batch batch;
    pack_batch(plan, batch);
    LaunchShape s1 = sh.s1, s2 = sh.s2;
    const int64_t nc1 = sh.nc1, nc2 = sh.nc2, ks = sh.ks, max1 = sh.max1, max2 = sh.max2;
    const unsigned count = static_cast<unsigned>(batch.count);

    if (fused) {  // the fused launch keeps blocks in launch order
        const size_t l1 = lds_bytes(1, s1.tpb, s1.tb, 1, s1.nw, s1.kc, nc1),
                     l2 = lds_bytes(2, s1.tpb, s1.tb, 1, s1.nw, s1.kc2, nc2, ks, static_cast<int>(tokens));
        s1.lds = l1 > l2 ? l1 : l2;
        s1.grid = dim3(static_cast<unsigned>(max1 > max2 ? max1 : max2), 2 * count);
        return enqueue_fused(batch, s1, stream);
    }
    s1.grid = dim3(xcd_grid(max1), count);
    if (stage0_path(tokens)) {
        // Stage 0 stages x * s_in once per (chunk, token block); stage 1 reads
        // its operands.
        LaunchShape s0 = s1;
        const int64_t items = nc1 * ((tokens + 3) / 4);
        s0.grid = dim3(static_cast<unsigned>((items + 3) / 4), count);
        st = enqueue_stage0(batch, s0, stream);
        if (st != NQ_OK) return st;
        s1.lds = static_cast<size_t>(nc1) * s1.tw * s1.tb * 64 * 4 + static_cast<size_t>(nc1) * kMaxTokens * 4;
        st = enqueue_stage1m(batch, s1, stream);
    } else {
        s1.lds = lds_bytes(1, s1.tpb, s1.tb, s1.tw, s1.nw, s1.kc, nc1);
        st = enqueue_stage1(batch, s1, stream);
    }
    if (st != NQ_OK) return st;
    s2.lds = lds_bytes(2, s2.tpb, s2.tb, s2.tw, s2.nw, s2.kc, nc2, ks, static_cast<int>(tokens));
    if (pair) {
        // Both members' partial sums in one workgroup: a second partial-sum area.
        s2.lds += static_cast<size_t>(nc2) * s2.tw * s2.tb * 64 * 4;
        s2.grid = dim3(xcd_grid(max2), 1);
        return enqueue_stage2_pair(batch, s2, stream);
    }
    s2.grid = dim3(xcd_grid(max2), count);
    return enqueue_stage2(batch, s2, stream);
}

}  // namespace
}  // namespace nqdec

using namespace nqdec;

namespace nq {

int64_t tiles_header_words() { return kHeaderWords; }

int64_t tiles_max_mid_word() { return line_word(kMiscLine) + kMiscMaxMid; }

int64_t decode_scratch_bytes(const nq_linear_desc* d, int64_t tokens) {
    if (!d->tiles) return 0;
    return scratch_bytes(geometry(d->in_features, d->out_features, d->rank), tokens);
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
                        hipStream_t stream, const nq_decode_fusion* fusion) {
    if (count < 1 || count > kMaxBatch) return NQ_ERR_SHAPE;
    if (tokens < 1 || tokens > kMaxTokens) return NQ_ERR_SHAPE;
    HostBatch batch{};
    batch.count = count;
    bool vector_ok = true;
    for (int i = 0; i < count; ++i) {
        if (descs[i]->decode_launch != descs[0]->decode_launch) return NQ_ERR_ARGUMENT;
        if (descs[i]->scale_dtype != descs[0]->scale_dtype) return NQ_ERR_DTYPE;
        int st = describe(descs[i], xs[i], x_dtype, tokens, ys[i], y_dtype, scratch[i], batch.p[i], vector_ok);
        if (st != NQ_OK) return st;
        if (fusion) {
            st = describe_fusion(*fusion, i, descs[i], batch.p[i]);
            if (st != NQ_OK) return st;
        }
    }
    int ak = kActGeneric;
    if (vector_ok) {
        ak = x_dtype == NQ_DTYPE_BF16 ? kActBf16 : (x_dtype == NQ_DTYPE_F16 ? kActF16 : kActF32);
    }
    bool pair = false;
    if (fusion) {
        // The fused forms have vector kernels only: one token, the split launch,
        // fp32 x and fp16 scales with the vector-load shape.
        if (tokens != 1 || descs[0]->decode_launch != NQ_DECODE_SPLIT) return NQ_ERR_UNSUPPORTED;
        if (fusion->output_kind == NQ_OUTPUT_SILU_PRODUCT) {
            const nq_linear_desc* a = descs[0];
            const nq_linear_desc* b = count == 2 ? descs[1] : nullptr;
            if (!b || fusion->residuals || a->out_features != b->out_features || a->rank != b->rank) return NQ_ERR_SHAPE;
            for (const nq_linear_desc* d : {a, b})
                if (d->salient_count > 0 || d->bias || d->patch_rank > 0 || d->row_count > 0) return NQ_ERR_UNSUPPORTED;
            pair = true;
        } else if (fusion->output_kind != NQ_OUTPUT_PLAIN) {
            return NQ_ERR_ARGUMENT;
        }
        if (fusion->input_kind != NQ_INPUT_PLAIN) {
            if (x_dtype != NQ_DTYPE_F32) return NQ_ERR_DTYPE;
            if (!vector_ok) return NQ_ERR_ALIGNMENT;
            if (fusion->input_kind == NQ_INPUT_ATTENTION) {
                // The fewest partial registers that hold every block; paired
                // (max, sum) loads for an even block count.
                const int64_t blocks = attn_blocks_of(fusion->attn_max_positions);
                const bool even = blocks % 2 == 0;
                ak = blocks <= attn_parts<kActAttn8>()    ? (even ? kActAttn8E : kActAttn8)
                     : blocks <= attn_parts<kActAttn12>() ? (even ? kActAttn12E : kActAttn12)
                                                          : (even ? kActAttn16E : kActAttn16);
            } else {
                ak = fusion->input_kind == NQ_INPUT_RMSNORM ? kActNormF32 : kActGatedF32;
            }
        }
    }
    return launch_batch(batch, tokens, ak, descs[0]->decode_launch == NQ_DECODE_FUSED, stream, pair);
}

}  // namespace nq

extern "C" int64_t nq_tiles_header_bytes(void) { return static_cast<int64_t>(kHeaderWords) * 4; }

extern "C" int64_t nq_tiles_bytes(int64_t in_features, int64_t out_features, int64_t rank) {
    if (in_features <= 0 || out_features <= 0 || rank <= 0) return -1;
    return tiles_bytes_of(geometry(in_features, out_features, rank));
}

extern "C" int nq_prepare_tiles(const nq_linear_desc* d, void* tiles, int64_t tiles_bytes, void* stream) {
    if (!d || !tiles || !d->right_words || !d->left_words || !d->scale_pre || !d->scale_mid) return NQ_ERR_ARGUMENT;
    if (d->in_features <= 0 || d->out_features <= 0 || d->rank <= 0) return NQ_ERR_SHAPE;
    if (!nq::is_float_dtype(d->scale_dtype)) return NQ_ERR_DTYPE;
    const TilesGeometry g = geometry(d->in_features, d->out_features, d->rank);
    if (tiles_bytes < tiles_bytes_of(g)) return NQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(tiles) % 256 != 0) return NQ_ERR_ALIGNMENT;
    auto s = static_cast<hipStream_t>(stream);
    uint32_t* base = static_cast<uint32_t*>(tiles);
    hipLaunchKernelGGL(k_init_header, dim3(1), dim3(256), 0, s, base, d->scale_mid, d->scale_dtype, d->rank);
    auto grid_for = [](int64_t n) {
        const int64_t b = (n + 255) / 256;
        return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
    };
    hipLaunchKernelGGL(k_build_tiles, dim3(grid_for(g.v_words)), dim3(256), 0, s,
                       reinterpret_cast<const uint32_t*>(d->right_words), d->rank, d->in_features,
                       base + kHeaderWords);
    hipLaunchKernelGGL(k_build_tiles, dim3(grid_for(g.u_words)), dim3(256), 0, s,
                       reinterpret_cast<const uint32_t*>(d->left_words), d->out_features, d->rank,
                       base + kHeaderWords + g.v_words);
    return nq::launch_status();
}


// Host-side exercise of the C ABI's argument checks and launch planning, built
// with AddressSanitizer and UndefinedBehaviorSanitizer on the host code of
// libnqamd (build_and_run.sh). It runs only where no GPU is visible: every call
// either returns an argument error before any device work, or plans its launch
// (descriptor checks, geometry, tile and wave choice, kernel-argument packing)
// and gets NQ_ERR_LAUNCH from the runtime. The fake device buffers below are
// host allocations that nothing dereferences on the host.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "nqamd.h"
#include "nqamd_shell.h"

namespace {

int failures = 0;

void expect(bool ok, const char* what, int got) {
    if (!ok) {
        std::fprintf(stderr, "FAIL %s (status %d)\n", what, got);
        ++failures;
    }
}

// A status from a call that reaches the launch without a device.
bool launch_refused(int st) { return st == NQ_ERR_LAUNCH || st == NQ_ERR_DEVICE; }

struct Buffer {
    void* p = nullptr;
    explicit Buffer(size_t bytes) { p = std::aligned_alloc(256, (bytes + 255) / 256 * 256); }
    ~Buffer() { std::free(p); }
};

nq_linear_desc desc_for(int64_t in, int64_t out, int64_t rank, const Buffer& words, const Buffer& scales,
                        const Buffer& tiles, int64_t tiles_bytes) {
    nq_linear_desc d;
    std::memset(&d, 0, sizeof(d));
    d.in_features = in;
    d.out_features = out;
    d.rank = rank;
    d.right_words = static_cast<const int32_t*>(words.p);
    d.left_words = static_cast<const int32_t*>(words.p);
    d.scale_pre = scales.p;
    d.scale_mid = scales.p;
    d.scale_post = scales.p;
    d.scale_dtype = NQ_DTYPE_F16;
    d.bias_dtype = NQ_DTYPE_F16;
    d.tiles = tiles.p;
    d.tiles_bytes = tiles_bytes;
    d.decode_launch = NQ_DECODE_SPLIT;
    d.prefill_operands = NQ_PREFILL_FP16;
    return d;
}

}  // namespace

int main() {
    nq_device_caps caps;
    if (nq_query_device(0, &caps) == NQ_OK) {
        std::printf("a GPU is visible: this host-only driver runs nothing\n");
        return 77;
    }
    expect(nq_abi_version() > 0, "abi version", 0);
    for (int s = -20; s <= 1; ++s) expect(nq_status_string(s) != nullptr, "status string", s);

    // Argument errors.
    expect(nq_unpack_signs(nullptr, 1, 1, 1, NQ_DTYPE_F32, nullptr, nullptr) == NQ_ERR_ARGUMENT, "unpack null", 0);
    expect(nq_tiles_bytes(0, 1, 1) < 0 && nq_tiles_bytes(1, 1, -1) < 0, "tiles bytes shape", 0);
    nq_linear_desc bad;
    std::memset(&bad, 0, sizeof(bad));
    expect(nq_linear_workspace_bytes(&bad, 1) == -1, "workspace of empty desc", 0);
    expect(nq_linear(&bad, nullptr, 0, 1, nullptr, 0, nullptr, 0, nullptr) != NQ_OK, "linear empty desc", 0);
    expect(nq_linear_batch(nullptr, 0, nullptr, 0, 1, nullptr, 0, nullptr, nullptr, nullptr) != NQ_OK, "batch null", 0);
    expect(nq_embedding(nullptr, 1, nullptr, NQ_DTYPE_BF16, 1, 8, nullptr, nullptr, nullptr) == NQ_ERR_ARGUMENT,
           "embedding null", 0);
    expect(nq_embedding_slots(nullptr, 1, nullptr, NQ_DTYPE_BF16, 1, 16, nullptr, nullptr, nullptr, nullptr) ==
               NQ_ERR_ARGUMENT, "embedding slots null", 0);
    expect(nq_add_rmsnorm(nullptr, nullptr, 0, nullptr, 0, 1e-6f, 1, 8, nullptr, 0, nullptr) == NQ_ERR_ARGUMENT,
           "add_rmsnorm null", 0);
    expect(nq_silu_mul(nullptr, nullptr, 8, nullptr, NQ_DTYPE_F32, nullptr) != NQ_OK, "silu null", 0);
    expect(nq_greedy_select(nullptr, 1, 8, nullptr, nullptr, 0, nullptr, nullptr, nullptr) == NQ_ERR_ARGUMENT,
           "greedy null", 0);
    expect(nq_decode_attention_workspace_bytes(32, 7, 128, NQ_DTYPE_BF16, 640) == -1, "attention heads", 0);
    expect(nq_output_projection_workspace_bytes(151936, 4096) > 0, "lm_head workspace", 0);
    expect(nq_attention_workspace_bytes(1, 32, 128, 640) > 0, "attention workspace", 0);

    // Launch planning of decode and prefill calls over the Qwen3-8B projection
    // shapes, every token count of the decode range and a few prefill ones.
    const int64_t shapes[][3] = {{4096, 4096, 2048}, {4096, 1024, 819}, {4096, 12288, 3072},
                                 {12288, 4096, 3072}, {1152, 6912, 768}, {35, 17, 5}};
    const int64_t token_counts[] = {1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 40, 64, 300};
    Buffer words(64 << 20), scales(1 << 20), x(64 << 20), y(64 << 20);
    for (const auto& sh : shapes) {
        const int64_t tb = nq_tiles_bytes(sh[0], sh[1], sh[2]);
        expect(tb > 0, "tiles bytes", 0);
        Buffer tiles(static_cast<size_t>(tb));
        for (int launch : {NQ_DECODE_SPLIT, NQ_DECODE_FUSED}) {
            nq_linear_desc d = desc_for(sh[0], sh[1], sh[2], words, scales, tiles, tb);
            d.decode_launch = launch;
            for (int64_t t : token_counts) {
                const int64_t wb = nq_linear_workspace_bytes(&d, t);
                expect(wb >= 0, "workspace bytes", static_cast<int>(wb));
                Buffer ws(static_cast<size_t>(wb > 0 ? wb : 1));
                for (int xd : {NQ_DTYPE_BF16, NQ_DTYPE_F32}) {
                    const int st = nq_linear(&d, x.p, xd, t, y.p, NQ_DTYPE_F32, ws.p, wb, nullptr);
                    expect(launch_refused(st), "linear launch", st);
                }
                const int st2 = nq_linear(&d, x.p, NQ_DTYPE_BF16, t, y.p, NQ_DTYPE_F32, ws.p, wb - 1, nullptr);
                expect(st2 == NQ_ERR_WORKSPACE, "linear short workspace", st2);
            }
        }
    }

    // A batch of the seven Qwen3-8B linears (one call per layer), and the
    // fused one-token forms the decoder uses.
    {
        const int64_t layer[7][3] = {{4096, 4096, 2048}, {4096, 1024, 819}, {4096, 1024, 819}, {4096, 4096, 2048},
                                     {4096, 12288, 3072}, {4096, 12288, 3072}, {12288, 4096, 3072}};
        std::vector<Buffer*> tiles, wss;
        std::vector<nq_linear_desc> descs(7);
        std::vector<const nq_linear_desc*> dp(7);
        std::vector<const void*> xs(7, x.p);
        std::vector<void*> ys(7, y.p), wp(7);
        std::vector<int64_t> wb(7);
        for (int i = 0; i < 7; ++i) {
            const int64_t tb = nq_tiles_bytes(layer[i][0], layer[i][1], layer[i][2]);
            tiles.push_back(new Buffer(static_cast<size_t>(tb)));
            descs[i] = desc_for(layer[i][0], layer[i][1], layer[i][2], words, scales, *tiles.back(), tb);
            dp[i] = &descs[i];
            wb[i] = nq_linear_workspace_bytes(&descs[i], 300);  // the largest token count below
            wss.push_back(new Buffer(static_cast<size_t>(wb[i])));
            wp[i] = wss.back()->p;
        }
        for (int64_t t : token_counts) {
            const int st = nq_linear_batch(dp.data(), 7, xs.data(), NQ_DTYPE_BF16, t, ys.data(), NQ_DTYPE_F32,
                                           wp.data(), wb.data(), nullptr);
            expect(launch_refused(st), "layer batch", st);
        }
        Buffer slots(1 << 16), colscale(1 << 20), residual(1 << 20);
        std::vector<const float*> cs(7, static_cast<const float*>(colscale.p));
        std::vector<const void*> ups(7, residual.p);
        std::vector<float*> res(7, static_cast<float*>(residual.p)), outs(7, static_cast<float*>(slots.p));
        nq_decode_fusion f;
        std::memset(&f, 0, sizeof(f));
        f.input_kind = NQ_INPUT_RMSNORM;
        f.eps = 1e-6f;
        f.col_scales = cs.data();
        f.norm_slots = static_cast<const float*>(slots.p);
        f.norm_slot_count = 256;
        int st = nq_linear_batch_fused(dp.data(), 3, xs.data(), NQ_DTYPE_F32, ys.data(), NQ_DTYPE_F32, wp.data(),
                                       wb.data(), &f, nullptr);
        expect(launch_refused(st), "fused qkv", st);
        f.output_kind = NQ_OUTPUT_SILU_PRODUCT;
        st = nq_linear_batch_fused(dp.data() + 4, 2, xs.data(), NQ_DTYPE_F32, ys.data(), NQ_DTYPE_BF16,
                                   wp.data() + 4, wb.data() + 4, &f, nullptr);
        expect(launch_refused(st), "fused gate/up", st);
        std::memset(&f, 0, sizeof(f));
        f.input_kind = NQ_INPUT_PLAIN;
        f.residuals = res.data();
        f.out_slots = outs.data();
        st = nq_linear_batch_fused(dp.data() + 6, 1, xs.data(), NQ_DTYPE_BF16, ys.data(), NQ_DTYPE_F32,
                                   wp.data() + 6, wb.data() + 6, &f, nullptr);
        expect(launch_refused(st), "fused down", st);
        f.input_kind = NQ_INPUT_SILU_GATE;
        f.ups = ups.data();
        st = nq_linear_batch_fused(dp.data() + 6, 1, xs.data(), NQ_DTYPE_F32, ys.data(), NQ_DTYPE_F32,
                                   wp.data() + 6, wb.data() + 6, &f, nullptr);
        expect(launch_refused(st), "fused gated down", st);
        for (Buffer* b : tiles) delete b;
        for (Buffer* b : wss) delete b;
    }

    // The other entry points, each planned up to its launch with buffers of the
    // sizes it checks (Qwen3-8B geometry where it has one).
    {
        Buffer big(64 << 20), ws(64 << 20), ids(64), pos(64), tok(64), hist(1024), stepb(64), counts(4096);
        int st = nq_embedding(static_cast<const int64_t*>(ids.p), 1, big.p, NQ_DTYPE_BF16, 151936, 4096, nullptr,
                              static_cast<float*>(ws.p), nullptr);
        expect(launch_refused(st), "embedding", st);
        st = nq_embedding_slots(static_cast<const int64_t*>(ids.p), 1, big.p, NQ_DTYPE_BF16, 151936, 4096, nullptr,
                                static_cast<float*>(ws.p), static_cast<float*>(x.p), nullptr);
        expect(launch_refused(st), "embedding slots", st);
        st = nq_embedding_slots(static_cast<const int64_t*>(ids.p), 1, big.p, NQ_DTYPE_BF16, 10, 24, nullptr,
                                static_cast<float*>(ws.p), static_cast<float*>(x.p), nullptr);
        expect(st == NQ_ERR_SHAPE, "embedding slots hidden % 16", st);
        for (int64_t t : {int64_t(1), int64_t(37)}) {
            st = nq_add_rmsnorm(static_cast<float*>(big.p), x.p, NQ_DTYPE_F32, scales.p, NQ_DTYPE_BF16, 1e-6f, t, 4096,
                                y.p, NQ_DTYPE_BF16, nullptr);
            expect(launch_refused(st), "add_rmsnorm", st);
        }
        st = nq_silu_mul(static_cast<const float*>(x.p), static_cast<const float*>(y.p), 12288, ws.p, NQ_DTYPE_BF16,
                         nullptr);
        expect(launch_refused(st), "silu_mul", st);
        const int64_t pw = nq_output_projection_workspace_bytes(151936, 4096);
        st = nq_output_projection(x.p, NQ_DTYPE_F32, big.p, 151936, 4096, static_cast<float*>(y.p), ws.p, pw, nullptr);
        expect(launch_refused(st), "output projection", st);
        st = nq_greedy_select(ws.p, 151936, 4096, static_cast<int64_t*>(tok.p), static_cast<int64_t*>(hist.p), 128,
                              static_cast<int32_t*>(stepb.p), static_cast<int32_t*>(pos.p), nullptr);
        expect(launch_refused(st), "greedy select", st);
        for (int64_t mp : {int64_t(128), int64_t(640), int64_t(1100)}) {
            for (int hd : {64, 128}) {
                const int64_t dw = nq_decode_attention_workspace_bytes(32, 8, hd, NQ_DTYPE_BF16, mp);
                expect(dw > 0, "decode attention workspace", static_cast<int>(dw));
                st = nq_decode_attention(static_cast<const float*>(x.p), static_cast<const float*>(x.p),
                                         static_cast<const float*>(x.p), 32, 8, hd, scales.p, scales.p, NQ_DTYPE_BF16,
                                         1e-6f, static_cast<const float*>(big.p), static_cast<const float*>(big.p),
                                         static_cast<const int32_t*>(pos.p), mp, ws.p, y.p, NQ_DTYPE_BF16, 0.088f,
                                         x.p, NQ_DTYPE_F32, words.p, dw, nullptr);
                expect(launch_refused(st), "decode attention", st);
                st = nq_decode_attention_partials(static_cast<const float*>(x.p), static_cast<const float*>(x.p),
                                                  static_cast<const float*>(x.p), 32, 8, hd, scales.p, scales.p,
                                                  NQ_DTYPE_BF16, 1e-6f, static_cast<const float*>(big.p),
                                                  static_cast<const float*>(big.p), static_cast<const int32_t*>(pos.p),
                                                  mp, ws.p, y.p, NQ_DTYPE_BF16, 0.088f, words.p, dw, nullptr);
                expect(launch_refused(st), "decode attention partials", st);
            }
            for (int64_t t : {int64_t(1), int64_t(17), int64_t(64)}) {
                const int64_t aw = nq_attention_workspace_bytes(t, 32, 128, mp);
                st = nq_qk_norm_rope_cache(static_cast<const float*>(x.p), static_cast<const float*>(x.p),
                                           static_cast<const float*>(x.p), t, 32, 8, 128, scales.p, scales.p,
                                           NQ_DTYPE_BF16, 1e-6f, static_cast<const float*>(big.p),
                                           static_cast<const float*>(big.p), static_cast<const int32_t*>(pos.p), mp,
                                           static_cast<float*>(y.p), ws.p, words.p, NQ_DTYPE_BF16, nullptr);
                expect(launch_refused(st), "qk norm rope cache", st);
                st = nq_attention(static_cast<const float*>(x.p), ws.p, words.p, NQ_DTYPE_BF16, t, 32, 8, 128,
                                  static_cast<const int32_t*>(pos.p), mp, 0.088f, y.p, NQ_DTYPE_BF16, big.p, aw,
                                  nullptr);
                expect(launch_refused(st), "attention", st);
            }
        }
        st = nq_unpack_signs(static_cast<const int32_t*>(words.p), 3072, 819, 26, NQ_DTYPE_BF16, ws.p, nullptr);
        expect(launch_refused(st), "unpack", st);
        st = nq_count_bad_padding(static_cast<const int32_t*>(words.p), 3072, 819, 26,
                                  static_cast<int32_t*>(counts.p), nullptr);
        expect(launch_refused(st), "bad padding", st);
        st = nq_transpose_signs(static_cast<const int32_t*>(words.p), 819, 3072, static_cast<int32_t*>(ws.p),
                                nullptr);
        expect(launch_refused(st) || st == NQ_OK, "transpose signs", st);
        const int64_t tb = nq_tiles_bytes(4096, 1024, 819);
        Buffer tiles(static_cast<size_t>(tb));
        nq_linear_desc d = desc_for(4096, 1024, 819, words, scales, tiles, tb);
        st = nq_prepare_tiles(&d, tiles.p, tb, nullptr);
        expect(launch_refused(st), "prepare tiles", st);
        for (int64_t t : {int64_t(1), int64_t(4), int64_t(16)}) {
            st = nq_linear_static(&d, x.p, NQ_DTYPE_BF16, t, y.p, NQ_DTYPE_F32, nullptr);
            expect(st != NQ_OK, "linear static", st);
        }
        st = nq_decode_mixed_v_words(nullptr, 0, nullptr, 0, nullptr, 819, 4096, nullptr, nullptr, nullptr);
        expect(st != NQ_OK, "mixed-v null", st);
        st = nq_decode_product_codebook_words(nullptr, 0, nullptr, 0, nullptr, nullptr, 819, 4096, nullptr, nullptr);
        expect(st != NQ_OK, "product codebook null", st);
        st = nq_read_stream(big.p, 1 << 20, static_cast<uint32_t*>(counts.p), 64, nullptr);
        expect(launch_refused(st), "read stream", st);
    }

    std::printf("%s: %d failed checks\n", failures ? "FAILED" : "ok", failures);
    return failures ? 1 : 0;
}

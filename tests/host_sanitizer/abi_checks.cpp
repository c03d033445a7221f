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

    std::printf("%s: %d failed checks\n", failures ? "FAILED" : "ok", failures);
    return failures ? 1 : 0;
}

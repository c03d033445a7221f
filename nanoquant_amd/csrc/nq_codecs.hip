// Prepare-time decoders of compact right factors into canonical sign words
// (layout llama.cpp-i32-lsb-v1), and a packed sign-matrix transpose. One
// thread per output word; these run once per layer when it is prepared.
//
//   mixed-V: rows < free_rows are copied; word w of coded row r is record
//     i = (r - free_rows) * words_per_row + w, the 19 bits at bit 19 i of the
//     payload (LSB-first): codebook[i & 1023] ^ (1 << a | 1 << b) where the
//     9-bit pair id enumerates (a, b), a < b < 32, lexicographically. Ids past
//     the 496 pairs are counted in *bad_records and leave the codebook word.
//   product codebook: record i is the 16-bit index at bit 16 i;
//     word = first[i & 255] | second[i >> 8] << 16.
//   transpose: out[c, r / 32] bit r % 32 = in[r, c / 32] bit c % 32, pad bits 0.
#include "nq_common.h"

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMixedPairs = 496;

__device__ __forceinline__ uint32_t record_bits(const uint32_t* __restrict__ payload, int64_t payload_words,
                                                int64_t index, int bits) {
    const int64_t pos = index * bits;
    const int64_t word = pos >> 5;
    const int shift = static_cast<int>(pos & 31);
    uint64_t v = payload[word];
    if (shift + bits > 32 && word + 1 < payload_words) v |= static_cast<uint64_t>(payload[word + 1]) << 32;
    return static_cast<uint32_t>((v >> shift) & ((1ull << bits) - 1));
}

// (a, b) of lexicographic pair id p over 32 positions: the rows before a hold
// 31 + 30 + ... + (32 - a) ids.
__device__ __forceinline__ uint32_t pair_mask(uint32_t p) {
    uint32_t a = 0;
    while (p >= 31u - a) {
        p -= 31u - a;
        ++a;
    }
    const uint32_t b = a + 1u + p;
    return (1u << a) | (1u << b);
}

__global__ __launch_bounds__(kThreads) void k_decode_mixed_v(const uint32_t* __restrict__ free_words, int64_t free_rows,
                                                             const uint32_t* __restrict__ payload, int64_t payload_words,
                                                             const uint32_t* __restrict__ codebook, int64_t rank,
                                                             int64_t words_per_row, uint32_t* __restrict__ out,
                                                             int32_t* __restrict__ bad_records) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= rank * words_per_row) return;
    const int64_t row = i / words_per_row;
    if (row < free_rows) {
        out[i] = free_words[i];
        return;
    }
    const uint32_t rec = record_bits(payload, payload_words, i - free_rows * words_per_row, 19);
    const uint32_t pair = rec >> 10;
    uint32_t word = codebook[rec & 1023u];
    if (pair < kMixedPairs) {
        word ^= pair_mask(pair);
    } else {
        atomicAdd(bad_records, 1);
    }
    out[i] = word;
}

__global__ __launch_bounds__(kThreads) void k_decode_product_codebook(
    const uint32_t* __restrict__ free_words, int64_t free_rows, const uint32_t* __restrict__ payload,
    int64_t payload_words, const uint16_t* __restrict__ first, const uint16_t* __restrict__ second, int64_t rank,
    int64_t words_per_row, uint32_t* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= rank * words_per_row) return;
    if (i / words_per_row < free_rows) {
        out[i] = free_words[i];
        return;
    }
    const uint32_t idx = record_bits(payload, payload_words, i - free_rows * words_per_row, 16);
    out[i] = static_cast<uint32_t>(first[idx & 255u]) | (static_cast<uint32_t>(second[idx >> 8]) << 16);
}

__global__ __launch_bounds__(kThreads) void k_transpose_signs(const uint32_t* __restrict__ in, int64_t rows,
                                                              int64_t cols, uint32_t* __restrict__ out) {
    const int64_t out_wpr = (rows + 31) / 32, in_wpr = (cols + 31) / 32;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= cols * out_wpr) return;
    const int64_t c = i / out_wpr, r0 = (i % out_wpr) * 32;
    uint32_t word = 0;
    for (int b = 0; b < 32 && r0 + b < rows; ++b)
        word |= ((in[(r0 + b) * in_wpr + c / 32] >> (c % 32)) & 1u) << b;
    out[i] = word;
}

__global__ void k_zero_count(int32_t* p) { *p = 0; }

int64_t blocks_for(int64_t n) { return (n + kThreads - 1) / kThreads; }

}  // namespace

extern "C" int nq_decode_mixed_v_words(const int32_t* free_words, int64_t free_rows, const int32_t* payload,
                                       int64_t payload_words, const int32_t* codebook, int64_t rank,
                                       int64_t in_features, int32_t* out_words, int32_t* bad_records, void* stream) {
    if (!payload || !codebook || !out_words || !bad_records || (free_rows > 0 && !free_words)) return NQ_ERR_ARGUMENT;
    const int64_t wpr = nq::words_for(in_features);
    if (rank <= 0 || in_features <= 0 || free_rows < 0 || free_rows >= rank) return NQ_ERR_SHAPE;
    if (payload_words != ((rank - free_rows) * wpr * 19 + 31) / 32) return NQ_ERR_SHAPE;
    const int64_t n = rank * wpr;
    if (blocks_for(n) > 0x7fffffff) return NQ_ERR_SHAPE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_zero_count, dim3(1), dim3(1), 0, st, bad_records);
    hipLaunchKernelGGL(k_decode_mixed_v, dim3(static_cast<unsigned>(blocks_for(n))), dim3(kThreads), 0, st,
                       reinterpret_cast<const uint32_t*>(free_words), free_rows,
                       reinterpret_cast<const uint32_t*>(payload), payload_words,
                       reinterpret_cast<const uint32_t*>(codebook), rank, wpr, reinterpret_cast<uint32_t*>(out_words),
                       bad_records);
    return nq::launch_status();
}

extern "C" int nq_decode_product_codebook_words(const int32_t* free_words, int64_t free_rows, const int32_t* payload,
                                                int64_t payload_words, const int16_t* first_half,
                                                const int16_t* second_half, int64_t rank, int64_t columns,
                                                int32_t* out_words, void* stream) {
    if (!payload || !first_half || !second_half || !out_words || (free_rows > 0 && !free_words))
        return NQ_ERR_ARGUMENT;
    const int64_t wpr = nq::words_for(columns);
    if (rank <= 0 || columns <= 0 || free_rows < 0 || free_rows >= rank) return NQ_ERR_SHAPE;
    if (payload_words != ((rank - free_rows) * wpr * 16 + 31) / 32) return NQ_ERR_SHAPE;
    const int64_t n = rank * wpr;
    if (blocks_for(n) > 0x7fffffff) return NQ_ERR_SHAPE;
    hipLaunchKernelGGL(k_decode_product_codebook, dim3(static_cast<unsigned>(blocks_for(n))), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t*>(free_words), free_rows,
                       reinterpret_cast<const uint32_t*>(payload), payload_words,
                       reinterpret_cast<const uint16_t*>(first_half), reinterpret_cast<const uint16_t*>(second_half),
                       rank, wpr, reinterpret_cast<uint32_t*>(out_words));
    return nq::launch_status();
}

extern "C" int nq_transpose_signs(const int32_t* words, int64_t rows, int64_t cols, int32_t* out_words, void* stream) {
    if (!words || !out_words) return NQ_ERR_ARGUMENT;
    if (rows <= 0 || cols <= 0) return NQ_ERR_SHAPE;
    const int64_t n = cols * nq::words_for(rows);
    if (blocks_for(n) > 0x7fffffff) return NQ_ERR_SHAPE;
    hipLaunchKernelGGL(k_transpose_signs, dim3(static_cast<unsigned>(blocks_for(n))), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t*>(words), rows, cols,
                       reinterpret_cast<uint32_t*>(out_words));
    return nq::launch_status();
}

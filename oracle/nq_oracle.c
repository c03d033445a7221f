/*
 * C restatement of the packed binary low-rank linear — TEST INFRASTRUCTURE ONLY.
 * Only tests/, the smoke check and the bench's CPU-baseline leg load it.
 *
 * Sign words (src/nanoquant/runtime/packed.py:170-218): column c of a row is
 * bit c % 32 of word c / 32, set bit = -1, pad bits 0.
 * Linear (src/nanoquant/runtime/reference.py:208-235), evaluated in double
 * straight from the words, with the salient columns' scale_pre masked to 0
 * (reference.py:101-106) and int8 salient values times their scales
 * (reference.py:93-98).
 */
#include <stdint.h>
#include <stddef.h>

static int64_t nq_words(int64_t cols) { return (cols + 31) / 32; }

static int sign_bit(const int32_t* words, int64_t stride, int64_t r, int64_t c) {
    uint32_t w = (uint32_t)words[r * stride + (c >> 5)];
    return (int)((w >> (c & 31)) & 1u);
}

/* Returns the number of rows with a non-zero pad bit (0 = valid). */
int64_t oracle_bad_padding_rows(const int32_t* words, int64_t rows, int64_t cols) {
    int64_t stride = nq_words(cols), bad = 0;
    int tail = (int)(cols % 32);
    if (tail == 0) return 0;
    for (int64_t r = 0; r < rows; ++r) {
        uint32_t last = (uint32_t)words[r * stride + stride - 1];
        if (last >> tail) ++bad;
    }
    return bad;
}

/* words [rows, ceil(cols/32)] -> signs int8 [rows, cols]; -1 on bad padding. */
int oracle_unpack(const int32_t* words, int64_t rows, int64_t cols, int8_t* signs) {
    if (oracle_bad_padding_rows(words, rows, cols)) return -1;
    int64_t stride = nq_words(cols);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            signs[r * cols + c] = (int8_t)(sign_bit(words, stride, r, c) ? -1 : 1);
    return 0;
}

/* signs int8 ±1 [rows, cols] -> words; pad bits zero. */
void oracle_pack(const int8_t* signs, int64_t rows, int64_t cols, int32_t* words) {
    int64_t stride = nq_words(cols);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t w = 0; w < stride; ++w) {
            uint32_t acc = 0;
            for (int b = 0; b < 32; ++b) {
                int64_t c = w * 32 + b;
                if (c < cols && signs[r * cols + c] < 0) acc |= (1u << b);
            }
            words[r * stride + w] = (int32_t)acc;
        }
    }
}

/*
 * y[t, o] for t < tokens, all operands as double:
 *   lm[r] = s_mid[r] * Σ_i sgn(V[r,i]) * x[t,i] * pre[i]      (pre zero at salient cols)
 *   y     = s_out[o] * Σ_r sgn(U[o,r]) * lm[r] + Σ_k x[t,idx_k] * sal[o,k] + bias[o]
 * sal already includes int8 scales; bias may be NULL; k may be 0.
 * latent_scratch holds `rank` doubles.
 */
void oracle_linear_f64(int64_t in, int64_t out, int64_t rank, const int32_t* left_words,
                       const int32_t* right_words, const double* s_pre, const double* s_mid,
                       const double* s_out, const double* bias, int64_t k, const int32_t* idx,
                       const double* sal, const double* x, int64_t tokens, double* y,
                       double* latent_scratch) {
    int64_t vs = nq_words(in), us = nq_words(rank);
    for (int64_t t = 0; t < tokens; ++t) {
        const double* xt = x + t * in;
        for (int64_t r = 0; r < rank; ++r) {
            double acc = 0.0;
            for (int64_t i = 0; i < in; ++i) {
                int masked = 0;
                for (int64_t s = 0; s < k; ++s) masked |= (idx[s] == i);
                double term = masked ? 0.0 : xt[i] * s_pre[i];
                acc += sign_bit(right_words, vs, r, i) ? -term : term;
            }
            latent_scratch[r] = acc * s_mid[r];
        }
        for (int64_t o = 0; o < out; ++o) {
            double acc = 0.0;
            for (int64_t r = 0; r < rank; ++r)
                acc += sign_bit(left_words, us, o, r) ? -latent_scratch[r] : latent_scratch[r];
            double v = acc * s_out[o];
            for (int64_t s = 0; s < k; ++s) v += xt[idx[s]] * sal[o * k + s];
            if (bias) v += bias[o];
            y[t * out + o] = v;
        }
    }
}

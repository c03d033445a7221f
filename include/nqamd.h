/*
 * nqamd.h — C ABI of the MI355X (gfx950) packed binary low-rank linear.
 *
 *   y = s_out ⊙ (U±1 · (s_mid ⊙ (V±1ᵀ · (s_in ⊙ x))))
 *       + Σ_k x[:, idx_k] · W_sal[:, k] (· scale_k)      salient input columns
 *       + patch_left · (patch_right · x)                  float low-rank patch
 *       + scatter(row_idx, row_scale · (Q_rows · x))      int8 output-row sidecar
 *       + bias
 *
 * U and V are sign matrices in layout llama.cpp-i32-lsb-v1: int32 words, column c
 * in word c/32 at bit c%32, bit set = -1, pad bits 0.
 *
 * Conventions shared by every entry point:
 *   - every pointer argument except `desc` and `out` parameters of the query
 *     functions is a DEVICE pointer owned by the caller;
 *   - `stream` is a hipStream_t passed as void*; kernels are enqueued on it and
 *     nothing synchronises, allocates or frees device memory;
 *   - the return value is an nq_status; nothing throws across the ABI.
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the NanoQuant repository).
 */
#ifndef NQAMD_H
#define NQAMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NQ_ABI_VERSION 3

typedef enum nq_dtype {
    NQ_DTYPE_F32 = 0,
    NQ_DTYPE_F16 = 1,
    NQ_DTYPE_BF16 = 2,
    NQ_DTYPE_I8 = 3,
    NQ_DTYPE_I32 = 4
} nq_dtype;

typedef enum nq_status {
    NQ_OK = 0,
    NQ_ERR_ARGUMENT = -1,    /* null pointer or inconsistent sizes          */
    NQ_ERR_DTYPE = -2,       /* dtype code not accepted for that operand     */
    NQ_ERR_SHAPE = -3,       /* dimension out of the supported range         */
    NQ_ERR_ALIGNMENT = -4,   /* pointer alignment the kernel needs is missing */
    NQ_ERR_WORKSPACE = -5,   /* workspace smaller than nq_linear_workspace_bytes */
    NQ_ERR_LAUNCH = -6,      /* hipLaunchKernel / hipGetLastError failure    */
    NQ_ERR_DEVICE = -7,      /* no HIP device or wrong architecture          */
    NQ_ERR_UNSUPPORTED = -8, /* valid request the library does not implement */
    NQ_ERR_SCRATCH = -9      /* nq_linear_static: the call needs more than
                                NQ_STATIC_SCRATCH_BYTES of workspace         */
} nq_status;

/* Size of the per-device static scratch array of nq_linear_static (4 MiB). */
#define NQ_STATIC_SCRATCH_BYTES (4 << 20)

/* Launch structure of the tiled decode path (tokens <= 16).
 *   NQ_DECODE_SPLIT: two kernels per call (stage 1 writes the rank-r
 *     intermediate, the kernel boundary publishes it, stage 2 reads it).
 *   NQ_DECODE_FUSED: one kernel; stage-2 workgroups wait on a grid-wide
 *     counter in the tiles header that stage-1 workgroups signal.
 * Both give bit-identical results. No reference counterpart (the reference
 * always launches two Triton kernels, cuda_kernels.py:816-874). */
typedef enum nq_decode_launch {
    NQ_DECODE_SPLIT = 0,
    NQ_DECODE_FUSED = 1
} nq_decode_launch;

/* Operands of the prefill path's fp16 MFMA GEMMs (tokens > 16).
 *   NQ_PREFILL_FP16: the row-scaled activations and the rank intermediate
 *     rounded to fp16 (11 bits; about 3e-4 rel-L2 against the fp32 forward).
 *   NQ_PREFILL_FP16_SPLIT: each as an fp16 high part plus an fp16 part of the
 *     remainder (about 22 bits), two MFMAs per product, for callers whose
 *     errors compound (a decoder's prompt pass).
 * Batch members must agree. No reference counterpart (the reference's
 * kernels compute in the activation dtype, cuda_kernels.py:65-162). */
typedef enum nq_prefill_operands {
    NQ_PREFILL_FP16 = 0,
    NQ_PREFILL_FP16_SPLIT = 1
} nq_prefill_operands;

/* Device facts used by the backend's capability check.
 * Replaces the CUDA capability probe of CudaPackedBackend.supports
 * (src/nanoquant/runtime/cuda_backend.py:174-197). */
typedef struct nq_device_caps {
    char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t compute_units;
    int32_t wavefront_size;
    int64_t lds_bytes_per_block;
    int64_t global_mem_bytes;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width_bits;
    int32_t is_gfx950;        /* 1 when the kernels in this library can run */
} nq_device_caps;

/* One packed linear. Sizes are element counts; word rows are contiguous.
 * Replaces the operand list of launch_packed_linear
 * (src/nanoquant/runtime/cuda_kernels.py:816-874) and the payload of
 * CudaPackedBackend (src/nanoquant/runtime/cuda_backend.py:35-48). */
typedef struct nq_linear_desc {
    int64_t in_features;
    int64_t out_features;
    int64_t rank;
    const int32_t* right_words;   /* V: [rank, ceil(in/32)]            */
    const int32_t* left_words;    /* U: [out,  ceil(rank/32)]          */
    const void* scale_pre;        /* [in]   (zero at salient columns)  */
    const void* scale_mid;        /* [rank]                            */
    const void* scale_post;       /* [out]                             */
    int32_t scale_dtype;          /* F32/F16/BF16: scales, salient and row scales */
    int32_t bias_dtype;           /* F32/F16/BF16                      */
    const void* bias;             /* [out] or NULL                     */
    int64_t salient_count;        /* k; 0 when absent                  */
    const int32_t* salient_indices; /* [k] strictly increasing, < in  */
    const void* salient_values;   /* [out, k]                          */
    int32_t salient_dtype;        /* I8/F16/BF16/F32                   */
    const void* salient_scales;   /* [k] (scale_dtype) when I8, else NULL */
    int64_t patch_rank;           /* p; 0 when absent                  */
    const void* patch_left;       /* [out, p]                          */
    const void* patch_right;      /* [p, in]                           */
    int32_t patch_dtype;          /* F32/F16/BF16                      */
    int64_t row_count;            /* output-row sidecar rows; 0 when absent */
    const int32_t* row_indices;   /* [row_count] strictly increasing, < out */
    const int8_t* row_values;     /* [row_count, in]                   */
    const void* row_scales;       /* [row_count] (scale_dtype)         */
    const void* tiles;            /* GPU layout from nq_prepare_tiles, or NULL */
    int64_t tiles_bytes;
    int32_t decode_launch;        /* nq_decode_launch; batch members must agree */
    int32_t prefill_operands;     /* nq_prefill_operands; batch members must agree */
} nq_linear_desc;

/* Library ABI version (NQ_ABI_VERSION). No reference counterpart. */
int nq_abi_version(void);

/* Human-readable text for a status code. No reference counterpart. */
const char* nq_status_string(int status);

/* Device query; see nq_device_caps. */
int nq_query_device(int device, nq_device_caps* out);

/* Bit-exact unpack of sign words to dense ±1 in F32/F16/BF16, row-major
 * [rows, cols]. Replaces unpack_sign_matrix
 * (src/nanoquant/runtime/packed.py:204-218) for device tensors. */
int nq_unpack_signs(const int32_t* words, int64_t rows, int64_t cols,
                    int64_t row_stride_words, int32_t out_dtype, void* out,
                    void* stream);

/* Count rows whose pad bits (columns >= cols in the last word) are non-zero;
 * writes one int32 to *bad_rows (device). Device form of the padding check in
 * _validate_packed_matrix (src/nanoquant/runtime/packed.py:189-201). */
int nq_count_bad_padding(const int32_t* words, int64_t rows, int64_t cols,
                         int64_t row_stride_words, int32_t* bad_rows, void* stream);

/* Bytes of the synchronisation header at the start of a tiles buffer. It holds
 * the fused launch's monotonic counters (never reset; graph replays are safe)
 * and, on its last 256-byte line, word 0 = sticky error flag (set if a fused
 * decode launch ever timed out waiting for its stage-1 results; the outputs of
 * the workgroups that timed out are NaN), word 1 = magic 0x4E515433, word 2 =
 * max|s_mid| as fp32 bits (bounds the stage-1 results so the decode epilogue
 * can pick their fixed-point exponent), word 3 = the fused launch's spin
 * limit (polls of the stage-1 signal before giving up; 2^22 from
 * nq_prepare_tiles, a caller may lower it). The
 * header is per layer: launches that use one prepared layer must not overlap
 * in time (one stream, or ordered streams). No reference counterpart. */
int64_t nq_tiles_header_bytes(void);

/* Prepare-time expansion of a mixed-V compact right factor
 * (mixed-v-free-k10-pair9-v1) to canonical words out_words[rank, ceil(in/32)]:
 * rows < free_rows copy free_words; every other word is one 19-bit record of
 * the LSB-first payload (payload_words = ceil(records * 19 / 32)),
 * codebook[index] with the two bits of its pair id flipped (ids enumerate
 * bit pairs a < b < 32 in lexicographic order). *bad_records (device) is set
 * to the count of ids past the 496 pairs. Replaces
 * launch_decode_mixed_v_right_words
 * (src/nanoquant/runtime/cuda_kernels.py:11-62,877-906). */
int nq_decode_mixed_v_words(const int32_t* free_words, int64_t free_rows, const int32_t* payload,
                            int64_t payload_words, const int32_t* codebook, int64_t rank,
                            int64_t in_features, int32_t* out_words, int32_t* bad_records,
                            void* stream);

/* Prepare-time expansion of a product-codebook right factor
 * (product-codebook-free-k16-v1): coded word = first_half[i & 255] |
 * second_half[i >> 8] << 16 for the 16-bit index i of its record
 * (payload_words = ceil(records / 2)). Device form of
 * decode_product_codebook_right_words
 * (src/nanoquant/runtime/product_codebook.py:102-128). */
int nq_decode_product_codebook_words(const int32_t* free_words, int64_t free_rows,
                                     const int32_t* payload, int64_t payload_words,
                                     const int16_t* first_half, const int16_t* second_half,
                                     int64_t rank, int64_t columns, int32_t* out_words,
                                     void* stream);

/* Packed sign-matrix transpose: out_words[cols, ceil(rows/32)] of the matrix
 * words[rows, ceil(cols/32)] transposed (pad bits zero). Device form of the
 * transposed-factorization conversion
 * (src/nanoquant/runtime/product_codebook.py:232-250). */
int nq_transpose_signs(const int32_t* words, int64_t rows, int64_t cols, int32_t* out_words,
                       void* stream);

/* Size in bytes of the GPU-private tiled weight layout for one linear:
 * header, V tiles, U tiles and 256 bytes of tail padding (the decode kernels
 * read whole 16-byte words per lane from clamped addresses). */
int64_t nq_tiles_bytes(int64_t in_features, int64_t out_features, int64_t rank);

/* Re-tile the canonical U and V words of `desc` into the GPU-private decode
 * layout at `tiles` (nq_tiles_bytes bytes). Prepare-time; replaces the
 * one-time device copy in CudaPackedBackend.prepare
 * (src/nanoquant/runtime/cuda_backend.py:199-241). */
int nq_prepare_tiles(const nq_linear_desc* desc, void* tiles, int64_t tiles_bytes,
                     void* stream);

/* Workspace bytes nq_linear needs for `tokens` token slots. */
int64_t nq_linear_workspace_bytes(const nq_linear_desc* desc, int64_t tokens);

/* y[tokens, out] = linear(x[tokens, in]). x dtype F32/F16/BF16; y dtype F32
 * (the reference backend's output) or BF16/F16. Decode kernels for
 * tokens <= 16, the MFMA prefill kernel above. Replaces launch_packed_linear
 * (src/nanoquant/runtime/cuda_kernels.py:816-874) and CudaPackedBackend.linear
 * (src/nanoquant/runtime/cuda_backend.py:243-278). */
int nq_linear(const nq_linear_desc* desc, const void* x, int32_t x_dtype,
              int64_t tokens, void* y, int32_t y_dtype, void* workspace,
              int64_t workspace_bytes, void* stream);

/* nq_linear without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation). No reference counterpart. The workspace is a
 * file-scope device array of NQ_STATIC_SCRATCH_BYTES per GPU, held until the
 * process ends; calls whose nq_linear_workspace_bytes exceeds it return
 * NQ_ERR_SCRATCH (decode token counts fit any Qwen3/Llama-sized layer;
 * larger prefill calls need nq_linear). Allocates nothing itself. All calls
 * on one GPU share the array: calls that overlap in time on one GPU race and
 * must not be issued (one stream, or streams ordered by the caller). */
int nq_linear_static(const nq_linear_desc* desc, const void* x, int32_t x_dtype,
                     int64_t tokens, void* y, int32_t y_dtype, void* stream);

/* Read `bytes` (a multiple of 16, 16-byte aligned) of device memory with the
 * decode kernels' load pattern and write, for each of min(sink_count,
 * ceil(bytes / 16384)) workgroups, the XOR of the 32-bit words it read to
 * sink[workgroup]. No reference counterpart: a measurement aid, the HBM read
 * ceiling the decode path is compared with. */
int nq_read_stream(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_count, void* stream);

/* One launch per kernel phase for `count` (1..8) packed linears with the same
 * token count and dtypes: y_i = linear_i(x_i). Up to 16 tokens the members
 * share the decode kernels' launches (no two descriptors may then share
 * tiles); above 16, the prefill row pass, both sign GEMMs and their split-K
 * reductions each take one launch for all members. Inputs may alias (Q/K/V
 * or gate/up share x); every descriptor must carry tiles.
 * workspaces[i] holds nq_linear_workspace_bytes(descs[i], tokens) bytes.
 * Replaces launch_grouped_packed_linears / grouped_cuda_projection
 * (src/nanoquant/runtime/cuda_kernels.py:301-374,
 * src/nanoquant/runtime/cuda_backend.py:123-144), generalised to distinct
 * inputs, any rank (no multiple-of-8 limit) and sidecars. */
int nq_linear_batch(const nq_linear_desc* const* descs, int32_t count, const void* const* xs,
                    int32_t x_dtype, int64_t tokens, void* const* ys, int32_t y_dtype,
                    void* const* workspaces, const int64_t* workspace_bytes, void* stream);

/* Input forms of a fused one-token decode call (nq_linear_batch_fused). */
typedef enum nq_input_kind {
    NQ_INPUT_PLAIN = 0,     /* x as in nq_linear_batch                                */
    NQ_INPUT_RMSNORM = 1,   /* x is an fp32 residual h [in]; member i sees RMSNorm(h) * w
                               through col_scales[i] = w * s_in (fp32 [in], replacing
                               its s_in) and 1 / RMS(h) from norm_slots               */
    NQ_INPUT_SILU_GATE = 2, /* x is the fp32 gate g [in], ups[i] the fp32 up u [in];
                               member i sees silu(g) * u                              */
    NQ_INPUT_ATTENTION = 3  /* x is the workspace of nq_decode_attention_partials
                               (include/nqamd_shell.h) for a cache of
                               attn_max_positions rows (at most 1024); input column k
                               is dimension k % attn_head_dim of head k / attn_head_dim
                               of the attention output, merged from the partials of
                               the blocks up to *attn_position; in_features = heads *
                               attn_head_dim <= 4096, heads * blocks even          */
} nq_input_kind;

/* Output forms of a fused one-token decode call (nq_linear_batch_fused). */
typedef enum nq_output_kind {
    NQ_OUTPUT_PLAIN = 0,        /* each member writes its y (or adds it to its residual) */
    NQ_OUTPUT_SILU_PRODUCT = 1  /* exactly two members of equal out and rank, no salient
                                   columns, bias, patch, row sidecar or residuals: ys[0]
                                   receives silu(y_0) * y_1 in y_dtype (ys[1] unused);
                                   the SiLU-gated MLP input of the next projection */
} nq_output_kind;

/* Decoder fusions around the packed linears of one decode token. */
typedef struct nq_decode_fusion {
    int32_t input_kind;              /* nq_input_kind                                   */
    float eps;                       /* RMSNORM: epsilon of the norm                    */
    const float* const* col_scales;  /* RMSNORM: [count] fp32 [in] column scales        */
    const float* norm_slots;         /* RMSNORM: sums of h^2 per 16-row tile of h, as
                                        written by a residual epilogue (out_slots)     */
    int64_t norm_slot_count;         /* RMSNORM: ceil(in / 16), a multiple of 4, <= 1024 */
    const void* const* ups;          /* SILU_GATE: [count] fp32 [in]                     */
    float* const* residuals;         /* NULL, or [count]: member i adds its output to
                                        residuals[i] (fp32 [out]) instead of writing y  */
    float* const* out_slots;         /* with residuals: [count] fp32 [ceil(out / 16)]
                                        sums of the new residual's squares per tile     */
    int32_t output_kind;             /* nq_output_kind                                  */
    const int32_t* attn_position;    /* ATTENTION: the token's cache row (device)       */
    int32_t attn_head_dim;           /* ATTENTION: 64, 128 or 256                       */
    int64_t attn_max_positions;      /* ATTENTION: rows of the cache                    */
} nq_decode_fusion;

/* One launch pair for `count` (1..8) packed linears of ONE token with the
 * decoder's neighbouring element-wise work fused in: the input RMSNorm (the
 * factor 1 / RMS(h) is applied to the rank intermediate, the weight is folded
 * into the column scale), the SiLU-gated product or the merge of the decode
 * attention's partial results (the attention's second pass), and the residual add of
 * the output with the per-tile sums of squares the next RMSNorm input needs.
 * x_dtype is F32 for every input but PLAIN; scales fp16; ys[i] may be
 * NULL with residuals; no patch or row sidecar, and no salient columns with a
 * non-plain input. Workspaces as for nq_linear_batch with tokens = 1.
 * No reference counterpart: the reference decoder runs the norms,
 * act_fn(gate) * up and the residual adds as separate torch operations around
 * its packed linears (src/nanoquant/runtime/torch_model.py:493-505 MLP,
 * :625-660 decoder layer; CudaPackedBackend.linear,
 * src/nanoquant/runtime/cuda_backend.py:243-278). */
int nq_linear_batch_fused(const nq_linear_desc* const* descs, int32_t count, const void* const* xs,
                          int32_t x_dtype, void* const* ys, int32_t y_dtype, void* const* workspaces,
                          const int64_t* workspace_bytes, const nq_decode_fusion* fusion, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NQAMD_H */

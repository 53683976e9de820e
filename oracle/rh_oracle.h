/*
 * rh_oracle.h -- CPU restatement of rusticide's quantized matrix-product
 * arithmetic. TEST INFRASTRUCTURE ONLY: this library is the checker that the
 * HIP path is compared against (and the CPU baseline timed beside it). The
 * product (rusticide_amd / librusticide_hip.so) never links or calls it.
 *
 * Every function names the reference file:line it restates. Paths are
 * relative to the rusticide repository root.
 */
#ifndef RH_ORACLE_H
#define RH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Q8Kind (crates/rusticide-kernels/src/q8_input.rs:33-50). Block (ggml Q8_0)
 * is out of scope: no format on this path pairs with it. */
enum { ORC_Q8_SUPER_BLOCK = 1, ORC_Q8_ROW = 2 };

/* Weights (crates/rusticide-kernels/src/matmul.rs:28-46). */
enum { ORC_DENSE = 0, ORC_BLOCKS = 1, ORC_TERNARY = 2 };

typedef struct {
    uint32_t kind;      /* ORC_DENSE / ORC_BLOCKS / ORC_TERNARY            */
    uint32_t type_id;   /* GGML type id for ORC_BLOCKS (12 Q4_K, 14 Q6_K)  */
    const void *data;   /* f32 rows (dense) or block bytes                 */
    size_t data_len;    /* elements (dense) or bytes                       */
    size_t width;       /* cols (dense) or row_bytes                       */
    float scale;        /* I2_S tensor scale (ternary)                     */
    float *out;         /* out[row * tokens + token]                       */
    size_t out_len;
} orc_job;

/* format.rs:31-92 / format.rs:102-104: 0 when unknown. */
int orc_block_format(uint32_t type_id, size_t *block_size, size_t *block_bytes,
                     size_t *trailer_bytes);
/* format.rs:151-165 (byte_len) and :193-198 (row_bytes); SIZE_MAX = None. */
size_t orc_byte_len(uint32_t type_id, size_t numel);
size_t orc_row_bytes(uint32_t type_id, size_t cols);

/* half_bits.rs:16-18 (half 2.7.1 f16::to_f32): exact widening. */
float orc_f16_to_f32(uint16_t bits);
/* half 2.7.1 f16::from_f32 (format.rs:210): round to nearest even. */
uint16_t orc_f32_to_f16(float value);

/* format.rs:219-226 with q4_k.rs:38-66, q6_k.rs:13-43, i2_s.rs:15-21. */
void orc_dequantize_row(uint32_t type_id, const uint8_t *row, size_t row_len,
                        float *out, size_t out_len);
/* i2_s.rs:26-30: little-endian f32 opening the trailer; 0 if too short. */
int orc_i2s_scale(const uint8_t *trailer, size_t len, float *scale);

/* Generators: format.rs:109-117, format.rs:204-214,
 * kernels/src/test_support.rs:72-92, bench/src/kernels.rs:27-35. */
void orc_pseudo_random_bytes(uint8_t *out, size_t len, uint32_t seed);
int orc_synthetic_blocks(uint32_t type_id, size_t blocks, uint32_t seed, uint8_t *out);
void orc_pseudo_random_values(float *out, size_t len, uint32_t seed);
void orc_bench_activations(float *out, size_t len, uint32_t seed);

/* portable/q8.rs:64-106: returns the number of 32-element blocks written. */
size_t orc_quantize(int kind, const float *x, size_t len, int8_t *quants,
                    float *scales, int32_t *sums);
/* q8_input.rs:72-93. */
void orc_q8_dequantize(int kind, const int8_t *quants, const float *scales,
                       size_t n_blocks, float *out);

/* portable/int_dot.rs:145-171 and :181-204 (dot_row, :36-47). */
float orc_q4k_dot(const uint8_t *row, size_t row_len, const int8_t *quants,
                  const float *scales, const int32_t *sums, size_t n_blocks);
float orc_q6k_dot(const uint8_t *row, size_t row_len, const int8_t *quants,
                  const float *scales, const int32_t *sums, size_t n_blocks);
/* portable/ternary.rs:21-42 (wrapping i32) and :48-58. */
int32_t orc_ternary_dot(const uint8_t *row, size_t row_len, const int8_t *quants,
                        const int32_t *sums, size_t n_blocks);
float orc_ternary_product(const uint8_t *row, size_t row_len, const int8_t *quants,
                          const float *scales, const int32_t *sums, size_t n_blocks,
                          float scale);
/* rusticide-simd/src/float.rs:23-36. */
float orc_dot_f32(const float *lhs, size_t lhs_len, const float *rhs, size_t rhs_len);

/* Dequantize-and-dot: quant_kernel_tests.rs:29-31,60-79 (sequential f32 sum
 * of dequantized weights x the given activation values). */
float orc_dequant_dot(uint32_t type_id, const uint8_t *row, size_t row_len,
                      const float *x, size_t x_len);

/* matmul.rs:229-248 (matmul_batch), rows split into threads*16 runs.
 * threads <= 0 picks 1. */
void orc_matmul_batch(const float *inputs, size_t inputs_len, size_t tokens,
                      const orc_job *jobs, size_t n_jobs, int threads);

/* Raw i32 accumulators of an I2_S matrix against Row-quantized tokens:
 * out[row * tokens + token] = ternary_dot(row, token). */
void orc_ternary_dot_matrix_i32(const uint8_t *data, size_t data_len, size_t row_bytes,
                                const float *inputs, size_t inputs_len, size_t tokens,
                                int32_t *out, size_t out_len);

/* ------------------------------------------- the avx2 adapter (rh_avx2.c)
 * The reference's x86 Q4_K / Q6_K kernels (crates/rusticide-simd/src/avx2/
 * {q4_k,q6_k}/vector.rs) over its eight-row units (group/{q4_k,q6_k}.rs),
 * for the CPU baseline. prepare: NULL unless the CPU has avx2 and fma, the
 * format is Q4_K / Q6_K and rows is a multiple of 8. matvec: one token
 * (Q8_K-quantized here) against every row, threads workers; 0 when the
 * activation holds the quant -128 (the reference then keeps the portable
 * kernel), else 1. */
typedef struct orc_avx2_matrix orc_avx2_matrix;
int orc_avx2_available(void);
orc_avx2_matrix *orc_avx2_prepare(uint32_t type_id, const uint8_t *data, size_t rows, size_t row_bytes);
void orc_avx2_free(orc_avx2_matrix *m);
int orc_avx2_matvec(const orc_avx2_matrix *m, const float *x, size_t len, float *out, size_t out_len, int threads);

/* ------------------------------------------------------------- decoder */

/* DecoderConfig (crates/rusticide-transformer/src/config.rs:19-33), llama
 * family: adjacent RoPE, SiLU, no biases or sub-norms. */
typedef struct {
    size_t embedding_length, block_count, feed_forward_length, head_count, head_count_kv, head_dim;
    size_t context_length, vocab_size;
    float rope_freq_base, rms_norm_eps;
} orc_decoder_config;

/* A weight matrix as Matrix holds it (model/src/weights.rs:17-38): GGML
 * type id (0 = f32 rows) and its row-major bytes. */
typedef struct {
    uint32_t type_id;
    const uint8_t *data;
    size_t rows, cols;
} orc_matrix;

/* BlockWeights / DecoderWeights (transformer/src/weights.rs); output NULL
 * is tied to token_embd. */
typedef struct {
    const float *attn_norm;
    orc_matrix attn_q, attn_k, attn_v, attn_output;
    const float *ffn_norm;
    orc_matrix ffn_gate, ffn_up, ffn_down;
} orc_block;

typedef struct {
    orc_matrix token_embd;
    const float *output_norm;
    const orc_matrix *output;
    const orc_block *blocks;
} orc_decoder_weights;

typedef struct orc_decoder orc_decoder;

/* Errors (ModelError / SamplingError kinds). */
enum {
    ORC_DEC_NO_TOKENS = 1,       /* InvalidConfig "no tokens to forward"   */
    ORC_DEC_CONTEXT_FULL = 2,    /* ContextFull                            */
    ORC_DEC_TOKEN_RANGE = 3,     /* InvalidConfig "token out of range"     */
    ORC_DEC_CACHE_POSITION = 4,  /* CachePosition                          */
    ORC_DEC_NO_VALID_TOKENS = 5, /* SamplingError::NoValidTokens           */
    ORC_DEC_NO_MEMORY = 6
};

orc_decoder *orc_decoder_new(const orc_decoder_config *c, const orc_decoder_weights *w, int threads);
void orc_decoder_free(orc_decoder *d);
/* Model::reset (cache.rs:79-83). */
void orc_decoder_reset(orc_decoder *d);
/* Model::forward_batch (transformer/src/decoder.rs:57-107): logits
 * [vocab_size] of the last token. */
int orc_decoder_forward_batch(orc_decoder *d, const uint32_t *tokens, size_t n, size_t start, float *logits);
/* Sampler::greedy_logits (sampling/src/sampler.rs:75-87). */
int orc_greedy(const float *logits, size_t n, uint32_t *token);
/* generate (model/src/generate.rs:35-124) at temperature 0. */
int orc_generate_greedy(orc_decoder *d, const uint32_t *prompt, size_t n, size_t max_tokens, uint32_t *out,
                        size_t *n_out);
/* The f32 pieces, exposed for their known-answer tests. */
void orc_normalize(const float *in, const float *weight, size_t n, float eps, float *out);
void orc_softmax(float *row, size_t n);
void orc_rope_adjacent(float *row, size_t len, size_t position, float theta, size_t dim_pairs);
void orc_rope_table(size_t positions, size_t columns, float theta, float *cos_out, float *sin_out);
void orc_expf_array(const float *x, float *y, size_t n);
void orc_silu_array(const float *x, float *y, size_t n);
void orc_dot_rows(const float *query, size_t qlen, const float *rows, size_t nrows, size_t stride, size_t offset,
                  float scale, float *out);
void orc_mix_rows(const float *weights, size_t nw, const float *rows, size_t nrows, size_t stride, size_t offset,
                  float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif

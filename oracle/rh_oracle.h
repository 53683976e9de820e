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

/* Q8Kind (crates/rusticide-kernels/src/q8_input.rs:86-100). Block (ggml Q8_0)
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

/* format.rs:219-226 with q4_k.rs:38-66, q6_k.rs:205-216, i2_s.rs:15-21. */
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
/* q8_input.rs:125-142. */
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

#ifdef __cplusplus
}
#endif
#endif

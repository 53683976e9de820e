/*
 * rusticide_hip.h -- C ABI of the MI355X (gfx950) quantized matrix-product
 * path: Q4_K / Q6_K / I2_S weights resident in HBM in their GGUF block
 * layouts, multiplied by f32 activations that are quantized on the device
 * exactly as rusticide's CPU kernels quantize them.
 *
 * The ABI is what a thin Rust crate (`rusticide-hip`) binds over FFI; each
 * entry point names the rusticide interface it stands in for (paths relative
 * to the rusticide repository root). Plain pointers and sizes only; no C++
 * exceptions cross it. A context owns one HIP stream and is externally
 * synchronized: calls on one context must not overlap.
 */
#ifndef RUSTICIDE_HIP_H
#define RUSTICIDE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. They mirror the error kinds of ModelError
 * (crates/rusticide-model/src/error.rs:11-44) and DispatchError
 * (crates/rusticide-dispatch/src/error.rs:7-21). */
typedef enum rh_status {
    RH_OK = 0,
    RH_ERR_INVALID_ARGUMENT = 1, /* null pointer, unknown kind, bad length  */
    RH_ERR_MISSING_KERNEL = 2,   /* ModelError::MissingKernel              */
    RH_ERR_INVALID_TENSOR = 3,   /* ModelError::InvalidTensor (I2_S scale)  */
    RH_ERR_SHAPE_MISMATCH = 4,   /* data too short for rows x cols          */
    RH_ERR_INVALID_CONFIG = 5,   /* ModelError::InvalidConfig (cols == 0)  */
    RH_ERR_DEVICE = 6,           /* a HIP runtime error; see rh_last_error  */
    RH_ERR_OUT_OF_MEMORY = 7,
    RH_ERR_NO_DEVICE = 8,        /* no gfx950 device: the caller falls back */
    RH_ERR_CONTEXT_FULL = 9,     /* ModelError::ContextFull                */
    RH_ERR_CACHE_POSITION = 10,  /* ModelError::CachePosition              */
    RH_ERR_NO_VALID_TOKENS = 11, /* SamplingError::NoValidTokens           */
    RH_ERR_GGUF = 12,            /* GgufError: rh_gguf_error says which     */
    RH_ERR_MISSING_METADATA = 13, /* ModelError::MissingMetadata            */
    RH_ERR_MISSING_TENSOR = 14,  /* ModelError::MissingTensor               */
    RH_ERR_UNKNOWN_ARCHITECTURE = 15 /* ModelError::UnknownArchitecture    */
} rh_status;

/* GGML type ids (crates/rusticide-quantize/src/format.rs:31-92), plus the
 * dense widths Matrix::load accepts (crates/rusticide-model/src/weights.rs:241-247). */
enum {
    RH_TYPE_F32 = 0,
    RH_TYPE_F16 = 1,
    RH_TYPE_Q4_K = 12,
    RH_TYPE_Q6_K = 14,
    RH_TYPE_I2_S = 36
};

/* Q8Kind (crates/rusticide-kernels/src/q8_input.rs:33-50). */
enum { RH_Q8_SUPER_BLOCK = 1, RH_Q8_ROW = 2 };

typedef struct rh_ctx rh_ctx;
typedef struct rh_matrix rh_matrix;

/* One entry of a batch: a matrix and the output it fills,
 * out[row * tokens + token]; out_len bounds what is written. The
 * (Weights, &mut [f32]) pair of matmul_batch
 * (crates/rusticide-kernels/src/matmul.rs:229). */
typedef struct rh_job {
    const rh_matrix *weights;
    float *out;
    size_t out_len;
} rh_job;

/* Opens device `device` and a stream on it. Stands in for the process-wide
 * adapter selection `active()` (crates/rusticide-kernels/src/adapter.rs:86-169):
 * RH_ERR_NO_DEVICE tells the caller to keep the CPU adapter. */
rh_status rh_init(int device, rh_ctx **out);
void rh_destroy(rh_ctx *ctx);
/* The message of the last failed call on this context ("" if none); with
 * NULL, of the last failed call this thread made without a context. */
const char *rh_last_error(const rh_ctx *ctx);
/* Adapter name, as `Adapter::name` (adapter.rs:40-45): "hip-gfx950". */
const char *rh_adapter_name(void);
/* The context's HIP stream (a hipStream_t), for rh_matmul_batch_device. */
void *rh_stream(rh_ctx *ctx);

/* Matrix::load_on (crates/rusticide-model/src/weights.rs:53-98) + the upload:
 * validates `len` against rows x cols for `type_id`, copies the blocks to
 * HBM once and for I2_S parses and validates the trailer scale
 * (weights.rs:190-202). F16 is widened to f32 as `widen` does
 * (weights.rs:241-247). I2_S and f32 rows sit at a 16-byte stride; Q4_K and
 * Q6_K blocks are regrouped on the host during the upload into groups of 16
 * consecutive blocks laid out the way the kernels' waves read them (the
 * same bytes, one copy; the in-place repack of Adapter::prepare_matrix,
 * crates/rusticide-kernels/src/adapter.rs:70-83). */
rh_status rh_matrix_load(rh_ctx *ctx, uint32_t type_id, const void *data, size_t len,
                         size_t rows, size_t cols, rh_matrix **out);
/* Frees the matrix; valid before or after its context is destroyed. */
void rh_matrix_free(rh_matrix *m);
size_t rh_matrix_rows(const rh_matrix *m);
size_t rh_matrix_cols(const rh_matrix *m);
uint32_t rh_matrix_type(const rh_matrix *m);
/* Weights::Ternary::scale (matmul.rs:41-45); 0 for other formats. */
float rh_matrix_ternary_scale(const rh_matrix *m);
/* Bytes of HBM the matrix occupies: its blocks (Q4_K / Q6_K rounded up to
 * whole groups of 16), plus 256 bytes of slack rounded to 256. */
size_t rh_matrix_device_bytes(const rh_matrix *m);

/* Matrix::copy_row (weights.rs:120-150): dequantizes row `index` into the
 * host buffer `out` (at most out_len values; I2_S rows are scaled by the
 * tensor scale). *found = 0 when the row does not exist. */
rh_status rh_matrix_copy_row(rh_ctx *ctx, const rh_matrix *m, size_t index, float *out,
                             size_t out_len, int *found);

/* matmul_batch (crates/rusticide-kernels/src/matmul.rs:229-248) on host
 * buffers: `inputs` holds `tokens` rows of inputs_len / tokens values; each
 * job's output gets out[row * tokens + token], bit-identical to a
 * rh_matvec_batch of that token alone. No-op when tokens == 0 or
 * tokens > inputs_len. Synchronous. */
rh_status rh_matmul_batch(rh_ctx *ctx, const float *inputs, size_t inputs_len, size_t tokens,
                          const rh_job *jobs, size_t n_jobs);
/* matvec_batch (matmul.rs:218-220). */
rh_status rh_matvec_batch(rh_ctx *ctx, const float *input, size_t len, const rh_job *jobs,
                          size_t n_jobs);
/* The device-resident form: `inputs` and every job's `out` are device
 * pointers; the work is queued on `stream` (a hipStream_t; NULL = the
 * context's stream) and the call returns without waiting. */
rh_status rh_matmul_batch_device(rh_ctx *ctx, const float *inputs, size_t inputs_len,
                                 size_t tokens, const rh_job *jobs, size_t n_jobs, void *stream);
/* No counterpart in the reference: rh_matmul_batch_device for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). It computes the same outputs,
 * bit for bit, and allocates nothing: the batch's quantized activations go
 * to a file-scope array of RH_NOALLOC_SCRATCH_BYTES on each GPU, whose
 * address rh_init looks up once per device, and K-split GEMMs run unsplit.
 * A batch whose quantized activations would not fit is refused with
 * RH_ERR_INVALID_ARGUMENT. They take, with W = width rounded up to a
 * multiple of 256 (at least 256), B = W / 32 rounded up to a multiple of 8
 * and r(n) = n rounded up to a multiple of 256:
 * 2 * r(tokens * W) + 6 * r(tokens * B * 4) bytes, about
 * 2.75 * tokens * width (4096 tokens x 256 values, or 1489 x 1024, fit). Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other contexts, other
 * threads) race, and must be ordered by the caller. */
enum { RH_NOALLOC_SCRATCH_BYTES = 4 << 20 };
rh_status rh_matmul_batch_device_noalloc(rh_ctx *ctx, const float *inputs, size_t inputs_len, size_t tokens,
                                         const rh_job *jobs, size_t n_jobs, void *stream);

/* A quantized activation batch on the device: Q8Input
 * (crates/rusticide-kernels/src/q8_input.rs:13-23), one per token. */
typedef struct rh_q8 rh_q8;
rh_status rh_q8_new(rh_ctx *ctx, rh_q8 **out);
void rh_q8_free(rh_q8 *q);
/* Q8Input::quantize (q8_input.rs:52-58) of every token of `inputs`, a
 * device pointer holding `tokens` rows of inputs_len / tokens values. Queued
 * on `stream` (NULL = the context's stream). */
rh_status rh_q8_quantize_device(rh_ctx *ctx, rh_q8 *q, int kind, const float *inputs,
                                size_t inputs_len, size_t tokens, void *stream);
/* QuantKernel::dot_matrix (crates/rusticide-kernels/src/quant_kernel.rs:106-119)
 * and dot_ternary_matrix (portable/ternary.rs:66-82): every row of `m`
 * against every token of `q` into the device buffer out[row * tokens + token].
 * `q` must hold the kind the matrix pairs with (SUPER_BLOCK for Q4_K/Q6_K,
 * ROW for I2_S). Queued on `stream`. */
rh_status rh_dot_matrix_device(rh_ctx *ctx, const rh_matrix *m, const rh_q8 *q, float *out,
                               size_t out_len, void *stream);

/* Test hook: Q8Input::quantize (q8_input.rs:52-58, portable/q8.rs:64-106)
 * on the device, for one row of `len` host values. Writes n_blocks =
 * whole 32-blocks (whole 256-blocks for SUPER_BLOCK) quants, scales, sums. */
rh_status rh_quantize(rh_ctx *ctx, int kind, const float *x, size_t len, int8_t *quants,
                      float *scales, int32_t *sums, size_t *n_blocks);

/* Test hook: the raw i32 accumulators of an I2_S matrix
 * (portable/ternary.rs:21-42) against Row-quantized tokens,
 * out[row * tokens + token], for the bit-exact check. */
rh_status rh_ternary_dot_i32(rh_ctx *ctx, const rh_matrix *m, const float *inputs,
                             size_t inputs_len, size_t tokens, int32_t *out, size_t out_len);

/* Token count from which rh_matmul_batch* run Q4_K, Q6_K and I2_S matrices on
 * the MFMA GEMMs instead of the GEMV kernels (both give the same bits); 9 by
 * default.
 * Process-wide. No counterpart in the reference (its row kernels serve every
 * batch size, crates/rusticide-kernels/src/matmul.rs:229-248). */
size_t rh_gemm_min_tokens(void);
void rh_set_gemm_min_tokens(size_t tokens);

/* Test hooks for the float functions of the decoder kernels, none of which
 * has a counterpart in the reference; they pin the kernels to the libm and
 * IEEE operations behind rusticide's f32 code:
 *   expf: the bits of the libm expf behind f32::exp (softmax, SiLU;
 *         crates/rusticide-kernels/src/portable/{norm.rs:17-30,elementwise.rs:6-9});
 *   sqrt: f32::sqrt, rounded to nearest (RMSNorm,
 *         crates/rusticide-kernels/src/portable/norm.rs:8-14);
 *   div:  f32 division, rounded to nearest.
 * rh_sqrt_host runs the device's correction from the given starts (which must
 * lie within one ulp of the result), or from the host's sqrt when start is
 * NULL. rh_math_device evaluates one function elementwise on the device
 * (b is read by RH_MATH_DIV only). */
enum { RH_MATH_EXPF = 0, RH_MATH_SQRT = 1, RH_MATH_DIV = 2 };
void rh_expf_host(const float *x, float *y, size_t n);
void rh_sqrt_host(const float *x, const float *start, float *y, size_t n);
rh_status rh_math_device(rh_ctx *ctx, uint32_t op, const float *a, const float *b, float *y, size_t n);
/* Bench hook with no reference counterpart: `launches` plain streaming reads
 * of `bytes` (a multiple of 16) of device memory, launch i reading
 * buffers[i % n_buffers] (16-byte aligned device pointers), queued on the
 * context's stream, asynchronous. It is the measured bandwidth ceiling the
 * GEMV kernels are compared with; `sink` (device memory of
 * RH_STREAM_READ_SINK_WORDS words) receives one word per workgroup. */
enum { RH_STREAM_READ_SINK_WORDS = 2048 };
rh_status rh_stream_read_device(rh_ctx *ctx, const void *const *buffers, size_t n_buffers, size_t bytes,
                                size_t launches, uint32_t *sink);
/* Bench hook with no reference counterpart: one wave that occupies `stream`
 * (NULL: the context's) for `microseconds` (at most RH_HOLD_MAX_US) of the
 * device's constant-rate clock, then exits. Queued ahead of a timed run, it
 * lets the host queue every launch before the first one starts, so events
 * around the run time the launches back to back and not the host's pace. */
enum { RH_HOLD_MAX_US = 100000 };
rh_status rh_hold_device(rh_ctx *ctx, uint32_t microseconds, void *stream);
/* Bench hook with no reference counterpart: `launches` calls of
 * rh_matmul_batch_device(ctx, inputs, inputs_len, tokens, {matrices[i %
 * n_matrices], out, out_len}, 1, stream), queued from C so that the host's
 * per-call cost does not pace launches shorter than it. */
rh_status rh_matmul_batch_device_repeat(rh_ctx *ctx, const float *inputs, size_t inputs_len, size_t tokens,
                                        const rh_matrix *const *matrices, size_t n_matrices, float *out,
                                        size_t out_len, size_t launches, void *stream);
/* Tuning hook with no reference counterpart: re-reads the RUSTICIDE_HIP_*
 * kernel switches from the environment (the process's first rh_init reads
 * them; a reload publishes a new snapshot, which launches on any thread
 * pick up whole). Every
 * switch gives the same bits; they select among equivalent kernels. */
void rh_reload_tuning(void);
/* Test hook with no reference counterpart: the ordered float sum the decoder
 * kernels form for RMSNorm, ((init + values[0]) + values[1]) + ... one IEEE
 * add at a time (the f32 `Sum` fold of
 * crates/rusticide-kernels/src/portable/norm.rs:8-14), computed on the device
 * by the same wave-parallel code; n <= 8192. `rounds` (may be NULL) receives
 * the guessing rounds it took; 7 means it finished with the sequential chain. */
rh_status rh_ordered_sum_device(rh_ctx *ctx, const float *values, size_t n, float init, float *sum,
                                uint32_t *rounds);
/* Test hook: the decoder's greedy pick over n logits on the device
 * (Sampler::greedy_logits, crates/rusticide-sampling/src/sampler.rs:75-87 with
 * filters.rs:37-43: NaN as -inf, f32::total_cmp, the last maximum wins);
 * `finite` receives whether any logit is finite (when none is, the decoder
 * reports RH_ERR_NO_VALID_TOKENS). */
rh_status rh_greedy_pick_device(rh_ctx *ctx, const float *logits, size_t n, uint32_t *token, uint32_t *finite);
/* Test hook with no reference counterpart: the same sum by the short form
 * the one-token attention step uses for its softmax denominator (four values
 * a lane); n <= 256. */
rh_status rh_ordered_sum4_device(rh_ctx *ctx, const float *values, size_t n, float init, float *sum,
                                 uint32_t *rounds);
/* Test hook: the RoPE angle table rh_decoder_new builds on the host,
 * cos/sin of position * theta^(-2p/columns) per (position, pair)
 * (crates/rusticide-kernels/src/portable/rope.rs:7-23). */
void rh_rope_table_host(size_t positions, size_t columns, float theta, float *cos_out, float *sin_out);

/* ---------------------------------------------------------------- decoder
 * The callers of the quantized products, on the device: the llama-family
 * Decoder (crates/rusticide-transformer/src/decoder.rs:17-136) and greedy
 * generation (crates/rusticide-model/src/generate.rs:35-124). */

/* DecoderConfig (crates/rusticide-transformer/src/config.rs:19-33) for the
 * llama family (adjacent RoPE, SiLU, no biases or sub-norms). */
typedef struct rh_decoder_config {
    size_t embedding_length, block_count, feed_forward_length, head_count, head_count_kv, head_dim;
    size_t context_length, vocab_size;
    float rope_freq_base, rms_norm_eps;
} rh_decoder_config;

/* BlockWeights (transformer/src/weights.rs): matrices already loaded with
 * rh_matrix_load (the decoder borrows them), norms as host f32 rows the
 * decoder copies. */
typedef struct rh_decoder_block {
    const float *attn_norm;
    const rh_matrix *attn_q, *attn_k, *attn_v, *attn_output;
    const float *ffn_norm;
    const rh_matrix *ffn_gate, *ffn_up, *ffn_down;
} rh_decoder_block;

/* DecoderWeights; output == NULL ties the output to token_embd. */
typedef struct rh_decoder_weights {
    const rh_matrix *token_embd;
    const float *output_norm;
    const rh_matrix *output;
    const rh_decoder_block *blocks; /* block_count of them */
} rh_decoder_weights;

typedef struct rh_decoder rh_decoder;

/* Decoder::new (decoder.rs:28-46): validates the config (config.rs:55-80;
 * this build also needs head_dim <= 128, embedding_length <= 8192 and the
 * attention weights of the whole context in one workgroup's LDS:
 * context_length <= 32,576 with gfx950's 160 KiB), copies
 * the norms, computes the RoPE
 * angle table and allocates the f32 KV cache for context_length positions. */
rh_status rh_decoder_new(rh_ctx *ctx, const rh_decoder_config *config, const rh_decoder_weights *weights,
                         rh_decoder **out);
void rh_decoder_free(rh_decoder *d);
/* Model::reset (cache.rs:79-83). */
void rh_decoder_reset(rh_decoder *d);
/* Positions the cache holds. */
size_t rh_decoder_position(const rh_decoder *d);
/* Model::forward_batch (decoder.rs:57-107): tokens at positions
 * start..start+n, the last token's logits into `logits` (logits_len values
 * at most). Errors, checked before the cache changes: INVALID_CONFIG (no
 * tokens, a token out of range), CONTEXT_FULL, CACHE_POSITION. */
rh_status rh_decoder_forward_batch(rh_decoder *d, const uint32_t *tokens, size_t n, size_t start, float *logits,
                                   size_t logits_len);
/* generate (generate.rs:35-124) at temperature 0, without a tokenizer: reset,
 * prefill in chunks of 64, then pick / forward up to max_tokens picks or the
 * context end. The picks stay on the device between steps. */
rh_status rh_decoder_generate_greedy(rh_decoder *d, const uint32_t *prompt, size_t n, size_t max_tokens,
                                     uint32_t *out, size_t *n_out);

/* ------------------------------------------------------------------- GGUF
 * GGUF v3 files held in memory (crates/rusticide-io/src/gguf) and the upload
 * of their tensors to HBM (crates/rusticide-model/src/weights.rs:40-98,
 * crates/rusticide-transformer/src/{hyperparameters.rs,loader.rs}). */

/* GgufError (crates/rusticide-io/src/error.rs:9-108), kind by kind. */
enum {
    RH_GGUF_OK = 0,
    RH_GGUF_INVALID_MAGIC = 1,
    RH_GGUF_UNSUPPORTED_VERSION = 2,     /* value: the version            */
    RH_GGUF_UNSUPPORTED_TENSOR_TYPE = 3, /* name, value: the type id       */
    RH_GGUF_CAST_OVERFLOW = 4,
    RH_GGUF_INVALID_ALIGNMENT = 5,
    RH_GGUF_DUPLICATE_KEY = 6,           /* name: the key                  */
    RH_GGUF_DUPLICATE_TENSOR = 7,        /* name                           */
    RH_GGUF_TOO_MANY_DIMENSIONS = 8,     /* value: the declared count      */
    RH_GGUF_SHAPE_OVERFLOW = 9,          /* name                           */
    RH_GGUF_MISALIGNED_TENSOR = 10,      /* name, value: the offset        */
    RH_GGUF_OVERLAPPING_TENSORS = 11,    /* name, other: the two, in data order */
    RH_GGUF_UNEXPECTED_EOF = 12,
    RH_GGUF_TENSOR_NOT_FOUND = 13,       /* name                           */
    RH_GGUF_INVALID_VALUE_TYPE = 14,     /* value: the type tag            */
    RH_GGUF_METADATA_TOO_LARGE = 15,     /* value: the element limit       */
    RH_GGUF_NESTING_TOO_DEEP = 16,       /* value: the depth limit         */
    RH_GGUF_NOT_A_FILE = 17,             /* name: the path                 */
    RH_GGUF_IO = 18                      /* name: the path, value: errno   */
};
typedef struct rh_gguf_error {
    uint32_t kind;
    uint64_t value;
    char name[128];  /* NUL-terminated, truncated */
    char other[128]; /* the second tensor of OVERLAPPING_TENSORS */
} rh_gguf_error;

typedef struct rh_gguf rh_gguf;

/* GgufFile::from_bytes (gguf/file.rs:39-62): parses a GGUF v3 file and keeps a
 * copy of its bytes. On RH_ERR_GGUF, *err (when given) says what failed. */
rh_status rh_gguf_parse(const void *bytes, size_t len, rh_gguf **out, rh_gguf_error *err);
/* GgufFile::load (gguf/file.rs:62-77): maps the file read-only (nothing is
 * copied; the mapping lasts until rh_gguf_free) and parses it. RH_ERR_GGUF
 * with NOT_A_FILE for a directory, device or pipe, IO when it cannot be
 * opened or mapped, else as rh_gguf_parse. */
rh_status rh_gguf_open(const char *path, rh_gguf **out, rh_gguf_error *err);
void rh_gguf_free(rh_gguf *g);
/* Metadata::len, GgufFile::tensor_count. */
size_t rh_gguf_metadata_count(const rh_gguf *g);
size_t rh_gguf_tensor_count(const rh_gguf *g);
/* tensor_names()[index] (sorted) and its TensorInfo:
 * the shape outermost first ([1] for a scalar; at most 4 dimensions), the
 * GGML type id and the offset in the data section. The name (`*name_len`
 * bytes, then a NUL) stays valid until rh_gguf_free
 * (gguf/tensor_info.rs:15-62). Every out-pointer may be NULL. */
rh_status rh_gguf_tensor_at(const rh_gguf *g, size_t index, const char **name, size_t *name_len,
                            uint32_t *type_id, size_t *n_dims, uint64_t shape[4], uint64_t *offset);
/* The index of a tensor name; RH_ERR_MISSING_TENSOR when absent. Names
 * here and in rh_gguf_tensor_data are NUL-terminated: a tensor whose name
 * holds a NUL byte is reachable by index only. */
rh_status rh_gguf_tensor_find(const rh_gguf *g, const char *name, size_t *index);
/* GgufFile::quantized_tensor / layout (gguf/load.rs:47-79): the tensor's bytes
 * inside the held file (blocks and any trailer; F32/F16 values), valid until
 * rh_gguf_free. RH_ERR_GGUF with TENSOR_NOT_FOUND, UNSUPPORTED_TENSOR_TYPE,
 * CAST_OVERFLOW or UNEXPECTED_EOF. */
rh_status rh_gguf_tensor_data(const rh_gguf *g, const char *name, const uint8_t **data, size_t *len,
                              rh_gguf_error *err);
/* Metadata::get: the value type tag of a key (0..12 as in the file; arrays
 * are 9); RH_ERR_MISSING_METADATA when absent. */
rh_status rh_gguf_meta_type(const rh_gguf *g, const char *key, uint32_t *value_type);
/* Metadata::arch_unsigned (gguf/metadata.rs:117-125): u32, u64, or a
 * non-negative i32/i64, as u64. */
rh_status rh_gguf_meta_uint(const rh_gguf *g, const char *key, uint64_t *out);
/* Metadata::arch_float (gguf/metadata.rs:128-134): f32, or f64 narrowed. */
rh_status rh_gguf_meta_float(const rh_gguf *g, const char *key, float *out);
/* A string value, its invalid UTF-8 replaced by U+FFFD (Cursor::string,
 * gguf/cursor.rs:57-60): `*len` bytes (when `len` is given; the value may
 * hold NULs) followed by a NUL, valid until rh_gguf_free. */
rh_status rh_gguf_meta_string(const rh_gguf *g, const char *key, const char **out, size_t *len);

/* DecoderConfig::from_source (crates/rusticide-transformer/src/hyperparameters.rs:80-120) for the llama
 * family (crates/rusticide-llama/src/variant.rs:41-49): the llama.* keys,
 * head_count_kv defaulting to head_count, rope.freq_base to 10000 and the
 * RMS epsilon to 1e-5, vocab_size from token_embd.weight. Errors:
 * MISSING_METADATA without general.architecture and UNKNOWN_ARCHITECTURE
 * when it is not "llama" (crates/rusticide-model/src/registry.rs:39-55),
 * MISSING_METADATA, MISSING_TENSOR, INVALID_CONFIG; the message names the
 * key or tensor, or gives the reason (rh_last_error of `ctx`, which may be
 * NULL). */
rh_status rh_gguf_decoder_config(rh_ctx *ctx, const rh_gguf *g, rh_decoder_config *out);

/* A decoder's weights uploaded from a GGUF file: DecoderWeights::from_source
 * (crates/rusticide-transformer/src/loader.rs:19-92) for the llama family.
 * Every matrix is checked against its expected shape and format as
 * rh_matrix_load checks it, in the reference's order, before any byte moves;
 * then all go up in one pass through two pinned staging buffers of the
 * context (host threads fill one while the DMA engine drains the other).
 * Norms are read as f32. output.weight is optional (tied to token_embd).
 * Bias and sub-norm tensors are rejected (MISSING_KERNEL): this decoder has
 * neither. Calls on one context must not overlap. */
typedef struct rh_gguf_model rh_gguf_model;
rh_status rh_gguf_model_load(rh_ctx *ctx, const rh_gguf *g, rh_gguf_model **out);
const rh_decoder_config *rh_gguf_model_config(const rh_gguf_model *m);
/* rh_decoder_new over the model's weights; free the decoder first. */
rh_status rh_gguf_model_decoder(rh_gguf_model *m, rh_decoder **out);
void rh_gguf_model_free(rh_gguf_model *m);

#ifdef __cplusplus
}
#endif
#endif

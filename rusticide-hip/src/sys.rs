//! Raw bindings of `include/rusticide_hip.h`, the C ABI of
//! `librusticide_hip.so`. Every non-hook entry point of the header is
//! declared here with the same name, arity and argument types;
//! `tests/test_rust_binding.py` in the HIP repository parses both files and
//! fails when they drift. The test, bench and tuning hooks are left out:
//! nothing in rusticide calls them.
#![allow(non_camel_case_types)]

use core::ffi::{c_char, c_int, c_void};

#[repr(C)]
pub struct rh_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rh_matrix {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rh_q8 {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rh_decoder {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rh_gguf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct rh_gguf_model {
    _p: [u8; 0],
}

/// `rh_status`: the error kinds of `ModelError`
/// (crates/rusticide-model/src/error.rs:11-44) and `DispatchError`.
#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum rh_status {
    Ok = 0,
    InvalidArgument = 1,
    MissingKernel = 2,
    InvalidTensor = 3,
    ShapeMismatch = 4,
    InvalidConfig = 5,
    Device = 6,
    OutOfMemory = 7,
    NoDevice = 8,
    ContextFull = 9,
    CachePosition = 10,
    NoValidTokens = 11,
    Gguf = 12,
    MissingMetadata = 13,
    MissingTensor = 14,
    UnknownArchitecture = 15,
}

pub const RH_TYPE_F32: u32 = 0;
pub const RH_TYPE_F16: u32 = 1;
pub const RH_TYPE_Q4_K: u32 = 12;
pub const RH_TYPE_Q6_K: u32 = 14;
pub const RH_TYPE_I2_S: u32 = 36;

/// `Q8Kind::SuperBlock` and `Q8Kind::Row` (q8_input.rs:33-50).
pub const RH_Q8_SUPER_BLOCK: c_int = 1;
pub const RH_Q8_ROW: c_int = 2;

pub const RH_NOALLOC_SCRATCH_BYTES: usize = 4 << 20;

/// One `(Weights, &mut [f32])` pair of `matmul_batch` (matmul.rs:229).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct rh_job {
    pub weights: *const rh_matrix,
    pub out: *mut f32,
    pub out_len: usize,
}

/// `DecoderConfig` (crates/rusticide-transformer/src/config.rs:19-33), llama family.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct rh_decoder_config {
    pub embedding_length: usize,
    pub block_count: usize,
    pub feed_forward_length: usize,
    pub head_count: usize,
    pub head_count_kv: usize,
    pub head_dim: usize,
    pub context_length: usize,
    pub vocab_size: usize,
    pub rope_freq_base: f32,
    pub rms_norm_eps: f32,
}

/// `BlockWeights`: borrowed device matrices and host norm rows.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct rh_decoder_block {
    pub attn_norm: *const f32,
    pub attn_q: *const rh_matrix,
    pub attn_k: *const rh_matrix,
    pub attn_v: *const rh_matrix,
    pub attn_output: *const rh_matrix,
    pub ffn_norm: *const f32,
    pub ffn_gate: *const rh_matrix,
    pub ffn_up: *const rh_matrix,
    pub ffn_down: *const rh_matrix,
}

/// `DecoderWeights`; a null `output` ties the output to `token_embd`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct rh_decoder_weights {
    pub token_embd: *const rh_matrix,
    pub output_norm: *const f32,
    pub output: *const rh_matrix,
    pub blocks: *const rh_decoder_block,
}

/// `GgufError` (crates/rusticide-io/src/error.rs:9-108): `kind` 1-16 in the
/// enum's order, 17 `NotAFile`, 18 `Io`.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct rh_gguf_error {
    pub kind: u32,
    pub value: u64,
    pub name: [c_char; 128],
    pub other: [c_char; 128],
}

unsafe extern "C" {
    // ------------------------------------------------------------ context
    pub fn rh_init(device: c_int, out: *mut *mut rh_ctx) -> rh_status;
    pub fn rh_destroy(ctx: *mut rh_ctx);
    pub fn rh_last_error(ctx: *const rh_ctx) -> *const c_char;
    pub fn rh_adapter_name() -> *const c_char;
    pub fn rh_stream(ctx: *mut rh_ctx) -> *mut c_void;

    // ----------------------------------------------------------- matrices
    pub fn rh_matrix_load(
        ctx: *mut rh_ctx,
        type_id: u32,
        data: *const c_void,
        len: usize,
        rows: usize,
        cols: usize,
        out: *mut *mut rh_matrix,
    ) -> rh_status;
    pub fn rh_matrix_free(m: *mut rh_matrix);
    pub fn rh_matrix_rows(m: *const rh_matrix) -> usize;
    pub fn rh_matrix_cols(m: *const rh_matrix) -> usize;
    pub fn rh_matrix_type(m: *const rh_matrix) -> u32;
    pub fn rh_matrix_ternary_scale(m: *const rh_matrix) -> f32;
    pub fn rh_matrix_device_bytes(m: *const rh_matrix) -> usize;
    pub fn rh_matrix_copy_row(
        ctx: *mut rh_ctx,
        m: *const rh_matrix,
        index: usize,
        out: *mut f32,
        out_len: usize,
        found: *mut c_int,
    ) -> rh_status;

    // ----------------------------------------------------------- products
    pub fn rh_matmul_batch(
        ctx: *mut rh_ctx,
        inputs: *const f32,
        inputs_len: usize,
        tokens: usize,
        jobs: *const rh_job,
        n_jobs: usize,
    ) -> rh_status;
    pub fn rh_matvec_batch(
        ctx: *mut rh_ctx,
        input: *const f32,
        len: usize,
        jobs: *const rh_job,
        n_jobs: usize,
    ) -> rh_status;
    pub fn rh_matmul_batch_device(
        ctx: *mut rh_ctx,
        inputs: *const f32,
        inputs_len: usize,
        tokens: usize,
        jobs: *const rh_job,
        n_jobs: usize,
        stream: *mut c_void,
    ) -> rh_status;
    /// For callers that cannot allocate (graph capture, serving loops): a
    /// 4 MiB per-GPU activation array; calls that overlap on one GPU race.
    pub fn rh_matmul_batch_device_noalloc(
        ctx: *mut rh_ctx,
        inputs: *const f32,
        inputs_len: usize,
        tokens: usize,
        jobs: *const rh_job,
        n_jobs: usize,
        stream: *mut c_void,
    ) -> rh_status;
    pub fn rh_gemm_min_tokens() -> usize;
    pub fn rh_set_gemm_min_tokens(tokens: usize);

    // ------------------------------- Q8Input and QuantKernel::dot_matrix
    pub fn rh_q8_new(ctx: *mut rh_ctx, out: *mut *mut rh_q8) -> rh_status;
    pub fn rh_q8_free(q: *mut rh_q8);
    pub fn rh_q8_quantize_device(
        ctx: *mut rh_ctx,
        q: *mut rh_q8,
        kind: c_int,
        inputs: *const f32,
        inputs_len: usize,
        tokens: usize,
        stream: *mut c_void,
    ) -> rh_status;
    pub fn rh_dot_matrix_device(
        ctx: *mut rh_ctx,
        m: *const rh_matrix,
        q: *const rh_q8,
        out: *mut f32,
        out_len: usize,
        stream: *mut c_void,
    ) -> rh_status;

    // ------------------------------------------------------------ decoder
    pub fn rh_decoder_new(
        ctx: *mut rh_ctx,
        config: *const rh_decoder_config,
        weights: *const rh_decoder_weights,
        out: *mut *mut rh_decoder,
    ) -> rh_status;
    pub fn rh_decoder_free(d: *mut rh_decoder);
    pub fn rh_decoder_reset(d: *mut rh_decoder);
    pub fn rh_decoder_position(d: *const rh_decoder) -> usize;
    pub fn rh_decoder_forward_batch(
        d: *mut rh_decoder,
        tokens: *const u32,
        n: usize,
        start: usize,
        logits: *mut f32,
        logits_len: usize,
    ) -> rh_status;
    pub fn rh_decoder_generate_greedy(
        d: *mut rh_decoder,
        prompt: *const u32,
        n: usize,
        max_tokens: usize,
        out: *mut u32,
        n_out: *mut usize,
    ) -> rh_status;

    // --------------------------------------------------------------- GGUF
    pub fn rh_gguf_parse(
        bytes: *const c_void,
        len: usize,
        out: *mut *mut rh_gguf,
        err: *mut rh_gguf_error,
    ) -> rh_status;
    pub fn rh_gguf_open(path: *const c_char, out: *mut *mut rh_gguf, err: *mut rh_gguf_error) -> rh_status;
    pub fn rh_gguf_free(g: *mut rh_gguf);
    pub fn rh_gguf_metadata_count(g: *const rh_gguf) -> usize;
    pub fn rh_gguf_tensor_count(g: *const rh_gguf) -> usize;
    pub fn rh_gguf_tensor_at(
        g: *const rh_gguf,
        index: usize,
        name: *mut *const c_char,
        name_len: *mut usize,
        type_id: *mut u32,
        n_dims: *mut usize,
        shape: *mut u64,
        offset: *mut u64,
    ) -> rh_status;
    pub fn rh_gguf_tensor_find(g: *const rh_gguf, name: *const c_char, index: *mut usize) -> rh_status;
    pub fn rh_gguf_tensor_data(
        g: *const rh_gguf,
        name: *const c_char,
        data: *mut *const u8,
        len: *mut usize,
        err: *mut rh_gguf_error,
    ) -> rh_status;
    pub fn rh_gguf_meta_type(g: *const rh_gguf, key: *const c_char, value_type: *mut u32) -> rh_status;
    pub fn rh_gguf_meta_uint(g: *const rh_gguf, key: *const c_char, out: *mut u64) -> rh_status;
    pub fn rh_gguf_meta_float(g: *const rh_gguf, key: *const c_char, out: *mut f32) -> rh_status;
    pub fn rh_gguf_meta_string(
        g: *const rh_gguf,
        key: *const c_char,
        out: *mut *const c_char,
        len: *mut usize,
    ) -> rh_status;
    pub fn rh_gguf_decoder_config(ctx: *mut rh_ctx, g: *const rh_gguf, out: *mut rh_decoder_config) -> rh_status;
    pub fn rh_gguf_model_load(ctx: *mut rh_ctx, g: *const rh_gguf, out: *mut *mut rh_gguf_model) -> rh_status;
    pub fn rh_gguf_model_config(m: *const rh_gguf_model) -> *const rh_decoder_config;
    pub fn rh_gguf_model_decoder(m: *mut rh_gguf_model, out: *mut *mut rh_decoder) -> rh_status;
    pub fn rh_gguf_model_free(m: *mut rh_gguf_model);
}

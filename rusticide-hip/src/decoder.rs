//! The llama-family decoder on the device: `Decoder::new`,
//! `Model::reset` and `Model::forward_batch`
//! (crates/rusticide-transformer/src/decoder.rs:28-136) and greedy
//! generation (crates/rusticide-model/src/generate.rs:35-124).
//!
//! rusticide-model implements its `Model` trait for [`HipDecoder`]
//! (`reset`, `forward_batch`, `forward`, `context_length` map one to one), so
//! `generate` runs unchanged on top of it with any sampler; temperature 0
//! may call [`HipDecoder::generate_greedy`] instead, which keeps the picks on
//! the device. Status 9-11 are `ModelError::ContextFull`, `CachePosition` and
//! `SamplingError::NoValidTokens`.

use crate::{Context, DeviceMatrix, HipError, Result, check, sys};

/// `DecoderConfig` for the llama family.
pub type DecoderConfig = sys::rh_decoder_config;

/// One block's weights: device matrices the decoder borrows, host norm rows
/// it copies.
pub struct BlockWeights<'a> {
    pub attn_norm: &'a [f32],
    pub attn_q: &'a DeviceMatrix,
    pub attn_k: &'a DeviceMatrix,
    pub attn_v: &'a DeviceMatrix,
    pub attn_output: &'a DeviceMatrix,
    pub ffn_norm: &'a [f32],
    pub ffn_gate: &'a DeviceMatrix,
    pub ffn_up: &'a DeviceMatrix,
    pub ffn_down: &'a DeviceMatrix,
}

/// `DecoderWeights`; `output: None` ties the output to `token_embd`.
pub struct DecoderWeights<'a> {
    pub token_embd: &'a DeviceMatrix,
    pub output_norm: &'a [f32],
    pub output: Option<&'a DeviceMatrix>,
    pub blocks: Vec<BlockWeights<'a>>,
}

/// A decoder whose KV cache and scratch live on the device. It borrows the
/// weights for its lifetime `'a`.
pub struct HipDecoder<'a> {
    raw: *mut sys::rh_decoder,
    ctx: *mut sys::rh_ctx,
    vocab: usize,
    context_length: usize,
    _weights: core::marker::PhantomData<&'a DeviceMatrix>,
}

impl<'a> HipDecoder<'a> {
    /// `Decoder::new` (decoder.rs:28-46): validates `config`
    /// (`InvalidConfig`), copies the norms and allocates the f32 KV cache.
    ///
    /// # Errors
    /// `InvalidConfig` when the norms are not `embedding_length` long or the
    /// block count differs from the config; the ABI's status otherwise.
    pub fn new(ctx: &'a mut Context, config: &DecoderConfig, weights: &DecoderWeights<'a>) -> Result<Self> {
        let width = config.embedding_length;
        let invalid = |message: &str| HipError { status: sys::rh_status::InvalidConfig, message: message.to_owned() };
        if weights.blocks.len() != config.block_count {
            return Err(invalid("block count differs from the config"));
        }
        if weights.output_norm.len() != width
            || weights.blocks.iter().any(|b| b.attn_norm.len() != width || b.ffn_norm.len() != width)
        {
            return Err(invalid("a norm is not embedding_length long"));
        }
        let blocks: Vec<sys::rh_decoder_block> = weights
            .blocks
            .iter()
            .map(|b| sys::rh_decoder_block {
                attn_norm: b.attn_norm.as_ptr(),
                attn_q: b.attn_q.raw(),
                attn_k: b.attn_k.raw(),
                attn_v: b.attn_v.raw(),
                attn_output: b.attn_output.raw(),
                ffn_norm: b.ffn_norm.as_ptr(),
                ffn_gate: b.ffn_gate.raw(),
                ffn_up: b.ffn_up.raw(),
                ffn_down: b.ffn_down.raw(),
            })
            .collect();
        let w = sys::rh_decoder_weights {
            token_embd: weights.token_embd.raw(),
            output_norm: weights.output_norm.as_ptr(),
            output: weights.output.map_or(core::ptr::null(), DeviceMatrix::raw),
            blocks: blocks.as_ptr(),
        };
        let mut raw = core::ptr::null_mut();
        // SAFETY: `config`, `w` and `blocks` are live for the call; the norms
        // are copied and the matrices borrowed for 'a, which the PhantomData
        // ties to this decoder.
        let status = unsafe { sys::rh_decoder_new(ctx.raw(), config, &raw const w, &raw mut raw) };
        check(ctx.raw(), status)?;
        Ok(Self::from_raw(raw, ctx.raw(), config))
    }

    pub(crate) const fn from_raw(raw: *mut sys::rh_decoder, ctx: *mut sys::rh_ctx, config: &DecoderConfig) -> Self {
        Self {
            raw,
            ctx,
            vocab: config.vocab_size,
            context_length: config.context_length,
            _weights: core::marker::PhantomData,
        }
    }

    /// `Model::reset` (cache.rs:79-83).
    pub fn reset(&mut self) {
        // SAFETY: self.raw is a live decoder.
        unsafe { sys::rh_decoder_reset(self.raw) };
    }

    /// Positions the cache holds.
    #[must_use]
    pub fn position(&self) -> usize {
        // SAFETY: self.raw is a live decoder.
        unsafe { sys::rh_decoder_position(self.raw) }
    }

    #[must_use]
    pub const fn context_length(&self) -> usize {
        self.context_length
    }

    /// `Model::forward_batch` (decoder.rs:57-107): `tokens` at positions
    /// `start..`, the last token's logits.
    ///
    /// # Errors
    /// `InvalidConfig` (no tokens, a token out of range), `ContextFull`,
    /// `CachePosition`, all checked before the cache changes.
    pub fn forward_batch(&mut self, tokens: &[u32], start: usize) -> Result<Vec<f32>> {
        let mut logits = vec![0.0f32; self.vocab];
        // SAFETY: `tokens` and `logits` are live host slices of the given
        // lengths; the call is synchronous.
        let status = unsafe {
            sys::rh_decoder_forward_batch(self.raw, tokens.as_ptr(), tokens.len(), start, logits.as_mut_ptr(), logits.len())
        };
        check(self.ctx, status)?;
        Ok(logits)
    }

    /// `Model::forward`: one token.
    ///
    /// # Errors
    /// As [`Self::forward_batch`].
    pub fn forward(&mut self, token: u32, position: usize) -> Result<Vec<f32>> {
        self.forward_batch(&[token], position)
    }

    /// `generate` at temperature 0 (generate.rs:35-124) without a tokenizer:
    /// reset, prefill in chunks of 64, then up to `max_tokens` greedy picks
    /// or the context end. The caller applies its end-of-generation check to
    /// the returned tokens.
    ///
    /// # Errors
    /// As [`Self::forward_batch`]; `NoValidTokens` when a pick finds no
    /// finite logit (sampler.rs:84-85).
    pub fn generate_greedy(&mut self, prompt: &[u32], max_tokens: usize) -> Result<Vec<u32>> {
        let mut out = vec![0u32; max_tokens];
        let mut n = 0usize;
        // SAFETY: `prompt` and `out` are live host slices; the library
        // writes at most `max_tokens` picks and their count to `n`.
        let status = unsafe {
            sys::rh_decoder_generate_greedy(self.raw, prompt.as_ptr(), prompt.len(), max_tokens, out.as_mut_ptr(), &raw mut n)
        };
        check(self.ctx, status)?;
        out.truncate(n);
        Ok(out)
    }
}

impl Drop for HipDecoder<'_> {
    fn drop(&mut self) {
        // SAFETY: self.raw came from rh_decoder_new or rh_gguf_model_decoder
        // and is freed once, before the weights it borrows.
        unsafe { sys::rh_decoder_free(self.raw) };
    }
}

//! GGUF v3 files parsed by the library (crates/rusticide-io/src/gguf) and
//! the upload of a llama model's tensors straight to HBM
//! (`DecoderWeights::from_source`, crates/rusticide-transformer/src/loader.rs:19-92).
//!
//! `rusticide_llama::load` (llama/src/model.rs:25-27) takes this route on a
//! GPU context: `GgufFile::open` maps the file, `GgufModel::load` checks every
//! tensor in the reference's order and streams them to the device, and
//! `GgufModel::decoder` builds the decoder over them. The tokenizer keeps
//! reading its metadata through the reference's own `GgufFile`. Drop order:
//! decoder, model, file.

use core::ffi::c_char;
use std::ffi::CString;
use std::path::Path;

use crate::decoder::{DecoderConfig, HipDecoder};
use crate::{Context, HipError, Result, check, sys};

/// A `GgufError` (crates/rusticide-io/src/error.rs:9-108) as the library
/// reports it: the kind (1-16 in the enum's order, 17 `NotAFile`, 18 `Io`),
/// its number (version, type id, offset, limit or errno) and names.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct GgufFailure {
    pub kind: u32,
    pub value: u64,
    pub name: String,
    pub other: String,
}

fn text(chars: &[c_char]) -> String {
    let bytes: Vec<u8> = chars.iter().take_while(|&&c| c != 0).map(|&c| c.to_ne_bytes()[0]).collect();
    String::from_utf8_lossy(&bytes).into_owned()
}

impl From<&sys::rh_gguf_error> for GgufFailure {
    fn from(e: &sys::rh_gguf_error) -> Self {
        Self { kind: e.kind, value: e.value, name: text(&e.name), other: text(&e.other) }
    }
}

/// Why opening or reading a file failed.
#[derive(Debug, Clone, PartialEq, Eq)]
pub enum GgufLoadError {
    Gguf(GgufFailure),
    Hip(HipError),
}

const fn empty_error() -> sys::rh_gguf_error {
    sys::rh_gguf_error { kind: 0, value: 0, name: [0; 128], other: [0; 128] }
}

fn gguf_result(status: sys::rh_status, err: &sys::rh_gguf_error) -> core::result::Result<(), GgufLoadError> {
    match status {
        sys::rh_status::Ok => Ok(()),
        sys::rh_status::Gguf => Err(GgufLoadError::Gguf(err.into())),
        s => Err(GgufLoadError::Hip(HipError { status: s, message: crate::message(core::ptr::null()) })),
    }
}

/// One tensor of the table: `TensorInfo` (gguf/tensor_info.rs:15-62).
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct TensorInfo {
    pub name: String,
    pub type_id: u32,
    /// Outermost first, as the reference reverses the stored order.
    pub shape: Vec<u64>,
    pub offset: u64,
}

/// A parsed GGUF file; its bytes stay mapped (or copied) until drop.
pub struct GgufFile {
    raw: *mut sys::rh_gguf,
}

// SAFETY: a parsed file is immutable; every accessor only reads it.
unsafe impl Send for GgufFile {}
// SAFETY: as above.
unsafe impl Sync for GgufFile {}

impl GgufFile {
    /// `GgufFile::load` (gguf/file.rs:62-77): maps `path` read-only.
    ///
    /// # Errors
    /// `GgufError` kinds as the reference reports them (`NotAFile`, `Io`,
    /// then the parse errors).
    pub fn open(path: &Path) -> core::result::Result<Self, GgufLoadError> {
        let c = CString::new(path.as_os_str().as_encoded_bytes()).map_err(|_| {
            GgufLoadError::Gguf(GgufFailure { kind: 17, value: 0, name: path.display().to_string(), other: String::new() })
        })?;
        let mut raw = core::ptr::null_mut();
        let mut err = empty_error();
        // SAFETY: `c` is NUL-terminated and live; `raw` and `err` are valid
        // out-pointers.
        let status = unsafe { sys::rh_gguf_open(c.as_ptr(), &raw mut raw, &raw mut err) };
        gguf_result(status, &err)?;
        Ok(Self { raw })
    }

    /// `GgufFile::from_bytes` (gguf/file.rs:39-62): parses a copy of `bytes`.
    ///
    /// # Errors
    /// The parse's `GgufError`.
    pub fn parse(bytes: &[u8]) -> core::result::Result<Self, GgufLoadError> {
        let mut raw = core::ptr::null_mut();
        let mut err = empty_error();
        // SAFETY: `bytes` is live for the call, which copies it.
        let status = unsafe { sys::rh_gguf_parse(bytes.as_ptr().cast(), bytes.len(), &raw mut raw, &raw mut err) };
        gguf_result(status, &err)?;
        Ok(Self { raw })
    }

    #[must_use]
    pub fn metadata_count(&self) -> usize {
        // SAFETY: self.raw is a live file.
        unsafe { sys::rh_gguf_metadata_count(self.raw) }
    }

    #[must_use]
    pub fn tensor_count(&self) -> usize {
        // SAFETY: self.raw is a live file.
        unsafe { sys::rh_gguf_tensor_count(self.raw) }
    }

    /// `tensor_names()[index]` (sorted) and its info.
    #[must_use]
    pub fn tensor_at(&self, index: usize) -> Option<TensorInfo> {
        let (mut name, mut name_len, mut type_id, mut n_dims) = (core::ptr::null(), 0usize, 0u32, 0usize);
        let (mut shape, mut offset) = ([0u64; 4], 0u64);
        // SAFETY: every out-pointer is valid; `shape` holds the 4 dimensions
        // the library writes at most.
        let status = unsafe {
            sys::rh_gguf_tensor_at(
                self.raw,
                index,
                &raw mut name,
                &raw mut name_len,
                &raw mut type_id,
                &raw mut n_dims,
                shape.as_mut_ptr(),
                &raw mut offset,
            )
        };
        if status != sys::rh_status::Ok || name.is_null() {
            return None;
        }
        // SAFETY: the name is `name_len` bytes owned by the file, live while
        // `self` is.
        let bytes = unsafe { core::slice::from_raw_parts(name.cast::<u8>(), name_len) };
        Some(TensorInfo {
            name: String::from_utf8_lossy(bytes).into_owned(),
            type_id,
            shape: shape[..n_dims.min(4)].to_vec(),
            offset,
        })
    }

    /// `GgufFile::quantized_tensor` (gguf/load.rs:47-79): the tensor's bytes
    /// inside the file (blocks and any trailer), borrowed from it.
    ///
    /// # Errors
    /// `TensorNotFound`, `UnsupportedTensorType`, `CastOverflow`, `UnexpectedEof`.
    pub fn tensor_data(&self, name: &str) -> core::result::Result<&[u8], GgufLoadError> {
        let c = CString::new(name).map_err(|_| {
            GgufLoadError::Gguf(GgufFailure { kind: 13, value: 0, name: name.to_owned(), other: String::new() })
        })?;
        let (mut data, mut len) = (core::ptr::null(), 0usize);
        let mut err = empty_error();
        // SAFETY: `c` is NUL-terminated; the out-pointers are valid.
        let status = unsafe { sys::rh_gguf_tensor_data(self.raw, c.as_ptr(), &raw mut data, &raw mut len, &raw mut err) };
        gguf_result(status, &err)?;
        if len == 0 {
            return Ok(&[]);
        }
        // SAFETY: the library returned `len` bytes inside the file it holds,
        // live while `self` is.
        Ok(unsafe { core::slice::from_raw_parts(data, len) })
    }

    fn key(key: &str) -> Option<CString> {
        CString::new(key).ok()
    }

    /// `Metadata::arch_unsigned` (gguf/metadata.rs:117-125).
    #[must_use]
    pub fn meta_uint(&self, key: &str) -> Option<u64> {
        let k = Self::key(key)?;
        let mut v = 0u64;
        // SAFETY: `k` is NUL-terminated, `v` a valid out-pointer.
        let status = unsafe { sys::rh_gguf_meta_uint(self.raw, k.as_ptr(), &raw mut v) };
        (status == sys::rh_status::Ok).then_some(v)
    }

    /// `Metadata::arch_float` (gguf/metadata.rs:128-134).
    #[must_use]
    pub fn meta_float(&self, key: &str) -> Option<f32> {
        let k = Self::key(key)?;
        let mut v = 0f32;
        // SAFETY: as in meta_uint.
        let status = unsafe { sys::rh_gguf_meta_float(self.raw, k.as_ptr(), &raw mut v) };
        (status == sys::rh_status::Ok).then_some(v)
    }

    /// The value type tag of a key (0..12; arrays are 9).
    #[must_use]
    pub fn meta_type(&self, key: &str) -> Option<u32> {
        let k = Self::key(key)?;
        let mut v = 0u32;
        // SAFETY: as in meta_uint.
        let status = unsafe { sys::rh_gguf_meta_type(self.raw, k.as_ptr(), &raw mut v) };
        (status == sys::rh_status::Ok).then_some(v)
    }

    /// A string value, invalid UTF-8 replaced as `Cursor::string` replaces it.
    #[must_use]
    pub fn meta_string(&self, key: &str) -> Option<String> {
        let k = Self::key(key)?;
        let (mut p, mut len): (*const c_char, usize) = (core::ptr::null(), 0);
        // SAFETY: as in meta_uint.
        let status = unsafe { sys::rh_gguf_meta_string(self.raw, k.as_ptr(), &raw mut p, &raw mut len) };
        if status != sys::rh_status::Ok || p.is_null() {
            return None;
        }
        // SAFETY: `len` bytes owned by the file, live while `self` is.
        let bytes = unsafe { core::slice::from_raw_parts(p.cast::<u8>(), len) };
        Some(String::from_utf8_lossy(bytes).into_owned())
    }

    /// `DecoderConfig::from_source` (transformer/src/hyperparameters.rs:80-120)
    /// for the llama family.
    ///
    /// # Errors
    /// `MissingMetadata`, `UnknownArchitecture`, `MissingTensor`,
    /// `InvalidConfig`, with the key, tensor or reason in the message.
    pub fn decoder_config(&self, ctx: Option<&mut Context>) -> Result<DecoderConfig> {
        let c = ctx.map_or(core::ptr::null_mut(), |c| c.raw());
        let mut out = DecoderConfig::default();
        // SAFETY: `out` is a valid out-pointer; a null context is allowed.
        let status = unsafe { sys::rh_gguf_decoder_config(c, self.raw, &raw mut out) };
        check(c, status)?;
        Ok(out)
    }

    #[must_use]
    pub fn name_of(&self, index: usize) -> Option<String> {
        self.tensor_at(index).map(|t| t.name)
    }
}

impl Drop for GgufFile {
    fn drop(&mut self) {
        // SAFETY: self.raw came from rh_gguf_open/parse and is freed once;
        // the models loaded from it copied their tensors to the device.
        unsafe { sys::rh_gguf_free(self.raw) };
    }
}

/// A llama decoder's weights, checked and uploaded to HBM from a file.
pub struct GgufModel<'c> {
    raw: *mut sys::rh_gguf_model,
    ctx: &'c mut Context,
}

impl<'c> GgufModel<'c> {
    /// `DecoderWeights::from_source` for the llama family: every tensor
    /// checked (`MissingTensor`, `ShapeMismatch`, `MissingKernel`,
    /// `InvalidTensor`) before any byte moves, then one pipelined upload.
    ///
    /// # Errors
    /// The first failing check, in the reference's order; device failures.
    pub fn load(ctx: &'c mut Context, file: &GgufFile) -> Result<Self> {
        let mut raw = core::ptr::null_mut();
        // SAFETY: both handles are live; `raw` is a valid out-pointer.
        let status = unsafe { sys::rh_gguf_model_load(ctx.raw(), file.raw, &raw mut raw) };
        check(ctx.raw(), status)?;
        Ok(Self { raw, ctx })
    }

    #[must_use]
    pub fn config(&self) -> DecoderConfig {
        // SAFETY: the model owns its config for its lifetime; it is copied.
        unsafe { *sys::rh_gguf_model_config(self.raw) }
    }

    /// `Decoder::new` over the uploaded weights; drop the decoder first.
    ///
    /// # Errors
    /// As `HipDecoder::new`.
    pub fn decoder(&mut self) -> Result<HipDecoder<'_>> {
        let mut d = core::ptr::null_mut();
        // SAFETY: self.raw is live; `d` is a valid out-pointer. The decoder
        // borrows `self` mutably, so the model outlives it.
        let status = unsafe { sys::rh_gguf_model_decoder(self.raw, &raw mut d) };
        check(self.ctx.raw(), status)?;
        let config = self.config();
        Ok(HipDecoder::from_raw(d, self.ctx.raw(), &config))
    }
}

impl Drop for GgufModel<'_> {
    fn drop(&mut self) {
        // SAFETY: self.raw came from rh_gguf_model_load and is freed once.
        unsafe { sys::rh_gguf_model_free(self.raw) };
    }
}

/// The name of a GGUF error kind, in `GgufError`'s order.
#[must_use]
pub const fn kind_name(kind: u32) -> &'static str {
    match kind {
        1 => "InvalidMagic",
        2 => "UnsupportedVersion",
        3 => "UnsupportedTensorType",
        4 => "CastOverflow",
        5 => "InvalidAlignment",
        6 => "DuplicateKey",
        7 => "DuplicateTensor",
        8 => "TooManyDimensions",
        9 => "ShapeOverflow",
        10 => "MisalignedTensor",
        11 => "OverlappingTensors",
        12 => "UnexpectedEof",
        13 => "TensorNotFound",
        14 => "InvalidValueType",
        15 => "MetadataTooLarge",
        16 => "NestingTooDeep",
        17 => "NotAFile",
        18 => "Io",
        _ => "Unknown",
    }
}

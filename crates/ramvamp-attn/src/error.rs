//! The error variants of the entry points this crate replaces, with their
//! payload fields: `KvError` as crates/core/src/kv/mod.rs:39-123 defines it,
//! `AttentionError` as crates/core/src/kernels/attention.rs:218-311. Inside
//! the ramvamp workspace these are the reference's own types (re-exported
//! from `ramvamp_core`); `KernelError` carries the primitive variants the
//! fused prologue reports (kernels/primitives/error.rs) plus `Device`, the
//! one variant with no reference counterpart (a null argument, a value the
//! device path does not support, a HIP runtime failure).
use thiserror::Error;

/// kv/mod.rs:39-123.
#[derive(Debug, Error, PartialEq, Eq)]
pub enum KvError {
    #[error(
        "invalid kv cache dims (n_layers {n_layers}, n_kv_heads {n_kv_heads}, \
         head_dim {head_dim}, capacity {capacity}): {reason}"
    )]
    InvalidDims { n_layers: usize, n_kv_heads: usize, head_dim: usize, capacity: usize, reason: &'static str },
    #[error("kv cache layer {layer} out of range: cache has {n_layers} layers")]
    LayerOutOfRange { layer: usize, n_layers: usize },
    #[error("kv cache {what} row has {got} floats, expected {expected} (n_kv_heads * head_dim)")]
    RowLenMismatch { what: &'static str, got: usize, expected: usize },
    #[error("kv cache layer {layer} is full: capacity {capacity} positions")]
    CapacityExceeded { layer: usize, capacity: usize },
    #[error("kv cache position {pos} out of range: layer {layer} holds {len} positions")]
    PositionOutOfRange { layer: usize, pos: usize, len: usize },
    #[error("kv cache layers hold unequal lengths ({shortest} vs {longest}): appends must advance every layer once per token")]
    RaggedLayers { shortest: usize, longest: usize },
    #[error("kv cache truncate to {requested} exceeds the {len} positions held: truncation only rewinds, it cannot extend")]
    TruncateBeyondLength { requested: usize, len: usize },
}

/// The primitive variants the fused prologue reports, and `Device`.
#[derive(Debug, Error, PartialEq, Eq)]
pub enum KernelError {
    #[error("invalid head_dim {head_dim}: must be nonzero and even")]
    InvalidHeadDim { head_dim: usize },
    #[error("{what}: length mismatch ({left} vs {right})")]
    LengthMismatch { what: &'static str, left: usize, right: usize },
    #[error("{what}: input is empty")]
    Empty { what: &'static str },
    /// No reference counterpart: the device path refused or failed (status
    /// code of include/ramvamp_attn.h, its first payload field).
    #[error("device: status {code} ({what}), value {value}")]
    Device { code: i32, what: &'static str, value: u64 },
}

/// attention.rs:218-311.
#[derive(Debug, Error, PartialEq, Eq)]
pub enum AttentionError {
    #[error(transparent)]
    Kv(#[from] KvError),
    #[error(transparent)]
    Kernel(#[from] KernelError),
    #[error("attention: q length {q_len} is not a nonzero multiple of head_dim {head_dim}")]
    QLenIndivisible { q_len: usize, head_dim: usize },
    #[error("attention: {n_q_heads} query heads do not group evenly over {n_kv_heads} kv heads")]
    GqaGroupMismatch { n_q_heads: usize, n_kv_heads: usize },
    #[error("attention: out length {out_len}, expected {expected} for this call")]
    OutLenMismatch { out_len: usize, expected: usize },
    #[error("attention: layer {layer} has no positions to attend over")]
    EmptyLayer { layer: usize },
    #[error("attention: kv head range {start}..{end} is not a sub-range of 0..{n_kv_heads}")]
    KvHeadRangeOutOfRange { start: usize, end: usize, n_kv_heads: usize },
    #[error("attention: scratch length {len}, need {need} f32 for this geometry")]
    ScratchTooShort { len: usize, need: usize },
}

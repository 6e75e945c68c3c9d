//! ramvamp's per-layer GQA attention and its KV cache on an MI355X (gfx950),
//! behind the reference's own interface: the twelve attention entry points of
//! crates/core/src/kernels/attention.rs:426-859 with their signatures, the
//! `KvCache` methods of crates/core/src/kv/mod.rs:163-487, `scratch_len`
//! (attention.rs:337-353) and `AttentionScratch` (attention.rs:360-400), and
//! every status of libramvamp_attn mapped back to the variant it stands for
//! (`error`). A caller switches by importing these names instead of the
//! reference's.
//!
//! What differs, and why:
//! - The cache lives in device memory. `k_row` / `v_row` return an owned
//!   copy of the row's f16 bits (`Vec<u16>`) instead of a borrow of host
//!   memory, and `k_layer` / `v_layer` a `DeviceSlice` (the device address
//!   and element count of the same view).
//! - Slices passed to the attention functions are host memory: each call
//!   copies `q` in and `out` back (RV_HOST_PTRS) and returns when `out` is
//!   written. Callers whose q and out already live on the GPU use the raw
//!   `ramvamp_attn_sys` calls with device pointers instead.
//! - The `_dispatch` twins take `force_scalar` and ignore it: it selects the
//!   reference's CPU body (AVX2 or scalar), which has no device meaning. The
//!   device results are one computation either way.
//! - The device keeps its own workspace, so `AttentionScratch` holds no
//!   buffer; the `_in` forms still take the caller's scratch slice and report
//!   `ScratchTooShort` exactly where the reference does.
//! - `KvCache::new` makes the reference's f16 cache on device 0;
//!   `KvCache::with_elem` also takes the element type (f32 planes keep the
//!   same indexing) and the device.
//!
//! A `KvCache` may move between threads but not be shared by them: calls on
//! one cache are serialised by its HIP stream and share its workspace.
#![allow(clippy::too_many_arguments)]

use std::ffi::{c_void, CStr};
use std::ops::Range;
use std::ptr::{self, NonNull};

use ramvamp_attn_sys as sys;

mod error;
pub use error::{AttentionError, KernelError, KvError};

/// Element type of a cache's planes.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Elem {
    /// The reference's format: f16 bits, round-to-nearest-even on append.
    F16,
    /// 4-byte f32 elements, the same [layer][capacity][kv_dim] indexing.
    F32,
}

fn no_error() -> sys::rv_error {
    sys::rv_error { code: 0, a: 0, b: 0, c: 0, d: 0, what: ptr::null() }
}

fn what_of(e: &sys::rv_error) -> &'static str {
    if e.what.is_null() {
        return "";
    }
    // The library's `what` strings are static and never freed.
    unsafe { CStr::from_ptr(e.what) }.to_str().unwrap_or("")
}

/// A KvError status (codes 1..=7) as its variant; anything else as None.
fn kv_error(e: &sys::rv_error) -> Option<KvError> {
    let (a, b, c, d) = (e.a as usize, e.b as usize, e.c as usize, e.d as usize);
    Some(match e.code {
        sys::RV_KV_INVALID_DIMS => {
            KvError::InvalidDims { n_layers: a, n_kv_heads: b, head_dim: c, capacity: d, reason: what_of(e) }
        }
        sys::RV_KV_LAYER_OUT_OF_RANGE => KvError::LayerOutOfRange { layer: a, n_layers: b },
        sys::RV_KV_ROW_LEN_MISMATCH => KvError::RowLenMismatch { what: what_of(e), got: a, expected: b },
        sys::RV_KV_CAPACITY_EXCEEDED => KvError::CapacityExceeded { layer: a, capacity: b },
        sys::RV_KV_POSITION_OUT_OF_RANGE => KvError::PositionOutOfRange { layer: a, pos: b, len: c },
        sys::RV_KV_RAGGED_LAYERS => KvError::RaggedLayers { shortest: a, longest: b },
        sys::RV_KV_TRUNCATE_BEYOND_LENGTH => KvError::TruncateBeyondLength { requested: a, len: b },
        _ => return None,
    })
}

fn kernel_error(e: &sys::rv_error) -> KernelError {
    match e.code {
        sys::RV_PRIM_INVALID_HEAD_DIM => KernelError::InvalidHeadDim { head_dim: e.a as usize },
        sys::RV_PRIM_LENGTH_MISMATCH => {
            KernelError::LengthMismatch { what: what_of(e), left: e.a as usize, right: e.b as usize }
        }
        sys::RV_PRIM_EMPTY => KernelError::Empty { what: what_of(e) },
        code => KernelError::Device { code, what: what_of(e), value: e.a },
    }
}

/// Any status as the AttentionError variant it stands for (a KvError passes
/// through as AttentionError::Kv, as attention.rs:220-221 wraps it).
fn attention_error(e: &sys::rv_error) -> AttentionError {
    if let Some(kv) = kv_error(e) {
        return AttentionError::Kv(kv);
    }
    let (a, b, c) = (e.a as usize, e.b as usize, e.c as usize);
    match e.code {
        sys::RV_ATTN_Q_LEN_INDIVISIBLE => AttentionError::QLenIndivisible { q_len: a, head_dim: b },
        sys::RV_ATTN_GQA_GROUP_MISMATCH => AttentionError::GqaGroupMismatch { n_q_heads: a, n_kv_heads: b },
        sys::RV_ATTN_OUT_LEN_MISMATCH => AttentionError::OutLenMismatch { out_len: a, expected: b },
        sys::RV_ATTN_EMPTY_LAYER => AttentionError::EmptyLayer { layer: a },
        sys::RV_ATTN_KV_HEAD_RANGE => AttentionError::KvHeadRangeOutOfRange { start: a, end: b, n_kv_heads: c },
        sys::RV_ATTN_SCRATCH_TOO_SHORT => AttentionError::ScratchTooShort { len: a, need: b },
        _ => AttentionError::Kernel(kernel_error(e)),
    }
}

/// A KvCache method's status: its KvError variant. The device-only statuses
/// (a HIP failure, an unsupported value) have no KvError variant; they are
/// reported as InvalidDims with the library's reason string, the one variant
/// that carries a reason.
fn kv_result(rc: i32, e: &sys::rv_error, geometry: (usize, usize, usize, usize)) -> Result<(), KvError> {
    if rc == 0 {
        return Ok(());
    }
    Err(kv_error(e).unwrap_or(KvError::InvalidDims {
        n_layers: geometry.0,
        n_kv_heads: geometry.1,
        head_dim: geometry.2,
        capacity: geometry.3,
        reason: what_of(e),
    }))
}

fn attn_result(rc: i32, e: &sys::rv_error) -> Result<(), AttentionError> {
    if rc == 0 {
        Ok(())
    } else {
        Err(attention_error(e))
    }
}

/// attention.rs:337-353: `(n_q_heads / n_kv_heads) * max_positions + 2 *
/// head_dim`, saturating and division-safe.
pub fn scratch_len(n_q_heads: usize, n_kv_heads: usize, head_dim: usize, max_positions: usize) -> usize {
    unsafe { sys::rv_scratch_len(n_q_heads, n_kv_heads, head_dim, max_positions) }
}

/// attention.rs:360-400. The device path keeps its own workspace, so this
/// holds no buffer; it exists so callers keep their types.
#[derive(Debug, Default)]
pub struct AttentionScratch {
    slots: usize,
}

impl AttentionScratch {
    /// attention.rs:376.
    pub fn new() -> Self {
        Self::default()
    }

    /// attention.rs:388 (the reservation is recorded, nothing is allocated).
    pub fn with_capacity(slots: usize) -> Self {
        Self { slots }
    }

    /// The slots reserved by `with_capacity`.
    pub fn reserved(&self) -> usize {
        self.slots
    }
}

/// A view of device memory: a layer plane's address and element count.
#[derive(Clone, Copy, Debug)]
pub struct DeviceSlice<'a> {
    pub ptr: *const c_void,
    pub len: usize,
    _cache: std::marker::PhantomData<&'a KvCache>,
}

/// kv/mod.rs:127-487 on one GPU: the K and V planes in device memory with
/// the reference's layout, per-layer cursors on the host.
pub struct KvCache {
    raw: NonNull<sys::rv_kv>,
    elem: Elem,
}

// The cache may move to another thread; it is not Sync (one stream, one
// workspace per cache).
unsafe impl Send for KvCache {}

impl Drop for KvCache {
    fn drop(&mut self) {
        unsafe { sys::rv_kv_free(self.raw.as_ptr()) }
    }
}

impl KvCache {
    /// kv/mod.rs:163-181: zeroed f16 planes on device 0, every cursor 0.
    pub fn new(n_layers: usize, n_kv_heads: usize, head_dim: usize, capacity: usize) -> Result<Self, KvError> {
        Self::with_elem(n_layers, n_kv_heads, head_dim, capacity, Elem::F16, 0)
    }

    /// `new` with the planes' element type and the device.
    pub fn with_elem(
        n_layers: usize,
        n_kv_heads: usize,
        head_dim: usize,
        capacity: usize,
        elem: Elem,
        device: i32,
    ) -> Result<Self, KvError> {
        let mut raw: *mut sys::rv_kv = ptr::null_mut();
        let mut e = no_error();
        let code = match elem {
            Elem::F16 => sys::RV_ELEM_F16,
            Elem::F32 => sys::RV_ELEM_F32,
        };
        let rc = unsafe { sys::rv_kv_new(n_layers, n_kv_heads, head_dim, capacity, code, device, &mut raw, &mut e) };
        kv_result(rc, &e, (n_layers, n_kv_heads, head_dim, capacity))?;
        Ok(Self { raw: NonNull::new(raw).expect("rv_kv_new returned RV_OK and no cache"), elem })
    }

    /// kv/mod.rs:237-259: the bytes `new` allocates for the planes.
    pub fn projected_bytes(n_layers: usize, n_kv_heads: usize, head_dim: usize, capacity: usize) -> Result<u64, KvError> {
        let mut bytes = 0u64;
        let mut e = no_error();
        let rc = unsafe {
            sys::rv_kv_projected_bytes(n_layers, n_kv_heads, head_dim, capacity, sys::RV_ELEM_F16, &mut bytes, &mut e)
        };
        kv_result(rc, &e, (n_layers, n_kv_heads, head_dim, capacity))?;
        Ok(bytes)
    }

    /// The raw handle, for the `ramvamp_attn_sys` calls this wrapper does
    /// not cover (device pointers, the fused steps, the token graph).
    pub fn raw(&self) -> *mut sys::rv_kv {
        self.raw.as_ptr()
    }

    fn geometry(&self) -> (usize, usize, usize, usize) {
        (self.n_layers(), self.n_kv_heads(), self.head_dim(), self.capacity())
    }

    /// kv/mod.rs:262.
    pub fn n_layers(&self) -> usize {
        unsafe { sys::rv_kv_n_layers(self.raw.as_ptr()) }
    }

    /// kv/mod.rs:267.
    pub fn n_kv_heads(&self) -> usize {
        unsafe { sys::rv_kv_n_kv_heads(self.raw.as_ptr()) }
    }

    /// kv/mod.rs:272.
    pub fn head_dim(&self) -> usize {
        unsafe { sys::rv_kv_head_dim(self.raw.as_ptr()) }
    }

    /// kv/mod.rs:277.
    pub fn capacity(&self) -> usize {
        unsafe { sys::rv_kv_capacity(self.raw.as_ptr()) }
    }

    /// kv/mod.rs:282.
    pub fn kv_dim(&self) -> usize {
        unsafe { sys::rv_kv_kv_dim(self.raw.as_ptr()) }
    }

    /// kv/mod.rs:291.
    pub fn len(&self, layer: usize) -> Result<usize, KvError> {
        let mut n = 0usize;
        let mut e = no_error();
        let rc = unsafe { sys::rv_kv_len(self.raw.as_ptr(), layer, &mut n, &mut e) };
        kv_result(rc, &e, self.geometry())?;
        Ok(n)
    }

    /// kv/mod.rs:297.
    pub fn is_empty(&self) -> bool {
        unsafe { sys::rv_kv_is_empty(self.raw.as_ptr()) != 0 }
    }

    /// kv/mod.rs:312.
    pub fn seq_len(&self) -> Result<usize, KvError> {
        let mut n = 0usize;
        let mut e = no_error();
        let rc = unsafe { sys::rv_kv_seq_len(self.raw.as_ptr(), &mut n, &mut e) };
        kv_result(rc, &e, self.geometry())?;
        Ok(n)
    }

    /// kv/mod.rs:336-368 (f16 planes: round to nearest even, the reference's
    /// bits).
    pub fn append(&mut self, layer: usize, k: &[f32], v: &[f32]) -> Result<(), KvError> {
        let mut e = no_error();
        let rc = unsafe {
            sys::rv_kv_append(self.raw.as_ptr(), layer, k.as_ptr(), k.len(), v.as_ptr(), v.len(), sys::RV_HOST_PTRS,
                              &mut e)
        };
        kv_result(rc, &e, self.geometry())
    }

    /// kv/mod.rs:383-385.
    pub fn clear(&mut self) {
        unsafe { sys::rv_kv_clear(self.raw.as_ptr()) }
    }

    /// kv/mod.rs:410-420.
    pub fn truncate(&mut self, new_len: usize) -> Result<(), KvError> {
        let mut e = no_error();
        let rc = unsafe { sys::rv_kv_truncate(self.raw.as_ptr(), new_len, &mut e) };
        kv_result(rc, &e, self.geometry())
    }

    fn row(&self, plane_v: i32, layer: usize, pos: usize) -> Result<Vec<u16>, KvError> {
        if self.elem != Elem::F16 {
            return Err(KvError::InvalidDims {
                n_layers: self.n_layers(),
                n_kv_heads: self.n_kv_heads(),
                head_dim: self.head_dim(),
                capacity: self.capacity(),
                reason: "f16 rows of an f32 cache: use k_row_f32 / v_row_f32",
            });
        }
        let mut out = vec![0u16; self.kv_dim()];
        let mut e = no_error();
        let rc = unsafe {
            sys::rv_kv_read_row(self.raw.as_ptr(), plane_v, layer, pos, out.as_mut_ptr() as *mut c_void, &mut e)
        };
        kv_result(rc, &e, self.geometry())?;
        Ok(out)
    }

    fn row_f32(&self, plane_v: i32, layer: usize, pos: usize) -> Result<Vec<f32>, KvError> {
        if self.elem != Elem::F32 {
            return Err(KvError::InvalidDims {
                n_layers: self.n_layers(),
                n_kv_heads: self.n_kv_heads(),
                head_dim: self.head_dim(),
                capacity: self.capacity(),
                reason: "f32 rows of an f16 cache: use k_row / v_row",
            });
        }
        let mut out = vec![0f32; self.kv_dim()];
        let mut e = no_error();
        let rc = unsafe {
            sys::rv_kv_read_row(self.raw.as_ptr(), plane_v, layer, pos, out.as_mut_ptr() as *mut c_void, &mut e)
        };
        kv_result(rc, &e, self.geometry())?;
        Ok(out)
    }

    /// kv/mod.rs:428: a copy of the row's f16 bits.
    pub fn k_row(&self, layer: usize, pos: usize) -> Result<Vec<u16>, KvError> {
        self.row(0, layer, pos)
    }

    /// kv/mod.rs:437: a copy of the row's f16 bits.
    pub fn v_row(&self, layer: usize, pos: usize) -> Result<Vec<u16>, KvError> {
        self.row(1, layer, pos)
    }

    /// `k_row` of an f32 cache.
    pub fn k_row_f32(&self, layer: usize, pos: usize) -> Result<Vec<f32>, KvError> {
        self.row_f32(0, layer, pos)
    }

    /// `v_row` of an f32 cache.
    pub fn v_row_f32(&self, layer: usize, pos: usize) -> Result<Vec<f32>, KvError> {
        self.row_f32(1, layer, pos)
    }

    fn layer_view(&self, plane_v: bool, layer: usize) -> Result<DeviceSlice<'_>, KvError> {
        let mut p: *const c_void = ptr::null();
        let mut n = 0usize;
        let mut e = no_error();
        let rc = unsafe {
            if plane_v {
                sys::rv_kv_v_layer(self.raw.as_ptr(), layer, &mut p, &mut n, &mut e)
            } else {
                sys::rv_kv_k_layer(self.raw.as_ptr(), layer, &mut p, &mut n, &mut e)
            }
        };
        kv_result(rc, &e, self.geometry())?;
        Ok(DeviceSlice { ptr: p, len: n, _cache: std::marker::PhantomData })
    }

    /// kv/mod.rs:449: the layer's K plane up to its length, in device memory.
    pub fn k_layer(&self, layer: usize) -> Result<DeviceSlice<'_>, KvError> {
        self.layer_view(false, layer)
    }

    /// kv/mod.rs:458: the layer's V plane up to its length, in device memory.
    pub fn v_layer(&self, layer: usize) -> Result<DeviceSlice<'_>, KvError> {
        self.layer_view(true, layer)
    }
}

/// attention.rs:426.
pub fn decode_attention(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    scale: f32,
    scratch: &mut AttentionScratch,
    out: &mut [f32],
) -> Result<(), AttentionError> {
    let _ = scratch;
    let mut e = no_error();
    let rc = unsafe {
        sys::rv_decode_attention(cache.raw(), q.as_ptr(), q.len(), layer, scale, out.as_mut_ptr(), out.len(),
                                 sys::RV_HOST_PTRS, &mut e)
    };
    attn_result(rc, &e)
}

/// attention.rs:452 (`force_scalar` has no device meaning).
pub fn decode_attention_dispatch(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    scale: f32,
    scratch: &mut AttentionScratch,
    out: &mut [f32],
    force_scalar: bool,
) -> Result<(), AttentionError> {
    let _ = force_scalar;
    decode_attention(q, cache, layer, scale, scratch, out)
}

/// attention.rs:484.
pub fn decode_attention_in(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    scale: f32,
    scratch: &mut [f32],
    out: &mut [f32],
) -> Result<(), AttentionError> {
    let mut e = no_error();
    let rc = unsafe {
        sys::rv_decode_attention_in(cache.raw(), q.as_ptr(), q.len(), layer, scale, scratch.len(), out.as_mut_ptr(),
                                    out.len(), sys::RV_HOST_PTRS, &mut e)
    };
    attn_result(rc, &e)
}

/// attention.rs:511.
pub fn decode_attention_in_dispatch(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    scale: f32,
    scratch: &mut [f32],
    out: &mut [f32],
    force_scalar: bool,
) -> Result<(), AttentionError> {
    let _ = force_scalar;
    decode_attention_in(q, cache, layer, scale, scratch, out)
}

/// attention.rs:586.
pub fn decode_attention_kv_range_in(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    scale: f32,
    kv_heads: Range<usize>,
    scratch: &mut [f32],
    out: &mut [f32],
) -> Result<(), AttentionError> {
    let mut e = no_error();
    let rc = unsafe {
        sys::rv_decode_attention_kv_range_in(cache.raw(), q.as_ptr(), q.len(), layer, scale, kv_heads.start,
                                             kv_heads.end, scratch.len(), out.as_mut_ptr(), out.len(),
                                             sys::RV_HOST_PTRS, &mut e)
    };
    attn_result(rc, &e)
}

/// attention.rs:605.
pub fn decode_attention_kv_range_in_dispatch(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    scale: f32,
    kv_heads: Range<usize>,
    scratch: &mut [f32],
    out: &mut [f32],
    force_scalar: bool,
) -> Result<(), AttentionError> {
    let _ = force_scalar;
    decode_attention_kv_range_in(q, cache, layer, scale, kv_heads, scratch, out)
}

/// attention.rs:666.
pub fn attention_at(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    positions: usize,
    scale: f32,
    scratch: &mut AttentionScratch,
    out: &mut [f32],
) -> Result<(), AttentionError> {
    let _ = scratch;
    let mut e = no_error();
    let rc = unsafe {
        sys::rv_attention_at(cache.raw(), q.as_ptr(), q.len(), layer, positions, scale, out.as_mut_ptr(), out.len(),
                             sys::RV_HOST_PTRS, &mut e)
    };
    attn_result(rc, &e)
}

/// attention.rs:685.
pub fn attention_at_dispatch(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    positions: usize,
    scale: f32,
    scratch: &mut AttentionScratch,
    out: &mut [f32],
    force_scalar: bool,
) -> Result<(), AttentionError> {
    let _ = force_scalar;
    attention_at(q, cache, layer, positions, scale, scratch, out)
}

/// attention.rs:732.
pub fn attention_at_in(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    positions: usize,
    scale: f32,
    scratch: &mut [f32],
    out: &mut [f32],
) -> Result<(), AttentionError> {
    let mut e = no_error();
    let rc = unsafe {
        sys::rv_attention_at_in(cache.raw(), q.as_ptr(), q.len(), layer, positions, scale, scratch.len(),
                                out.as_mut_ptr(), out.len(), sys::RV_HOST_PTRS, &mut e)
    };
    attn_result(rc, &e)
}

/// attention.rs:761.
pub fn attention_at_in_dispatch(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    positions: usize,
    scale: f32,
    scratch: &mut [f32],
    out: &mut [f32],
    force_scalar: bool,
) -> Result<(), AttentionError> {
    let _ = force_scalar;
    attention_at_in(q, cache, layer, positions, scale, scratch, out)
}

/// attention.rs:807.
pub fn attention_at_kv_range_in(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    positions: usize,
    scale: f32,
    kv_heads: Range<usize>,
    scratch: &mut [f32],
    out: &mut [f32],
) -> Result<(), AttentionError> {
    let mut e = no_error();
    let rc = unsafe {
        sys::rv_attention_at_kv_range_in(cache.raw(), q.as_ptr(), q.len(), layer, positions, scale, kv_heads.start,
                                         kv_heads.end, scratch.len(), out.as_mut_ptr(), out.len(),
                                         sys::RV_HOST_PTRS, &mut e)
    };
    attn_result(rc, &e)
}

/// attention.rs:837.
pub fn attention_at_kv_range_in_dispatch(
    q: &[f32],
    cache: &KvCache,
    layer: usize,
    positions: usize,
    scale: f32,
    kv_heads: Range<usize>,
    scratch: &mut [f32],
    out: &mut [f32],
    force_scalar: bool,
) -> Result<(), AttentionError> {
    let _ = force_scalar;
    attention_at_kv_range_in(q, cache, layer, positions, scale, kv_heads, scratch, out)
}

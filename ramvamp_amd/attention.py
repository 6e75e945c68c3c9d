"""Python mirror of ramvamp's attention interface over the gfx950 C ABI.

Names, argument meaning, validation order and error variants follow the
reference's Rust API (crates/core/src/kernels/attention.rs:218-859 and
crates/core/src/kv/mod.rs:39-487), so code and tests written against the
reference read the same here. Differences, all forced by the device:

- ``KvCache`` lives on a GPU (planes in HBM, cursors on the host) and takes
  an element type: ``"f16"`` is the reference's format, ``"f32"`` keeps the
  same layout with 4-byte elements.
- Tensors are either torch tensors on the cache's GPU (device pointers; the
  call is queued on torch's current stream) or numpy arrays (host pointers;
  the call copies in, computes, copies out and returns when done). One call
  never mixes the two.
- ``scratch`` is validated exactly as the reference validates it (the ``_in``
  forms report ``ScratchTooShort``) but never touched: the device keeps its
  own workspace.
- ``*_dispatch(force_scalar)`` has no counterpart: there is one device path.
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_double, c_int32, c_size_t, c_uint64, c_void_p

import numpy as np

from . import _lib as L

# code -> (error class name, variant, payload field names in a, b, c, d order)
_VARIANTS = {
    1: ("KvError", "InvalidDims", ("n_layers", "n_kv_heads", "head_dim", "capacity")),
    2: ("KvError", "LayerOutOfRange", ("layer", "n_layers")),
    3: ("KvError", "RowLenMismatch", ("got", "expected")),
    4: ("KvError", "CapacityExceeded", ("layer", "capacity")),
    5: ("KvError", "PositionOutOfRange", ("layer", "pos", "len")),
    6: ("KvError", "RaggedLayers", ("shortest", "longest")),
    7: ("KvError", "TruncateBeyondLength", ("requested", "len")),
    16: ("AttentionError", "QLenIndivisible", ("q_len", "head_dim")),
    17: ("AttentionError", "GqaGroupMismatch", ("n_q_heads", "n_kv_heads")),
    18: ("AttentionError", "OutLenMismatch", ("out_len", "expected")),
    19: ("AttentionError", "EmptyLayer", ("layer",)),
    20: ("AttentionError", "KvHeadRangeOutOfRange", ("start", "end", "n_kv_heads")),
    21: ("AttentionError", "ScratchTooShort", ("len", "need")),
    24: ("PrimitiveError", "InvalidHeadDim", ("head_dim",)),
    25: ("PrimitiveError", "LengthMismatch", ("left", "right")),
    26: ("PrimitiveError", "Empty", ()),
    32: ("DeviceError", "NullArgument", ()),
    33: ("DeviceError", "Unsupported", ("value",)),
    34: ("DeviceError", "Hip", ("hip_error",)),
    35: ("DeviceError", "BadElem", ("elem",)),
    40: ("KernelError", "IndivisibleRow", ("format", "in_dim", "block_weights")),
    41: ("KernelError", "RowBytesNotBlockMultiple", ("format", "len", "block_bytes")),
    42: ("KernelError", "BlockCountMismatch", ("weight_blocks", "activation_blocks")),
    43: ("KernelError", "QuantizeLenMismatch", ("format", "floats", "out_blocks")),
    44: ("KernelError", "UnsupportedFormat", ("format",)),
    48: ("ForwardError", "InvalidTopK", ("top_k", "n_experts")),
}


class RamvampError(Exception):
    """A typed failure: ``variant`` names the reference variant, ``fields`` its payload."""

    def __init__(self, code: int, err: L.RvError):
        self.code = int(code)
        _, self.variant, names = _VARIANTS.get(self.code, ("RamvampError", "Unknown", ()))
        vals = (int(err.a), int(err.b), int(err.c), int(err.d))
        self.fields = dict(zip(names, vals))
        self.what = err.what.decode() if err.what else None
        if self.what is not None:
            self.fields["what"] = self.what
        self.raw = (self.code, *vals, self.what)
        super().__init__(f"{self.variant} {self.fields}")


class KvError(RamvampError):
    """kv/mod.rs:39-123 (passes through attention transparently, as AttentionError::Kv does)."""


class AttentionError(RamvampError):
    """attention.rs:218-311."""


class PrimitiveError(RamvampError):
    """primitives/error.rs (the fused prologue's RoPE / RMSNorm checks)."""


class DeviceError(RamvampError):
    """Failures of the device path itself (HIP errors, null arguments, unsupported shapes)."""


class KernelError(RamvampError):
    """kernels/error.rs: the quantized projections' geometry errors (LengthMismatch
    arrives as PrimitiveError's LengthMismatch with its ``what``)."""


_CLASSES = {"KvError": KvError, "AttentionError": AttentionError, "PrimitiveError": PrimitiveError,
            "DeviceError": DeviceError, "KernelError": KernelError}


def _check(rc: int, err: L.RvError):
    if rc:
        cls = _CLASSES.get(_VARIANTS.get(int(rc), ("DeviceError",))[0], RamvampError)
        raise cls(rc, err)


def _lib():
    return L.load()


_F32 = None
_RAW_STREAM = None


def _torch_f32():
    global _F32
    if _F32 is None:
        import torch

        _F32 = torch.float32
    return _F32


def _raw_stream(device: int) -> int:
    """The current HIP stream of `device` as an address: torch's raw-stream
    query (one call, no Stream object) when this torch build has it."""
    global _RAW_STREAM
    if _RAW_STREAM is None:
        import torch

        _RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
            lambda d: torch.cuda.current_stream(d).cuda_stream)
    return _RAW_STREAM(device)


class _Arg:
    """One tensor argument: device (torch) or host (numpy) pointer plus length."""

    __slots__ = ("ptr", "n", "host", "keep")

    def __init__(self, x, writable=False, dtype=np.float32):
        if x is None:
            self.ptr, self.n, self.host, self.keep = None, 0, None, None
            return
        if type(x).__module__.startswith("torch"):
            # The per-call cost matters here (a decode step marshals six of
            # these): cached dtype, is_cuda instead of a device object, and
            # the raw address handed to ctypes as an int.
            if x.dtype is not _torch_f32() or not x.is_contiguous():
                raise TypeError("device tensors must be contiguous torch.float32")
            if not x.is_cuda:
                raise TypeError("torch tensors must live on the GPU; pass numpy arrays for host memory")
            self.ptr, self.n, self.host, self.keep = x.data_ptr(), x.numel(), False, x
        else:
            a = x if isinstance(x, np.ndarray) else np.asarray(x, dtype=dtype)
            if a.dtype != dtype or not a.flags["C_CONTIGUOUS"]:
                if writable:
                    raise TypeError("host output arrays must be C-contiguous float32")
                a = np.ascontiguousarray(a, dtype=dtype)
            if writable and not a.flags["WRITEABLE"]:
                raise TypeError("host output array is read-only")
            self.ptr, self.n, self.host, self.keep = a.ctypes.data_as(c_void_p), a.size, True, a


def _flags(cache: "KvCache", args) -> int:
    kinds = {a.host for a in args if a.host is not None}
    if len(kinds) > 1:
        raise TypeError("one call takes either device tensors or host arrays, not both")
    if kinds == {True}:
        return L.RV_HOST_PTRS
    cache._bind_stream()
    return 0


def _elem_code(elem) -> int:
    if elem in ("f16", L.RV_ELEM_F16):
        return L.RV_ELEM_F16
    if elem in ("f32", L.RV_ELEM_F32):
        return L.RV_ELEM_F32
    raise ValueError(f"elem must be 'f16' or 'f32', got {elem!r}")


class KvCache:
    """kv/mod.rs `KvCache` on one GPU: planes ``[n_layers][capacity][n_kv_heads*head_dim]``."""

    def __init__(self, n_layers: int, n_kv_heads: int, head_dim: int, capacity: int, elem="f16", device: int = 0):
        self._h = c_void_p()
        err = L.RvError()
        _check(_lib().rv_kv_new(n_layers, n_kv_heads, head_dim, capacity, _elem_code(elem), device, byref(self._h),
                                byref(err)), err)
        self.device = device
        self.elem = "f16" if _elem_code(elem) == L.RV_ELEM_F16 else "f32"
        self._stream = None

    new = classmethod(lambda cls, *a, **k: cls(*a, **k))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib().rv_kv_free(h)
            except Exception:
                pass
            self._h = None

    def close(self):
        self.__del__()

    @property
    def handle(self):
        return self._h

    def _bind_stream(self):
        s = _raw_stream(self.device)
        if s != self._stream:
            err = L.RvError()
            _check(_lib().rv_kv_set_stream(self._h, c_void_p(s), byref(err)), err)
            self._stream = s

    @staticmethod
    def projected_bytes(n_layers, n_kv_heads, head_dim, capacity, elem="f16") -> int:
        out, err = c_uint64(), L.RvError()
        _check(_lib().rv_kv_projected_bytes(n_layers, n_kv_heads, head_dim, capacity, _elem_code(elem), byref(out),
                                            byref(err)), err)
        return int(out.value)

    def n_layers(self):
        return int(_lib().rv_kv_n_layers(self._h))

    def n_kv_heads(self):
        return int(_lib().rv_kv_n_kv_heads(self._h))

    def head_dim(self):
        return int(_lib().rv_kv_head_dim(self._h))

    def capacity(self):
        return int(_lib().rv_kv_capacity(self._h))

    def kv_dim(self):
        return int(_lib().rv_kv_kv_dim(self._h))

    def len(self, layer: int) -> int:
        n, err = c_size_t(), L.RvError()
        _check(_lib().rv_kv_len(self._h, layer, byref(n), byref(err)), err)
        return n.value

    def is_empty(self) -> bool:
        return bool(_lib().rv_kv_is_empty(self._h))

    def seq_len(self) -> int:
        n, err = c_size_t(), L.RvError()
        _check(_lib().rv_kv_seq_len(self._h, byref(n), byref(err)), err)
        return n.value

    def append(self, layer: int, k, v):
        ka, va = _Arg(k), _Arg(v)
        err = L.RvError()
        _check(_lib().rv_kv_append(self._h, layer, ka.ptr, ka.n, va.ptr, va.n, _flags(self, (ka, va)), byref(err)),
               err)

    def append_rows(self, layer: int, k_rows, v_rows):
        """The loop of model/prefill.rs:2081-2087 in one call (all rows or none)."""
        ka, va = _Arg(k_rows), _Arg(v_rows)
        kv_dim = self.kv_dim()
        if ka.n != va.n or ka.n % kv_dim:
            raise ValueError("k_rows and v_rows must both be rows x kv_dim")
        err = L.RvError()
        _check(_lib().rv_kv_append_rows(self._h, layer, ka.ptr, va.ptr, ka.n // kv_dim, kv_dim,
                                        _flags(self, (ka, va)), byref(err)), err)

    def clear(self):
        _lib().rv_kv_clear(self._h)

    def truncate(self, new_len: int):
        err = L.RvError()
        _check(_lib().rv_kv_truncate(self._h, new_len, byref(err)), err)

    def commit(self, layer: int, rows: int):
        """rv_kv_commit (no reference counterpart): adds the rows that
        device-position steps wrote to the layer's length; a step refused on
        the device (its position past max_position) raises KvError
        CapacityExceeded here, as device_status does."""
        self._bind_stream()
        err = L.RvError()
        _check(_lib().rv_kv_commit(self._h, layer, rows, byref(err)), err)

    def device_status(self):
        """rv_kv_device_status (no reference counterpart): waits for the
        cache's stream; raises KvError CapacityExceeded (layer, planned
        positions) when a device-position step refused its position since the
        last read, and clears the status."""
        self._bind_stream()
        err = L.RvError()
        _check(_lib().rv_kv_device_status(self._h, byref(err)), err)

    def device_bytes(self):
        """rv_kv_device_bytes: (bytes allocated now, bound with every layer's
        staged copy at capacity) of device memory this cache holds."""
        now, bound, err = c_uint64(), c_uint64(), L.RvError()
        _check(_lib().rv_kv_device_bytes(self._h, byref(now), byref(bound), byref(err)), err)
        return now.value, bound.value

    @staticmethod
    def projected_device_bytes(n_layers, n_kv_heads, head_dim, capacity, elem="f16") -> int:
        """rv_kv_projected_device_bytes: device_bytes()'s bound for a fresh
        cache of this geometry (planes, decode workspace, tickets, an EXACT
        staged copy per layer, the (cos, sin) table), from the geometry alone."""
        out, err = c_uint64(), L.RvError()
        _check(_lib().rv_kv_projected_device_bytes(n_layers, n_kv_heads, head_dim, capacity, _elem_code(elem),
                                                   byref(out), byref(err)), err)
        return int(out.value)

    def xcd_ok(self) -> bool:
        """rv_kv_xcd_dealing: whether the device deals a launch's workgroups
        to its XCDs round robin (the in-launch XCD merge needs it)."""
        ok, err = c_int32(), L.RvError()
        _check(_lib().rv_kv_xcd_dealing(self._h, byref(ok), byref(err)), err)
        return bool(ok.value)

    def _row(self, plane_v: int, layer: int, pos: int) -> np.ndarray:
        self._bind_stream()  # the copy is ordered after work queued on torch's current stream
        out = np.empty(self.kv_dim(), dtype=np.uint16 if self.elem == "f16" else np.float32)
        err = L.RvError()
        _check(_lib().rv_kv_read_row(self._h, plane_v, layer, pos, out.ctypes.data_as(c_void_p), byref(err)), err)
        return out

    def k_row(self, layer: int, pos: int) -> np.ndarray:
        return self._row(0, layer, pos)

    def v_row(self, layer: int, pos: int) -> np.ndarray:
        return self._row(1, layer, pos)

    def _layer(self, fn, layer):
        p, n, err = c_void_p(), c_size_t(), L.RvError()
        _check(fn(self._h, layer, byref(p), byref(n), byref(err)), err)
        return p.value, n.value

    def k_layer(self, layer: int):
        """(device address, element count) of layer's K view (kv/mod.rs:449)."""
        return self._layer(_lib().rv_kv_k_layer, layer)

    def v_layer(self, layer: int):
        return self._layer(_lib().rv_kv_v_layer, layer)

    def set_tuning(self, knob: int, value: int):
        err = L.RvError()
        _check(_lib().rv_kv_set_tuning(self._h, knob, value, byref(err)), err)

    def synchronize(self):
        self._bind_stream()
        err = L.RvError()
        _check(_lib().rv_kv_synchronize(self._h, byref(err)), err)

    def kernel_time(self):
        """(total milliseconds, launches) of the dominant kernels timed since
        the last read (RV_TUNE_KERNEL_TIMING on); resets the tally."""
        self._bind_stream()
        ms, n, err = c_double(), c_uint64(), L.RvError()
        _check(_lib().rv_kv_kernel_time(self._h, byref(ms), byref(n), byref(err)), err)
        return ms.value, n.value


def scratch_len(n_q_heads: int, n_kv_heads: int, head_dim: int, max_positions: int) -> int:
    """attention.rs:337-353 (the reference CPU carve; pinned, saturating)."""
    return int(_lib().rv_scratch_len(n_q_heads, n_kv_heads, head_dim, max_positions))


class AttentionScratch:
    """attention.rs:369-400. Kept for signature parity; the device has its own workspace."""

    def __init__(self, slots: int = 0):
        self.slots = slots

    @classmethod
    def with_capacity(cls, slots: int):
        return cls(slots)


def _scratch_len(scratch) -> int:
    if isinstance(scratch, int):
        return scratch
    if isinstance(scratch, AttentionScratch):
        return scratch.slots
    return int(getattr(scratch, "size", None) or len(scratch))


def _attn(fn_name, q, cache, layer, extra, out):
    qa, oa = _Arg(q), _Arg(out, writable=True)
    err = L.RvError()
    flags = _flags(cache, (qa, oa))
    fn = getattr(_lib(), fn_name)
    _check(fn(cache.handle, qa.ptr, qa.n, layer, *extra, oa.ptr, oa.n, flags, byref(err)), err)
    return out


def decode_attention(q, cache: KvCache, layer: int, scale: float, scratch, out):
    """attention.rs:426: every position the layer holds."""
    return _attn("rv_decode_attention", q, cache, layer, (scale,), out)


def decode_attention_noalloc(q, cache: KvCache, layer: int, scale: float, out):
    """rv_decode_attention_noalloc (no reference counterpart): decode_attention
    with its split partials in the library's fixed device scratch, allocating
    nothing; device tensors only (host arrays are refused)."""
    return _attn("rv_decode_attention_noalloc", q, cache, layer, (scale,), out)


def decode_attention_in(q, cache: KvCache, layer: int, scale: float, scratch, out):
    """attention.rs:484."""
    return _attn("rv_decode_attention_in", q, cache, layer, (scale, _scratch_len(scratch)), out)


def decode_attention_kv_range_in(q, cache: KvCache, layer: int, scale: float, kv_heads: range, scratch, out):
    """attention.rs:586: ``out`` is the range's own buffer, written from index 0."""
    return _attn("rv_decode_attention_kv_range_in", q, cache, layer,
                 (scale, kv_heads.start, kv_heads.stop, _scratch_len(scratch)), out)


def attention_at(q, cache: KvCache, layer: int, positions: int, scale: float, scratch, out):
    """attention.rs:666: positions 0..positions only."""
    return _attn("rv_attention_at", q, cache, layer, (positions, scale), out)


def attention_at_in(q, cache: KvCache, layer: int, positions: int, scale: float, scratch, out):
    """attention.rs:732."""
    return _attn("rv_attention_at_in", q, cache, layer, (positions, scale, _scratch_len(scratch)), out)


def attention_at_kv_range_in(q, cache: KvCache, layer: int, positions: int, scale: float, kv_heads: range, scratch,
                             out):
    """attention.rs:807."""
    return _attn("rv_attention_at_kv_range_in", q, cache, layer,
                 (positions, scale, kv_heads.start, kv_heads.stop, _scratch_len(scratch)), out)


_MODES = {"exact": L.RV_PREFILL_EXACT, "f16": L.RV_PREFILL_F16, "bf16": L.RV_PREFILL_BF16}


def attention_at_rows(q_rows, cache: KvCache, layer: int, start: int, scale: float, out, mode: str = "exact"):
    """model/prefill.rs:1322 `scatter_attention`: row r attends start + r + 1 positions."""
    qa, oa = _Arg(q_rows), _Arg(out, writable=True)
    q_dim = _row_width(q_rows, cache)
    rows = qa.n // q_dim if q_dim else 0
    if oa.n != qa.n:
        raise ValueError("out must have the shape of q_rows")
    err = L.RvError()
    flags = _flags(cache, (qa, oa)) | _MODES[mode]
    _check(_lib().rv_attention_at_rows(cache.handle, qa.ptr, rows, q_dim, layer, start, scale, oa.ptr, flags,
                                       byref(err)), err)
    return out


def _row_width(x, cache: KvCache) -> int:
    shape = tuple(x.shape)
    if len(shape) != 2:
        raise ValueError("row-batched inputs are 2-D: rows x width")
    return int(shape[1])


def decode_step(cache: KvCache, layer: int, q, k, v, q_norm_w, k_norm_w, eps: float, theta: float, position: int,
                scale: float, out):
    """model/forward.rs:2622-2633: q/k RMSNorm + RoPE, append, decode attention."""
    qa, ka, va, wq, wk, oa = _Arg(q), _Arg(k), _Arg(v), _Arg(q_norm_w), _Arg(k_norm_w), _Arg(out, writable=True)
    err = L.RvError()
    flags = _flags(cache, (qa, ka, va, wq, wk, oa))
    _check(_lib().rv_decode_step(cache.handle, layer, qa.ptr, qa.n, ka.ptr, ka.n, va.ptr, va.n, wq.ptr, wq.n, wk.ptr,
                                 wk.n, eps, theta, position, scale, oa.ptr, oa.n, flags, byref(err)), err)
    return out


def _position_ptr(d_position) -> int:
    """Address of a one-element int32 device tensor holding a token position."""
    import torch

    if not (isinstance(d_position, torch.Tensor) and d_position.is_cuda and d_position.dtype == torch.int32
            and d_position.numel() >= 1):
        raise TypeError("d_position must be an int32 device tensor with at least one element")
    return d_position.data_ptr()


def decode_step_dev(cache: KvCache, layer: int, q, k, v, q_norm_w, k_norm_w, eps: float, theta: float, d_position,
                    max_position: int, scale: float, out):
    """rv_decode_step_dev (no reference counterpart): decode_step at the
    position ``d_position`` (int32 device tensor) holds when the step runs,
    planned for ``max_position``; the layer's length does not move
    (``KvCache.commit``). Device tensors only. For a token graph captured once
    and replayed per token."""
    qa, ka, va, wq, wk, oa = _Arg(q), _Arg(k), _Arg(v), _Arg(q_norm_w), _Arg(k_norm_w), _Arg(out, writable=True)
    err = L.RvError()
    flags = _flags(cache, (qa, ka, va, wq, wk, oa))
    _check(_lib().rv_decode_step_dev(cache.handle, layer, qa.ptr, qa.n, ka.ptr, ka.n, va.ptr, va.n, wq.ptr, wq.n,
                                     wk.ptr, wk.n, eps, theta, _position_ptr(d_position), max_position, scale, oa.ptr,
                                     oa.n, flags, byref(err)), err)
    return out


def position_advance(cache: KvCache, d_position, n: int = 1):
    """rv_position_advance: queues ``d_position += n`` on the cache's stream."""
    cache._bind_stream()
    err = L.RvError()
    _check(_lib().rv_position_advance(cache.handle, _position_ptr(d_position), n, byref(err)), err)


def prefill_chunk(cache: KvCache, layer: int, q_rows, k_rows, v_rows, q_norm_w, k_norm_w, eps: float, theta: float,
                  start: int, scale: float, out, mode: str = "exact"):
    """model/prefill.rs:2055-2111 steps (d)-(f) for one layer."""
    qa, ka, va, wq, wk, oa = (_Arg(q_rows), _Arg(k_rows), _Arg(v_rows), _Arg(q_norm_w), _Arg(k_norm_w),
                              _Arg(out, writable=True))
    q_dim = _row_width(q_rows, cache)
    rows = qa.n // q_dim
    if oa.n != qa.n or ka.n != va.n or ka.n != rows * cache.kv_dim():
        raise ValueError("q_rows/out are rows x q_dim, k_rows/v_rows rows x kv_dim")
    err = L.RvError()
    flags = _flags(cache, (qa, ka, va, wq, wk, oa)) | _MODES[mode]
    _check(_lib().rv_prefill_chunk(cache.handle, layer, qa.ptr, ka.ptr, va.ptr, rows, q_dim, wq.ptr, wq.n, wk.ptr,
                                   wk.n, eps, theta, start, scale, oa.ptr, flags, byref(err)), err)
    return out

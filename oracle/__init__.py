"""ctypes wrapper over the CPU oracle (liboracle.so, built by oracle/Makefile).

TEST INFRASTRUCTURE ONLY. The oracle is a C restatement of ramvamp's CPU
attention path (crates/core/src/kernels/attention.rs and attention/x86.rs,
kv/mod.rs, primitives/{softmax,norm,rope}.rs, quants/f16.rs and the callers in
model/forward.rs and model/prefill.rs). Only tests/, ``__graft_entry__.smoke``
and bench.py's ``cpu_baseline`` leg may import it, and only as the checker or
the timed CPU baseline; the product (``ramvamp_amd``) never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_int32, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

RV_ELEM_F16 = 1
RV_ELEM_F32 = 2


class RvError(ctypes.Structure):
    _fields_ = [
        ("code", c_int32),
        ("a", c_uint64),
        ("b", c_uint64),
        ("c", c_uint64),
        ("d", c_uint64),
        ("what", c_char_p),
    ]


class OracleError(Exception):
    """A nonzero status from the oracle, with the reference variant's payload."""

    def __init__(self, code: int, err: RvError | None = None):
        self.code = int(code)
        self.a = int(err.a) if err else 0
        self.b = int(err.b) if err else 0
        self.c = int(err.c) if err else 0
        self.d = int(err.d) if err else 0
        self.what = err.what.decode() if (err and err.what) else None
        super().__init__(f"oracle status {self.code} ({self.a}, {self.b}, {self.c}, {self.d}, {self.what})")

    def payload(self):
        return (self.code, self.a, self.b, self.c, self.d, self.what)


_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    fp = POINTER(c_float)
    E = POINTER(RvError)
    sig = {
        "rvo_f16_to_f32": (c_float, [c_uint16]),
        "rvo_f32_to_f16": (c_uint16, [c_float]),
        "rvo_f16_to_f32_n": (None, [c_void_p, c_void_p, c_size_t]),
        "rvo_f32_to_f16_n": (None, [c_void_p, c_void_p, c_size_t]),
        "rvo_kv_projected_bytes": (c_int32, [c_size_t, c_size_t, c_size_t, c_size_t, c_int, POINTER(c_uint64), E]),
        "rvo_kv_new": (c_int32, [c_size_t, c_size_t, c_size_t, c_size_t, c_int, POINTER(c_void_p), E]),
        "rvo_kv_free": (None, [c_void_p]),
        "rvo_kv_len": (c_int32, [c_void_p, c_size_t, POINTER(c_size_t), E]),
        "rvo_kv_is_empty": (c_int, [c_void_p]),
        "rvo_kv_seq_len": (c_int32, [c_void_p, POINTER(c_size_t), E]),
        "rvo_kv_append": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, E]),
        "rvo_kv_clear": (None, [c_void_p]),
        "rvo_kv_truncate": (c_int32, [c_void_p, c_size_t, E]),
        "rvo_kv_read_row": (c_int32, [c_void_p, c_int, c_size_t, c_size_t, c_void_p, E]),
        "rvo_softmax": (c_int32, [c_void_p, c_size_t]),
        "rvo_rmsnorm_in_place": (c_int32, [c_void_p, c_void_p, c_size_t, c_float]),
        "rvo_rope_neox_heads": (c_int32, [c_void_p, c_size_t, c_size_t, c_size_t, c_uint32, c_float]),
        "rvo_norm_rope_heads": (c_int32, [c_void_p, c_size_t, c_size_t, c_void_p, c_float, c_float, c_uint32]),
        "rvo_scratch_len": (c_size_t, [c_size_t, c_size_t, c_size_t, c_size_t]),
        "rvo_attention": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, c_int, c_size_t, c_float, c_size_t,
                                    c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, c_int, E]),
        "rvo_avx2_path_covers": (c_int, [c_size_t]),
        "rvo_kv_head_range": (None, [c_size_t, c_size_t, c_size_t, c_size_t, POINTER(c_size_t), POINTER(c_size_t)]),
        "rvo_attention_shard_range": (None, [c_size_t, c_size_t, c_size_t, c_size_t, POINTER(c_size_t),
                                             POINTER(c_size_t)]),
        "rvo_pool_decode_attention": (c_int32, [c_void_p, c_size_t, c_float, c_void_p, c_size_t, c_void_p, c_size_t,
                                                c_size_t, c_int, E]),
        "rvo_scatter_attention": (c_int32, [c_void_p, c_size_t, c_size_t, c_size_t, c_size_t, c_float, c_void_p,
                                            c_void_p, c_size_t, c_int, E]),
        "rvo_decode_step": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_size_t,
                                      c_void_p, c_size_t, c_float, c_float, c_uint32, c_float, c_void_p, c_size_t,
                                      c_int, E]),
        "rvo_prefill_chunk": (c_int32, [c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t,
                                        c_void_p, c_size_t, c_void_p, c_size_t, c_float, c_float, c_size_t, c_float,
                                        c_void_p, c_size_t, c_int, E]),
        "rvo_quant_block_weights": (c_size_t, [c_uint32]),
        "rvo_quant_block_bytes": (c_size_t, [c_uint32]),
        "rvo_quant_row_bytes": (c_int32, [c_uint32, c_size_t, POINTER(c_size_t), E]),
        "rvo_quantize_row_q8_0": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, E]),
        "rvo_quantize_row_q8_k": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, E]),
        "rvo_dequantize_row": (c_int32, [c_uint32, c_void_p, c_size_t, c_void_p, E]),
        "rvo_vec_dot_q8_k": (c_int32, [c_uint32, c_void_p, c_size_t, c_void_p, c_size_t, fp, E]),
        "rvo_vec_dot_q8_0": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, fp, E]),
        "rvo_gemv_q8_k": (c_int32, [c_uint32, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_size_t, c_size_t,
                                    c_size_t, c_size_t, c_void_p, c_size_t, E]),
        "rvo_router_topk": (c_int32, [c_void_p, c_size_t, c_void_p, c_size_t, c_size_t, c_int, c_void_p, c_void_p,
                                      c_void_p]),
        "rvo_gemv_q8_0": (c_int32, [c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_size_t, c_size_t, c_size_t,
                                    c_size_t, c_void_p, c_size_t, E]),
    }
    del fp
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(c_void_p)


def _check(rc: int, err: RvError):
    if rc:
        raise OracleError(rc, err)


# ---- f16 ---------------------------------------------------------------------

def f16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().rvo_f16_to_f32_n(_ptr(b), _ptr(out), b.size)
    return out


def f32_to_f16(x) -> np.ndarray:
    a = _f32(x)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().rvo_f32_to_f16_n(_ptr(a), _ptr(out), a.size)
    return out


# ---- primitives -----------------------------------------------------------------

def softmax(x) -> np.ndarray:
    a = _f32(x).copy()
    rc = lib().rvo_softmax(_ptr(a), a.size)
    if rc:
        raise OracleError(rc)
    return a


def rmsnorm(x, w, eps: float) -> np.ndarray:
    a = _f32(x).copy()
    ww = _f32(w)
    rc = lib().rvo_rmsnorm_in_place(_ptr(a), _ptr(ww), a.size, eps)
    if rc:
        raise OracleError(rc)
    return a


def rope_neox_heads(x, n_heads: int, head_dim: int, position: int, theta: float) -> np.ndarray:
    a = _f32(x).copy()
    rc = lib().rvo_rope_neox_heads(_ptr(a), a.size, n_heads, head_dim, position, theta)
    if rc:
        raise OracleError(rc)
    return a


def norm_rope_heads(x, n_heads: int, head_dim: int, w, eps: float, theta: float, position: int) -> np.ndarray:
    a = _f32(x).copy()
    ww = _f32(w)
    rc = lib().rvo_norm_rope_heads(_ptr(a), n_heads, head_dim, _ptr(ww), eps, theta, position)
    if rc:
        raise OracleError(rc)
    return a


def scratch_len(n_q_heads, n_kv_heads, head_dim, max_positions) -> int:
    return int(lib().rvo_scratch_len(n_q_heads, n_kv_heads, head_dim, max_positions))


def avx2_path_covers(head_dim: int) -> bool:
    return bool(lib().rvo_avx2_path_covers(head_dim))


def kv_head_range(n_kv_heads, units, slot_lo, slot_hi):
    lo, hi = c_size_t(), c_size_t()
    lib().rvo_kv_head_range(n_kv_heads, units, slot_lo, slot_hi, byref(lo), byref(hi))
    return range(lo.value, hi.value)


def attention_shard_range(rows, start, shards, index):
    lo, hi = c_size_t(), c_size_t()
    lib().rvo_attention_shard_range(rows, start, shards, index, byref(lo), byref(hi))
    return range(lo.value, hi.value)


def projected_bytes(n_layers, n_kv_heads, head_dim, capacity, elem=RV_ELEM_F16) -> int:
    out, err = c_uint64(), RvError()
    _check(lib().rvo_kv_projected_bytes(n_layers, n_kv_heads, head_dim, capacity, elem, byref(out), byref(err)), err)
    return int(out.value)


# ---- KV cache + attention ---------------------------------------------------------

class KvCache:
    """kv/mod.rs `KvCache`, in host memory, f16 (reference) or f32 elements."""

    def __init__(self, n_layers, n_kv_heads, head_dim, capacity, elem=RV_ELEM_F16):
        self._h = c_void_p()
        err = RvError()
        _check(lib().rvo_kv_new(n_layers, n_kv_heads, head_dim, capacity, elem, byref(self._h), byref(err)), err)
        self.n_layers, self.n_kv_heads, self.head_dim, self.capacity = n_layers, n_kv_heads, head_dim, capacity
        self.kv_dim = n_kv_heads * head_dim
        self.elem = elem

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and h.value and lib is not None:
            try:
                lib().rvo_kv_free(h)
            except Exception:
                pass
            self._h = None

    @property
    def handle(self):
        return self._h

    def append(self, layer, k, v):
        k, v = _f32(k), _f32(v)
        err = RvError()
        _check(lib().rvo_kv_append(self._h, layer, _ptr(k), k.size, _ptr(v), v.size, byref(err)), err)

    def append_rows(self, layer, k_rows, v_rows):
        k_rows, v_rows = _f32(k_rows).reshape(-1, self.kv_dim), _f32(v_rows).reshape(-1, self.kv_dim)
        for r in range(k_rows.shape[0]):
            self.append(layer, k_rows[r], v_rows[r])

    def len(self, layer):
        n, err = c_size_t(), RvError()
        _check(lib().rvo_kv_len(self._h, layer, byref(n), byref(err)), err)
        return n.value

    def is_empty(self):
        return bool(lib().rvo_kv_is_empty(self._h))

    def seq_len(self):
        n, err = c_size_t(), RvError()
        _check(lib().rvo_kv_seq_len(self._h, byref(n), byref(err)), err)
        return n.value

    def truncate(self, new_len):
        err = RvError()
        _check(lib().rvo_kv_truncate(self._h, new_len, byref(err)), err)

    def clear(self):
        lib().rvo_kv_clear(self._h)

    def read_row(self, plane_v: bool, layer, pos):
        dt = np.uint16 if self.elem == RV_ELEM_F16 else np.float32
        out = np.empty(self.kv_dim, dtype=dt)
        err = RvError()
        _check(lib().rvo_kv_read_row(self._h, int(bool(plane_v)), layer, pos, _ptr(out), byref(err)), err)
        return out

    def attention(self, q, layer, scale, positions=None, kv_range=None, scratch_len=None, out_len=None,
                  force_scalar=False):
        """One of the twelve reference entry points (attention.rs:426-859)."""
        q = _f32(q)
        lo, hi = (0, self.n_kv_heads) if kv_range is None else (kv_range.start, kv_range.stop)
        n_q = q.size // self.head_dim if self.head_dim else 0
        group = n_q // self.n_kv_heads if self.n_kv_heads else 0
        if out_len is None:
            out_len = max(hi - lo, 0) * group * self.head_dim if kv_range is not None else q.size
        out = np.full(max(out_len, 1), np.nan, dtype=np.float32)
        scratch = None
        if scratch_len is not None:
            scratch = np.zeros(max(scratch_len, 1), dtype=np.float32)
        err = RvError()
        rc = lib().rvo_attention(_ptr(q), q.size, self._h, layer, int(positions is not None),
                                 0 if positions is None else positions, scale, lo, hi,
                                 None if scratch is None else _ptr(scratch), 0 if scratch_len is None else scratch_len,
                                 _ptr(out), out_len, int(force_scalar), byref(err))
        _check(rc, err)
        return out[:out_len]

    def pool_decode_attention(self, q, layer, scale, threads, force_scalar=False):
        q = _f32(q)
        out = np.full(q.size, np.nan, dtype=np.float32)
        err = RvError()
        _check(lib().rvo_pool_decode_attention(self._h, layer, scale, _ptr(q), q.size, _ptr(out), q.size, threads,
                                               int(force_scalar), byref(err)), err)
        return out

    def scatter_attention(self, q_rows, layer, start, scale, threads, force_scalar=False):
        q_rows = _f32(q_rows)
        rows, q_dim = q_rows.shape
        out = np.full(q_rows.shape, np.nan, dtype=np.float32)
        err = RvError()
        _check(lib().rvo_scatter_attention(self._h, layer, start, rows, q_dim, scale, _ptr(q_rows), _ptr(out), threads,
                                           int(force_scalar), byref(err)), err)
        return out

    def decode_step(self, layer, q, k, v, q_norm_w, k_norm_w, eps, theta, position, scale, threads=1,
                    force_scalar=False):
        q, k, v = _f32(q).copy(), _f32(k).copy(), _f32(v)
        wq, wk = _f32(q_norm_w), _f32(k_norm_w)
        out = np.full(q.size, np.nan, dtype=np.float32)
        err = RvError()
        _check(lib().rvo_decode_step(self._h, layer, _ptr(q), q.size, _ptr(k), _ptr(v), _ptr(wq), wq.size, _ptr(wk),
                                     wk.size, eps, theta, position, scale, _ptr(out), threads, int(force_scalar),
                                     byref(err)), err)
        return out

    def prefill_chunk(self, layer, q_rows, k_rows, v_rows, q_norm_w, k_norm_w, eps, theta, start, scale, threads=1,
                      force_scalar=False):
        q_rows, k_rows, v_rows = _f32(q_rows).copy(), _f32(k_rows).copy(), _f32(v_rows)
        rows, q_dim = q_rows.shape
        wq, wk = _f32(q_norm_w), _f32(k_norm_w)
        out = np.full(q_rows.shape, np.nan, dtype=np.float32)
        err = RvError()
        _check(lib().rvo_prefill_chunk(self._h, layer, _ptr(q_rows), _ptr(k_rows), _ptr(v_rows), rows, q_dim, _ptr(wq),
                                       wq.size, _ptr(wk), wk.size, eps, theta, start, scale, _ptr(out), threads,
                                       int(force_scalar), byref(err)), err)
        return out


# ---- quantized projections (rv_oracle_quant.c; kernels/quants, kernels/gemv.rs) ----

RV_QF_Q4_K, RV_QF_Q5_K, RV_QF_Q6_K, RV_QF_Q8_0, RV_QF_Q8_K = 1, 2, 3, 4, 5
# The ABI's activation blocks (include/ramvamp_gemv.h): ggml field order, no padding.
BLOCK_Q8_K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
BLOCK_Q8_0 = np.dtype([("d", "<f4"), ("qs", "i1", (32,))])
assert BLOCK_Q8_K.itemsize == 292 and BLOCK_Q8_0.itemsize == 36


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


def quant_block_weights(fmt: int) -> int:
    return int(lib().rvo_quant_block_weights(fmt))


def quant_block_bytes(fmt: int) -> int:
    return int(lib().rvo_quant_block_bytes(fmt))


def quant_row_bytes(fmt: int, in_dim: int) -> int:
    n, err = c_size_t(), RvError()
    _check(lib().rvo_quant_row_bytes(fmt, in_dim, byref(n), byref(err)), err)
    return int(n.value)


def quantize_row_q8_0(x, n_blocks=None) -> np.ndarray:
    x = _f32(x).ravel()
    n = x.size // 32 if n_blocks is None else n_blocks
    out = np.zeros(n, dtype=BLOCK_Q8_0)
    err = RvError()
    _check(lib().rvo_quantize_row_q8_0(_ptr(x), x.size, out.ctypes.data, n, byref(err)), err)
    return out


def quantize_row_q8_k(x, n_blocks=None) -> np.ndarray:
    x = _f32(x).ravel()
    n = x.size // 256 if n_blocks is None else n_blocks
    out = np.zeros(n, dtype=BLOCK_Q8_K)
    err = RvError()
    _check(lib().rvo_quantize_row_q8_k(_ptr(x), x.size, out.ctypes.data, n, byref(err)), err)
    return out


def dequantize_row(fmt: int, row) -> np.ndarray:
    row = _u8(row).ravel()
    bb = max(1, quant_block_bytes(fmt))
    out = np.zeros(row.size // bb * quant_block_weights(fmt), dtype=np.float32)
    err = RvError()
    _check(lib().rvo_dequantize_row(fmt, row.ctypes.data, row.size, _ptr(out), byref(err)), err)
    return out


def vec_dot(fmt: int, row, acts) -> float:
    row = _u8(row).ravel()
    r, err = c_float(), RvError()
    if fmt == RV_QF_Q8_0:
        _check(lib().rvo_vec_dot_q8_0(row.ctypes.data, row.size, acts.ctypes.data, acts.size, byref(r), byref(err)),
               err)
    else:
        _check(lib().rvo_vec_dot_q8_k(fmt, row.ctypes.data, row.size, acts.ctypes.data, acts.size, byref(r),
                                      byref(err)), err)
    return float(np.float32(r.value))


def gemv(fmt: int, weight, in_dim: int, out_dim: int, acts, n_acts: int = 1, rows=None) -> np.ndarray:
    """gemv.rs: out[(r - lo) * n_acts + a] = weight_row(r) . act_row(a) for r in rows."""
    weight = _u8(weight).ravel()
    lo, hi = (0, out_dim) if rows is None else rows
    out = np.full(max(0, hi - lo) * n_acts, np.nan, dtype=np.float32)
    err = RvError()
    if fmt == RV_QF_Q8_0:
        rc = lib().rvo_gemv_q8_0(weight.ctypes.data, weight.size, in_dim, out_dim, acts.ctypes.data, acts.size, n_acts,
                                 lo, hi, _ptr(out), out.size, byref(err))
    else:
        rc = lib().rvo_gemv_q8_k(fmt, weight.ctypes.data, weight.size, in_dim, out_dim, acts.ctypes.data, acts.size,
                                 n_acts, lo, hi, _ptr(out), out.size, byref(err))
    _check(rc, err)
    return out


RV_FWD_INVALID_TOP_K = 48
RV_PRIM_LENGTH_MISMATCH = 25
RV_PRIM_EMPTY = 26


def router_topk(x, router, n_experts: int, top_k: int, norm: bool):
    """forward.rs:2658-2705 for one row: (experts uint32 [top_k], weights float32 [top_k])."""
    x, router = _f32(x).ravel(), _f32(router).ravel()
    probs = np.zeros(max(1, n_experts), np.float32)
    experts = np.zeros(max(1, top_k), np.uint32)
    weights = np.zeros(max(1, top_k), np.float32)
    rc = lib().rvo_router_topk(_ptr(x), x.size, _ptr(router), n_experts, top_k, int(bool(norm)), _ptr(probs),
                               experts.ctypes.data, _ptr(weights))
    if rc:
        raise OracleError(rc)
    return experts[:top_k], weights[:top_k]


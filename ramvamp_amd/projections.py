"""Python mirror of ramvamp's quantized projections over the gfx950 C ABI
(include/ramvamp_gemv.h).

Names, argument meaning, validation order and error variants follow
crates/core/src/kernels/quants/{quantize,mod}.rs and kernels/gemv.rs, and the
two per-layer helpers follow model/forward.rs:2574-2646. Device-only: every
tensor is a torch tensor on the current GPU (weights and activation blocks as
``uint8`` byte tensors, rows as ``float32``); calls are queued on torch's
current stream. Activation blocks use the ABI layout of rv_block_q8_k (292
bytes) and rv_block_q8_0 (36 bytes). Results are bit-identical to the
reference's scalar kernels.
"""
from __future__ import annotations

from ctypes import byref, c_size_t, c_void_p

from . import _lib as L
from .attention import _check, _raw_stream

Q4_K, Q5_K, Q6_K, Q8_0, Q8_K = L.RV_QF_Q4_K, L.RV_QF_Q5_K, L.RV_QF_Q6_K, L.RV_QF_Q8_0, L.RV_QF_Q8_K
Q8_K_BLOCK_BYTES = 292  # sizeof(rv_block_q8_k)
Q8_0_BLOCK_BYTES = 36   # sizeof(rv_block_q8_0)


def _lib():
    return L.load()


def _stream():
    import torch
    return c_void_p(_raw_stream(torch.cuda.current_device()))


def _dev(t, what):
    if not (hasattr(t, "is_cuda") and t.is_cuda):
        raise TypeError(f"{what} must be a torch tensor on the GPU (device pointers only)")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return c_void_p(t.data_ptr())


def _blocks(t, size, what) -> int:
    n = t.numel() * t.element_size()
    if n % size:
        raise ValueError(f"{what}: {n} bytes is not a whole number of {size}-byte blocks")
    return n // size


def block_weights(fmt: int) -> int:
    """QuantFormat::block_weights (quants/mod.rs:75-81)."""
    return int(_lib().rv_quant_block_weights(fmt))


def block_bytes(fmt: int) -> int:
    """QuantFormat::block_bytes (quants/mod.rs:83-93)."""
    return int(_lib().rv_quant_block_bytes(fmt))


def row_bytes(fmt: int, in_dim: int) -> int:
    """QuantFormat::row_bytes (quants/mod.rs:95-105)."""
    n, err = c_size_t(), L.RvError()
    _check(_lib().rv_quant_row_bytes(fmt, in_dim, byref(n), byref(err)), err)
    return int(n.value)


def q8_k_buffer(n_blocks: int, device=None):
    """Room for n_blocks Q8_K activation blocks."""
    import torch
    return torch.empty(n_blocks * Q8_K_BLOCK_BYTES, dtype=torch.uint8, device=device or "cuda")


def q8_0_buffer(n_blocks: int, device=None):
    import torch
    return torch.empty(n_blocks * Q8_0_BLOCK_BYTES, dtype=torch.uint8, device=device or "cuda")


def quantize_row_q8_0(x, out):
    """quantize.rs:37-55: x (float32, 32 * n) into n Q8_0 blocks."""
    err = L.RvError()
    _check(_lib().rv_quantize_row_q8_0(_dev(x, "x"), x.numel(), _dev(out, "out"),
                                       _blocks(out, Q8_0_BLOCK_BYTES, "out"), _stream(), 0, byref(err)), err)
    return out


def quantize_row_q8_k(x, out):
    """quantize.rs:71-106: x (float32, 256 * n) into n Q8_K blocks."""
    err = L.RvError()
    _check(_lib().rv_quantize_row_q8_k(_dev(x, "x"), x.numel(), _dev(out, "out"),
                                       _blocks(out, Q8_K_BLOCK_BYTES, "out"), _stream(), 0, byref(err)), err)
    return out


def gemv_q8_k_rows(fmt: int, weight, in_dim: int, out_dim: int, acts, rows, out):
    """gemv.rs:386-411: out[i] = weight_row(rows[0] + i) . acts."""
    lo, hi = rows
    err = L.RvError()
    _check(_lib().rv_gemv_q8_k_rows(fmt, _dev(weight, "weight"), weight.numel(), in_dim, out_dim, _dev(acts, "acts"),
                                    _blocks(acts, Q8_K_BLOCK_BYTES, "acts"), lo, hi, _dev(out, "out"), out.numel(),
                                    _stream(), 0, byref(err)), err)
    return out


def gemv_q8_k(fmt: int, weight, in_dim: int, out_dim: int, acts, out):
    """gemv.rs:347-368."""
    err = L.RvError()
    _check(_lib().rv_gemv_q8_k(fmt, _dev(weight, "weight"), weight.numel(), in_dim, out_dim, _dev(acts, "acts"),
                               _blocks(acts, Q8_K_BLOCK_BYTES, "acts"), _dev(out, "out"), out.numel(), _stream(), 0,
                               byref(err)), err)
    return out


def gemv_q8_0_rows(weight, in_dim: int, out_dim: int, acts, rows, out):
    """gemv.rs:579-615."""
    lo, hi = rows
    err = L.RvError()
    _check(_lib().rv_gemv_q8_0_rows(_dev(weight, "weight"), weight.numel(), in_dim, out_dim, _dev(acts, "acts"),
                                    _blocks(acts, Q8_0_BLOCK_BYTES, "acts"), lo, hi, _dev(out, "out"), out.numel(),
                                    _stream(), 0, byref(err)), err)
    return out


def gemv_q8_0(weight, in_dim: int, out_dim: int, acts, out):
    """gemv.rs:544-577."""
    err = L.RvError()
    _check(_lib().rv_gemv_q8_0(_dev(weight, "weight"), weight.numel(), in_dim, out_dim, _dev(acts, "acts"),
                               _blocks(acts, Q8_0_BLOCK_BYTES, "acts"), _dev(out, "out"), out.numel(), _stream(), 0,
                               byref(err)), err)
    return out


def gemv_q8_k_batched(fmt: int, weight, in_dim: int, out_dim: int, acts, n_acts: int, rows, out):
    """gemv.rs:444-478: out[i * n_acts + a] = weight_row(rows[0] + i) . act_row(a)."""
    lo, hi = rows
    err = L.RvError()
    _check(_lib().rv_gemv_q8_k_batched(fmt, _dev(weight, "weight"), weight.numel(), in_dim, out_dim,
                                       _dev(acts, "acts"), _blocks(acts, Q8_K_BLOCK_BYTES, "acts"), n_acts, lo, hi,
                                       _dev(out, "out"), out.numel(), _stream(), 0, byref(err)), err)
    return out


def gemv_q8_0_batched(weight, in_dim: int, out_dim: int, acts, n_acts: int, rows, out):
    """gemv.rs:616-651, the Q8_0 sibling."""
    lo, hi = rows
    err = L.RvError()
    _check(_lib().rv_gemv_q8_0_batched(_dev(weight, "weight"), weight.numel(), in_dim, out_dim, _dev(acts, "acts"),
                                       _blocks(acts, Q8_0_BLOCK_BYTES, "acts"), n_acts, lo, hi, _dev(out, "out"),
                                       out.numel(), _stream(), 0, byref(err)), err)
    return out


def attn_in_proj_scratch_bytes(hidden: int) -> int:
    return int(_lib().rv_attn_in_proj_scratch_bytes(hidden))


def attn_out_proj_scratch_bytes(q_dim: int) -> int:
    return int(_lib().rv_attn_out_proj_scratch_bytes(q_dim))


def attn_in_proj(normed, q_format: int, wq, q, wk, k, v_format: int, wv, v, scratch=None):
    """forward.rs:2574-2612: q = Wq.x (k-quant), k = Wk.x (Q8_0), v = Wv.x
    (k-quant) for one normed hidden row x, quantized both ways into scratch."""
    import torch
    hidden = normed.numel()
    if scratch is None:
        scratch = torch.empty(max(16, attn_in_proj_scratch_bytes(hidden)), dtype=torch.uint8, device=normed.device)
    err = L.RvError()
    _check(_lib().rv_attn_in_proj(_dev(normed, "normed"), hidden, q_format, _dev(wq, "wq"), wq.numel(), _dev(q, "q"),
                                  q.numel(), _dev(wk, "wk"), wk.numel(), _dev(k, "k"), k.numel(), v_format,
                                  _dev(wv, "wv"), wv.numel(), _dev(v, "v"), _dev(scratch, "scratch"), scratch.numel(),
                                  _stream(), 0, byref(err)), err)
    return q, k, v


def attn_out_proj(attn_out, o_format: int, wo, o, scratch=None):
    """forward.rs:2630-2646: o = Wo . quantize_q8_k(attn_out)."""
    import torch
    q_dim = attn_out.numel()
    if scratch is None:
        scratch = torch.empty(max(16, attn_out_proj_scratch_bytes(q_dim)), dtype=torch.uint8, device=attn_out.device)
    err = L.RvError()
    _check(_lib().rv_attn_out_proj(_dev(attn_out, "attn_out"), q_dim, o_format, _dev(wo, "wo"), wo.numel(),
                                   _dev(o, "o"), o.numel(), _dev(scratch, "scratch"), scratch.numel(), _stream(), 0,
                                   byref(err)), err)
    return o


def attn_in_proj_rows(normed_rows, q_format: int, wq, q_rows, wk, k_rows, v_format: int, wv, v_rows, scratch=None):
    """prefill.rs:1985-2053: q/k/v rows [n][dim] of a chunk's normed rows [n][hidden]."""
    import torch
    n, hidden = normed_rows.shape
    if scratch is None:
        scratch = torch.empty(max(16, int(_lib().rv_attn_in_proj_rows_scratch_bytes(n, hidden))), dtype=torch.uint8,
                              device=normed_rows.device)
    err = L.RvError()
    _check(_lib().rv_attn_in_proj_rows(_dev(normed_rows, "normed_rows"), n, hidden, q_format, _dev(wq, "wq"),
                                       wq.numel(), _dev(q_rows, "q_rows"), q_rows.shape[1], _dev(wk, "wk"), wk.numel(),
                                       _dev(k_rows, "k_rows"), k_rows.shape[1], v_format, _dev(wv, "wv"), wv.numel(),
                                       _dev(v_rows, "v_rows"), _dev(scratch, "scratch"), scratch.numel(), _stream(),
                                       0, byref(err)), err)
    return q_rows, k_rows, v_rows


def attn_out_proj_rows(attn_rows, o_format: int, wo, residual_rows, scratch=None):
    """prefill.rs:2113-2154: residual_rows[n][hidden] += Wo . quantize_q8_k(attn_rows[n][q_dim])."""
    import torch
    n, q_dim = attn_rows.shape
    if scratch is None:
        scratch = torch.empty(max(16, int(_lib().rv_attn_out_proj_rows_scratch_bytes(n, q_dim))), dtype=torch.uint8,
                              device=attn_rows.device)
    err = L.RvError()
    _check(_lib().rv_attn_out_proj_rows(_dev(attn_rows, "attn_rows"), n, q_dim, o_format, _dev(wo, "wo"), wo.numel(),
                                        _dev(residual_rows, "residual_rows"), residual_rows.shape[1],
                                        _dev(scratch, "scratch"), scratch.numel(), _stream(), 0, byref(err)), err)
    return residual_rows


"""One layer's attention block for one token on the GPU (include/ramvamp_block.h).

model/forward.rs:2570-2650 as one call: RMSNorm of the residual, the q/k/v
projections, per-head QK-RMSNorm and RoPE, the KV append, decode attention,
the output projection and the residual add, all on device tensors and
queued on torch's current stream (which the cache is bound to). Five
launches, no host round trip; capture a token's layers into one graph with
``torch.cuda.graph`` after one eager call (the first call sizes the cache's
workspaces).
"""
from __future__ import annotations

from ctypes import byref, c_void_p
from dataclasses import dataclass

from . import _lib as L
from .attention import KvCache, _check


@dataclass
class AttnBlockWeights:
    """One layer's attention weights (device tensors): attn_norm, q_norm and
    k_norm float32; wq, wk (Q8_0), wv and wo as uint8 packed rows."""
    attn_norm: object
    q_format: int
    wq: object
    wk: object
    v_format: int
    wv: object
    q_norm: object
    k_norm: object
    o_format: int
    wo: object

    def _c(self) -> L.RvAttnBlockWeights:
        def p(t):
            if t is None:
                return None
            if not (hasattr(t, "is_cuda") and t.is_cuda and t.is_contiguous()):
                raise TypeError("attention weights must be contiguous torch tensors on the GPU")
            return t.data_ptr()
        return L.RvAttnBlockWeights(p(self.attn_norm), self.q_format, p(self.wq), self.wq.numel(), p(self.wk),
                                    self.wk.numel(), self.v_format, p(self.wv), self.wv.numel(), p(self.q_norm),
                                    p(self.k_norm), self.o_format, p(self.wo), self.wo.numel(), self.q_norm.numel(),
                                    self.k_norm.numel())


def scratch_bytes(hidden: int, q_dim: int, kv_dim: int) -> int:
    return int(L.load().rv_attn_block_scratch_bytes(hidden, q_dim, kv_dim))


def attn_block_decode(cache: KvCache, layer: int, residual, q_dim: int, w: AttnBlockWeights, eps: float,
                      theta: float, position: int, scale: float, scratch=None):
    """forward.rs:2570-2650 for `layer`: residual (float32 [hidden], device)
    is updated in place; returns it."""
    import torch
    if not (hasattr(residual, "is_cuda") and residual.is_cuda and residual.is_contiguous()):
        raise TypeError("residual must be a contiguous torch tensor on the GPU")
    hidden = residual.numel()
    if scratch is None:
        scratch = torch.empty(max(256, scratch_bytes(hidden, q_dim, cache.kv_dim())), dtype=torch.uint8,
                              device=residual.device)
    cache._bind_stream()
    err = L.RvError()
    cw = w._c()
    _check(L.load().rv_attn_block_decode(cache.handle, layer, c_void_p(residual.data_ptr()), hidden, q_dim, byref(cw),
                                         eps, theta, position, scale, c_void_p(scratch.data_ptr()), scratch.numel(),
                                         0, byref(err)), err)
    return residual


def attn_block_decode_dev(cache: KvCache, layer: int, residual, q_dim: int, w: AttnBlockWeights, eps: float,
                          theta: float, d_position, max_position: int, scale: float, scratch):
    """rv_attn_block_decode_dev (no reference counterpart): attn_block_decode
    at the position ``d_position`` (int32 device tensor) holds when the step
    runs, planned for ``max_position``; the layer's length does not move
    (``KvCache.commit``). ``scratch`` is required: a token graph keeps it."""
    from .attention import _position_ptr
    if not (hasattr(residual, "is_cuda") and residual.is_cuda and residual.is_contiguous()):
        raise TypeError("residual must be a contiguous torch tensor on the GPU")
    cache._bind_stream()
    err = L.RvError()
    cw = w._c()
    _check(L.load().rv_attn_block_decode_dev(cache.handle, layer, c_void_p(residual.data_ptr()), residual.numel(),
                                             q_dim, byref(cw), eps, theta, _position_ptr(d_position), max_position,
                                             scale, c_void_p(scratch.data_ptr()), scratch.numel(), 0, byref(err)),
           err)
    return residual


_MODES ={"exact": L.RV_PREFILL_EXACT, "f16": L.RV_PREFILL_F16, "bf16": L.RV_PREFILL_BF16}


def prefill_scratch_bytes(n_rows: int, hidden: int, q_dim: int, kv_dim: int) -> int:
    return int(L.load().rv_attn_block_prefill_scratch_bytes(n_rows, hidden, q_dim, kv_dim))


def attn_block_prefill(cache: KvCache, layer: int, residual_rows, q_dim: int, w: AttnBlockWeights, eps: float,
                       theta: float, start: int, scale: float, mode: str = "exact", scratch=None):
    """prefill.rs:1975-2154 (the attention half of a layer) for a chunk:
    residual_rows (float32 [n][hidden], device) is updated in place."""
    import torch
    if not (hasattr(residual_rows, "is_cuda") and residual_rows.is_cuda and residual_rows.is_contiguous()):
        raise TypeError("residual_rows must be a contiguous torch tensor on the GPU")
    n, hidden = residual_rows.shape
    if scratch is None:
        scratch = torch.empty(max(256, prefill_scratch_bytes(n, hidden, q_dim, cache.kv_dim())), dtype=torch.uint8,
                              device=residual_rows.device)
    cache._bind_stream()
    err = L.RvError()
    cw = w._c()
    _check(L.load().rv_attn_block_prefill(cache.handle, layer, c_void_p(residual_rows.data_ptr()), n, hidden, q_dim,
                                          byref(cw), eps, theta, start, scale, c_void_p(scratch.data_ptr()),
                                          scratch.numel(), _MODES[mode], byref(err)), err)
    return residual_rows


"""The MoE router's decision on the GPU (include/ramvamp_router.h).

model/forward.rs:2658-2705: per row, the router matrix times the normed row
(one serial f32 sum per expert), softmax over the experts, the top_k
largest probabilities (first index wins ties), renormalized when
norm_topk_prob. Device tensors, torch's current stream; the same values as
the reference, bit for bit.
"""
from __future__ import annotations

from ctypes import byref, c_void_p

from . import _lib as L
from .attention import _check, _raw_stream


def router_topk(x, router, top_k: int, norm_topk_prob: bool, experts=None, weights=None):
    """x: float32 [n_rows][hidden] (or [hidden]); router: float32 [n_experts][hidden].
    Returns (experts uint32-as-int32 [n_rows][top_k], weights float32 [n_rows][top_k])."""
    import torch
    for t, what in ((x, "x"), (router, "router")):
        if not (hasattr(t, "is_cuda") and t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
            raise TypeError(f"{what} must be a contiguous float32 torch tensor on the GPU")
    rows = x.reshape(-1, x.shape[-1])
    n_rows, hidden = rows.shape
    n_experts = router.shape[0]
    if experts is None:
        experts = torch.empty(n_rows, top_k, dtype=torch.int32, device=x.device)
    if weights is None:
        weights = torch.empty(n_rows, top_k, dtype=torch.float32, device=x.device)
    err = L.RvError()
    _check(L.load().rv_router_topk(c_void_p(rows.data_ptr()), n_rows, hidden, c_void_p(router.data_ptr()),
                                   router.numel(), n_experts, top_k, int(bool(norm_topk_prob)),
                                   c_void_p(experts.data_ptr()), c_void_p(weights.data_ptr()),
                                   c_void_p(_raw_stream(torch.cuda.current_device())), 0, byref(err)), err)
    return experts, weights

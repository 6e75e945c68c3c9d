"""Loads libramvamp_attn.so (the gfx950 HIP library) and declares its C ABI.

The library is built in-tree by ``ramvamp_amd.build`` (hipcc --offload-arch=gfx950).
There is no fallback: if the library is missing, importing the compute API
raises, so nothing can silently run on the CPU instead.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libramvamp_attn.so")

RV_HOST_PTRS = 0x1
RV_SYNC = 0x2
RV_PREFILL_EXACT = 0x00
RV_PREFILL_F16 = 0x10
RV_PREFILL_BF16 = 0x20
RV_ELEM_F16 = 1
RV_ELEM_F32 = 2
RV_TUNE_DECODE_SPLIT_LEN = 1
RV_TUNE_PREFILL_KV_SPLIT = 2
RV_TUNE_DECODE_WAVES = 3
RV_TUNE_PREFILL_ROWS = 4
RV_TUNE_DECODE_HG = 5
RV_TUNE_DECODE_IMPL = 6
RV_TUNE_KERNEL_TIMING = 7
RV_TUNE_DECODE_DEPTH = 9
RV_TUNE_DECODE_MERGE = 11
RV_NOALLOC_SCRATCH_BYTES = 8 << 20
# include/ramvamp_gemv.h
RV_QF_Q4_K = 1
RV_QF_Q5_K = 2
RV_QF_Q6_K = 3
RV_QF_Q8_0 = 4
RV_QF_Q8_K = 5
# include/ramvamp_floors.h
RV_FLOOR_MFMA_F16_16X16X32 = 0
RV_FLOOR_MFMA_F16_32X32X16 = 1
RV_FLOOR_MFMA_F32_16X16X4 = 2
RV_FLOOR_VALU_FMA = 0
RV_FLOOR_VALU_EXP = 1


class RvError(ctypes.Structure):
    _fields_ = [("code", c_int32), ("a", c_uint64), ("b", c_uint64), ("c", c_uint64), ("d", c_uint64),
                ("what", c_char_p)]


class RvAttnBlockWeights(ctypes.Structure):
    """rv_attn_block_weights (include/ramvamp_block.h)."""
    _fields_ = [("attn_norm", c_void_p), ("q_format", c_uint32), ("wq", c_void_p), ("wq_len", c_size_t),
                ("wk", c_void_p), ("wk_len", c_size_t), ("v_format", c_uint32), ("wv", c_void_p),
                ("wv_len", c_size_t), ("q_norm", c_void_p), ("k_norm", c_void_p), ("o_format", c_uint32),
                ("wo", c_void_p), ("wo_len", c_size_t), ("q_norm_len", c_size_t), ("k_norm_len", c_size_t)]


# Every symbol include/*.h declares: name -> (restype, argtypes).
_E = POINTER(RvError)
_P = c_void_p
SIGNATURES = {
    "rv_abi_version": (c_uint32, []),
    "rv_status_name": (c_char_p, [c_int32]),
    "rv_scratch_len": (c_size_t, [c_size_t, c_size_t, c_size_t, c_size_t]),
    "rv_kv_projected_bytes": (c_int32, [c_size_t, c_size_t, c_size_t, c_size_t, c_int, POINTER(c_uint64), _E]),
    "rv_kv_new": (c_int32, [c_size_t, c_size_t, c_size_t, c_size_t, c_int, c_int, POINTER(c_void_p), _E]),
    "rv_kv_free": (None, [_P]),
    "rv_kv_set_stream": (c_int32, [_P, _P, _E]),
    "rv_kv_synchronize": (c_int32, [_P, _E]),
    "rv_kv_n_layers": (c_size_t, [_P]),
    "rv_kv_n_kv_heads": (c_size_t, [_P]),
    "rv_kv_head_dim": (c_size_t, [_P]),
    "rv_kv_capacity": (c_size_t, [_P]),
    "rv_kv_kv_dim": (c_size_t, [_P]),
    "rv_kv_elem": (c_int32, [_P]),
    "rv_kv_len": (c_int32, [_P, c_size_t, POINTER(c_size_t), _E]),
    "rv_kv_is_empty": (c_int, [_P]),
    "rv_kv_seq_len": (c_int32, [_P, POINTER(c_size_t), _E]),
    "rv_kv_append": (c_int32, [_P, c_size_t, _P, c_size_t, _P, c_size_t, c_uint32, _E]),
    "rv_kv_append_rows": (c_int32, [_P, c_size_t, _P, _P, c_size_t, c_size_t, c_uint32, _E]),
    "rv_kv_clear": (None, [_P]),
    "rv_kv_truncate": (c_int32, [_P, c_size_t, _E]),
    "rv_kv_k_layer": (c_int32, [_P, c_size_t, POINTER(c_void_p), POINTER(c_size_t), _E]),
    "rv_kv_v_layer": (c_int32, [_P, c_size_t, POINTER(c_void_p), POINTER(c_size_t), _E]),
    "rv_kv_read_row": (c_int32, [_P, c_int, c_size_t, c_size_t, _P, _E]),
    "rv_decode_attention": (c_int32, [_P, _P, c_size_t, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_decode_attention_in": (c_int32, [_P, _P, c_size_t, c_size_t, c_float, c_size_t, _P, c_size_t, c_uint32, _E]),
    "rv_decode_attention_kv_range_in": (c_int32, [_P, _P, c_size_t, c_size_t, c_float, c_size_t, c_size_t, c_size_t,
                                                  _P, c_size_t, c_uint32, _E]),
    "rv_attention_at": (c_int32, [_P, _P, c_size_t, c_size_t, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_attention_at_in": (c_int32, [_P, _P, c_size_t, c_size_t, c_size_t, c_float, c_size_t, _P, c_size_t, c_uint32,
                                     _E]),
    "rv_attention_at_kv_range_in": (c_int32, [_P, _P, c_size_t, c_size_t, c_size_t, c_float, c_size_t, c_size_t,
                                              c_size_t, _P, c_size_t, c_uint32, _E]),
    "rv_attention_at_rows": (c_int32, [_P, _P, c_size_t, c_size_t, c_size_t, c_size_t, c_float, _P, c_uint32, _E]),
    "rv_decode_step": (c_int32, [_P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t,
                                 c_float, c_float, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_decode_step_dev": (c_int32, [_P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P,
                                     c_size_t, c_float, c_float, _P, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_kv_commit": (c_int32, [_P, c_size_t, c_size_t, _E]),
    "rv_position_advance": (c_int32, [_P, _P, c_uint32, _E]),
    "rv_prefill_chunk": (c_int32, [_P, c_size_t, _P, _P, _P, c_size_t, c_size_t, _P, c_size_t, _P, c_size_t, c_float,
                                   c_float, c_size_t, c_float, _P, c_uint32, _E]),
    "rv_decode_attention_noalloc": (c_int32, [_P, _P, c_size_t, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_kv_set_tuning": (c_int32, [_P, c_int32, c_int64, _E]),
    "rv_kv_kernel_time": (c_int32, [_P, POINTER(c_double), POINTER(c_uint64), _E]),
    "rv_kv_device_status": (c_int32, [_P, _E]),
    "rv_kv_device_bytes": (c_int32, [_P, POINTER(c_uint64), POINTER(c_uint64), _E]),
    "rv_kv_xcd_dealing": (c_int32, [_P, POINTER(c_int32), _E]),
    "rv_kv_projected_device_bytes": (c_int32, [c_size_t, c_size_t, c_size_t, c_size_t, c_int, POINTER(c_uint64), _E]),
    # include/ramvamp_gemv.h
    "rv_quant_block_weights": (c_size_t, [c_uint32]),
    "rv_quant_block_bytes": (c_size_t, [c_uint32]),
    "rv_quant_row_bytes": (c_int32, [c_uint32, c_size_t, POINTER(c_size_t), _E]),
    "rv_quantize_row_q8_0": (c_int32, [_P, c_size_t, _P, c_size_t, _P, c_uint32, _E]),
    "rv_quantize_row_q8_k": (c_int32, [_P, c_size_t, _P, c_size_t, _P, c_uint32, _E]),
    "rv_gemv_q8_k_rows": (c_int32, [c_uint32, _P, c_size_t, c_size_t, c_size_t, _P, c_size_t, c_size_t, c_size_t, _P,
                                    c_size_t, _P, c_uint32, _E]),
    "rv_gemv_q8_k": (c_int32, [c_uint32, _P, c_size_t, c_size_t, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_uint32,
                               _E]),
    "rv_gemv_q8_0_rows": (c_int32, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, c_size_t, c_size_t, _P, c_size_t,
                                    _P, c_uint32, _E]),
    "rv_gemv_q8_0": (c_int32, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_uint32, _E]),
    "rv_gemv_q8_k_batched": (c_int32, [c_uint32, _P, c_size_t, c_size_t, c_size_t, _P, c_size_t, c_size_t, c_size_t,
                                       c_size_t, _P, c_size_t, _P, c_uint32, _E]),
    "rv_gemv_q8_0_batched": (c_int32, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, c_size_t, c_size_t, c_size_t,
                                       _P, c_size_t, _P, c_uint32, _E]),
    "rv_attn_in_proj_rows_scratch_bytes": (c_size_t, [c_size_t, c_size_t]),
    "rv_attn_in_proj_rows": (c_int32, [_P, c_size_t, c_size_t, c_uint32, _P, c_size_t, _P, c_size_t, _P, c_size_t,
                                       _P, c_size_t, c_uint32, _P, c_size_t, _P, _P, c_size_t, _P, c_uint32, _E]),
    "rv_attn_out_proj_rows_scratch_bytes": (c_size_t, [c_size_t, c_size_t]),
    "rv_attn_out_proj_rows": (c_int32, [_P, c_size_t, c_size_t, c_uint32, _P, c_size_t, _P, c_size_t, _P, c_size_t,
                                        _P, c_uint32, _E]),
    "rv_attn_in_proj_scratch_bytes": (c_size_t, [c_size_t]),
    "rv_attn_in_proj": (c_int32, [_P, c_size_t, c_uint32, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t,
                                  c_uint32, _P, c_size_t, _P, _P, c_size_t, _P, c_uint32, _E]),
    "rv_attn_out_proj_scratch_bytes": (c_size_t, [c_size_t]),
    "rv_attn_out_proj": (c_int32, [_P, c_size_t, c_uint32, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_uint32,
                                   _E]),
    "rv_router_topk": (c_int32, [_P, c_size_t, c_size_t, _P, c_size_t, c_size_t, c_size_t, c_int, _P, _P, _P,
                                 c_uint32, _E]),
    "rv_attn_block_scratch_bytes": (c_size_t, [c_size_t, c_size_t, c_size_t]),
    "rv_attn_block_prefill_scratch_bytes": (c_size_t, [c_size_t, c_size_t, c_size_t, c_size_t]),
    "rv_attn_block_prefill": (c_int32, [_P, c_size_t, _P, c_size_t, c_size_t, c_size_t, POINTER(RvAttnBlockWeights),
                                        c_float, c_float, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_attn_block_decode": (c_int32, [_P, c_size_t, _P, c_size_t, c_size_t, POINTER(RvAttnBlockWeights), c_float,
                                       c_float, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    "rv_attn_block_decode_dev": (c_int32, [_P, c_size_t, _P, c_size_t, c_size_t, POINTER(RvAttnBlockWeights),
                                           c_float, c_float, _P, c_size_t, c_float, _P, c_size_t, c_uint32, _E]),
    # include/ramvamp_floors.h
    "rv_floor_empty": (c_int32, [_P, _E]),
    "rv_floor_stream_read": (c_int32, [_P, c_size_t, c_uint32, _P, _P, _E]),
    "rv_floor_mfma": (c_int32, [c_int32, c_uint32, c_uint32, c_uint32, _P, _P, _E]),
    "rv_floor_mfma_valu": (c_int32, [c_int32, c_uint32, c_uint32, c_uint32, _P, _P, _E]),
}

_lib = None


def load(path: str = LIB_PATH):
    """The library with every ABI symbol typed. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build the gfx950 HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()'). There is no CPU fallback.")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib

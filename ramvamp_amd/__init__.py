"""ramvamp_amd — MI355X-native (gfx950) GQA attention hot path of ramvamp.

The product is ``libramvamp_attn.so`` (hand-written HIP kernels behind the C
ABI in include/ramvamp_attn.h, ramvamp_gemv.h and ramvamp_block.h). This package
builds it (``build``), loads it (``_lib``), mirrors the reference's Rust
attention API (``attention``) and quantized projections (``projections``)
over it, one layer's attention block as a single device call (``block``),
and makes seeded synthetic inputs (``synth``).
"""
from .attention import (  # noqa: F401
    AttentionError,
    AttentionScratch,
    DeviceError,
    KernelError,
    KvCache,
    KvError,
    PrimitiveError,
    RamvampError,
    attention_at,
    attention_at_in,
    attention_at_kv_range_in,
    attention_at_rows,
    decode_attention,
    decode_attention_in,
    decode_attention_kv_range_in,
    decode_attention_noalloc,
    decode_step,
    decode_step_dev,
    position_advance,
    prefill_chunk,
    scratch_len,
)
from ._lib import (  # noqa: F401  (knobs of KvCache.set_tuning)
    RV_TUNE_DECODE_DEPTH,
    RV_TUNE_DECODE_HG,
    RV_TUNE_DECODE_IMPL,
    RV_TUNE_DECODE_MERGE,
    RV_TUNE_DECODE_SPLIT_LEN,
    RV_TUNE_DECODE_WAVES,
    RV_TUNE_KERNEL_TIMING,
    RV_TUNE_PREFILL_KV_SPLIT,
    RV_TUNE_PREFILL_ROWS,
)
from . import block, projections, router  # noqa: F401,E402

"""Seeded synthetic inputs for the five benchmark configurations.

N(0,1) draws come from a counter-based generator, so any slice of a tensor
can be regenerated independently and the whole thing vectorises in numpy:
value pair i of a stream is Box-Muller (f64) of splitmix64(key + 2i) and
splitmix64(key + 2i + 1), key = splitmix64(seed). Seeds follow one scheme,
``0x5EED0000 | cfg << 8 | tensor``, with the layer mixed into bits 32 and up
(tensor ids: q 1, k 2, v 3, q_norm 4, k_norm 5, k cache 6, v cache 7).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

N_Q_HEADS, N_KV_HEADS, HEAD_DIM = 32, 4, 128
Q_DIM, KV_DIM = N_Q_HEADS * HEAD_DIM, N_KV_HEADS * HEAD_DIM
EPS = np.float32(1e-6)
THETA = np.float32(1e6)
SCALE = np.float32(1.0) / np.sqrt(np.float32(HEAD_DIM))  # forward.rs:2475, in f32

T_Q, T_K, T_V, T_QN, T_KN, T_KC, T_VC = 1, 2, 3, 4, 5, 6, 7

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def seed(cfg: int, tensor: int, layer: int = 0) -> int:
    return (0x5EED0000 | (cfg << 8) | tensor) ^ (layer << 32)


def normal(seed_: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n float32 draws of N(mean, std^2)."""
    pairs = (n + 1) // 2
    key = _splitmix64(np.array([seed_ & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))[0]
    i = np.arange(pairs, dtype=np.uint64)
    with np.errstate(over="ignore"):
        a = _splitmix64(key + np.uint64(2) * i)
        b = _splitmix64(key + np.uint64(2) * i + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)  # (0, 1]
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)          # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * math.pi * u2)
    z[1::2] = r * np.sin(2.0 * math.pi * u2)
    return (z[:n] * std + mean).astype(np.float32)


def rope_f64(x: np.ndarray, head_dim: int, position: int, theta: float) -> np.ndarray:
    """NeoX RoPE of every head of x at one position (setup only: f64 angles, f32 result)."""
    h = np.asarray(x, dtype=np.float64).reshape(-1, head_dim)
    half = head_dim // 2
    i = np.arange(half, dtype=np.float64)
    ang = position * np.power(float(np.float32(theta)), -2.0 * i / head_dim)
    c, s = np.cos(ang), np.sin(ang)
    out = np.empty_like(h)
    out[:, :half] = h[:, :half] * c - h[:, half:] * s
    out[:, half:] = h[:, :half] * s + h[:, half:] * c
    return out.reshape(-1).astype(np.float32)


@dataclass
class Config:
    """One BASELINE.json configuration (index 1..5)."""

    cfg: int
    name: str
    kind: str            # "decode_step" | "decode" | "prefill"
    layers: int
    context: int         # cached positions before the timed op
    rows: int            # new rows (decode: 1)
    elem: str            # KV element type
    capacity: int
    notes: str = ""
    extra: dict = field(default_factory=dict)


CONFIGS = {
    1: Config(1, "decode ctx 512 + 1 (fused prologue)", "decode_step", 1, 512, 1, "f32", 513,
              "cached K/V normed+RoPE'd from pre-norm N(0,1) at 0..511; new pre-norm q,k,v at 512"),
    2: Config(2, "decode ctx 4096 x 48 layers", "decode", 48, 4096, 1, "f32", 4096,
              "post-RoPE N(0,1) K/V at 0..4095 per layer; q N(0,1) per layer"),
    3: Config(3, "causal prefill 512 (empty cache)", "prefill", 1, 0, 512, "f32", 512,
              "pre-norm N(0,1) Q/K/V rows at 0..511"),
    4: Config(4, "prefix-reuse prefill 512 at 3449", "prefill", 1, 3449, 512, "f32", 3961,
              "post-RoPE N(0,1) K/V at 0..3448; pre-norm Q/K/V rows at 3449..3960"),
    5: Config(5, "split-K decode ctx 32768 (f16 KV)", "decode", 1, 32768, 1, "f16", 32768,
              "f16 cast of post-RoPE N(0,1) K/V at 0..32767; q N(0,1) RoPE'd at 32768"),
}


def norm_weight(cfg: int, tensor: int, layer: int = 0) -> np.ndarray:
    return normal(seed(cfg, tensor, layer), HEAD_DIM, 1.0, 0.02)


def cached_kv(cfg: int, layer: int, positions: int):
    """Post-RoPE K and V rows 0..positions of one layer, each (positions, KV_DIM) f32."""
    k = normal(seed(cfg, T_KC, layer), positions * KV_DIM)
    v = normal(seed(cfg, T_VC, layer), positions * KV_DIM)
    return k.reshape(positions, KV_DIM), v.reshape(positions, KV_DIM)


def new_rows(cfg: int, rows: int, layer: int = 0):
    """Pre-norm q (rows, Q_DIM), k and v (rows, KV_DIM)."""
    q = normal(seed(cfg, T_Q, layer), rows * Q_DIM).reshape(rows, Q_DIM)
    k = normal(seed(cfg, T_K, layer), rows * KV_DIM).reshape(rows, KV_DIM)
    v = normal(seed(cfg, T_V, layer), rows * KV_DIM).reshape(rows, KV_DIM)
    return q, k, v

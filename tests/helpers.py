"""Shared test helpers, restating the reference's own test scaffolding.

- ``Rng``: the xorshift64* generator of crates/core/src/kernels/attention.rs:1317-1341
  (same as kernels/primitives/testutil.rs:5-34): seeds and draws match the
  reference tests bit for bit.
- ``assert_close``: the mixed rel/abs gate of attention.rs:1345-1356.
- ``reference_attention``: the naive f64 attention of attention.rs:1360-1403,
  vectorised with numpy (a textbook routine, not the reference's kernel).
- ``round_trip``: one f16 round trip (attention.rs:1406-1410), through numpy's
  IEEE float16 conversion.
"""
from __future__ import annotations

import numpy as np

MASK64 = (1 << 64) - 1


class Rng:
    def __init__(self, seed: int):
        self.s = (seed | 1) & MASK64

    def next_u64(self) -> int:
        x = self.s
        x ^= (x << 13) & MASK64
        x ^= x >> 7
        x ^= (x << 17) & MASK64
        self.s = x
        return (x * 0x2545F4914F6CDD1D) & MASK64

    def f32_in(self, lo: float, hi: float) -> np.float32:
        unit = np.float32(self.next_u64() >> 40) / np.float32(1 << 24)
        return np.float32(lo) + (np.float32(hi) - np.float32(lo)) * unit

    def vec_in(self, n: int, lo: float, hi: float) -> np.ndarray:
        raw = np.fromiter((self.next_u64() >> 40 for _ in range(n)), dtype=np.uint64, count=n)
        unit = raw.astype(np.float32) / np.float32(1 << 24)
        return (np.float32(lo) + (np.float32(hi) - np.float32(lo)) * unit).astype(np.float32)


def assert_close(actual, expected, rel_tol: float, abs_tol: float, what: str = ""):
    """Elementwise: |a-e| <= abs_tol or |a-e|/|e| <= rel_tol (attention.rs:1345-1356)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    diff = np.abs(a - e)
    rel = diff / np.maximum(np.abs(e), np.finfo(np.float64).tiny)
    bad = ~((diff <= abs_tol) | (rel <= rel_tol))
    if np.any(bad):
        i = int(np.flatnonzero(bad.ravel())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance; first at {i}: "
            f"actual {a.ravel()[i]!r} expected {e.ravel()[i]!r} rel {rel.ravel()[i]:.3e} > {rel_tol:.1e} "
            f"(abs {diff.ravel()[i]:.3e} > {abs_tol:.1e})")


def max_rel_err(actual, expected, floor: float) -> float:
    """max |a-e| / max(|e|, floor): the fp32-mode parity metric."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(np.abs(e), floor))) if a.size else 0.0


def round_trip(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def reference_attention(q, k_rows, v_rows, n_kv_heads: int, head_dim: int, scale: float) -> np.ndarray:
    """f64 textbook GQA attention. q [n_q*d]; k_rows/v_rows [len, n_kv*d]."""
    q = np.asarray(q, dtype=np.float64).reshape(-1, head_dim)
    K = np.asarray(k_rows, dtype=np.float64).reshape(-1, n_kv_heads, head_dim)
    V = np.asarray(v_rows, dtype=np.float64).reshape(-1, n_kv_heads, head_dim)
    n_q = q.shape[0]
    group = n_q // n_kv_heads
    out = np.zeros((n_q, head_dim))
    for h in range(n_q):
        j = h // group
        s = (K[:, j, :] @ q[h]) * float(np.float32(scale))
        s = np.exp(s - s.max())
        s /= s.sum()
        out[h] = s @ V[:, j, :]
    return out.reshape(-1)


def reference_causal_rows(q_rows, k_rows, v_rows, n_kv_heads: int, head_dim: int, scale: float, start: int):
    """Row r attends positions 0..start+r+1 (model/prefill.rs:1394), f64."""
    q_rows = np.asarray(q_rows, dtype=np.float64)
    out = np.zeros_like(q_rows)
    for r in range(q_rows.shape[0]):
        n = start + r + 1
        out[r] = reference_attention(q_rows[r], k_rows[:n], v_rows[:n], n_kv_heads, head_dim, scale)
    return out

"""Test helpers for the quantized projections: the reference's seeded LCG and
its test-only weight quantizers (kernels/quants/test_support.rs), and random
packed weight rows for the GPU parity tests.

The weight quantizers exist only to make valid, representative blocks (the
runtime never quantizes weights); they follow test_support.rs:21-234 with f32
arithmetic via numpy float32 and the oracle's f16 conversions.
"""
from __future__ import annotations

import numpy as np

import oracle

F32 = np.float32
M64 = (1 << 64) - 1


class Lcg:
    """test_support.rs:21-40: Knuth MMIX LCG; next_f32 in [-1, 1)."""

    def __init__(self, seed: int):
        self.s = seed & M64

    def next_u64(self) -> int:
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & M64
        return self.s

    def next_f32(self) -> np.float32:
        return F32(F32(self.next_u64() >> 40) / F32(1 << 24)) * F32(2.0) - F32(1.0)

    def f32s(self, n: int, scale: float) -> np.ndarray:
        return np.array([self.next_f32() * F32(scale) for _ in range(n)], dtype=F32)


def round_away(t) -> float:
    """Rust's f32::round (half away from zero), exactly: in f64, where
    |t| + 0.5 cannot round for an f32 t."""
    t = float(t)
    return float(np.sign(t) * np.floor(abs(t) + 0.5))


def f16r(x) -> np.float32:
    """f32 -> f16 (RNE) -> f32 through the oracle's pinned conversions."""
    return F32(oracle.f16_to_f32(oracle.f32_to_f16(np.float32(x)))[0])


def f16_bytes(x) -> bytes:
    return int(oracle.f32_to_f16(np.float32(x))[0]).to_bytes(2, "little")


def pack_scales_k4(ls, lm) -> bytes:
    """test_support.rs:45-58: inverse of get_scale_min_k4."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] = ls[j] & 63
            s[j + 4] = lm[j] & 63
        else:
            s[j + 4] = (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            s[j - 4] |= (ls[j] >> 4) << 6
            s[j] |= (lm[j] >> 4) << 6
    return bytes(v & 0xFF for v in s)


def _affine_scales(x, levels):
    """test_support.rs:66-98."""
    levels = F32(levels)
    scale_f, min_f = [], []
    for j in range(8):
        sub = x[32 * j:32 * j + 32]
        vmin, vmax = F32(sub.min()), F32(sub.max())
        mn = max(F32(-vmin), F32(0))
        min_f.append(mn)
        scale_f.append(max(F32((vmax + mn) / levels), F32(0)))
    d = f16r(F32(max(scale_f + [F32(0)]) / F32(63)))
    dmin = f16r(F32(max(min_f + [F32(0)]) / F32(63)))
    ls = [int(min(max(np.ceil(F32(sf / d)), 0), 63)) if d > 0 else 0 for sf in scale_f]
    lm = [int(min(max(round_away(F32(mf / dmin)), 0), 63)) if dmin > 0 else 0 for mf in min_f]
    decoded = [(F32(d * F32(ls[j])), F32(dmin * F32(lm[j]))) for j in range(8)]
    return pack_scales_k4(ls, lm), d, dmin, decoded


def _affine_q(v, step, mn, levels):
    """test_support.rs:101-106 (f32 round half away from zero)."""
    if step <= 0:
        return 0
    return int(min(max(round_away(F32(F32(v + mn) / step)), 0), levels))


def quantize_row_q4_k_test(x) -> bytes:
    """test_support.rs:108-126."""
    out = bytearray()
    for xs in np.asarray(x, dtype=F32).reshape(-1, 256):
        scales, d, dmin, dec = _affine_scales(xs, 15)
        q = [_affine_q(xs[32 * j + l], dec[j][0], dec[j][1], 15) for j in range(8) for l in range(32)]
        out += f16_bytes(d) + f16_bytes(dmin) + scales
        for span in range(4):
            out += bytes(q[64 * span + l] | (q[64 * span + 32 + l] << 4) for l in range(32))
    return bytes(out)


def quantize_row_q5_k_test(x) -> bytes:
    """test_support.rs:129-159."""
    out = bytearray()
    for xs in np.asarray(x, dtype=F32).reshape(-1, 256):
        scales, d, dmin, dec = _affine_scales(xs, 31)
        q = [_affine_q(xs[32 * j + l], dec[j][0], dec[j][1], 31) for j in range(8) for l in range(32)]
        qh = [0] * 32
        for j in range(8):
            for l in range(32):
                if q[32 * j + l] >= 16:
                    qh[l] |= 1 << j
        out += f16_bytes(d) + f16_bytes(dmin) + scales + bytes(qh)
        for span in range(4):
            out += bytes((q[64 * span + l] & 0xF) | ((q[64 * span + 32 + l] & 0xF) << 4) for l in range(32))
    return bytes(out)


def quantize_row_q6_k_test(x) -> bytes:
    """test_support.rs:162-218."""
    out = bytearray()
    for xs in np.asarray(x, dtype=F32).reshape(-1, 256):
        scale_f = [F32(np.abs(xs[16 * g:16 * g + 16]).max() / F32(31)) for g in range(16)]
        d = f16r(F32(max(scale_f) / F32(127)))
        ls = [int(min(max(np.ceil(F32(s / d)), 0), 127)) if d > 0 else 0 for s in scale_f]
        q = []
        for g in range(16):
            step = F32(d * F32(ls[g]))
            for l in range(16):
                if step > 0:
                    v = int(min(max(round_away(F32(xs[16 * g + l] / step)), -32), 31))
                else:
                    v = 0
                q.append(v + 32)
        ql, qh = [0] * 128, [0] * 64
        for half in range(2):
            base = 128 * half
            for l in range(32):
                v1, v2, v3, v4 = q[base + l], q[base + l + 32], q[base + l + 64], q[base + l + 96]
                ql[64 * half + l] = (v1 & 0xF) | ((v3 & 0xF) << 4)
                ql[64 * half + l + 32] = (v2 & 0xF) | ((v4 & 0xF) << 4)
                qh[32 * half + l] = (v1 >> 4) | ((v2 >> 4) << 2) | ((v3 >> 4) << 4) | ((v4 >> 4) << 6)
        out += bytes(ql) + bytes(qh) + bytes(ls) + f16_bytes(d)
    return bytes(out)


def quantize_row_q8_0_test(x) -> bytes:
    """test_support.rs:222-234: the activation quantizer's blocks, packed."""
    blocks = oracle.quantize_row_q8_0(np.asarray(x, dtype=F32))
    out = bytearray()
    for b in blocks:
        out += f16_bytes(b["d"]) + b["qs"].astype(np.int8).tobytes()
    return bytes(out)


def random_weight_rows(fmt: int, rows: int, in_dim: int, rng: np.random.Generator, scale_lo=1e-3, scale_hi=0.05):
    """Random packed rows: every quant/scale byte uniform, the f16 scales (d,
    dmin) random finite values in [scale_lo, scale_hi) with random sign for d
    of Q6_K / Q8_0 (their d is signed in general)."""
    bb = oracle.quant_block_bytes(fmt)
    nb = in_dim // oracle.quant_block_weights(fmt)
    w = rng.integers(0, 256, size=(rows, nb, bb), dtype=np.uint8)

    def put_f16(off, signed):
        v = rng.uniform(scale_lo, scale_hi, size=(rows, nb)).astype(F32)
        if signed:
            v *= rng.choice(np.array([-1, 1], dtype=F32), size=(rows, nb))
        bits = oracle.f32_to_f16(v.ravel()).reshape(rows, nb)
        w[:, :, off] = bits & 0xFF
        w[:, :, off + 1] = bits >> 8

    if fmt in (oracle.RV_QF_Q4_K, oracle.RV_QF_Q5_K):
        put_f16(0, False)
        put_f16(2, False)
    elif fmt == oracle.RV_QF_Q6_K:
        put_f16(208, True)
    else:
        put_f16(0, True)
    return w.reshape(rows, nb * bb)

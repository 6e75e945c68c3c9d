"""Pins the oracle's quantized-projection functions (oracle/rv_oracle_quant.c)
with the reference's own known-answer and ground-truth tests
(kernels/quants/quantize.rs:108-203, quants/tests.rs, kernels/gemv.rs), plus
closed forms the code fixes: exact integer identities (bsums, zero
activations), row-range and batch partitions that must be bit-identical.
"""
import numpy as np
import pytest

import oracle
from oracle import RV_QF_Q4_K, RV_QF_Q5_K, RV_QF_Q6_K, RV_QF_Q8_0, RV_QF_Q8_K, OracleError
from quant_util import (Lcg, f16_bytes, quantize_row_q4_k_test, quantize_row_q5_k_test, quantize_row_q6_k_test,
                        quantize_row_q8_0_test, random_weight_rows)

F32 = np.float32
RV_PRIM_LENGTH_MISMATCH = 25
IND, RBN, BCM, QLM, UNS = 40, 41, 42, 43, 44
K_QUANTS = [RV_QF_Q4_K, RV_QF_Q5_K, RV_QF_Q6_K]
TEST_QUANT = {RV_QF_Q4_K: quantize_row_q4_k_test, RV_QF_Q5_K: quantize_row_q5_k_test,
              RV_QF_Q6_K: quantize_row_q6_k_test, RV_QF_Q8_0: quantize_row_q8_0_test}


def dequant_acts(blocks) -> np.ndarray:
    """quants/tests.rs:12-26: d * q per value."""
    return (blocks["d"][:, None] * blocks["qs"].astype(F32)).astype(F32).ravel()


def assert_dot_close(dot, w, a):
    """quants/tests.rs:28-47: within 1e-5 of the f64 dot, relative to the sum
    of term magnitudes."""
    p = w.astype(np.float64) * a.astype(np.float64)
    r, mag = p.sum(), np.abs(p).sum()
    tol = 1e-5 * max(mag, 1e-20)
    assert abs(float(dot) - r) <= tol, (dot, r, tol)


def raises(code, fn, *args, **kw):
    with pytest.raises(OracleError) as e:
        fn(*args, **kw)
    assert e.value.code == code, e.value.payload()
    return e.value


# ---- geometry -----------------------------------------------------------------


def test_row_bytes_known_answers():
    # quants/tests.rs:444-465
    assert oracle.quant_row_bytes(RV_QF_Q4_K, 2048) == 1152
    assert oracle.quant_row_bytes(RV_QF_Q5_K, 768) == 528
    assert oracle.quant_row_bytes(RV_QF_Q6_K, 768) == 630
    assert oracle.quant_row_bytes(RV_QF_Q8_0, 2048) == 2176
    assert oracle.quant_row_bytes(RV_QF_Q8_K, 256) == 292
    assert oracle.quant_row_bytes(RV_QF_Q4_K, 0) == 0
    assert raises(IND, oracle.quant_row_bytes, RV_QF_Q4_K, 100).payload()[1:4] == (RV_QF_Q4_K, 100, 256)
    assert raises(IND, oracle.quant_row_bytes, RV_QF_Q8_0, 33).payload()[1:4] == (RV_QF_Q8_0, 33, 32)
    assert [oracle.quant_block_bytes(f) for f in (1, 2, 3, 4, 5)] == [144, 176, 210, 34, 292]


# ---- activation quantizers ----------------------------------------------------


def test_q8_0_known_answers():
    # quantize.rs:112-127
    x = np.zeros(32, F32)
    x[0], x[1], x[31] = 2.0, -1.0, 0.5
    b = oracle.quantize_row_q8_0(x)[0]
    assert b["d"] == oracle.f16_to_f32(oracle.f32_to_f16(F32(2.0) / F32(127.0)))[0]
    assert (b["qs"][0], b["qs"][1], b["qs"][31], b["qs"][2]) == (127, -64, 32, 0)  # -63.5 -> -64: half away
    # quantize.rs:130-143
    z = oracle.quantize_row_q8_0(np.zeros(64, F32))
    assert (z["d"] == 0).all() and (z["qs"] == 0).all()


def test_q8_k_known_answers():
    # quantize.rs:146-158: the negative extreme lands on -127, d > 0
    x = np.zeros(256, F32)
    x[10], x[20] = -3.0, 1.5
    b = oracle.quantize_row_q8_k(x)[0]
    assert b["qs"][10] == -127 and b["qs"][20] == 64  # 63.5 ties to even
    assert b["d"] == F32(1.0) / (F32(-127.0) / F32(-3.0))
    # quantize.rs:161-171: a positive extreme also maps to -127, d < 0
    x = np.zeros(256, F32)
    x[0], x[1] = 4.0, -2.0
    b = oracle.quantize_row_q8_k(x)[0]
    assert b["qs"][0] == -127 and b["qs"][1] == 64
    assert b["d"] == F32(1.0) / (F32(-127.0) / F32(4.0))
    # quantize.rs:174-184: a zero row zeroes d, qs and bsums
    z = oracle.quantize_row_q8_k(np.zeros(256, F32))[0]
    assert z["d"] == 0 and (z["qs"] == 0).all() and (z["bsums"] == 0).all()
    # `av > amax` is strict (quantize.rs:78-83): of equal magnitudes the first wins
    x = np.zeros(256, F32)
    x[3], x[7] = -2.0, 2.0
    b = oracle.quantize_row_q8_k(x)[0]
    assert b["qs"][3] == -127 and b["qs"][7] == 127 and b["d"] > 0


def test_quantize_length_mismatch_payloads():
    # quantize.rs:187-202
    e = raises(QLM, oracle.quantize_row_q8_0, np.zeros(100, F32), 3)
    assert e.payload()[1:4] == (RV_QF_Q8_0, 100, 3)
    e = raises(QLM, oracle.quantize_row_q8_k, np.zeros(100, F32), 1)
    assert e.payload()[1:4] == (RV_QF_Q8_K, 100, 1)


def test_q8_k_bsums_are_the_group_sums():
    # quants/tests.rs:349-364
    rng = Lcg(0xB5)
    for _ in range(4):
        b = oracle.quantize_row_q8_k(rng.f32s(256, 5.0))[0]
        assert b["d"] != 0
        assert (b["bsums"] == b["qs"].astype(np.int32).reshape(16, 16).sum(1)).all()
        assert b["qs"].min() >= -128 and b["qs"].max() <= 127
        assert -127 in b["qs"]  # the anchored extreme


def test_quantizers_round_trip_within_half_a_step():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(4096).astype(F32)
    k = oracle.quantize_row_q8_k(x)
    assert np.abs(dequant_acts(k) - x).max() <= np.abs(k["d"]).max() * 0.5001
    q = oracle.quantize_row_q8_0(x)
    # d is f16-rounded after the integers are chosen: half a step plus the d rounding
    err = np.abs(dequant_acts(q) - x).reshape(-1, 32).max(1)
    assert (err <= q["d"] * 0.5 + 127 * q["d"] * 2.0 ** -11 + 1e-7).all()


# ---- dequantizers: round trips of the reference's test quantizers --------------


@pytest.mark.parametrize("fmt,seed", [(RV_QF_Q4_K, 42), (RV_QF_Q5_K, 43)])
def test_round_trip_affine(fmt, seed):
    # quants/tests.rs:50-92: error within one step plus one min step
    x = Lcg(seed).f32s(512, 8.0)
    bts = np.frombuffer(TEST_QUANT[fmt](x), np.uint8)
    w = oracle.dequantize_row(fmt, bts)
    bb = oracle.quant_block_bytes(fmt)
    for bi in range(2):
        blk = bts[bb * bi:bb * (bi + 1)]
        d = oracle.f16_to_f32(blk[0] | (blk[1].astype(np.uint16) << 8))[0]
        dmin = oracle.f16_to_f32(blk[2] | (blk[3].astype(np.uint16) << 8))[0]
        s = blk[4:16]
        for j in range(8):
            sc = (s[j] & 63) if j < 4 else ((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4))
            tol = d * F32(sc) + dmin + F32(1e-6)
            i = slice(256 * bi + 32 * j, 256 * bi + 32 * j + 32)
            assert (np.abs(w[i] - x[i]) <= tol).all()


def test_round_trip_q6_k_and_q8_0():
    # quants/tests.rs:95-134
    x = Lcg(44).f32s(512, 8.0)
    bts = np.frombuffer(quantize_row_q6_k_test(x), np.uint8)
    w = oracle.dequantize_row(RV_QF_Q6_K, bts)
    for bi in range(2):
        blk = bts[210 * bi:210 * (bi + 1)]
        d = oracle.f16_to_f32(blk[208] | (blk[209].astype(np.uint16) << 8))[0]
        for g in range(16):
            tol = abs(d * F32(np.int8(blk[192 + g]))) + F32(1e-6)
            i = slice(256 * bi + 16 * g, 256 * bi + 16 * g + 16)
            assert (np.abs(w[i] - x[i]) <= tol).all()
    x = Lcg(45).f32s(128, 8.0)
    bts = np.frombuffer(quantize_row_q8_0_test(x), np.uint8)
    w = oracle.dequantize_row(RV_QF_Q8_0, bts)
    for bi in range(4):
        d = oracle.f16_to_f32(bts[34 * bi] | (bts[34 * bi + 1].astype(np.uint16) << 8))[0]
        assert (np.abs(w[32 * bi:32 * bi + 32] - x[32 * bi:32 * bi + 32]) <= d + F32(1e-6)).all()


def test_round_trip_flat_blocks():
    # quants/tests.rs:137-159
    for c in (0.0, -3.75, 12.5):
        x = np.full(256, c, F32)
        tol45 = abs(c) / 63.0 + 1e-3
        for fmt in (RV_QF_Q4_K, RV_QF_Q5_K):
            w = oracle.dequantize_row(fmt, np.frombuffer(TEST_QUANT[fmt](x), np.uint8))
            assert (np.abs(w - c) <= tol45).all()
        w = oracle.dequantize_row(RV_QF_Q6_K, np.frombuffer(quantize_row_q6_k_test(x), np.uint8))
        assert (np.abs(w - c) <= abs(c) / 31.0 + 1e-3).all()


# ---- scalar dots: f64 ground truth and adversarial blocks ----------------------


@pytest.mark.parametrize("fmt,seed", [(RV_QF_Q4_K, 0xA4), (RV_QF_Q5_K, 0xA5), (RV_QF_Q6_K, 0xA6)])
def test_dot_ground_truth_k_quants(fmt, seed):
    # quants/tests.rs:162-208
    for n in (2048, 768):
        rng = Lcg(seed ^ n)
        xw, xa = rng.f32s(n, 4.0), rng.f32s(n, 3.0)
        wb = np.frombuffer(TEST_QUANT[fmt](xw), np.uint8)
        acts = oracle.quantize_row_q8_k(xa)
        assert_dot_close(oracle.vec_dot(fmt, wb, acts), oracle.dequantize_row(fmt, wb), dequant_acts(acts))


def test_dot_ground_truth_q8_0():
    # quants/tests.rs:211-228
    for n in (2048, 768):
        rng = Lcg(0x80 ^ n)
        xw, xa = rng.f32s(n, 4.0), rng.f32s(n, 3.0)
        wb = np.frombuffer(quantize_row_q8_0_test(xw), np.uint8)
        acts = oracle.quantize_row_q8_0(xa)
        assert_dot_close(oracle.vec_dot(RV_QF_Q8_0, wb, acts), oracle.dequantize_row(RV_QF_Q8_0, wb),
                         dequant_acts(acts))


@pytest.mark.parametrize("fmt", [RV_QF_Q4_K, RV_QF_Q5_K, RV_QF_Q6_K, RV_QF_Q8_0])
def test_dot_ground_truth_on_random_bytes(fmt):
    """Every bit pattern of the quants and scales (not only what the test
    quantizers emit), against the f64 dot of the dequantized rows."""
    rng = np.random.default_rng(0xD0 + fmt)
    for in_dim in (256, 2048, 4096):
        w = random_weight_rows(fmt, 6, in_dim, rng)
        x = rng.standard_normal(in_dim).astype(F32)
        acts = oracle.quantize_row_q8_0(x) if fmt == RV_QF_Q8_0 else oracle.quantize_row_q8_k(x)
        a = dequant_acts(acts)
        for r in range(6):
            assert_dot_close(oracle.vec_dot(fmt, w[r], acts), oracle.dequantize_row(fmt, w[r]), a)


def _q8k_random(seed):
    return oracle.quantize_row_q8_k(Lcg(seed).f32s(256, 2.0))


ALL_MIN = bytes([0, 0, 0, 0, 0xFF, 0xFF, 0xFF, 0xFF, 0xF0, 0xF0, 0xF0, 0xF0])


def test_dot_adversarial_blocks():
    # quants/tests.rs:231-346
    def q4k(d, dmin, scales, qs):
        return np.frombuffer(f16_bytes(d) + f16_bytes(dmin) + bytes(scales) + bytes([qs] * 128), np.uint8)

    def q5k(d, dmin, scales, qh, qs):
        return np.frombuffer(f16_bytes(d) + f16_bytes(dmin) + bytes(scales) + bytes([qh] * 32) + bytes([qs] * 128),
                             np.uint8)

    def q6k(ql, qh, scale, d):
        return np.frombuffer(bytes([ql] * 128) + bytes([qh] * 64) + bytes([scale & 0xFF] * 16) + f16_bytes(d), np.uint8)

    acts = _q8k_random(0xD4)
    cases4 = [q4k(1.0, 0.5, [0xFF] * 12, 0xFF), q4k(4.0, 2.0, [0] * 12, 0x5A), q4k(0.0, 0.0, [0x3F] * 12, 0xFF),
              q4k(1.0, 0.5, ALL_MIN, 0x00)]
    for b in cases4:
        assert_dot_close(oracle.vec_dot(RV_QF_Q4_K, b, acts), oracle.dequantize_row(RV_QF_Q4_K, b), dequant_acts(acts))
    assert oracle.vec_dot(RV_QF_Q4_K, cases4[1], np.zeros(1, oracle.BLOCK_Q8_K)) == 0.0
    acts = _q8k_random(0xD5)
    for b in [q5k(1.0, 0.5, [0xFF] * 12, 0xFF, 0xFF), q5k(1.0, 0.5, [0xFF] * 12, 0x00, 0xFF),
              q5k(4.0, 2.0, [0] * 12, 0xAA, 0x5A), q5k(1.0, 0.5, ALL_MIN, 0xAA, 0x00)]:
        assert_dot_close(oracle.vec_dot(RV_QF_Q5_K, b, acts), oracle.dequantize_row(RV_QF_Q5_K, b), dequant_acts(acts))
    acts = _q8k_random(0xD6)
    for b in [q6k(0xFF, 0xFF, -128, 1.0), q6k(0xFF, 0xFF, 127, 0.25), q6k(0x00, 0x00, 127, 1.0),
              q6k(0x5A, 0xA5, 0, 4.0)]:
        assert_dot_close(oracle.vec_dot(RV_QF_Q6_K, b, acts), oracle.dequantize_row(RV_QF_Q6_K, b), dequant_acts(acts))
    wb = np.frombuffer((0x7BFF).to_bytes(2, "little") + bytes([0x80] * 32), np.uint8)  # d = 65504, q = -128
    a = np.zeros(1, oracle.BLOCK_Q8_0)
    a["d"], a["qs"] = 65504.0, 127
    assert_dot_close(oracle.vec_dot(RV_QF_Q8_0, wb, a), oracle.dequantize_row(RV_QF_Q8_0, wb), dequant_acts(a))
    assert oracle.vec_dot(RV_QF_Q8_0, wb, np.zeros(1, oracle.BLOCK_Q8_0)) == 0.0


def test_dot_and_dequant_length_errors():
    # quants/tests.rs:369-441
    for fmt, bb in ((RV_QF_Q4_K, 144), (RV_QF_Q5_K, 176), (RV_QF_Q6_K, 210), (RV_QF_Q8_0, 34)):
        assert raises(RBN, oracle.dequantize_row, fmt, np.zeros(bb + 1, np.uint8)).payload()[1:4] == (fmt, bb + 1, bb)
        assert oracle.dequantize_row(fmt, np.zeros(0, np.uint8)).size == 0
    acts = np.zeros(2, oracle.BLOCK_Q8_K)
    assert raises(BCM, oracle.vec_dot, RV_QF_Q4_K, np.zeros(144, np.uint8), acts).payload()[1:3] == (1, 2)
    assert raises(RBN, oracle.vec_dot, RV_QF_Q6_K, np.zeros(100, np.uint8), acts).payload()[1:4] == (RV_QF_Q6_K, 100,
                                                                                                     210)
    assert oracle.vec_dot(RV_QF_Q8_0, np.zeros(272, np.uint8), np.zeros(8, oracle.BLOCK_Q8_0)) == 0.0


# ---- GEMV -----------------------------------------------------------------------


@pytest.mark.parametrize("fmt", [RV_QF_Q4_K, RV_QF_Q5_K, RV_QF_Q6_K, RV_QF_Q8_0])
def test_gemv_rows_and_batches_are_bit_identical_to_single_dots(fmt):
    """gemv.rs:18-35 and :55-79: every output is one vec_dot of one weight row
    against one activation row, so any row range and any batch reproduces
    the single dots bit for bit."""
    rng = np.random.default_rng(0x6E + fmt)
    in_dim, out_dim, n_acts = 512, 13, 3
    w = random_weight_rows(fmt, out_dim, in_dim, rng)
    quant = oracle.quantize_row_q8_0 if fmt == RV_QF_Q8_0 else oracle.quantize_row_q8_k
    acts = quant(rng.standard_normal(n_acts * in_dim).astype(F32))
    nb = acts.size // n_acts
    whole = oracle.gemv(fmt, w, in_dim, out_dim, acts[:nb])
    single = np.array([oracle.vec_dot(fmt, w[r], acts[:nb]) for r in range(out_dim)], F32)
    assert whole.tobytes() == single.tobytes()
    parts = np.concatenate([oracle.gemv(fmt, w, in_dim, out_dim, acts[:nb], rows=(lo, hi))
                            for lo, hi in ((0, 5), (5, 5), (5, 12), (12, 13))])
    assert parts.tobytes() == whole.tobytes()
    batched = oracle.gemv(fmt, w, in_dim, out_dim, acts, n_acts=n_acts, rows=(2, 11)).reshape(9, n_acts)
    for a in range(n_acts):
        assert batched[:, a].tobytes() == oracle.gemv(fmt, w, in_dim, out_dim, acts[a * nb:(a + 1) * nb],
                                                      rows=(2, 11)).tobytes()


def test_gemv_validation_order_and_payloads():
    """gemv.rs:212-266 in order: row bytes, whole-matrix bytes, range order,
    range bound, out length, block count; a non-k-quant format first."""
    L = oracle.lib()
    err = oracle.RvError()
    acts = np.zeros(8, oracle.BLOCK_Q8_K)
    w = np.zeros(4 * 1152, np.uint8)
    out = np.zeros(4, F32)

    def call(fmt=RV_QF_Q4_K, wlen=w.size, in_dim=2048, out_dim=4, nacts=8, lo=0, hi=4, olen=4):
        rc = L.rvo_gemv_q8_k(fmt, w.ctypes.data, wlen, in_dim, out_dim, acts.ctypes.data, nacts, 1, lo, hi,
                             out.ctypes.data_as(oracle.POINTER(oracle.c_float)), olen, oracle.byref(err))
        return rc, (err.a, err.b, err.c), err.what.decode() if err.what else None

    assert call()[0] == 0
    assert call(fmt=RV_QF_Q8_0)[0] == UNS
    assert call(in_dim=100)[0:2] == (IND, (RV_QF_Q4_K, 100, 256))
    rc, ab, what = call(wlen=w.size - 1)
    assert rc == RV_PRIM_LENGTH_MISMATCH and ab[:2] == (w.size - 1, w.size) and what.startswith("gemv_q8_k")
    assert call(lo=3, hi=2)[0:3] == (RV_PRIM_LENGTH_MISMATCH, (3, 2, 0), "gemv rows: row range start vs end")
    assert call(hi=5)[0:3] == (RV_PRIM_LENGTH_MISMATCH, (5, 4, 0), "gemv rows: row range end vs out_dim")
    assert call(olen=3)[0:2] == (RV_PRIM_LENGTH_MISMATCH, (3, 4, 0))
    assert call(nacts=7)[0:2] == (BCM, (8, 7, 0))
    # precedence: a bad row size is reported before a bad range or out length
    assert call(in_dim=100, lo=3, hi=2, olen=0)[0] == IND

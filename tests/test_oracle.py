"""Pins the CPU oracle (oracle/rv_oracle.c) before anything is checked against it.

Each check is one the reference's own tests make (cited file:line into
ramvamp's crates/core/src), a closed form, or an independent library routine
(numpy float16 / float64), chosen so that a plausible slip in the restatement
(a dropped term, a swapped index, a wrong rounding) fails one of them.
"""
import math

import numpy as np
import pytest

import json
import os

import oracle
from helpers import Rng, assert_close, reference_attention, round_trip

# Known answers the reference's own tests assert, kept as data.
with open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")) as _f:
    KATS = json.load(_f)

F16_SUBNORMAL_ULP = np.float32(2.0 ** -24)


# ---- f16 (kernels/quants/f16.rs:97-160) ---------------------------------------

def _f32(bits_hex):
    return np.array([int(bits_hex, 16)], dtype=np.uint32).view(np.float32)[0]


def test_f16_to_f32_known_vectors():
    kat = KATS["f16_to_f32"]  # f16.rs:97-113
    for case in kat["cases"]:
        got = oracle.f16_to_f32([int(case["f16"], 16)])[0]
        assert np.float32(got).view(np.uint32) == _f32(case["f32_bits"]).view(np.uint32), case
    for bits in kat["nan_inputs"]:
        assert np.isnan(oracle.f16_to_f32([int(bits, 16)])[0])


def test_f32_to_f16_known_vectors():
    kat = KATS["f32_to_f16"]  # f16.rs:116-133, ties to even :153-160
    for case in kat["cases"]:
        assert int(oracle.f32_to_f16([_f32(case["f32_bits"])])[0]) == int(case["f16"], 16), case
    for bits in kat["nan_inputs_f32_bits"]:
        assert np.isnan(oracle.f16_to_f32(oracle.f32_to_f16([_f32(bits)]))[0])


def test_f16_round_trip_all_finite_and_ties_to_even():
    # f16.rs:136-150 and :153-160
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    finite = ((bits >> 10) & 0x1F) != 0x1F
    widened = oracle.f16_to_f32(bits[finite])
    assert np.array_equal(oracle.f32_to_f16(widened), bits[finite])
    assert int(oracle.f32_to_f16([np.float32(1.0004883)])[0]) == 0x3C00
    assert int(oracle.f32_to_f16([np.float32(1.0004884)])[0]) == 0x3C01
    assert int(oracle.f32_to_f16([np.float32(1.0014648)])[0]) == 0x3C02


def test_f16_matches_ieee_library_conversion():
    # Independent routine: numpy's IEEE binary16 conversion (RNE), all 65,536
    # widenings and 4M narrowings spread over every f32 exponent.
    bits = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    finite = ((bits >> 10) & 0x1F) != 0x1F
    lib_w = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(oracle.f16_to_f32(bits)[finite].view(np.uint32), lib_w[finite].view(np.uint32))
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 2 ** 32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    x = raw.view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        lib_n = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x), lib_n)


# ---- softmax / rmsnorm / rope ----------------------------------------------------

def test_softmax_closed_forms_and_f64_reference():
    kat = KATS["softmax_single_element"]  # softmax.rs:103-107
    assert oracle.softmax(kat["input"])[0] == np.float32(kat["expected"][0])
    for n in (1, 3, 1000):  # softmax.rs:90-100
        assert_close(oracle.softmax(np.full(n, 42.5, np.float32)), np.full(n, 1.0 / n), 1e-6, 0.0, "all equal")
    a = np.float32(0.7)
    got = oracle.softmax([0.0, a])
    assert_close(got[1], 1.0 / (1.0 + math.exp(-float(a))), 1e-6, 0.0, "two-element sigmoid")
    rng = Rng(0x50F7)  # softmax.rs:58-69
    for n in (2, 20, 128, 2048):
        x = rng.vec_in(n, -10.0, 10.0)
        e = np.exp(x.astype(np.float64) - x.max())
        assert_close(oracle.softmax(x), e / e.sum(), 1e-6, 1e-10, f"softmax n={n}")
    with pytest.raises(oracle.OracleError):
        oracle.softmax(np.zeros(0, np.float32))


def test_rmsnorm_closed_forms():
    eps = np.float32(1e-6)
    rng = Rng(0xA11CE)  # norm.rs:130-141
    for n in (1, 2, 128, 2048):
        x = rng.vec_in(n, -4.0, 4.0)
        w = rng.vec_in(n, 0.25, 2.0)
        xd = x.astype(np.float64)
        want = xd / np.sqrt(np.mean(xd * xd) + float(eps)) * w
        assert_close(oracle.rmsnorm(x, w, eps), want, 1e-6, 1e-30, f"rmsnorm n={n}")
    kat = KATS["rmsnorm_zero_weight"]  # norm.rs:184-191
    assert np.array_equal(oracle.rmsnorm(kat["input"], kat["weight"], eps), np.asarray(kat["expected"], np.float32))
    assert_close(oracle.rmsnorm(np.full(512, 3.0), np.ones(512), eps), np.ones(512), 1e-6, 0.0, "all equal")


def test_rope_known_angles_head_dim_4_theta_1e7():
    kat = KATS["rope_neox_head_dim4_theta_1e7"]  # rope.rs:144-175: hand-computed f64 values
    for case in kat["cases"]:
        got = oracle.rope_neox_heads(kat["input"], 1, 4, case["position"], kat["theta"])
        assert_close(got, case["expected"], kat["tolerance"]["rel"], 1e-30, f"rope pos {case['position']}")


def test_rope_identity_magnitude_and_f64_reference():
    rng = Rng(0x0)
    for d in (4, 128):  # rope.rs:132-141
        x = rng.vec_in(d, -5.0, 5.0)
        assert np.array_equal(oracle.rope_neox_heads(x, 1, d, 0, 1e7), x)
    rng = Rng(0xF00D)  # rope.rs:195-210
    x = rng.vec_in(128, -8.0, 8.0)
    y = oracle.rope_neox_heads(x, 1, 128, 90_210, 1e7).astype(np.float64)
    xd = x.astype(np.float64)
    assert_close(np.hypot(y[:64], y[64:]), np.hypot(xd[:64], xd[64:]), 1e-5, 1e-30, "pair magnitude")
    rng = Rng(0xD1)  # rope.rs:178-193 (f64 reference, NeoX pairs (i, i+64))
    for pos in (1, 2, 17, 4096, 100_000):
        x = rng.vec_in(128, -3.0, 3.0).astype(np.float64)
        i = np.arange(64, dtype=np.float64)
        ang = pos * np.power(float(np.float32(1e7)), -2.0 * i / 128.0)
        want = np.concatenate([x[:64] * np.cos(ang) - x[64:] * np.sin(ang), x[:64] * np.sin(ang) + x[64:] * np.cos(ang)])
        assert_close(oracle.rope_neox_heads(x, 1, 128, pos, 1e7), want, 1e-6, 1e-6, f"rope pos {pos}")
    # The multi-head form is the single-head form per head (rope.rs:213-223).
    x = Rng(0xCAFE).vec_in(4 * 128, -2.0, 2.0)
    per = np.concatenate([oracle.rope_neox_heads(x[h * 128:(h + 1) * 128], 1, 128, 7, 1e7) for h in range(4)])
    assert np.array_equal(oracle.rope_neox_heads(x, 4, 128, 7, 1e7), per)
    with pytest.raises(oracle.OracleError):
        oracle.rope_neox_heads(np.zeros(3, np.float32), 1, 3, 1, 1e7)


# ---- KV cache (kv/mod.rs) ------------------------------------------------------------

def test_kv_projected_bytes_and_dims():
    for cap in (1, 512, 4096, 16_384):  # kv/mod.rs:552-563
        assert oracle.projected_bytes(48, 4, 128, cap) == cap * 96 * 1024
    assert oracle.projected_bytes(48, 4, 128, 4096) == 384 << 20
    assert oracle.projected_bytes(48, 4, 128, 4096, oracle.RV_ELEM_F32) == 768 << 20
    for dims in [(0, 4, 128, 8), (1, 0, 128, 8), (1, 4, 0, 8), (1, 4, 128, 0)]:
        with pytest.raises(oracle.OracleError) as e:
            oracle.KvCache(*dims)
        assert e.value.code == 1 and e.value.what == "all dims must be nonzero"
    with pytest.raises(oracle.OracleError) as e:
        oracle.projected_bytes(2, 2 ** 62, 4, 1)
    assert e.value.what == "row width overflows usize"
    with pytest.raises(oracle.OracleError) as e:
        oracle.projected_bytes(2, 2 ** 61, 2, 1)
    assert e.value.what == "total size in bytes overflows usize"


def test_kv_append_errors_truncate_clear():
    kv = oracle.KvCache(2, 2, 4, 3)
    row = np.arange(8, dtype=np.float32) * 0.5
    kv.append(0, row, -row)
    assert kv.len(0) == 1 and kv.len(1) == 0
    with pytest.raises(oracle.OracleError) as e:
        kv.seq_len()
    assert e.value.payload()[:3] == (6, 0, 1)  # RaggedLayers { shortest 0, longest 1 }
    with pytest.raises(oracle.OracleError) as e:
        kv.append(2, row, row)
    assert e.value.payload()[:3] == (2, 2, 2)
    with pytest.raises(oracle.OracleError) as e:
        kv.append(0, row[:7], row)
    assert e.value.payload() == (3, 7, 8, 0, 0, "k")
    with pytest.raises(oracle.OracleError) as e:
        kv.append(0, row, row[:5])
    assert e.value.payload() == (3, 5, 8, 0, 0, "v")
    with pytest.raises(oracle.OracleError) as e:
        kv.truncate(0)  # ragged refused before the target is looked at
    assert e.value.code == 6
    kv.append(1, row, row)
    kv.truncate(1)
    with pytest.raises(oracle.OracleError) as e:
        kv.truncate(2)
    assert e.value.payload()[:3] == (7, 2, 1)
    kv.append(0, row, row)
    kv.append(0, row, row)
    with pytest.raises(oracle.OracleError) as e:
        kv.append(0, row, row)
    assert e.value.payload()[:3] == (4, 0, 3)
    assert np.array_equal(kv.read_row(False, 0, 0), oracle.f32_to_f16(row))
    assert np.array_equal(kv.read_row(True, 0, 0), oracle.f32_to_f16(-row))
    with pytest.raises(oracle.OracleError) as e:
        kv.read_row(False, 1, 1)
    assert e.value.payload()[:4] == (5, 1, 1, 1)
    kv.clear()
    assert kv.is_empty() and kv.seq_len() == 0


# ---- attention (kernels/attention.rs tests) ----------------------------------------------

def _cache_from_rng(rng, n_layers, n_kv, head_dim, n_pos, elem=oracle.RV_ELEM_F16, cap=None):
    kv_dim = n_kv * head_dim
    rows = [[(rng.vec_in(kv_dim, -1.0, 1.0), rng.vec_in(kv_dim, -1.0, 1.0)) for _ in range(n_pos)]
            for _ in range(n_layers)]
    kv = oracle.KvCache(n_layers, n_kv, head_dim, cap or max(n_pos, 1), elem)
    for layer, layer_rows in enumerate(rows):
        for k, v in layer_rows:
            kv.append(layer, k, v)
    return kv, rows


def test_matches_f64_reference_across_layers_and_lengths():
    # attention.rs:1419-1473, the v0 pin 32:4:128, three layers, lens 1/2/17/256.
    n_layers, n_kv, n_q, hd, cap = 3, 4, 32, 128, 256
    kv_dim = n_kv * hd
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    rng = Rng(0xA77E)
    for elem in (oracle.RV_ELEM_F16, oracle.RV_ELEM_F32):
        kv = oracle.KvCache(n_layers, n_kv, hd, cap, elem)
        ks = [[] for _ in range(n_layers)]
        vs = [[] for _ in range(n_layers)]
        appended = 0
        for target in (1, 2, 17, 256):
            while appended < target:
                for layer in range(n_layers):
                    k = rng.vec_in(kv_dim, -1.0, 1.0)
                    v = rng.vec_in(kv_dim, -1.0, 1.0)
                    kv.append(layer, k, v)
                    ks[layer].append(k)
                    vs[layer].append(v)
                appended += 1
            assert kv.seq_len() == target
            for layer in range(n_layers):
                q = rng.vec_in(n_q * hd, -1.0, 1.0)
                out = kv.attention(q, layer, scale)
                K, V = np.array(ks[layer]), np.array(vs[layer])
                assert_close(out, reference_attention(q, K, V, n_kv, hd, scale), 1e-3, 1.5e-3, "vs exact")
                if elem == oracle.RV_ELEM_F16:
                    K, V = round_trip(K), round_trip(V)
                assert_close(out, reference_attention(q, K, V, n_kv, hd, scale), 1e-4, 5e-5, "vs stored")


def test_gqa_maps_query_head_h_to_kv_head_h_div_8():
    # attention.rs:1483-1516
    n_kv, n_q, hd = 4, 32, 16
    kv = oracle.KvCache(1, n_kv, hd, 4)
    marker = lambda j, t: np.float32((10 * j + t) * 0.01)
    for t in range(4):
        k = np.zeros(n_kv * hd, np.float32)
        v = np.zeros(n_kv * hd, np.float32)
        for j in range(n_kv):
            k[j * hd:(j + 1) * hd] = (1.0 if t == j else -1.0) * 8.0 / hd
            v[j * hd:(j + 1) * hd] = marker(j, t)
        kv.append(0, k, v)
    out = kv.attention(np.ones(n_q * hd, np.float32), 0, 1.0).reshape(n_q, hd)
    for h in range(n_q):
        assert np.all(np.abs(out[h] - marker(h // 8, h // 8)) < 1e-3), h


def test_single_position_returns_v_row_bit_exact():
    # attention.rs:1523-1554
    n_kv, n_q, hd = 4, 32, 128
    rng = Rng(0x5EED)
    kv = oracle.KvCache(2, n_kv, hd, 8)
    vs = []
    for layer in range(2):
        k, v = rng.vec_in(n_kv * hd, -1.0, 1.0), rng.vec_in(n_kv * hd, -1.0, 1.0)
        kv.append(layer, k, v)
        vs.append(v)
    q = rng.vec_in(n_q * hd, -1.0, 1.0)
    for layer, v in enumerate(vs):
        out = kv.attention(q, layer, np.float32(1.0) / np.sqrt(np.float32(hd))).reshape(n_q, hd)
        for h in range(n_q):
            col = (h // 8) * hd
            assert np.array_equal(out[h], round_trip(v[col:col + hd]))


def test_doubling_scale_squares_the_odds_ratio():
    # attention.rs:1894-1918
    kv = oracle.KvCache(1, 1, 4, 2)
    kv.append(0, [0, 0, 0, 0], [0] * 4)
    kv.append(0, [1, 0, 0, 0], [1] * 4)
    q = [1.0, 0, 0, 0]
    s = np.float32(0.7)
    p1 = float(kv.attention(q, 0, s)[0])
    p2 = float(kv.attention(q, 0, np.float32(2.0) * s)[0])
    sig = lambda x: 1.0 / (1.0 + math.exp(-x))
    assert_close(p1, sig(float(s)), 1e-5, 0.0)
    assert_close(p2, sig(2.0 * float(s)), 1e-5, 0.0)
    odds = lambda p: p / (1.0 - p)
    assert_close(odds(p2), odds(p1) ** 2, 1e-4, 0.0)


def test_scratch_len_pins():
    kat = KATS["scratch_len"]  # attention.rs:2330-2342
    assert oracle.scratch_len(*kat["args"]) == kat["expected"]
    assert oracle.scratch_len(32, 4, 8, 17) == 8 * 17 + 2 * 8
    assert oracle.scratch_len(32, 0, 8, 17) == 16
    assert oracle.scratch_len(2 ** 63, 1, 2, 4) == 2 ** 64 - 1


LIMITED = [(2, 4, 32, 128, 5), (1, 2, 2, 16, 9), (1, 1, 8, 8, 7), (2, 3, 6, 4, 12)]  # attention.rs:1971-1976


def dispatch_geometries():  # attention.rs:2621-2634
    return LIMITED + [(1, 4, 32, 128, 67), (1, 1, 8, 9, 11), (2, 3, 6, 9, 13), (1, 1, 32, 128, 9),
                      (1, 2, 34, 16, 13), (1, 1, 12, 9, 11), (1, 1, 8, 256, 5), (1, 2, 4, 255, 3)]


def dispatch_lengths(n_pos):  # attention.rs:2670-2679
    return [p for p in (1, 2, 3, 4, 5, 6, 7, 8, 9, 11, 12, 13, 14, 15, 16, 17, 23, 24, 25, 31, 61) if p < n_pos] + [n_pos]


def test_attention_at_is_bit_identical_to_truncated_decode():
    # attention.rs:2019-2058
    rng = Rng(0xB17DE17E)
    for n_layers, n_kv, n_q, hd, n_pos in LIMITED:
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        full, rows = _cache_from_rng(rng, n_layers, n_kv, hd, n_pos)
        q = rng.vec_in(n_q * hd, -1.0, 1.0)
        for layer, layer_rows in enumerate(rows):
            for n in range(1, n_pos + 1):
                trunc = oracle.KvCache(n_layers, n_kv, hd, n)
                for k, v in layer_rows[:n]:
                    trunc.append(layer, k, v)
                got = full.attention(q, layer, scale, positions=n)
                want = trunc.attention(q, layer, scale)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.skipif(not oracle.avx2_path_covers(128), reason="host lacks AVX2+F16C")
def test_simd_matches_scalar_bit_for_bit():
    # attention.rs:2739: both bodies over every geometry and length class.
    classes = {p % 8 for *_, n in dispatch_geometries() for p in dispatch_lengths(n)}
    assert classes == set(range(8))  # attention.rs:2694-2713
    rng = Rng(0x51AD)
    for elem in (oracle.RV_ELEM_F16, oracle.RV_ELEM_F32):
        for n_layers, n_kv, n_q, hd, n_pos in dispatch_geometries():
            scale = np.float32(1.0) / np.sqrt(np.float32(hd))
            kv, _ = _cache_from_rng(rng, n_layers, n_kv, hd, n_pos, elem)
            q = rng.vec_in(n_q * hd, -1.0, 1.0)
            for layer in range(n_layers):
                for p in dispatch_lengths(n_pos):
                    a = kv.attention(q, layer, scale, positions=p, force_scalar=False)
                    b = kv.attention(q, layer, scale, positions=p, force_scalar=True)
                    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (hd, n_q, p)


def test_kv_range_union_is_bit_identical_to_the_whole_call():
    # attention.rs:3002; forward.rs:3022-3122 (shards 1-8)
    rng = Rng(0x7A16)
    kv, _ = _cache_from_rng(rng, 1, 4, 128, 67)
    q = rng.vec_in(32 * 128, -1.0, 1.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    whole = kv.attention(q, 0, scale)
    need = oracle.scratch_len(32, 4, 128, 67)
    for units in range(1, 9):
        got = np.full_like(whole, np.nan)
        for u in range(units):
            r = oracle.kv_head_range(4, units, u, u + 1)
            if len(r):
                got[r.start * 1024:r.stop * 1024] = kv.attention(q, 0, scale, kv_range=r, scratch_len=need)
        assert np.array_equal(got.view(np.uint32), whole.view(np.uint32)), units
        pooled = kv.pool_decode_attention(q, 0, scale, threads=units)
        assert np.array_equal(pooled.view(np.uint32), whole.view(np.uint32)), units


def test_error_precedence_is_pinned_from_q_to_out():
    # attention.rs:1640-1888 (condensed: one probe per level, every entry form)
    n_kv, n_q, hd = 4, 8, 8
    kv = oracle.KvCache(2, n_kv, hd, 4)
    row = np.full(n_kv * hd, 0.5, np.float32)
    for _ in range(3):
        kv.append(0, row, row)
    q = np.full(n_q * hd, 0.25, np.float32)
    need = oracle.scratch_len(n_q, n_kv, hd, 4)

    def codes(q_arg, layer, positions, out_len, kv_range, scratch_len=need):
        got = []
        for form in ("decode", "decode_in", "at", "at_in", "decode_range", "at_range"):
            kw = dict(out_len=out_len)
            if form.endswith("_in") or "range" in form:
                kw["scratch_len"] = scratch_len
            if form.startswith("at"):
                kw["positions"] = positions
            if "range" in form:
                kw["kv_range"] = kv_range
            with pytest.raises(oracle.OracleError) as e:
                kv.attention(q_arg, layer, 0.5, **kw)
            got.append(e.value.code)
        return got

    bad = range(5, 5)
    assert codes(q[:13], 9, 0, 7, bad) == [16] * 6                       # q length first
    assert codes(q[:5 * hd], 9, 0, 7, bad) == [17] * 6                   # then GQA
    assert codes(q, 9, 0, 7, bad) == [2] * 6                             # then layer
    assert codes(q, 1, 0, 7, bad) == [19] * 6                            # empty layer / positions 0
    assert codes(q, 0, 9, 7, bad) == [18, 18, 5, 5, 20, 5]               # positions past the end
    assert codes(q, 0, 2, 7, bad) == [18, 18, 18, 18, 20, 20]            # kv range before out
    assert codes(q, 0, 2, 7, range(0, 4)) == [18] * 6                    # out length
    # scratch is checked last, against this call's own geometry (group * positions + 2 * head_dim)
    for positions, kv_range in ((None, None), (2, None), (None, range(0, 4)), (2, range(0, 4))):
        p = 3 if positions is None else positions
        with pytest.raises(oracle.OracleError) as e:
            kv.attention(q, 0, 0.5, positions=positions, kv_range=kv_range, scratch_len=2 * p + 2 * hd - 1)
        assert e.value.payload()[:3] == (21, 2 * p + 2 * hd - 1, 2 * p + 2 * hd)
        kv.attention(q, 0, 0.5, positions=positions, kv_range=kv_range, scratch_len=2 * p + 2 * hd)


def test_attention_split_partitions_balances_and_kv_head_split_tiles():
    # prefill.rs:4009-4090 and forward.rs:2944
    for rows in (0, 1, 2, 5, 6, 7, 8, 63, 512, 1891):
        for start in (0, 1, 7, 512, 4095):
            for shards in (1, 2, 3, 6, 8, 16):
                nxt, seen = 0, np.zeros(rows, int)
                for i in range(shards):
                    r = oracle.attention_shard_range(rows, start, shards, i)
                    assert r.start == nxt and r.stop <= rows
                    nxt = r.stop
                    seen[r.start:r.stop] += 1
                assert nxt == rows and np.all(seen == 1)
    cost = lambda r, s: r * s + r * (r + 1) // 2
    total = cost(512, 0)
    assert total == 131_328
    widest = 0
    for i in range(6):
        r = oracle.attention_shard_range(512, 0, 6, i)
        c = cost(r.stop, 0) - cost(r.start, 0)
        assert abs(c - total // 6) <= 512
        widest = max(widest, c)
    assert len(oracle.attention_shard_range(512, 0, 6, 0)) > 2 * len(oracle.attention_shard_range(512, 0, 6, 5))
    assert widest * 3 < (cost(512, 0) - cost(512 - 512 // 6, 0)) * 2
    for n_kv, units in ((4, 6), (4, 4), (4, 32), (4, 3), (4, 2), (3, 2), (8, 6), (1, 6), (0, 6)):
        covered, empty = np.zeros(n_kv, int), 0
        for slot in range(units):
            r = oracle.kv_head_range(n_kv, units, slot, slot + 1)
            assert r.start <= r.stop <= n_kv
            empty += len(r) == 0
            covered[r.start:r.stop] += 1
        assert np.all(covered == 1) and empty == units - min(n_kv, units)
        assert oracle.kv_head_range(n_kv, units, 0, units) == range(0, n_kv)


def test_scatter_attention_matches_per_row_attention_at():
    # prefill.rs:1390-1398: row r attends start + r + 1; shard count moves no bit
    # (forward.rs:3203 / prefill.rs:2963 spirit).
    rng = Rng(0x5CA7)
    n_kv, n_q, hd, start, rows = 2, 8, 16, 5, 11
    kv, kvrows = _cache_from_rng(rng, 1, n_kv, hd, start + rows, elem=oracle.RV_ELEM_F32)
    q = rng.vec_in(rows * n_q * hd, -1.0, 1.0).reshape(rows, -1)
    scale = np.float32(0.25)
    want = np.stack([kv.attention(q[r], 0, scale, positions=start + r + 1) for r in range(rows)])
    for threads in (1, 2, 3, 8):
        got = kv.scatter_attention(q, 0, start, scale, threads)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), threads


# ---- fused callers (model/forward.rs:2622-2633, model/prefill.rs:2057-2109) -------------

def _norm_rope_f64(x, n_heads, hd, w, eps, theta, pos):
    """f64 textbook of one token's per-head RMSNorm then NeoX RoPE at `pos`."""
    h = np.asarray(x, np.float64).reshape(n_heads, hd)
    h = h / np.sqrt(np.mean(h * h, axis=1, keepdims=True) + float(eps)) * np.asarray(w, np.float64)
    half = hd // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos * np.power(float(np.float32(theta)), -2.0 * i / hd)
    a, b = h[:, :half], h[:, half:]
    return np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], axis=1).reshape(-1)


def test_decode_step_and_prefill_chunk_match_the_f64_composition():
    # The order the callers fix: q and k heads normed, then rotated at the
    # token's position (= the layer's length before the append), k and v
    # appended, then attention over every position including the new one; a
    # prefill row r sits at start + r and attends start + r + 1 positions.
    n_kv, n_q, hd, eps, theta = 2, 8, 16, np.float32(1e-6), np.float32(1e6)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    rng = Rng(0xF05E)
    wq, wk = rng.vec_in(hd, 0.5, 1.5), rng.vec_in(hd, 0.5, 1.5)
    start = 9
    cached_k = rng.vec_in(start * n_kv * hd, -1.0, 1.0).reshape(start, -1)
    cached_v = rng.vec_in(start * n_kv * hd, -1.0, 1.0).reshape(start, -1)
    # decode step
    kv = oracle.KvCache(1, n_kv, hd, start + 8, oracle.RV_ELEM_F32)
    kv.append_rows(0, cached_k, cached_v)
    q, k, v = rng.vec_in(n_q * hd, -2.0, 2.0), rng.vec_in(n_kv * hd, -2.0, 2.0), rng.vec_in(n_kv * hd, -1.0, 1.0)
    got = kv.decode_step(0, q, k, v, wq, wk, eps, theta, start, scale)
    kn = _norm_rope_f64(k, n_kv, hd, wk, eps, theta, start)
    qn = _norm_rope_f64(q, n_q, hd, wq, eps, theta, start)
    assert kv.len(0) == start + 1
    assert_close(kv.read_row(False, 0, start), kn, 1e-5, 1e-6, "appended k row")
    assert np.array_equal(kv.read_row(True, 0, start), v)
    want = reference_attention(qn, np.vstack([cached_k, kn]), np.vstack([cached_v, v]), n_kv, hd, scale)
    assert_close(got, want, 1e-4, 5e-5, "decode step")
    # prefill chunk of 5 rows after the same prefix
    rows = 5
    kv = oracle.KvCache(1, n_kv, hd, start + rows, oracle.RV_ELEM_F32)
    kv.append_rows(0, cached_k, cached_v)
    qr = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
    kr = rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1)
    vr = rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1)
    got = kv.prefill_chunk(0, qr, kr, vr, wq, wk, eps, theta, start, scale)
    kall = np.vstack([cached_k] + [_norm_rope_f64(kr[r], n_kv, hd, wk, eps, theta, start + r) for r in range(rows)])
    vall = np.vstack([cached_v, vr])
    for r in range(rows):
        qn = _norm_rope_f64(qr[r], n_q, hd, wq, eps, theta, start + r)
        n = start + r + 1
        assert_close(got[r], reference_attention(qn, kall[:n], vall[:n], n_kv, hd, scale), 1e-4, 5e-5, f"row {r}")


def test_norm_weight_lengths_are_checked_q_first_then_k():
    # primitives/norm.rs:72-83: rmsnorm_in_place refuses a weight whose length
    # differs from the head's, LengthMismatch {left: head_dim, right: len}; the
    # callers normalise every q head before any k head (forward.rs:2622-2627,
    # prefill.rs:2057-2076). Nothing is appended on the error.
    n_kv, n_q, hd = 2, 4, 8
    rng = Rng(0x11E7)
    w = rng.vec_in(hd, 0.5, 1.5)
    q, k, v = rng.vec_in(n_q * hd, -1.0, 1.0), rng.vec_in(n_kv * hd, -1.0, 1.0), rng.vec_in(n_kv * hd, -1.0, 1.0)
    cases = [(w[:hd - 1], w, (oracle.RV_PRIM_LENGTH_MISMATCH, hd, hd - 1)),
             (np.concatenate([w, w]), w[:3], (oracle.RV_PRIM_LENGTH_MISMATCH, hd, 2 * hd)),
             (w, w[:3], (oracle.RV_PRIM_LENGTH_MISMATCH, hd, 3)),
             (w, np.concatenate([w, w[:1]]), (oracle.RV_PRIM_LENGTH_MISMATCH, hd, hd + 1))]
    for wq, wk, want in cases:
        kv = oracle.KvCache(1, n_kv, hd, 4, oracle.RV_ELEM_F32)
        with pytest.raises(oracle.OracleError) as e:
            kv.decode_step(0, q, k, v, wq, wk, 1e-6, 1e6, 0, 0.5)
        assert e.value.payload()[:3] == want and e.value.what == "rmsnorm_in_place: x vs weight"
        assert kv.len(0) == 0
        with pytest.raises(oracle.OracleError) as e:
            kv.prefill_chunk(0, q.reshape(1, -1), k.reshape(1, -1), v.reshape(1, -1), wq, wk, 1e-6, 1e6, 0, 0.5)
        assert e.value.payload()[:3] == want
        assert kv.len(0) == 0
    # an empty chunk normalises nothing, so it reports nothing
    kv = oracle.KvCache(1, n_kv, hd, 4, oracle.RV_ELEM_F32)
    out = kv.prefill_chunk(0, np.zeros((0, n_q * hd), np.float32), np.zeros((0, n_kv * hd), np.float32),
                           np.zeros((0, n_kv * hd), np.float32), w[:1], w[:1], 1e-6, 1e6, 0, 0.5)
    assert out.size == 0

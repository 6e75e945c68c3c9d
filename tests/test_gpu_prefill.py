"""Chunked causal prefill on the GPU vs the oracle (model/prefill.rs:2055-2111).

Modes and their stated bounds against the oracle on the same cache, each
applied as both the reference-style elementwise gate (abs or rel) and the
scale-normalised max|err|/max|ref| (tests/gpu_util.py `gate`):
  exact (split-f16 MFMA): rel 1e-4 / abs 5e-5, scaled 1e-5 (the fp32-mode gate);
  f16  (one f16 MFMA per product): rel 4e-3 / abs 4e-3, scaled 2e-3;
  bf16 (one bf16 MFMA per product): rel 3e-2 / abs 3e-2, scaled 1.5e-2.
"""
import os

import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import dev, elem_code, gate, host, rel_err, say, torch_cuda
from helpers import Rng
from ramvamp_amd import synth

pytestmark = pytest.mark.gpu

BOUNDS = {"exact": 1e-4, "f16": 4e-3, "bf16": 3e-2}
ABS = {"exact": 5e-5, "f16": 4e-3, "bf16": 3e-2}  # the reference gate's abs term scales with the mode
SCALE = {"exact": 1e-5, "f16": 2e-3, "bf16": 1.5e-2}  # max|err| / max|ref|
THREADS = min(16, os.cpu_count() or 1)


def twin(rng, n_kv, hd, n_pos, cap, elem):
    kv = rv.KvCache(1, n_kv, hd, cap, elem)
    ref = oracle.KvCache(1, n_kv, hd, cap, elem_code(elem))
    if n_pos:
        K = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        V = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        kv.append_rows(0, K, V)
        ref.append_rows(0, K, V)
    return kv, ref


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("mode", ["exact", "f16", "bf16"])
@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_rows_match_per_row_attention_at(mode, elem, splits):
    # splits (RV_TUNE_PREFILL_KV_SPLIT): 0 the launch plan's choice, 1 none,
    # 3 (the F16/BF16 kernel folds a block's splits inside its launch).
    torch_cuda()
    rng = Rng(0xC0FFEE)
    for n_kv, n_q, hd, start, rows in [(4, 32, 128, 0, 37), (4, 32, 128, 100, 70), (2, 8, 128, 5, 16),
                                       (1, 1, 128, 3, 50), (4, 16, 128, 0, 1), (2, 4, 128, 31, 33),
                                       (1, 16, 128, 7, 21), (1, 32, 128, 64, 9), (3, 9, 128, 2, 5),
                                       (1, 8, 16, 4, 9), (3, 6, 9, 0, 7)]:
        say(f"case rows {(n_kv, n_q, hd, start, rows)} mode={mode} elem={elem}")
        kv, ref = twin(rng, n_kv, hd, start + rows, start + rows, elem)
        kv.set_tuning(rv.RV_TUNE_PREFILL_KV_SPLIT, splits)
        q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        out = dev(np.zeros(q.shape))
        rv.attention_at_rows(dev(q), kv, 0, start, scale, out, mode=mode)
        want = ref.scatter_attention(q, 0, start, scale, THREADS)
        bound = BOUNDS[mode] if hd == 128 else 1e-4  # other head dims run the fp32 decode kernel per row
        e = gate(host(out), want, rel=bound, abs_tol=ABS[mode] if hd == 128 else 5e-5,
                 scale=SCALE[mode] if hd == 128 else 1e-5,
                 what=f"rows {(n_kv, n_q, hd, start, rows)} {mode}")
        say(f"  max rel err {e:.3e}")


@pytest.mark.parametrize("mode", ["f16", "bf16"])
def test_ragged_chunk_shapes_match_the_oracle(mode):
    # Chunk sizes other than 512 rows: partial 256-vector blocks and KV
    # split counts the launch plan picks for them (448, 520, 768 rows).
    torch_cuda()
    rng = Rng(0x4A66ED)
    for start, rows in [(700, 448), (700, 520), (200, 768)]:
        say(f"case ragged chunk start={start} rows={rows} mode={mode}")
        kv, ref = twin(rng, 4, 128, start + rows, start + rows, "f32")
        q = rng.vec_in(rows * 32 * 128, -2.0, 2.0).reshape(rows, -1)
        scale = np.float32(1.0) / np.sqrt(np.float32(128))
        out = dev(np.zeros(q.shape))
        rv.attention_at_rows(dev(q), kv, 0, start, scale, out, mode=mode)
        want = ref.scatter_attention(q, 0, start, scale, THREADS)
        e = gate(host(out), want, rel=BOUNDS[mode], abs_tol=ABS[mode], scale=SCALE[mode],
                 what=f"ragged chunk {(start, rows)} {mode}")
        say(f"  max rel err {e:.3e}")


@pytest.mark.parametrize("mode", ["exact", "f16", "bf16"])
def test_config3_prefill_chunk_matches_the_oracle(mode):
    torch_cuda()
    say(f"case config 3 mode={mode}")
    kv = rv.KvCache(1, 4, 128, 512, "f32")
    ref = oracle.KvCache(1, 4, 128, 512, oracle.RV_ELEM_F32)
    q, k, v = synth.new_rows(3, 512)
    wq, wk = synth.norm_weight(3, synth.T_QN), synth.norm_weight(3, synth.T_KN)
    out = dev(np.zeros(q.shape))
    rv.prefill_chunk(kv, 0, dev(q), dev(k), dev(v), dev(wq), dev(wk), synth.EPS, synth.THETA, 0, synth.SCALE, out,
                     mode=mode)
    want = ref.prefill_chunk(0, q, k, v, wq, wk, synth.EPS, synth.THETA, 0, synth.SCALE, threads=THREADS)
    e = gate(host(out), want, rel=BOUNDS[mode], abs_tol=ABS[mode], scale=SCALE[mode], what=f"config 3 {mode}")
    say(f"config 3 {mode} max rel err {e:.3e}")
    assert kv.len(0) == 512
    for pos in (0, 511):
        gate(kv.k_row(0, pos), ref.read_row(False, 0, pos), rel=2e-7, floor=1e-6, what="cache K")


@pytest.mark.parametrize("splits", [0, 2])
@pytest.mark.parametrize("mode", ["exact", "f16"])
@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_prefill_chunk_matches_the_oracle_across_geometries(mode, elem, splits):
    """The fused path (k/v prologue + append, q prologue inside the attention
    kernels' query loads) for groups 1..8, and the fallback path (full row
    prologue, then per-row decode) where the prefill kernels do not apply
    (group 3, head_dim 16 and 256)."""
    torch_cuda()
    rng = Rng(0xFEED + 7 * splits + (elem == "f16"))
    for n_kv, n_q, hd, start, rows in [(4, 32, 128, 0, 37), (2, 8, 128, 5, 16), (1, 1, 128, 3, 20),
                                       (4, 16, 128, 100, 9), (2, 4, 128, 31, 33), (3, 9, 128, 2, 5),
                                       (1, 8, 16, 4, 9), (2, 4, 256, 7, 6)]:
        say(f"case prefill_chunk {(n_kv, n_q, hd, start, rows)} mode={mode} elem={elem} splits={splits}")
        kv, ref = twin(rng, n_kv, hd, start, start + rows, elem)
        kv.set_tuning(rv.RV_TUNE_PREFILL_KV_SPLIT, splits)
        q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
        k = rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1)
        v = rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1)
        wq, wk = rng.vec_in(hd, 0.9, 1.1), rng.vec_in(hd, 0.9, 1.1)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        out = dev(np.full(q.shape, np.nan))
        rv.prefill_chunk(kv, 0, dev(q), dev(k), dev(v), dev(wq), dev(wk), 1e-6, 1e6, start, scale, out, mode=mode)
        want = ref.prefill_chunk(0, q, k, v, wq, wk, 1e-6, 1e6, start, scale, threads=THREADS)
        fast = hd == 128 and 64 % (n_q // n_kv) == 0
        # f16 planes: a new K row may round one ulp apart (f64 sin/cos of two libms).
        loose = elem == "f16"
        rel = BOUNDS[mode] if fast else 1e-4
        e = gate(host(out), want, rel=max(rel, 1e-3) if loose else rel,
                 abs_tol=max(ABS[mode] if fast else 5e-5, 1.5e-3 if loose else 0),
                 scale=max(SCALE[mode] if fast else 1e-5, 1e-3 if loose else 0),
                 what=f"prefill_chunk {(n_kv, n_q, hd, start, rows)} {mode}")
        say(f"  max rel err {e:.3e}")
        assert kv.len(0) == start + rows


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_chunked_prefill_truncation_and_mode_changes_keep_the_staged_copy_current(elem):
    """The prefill kernels keep a staged copy of each layer's K/V across calls:
    a chunk's row prologue writes its own rows into it, rows that reached the
    cache otherwise are staged from the cache, and attention over existing
    rows restages from the first tile at or past the current prefix. A
    sequence of chunks, a truncation (server prefix reuse), a change of
    arithmetic mode, rows added by decode steps and plain appends, attention
    over a shorter prefix and a cleared cache must each match the oracle
    running the same sequence."""
    torch_cuda()
    rng = Rng(0x57A6E + (elem == "f16"))
    n_kv, n_q, hd = 2, 16, 128
    kv = rv.KvCache(2, n_kv, hd, 448, elem)
    ref = oracle.KvCache(2, n_kv, hd, 448, elem_code(elem))
    wq, wk = rng.vec_in(hd, 0.9, 1.1), rng.vec_in(hd, 0.9, 1.1)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    loose = elem == "f16"

    def chunk(layer, start, rows, mode):
        q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
        k = rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1)
        v = rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1)
        out = dev(np.full(q.shape, np.nan))
        rv.prefill_chunk(kv, layer, dev(q), dev(k), dev(v), dev(wq), dev(wk), 1e-6, 1e6, start, scale, out, mode=mode)
        want = ref.prefill_chunk(layer, q, k, v, wq, wk, 1e-6, 1e6, start, scale, threads=THREADS)
        gate(host(out), want, rel=max(BOUNDS[mode], 1e-3 if loose else 0), abs_tol=max(ABS[mode], 1.5e-3 if loose else 0),
             scale=max(SCALE[mode], 1e-3 if loose else 0), what=f"chunk {layer} {start}+{rows} {mode}")

    for layer in (0, 1):
        say(f"case chunked prefill layer {layer} elem={elem}")
        chunk(layer, 0, 100, "f16")     # tiles 0-1 staged, tile 1 partly
        chunk(layer, 100, 70, "f16")    # restage from tile 1
    kv.truncate(130)
    ref.truncate(130)
    for layer in (0, 1):
        chunk(layer, 130, 90, "f16")    # rows 130.. rewritten: restage from tile 2
        chunk(layer, 220, 33, "exact")  # a mode change restages everything
    # Rows that reach the cache outside a chunk (decode steps, plain appends)
    # are staged from it before the next chunk writes its own rows; chunks
    # ending on a tile boundary leave no tail to zero.
    for layer in (0, 1):
        pos = kv.len(layer)
        for _ in range(3):
            q1 = rng.vec_in(n_q * hd, -2.0, 2.0)
            k1, v1 = rng.vec_in(n_kv * hd, -2.0, 2.0), rng.vec_in(n_kv * hd, -1.0, 1.0)
            out = dev(np.full(q1.shape, np.nan))
            rv.decode_step(kv, layer, dev(q1), dev(k1), dev(v1), dev(wq), dev(wk), 1e-6, 1e6, pos, scale, out)
            ref.decode_step(layer, q1, k1, v1, wq, wk, 1e-6, 1e6, pos, scale, threads=THREADS)
            pos += 1
        assert pos == 256
        chunk(layer, 256, 64, "exact")   # starts and ends on tile boundaries
        k2, v2 = rng.vec_in(9 * n_kv * hd, -2.0, 2.0), rng.vec_in(9 * n_kv * hd, -1.0, 1.0)
        kv.append_rows(layer, k2, v2)
        ref.append_rows(layer, k2, v2)
        chunk(layer, 329, 55, "bf16")    # a mode change after plain appends
        chunk(layer, 384, 17, "bf16")
    # attention over a shorter prefix of the staged layer, then the full one
    q = rng.vec_in(20 * n_q * hd, -2.0, 2.0).reshape(20, -1)
    for start in (40, 381):
        out = dev(np.full(q.shape, np.nan))
        rv.attention_at_rows(dev(q), kv, 1, start, scale, out, mode="f16")
        want = ref.scatter_attention(q, 1, start, scale, THREADS)
        gate(host(out), want, rel=max(BOUNDS["f16"], 1e-3 if loose else 0), abs_tol=ABS["f16"],
             scale=SCALE["f16"], what=f"attention_at_rows start {start}")
    kv.clear()
    ref.clear()
    chunk(0, 0, 64, "f16")
    assert kv.len(0) == 64


@pytest.fixture(scope="module")
def config4_oracle():
    """Config 4's inputs and the oracle's output for all 512 rows (the
    reference's prefill composition, prefill.rs:2055-2111), computed once."""
    start, rows = 3449, 512
    K, V = synth.cached_kv(4, 0, start)
    q, k, v = synth.new_rows(4, rows)
    wq, wk = synth.norm_weight(4, synth.T_QN), synth.norm_weight(4, synth.T_KN)
    ref = oracle.KvCache(1, 4, 128, start + rows, oracle.RV_ELEM_F32)
    ref.append_rows(0, K, V)
    want = ref.prefill_chunk(0, q, k, v, wq, wk, synth.EPS, synth.THETA, start, synth.SCALE, threads=THREADS)
    return start, rows, K, V, q, k, v, wq, wk, want


@pytest.mark.parametrize("mode", ["exact", "f16", "bf16"])
def test_config4_prefix_reuse_prefill_matches_the_oracle(mode, config4_oracle):
    # Every one of the chunk's 512 rows against the oracle, in each mode.
    torch_cuda()
    say(f"case config 4 mode={mode}")
    start, rows, K, V, q, k, v, wq, wk, want = config4_oracle
    kv = rv.KvCache(1, 4, 128, start + rows, "f32")
    kv.append_rows(0, K, V)
    out = dev(np.full(q.shape, np.nan, np.float32))
    rv.prefill_chunk(kv, 0, dev(q), dev(k), dev(v), dev(wq), dev(wk), synth.EPS, synth.THETA, start, synth.SCALE,
                     out, mode=mode)
    got = host(out)
    e = gate(got, want, rel=BOUNDS[mode], abs_tol=ABS[mode], scale=SCALE[mode], what=f"config 4 {mode}")
    say(f"config 4 {mode} max rel err over all {rows} rows {e:.3e}")


def test_prefill_rows_equal_decode_with_the_row_limit():
    # attention.rs:2019-2058 in spirit: the masked (prefill) form equals the
    # position-limited decode form row by row (two different device kernels).
    torch_cuda()
    say("case prefill vs attention_at")
    rng = Rng(0xCA5A)
    kv, _ = twin(rng, 4, 128, 900, 900, "f32")
    start, rows = 700, 200
    q = rng.vec_in(rows * 4096, -1.0, 1.0).reshape(rows, -1)
    out = np.zeros(q.shape, np.float32)
    rv.attention_at_rows(q, kv, 0, start, 0.1, out, mode="exact")
    for r in (0, 1, 99, 199):
        one = np.zeros(4096, np.float32)
        rv.attention_at(q[r], kv, 0, start + r + 1, 0.1, None, one)
        gate(out[r], one, rel=1e-4, what=f"row {r}")


def test_prefill_errors_and_first_row_semantics():
    torch_cuda()
    say("case prefill errors")
    kv = rv.KvCache(2, 4, 128, 64, "f32")
    rng = Rng(3)
    K = rng.vec_in(10 * 512, -1, 1).reshape(10, -1)
    kv.append_rows(0, K, K)
    q = rng.vec_in(8 * 4096, -1, 1).reshape(8, -1)
    out = np.full(q.shape, np.nan, np.float32)
    with pytest.raises(rv.KvError) as e:  # row 7 would attend 11 positions of 10
        rv.attention_at_rows(q, kv, 0, 3, 0.1, out)
    assert e.value.variant == "PositionOutOfRange" and e.value.fields["pos"] == 10 and e.value.fields["len"] == 10
    assert np.all(np.isnan(out))
    with pytest.raises(rv.KvError):
        rv.attention_at_rows(q, kv, 2, 0, 0.1, out)
    with pytest.raises(rv.AttentionError) as e:
        rv.attention_at_rows(np.ascontiguousarray(q[:, :100]), kv, 0, 0, 0.1, np.zeros((8, 100), np.float32))
    assert e.value.variant == "QLenIndivisible"
    rv.attention_at_rows(q[:0], kv, 0, 0, 0.1, out[:0])  # zero rows: a no-op
    rv.attention_at_rows(q[:1], kv, 0, 0, 0.1, out[:1])  # row 0 at start 0 sees only position 0
    # the split mode reproduces V to ~2^-22 relative (hi + lo f16 of the
    # f32, scaled by its tile column's exponent)
    assert np.allclose(out[0].reshape(4, 8, 128), np.broadcast_to(K[0].reshape(4, 1, 128), (4, 8, 128)), rtol=1e-6,
                       atol=0)


@pytest.mark.parametrize("mode", ["exact", "f16", "bf16"])
@pytest.mark.parametrize("vectors_rows,splits", [(0, 0), (8, 1), (16, 1), (16, 2), (8, 3), (8, 4), (16, 5), (8, 6),
                                                 (16, 7), (16, 8)])
def test_tile_shapes_and_kv_splits_agree(mode, vectors_rows, splits):
    """1..8 KV splits (some empty) over a chunk whose rows cross several
    64-position tiles and end in a partial block of query vectors: EXACT at
    64 or 128 query vectors per workgroup (each split count has its own
    merge kernel), F16/BF16 at 256 (the splits folded inside the launch;
    the vector count is EXACT's knob only)."""
    torch_cuda()
    say(f"case tiles rows={vectors_rows} splits={splits} mode={mode}")
    rng = Rng(0x711E + 31 * splits + vectors_rows)
    n_kv, n_q, hd, start, rows = 4, 32, 128, 200, 130
    kv, ref = twin(rng, n_kv, hd, start + rows, start + rows, "f32")
    kv.set_tuning(rv.RV_TUNE_PREFILL_ROWS, vectors_rows)
    kv.set_tuning(rv.RV_TUNE_PREFILL_KV_SPLIT, splits)
    q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = dev(np.full(q.shape, np.nan))
    rv.attention_at_rows(dev(q), kv, 0, start, scale, out, mode=mode)
    want = ref.scatter_attention(q, 0, start, scale, THREADS)
    got = host(out)
    e = gate(got, want, rel=BOUNDS[mode], abs_tol=ABS[mode], scale=SCALE[mode],
             what=f"tiles {vectors_rows}/{splits} {mode}")
    say(f"  max rel err {e:.3e}")
    # Again: the same bits (each split fold's ticket is reset by its last
    # arriver, and the fold runs in split order whichever split finishes last).
    out2 = dev(np.full(q.shape, np.nan))
    rv.attention_at_rows(dev(q), kv, 0, start, scale, out2, mode=mode)
    assert np.array_equal(host(out2).view(np.uint32), got.view(np.uint32))


def weighted_magnitude(q, K, V, n_kv, hd, start, scale):
    """f64 sum_t p_t |V[t][d]| per output element: the size of the terms each
    output sums, which bounds what fp32 arithmetic can resolve in it."""
    rows, q_dim = q.shape
    n_q = q_dim // hd
    group = n_q // n_kv
    qh = q.astype(np.float64).reshape(rows, n_q, hd)
    Kh = K.astype(np.float64).reshape(-1, n_kv, hd)
    Vh = np.abs(V.astype(np.float64)).reshape(-1, n_kv, hd)
    mag = np.zeros((rows, n_q, hd))
    for r in range(rows):
        n = start + r + 1
        for h in range(n_q):
            s = Kh[:n, h // group] @ qh[r, h] * float(scale)
            p = np.exp(s - s.max())
            mag[r, h] = (p / p.sum()) @ Vh[:n, h // group]
    return mag.reshape(rows, q_dim)


@pytest.mark.parametrize("case", ["v_1e6", "v_1e-30", "v_rows_1e-30_to_1e6", "k_rows_1e-25_to_1", "q_1e-20"])
def test_exact_mode_covers_finite_fp32(case):
    """The fp32 parity mode over values far outside f16's range (attention.rs
    takes any finite f32): |V| up to 1e6 and down to 1e-30, V and K rows
    whose magnitudes span many decades within one 64-position tile, and tiny
    q. Every output element must match the oracle to 1e-5 of the magnitude
    of the terms it sums (sum_t p_t |V[t][d]|, in f64), which fp32 itself
    only resolves to a few 1e-7. Scores stay O(10) in size: the mode's
    scores carry ~2^-21 of |q| |k| (fp32's: ~2^-24), so scores of size S
    move the softmax weights by ~S * 2^-21 relative."""
    torch_cuda()
    say(f"case exact range {case}")
    rng = Rng(0xE7AC7 + len(case))
    n_kv, n_q, hd, start, rows = 4, 32, 128, 70, 50
    n_pos = start + rows
    K = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
    V = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
    q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
    decades = rng.vec_in(n_pos, 0.0, 1.0).reshape(n_pos, 1)
    if case == "v_1e6":
        V = V * np.float32(1e6)
    elif case == "v_1e-30":
        V = V * np.float32(1e-30)
    elif case == "v_rows_1e-30_to_1e6":
        V = (V * np.power(10.0, -30.0 + 36.0 * decades)).astype(np.float32)
    elif case == "k_rows_1e-25_to_1":
        K = (K * np.power(10.0, -25.0 + 25.0 * decades)).astype(np.float32)
    elif case == "q_1e-20":
        q = q * np.float32(1e-20)
    kv = rv.KvCache(1, n_kv, hd, n_pos, "f32")
    ref = oracle.KvCache(1, n_kv, hd, n_pos, oracle.RV_ELEM_F32)
    kv.append_rows(0, K, V)
    ref.append_rows(0, K, V)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = dev(np.full(q.shape, np.nan))
    rv.attention_at_rows(dev(q), kv, 0, start, scale, out, mode="exact")
    want = ref.scatter_attention(q, 0, start, scale, THREADS)
    got = host(out)
    assert np.all(np.isfinite(got)), f"{case}: non-finite output"
    mag = weighted_magnitude(q, K, V, n_kv, hd, start, scale)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = float(np.max(err / np.maximum(mag, np.finfo(np.float64).tiny)))
    say(f"  max |err| / sum p|v| = {worst:.3e}")
    assert worst <= 1e-5, f"{case}: max |err| / sum_t p_t |v_t| = {worst:.3e} > 1e-5"


def test_exact_prefill_chunk_with_large_values():
    """prefill_chunk (RMSNorm + RoPE prologue, append, staged rows) in the
    fp32 parity mode with V rows up to 1e6 and down to 1e-30 in magnitude:
    the chunk's own rows go through the row prologue's staging (per-row K
    exponents, bf16 V planes), the cached prefix through the stage kernel."""
    torch_cuda()
    say("case exact prefill_chunk wide V")
    rng = Rng(0xB16)
    n_kv, n_q, hd, start, rows = 4, 32, 128, 90, 70
    kv, ref = twin(rng, n_kv, hd, 0, start + rows, "f32")
    K0 = rng.vec_in(start * n_kv * hd, -1.0, 1.0).reshape(start, -1)
    V0 = (rng.vec_in(start * n_kv * hd, -1.0, 1.0).reshape(start, -1) *
          np.power(10.0, -30.0 + 36.0 * rng.vec_in(start, 0.0, 1.0).reshape(start, 1))).astype(np.float32)
    kv.append_rows(0, K0, V0)
    ref.append_rows(0, K0, V0)
    q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
    k = rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1)
    v = (rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1) *
         np.power(10.0, -30.0 + 36.0 * rng.vec_in(rows, 0.0, 1.0).reshape(rows, 1))).astype(np.float32)
    wq, wk = rng.vec_in(hd, 0.9, 1.1), rng.vec_in(hd, 0.9, 1.1)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = dev(np.full(q.shape, np.nan))
    rv.prefill_chunk(kv, 0, dev(q), dev(k), dev(v), dev(wq), dev(wk), 1e-6, 1e6, start, scale, out, mode="exact")
    want = ref.prefill_chunk(0, q, k, v, wq, wk, 1e-6, 1e6, start, scale, threads=THREADS)
    got = host(out)
    assert np.all(np.isfinite(got))
    # The magnitudes from the post-prologue q (RMSNorm + NeoX RoPE in f64,
    # close enough to weight the terms) and the cache's K and V rows.
    x = q.astype(np.float64).reshape(rows, n_q, hd)
    x = x / np.sqrt(np.mean(x * x, axis=2, keepdims=True) + 1e-6) * wq.astype(np.float64)
    ang = (start + np.arange(rows))[:, None] * np.power(1e6, -2.0 * np.arange(hd // 2) / hd)[None, :]
    c, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    qp = np.concatenate([x[..., :hd // 2] * c - x[..., hd // 2:] * sn, x[..., :hd // 2] * sn + x[..., hd // 2:] * c],
                        axis=2).reshape(rows, -1)
    Kall = np.stack([kv.k_row(0, t) for t in range(start + rows)])
    Vall = np.stack([kv.v_row(0, t) for t in range(start + rows)])
    mag = weighted_magnitude(qp, Kall, Vall, n_kv, hd, start, scale)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    worst = float(np.max(err / np.maximum(mag, np.finfo(np.float64).tiny)))
    say(f"  max |err| / sum p|v| = {worst:.3e}")
    assert worst <= 1e-5
    for pos in (0, start - 1, start, start + rows - 1):
        gate(kv.k_row(0, pos), ref.read_row(False, 0, pos), rel=2e-7, floor=1e-6, what="cache K")
        gate(kv.v_row(0, pos), ref.read_row(True, 0, pos), rel=0, floor=1e-38, what="cache V")

"""A prefill chunk whose attention launch appends its own k/v rows
(RV_TUNE_PREFILL_FUSE 2, F16/BF16) against the same chunk with the
row-prologue launch before it (the default), on twin caches, and against the
oracle.

Both paths run the same attention arithmetic; they differ only where the k
rows' RMSNorm sums its squares (two f64 orders) and where (cos, sin) come from
(the host's f64 sincos for the fused launch, the device's for the row
prologue), each rounded to f32 afterwards. So the cache rows and outputs are
expected to be bit-identical except, rarely, one f32 ulp in a K value. Held:
V rows bit-identical; K rows within 1 ulp with at most 1 in 10^4 values
apart; outputs within 1e-6 of the output's scale. Covers chunks from an empty
cache, starts inside a tile, chunks crossing tiles, single rows, groups 1..64
(row blocks of 64 down to one row), KV splits, 64 or 128 vectors per
workgroup, both attention kernels, chunk after chunk, and later reads of the
staged copy (attention over the rows, and a decode step). Against the
oracle, config 3 and a chunk starting inside a tile are held to
test_gpu_prefill.py's f16/bf16 bounds.
"""
import numpy as np
import pytest

import ramvamp_amd as rv
from gpu_util import dev, host, say, torch_cuda
from helpers import Rng

pytestmark = pytest.mark.gpu


def _k_close(a, b, elem, what):
    if elem == "f16":
        x, y = a.view(np.uint16).astype(np.int32), b.view(np.uint16).astype(np.int32)
    else:
        x, y = a.view(np.int32).astype(np.int64), b.view(np.int32).astype(np.int64)
    d = np.abs(x - y)
    assert d.max() <= 1, f"{what}: K rows {int(d.max())} ulps apart"
    assert np.count_nonzero(d) <= max(1, d.size // 10000), f"{what}: {np.count_nonzero(d)} K values 1 ulp apart"


def _run(torch, elem, mode, n_kv, n_q, prefix, chunks, cap, tune, seed):
    hd = 128
    rng = Rng(seed)
    caches = [rv.KvCache(1, n_kv, hd, cap, elem) for _ in range(2)]
    caches[0].set_tuning(rv.RV_TUNE_PREFILL_FUSE, 2)
    for kv in caches:
        for knob, val in tune.items():
            kv.set_tuning(knob, val)
    if prefix:
        K = rng.vec_in(prefix * n_kv * hd, -1.0, 1.0).reshape(prefix, -1)
        V = rng.vec_in(prefix * n_kv * hd, -1.0, 1.0).reshape(prefix, -1)
        for kv in caches:
            kv.append_rows(0, K, V)
    wq, wk = dev(rng.vec_in(hd, 0.9, 1.1)), dev(rng.vec_in(hd, 0.9, 1.1))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    start = prefix
    for rows in chunks:
        what = f"{elem} {mode} kv{n_kv} q{n_q} start {start} rows {rows} {tune}"
        say(f"case fused chunk {what}")
        q = dev(rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1))
        k = dev(rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1))
        v = dev(rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1))
        outs = []
        for kv in caches:
            out = dev(np.full((rows, n_q * hd), np.nan, np.float32))
            rv.prefill_chunk(kv, 0, q, k, v, wq, wk, 1e-6, 1e6, start, scale, out, mode=mode)
            outs.append(host(out).copy())
        a, b = outs
        assert np.all(np.isfinite(a)), what
        err = float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))
        same = float(np.mean(a.view(np.uint32) == b.view(np.uint32)))
        say(f"  out max|diff|/max|out| {err:.2e}, {100 * same:.3f}% bit-identical")
        assert err <= 1e-6, what
        for p in range(start, start + rows):
            assert np.array_equal(caches[0].v_row(0, p), caches[1].v_row(0, p)), (what, p)
        ka = np.stack([caches[0].k_row(0, p) for p in range(start, start + rows)])
        kb = np.stack([caches[1].k_row(0, p) for p in range(start, start + rows)])
        _k_close(ka, kb, elem, what)
        start += rows
        assert caches[0].len(0) == start == caches[1].len(0)
    # The staged copy the fused launches wrote (rows and the zeroed tail of
    # the last tile), read by attention over the existing rows ...
    nr = min(start, 40)
    qr_ = dev(rng.vec_in(nr * n_q * hd, -2.0, 2.0).reshape(nr, -1))
    outs = []
    for kv in caches:
        out = dev(np.full((nr, n_q * hd), np.nan, np.float32))
        rv.attention_at_rows(qr_, kv, 0, start - nr, scale, out, mode=mode)
        outs.append(host(out).copy())
    err = float(np.max(np.abs(outs[0].astype(np.float64) - outs[1])) / np.max(np.abs(outs[1])))
    assert err <= 1e-6, f"attention_at_rows after the chunks: {err:.2e}"
    # ... and the cache by a decode step.
    if start < cap:
        q1, k1, v1 = (dev(rng.vec_in(n * hd, -2.0, 2.0)) for n in (n_q, n_kv, n_kv))
        outs = []
        for kv in caches:
            out = dev(np.full(n_q * hd, np.nan, np.float32))
            rv.decode_step(kv, 0, q1, k1, v1, wq, wk, 1e-6, 1e6, start, scale, out)
            outs.append(host(out).copy())
        err = float(np.max(np.abs(outs[0].astype(np.float64) - outs[1])) / np.max(np.abs(outs[1])))
        assert err <= 1e-6, f"decode step after the chunks: {err:.2e}"


@pytest.mark.parametrize("mode", ["f16", "bf16"])
@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_fused_chunks_follow_the_row_prologue_path(elem, mode):
    torch = torch_cuda()
    P = rv.RV_TUNE_PREFILL_IMPL
    cases = [
        # (n_kv, n_q, prefix, chunks, cap, tune)
        (4, 32, 0, [512], 600, {}),                      # config 3's shape
        (4, 32, 57, [9, 100, 1, 70], 300, {}),          # starts inside tiles, chunk after chunk
        (4, 32, 200, [130], 400, {2: 3, 4: 16, P: 1}),   # 3 KV splits, 128 vectors, two-group kernel
        (4, 32, 200, [130], 400, {2: 2, P: 2}),          # 2 KV splits, pipelined kernel
        (2, 8, 63, [1, 64, 65], 256, {}),                # group 4
        (1, 1, 5, [33], 64, {P: 1}),                     # group 1, a full cache
        (1, 16, 3, [40], 128, {}),                       # group 16: 4-row blocks
        (1, 64, 10, [70], 128, {}),                      # group 64: one-row blocks
    ]
    for i, (n_kv, n_q, prefix, chunks, cap, tune) in enumerate(cases):
        _run(torch, elem, mode, n_kv, n_q, prefix, chunks, cap, tune, 0xF05E + 17 * i + (elem == "f16"))


def test_fused_config4_shape():
    # BASELINE config 4's chunk after its 3449-row prefix (KV range 62 tiles).
    torch = torch_cuda()
    _run(torch, "f32", "f16", 4, 32, 3449, [512], 4096, {}, 0xC0F4)


def test_a_captured_chunk_takes_the_row_prologue_path():
    # Graph capture keeps the row-prologue launch (the fused path's flags
    # carry an epoch the host sets per call): the captured chunk equals the
    # eager fused one.
    torch = torch_cuda()
    say("case captured prefill chunk")
    rng = Rng(0xCA97)
    n_kv, n_q, hd, prefix, rows = 4, 32, 128, 70, 50
    K = rng.vec_in(prefix * n_kv * hd, -1.0, 1.0).reshape(prefix, -1)
    V = rng.vec_in(prefix * n_kv * hd, -1.0, 1.0).reshape(prefix, -1)
    caches = [rv.KvCache(1, n_kv, hd, 256, "f32") for _ in range(2)]
    for kv in caches:
        kv.set_tuning(rv.RV_TUNE_PREFILL_FUSE, 2)
        kv.append_rows(0, K, V)
    q = dev(rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1))
    k = dev(rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1))
    v = dev(rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1))
    wq, wk = dev(rng.vec_in(hd, 0.9, 1.1)), dev(rng.vec_in(hd, 0.9, 1.1))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    eager = dev(np.full((rows, n_q * hd), np.nan, np.float32))
    rv.prefill_chunk(caches[0], 0, q, k, v, wq, wk, 1e-6, 1e6, prefix, scale, eager, mode="f16")
    want = host(eager).copy()
    out = dev(np.full((rows, n_q * hd), np.nan, np.float32))
    # One eager call sizes the cache's workspace and q buffer (a capture may
    # not allocate); the rows it appended are dropped again.
    rv.prefill_chunk(caches[1], 0, q, k, v, wq, wk, 1e-6, 1e6, prefix, scale, out, mode="f16")
    caches[1].truncate(prefix)
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rv.prefill_chunk(caches[1], 0, q, k, v, wq, wk, 1e-6, 1e6, prefix, scale, out, mode="f16")
    g.replay()
    got = host(out)
    err = float(np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)))
    assert err <= 1e-6, err
    assert caches[1].len(0) == prefix + rows


@pytest.mark.parametrize("mode", ["f16", "bf16"])
@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_fused_chunks_match_the_oracle(elem, mode):
    import oracle
    from gpu_util import elem_code, gate
    from test_gpu_prefill import ABS, BOUNDS, SCALE, THREADS

    torch_cuda()
    rng = Rng(0xF0A1 + (elem == "f16") + 2 * (mode == "bf16"))
    loose = elem == "f16"
    for n_kv, n_q, prefix, rows in ((4, 32, 0, 512), (2, 16, 57, 90)):
        say(f"case fused chunk vs oracle {elem} {mode} kv{n_kv} q{n_q} start {prefix} rows {rows}")
        hd = 128
        kv = rv.KvCache(1, n_kv, hd, prefix + rows, elem)
        kv.set_tuning(rv.RV_TUNE_PREFILL_FUSE, 2)
        ref = oracle.KvCache(1, n_kv, hd, prefix + rows, elem_code(elem))
        if prefix:
            K = rng.vec_in(prefix * n_kv * hd, -1.0, 1.0).reshape(prefix, -1)
            V = rng.vec_in(prefix * n_kv * hd, -1.0, 1.0).reshape(prefix, -1)
            kv.append_rows(0, K, V)
            ref.append_rows(0, K, V)
        q = rng.vec_in(rows * n_q * hd, -2.0, 2.0).reshape(rows, -1)
        k = rng.vec_in(rows * n_kv * hd, -2.0, 2.0).reshape(rows, -1)
        v = rng.vec_in(rows * n_kv * hd, -1.0, 1.0).reshape(rows, -1)
        wq, wk = rng.vec_in(hd, 0.9, 1.1), rng.vec_in(hd, 0.9, 1.1)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        out = dev(np.full(q.shape, np.nan))
        rv.prefill_chunk(kv, 0, dev(q), dev(k), dev(v), dev(wq), dev(wk), 1e-6, 1e6, prefix, scale, out, mode=mode)
        want = ref.prefill_chunk(0, q, k, v, wq, wk, 1e-6, 1e6, prefix, scale, threads=THREADS)
        e = gate(host(out), want, rel=max(BOUNDS[mode], 1e-3 if loose else 0),
                 abs_tol=max(ABS[mode], 1.5e-3 if loose else 0), scale=max(SCALE[mode], 1e-3 if loose else 0),
                 what=f"fused chunk {elem} {mode} {prefix}+{rows}")
        say(f"  max rel err {e:.3e}")
        for p in range(prefix, prefix + rows):
            assert np.array_equal(kv.v_row(0, p), ref.read_row(True, 0, p)), p

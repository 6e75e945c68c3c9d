"""Token graph: one token's layer steps captured once into a HIP graph with
the token's position in device memory (rv_decode_step_dev,
rv_attn_block_decode_dev, rv_position_advance) and replayed for every
following token, the inputs refilled and the outputs NaN-filled between
replays.

Each replay is held to three references: eager device-position steps on a
twin cache (bit for bit: the same launches), eager rv_decode_step /
rv_attn_block_decode on a third cache at the host position (fp32 gate: the
device-position launch is planned for max_position, so its splits and
therefore its summation order differ), and the oracle's decode step
(model/forward.rs:2622-2633). After the replays the layers' lengths have not
moved until rv_kv_commit adds the rows, and the rows the graph wrote equal the
eager steps' bit for bit.
"""
import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import FP32_FLOOR, FP32_REL, dev, elem_code, gate, host, say, torch_cuda
from helpers import Rng
from ramvamp_amd import block as B

pytestmark = pytest.mark.gpu

EPS, THETA = 1e-6, 1e6


def _caches(rng, n, n_layers, n_kv, hd, n_pos, cap, elem):
    devs = [rv.KvCache(n_layers, n_kv, hd, cap, elem) for _ in range(n)]
    ref = oracle.KvCache(n_layers, n_kv, hd, cap, elem_code(elem))
    for layer in range(n_layers):
        K = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        V = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        for kv in devs:
            kv.append_rows(layer, K, V)
        ref.append_rows(layer, K, V)
    return devs, ref


def _bits(a):
    return np.asarray(a).view(np.uint32 if np.asarray(a).dtype == np.float32 else np.uint16)


@pytest.mark.parametrize("elem,n_pos,cap", [("f32", 1000, 1200), ("f16", 1000, 1200), ("f32", 5, 8192),
                                           ("f16", 100, 180)])
def test_decode_step_graph_replays_follow_the_eager_steps(elem, n_pos, cap):
    # (f32, 5, 8192): the launch is planned for 8192 positions while the
    # layers hold 5..10: almost every split is empty and must contribute
    # nothing to the merge. (f16, 100, 180): planned for 179 positions, one
    # split per kv head and no merge, the layers holding 100..106.
    torch = torch_cuda()
    say(f"case token graph decode_step_dev elem={elem} n_pos={n_pos} cap={cap}")
    rng = Rng(0x70C0 + n_pos)
    n_layers, n_kv, n_q, hd, n_tok = 3, 4, 32, 128, 6
    (kv_g, kv_d, kv_e), ref = _caches(rng, 3, n_layers, n_kv, hd, n_pos, cap, elem)
    wq, wk = rng.vec_in(hd, 0.9, 1.1), rng.vec_in(hd, 0.9, 1.1)
    dwq, dwk = dev(wq), dev(wk)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    max_pos = cap - 1
    qb = torch.zeros(n_layers, n_q * hd, device="cuda")
    kb = torch.zeros(n_layers, n_kv * hd, device="cuda")
    vb = torch.zeros(n_layers, n_kv * hd, device="cuda")
    out_g, out_d, out_e = (torch.zeros(n_layers, n_q * hd, device="cuda") for _ in range(3))
    pos_g = torch.tensor([n_pos], dtype=torch.int32, device="cuda")
    pos_d = torch.tensor([n_pos], dtype=torch.int32, device="cuda")

    def token(kv, pos_t, out):
        for layer in range(n_layers):
            rv.decode_step_dev(kv, layer, qb[layer], kb[layer], vb[layer], dwq, dwk, EPS, THETA, pos_t, max_pos,
                               scale, out[layer])
        rv.position_advance(kv, pos_t, 1)

    f16 = elem == "f16"
    g = None
    for t in range(n_tok):
        pos = n_pos + t
        q = rng.vec_in(n_layers * n_q * hd, -2.0, 2.0).reshape(n_layers, -1)
        k = rng.vec_in(n_layers * n_kv * hd, -2.0, 2.0).reshape(n_layers, -1)
        v = rng.vec_in(n_layers * n_kv * hd, -2.0, 2.0).reshape(n_layers, -1)
        qb.copy_(dev(q))
        kb.copy_(dev(k))
        vb.copy_(dev(v))
        for o in (out_g, out_d, out_e):
            o.fill_(float("nan"))
        if t == 0:
            token(kv_g, pos_g, out_g)  # the first token runs eagerly: it builds the (cos, sin) table
        else:
            if g is None:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    token(kv_g, pos_g, out_g)
            g.replay()
        got = host(out_g).copy()
        token(kv_d, pos_d, out_d)  # eager work between replays
        for layer in range(n_layers):
            rv.decode_step(kv_e, layer, qb[layer], kb[layer], vb[layer], dwq, dwk, EPS, THETA, pos, scale,
                           out_e[layer])
        assert np.array_equal(_bits(got), _bits(host(out_d))), f"token {t}: replay vs eager device-position step"
        eager = host(out_e)
        for layer in range(n_layers):
            gate(got[layer], eager[layer], what=f"token {t} layer {layer} vs rv_decode_step")
            want = ref.decode_step(layer, q[layer], k[layer], v[layer], wq, wk, EPS, THETA, pos, scale)
            gate(got[layer], want, rel=1e-3 if f16 else FP32_REL, abs_tol=1.5e-3 if f16 else FP32_FLOOR,
                 what=f"token {t} layer {layer} vs oracle")
        say(f"token {t} position {pos}: replay == eager device-position step")
    assert int(pos_g.item()) == n_pos + n_tok and int(pos_d.item()) == n_pos + n_tok
    for layer in range(n_layers):
        assert kv_g.len(layer) == n_pos and kv_e.len(layer) == n_pos + n_tok
        kv_g.commit(layer, n_tok)
        kv_d.commit(layer, n_tok)
        assert kv_g.len(layer) == n_pos + n_tok
        for p in range(n_pos, n_pos + n_tok):
            kg, vg = kv_g.k_row(layer, p), kv_g.v_row(layer, p)
            assert np.array_equal(kg, kv_d.k_row(layer, p)) and np.array_equal(vg, kv_d.v_row(layer, p)), (layer, p)
            assert np.array_equal(kg, kv_e.k_row(layer, p)) and np.array_equal(vg, kv_e.v_row(layer, p)), (layer, p)
            assert np.array_equal(vg, ref.read_row(True, layer, p)), (layer, p)
            gate(kg.view(np.float16).astype(np.float32) if f16 else kg,
                 ref.read_row(False, layer, p).view(np.float16).astype(np.float32) if f16 else
                 ref.read_row(False, layer, p), rel=1e-3 if f16 else 2e-7, floor=1e-6, what=f"K row {layer} {p}")
    # Committed, the cache continues with ordinary steps: the next token on
    # the graph's cache equals the one on the eager cache bit for bit.
    pos = n_pos + n_tok
    q = dev(rng.vec_in(n_q * hd, -2.0, 2.0))
    k, v = dev(rng.vec_in(n_kv * hd, -2.0, 2.0)), dev(rng.vec_in(n_kv * hd, -2.0, 2.0))
    a, b = torch.zeros(n_q * hd, device="cuda"), torch.zeros(n_q * hd, device="cuda")
    rv.decode_step(kv_g, 1, q, k, v, dwq, dwk, EPS, THETA, pos, scale, a)
    rv.decode_step(kv_e, 1, q, k, v, dwq, dwk, EPS, THETA, pos, scale, b)
    assert np.array_equal(_bits(host(a)), _bits(host(b)))
    with pytest.raises(rv.KvError) as ei:
        kv_g.commit(0, cap)
    assert ei.value.variant == "CapacityExceeded" and kv_g.len(0) == n_pos + n_tok


def test_decode_step_dev_rejections():
    torch = torch_cuda()
    say("case decode_step_dev rejections")
    rng = Rng(0x70C9)
    (kv,), _ = _caches(rng, 1, 1, 2, 128, 4, 16, "f32")
    q, k, v = dev(rng.vec_in(8 * 128, -1, 1)), dev(rng.vec_in(256, -1, 1)), dev(rng.vec_in(256, -1, 1))
    w = dev(np.ones(128, np.float32))
    out = torch.zeros(8 * 128, device="cuda")
    pos = torch.tensor([4], dtype=torch.int32, device="cuda")

    def call(**kw):
        a = dict(q=q, k=k, v=v, w=w, out=out, pos=pos, max_pos=15)
        a.update(kw)
        rv.decode_step_dev(kv, 0, a["q"], a["k"], a["v"], a["w"], a["w"], EPS, THETA, a["pos"], a["max_pos"], 0.1,
                           a["out"])

    with pytest.raises(rv.KvError) as ei:
        call(max_pos=16)  # no row left for position 16 in a 16-row layer
    assert ei.value.variant == "CapacityExceeded"
    with pytest.raises(rv.DeviceError) as ei:
        call(q=dev(rng.vec_in(34 * 128, -1, 1)), out=torch.zeros(34 * 128, device="cuda"))  # group 17
    assert ei.value.variant == "Unsupported"
    with pytest.raises(rv.DeviceError) as ei:  # host arrays: device pointers only
        call(q=rng.vec_in(8 * 128, -1, 1), k=rng.vec_in(256, -1, 1), v=rng.vec_in(256, -1, 1),
             w=np.ones(128, np.float32), out=np.zeros(8 * 128, np.float32))
    assert ei.value.variant == "Unsupported"
    with pytest.raises(TypeError):
        call(pos=torch.tensor([4], dtype=torch.int64, device="cuda"))
    torch.cuda.synchronize()
    assert kv.len(0) == 4
    call()  # a valid call writes row 4 and leaves the length
    torch.cuda.synchronize()
    assert kv.len(0) == 4
    kv.commit(0, 1)
    assert kv.len(0) == 5


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_a_device_position_past_the_plan_is_refused_on_the_device(elem):
    """A device-position step whose *d_position (read as unsigned) is past
    its max_position writes no cache row and leaves `out` as it was, eagerly
    and in a graph replay, and records CapacityExceeded (layer, max_position +
    1) in the cache's device status, as KvCache::append refuses a full layer
    (kv/mod.rs:352-357); rv_kv_commit reports it too and moves no cursor. An
    int32 -1 (0xFFFFFFFF) is past every plan. The attention block's device
    form leaves the residual untouched the same way."""
    torch = torch_cuda()
    say(f"case device position past the plan elem={elem}")
    rng = Rng(0x70CA)
    (kv,), _ = _caches(rng, 1, 2, 2, 128, 4, 16, elem)
    q, k, v = dev(rng.vec_in(8 * 128, -1, 1)), dev(rng.vec_in(256, -1, 1)), dev(rng.vec_in(256, -1, 1))
    w = dev(np.ones(128, np.float32))
    out = torch.zeros(8 * 128, device="cuda")
    max_pos = 9
    # Rows past a layer's length cannot be read until committed; the planes
    # start zeroed (rv_kv_new), so every row a step did not write stays zero.
    rows_before = [(kv.k_row(layer, p), kv.v_row(layer, p)) for layer in range(2) for p in range(4)]
    for bad in (10, 15, -1):
        pos = torch.tensor([bad], dtype=torch.int32, device="cuda")
        out.fill_(float("nan"))
        rv.decode_step_dev(kv, 1, q, k, v, w, w, EPS, THETA, pos, max_pos, 0.1, out)
        torch.cuda.synchronize()
        assert bool(torch.isnan(out).all()), bad
        with pytest.raises(rv.KvError) as ei:
            kv.device_status()
        assert ei.value.variant == "CapacityExceeded" and ei.value.fields["layer"] == 1
        assert ei.value.fields["capacity"] == max_pos + 1 and ei.value.raw[3] == (bad & 0xFFFFFFFF)
        kv.device_status()  # read once, cleared
    # In a graph: the first replay at position 9 writes row 9, the second (10)
    # is refused.
    pos = torch.tensor([max_pos], dtype=torch.int32, device="cuda")
    rv.decode_step_dev(kv, 0, q, k, v, w, w, EPS, THETA, pos, max_pos, 0.1, out)  # builds the table
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rv.decode_step_dev(kv, 0, q, k, v, w, w, EPS, THETA, pos, max_pos, 0.1, out)
        rv.position_advance(kv, pos, 1)
    out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert not bool(torch.isnan(out).any())
    kv.device_status()
    out.fill_(float("nan"))
    g.replay()  # position 10
    torch.cuda.synchronize()
    assert bool(torch.isnan(out).all()) and int(pos.item()) == max_pos + 2
    with pytest.raises(rv.KvError) as ei:
        kv.commit(0, 1)
    assert ei.value.variant == "CapacityExceeded" and ei.value.fields["layer"] == 0 and kv.len(0) == 4
    kv.commit(0, 12)  # the status was read and cleared: every row becomes readable
    kv.commit(1, 12)
    assert np.any(kv.k_row(0, 9) != 0) and np.any(kv.v_row(0, 9) != 0)
    for layer in range(2):
        for p in range(16):
            k_, v_ = kv.k_row(layer, p), kv.v_row(layer, p)
            if p < 4:
                k0, v0 = rows_before[layer * 4 + p]
                assert np.array_equal(k_, k0) and np.array_equal(v_, v0), (layer, p)
            elif (layer, p) != (0, 9):  # the accepted steps' row
                assert not np.any(k_) and not np.any(v_), (layer, p)

    from test_gpu_block import Layer

    Q = oracle
    hd, n_heads, n_kv, hidden, cap = 128, 32, 4, 2048, 64
    q_dim, kv_dim = n_heads * hd, n_kv * hd
    nrng = np.random.default_rng(0xB70E)
    lay = Layer(torch, nrng, hidden, q_dim, kv_dim, hd, Q.RV_QF_Q4_K, Q.RV_QF_Q6_K, Q.RV_QF_Q5_K)
    (kb,), _ = _caches(Rng(0xB70F), 1, 1, n_kv, hd, 8, cap, elem)
    sc = torch.empty(B.scratch_bytes(hidden, q_dim, kv_dim), dtype=torch.uint8, device="cuda")
    res = torch.from_numpy((1.5 * nrng.standard_normal(hidden)).astype(np.float32)).cuda()
    keep = res.clone()
    pos = torch.tensor([40], dtype=torch.int32, device="cuda")
    B.attn_block_decode_dev(kb, 0, res, q_dim, lay.dev, EPS, THETA, pos, 20, 0.088, sc)
    torch.cuda.synchronize()
    assert torch.equal(res, keep)
    with pytest.raises(rv.KvError) as ei:
        kb.device_status()
    assert ei.value.variant == "CapacityExceeded" and ei.value.fields["capacity"] == 21


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_block_graph_replays_follow_the_eager_blocks(elem):
    """The attention block of two layers per token captured once with the
    position on the device; each replay's residual equals eager
    rv_attn_block_decode_dev's bit for bit and eager rv_attn_block_decode's
    within 2e-3 of the output projection's scale (the two launches' different
    split orders can move one quantized attention value by one step)."""
    from test_gpu_block import Layer

    torch = torch_cuda()
    say(f"case token graph attn_block_decode_dev elem={elem}")
    Q = oracle
    hd, n_heads, n_kv, hidden, n_pos, n_tok, cap = 128, 32, 4, 2048, 300, 5, 512
    q_dim, kv_dim = n_heads * hd, n_kv * hd
    nrng = np.random.default_rng(0xB70C)
    lays = [Layer(torch, nrng, hidden, q_dim, kv_dim, hd, Q.RV_QF_Q4_K, Q.RV_QF_Q6_K, Q.RV_QF_Q5_K)
            for _ in range(2)]
    (kv_g, kv_d, kv_e), _ = _caches(Rng(0xB70D), 3, 2, n_kv, hd, n_pos, cap, elem)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    nb = B.scratch_bytes(hidden, q_dim, kv_dim)
    sc_g, sc_d, sc_e = (torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(3))
    res_g, res_d, res_e = (torch.zeros(hidden, device="cuda") for _ in range(3))
    pos_g = torch.tensor([n_pos], dtype=torch.int32, device="cuda")
    pos_d = torch.tensor([n_pos], dtype=torch.int32, device="cuda")

    def token(kv, res, pos_t, sc):
        for layer in range(2):
            B.attn_block_decode_dev(kv, layer, res, q_dim, lays[layer].dev, EPS, THETA, pos_t, cap - 1, scale, sc)
        rv.position_advance(kv, pos_t, 1)

    g = None
    for t in range(n_tok):
        x = torch.from_numpy((1.5 * nrng.standard_normal(hidden)).astype(np.float32)).cuda()
        for r in (res_g, res_d, res_e):
            r.copy_(x)
        if t == 0:
            token(kv_g, res_g, pos_g, sc_g)
        else:
            if g is None:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    token(kv_g, res_g, pos_g, sc_g)
            g.replay()
        got = host(res_g).copy()
        token(kv_d, res_d, pos_d, sc_d)
        for layer in range(2):
            B.attn_block_decode(kv_e, layer, res_e, q_dim, lays[layer].dev, EPS, THETA, n_pos + t, scale,
                                scratch=sc_e)
        assert np.array_equal(_bits(got), _bits(host(res_d))), f"token {t}: replay vs eager device-position block"
        delta = host(res_e).astype(np.float64) - host(x).astype(np.float64)
        err = np.max(np.abs(got.astype(np.float64) - host(res_e))) / np.max(np.abs(delta))
        say(f"token {t}: residual max|err|/max|o| vs host-position block {err:.2e}")
        assert err <= 2e-3, f"token {t}"
    assert int(pos_g.item()) == n_pos + n_tok
    for layer in range(2):
        assert kv_g.len(layer) == n_pos
        kv_g.commit(layer, n_tok)
        kv_d.commit(layer, n_tok)
        for p in range(n_pos, n_pos + n_tok):
            assert np.array_equal(kv_g.k_row(layer, p), kv_d.k_row(layer, p)), (layer, p)
            assert np.array_equal(kv_g.v_row(layer, p), kv_d.v_row(layer, p)), (layer, p)
    # Layer 0's k and v come from the token's residual alone: the same rows
    # as the host-position blocks wrote.
    for p in range(n_pos, n_pos + n_tok):
        assert np.array_equal(kv_g.k_row(0, p), kv_e.k_row(0, p)), p
        assert np.array_equal(kv_g.v_row(0, p), kv_e.v_row(0, p)), p

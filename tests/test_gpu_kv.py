"""Device KV cache vs the oracle (kv/mod.rs): bit-exact rows, cursors, errors."""
import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import dev, say, torch_cuda
from helpers import Rng

pytestmark = pytest.mark.gpu


def special_values():
    f16_ulp = np.float32(2.0 ** -24)
    vals = [0.0, -0.0, 1.0, -2.5, 65504.0, 65519.0, 65520.0, 1e9, np.inf, -np.inf, f16_ulp, 0.5 * f16_ulp,
            0.75 * f16_ulp, 1.5 * f16_ulp, 2.5 * f16_ulp, 1e-10, -1e-10, np.float32(1.0004883), np.float32(1.0004884),
            np.float32(1.0014648), np.float32(6.1035156e-05), np.float32(6.0975552e-05), np.nan]
    payload = np.array([0x7F800001, 0xFFC00123, 0x7FBFFFFF], dtype=np.uint32).view(np.float32)
    return np.concatenate([np.array(vals, np.float32), payload])


@pytest.mark.parametrize("elem", ["f16", "f32"])
@pytest.mark.parametrize("io", ["device", "host"])
def test_append_rows_are_the_oracles_bits(elem, io):
    torch_cuda()
    say(f"case append elem={elem} io={io}")
    n_layers, n_kv, hd, cap = 2, 4, 128, 64
    kv_dim = n_kv * hd
    kv = rv.KvCache(n_layers, n_kv, hd, cap, elem)
    ref = oracle.KvCache(n_layers, n_kv, hd, cap, oracle.RV_ELEM_F16 if elem == "f16" else oracle.RV_ELEM_F32)
    rng = np.random.default_rng(1)
    rows = []
    sp = special_values()
    for r in range(7):
        k = (rng.standard_normal(kv_dim) * 10 ** rng.uniform(-6, 4)).astype(np.float32)
        v = rng.integers(0, 2 ** 32, kv_dim, dtype=np.uint64).astype(np.uint32).view(np.float32).copy()
        k[:sp.size] = sp
        rows.append((k, v))
    for k, v in rows[:3]:
        if io == "device":
            kv.append(1, dev(k), dev(v))
        else:
            kv.append(1, k, v)
        ref.append(1, k, v)
    K = np.stack([r[0] for r in rows[3:]])
    V = np.stack([r[1] for r in rows[3:]])
    if io == "device":
        kv.append_rows(1, dev(K), dev(V))
    else:
        kv.append_rows(1, K, V)
    ref.append_rows(1, K, V)
    kv.synchronize()
    assert kv.len(1) == ref.len(1) == 7 and kv.len(0) == 0
    for pos in range(7):
        for plane_v in (False, True):
            got = kv.v_row(1, pos) if plane_v else kv.k_row(1, pos)
            want = ref.read_row(plane_v, 1, pos)
            assert np.array_equal(got.view(np.uint16 if elem == "f16" else np.uint32),
                                  want.view(np.uint16 if elem == "f16" else np.uint32)), (pos, plane_v)


def test_errors_cursors_truncate_clear_match_the_oracle():
    torch_cuda()
    say("case kv errors")
    kv = rv.KvCache(2, 2, 4, 3, "f16")
    ref = oracle.KvCache(2, 2, 4, 3)
    row = np.arange(8, dtype=np.float32) * 0.5

    def both(fn_dev, fn_ref):
        got = want = None
        try:
            fn_dev()
        except rv.RamvampError as e:
            got = e.raw
        try:
            fn_ref()
        except oracle.OracleError as e:
            want = e.payload()
        assert got == want, (got, want)

    both(lambda: kv.append(0, row, -row), lambda: ref.append(0, row, -row))
    both(lambda: kv.seq_len(), lambda: ref.seq_len())
    both(lambda: kv.append(2, row, row), lambda: ref.append(2, row, row))
    both(lambda: kv.append(0, row[:7], row), lambda: ref.append(0, row[:7], row))
    both(lambda: kv.append(0, row, row[:5]), lambda: ref.append(0, row, row[:5]))
    both(lambda: kv.truncate(0), lambda: ref.truncate(0))
    both(lambda: kv.append(1, row, row), lambda: ref.append(1, row, row))
    both(lambda: kv.truncate(1), lambda: ref.truncate(1))
    both(lambda: kv.truncate(2), lambda: ref.truncate(2))
    for _ in range(3):
        both(lambda: kv.append(0, row, row), lambda: ref.append(0, row, row))
    both(lambda: kv.k_row(1, 1), lambda: ref.read_row(False, 1, 1))
    assert kv.len(0) == ref.len(0) and kv.len(1) == ref.len(1)
    kv.clear()
    ref.clear()
    assert kv.is_empty() and kv.seq_len() == 0
    with pytest.raises(rv.KvError) as e:
        rv.KvCache(0, 4, 128, 8)
    assert e.value.variant == "InvalidDims" and e.value.what == "all dims must be nonzero"
    assert rv.KvCache.projected_bytes(48, 4, 128, 4096) == 384 << 20


def test_layer_views_cover_exactly_the_cursor():
    torch = torch_cuda()
    say("case layer views")
    rng = Rng(0x1A7E)
    kv = rv.KvCache(3, 2, 16, 10, "f32")
    for layer, n in ((0, 3), (2, 5)):
        for _ in range(n):
            kv.append(layer, rng.vec_in(32, -1, 1), rng.vec_in(32, -1, 1))
    for layer, n in ((0, 3), (1, 0), (2, 5)):
        p, cnt = kv.k_layer(layer)
        assert cnt == n * 32 and p
    p0, _ = kv.k_layer(0)
    p2, _ = kv.k_layer(2)
    assert p2 - p0 == 2 * 10 * 32 * 4  # layer * capacity * kv_dim * 4 bytes
    torch.cuda.synchronize()


@pytest.mark.parametrize("elem", ["f16", "f32"])
def test_device_bytes_account_for_everything_the_cache_allocates(elem):
    """rv_kv_device_bytes: a fresh cache holds its planes, workspace and
    tickets, and its bound is rv_kv_projected_device_bytes of its geometry;
    prefill chunks add one staged copy per layer they touch (within the
    bound when in the bound's EXACT mode; an F16 copy is smaller), and the
    device-position step's (cos, sin) table. `now` never exceeds `bound`
    while nothing outgrows the bound's assumptions."""
    torch = torch_cuda()
    say(f"case device bytes elem={elem}")
    n_layers, n_kv, hd, cap = 3, 4, 128, 256
    kv = rv.KvCache(n_layers, n_kv, hd, cap, elem)
    now0, bound0 = kv.device_bytes()
    planes = rv.KvCache.projected_bytes(n_layers, n_kv, hd, cap, elem)
    assert bound0 == rv.KvCache.projected_device_bytes(n_layers, n_kv, hd, cap, elem)
    assert planes < now0 < bound0
    rng = Rng(0xB17E)
    rows = 64
    q = dev(rng.vec_in(rows * 32 * hd, -1, 1)).reshape(rows, 32 * hd)
    k = dev(rng.vec_in(rows * n_kv * hd, -1, 1)).reshape(rows, n_kv * hd)
    v = dev(rng.vec_in(rows * n_kv * hd, -1, 1)).reshape(rows, n_kv * hd)
    w = dev(np.ones(hd, np.float32))
    out = torch.zeros(rows, 32 * hd, device="cuda")
    # The device-position step first: it builds the cache's (cos, sin)
    # table for the capacity (the F16 chunk below reads the same table).
    pos = torch.tensor([0], dtype=torch.int32, device="cuda")
    q1 = dev(rng.vec_in(32 * hd, -1, 1))
    k1, v1 = dev(rng.vec_in(n_kv * hd, -1, 1)), dev(rng.vec_in(n_kv * hd, -1, 1))
    o1 = torch.zeros(32 * hd, device="cuda")
    rv.decode_step_dev(kv, 2, q1, k1, v1, w, w, 1e-6, 1e6, pos, cap - 1, 0.088, o1)
    torch.cuda.synchronize()
    now1, bound1 = kv.device_bytes()
    assert now1 - now0 >= cap * hd * 4 and now1 <= bound1, (now1 - now0)
    rv.prefill_chunk(kv, 0, q, k, v, w, w, 1e-6, 1e6, 0, 0.088, out, mode="exact")
    rv.prefill_chunk(kv, 1, q, k, v, w, w, 1e-6, 1e6, 0, 0.088, out, mode="f16")
    torch.cuda.synchronize()
    now2, bound2 = kv.device_bytes()
    tiles = (cap + 63) // 64
    exact_copy, f16_copy = n_kv * tiles * (4 * 16384 + 4096), n_kv * tiles * 2 * 16384
    qbuf = rows * hd * 4  # at least the chunk's (cos, sin) rows, or its prepared queries
    assert now2 - now1 >= exact_copy + f16_copy + qbuf, (now2 - now1)
    assert now2 <= bound2 and bound2 >= bound0

"""rv_decode_attention_noalloc (no reference counterpart) against
rv_decode_attention: the same kernels on the library's fixed device scratch
instead of the cache's workspace, so the outputs must agree bit for bit, on
two calls in a row (the second over fewer positions), on every decode path
(MFMA tiles, VALU subgroups, the generic head_dim path); over-size calls and
host pointers are refused with RV_ERR_UNSUPPORTED and leave out untouched.
"""
import numpy as np
import pytest

import ramvamp_amd as rv
from ramvamp_amd import _lib as L
from gpu_util import dev, host, say, torch_cuda
from helpers import Rng

pytestmark = pytest.mark.gpu

RV_ERR_UNSUPPORTED = 33

CASES = [  # (n_kv, n_q, head_dim, elem, positions of call 1, positions of call 2)
    (4, 32, 128, "f32", 3000, 700),   # MFMA tile path (config 2's geometry)
    (4, 32, 128, "f16", 9000, 33),    # MFMA tile path, f16 planes
    (2, 68, 128, "f32", 1500, 90),    # VALU subgroup path (group 34)
    (2, 8, 64, "f16", 1200, 5),       # generic path (head_dim 64)
]


@pytest.mark.parametrize("n_kv,n_q,hd,elem,p1,p2", CASES)
def test_noalloc_matches_decode_attention_bit_for_bit(n_kv, n_q, hd, elem, p1, p2):
    torch = torch_cuda()
    say(f"case noalloc {(n_kv, n_q, hd, elem, p1, p2)}")
    rng = Rng(0x0A110C + p1)
    kv = rv.KvCache(2, n_kv, hd, p1, elem)
    for layer in range(2):
        K = rng.vec_in(p1 * n_kv * hd, -1.0, 1.0).reshape(p1, -1)
        V = rng.vec_in(p1 * n_kv * hd, -1.0, 1.0).reshape(p1, -1)
        kv.append_rows(layer, K, V)
    q = dev(rng.vec_in(n_q * hd, -1.0, 1.0))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    for positions in (p1, p2):  # the second call over fewer positions
        kv.truncate(positions)
        for layer in range(2):
            want = torch.full_like(q, float("nan"))
            got = torch.full_like(q, float("nan"))
            rv.decode_attention(q, kv, layer, scale, None, want)
            rv.decode_attention_noalloc(q, kv, layer, scale, got)
            w, g = host(want), host(got)
            assert not np.any(np.isnan(w))
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (positions, layer)


def test_noalloc_refuses_oversize_calls_and_host_pointers():
    torch = torch_cuda()
    say("case noalloc refusals")
    rng = Rng(0x0A110D)
    # generic path: scores need n_q * positions * 4 bytes > the 8 MiB array
    n_kv, n_q, hd, n = 2, 64, 32, 40000
    kv = rv.KvCache(1, n_kv, hd, n, "f16")
    kv.append_rows(0, np.zeros((n, n_kv * hd), np.float32), np.zeros((n, n_kv * hd), np.float32))
    q = dev(rng.vec_in(n_q * hd, -1.0, 1.0))
    out = torch.full_like(q, float("nan"))
    with pytest.raises(rv.RamvampError) as e:
        rv.decode_attention_noalloc(q, kv, 0, 0.5, out)
    assert e.value.code == RV_ERR_UNSUPPORTED
    assert e.value.raw[1] == n_q * n * 4 and e.value.raw[2] == L.RV_NOALLOC_SCRATCH_BYTES
    assert np.all(np.isnan(host(out)))
    # host pointers (their staging would allocate)
    qh = rng.vec_in(n_q * hd, -1.0, 1.0)
    outh = np.full(qh.size, np.nan, np.float32)
    with pytest.raises(rv.RamvampError) as e:
        rv.decode_attention_noalloc(qh, kv, 0, 0.5, outh)
    assert e.value.code == RV_ERR_UNSUPPORTED
    assert np.all(np.isnan(outh))

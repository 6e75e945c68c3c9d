"""Decode calls captured into a HIP graph: every replay matches the eager
result bit for bit (the calls queue no memset and allocate nothing once the
cache's workspace exists), with eager work and synchronisations between
replays; and the kernel-timing instrumentation counts what it brackets."""
import numpy as np
import pytest

import ramvamp_amd as rv
from gpu_util import dev, host, say, torch_cuda
from helpers import Rng

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_graph_replays_match_eager(elem):
    torch = torch_cuda()
    say(f"case graph replay elem={elem}")
    rng = Rng(0x6A7F)
    n_layers, n_pos = 3, 1000
    kv = rv.KvCache(n_layers, 4, 128, n_pos, elem)
    for layer in range(n_layers):
        K = rng.vec_in(n_pos * 512, -1.0, 1.0).reshape(n_pos, -1)
        V = rng.vec_in(n_pos * 512, -1.0, 1.0).reshape(n_pos, -1)
        kv.append_rows(layer, K, V)
    q = dev(rng.vec_in(n_layers * 4096, -1.0, 1.0).reshape(n_layers, 4096))
    out = torch.zeros_like(q)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))

    def eager_ref():
        out.zero_()
        for layer in range(n_layers):
            rv.decode_attention(q[layer], kv, layer, scale, None, out[layer])
        return host(out).copy()

    want = eager_ref()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for layer in range(n_layers):
            rv.decode_attention(q[layer], kv, layer, scale, None, out[layer])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for layer in range(n_layers):
            rv.decode_attention(q[layer], kv, layer, scale, None, out[layer])
    for rep in range(5):
        out.fill_(float("nan"))
        g.replay()
        got = host(out)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
        again = eager_ref()  # eager work between replays
        assert np.array_equal(again.view(np.uint32), want.view(np.uint32)), f"eager after replay {rep}"


def test_kernel_timing_counts_bracketed_launches():
    torch = torch_cuda()
    say("case kernel timing")
    rng = Rng(0x71E)
    kv = rv.KvCache(1, 4, 128, 512, "f32")
    K = rng.vec_in(512 * 512, -1.0, 1.0).reshape(512, -1)
    kv.append_rows(0, K, K)
    q = dev(rng.vec_in(4096, -1.0, 1.0))
    out = torch.zeros_like(q)
    assert kv.kernel_time() == (0.0, 0)
    rv.decode_attention(q, kv, 0, 0.1, None, out)
    assert kv.kernel_time() == (0.0, 0)  # timing off: nothing recorded
    kv.set_tuning(7, 1)
    for _ in range(3):
        rv.decode_attention(q, kv, 0, 0.1, None, out)
    ms, n = kv.kernel_time()
    assert n == 3 and ms > 0.0, (ms, n)
    assert kv.kernel_time() == (0.0, 0)  # reset by the read
    kv.set_tuning(7, 0)


@pytest.mark.parametrize("mode", ["f16", "exact"])
def test_prefill_graph_replays_match_eager_and_leave_the_staged_copy_sound(mode):
    """Prefill keeps a staged copy of the layer's K/V across eager calls; a
    captured call stages what it reads into the workspace on every replay and
    leaves that copy alone. Replays interleaved with eager calls over a longer
    prefix (before and after the capture) match eager results bit for bit."""
    torch = torch_cuda()
    say(f"case prefill graph mode={mode}")
    rng = Rng(0x9A9F)
    n_pos = 300
    kv = rv.KvCache(1, 4, 128, 700, "f32")
    kv.append_rows(0, rng.vec_in(n_pos * 512, -1.0, 1.0).reshape(n_pos, -1),
                   rng.vec_in(n_pos * 512, -1.0, 1.0).reshape(n_pos, -1))
    q = dev(rng.vec_in(40 * 4096, -1.0, 1.0).reshape(40, 4096))
    out = torch.zeros_like(q)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))

    def eager(start):
        out.fill_(float("nan"))
        rv.attention_at_rows(q, kv, 0, start, scale, out, mode=mode)
        return host(out).copy()

    want_long = eager(260)  # stages every tile of positions 0..299
    want_short = eager(100)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        rv.attention_at_rows(q, kv, 0, 100, scale, out, mode=mode)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rv.attention_at_rows(q, kv, 0, 100, scale, out, mode=mode)
    again = eager(260)
    assert np.array_equal(again.view(np.uint32), want_long.view(np.uint32)), "eager after capture"
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        got = host(out)
        assert np.array_equal(got.view(np.uint32), want_short.view(np.uint32)), f"replay {rep}"
        again = eager(260)  # restages past the replay's zeroed rows
        assert np.array_equal(again.view(np.uint32), want_long.view(np.uint32)), f"eager after replay {rep}"


def test_a_graph_captured_early_stays_valid_as_the_context_grows():
    # The workspace is sized for the cache's capacity and never freed while
    # the cache lives: a decode graph captured at ctx 512 on a fresh cache
    # (no warm-up call) still replays correctly after eager calls at ctx
    # 8192, into a NaN-filled out, bit for bit the eager result at 512.
    torch = torch_cuda()
    say("case early capture, context grows to 8192")
    rng = Rng(0x6A80)
    cap = 8192
    kv = rv.KvCache(1, 4, 128, cap, "f32")
    K = rng.vec_in(cap * 512, -1.0, 1.0).reshape(cap, -1)
    V = rng.vec_in(cap * 512, -1.0, 1.0).reshape(cap, -1)
    kv.append_rows(0, K[:512], V[:512])
    q = dev(rng.vec_in(4096, -1.0, 1.0))
    out = torch.full_like(q, float("nan"))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rv.decode_attention(q, kv, 0, scale, None, out)
    out.fill_(float("nan"))
    rv.decode_attention(q, kv, 0, scale, None, out)
    want = host(out).copy()
    for n in (1024, 4096, 8192):
        kv.append_rows(0, K[kv.len(0):n], V[kv.len(0):n])
        eager = torch.full_like(q, float("nan"))
        rv.decode_attention(q, kv, 0, scale, None, eager)
        assert not np.any(np.isnan(host(eager))), n
        for rep in range(2):
            out.fill_(float("nan"))
            g.replay()
            got = host(out)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, rep)

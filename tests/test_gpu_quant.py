"""The quantized projections on the GPU vs the oracle (kernels/quants,
kernels/gemv.rs, model/forward.rs:2574-2646).

Bar: bit-identical. The activation quantizers produce the oracle's bytes
(d, qs, bsums); each GEMV output is the oracle's f32 bit for bit, since the
integer sub-block sums are exact and the float steps are the scalar dot's
in the same order. Inputs cover every quant/scale bit pattern (random bytes),
the reference's known answers and adversarial blocks, 2-byte-aligned blocks
(Q6_K, Q8_0), odd row counts and sub-ranges.
"""
import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import say, torch_cuda
from quant_util import Lcg, f16_bytes, random_weight_rows
from ramvamp_amd import projections as P

pytestmark = pytest.mark.gpu
F32 = np.float32
FORMATS = [oracle.RV_QF_Q4_K, oracle.RV_QF_Q5_K, oracle.RV_QF_Q6_K, oracle.RV_QF_Q8_0]


def u8(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).ravel().copy()).cuda()


def f32(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=F32).ravel().copy()).cuda()


def gpu_quantize(torch, fmt, x):
    xd = f32(torch, x)
    if fmt == oracle.RV_QF_Q8_K:
        out = P.q8_k_buffer(x.size // 256)
        P.quantize_row_q8_k(xd, out)
        return out.cpu().numpy().view(oracle.BLOCK_Q8_K)
    out = P.q8_0_buffer(x.size // 32)
    P.quantize_row_q8_0(xd, out)
    return out.cpu().numpy().view(oracle.BLOCK_Q8_0)


def special_rows(n):
    """Rows that stress the quantizers: ties of magnitude with both signs,
    zero blocks, one huge value, tiny values, exact halves."""
    rows = []
    x = np.zeros(n, F32)
    x[3], x[7] = -2.0, 2.0  # first of equal magnitudes wins
    rows.append(x)
    x = np.zeros(n, F32)
    x[100 % n] = 1e30
    x[5] = 1e-30
    rows.append(x)
    x = np.zeros(n, F32)
    x[0], x[1] = 4.0, -2.0  # 63.5: ties to even / away from zero
    x[31] = 0.5
    rows.append(x)
    rows.append(np.zeros(n, F32))
    rows.append((np.arange(n, dtype=F32) - n / 2) / F32(7.0))
    return rows


@pytest.mark.parametrize("fmt", [oracle.RV_QF_Q8_K, oracle.RV_QF_Q8_0])
def test_quantizers_are_bit_identical(fmt):
    torch = torch_cuda()
    rng = np.random.default_rng(0x51 + fmt)
    quant = oracle.quantize_row_q8_k if fmt == oracle.RV_QF_Q8_K else oracle.quantize_row_q8_0
    cases = special_rows(2048) + [rng.standard_normal(4096).astype(F32) * s for s in (1e-3, 1.0, 300.0)]
    cases.append(Lcg(0xB5).f32s(256 * 7, 5.0))
    for x in cases:
        say(f"case quantize fmt={fmt} n={x.size}")
        got, want = gpu_quantize(torch, fmt, x), quant(x)
        assert got.tobytes() == want.tobytes()


def test_quantizer_known_answers_on_the_gpu():
    """quantize.rs:112-184, through the device path."""
    torch = torch_cuda()
    x = np.zeros(32, F32)
    x[0], x[1], x[31] = 2.0, -1.0, 0.5
    b = gpu_quantize(torch, oracle.RV_QF_Q8_0, x)[0]
    assert (b["qs"][0], b["qs"][1], b["qs"][31]) == (127, -64, 32)
    assert b["d"] == oracle.f16_to_f32(oracle.f32_to_f16(F32(2.0) / F32(127.0)))[0]
    x = np.zeros(256, F32)
    x[10], x[20] = -3.0, 1.5
    b = gpu_quantize(torch, oracle.RV_QF_Q8_K, x)[0]
    assert b["qs"][10] == -127 and b["qs"][20] == 64 and b["d"] == F32(1.0) / (F32(-127.0) / F32(-3.0))
    z = gpu_quantize(torch, oracle.RV_QF_Q8_K, np.zeros(512, F32))
    assert (z.view(np.uint8) == 0).all()


def run_gemv(torch, fmt, w, in_dim, out_dim, acts, rows=None, offset=0):
    """The device GEMV over rows (default all); the weight matrix placed
    `offset` bytes into its buffer."""
    lo, hi = (0, out_dim) if rows is None else rows
    buf = torch.zeros(w.size + offset, dtype=torch.uint8, device="cuda")
    buf[offset:] = u8(torch, w)
    wd = buf[offset:]
    ad = u8(torch, acts)
    out = torch.full((hi - lo,), float("nan"), device="cuda")
    if fmt == oracle.RV_QF_Q8_0:
        P.gemv_q8_0_rows(wd, in_dim, out_dim, ad, (lo, hi), out)
    else:
        P.gemv_q8_k_rows(fmt, wd, in_dim, out_dim, ad, (lo, hi), out)
    return out.cpu().numpy()


@pytest.mark.parametrize("fmt", FORMATS)
def test_gemv_is_bit_identical_to_the_scalar_reference(fmt):
    torch = torch_cuda()
    rng = np.random.default_rng(0x6E0 + fmt)
    shapes = [(256, 5), (768, 7), (2048, 33), (4096, 9), (2304, 3)]
    if fmt == oracle.RV_QF_Q8_0:
        shapes += [(32, 3), (96, 5), (4128, 2)]  # odd block counts, > 64 blocks per pass
    for in_dim, out_dim in shapes:
        say(f"case gemv fmt={fmt} in={in_dim} out={out_dim}")
        w = random_weight_rows(fmt, out_dim, in_dim, rng)
        x = rng.standard_normal(in_dim).astype(F32)
        acts = oracle.quantize_row_q8_0(x) if fmt == oracle.RV_QF_Q8_0 else oracle.quantize_row_q8_k(x)
        want = oracle.gemv(fmt, w, in_dim, out_dim, acts)
        got = run_gemv(torch, fmt, w, in_dim, out_dim, acts)
        assert got.tobytes() == want.tobytes(), np.abs(got - want).max()
        lo, hi = 1, out_dim - 1
        got = run_gemv(torch, fmt, w, in_dim, out_dim, acts, rows=(lo, hi), offset=4)
        assert got.tobytes() == want[lo:hi].tobytes()


def test_gemv_reference_adversarial_blocks():
    """quants/tests.rs:231-346 blocks (maxed scales, all-min, zero d, extreme
    Q8_0), plus zero activations, bit for bit."""
    torch = torch_cuda()
    all_min = bytes([0, 0, 0, 0, 0xFF, 0xFF, 0xFF, 0xFF, 0xF0, 0xF0, 0xF0, 0xF0])
    q4 = [f16_bytes(1.0) + f16_bytes(0.5) + bytes([0xFF] * 12) + bytes([0xFF] * 128),
          f16_bytes(4.0) + f16_bytes(2.0) + bytes(12) + bytes([0x5A] * 128),
          f16_bytes(0.0) + f16_bytes(0.0) + bytes([0x3F] * 12) + bytes([0xFF] * 128),
          f16_bytes(1.0) + f16_bytes(0.5) + all_min + bytes(128)]
    q5 = [f16_bytes(1.0) + f16_bytes(0.5) + bytes([0xFF] * 12) + bytes([0xFF] * 32) + bytes([0xFF] * 128),
          f16_bytes(1.0) + f16_bytes(0.5) + bytes([0xFF] * 12) + bytes(32) + bytes([0xFF] * 128),
          f16_bytes(1.0) + f16_bytes(0.5) + all_min + bytes([0xAA] * 32) + bytes(128)]
    q6 = [bytes([0xFF] * 128) + bytes([0xFF] * 64) + bytes([0x80] * 16) + f16_bytes(1.0),
          bytes([0xFF] * 192) + bytes([127] * 16) + f16_bytes(0.25),
          bytes(192) + bytes([127] * 16) + f16_bytes(1.0)]
    acts = oracle.quantize_row_q8_k(Lcg(0xD4).f32s(256, 2.0))
    for fmt, blocks in ((oracle.RV_QF_Q4_K, q4), (oracle.RV_QF_Q5_K, q5), (oracle.RV_QF_Q6_K, q6)):
        w = np.frombuffer(b"".join(blocks), np.uint8).reshape(len(blocks), -1)
        for a in (acts, np.zeros(1, oracle.BLOCK_Q8_K)):
            want = oracle.gemv(fmt, w, 256, len(blocks), a)
            assert run_gemv(torch, fmt, w, 256, len(blocks), a).tobytes() == want.tobytes()
    w = np.frombuffer((0x7BFF).to_bytes(2, "little") + bytes([0x80] * 32), np.uint8).reshape(1, -1)
    a = np.zeros(1, oracle.BLOCK_Q8_0)
    a["d"], a["qs"] = 65504.0, 127
    assert run_gemv(torch, oracle.RV_QF_Q8_0, w, 32, 1, a).tobytes() == oracle.gemv(oracle.RV_QF_Q8_0, w, 32, 1,
                                                                                    a).tobytes()


def test_attention_projections_match_the_separate_calls():
    """forward.rs:2574-2646 at the model's shapes (hidden 2048, q_dim 4096,
    kv_dim 512): Q4_K q, Q8_0 k, Q6_K (and Q4_K) v, Q5_K o."""
    torch = torch_cuda()
    rng = np.random.default_rng(0xA77)
    hidden, q_dim, kv_dim = 2048, 4096, 512
    x = rng.standard_normal(hidden).astype(F32)
    a = rng.standard_normal(q_dim).astype(F32)
    wq = random_weight_rows(oracle.RV_QF_Q4_K, q_dim, hidden, rng)
    wk = random_weight_rows(oracle.RV_QF_Q8_0, kv_dim, hidden, rng)
    wo = random_weight_rows(oracle.RV_QF_Q5_K, hidden, q_dim, rng)
    acts_k, acts_0 = oracle.quantize_row_q8_k(x), oracle.quantize_row_q8_0(x)
    for v_fmt in (oracle.RV_QF_Q6_K, oracle.RV_QF_Q4_K):
        say(f"case attn_in_proj v_fmt={v_fmt}")
        wv = random_weight_rows(v_fmt, kv_dim, hidden, rng)
        q = torch.full((q_dim,), float("nan"), device="cuda")
        k = torch.full((kv_dim,), float("nan"), device="cuda")
        v = torch.full((kv_dim,), float("nan"), device="cuda")
        P.attn_in_proj(f32(torch, x), oracle.RV_QF_Q4_K, u8(torch, wq), q, u8(torch, wk), k, v_fmt, u8(torch, wv), v)
        assert q.cpu().numpy().tobytes() == oracle.gemv(oracle.RV_QF_Q4_K, wq, hidden, q_dim, acts_k).tobytes()
        assert k.cpu().numpy().tobytes() == oracle.gemv(oracle.RV_QF_Q8_0, wk, hidden, kv_dim, acts_0).tobytes()
        assert v.cpu().numpy().tobytes() == oracle.gemv(v_fmt, wv, hidden, kv_dim, acts_k).tobytes()
    o = torch.full((hidden,), float("nan"), device="cuda")
    P.attn_out_proj(f32(torch, a), oracle.RV_QF_Q5_K, u8(torch, wo), o)
    want = oracle.gemv(oracle.RV_QF_Q5_K, wo, q_dim, hidden, oracle.quantize_row_q8_k(a))
    assert o.cpu().numpy().tobytes() == want.tobytes()


def test_gemv_errors_match_the_oracle_and_write_nothing():
    """gemv.rs `validate` order and payloads, host-checked before any launch."""
    torch = torch_cuda()
    w = torch.zeros(4 * 1152, dtype=torch.uint8, device="cuda")
    acts = P.q8_k_buffer(8)
    out = torch.full((4,), 7.0, device="cuda")
    cases = [dict(fmt=oracle.RV_QF_Q8_0), dict(in_dim=100), dict(wlen=w.numel() - 1), dict(rows=(3, 2)),
             dict(rows=(0, 5)), dict(olen=3), dict(nacts=7)]
    L = rv._lib.load()
    host_w = np.zeros(4 * 1152, np.uint8)
    for c in cases:
        fmt, in_dim = c.get("fmt", oracle.RV_QF_Q4_K), c.get("in_dim", 2048)
        lo, hi = c.get("rows", (0, 4))
        wlen, olen, nacts = c.get("wlen", w.numel()), c.get("olen", 4), c.get("nacts", 8)
        err = rv._lib.RvError()
        rc = L.rv_gemv_q8_k_rows(fmt, w.data_ptr(), wlen, in_dim, 4, acts.data_ptr(), nacts, lo, hi, out.data_ptr(),
                                 olen, None, 0, err)
        oerr = oracle.RvError()
        orc = oracle.lib().rvo_gemv_q8_k(fmt, host_w.ctypes.data, wlen, in_dim, 4, None, nacts, 1, lo, hi, None, olen,
                                         oracle.byref(oerr))
        assert rc == orc != 0, c
        assert (err.a, err.b, err.c) == (oerr.a, oerr.b, oerr.c), c
        if err.what or oerr.what:
            assert err.what.decode().split(":")[0].startswith(oerr.what.decode().split(":")[0][:4]), c
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()
    with pytest.raises(rv.KernelError) as e:
        P.gemv_q8_k(oracle.RV_QF_Q4_K, w, 2048, 4, P.q8_k_buffer(7), out)
    assert e.value.variant == "BlockCountMismatch"
    with pytest.raises(rv.KernelError) as e:
        P.quantize_row_q8_k(torch.zeros(100, device="cuda"), P.q8_k_buffer(1))
    assert e.value.variant == "QuantizeLenMismatch" and e.value.fields["floats"] == 100


def test_projections_quantize_in_the_wave_like_the_quantizers():
    """The fused projections quantize each activation block inside the GEMV
    wave; on rows built to stress the quantizers (a zero block, magnitude
    ties of both signs in different lanes, one huge value, exact halves) the
    outputs stay bit-identical to the oracle's quantize-then-GEMV."""
    torch = torch_cuda()
    rng = np.random.default_rng(0xF0)
    hidden, q_dim, kv_dim = 1024, 256, 64
    x = rng.standard_normal(hidden).astype(F32)
    x[0:256] = 0.0                      # a zero Q8_K block (and eight zero Q8_0 blocks)
    x[256 + 3], x[256 + 200] = -2.5, 2.5  # tie across lanes: the first (negative) one anchors
    x[256 + 100] = 2.5
    x[512:768] = np.round(x[512:768] * 2) / 2  # exact halves
    x[800] = 3e4
    wq = random_weight_rows(oracle.RV_QF_Q4_K, q_dim, hidden, rng)
    wk = random_weight_rows(oracle.RV_QF_Q8_0, kv_dim, hidden, rng)
    wv = random_weight_rows(oracle.RV_QF_Q6_K, kv_dim, hidden, rng)
    wo = random_weight_rows(oracle.RV_QF_Q5_K, kv_dim, hidden, rng)
    acts_k, acts_0 = oracle.quantize_row_q8_k(x), oracle.quantize_row_q8_0(x)
    q = torch.empty(q_dim, device="cuda")
    k = torch.empty(kv_dim, device="cuda")
    v = torch.empty(kv_dim, device="cuda")
    P.attn_in_proj(f32(torch, x), oracle.RV_QF_Q4_K, u8(torch, wq), q, u8(torch, wk), k, oracle.RV_QF_Q6_K,
                   u8(torch, wv), v)
    assert q.cpu().numpy().tobytes() == oracle.gemv(oracle.RV_QF_Q4_K, wq, hidden, q_dim, acts_k).tobytes()
    assert k.cpu().numpy().tobytes() == oracle.gemv(oracle.RV_QF_Q8_0, wk, hidden, kv_dim, acts_0).tobytes()
    assert v.cpu().numpy().tobytes() == oracle.gemv(oracle.RV_QF_Q6_K, wv, hidden, kv_dim, acts_k).tobytes()
    o = torch.empty(kv_dim, device="cuda")
    P.attn_out_proj(f32(torch, x), oracle.RV_QF_Q5_K, u8(torch, wo), o)
    assert o.cpu().numpy().tobytes() == oracle.gemv(oracle.RV_QF_Q5_K, wo, hidden, kv_dim, acts_k).tobytes()

"""GPU parity of the batched GEMVs (gemv.rs:444-478 `gemv_q8_k_batched`,
:616-651 `gemv_q8_0_batched`): every output bit-identical to the oracle's
scalar dot of that weight row and activation row, over ragged row ranges
and activation counts (partial 32-row and 32-activation tiles), the model's
prefill shapes (512 activation rows), and the reference's adversarial blocks
(maxed and negative scales, where the folded int8 planes reach their
extremes), plus the validation order of the batched forms."""
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


def dev_u8(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).ravel().copy()).cuda()


def quantize_rows(fmt, x):
    q = oracle.quantize_row_q8_0 if fmt == oracle.RV_QF_Q8_0 else oracle.quantize_row_q8_k
    return np.concatenate([q(r) for r in x])


def run_batched(torch, fmt, w, in_dim, out_dim, acts, n_acts, rows):
    lo, hi = rows
    out = torch.full(((hi - lo) * n_acts,), float("nan"), device="cuda")
    wd, ad = dev_u8(torch, w), dev_u8(torch, acts)
    if fmt == oracle.RV_QF_Q8_0:
        P.gemv_q8_0_batched(wd, in_dim, out_dim, ad, n_acts, rows, out)
    else:
        P.gemv_q8_k_batched(fmt, wd, in_dim, out_dim, ad, n_acts, rows, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(torch, fmt, w, in_dim, out_dim, acts, n_acts, rows=None):
    rows = rows or (0, out_dim)
    want = oracle.gemv(fmt, w, in_dim, out_dim, acts, n_acts=n_acts, rows=rows)
    got = run_batched(torch, fmt, w, in_dim, out_dim, acts, n_acts, rows)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (f"fmt {fmt}: {bad.size} of {want.size} differ, first at {bad[0]}: "
                           f"{got[bad[0]]!r} vs {want[bad[0]]!r}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_batched_gemv_is_bit_identical_to_the_scalar_dots(fmt):
    torch = torch_cuda()
    rng = np.random.default_rng(0xBA7 + fmt)
    # (out_dim, in_dim, n_acts, rows): partial row and activation tiles, one
    # activation, more activations than one workgroup covers, row windows.
    cases = [(64, 512, 33, None), (100, 1024, 1, (3, 97)), (72, 256, 257, (5, 70)), (40, 2048, 70, None),
             (33, 768, 130, (1, 33))]
    if fmt == oracle.RV_QF_Q8_0:
        cases += [(35, 32, 9, None), (64, 288, 40, None)]  # 1 and 9 blocks: partial groups of eight
    for out_dim, in_dim, n_acts, rows in cases:
        say(f"case batched fmt={fmt} out={out_dim} in={in_dim} n_acts={n_acts} rows={rows}")
        w = random_weight_rows(fmt, out_dim, in_dim, rng)
        acts = quantize_rows(fmt, rng.standard_normal((n_acts, in_dim)).astype(F32))
        check(torch, fmt, w, in_dim, out_dim, acts, n_acts, rows)


@pytest.mark.parametrize("fmt,out_dim,in_dim", [(oracle.RV_QF_Q4_K, 4096, 2048), (oracle.RV_QF_Q8_0, 512, 2048),
                                                (oracle.RV_QF_Q6_K, 512, 2048), (oracle.RV_QF_Q5_K, 2048, 4096)])
def test_batched_gemv_at_the_prefill_shapes(fmt, out_dim, in_dim):
    # prefill.rs:1999-2053: a 512-row chunk's q (Q4_K), k (Q8_0), v (Q6_K)
    # and o (Q5_K) projections.
    torch = torch_cuda()
    say(f"case batched prefill shape fmt={fmt} {out_dim}x{in_dim} x 512")
    rng = np.random.default_rng(0x512 + fmt)
    w = random_weight_rows(fmt, out_dim, in_dim, rng)
    acts = quantize_rows(fmt, rng.standard_normal((512, in_dim)).astype(F32))
    # The whole matrix on the GPU (every workgroup of the full grid); the
    # oracle checks three 64-row windows of it (the full scalar product
    # takes it 10-15 s).
    got = run_batched(torch, fmt, w, in_dim, out_dim, acts, 512, (0, out_dim)).reshape(out_dim, 512)
    for lo in (0, out_dim // 2 - 32, out_dim - 64):
        want = oracle.gemv(fmt, w, in_dim, out_dim, acts, n_acts=512, rows=(lo, lo + 64)).reshape(64, 512)
        assert got[lo:lo + 64].tobytes() == want.tobytes(), f"rows {lo}..{lo + 64}"


def test_batched_gemv_reference_adversarial_blocks():
    """quants/tests.rs:231-346 blocks (maxed scales, all-min, zero d, signed
    Q6_K scales at -128 and 127) against 40 random and one zero activation
    row: the folded int8 planes at their extremes."""
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
    lcg = Lcg(0xD5)
    rows = [lcg.f32s(512, 2.0) for _ in range(40)] + [np.zeros(512, F32)]
    acts = quantize_rows(oracle.RV_QF_Q4_K, rows)
    for fmt, blocks in ((oracle.RV_QF_Q4_K, q4), (oracle.RV_QF_Q5_K, q5), (oracle.RV_QF_Q6_K, q6)):
        # Two blocks per row (in_dim 512): each block paired with every other.
        pairs = [a + b for a in blocks for b in blocks]
        w = np.frombuffer(b"".join(pairs), np.uint8).reshape(len(pairs), -1)
        say(f"case batched adversarial fmt={fmt} rows={len(pairs)}")
        check(torch, fmt, w, 512, len(pairs), acts, len(rows))
    w = np.frombuffer(((0x7BFF).to_bytes(2, "little") + bytes([0x80] * 32)) * 2, np.uint8).reshape(1, -1)
    a = np.zeros(6, oracle.BLOCK_Q8_0)
    a["d"], a["qs"] = 65504.0, 127
    check(torch, oracle.RV_QF_Q8_0, w, 64, 1, a, 3)


def test_batched_gemv_validation_order():
    torch = torch_cuda()
    rng = np.random.default_rng(7)
    w = dev_u8(torch, random_weight_rows(oracle.RV_QF_Q4_K, 8, 256, rng))
    acts = dev_u8(torch, quantize_rows(oracle.RV_QF_Q4_K, rng.standard_normal((3, 256)).astype(F32)))
    out = torch.zeros(8 * 3, device="cuda")

    def raises(variant, fn, what=None):
        with pytest.raises(rv.RamvampError) as ei:
            fn()
        assert ei.value.variant == variant, ei.value
        if what:
            assert what in ei.value.what, ei.value

    raises("UnsupportedFormat", lambda: P.gemv_q8_k_batched(oracle.RV_QF_Q8_0, w, 256, 8, acts, 3, (0, 8), out))
    raises("LengthMismatch", lambda: P.gemv_q8_k_batched(oracle.RV_QF_Q4_K, w, 256, 9, acts, 3, (0, 9), out),
           "x n_acts")
    raises("LengthMismatch", lambda: P.gemv_q8_k_batched(oracle.RV_QF_Q4_K, w, 256, 8, acts, 3, (0, 7), out),
           "x n_acts")
    raises("BlockCountMismatch", lambda: P.gemv_q8_k_batched(oracle.RV_QF_Q4_K, w, 256, 8, acts, 4, (0, 6), out))
    raises("LengthMismatch", lambda: P.gemv_q8_k_batched(oracle.RV_QF_Q4_K, w, 256, 8, acts, 3, (5, 4), out),
           "row range")
    assert np.all(out.cpu().numpy() == 0)  # nothing written on error
    # Empty ranges and no activations are valid and write nothing.
    empty = torch.zeros(0, device="cuda")
    P.gemv_q8_k_batched(oracle.RV_QF_Q4_K, w, 256, 8, acts[:0], 0, (0, 8), empty)
    P.gemv_q8_k_batched(oracle.RV_QF_Q4_K, w, 256, 8, acts, 3, (4, 4), empty)
    torch.cuda.synchronize()


@pytest.mark.parametrize("n", [1, 37, 130])
def test_prefill_chunk_projections_match_the_single_row_gemvs(n):
    """prefill.rs:1985-2053 and :2113-2154 at the model's shapes: each row of
    q/k/v equals the single-row GEMV of that row's quantized normed input,
    and each residual row gains exactly its o row (one f32 add)."""
    torch = torch_cuda()
    rng = np.random.default_rng(0xC4 + n)
    hidden, q_dim, kv_dim = 2048, 4096, 512
    Q = oracle
    wq = random_weight_rows(Q.RV_QF_Q4_K, q_dim, hidden, rng)
    wk = random_weight_rows(Q.RV_QF_Q8_0, kv_dim, hidden, rng)
    wv = random_weight_rows(Q.RV_QF_Q6_K, kv_dim, hidden, rng)
    wo = random_weight_rows(Q.RV_QF_Q5_K, hidden, q_dim, rng)
    x = rng.standard_normal((n, hidden)).astype(F32)
    attn = rng.standard_normal((n, q_dim)).astype(F32)
    res = rng.standard_normal((n, hidden)).astype(F32)
    say(f"case prefill chunk projections n={n}")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    q, k, v = (torch.full((n, m), float("nan"), device="cuda") for m in (q_dim, kv_dim, kv_dim))
    P.attn_in_proj_rows(d(x), Q.RV_QF_Q4_K, dev_u8(torch, wq), q, dev_u8(torch, wk), k, Q.RV_QF_Q6_K,
                        dev_u8(torch, wv), v)
    r_dev = d(res)
    P.attn_out_proj_rows(d(attn), Q.RV_QF_Q5_K, dev_u8(torch, wo), r_dev)
    torch.cuda.synchronize()
    q, k, v, r_got = (t.cpu().numpy() for t in (q, k, v, r_dev))
    for r in range(n):
        ak, a0 = oracle.quantize_row_q8_k(x[r]), oracle.quantize_row_q8_0(x[r])
        assert q[r].tobytes() == oracle.gemv(Q.RV_QF_Q4_K, wq, hidden, q_dim, ak).tobytes(), f"q row {r}"
        assert k[r].tobytes() == oracle.gemv(Q.RV_QF_Q8_0, wk, hidden, kv_dim, a0).tobytes(), f"k row {r}"
        assert v[r].tobytes() == oracle.gemv(Q.RV_QF_Q6_K, wv, hidden, kv_dim, ak).tobytes(), f"v row {r}"
        o = oracle.gemv(Q.RV_QF_Q5_K, wo, q_dim, hidden, oracle.quantize_row_q8_k(attn[r]))
        assert r_got[r].tobytes() == (res[r] + o).astype(F32).tobytes(), f"residual row {r}"

"""GPU parity of one layer's attention block (include/ramvamp_block.h) against
the oracle's composition of the same steps (model/forward.rs:2570-2650):
rmsnorm -> Q8_K/Q8_0 quantize -> q/k/v GEMVs -> decode_step (QK norm, RoPE,
append, attention) -> quantize attn_out -> o GEMV -> residual add.

What each intermediate is held to: the q/k/v projections (read back from the
call's scratch) bit-identical to the oracle's GEMVs on the oracle's
normalized row; the attention output to the fp32 gate; the updated residual
to 2e-3 of max|o|, since a one-step change in one quantized attn_out value
(the attention is exact only to a tolerance) moves o by one quantum of that
block. Weights are random k-quant rows (quant_util); the cache holds random
rows before the tokens run.
"""
import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import FP32_FLOOR, FP32_REL, elem_code, gate, say, torch_cuda
from helpers import Rng
from quant_util import random_weight_rows
from ramvamp_amd import block as B

pytestmark = pytest.mark.gpu

EPS, THETA = 1e-6, 1e6


class Layer:
    """One layer's weights, host bytes and device tensors."""

    def __init__(self, torch, rng, hidden, q_dim, kv_dim, hd, q_fmt, v_fmt, o_fmt):
        self.hidden, self.q_dim, self.kv_dim = hidden, q_dim, kv_dim
        self.q_fmt, self.v_fmt, self.o_fmt = q_fmt, v_fmt, o_fmt
        self.attn_norm = (1.0 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
        self.q_norm = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        self.k_norm = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        self.wq = random_weight_rows(q_fmt, q_dim, hidden, rng)
        self.wk = random_weight_rows(oracle.RV_QF_Q8_0, kv_dim, hidden, rng)
        self.wv = random_weight_rows(v_fmt, kv_dim, hidden, rng)
        self.wo = random_weight_rows(o_fmt, hidden, q_dim, rng)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a).ravel()).cuda()
        self.dev = B.AttnBlockWeights(d(self.attn_norm), q_fmt, d(self.wq), d(self.wk), v_fmt, d(self.wv),
                                      d(self.q_norm), d(self.k_norm), o_fmt, d(self.wo))

    def oracle_step(self, ref, layer, residual, position, scale):
        normed = oracle.rmsnorm(residual, self.attn_norm, EPS)
        acts_k, acts_0 = oracle.quantize_row_q8_k(normed), oracle.quantize_row_q8_0(normed)
        q = oracle.gemv(self.q_fmt, self.wq, self.hidden, self.q_dim, acts_k)
        k = oracle.gemv(oracle.RV_QF_Q8_0, self.wk, self.hidden, self.kv_dim, acts_0)
        v = oracle.gemv(self.v_fmt, self.wv, self.hidden, self.kv_dim, acts_k)
        attn = ref.decode_step(layer, q, k, v, self.q_norm, self.k_norm, EPS, THETA, position, scale)
        o = oracle.gemv(self.o_fmt, self.wo, self.q_dim, self.hidden, oracle.quantize_row_q8_k(attn))
        return (q, k, v), attn, o, (residual + o).astype(np.float32)


def twin(rng, n_layers, n_kv, hd, n_pos, cap, elem):
    kv = rv.KvCache(n_layers, n_kv, hd, cap, elem)
    ref = oracle.KvCache(n_layers, n_kv, hd, cap, elem_code(elem))
    for layer in range(n_layers):
        K = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        V = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        kv.append_rows(layer, K, V)
        ref.append_rows(layer, K, V)
    return kv, ref


def run_tokens(torch, case, n_heads, n_kv, hidden, fmts, elem, n_pos, n_tok, seed):
    hd = 128
    q_dim, kv_dim = n_heads * hd, n_kv * hd
    rng = np.random.default_rng(seed)
    lay = Layer(torch, rng, hidden, q_dim, kv_dim, hd, *fmts)
    kv, ref = twin(Rng(seed), 2, n_kv, hd, n_pos, n_pos + n_tok, elem)
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    residual = (1.5 * rng.standard_normal(hidden)).astype(np.float32)
    res_dev = torch.from_numpy(residual.copy()).cuda()
    nbytes = B.scratch_bytes(hidden, q_dim, kv_dim)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    f16 = elem == "f16"
    for t in range(n_tok):
        pos = n_pos + t
        say(f"case {case} token {t} position {pos}")
        B.attn_block_decode(kv, 1, res_dev, q_dim, lay.dev, EPS, THETA, pos, scale, scratch=scratch)
        torch.cuda.synchronize()
        (q, k, v), attn, o, want = lay.oracle_step(ref, 1, residual, pos, scale)
        sc = scratch.cpu().numpy()
        off = lambda n: (n * 4 + 255) // 256 * 256
        got_q = sc[:q_dim * 4].view(np.float32)
        got_k = sc[off(q_dim):off(q_dim) + kv_dim * 4].view(np.float32)
        got_v = sc[off(q_dim) + off(kv_dim):off(q_dim) + off(kv_dim) + kv_dim * 4].view(np.float32)
        a0 = off(q_dim) + 2 * off(kv_dim)
        got_attn = sc[a0:a0 + q_dim * 4].view(np.float32)
        assert got_q.tobytes() == q.tobytes(), f"{case}: q projection"
        assert got_k.tobytes() == k.tobytes(), f"{case}: k projection"
        assert got_v.tobytes() == v.tobytes(), f"{case}: v projection"
        gate(got_attn, attn, rel=1e-3 if f16 else FP32_REL, abs_tol=1.5e-3 if f16 else FP32_FLOOR,
             what=f"{case} attention")
        got = res_dev.cpu().numpy()
        err = np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(o))
        same = int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
        say(f"{case} token {t}: residual max|err|/max|o| {err:.2e}, {same}/{hidden} bit-identical")
        assert err <= 2e-3, f"{case}: residual"
        assert kv.len(1) == pos + 1 and kv.len(0) == n_pos
        residual = want  # the next token starts from the oracle's residual
        res_dev.copy_(torch.from_numpy(residual.copy()))


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_attn_block_matches_the_oracle_composition(elem):
    torch = torch_cuda()
    Q = oracle
    run_tokens(torch, f"model block {elem}", 32, 4, 2048, (Q.RV_QF_Q4_K, Q.RV_QF_Q6_K, Q.RV_QF_Q5_K), elem, 300, 3,
               0xB10C)


def test_attn_block_other_formats_and_geometry():
    # v as Q4_K and o as Q6_K (both appear in the v0 model), 16 q heads over 2 kv heads.
    torch = torch_cuda()
    Q = oracle
    run_tokens(torch, "formats", 16, 2, 1024, (Q.RV_QF_Q5_K, Q.RV_QF_Q4_K, Q.RV_QF_Q6_K), "f32", 65, 2, 0xB10D)


def test_attn_block_wide_rows_take_the_unfused_path():
    # hidden 8448 and q_dim 9216 exceed the 8192-value in-LDS quantization, so
    # the norm, the quantizers and the residual add run as kernels of their
    # own; group 18 takes the VALU decode kernel.
    torch = torch_cuda()
    Q = oracle
    run_tokens(torch, "wide", 72, 4, 8448, (Q.RV_QF_Q4_K, Q.RV_QF_Q6_K, Q.RV_QF_Q5_K), "f32", 40, 2, 0xB10E)


def test_attn_block_errors_leave_residual_and_cache_untouched():
    torch = torch_cuda()
    Q = oracle
    rng = np.random.default_rng(0xE77)
    hidden, n_heads, n_kv, hd = 512, 8, 2, 128
    q_dim, kv_dim = n_heads * hd, n_kv * hd
    lay = Layer(torch, rng, hidden, q_dim, kv_dim, hd, Q.RV_QF_Q4_K, Q.RV_QF_Q6_K, Q.RV_QF_Q5_K)
    kv, _ = twin(Rng(3), 2, n_kv, hd, 4, 5, "f32")
    res = torch.from_numpy(rng.standard_normal(hidden).astype(np.float32)).cuda()
    before = res.cpu().numpy().copy()
    w = lay.dev

    def expect(variant, what=None, **kw):
        args = dict(cache=kv, layer=1, residual=res, q_dim=q_dim, w=w, position=4)
        args.update(kw)
        with pytest.raises(rv.RamvampError) as ei:
            B.attn_block_decode(args["cache"], args["layer"], args["residual"], args["q_dim"], args["w"], EPS, THETA,
                                args["position"], 0.1, scratch=kw.get("scratch"))
        assert ei.value.variant == variant, (variant, ei.value)
        if what:
            assert what in (ei.value.what or ""), ei.value
        torch.cuda.synchronize()
        assert np.array_equal(res.cpu().numpy(), before)
        assert kv.len(1) == 4 and kv.len(0) == 4

    empty = torch.empty(0, dtype=torch.float32, device="cuda")
    expect("Empty", "rmsnorm", residual=empty)
    short_wq = B.AttnBlockWeights(w.attn_norm, w.q_format, w.wq[:-144], w.wk, w.v_format, w.wv, w.q_norm, w.k_norm,
                                  w.o_format, w.wo)
    expect("LengthMismatch", "attn_in_proj q", w=short_wq)
    bad_v = B.AttnBlockWeights(w.attn_norm, w.q_format, w.wq, w.wk, Q.RV_QF_Q8_0, w.wv, w.q_norm, w.k_norm,
                               w.o_format, w.wo)
    expect("UnsupportedFormat", w=bad_v)
    # q_dim off by one fails the q projection's length check first (the
    # reference validates each GEMV before attention sees q) ...
    expect("LengthMismatch", "attn_in_proj q", q_dim=q_dim - 1)
    # ... and with weights of that many rows, attention's q-length checks.
    rb = hidden // 256 * 144

    def rows_of(n):
        return B.AttnBlockWeights(w.attn_norm, w.q_format, w.wq[:n * rb], w.wk, w.v_format, w.wv, w.q_norm,
                                  w.k_norm, w.o_format, w.wo)

    expect("QLenIndivisible", q_dim=1000, w=rows_of(1000))
    expect("GqaGroupMismatch", q_dim=384, w=rows_of(384))
    expect("LayerOutOfRange", layer=2)
    short_wo = B.AttnBlockWeights(w.attn_norm, w.q_format, w.wq, w.wk, w.v_format, w.wv, w.q_norm, w.k_norm,
                                  w.o_format, w.wo[:-176])
    expect("LengthMismatch", "attn_out_proj", w=short_wo)
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    expect("LengthMismatch", "attn_block scratch", scratch=small)
    # A full layer: capacity 5 holds 4 rows and this token; a second token fails.
    B.attn_block_decode(kv, 1, res, q_dim, w, EPS, THETA, 4, 0.1)
    torch.cuda.synchronize()
    before = res.cpu().numpy().copy()
    with pytest.raises(rv.KvError) as ei:
        B.attn_block_decode(kv, 1, res, q_dim, w, EPS, THETA, 5, 0.1)
    assert ei.value.variant == "CapacityExceeded"
    assert np.array_equal(res.cpu().numpy(), before) and kv.len(1) == 5


@pytest.mark.parametrize("mode,tol", [("exact", 2e-3), ("f16", 1e-2)])
def test_attn_block_prefill_matches_the_oracle_composition(mode, tol):
    """prefill.rs:1975-2154 for a 37-row chunk after 40 cached rows, then a
    second chunk: per-row rmsnorm, quantizations, batched q/k/v (bit-identical
    to the oracle's GEMVs on the oracle's normalized rows), the chunk's
    attention (EXACT: fp32-equivalent; F16: f16 MFMA inputs) and the batched
    o projection added into the residual rows. The residual is held to tol of
    max|o| (one quantum of a quantized attention value moves o by one step)."""
    torch = torch_cuda()
    Q = oracle
    rng = np.random.default_rng(0xB10F)
    hidden, n_heads, n_kv, hd = 2048, 32, 4, 128
    q_dim, kv_dim = n_heads * hd, n_kv * hd
    lay = Layer(torch, rng, hidden, q_dim, kv_dim, hd, Q.RV_QF_Q4_K, Q.RV_QF_Q6_K, Q.RV_QF_Q5_K)
    n_pos, n = 40, 37
    kv, ref = twin(Rng(0xB1), 2, n_kv, hd, n_pos, n_pos + 2 * n, "f32")
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    start = n_pos
    for chunk in range(2):
        say(f"case prefill block mode={mode} chunk {chunk} start {start}")
        res = (1.5 * rng.standard_normal((n, hidden))).astype(np.float32)
        res_dev = torch.from_numpy(res.copy()).cuda()
        B.attn_block_prefill(kv, 1, res_dev, q_dim, lay.dev, EPS, THETA, start, scale, mode=mode)
        torch.cuda.synchronize()
        got = res_dev.cpu().numpy()
        normed = [oracle.rmsnorm(res[r], lay.attn_norm, EPS) for r in range(n)]
        ak = [oracle.quantize_row_q8_k(x) for x in normed]
        a0 = [oracle.quantize_row_q8_0(x) for x in normed]
        q = np.stack([oracle.gemv(lay.q_fmt, lay.wq, hidden, q_dim, a) for a in ak])
        k = np.stack([oracle.gemv(Q.RV_QF_Q8_0, lay.wk, hidden, kv_dim, a) for a in a0])
        v = np.stack([oracle.gemv(lay.v_fmt, lay.wv, hidden, kv_dim, a) for a in ak])
        attn = ref.prefill_chunk(1, q, k, v, lay.q_norm, lay.k_norm, EPS, THETA, start, scale)
        o = np.stack([oracle.gemv(lay.o_fmt, lay.wo, q_dim, hidden, oracle.quantize_row_q8_k(attn[r]))
                      for r in range(n)])
        want = (res + o).astype(np.float32)
        err = np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(o))
        say(f"prefill block {mode} chunk {chunk}: residual max|err|/max|o| {err:.2e}")
        assert err <= tol, f"{mode} chunk {chunk}"
        assert kv.len(1) == start + n and kv.len(0) == n_pos
        start += n

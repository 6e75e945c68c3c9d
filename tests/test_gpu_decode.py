"""Decode attention on the GPU vs the oracle (kernels/attention.rs gates).

Tolerances (tests/gpu_util.py `gate`): fp32 KV — the reference's elementwise
gate rel 1e-4 / abs 5e-5 (attention.rs:1469) and max|err|/max|ref| <= 1e-5
against the oracle on the same fp32 cache. f16 KV — the same against the
oracle on the same f16 cache, and the reference's own looser gate (rel 1e-3 /
abs 1.5e-3, attention.rs:1457) against the oracle on the unrounded fp32 values.
"""
import math

import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import FP32_FLOOR, FP32_REL, dev, elem_code, gate, host, rel_err, say, torch_cuda
from helpers import Rng, assert_close, reference_attention, round_trip
from ramvamp_amd import synth

pytestmark = pytest.mark.gpu


def twin_caches(rng, n_layers, n_kv, hd, n_pos, elem, cap=None):
    """A device cache and an oracle cache holding the same rows."""
    cap = cap or max(n_pos, 1)
    kv = rv.KvCache(n_layers, n_kv, hd, cap, elem)
    ref = oracle.KvCache(n_layers, n_kv, hd, cap, elem_code(elem))
    for layer in range(n_layers):
        K = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        V = rng.vec_in(n_pos * n_kv * hd, -1.0, 1.0).reshape(n_pos, -1)
        kv.append_rows(layer, K, V)
        ref.append_rows(layer, K, V)
    return kv, ref


GEOMETRIES = [  # (n_layers, n_kv, n_q, head_dim, n_pos): fast path (d 128, group 1/2/4/8) and generic
    (1, 4, 32, 128, 67), (2, 4, 32, 128, 300), (1, 2, 2, 128, 9), (1, 1, 8, 128, 130), (1, 4, 16, 128, 33),
    (2, 4, 32, 128, 5), (1, 2, 2, 16, 9), (1, 1, 8, 8, 7), (2, 3, 6, 4, 12), (1, 1, 8, 9, 11), (2, 3, 6, 9, 13),
    (1, 1, 32, 128, 9), (1, 2, 34, 16, 13), (1, 1, 12, 9, 11), (1, 1, 8, 256, 5), (1, 2, 4, 255, 3),
]


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_decode_and_limited_forms_match_the_oracle_across_geometries(elem):
    torch_cuda()
    rng = Rng(0xDEC0DE)
    for n_layers, n_kv, n_q, hd, n_pos in GEOMETRIES:
        say(f"case geometry {(n_layers, n_kv, n_q, hd, n_pos)} elem={elem}")
        kv, ref = twin_caches(rng, n_layers, n_kv, hd, n_pos, elem)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        q = rng.vec_in(n_q * hd, -1.0, 1.0)
        qd = dev(q)
        for layer in range(n_layers):
            out = dev(np.zeros(q.size))
            rv.decode_attention(qd, kv, layer, scale, None, out)
            gate(host(out), ref.attention(q, layer, scale), what=f"decode {(n_kv, n_q, hd, n_pos)}")
            for p in sorted({1, 2, 3, 8, 9, 17, n_pos // 2 + 1, n_pos}):
                if p > n_pos:
                    continue
                out = dev(np.zeros(q.size))
                rv.attention_at(qd, kv, layer, p, scale, None, out)
                gate(host(out), ref.attention(q, layer, scale, positions=p), what=f"attention_at p={p}")


def test_matches_f64_reference_across_layers_and_lengths():
    # attention.rs:1419-1473 on the device (f16 cache, v0 pin geometry).
    torch_cuda()
    n_layers, n_kv, n_q, hd, cap = 3, 4, 32, 128, 256
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    rng = Rng(0xA77E)
    kv = rv.KvCache(n_layers, n_kv, hd, cap, "f16")
    ks, vs = [[] for _ in range(n_layers)], [[] for _ in range(n_layers)]
    appended = 0
    for target in (1, 2, 17, 256):
        say(f"case f64 reference len={target}")
        while appended < target:
            for layer in range(n_layers):
                k, v = rng.vec_in(n_kv * hd, -1.0, 1.0), rng.vec_in(n_kv * hd, -1.0, 1.0)
                kv.append(layer, k, v)
                ks[layer].append(k)
                vs[layer].append(v)
            appended += 1
        for layer in range(n_layers):
            q = rng.vec_in(n_q * hd, -1.0, 1.0)
            out = np.zeros(q.size, np.float32)
            rv.decode_attention(q, kv, layer, scale, None, out)  # host-pointer path
            K, V = np.array(ks[layer]), np.array(vs[layer])
            assert_close(out, reference_attention(q, K, V, n_kv, hd, scale), 1e-3, 1.5e-3, "vs exact")
            assert_close(out, reference_attention(q, round_trip(K), round_trip(V), n_kv, hd, scale), 1e-4, 5e-5,
                         "vs stored")


def test_gqa_marker_single_position_and_odds_ratio():
    torch_cuda()
    say("case gqa marker")
    n_kv, n_q, hd = 4, 32, 16  # attention.rs:1483-1516 (generic path: head_dim 16)
    for head_dim in (hd, 128):  # and the fast path
        kv = rv.KvCache(1, n_kv, head_dim, 4, "f16")
        marker = lambda j, t: np.float32((10 * j + t) * 0.01)
        for t in range(4):
            k = np.zeros(n_kv * head_dim, np.float32)
            v = np.zeros(n_kv * head_dim, np.float32)
            for j in range(n_kv):
                k[j * head_dim:(j + 1) * head_dim] = (1.0 if t == j else -1.0) * 8.0 / head_dim
                v[j * head_dim:(j + 1) * head_dim] = marker(j, t)
            kv.append(0, k, v)
        out = np.zeros(n_q * head_dim, np.float32)
        rv.decode_attention(np.ones(n_q * head_dim, np.float32), kv, 0, 1.0, None, out)
        out = out.reshape(n_q, head_dim)
        for h in range(n_q):
            assert np.all(np.abs(out[h] - marker(h // 8, h // 8)) < 1e-3), (head_dim, h)

    say("case single position")  # attention.rs:1523-1554: bit-exact V row
    rng = Rng(0x5EED)
    for elem in ("f16", "f32"):
        kv = rv.KvCache(2, 4, 128, 8, elem)
        vs = []
        for layer in range(2):
            k, v = rng.vec_in(512, -1.0, 1.0), rng.vec_in(512, -1.0, 1.0)
            kv.append(layer, k, v)
            vs.append(v)
        q = rng.vec_in(32 * 128, -1.0, 1.0)
        for layer, v in enumerate(vs):
            out = np.zeros(q.size, np.float32)
            rv.decode_attention(q, kv, layer, np.float32(1.0) / np.sqrt(np.float32(128)), None, out)
            stored = round_trip(v) if elem == "f16" else v
            for h in range(32):
                assert np.array_equal(out.reshape(32, 128)[h], stored[(h // 8) * 128:(h // 8 + 1) * 128]), (elem, h)

    say("case odds ratio")  # attention.rs:1894-1918
    kv = rv.KvCache(1, 1, 4, 2, "f16")
    kv.append(0, [0, 0, 0, 0], [0] * 4)
    kv.append(0, [1, 0, 0, 0], [1] * 4)
    q = np.array([1.0, 0, 0, 0], np.float32)
    s = np.float32(0.7)
    p = []
    for sc in (s, np.float32(2.0) * s):
        out = np.zeros(4, np.float32)
        rv.decode_attention(q, kv, 0, sc, None, out)
        p.append(float(out[0]))
    sig = lambda x: 1.0 / (1.0 + math.exp(-x))
    assert_close(p[0], sig(float(s)), 1e-5, 0.0)
    assert_close(p[1], sig(2.0 * float(s)), 1e-5, 0.0)
    odds = lambda x: x / (1.0 - x)
    assert_close(odds(p[1]), odds(p[0]) ** 2, 1e-4, 0.0)


def test_error_precedence_matches_the_oracle_for_every_form():
    # attention.rs:1640-1888: same first failure, same payload, out untouched.
    torch_cuda()
    say("case precedence")
    n_kv, n_q, hd, cap = 4, 8, 8, 4
    kv = rv.KvCache(2, n_kv, hd, cap, "f16")
    ref = oracle.KvCache(2, n_kv, hd, cap)
    row = np.full(n_kv * hd, 0.5, np.float32)
    for _ in range(3):
        kv.append(0, row, row)
        ref.append(0, row, row)
    q = np.full(n_q * hd, 0.25, np.float32)
    need = oracle.scratch_len(n_q, n_kv, hd, cap)
    probes = [(q[:13], 9, 0, 7, range(5, 5)), (q[:5 * hd], 9, 0, 7, range(5, 5)), (q, 9, 0, 7, range(5, 5)),
              (q, 1, 0, 7, range(5, 5)), (q, 0, 9, 7, range(5, 5)), (q, 0, 2, 7, range(5, 5)),
              (q, 0, 2, 7, range(0, 4)), (q, 0, 2, 64, range(3, 1)), (q[:0], 0, 1, 0, range(0, 1))]
    for q_arg, layer, positions, out_len, kvr in probes:
        for form in ("decode", "decode_in", "at", "at_in", "decode_range", "at_range"):
            for scratch in ((need,) if form in ("decode", "at") else (need, 3)):
                out = np.full(max(out_len, 1), np.nan, np.float32)[:out_len]
                kw = {}
                if "range" in form:
                    kw["kv_range"] = kvr
                if form.startswith("at"):
                    kw["positions"] = positions
                if form not in ("decode", "at"):
                    kw["scratch_len"] = scratch
                try:
                    ref.attention(q_arg, layer, 0.5, out_len=out_len, **kw)
                    want = None
                except oracle.OracleError as e:
                    want = e.payload()
                fn = {"decode": lambda: rv.decode_attention(q_arg, kv, layer, 0.5, None, out),
                      "decode_in": lambda: rv.decode_attention_in(q_arg, kv, layer, 0.5, scratch, out),
                      "at": lambda: rv.attention_at(q_arg, kv, layer, positions, 0.5, None, out),
                      "at_in": lambda: rv.attention_at_in(q_arg, kv, layer, positions, 0.5, scratch, out),
                      "decode_range": lambda: rv.decode_attention_kv_range_in(q_arg, kv, layer, 0.5, kvr, scratch,
                                                                              out),
                      "at_range": lambda: rv.attention_at_kv_range_in(q_arg, kv, layer, positions, 0.5, kvr, scratch,
                                                                      out)}[form]
                try:
                    fn()
                    got = None
                except rv.RamvampError as e:
                    got = e.raw
                assert got == want, (form, layer, positions, out_len, kvr, scratch, got, want)
                if got is not None:
                    assert np.all(np.isnan(out)), "an error path wrote out"


def test_kv_range_union_is_bit_identical_to_the_whole_call():
    # attention.rs:3002 / forward.rs:3022-3122, with the split length pinned so
    # every kv head takes the same reduction tree in both calls.
    torch_cuda()
    say("case kv range union")
    rng = Rng(0x7A16)
    kv, ref = twin_caches(rng, 1, 4, 128, 700, "f16")
    kv.set_tuning(1, 64)
    q = rng.vec_in(32 * 128, -1.0, 1.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    whole = np.zeros(q.size, np.float32)
    rv.decode_attention(q, kv, 0, scale, None, whole)
    gate(whole, ref.attention(q, 0, scale), what="whole")
    for units in range(1, 9):
        got = np.full(q.size, np.nan, np.float32)
        for u in range(units):
            r = oracle.kv_head_range(4, units, u, u + 1)
            part = np.full(len(r) * 1024, np.nan, np.float32)
            rv.decode_attention_kv_range_in(q, kv, 0, scale, r, 10 ** 6, part)
            got[r.start * 1024:r.stop * 1024] = part
        assert np.array_equal(got.view(np.uint32), whole.view(np.uint32)), units


def test_decode_across_the_split_plan_regimes():
    # The default plan changes shape at these lengths (4 kv heads): whole
    # 64-position splits up to 4096, then even 16-position shares on one
    # workgroup per CU up to 448 positions each (28672), then on two.
    torch_cuda()
    rng = Rng(0x5A1F)
    kv, ref = twin_caches(rng, 1, 4, 128, 28673, "f16")
    q = rng.vec_in(32 * 128, -1.0, 1.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    for p in (4096, 4097, 8192, 8193, 28672, 28673):
        say(f"case split plan regime positions={p}")
        out = np.full(q.size, np.nan, np.float32)
        rv.attention_at(q, kv, 0, p, scale, None, out)
        gate(out, ref.attention(q, 0, scale, positions=p), what=f"positions {p}")


@pytest.mark.parametrize("elem,lengths", [("f16", (64, 65, 150, 192, 193)), ("f32", (64, 65, 128, 129))])
def test_decode_short_contexts_in_one_split(elem, lengths):
    # Up to 3 tiles per wave and 128 KiB of K and V per kv head (f16: 192
    # positions, fp32: 128) the default plan takes one split per kv head
    # with no merge launch, each wave walking several tiles; one position
    # more goes back to 64-position splits and the merge.
    torch_cuda()
    rng = Rng(0x5B07 + len(elem))
    kv, ref = twin_caches(rng, 1, 4, 128, max(lengths), elem)
    q = rng.vec_in(32 * 128, -1.0, 1.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    for p in lengths:
        say(f"case short context {elem} positions={p}")
        out = np.full(q.size, np.nan, np.float32)
        rv.attention_at(q, kv, 0, p, scale, None, out)
        gate(out, ref.attention(q, 0, scale, positions=p), what=f"{elem} positions {p}")


@pytest.mark.parametrize("elem,n_pos,waves,split_len", [
    ("f32", 4096, 4, 0), ("f32", 4096, 2, 32), ("f32", 4096, 1, 16), ("f16", 32768, 4, 0), ("f16", 300, 4, 0),
    ("f32", 1000, 4, 64), ("f16", 20000, 1, 0), ("f32", 129, 1, 16), ("f16", 8193, 2, 0)])
def test_in_launch_xcd_merge_matches_the_oracle(elem, n_pos, waves, split_len):
    # RV_TUNE_DECODE_MERGE 1: the splits of a kv head that share an XCD (s =
    # r mod 8) are folded inside that XCD's L2 by the last to finish, then
    # the last of the <= 8 group rows folds them across XCDs. Shapes: whole
    # and partial groups of 8 (4096 / 64: 8 per group; 1000 / 64: 16 splits;
    # 300: 5 splits, each its own group; 129 / 16: 9 splits, one group of
    # 2), 1-, 2- and 4-wave workgroups. Three calls in a row give the same
    # bits (every ticket is reset by its last arriver), the kv-range union is
    # bit-identical to the whole call, and the result is within the fp32 gate
    # of the oracle and of the separate merge kernel.
    torch_cuda()
    say(f"case xcd merge elem={elem} n_pos={n_pos} waves={waves} split_len={split_len}")
    rng = Rng(0x8CD + n_pos + 7 * waves + split_len)
    kv, ref = twin_caches(rng, 1, 4, 128, n_pos, elem)
    if not kv.xcd_ok():
        pytest.skip("the device does not deal workgroups to XCDs round robin")
    q = rng.vec_in(32 * 128, -1.0, 1.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    want = ref.attention(q, 0, scale)
    kv.set_tuning(rv.RV_TUNE_DECODE_WAVES, waves)
    if split_len:
        kv.set_tuning(rv.RV_TUNE_DECODE_SPLIT_LEN, split_len)
    kv.set_tuning(rv.RV_TUNE_DECODE_MERGE, 2)
    sep = np.full(q.size, np.nan, np.float32)
    rv.decode_attention(q, kv, 0, scale, None, sep)
    kv.set_tuning(rv.RV_TUNE_DECODE_MERGE, 1)
    outs = []
    for _ in range(3):
        out = np.full(q.size, np.nan, np.float32)
        rv.decode_attention(q, kv, 0, scale, None, out)
        outs.append(out)
    gate(outs[0], want, what=f"xcd merge {elem} {n_pos}")
    gate(outs[0], sep.astype(np.float64), what="xcd merge vs merge kernel")
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    got = np.full(q.size, np.nan, np.float32)
    for u in range(4):
        r = oracle.kv_head_range(4, 4, u, u + 1)
        part = np.full(len(r) * 1024, np.nan, np.float32)
        rv.decode_attention_kv_range_in(q, kv, 0, scale, r, 10 ** 6, part)
        got[r.start * 1024:r.stop * 1024] = part
    assert np.array_equal(got.view(np.uint32), outs[0].view(np.uint32))
    for p in (1, 17, n_pos // 2 + 1):
        out = np.full(q.size, np.nan, np.float32)
        rv.attention_at(q, kv, 0, p, scale, None, out)
        gate(out, ref.attention(q, 0, scale, positions=p), what=f"xcd merge attention_at p={p}")


@pytest.mark.parametrize("n_pos", [5000, 20000])
def test_kv_range_union_matches_the_whole_call_with_the_default_plan(n_pos):
    # The default split length is sized for the cache's kv heads, not the
    # range's, so each head's reduction tree is the whole call's at any
    # length (here past one workgroup per CU, where it grows in 16-position
    # steps).
    torch_cuda()
    say(f"case kv range union, default plan, n_pos={n_pos}")
    rng = Rng(0x7A17 + n_pos)
    kv, ref = twin_caches(rng, 1, 4, 128, n_pos, "f16")
    q = rng.vec_in(32 * 128, -1.0, 1.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    whole = np.zeros(q.size, np.float32)
    rv.decode_attention(q, kv, 0, scale, None, whole)
    gate(whole, ref.attention(q, 0, scale), what="whole")
    for units in (1, 2, 4):
        got = np.full(q.size, np.nan, np.float32)
        for u in range(units):
            r = oracle.kv_head_range(4, units, u, u + 1)
            part = np.full(len(r) * 1024, np.nan, np.float32)
            rv.decode_attention_kv_range_in(q, kv, 0, scale, r, 10 ** 6, part)
            got[r.start * 1024:r.stop * 1024] = part
        assert np.array_equal(got.view(np.uint32), whole.view(np.uint32)), units


@pytest.mark.parametrize("split_len", [16, 32, 48, 64, 128, 1024, 0])
def test_split_lengths_agree_within_tolerance(split_len):
    torch_cuda()
    say(f"case split_len={split_len}")
    rng = Rng(0x5711)
    kv, ref = twin_caches(rng, 1, 4, 128, 1537, "f32")
    kv.set_tuning(1, split_len)
    q = rng.vec_in(32 * 128, -2.0, 2.0)
    want = ref.attention(q, 0, 0.3)
    for p in (1, 16, 17, 1000, 1537):
        out = np.zeros(q.size, np.float32)
        rv.attention_at(q, kv, 0, p, 0.3, None, out)
        gate(out, ref.attention(q, 0, 0.3, positions=p), what=f"split {split_len} p {p}")
    out = np.zeros(q.size, np.float32)
    rv.decode_attention(q, kv, 0, 0.3, None, out)
    gate(out, want, what="decode")


@pytest.mark.parametrize("impl,waves", [(0, 4), (0, 8), (1, 4), (1, 8)])
@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_kernel_variants_agree_with_the_oracle(impl, waves, elem):
    """Both fast kernels (MFMA tiles, VALU subgroups) at both workgroup sizes,
    with splits of one and of several tiles per wave."""
    torch_cuda()
    say(f"case impl={impl} waves={waves} elem={elem}")
    rng = Rng(0x7EA1 + 16 * impl + waves)
    kv, ref = twin_caches(rng, 1, 4, 128, 2049, elem)
    kv.set_tuning(6, impl)
    kv.set_tuning(3, waves)
    q = rng.vec_in(32 * 128, -2.0, 2.0)
    for split_len in (0, 64, 200, 4096):
        kv.set_tuning(1, split_len)
        for p in (1, 15, 16, 65, 2049):
            out = np.zeros(q.size, np.float32)
            rv.attention_at(q, kv, 0, p, 0.3, None, out)
            gate(out, ref.attention(q, 0, 0.3, positions=p), what=f"impl {impl} waves {waves} split {split_len} p {p}")


@pytest.mark.parametrize("hg", [1, 2, 4, 8])
def test_valu_head_groups_agree_with_the_oracle(hg):
    """RV_TUNE_DECODE_HG: the VALU kernel's query heads per workgroup (the
    largest of 8/4/2/1 dividing the group, up to the tuned count), for a
    group of 8 and a group of 20, which only the VALU kernel takes."""
    torch_cuda()
    for n_q in (32, 80):
        say(f"case VALU head groups hg={hg} n_q={n_q}")
        rng = Rng(0x46A0 + 8 * hg + n_q)
        kv, ref = twin_caches(rng, 1, 4, 128, 700, "f32")
        kv.set_tuning(6, 1)
        kv.set_tuning(5, hg)
        q = rng.vec_in(n_q * 128, -2.0, 2.0)
        for p in (1, 64, 700):
            out = np.zeros(q.size, np.float32)
            rv.attention_at(q, kv, 0, p, 0.3, None, out)
            gate(out, ref.attention(q, 0, 0.3, positions=p), what=f"hg {hg} n_q {n_q} p {p}")


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_ring_depths_are_bit_identical(elem):
    """The tile kernel's register ring (RV_TUNE_DECODE_DEPTH 2 and 4; the
    default takes one tile at a time) changes only how many tiles' loads are
    in flight, never the arithmetic order: every depth gives depth 1's bits,
    and those pass the oracle gate."""
    torch_cuda()
    say(f"case ring depths elem={elem}")
    rng = Rng(0xDE97 + (elem == "f16"))
    kv, ref = twin_caches(rng, 1, 4, 128, 2049, elem)
    q = rng.vec_in(32 * 128, -2.0, 2.0)
    for waves in (4, 8):
        kv.set_tuning(rv.RV_TUNE_DECODE_WAVES, waves)
        for split_len in (0, 256, 4096):
            kv.set_tuning(rv.RV_TUNE_DECODE_SPLIT_LEN, split_len)
            outs = {}
            for depth in (1, 2, 4):
                kv.set_tuning(rv.RV_TUNE_DECODE_DEPTH, depth)
                out = np.full(q.size, np.nan, np.float32)
                rv.decode_attention(q, kv, 0, 0.3, None, out)
                outs[depth] = out
            what = f"waves {waves} split {split_len}"
            gate(outs[1], ref.attention(q, 0, 0.3), what=what)
            for depth in (2, 4):
                assert np.array_equal(outs[depth].view(np.uint32), outs[1].view(np.uint32)), f"{what} depth {depth}"


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_lds_staged_tiles_give_the_register_form_bits(elem):
    """RV_TUNE_DECODE_IMPL 3 stages each 64-position step through LDS with
    direct-to-LDS loads; the MFMA operands (and their clamping past a split's
    end) are the register form's, so the outputs are its bits, at one tile
    per split, ragged splits and long ones."""
    torch_cuda()
    say(f"case lds-staged elem={elem}")
    rng = Rng(0x1D5 + (elem == "f16"))
    kv, ref = twin_caches(rng, 1, 4, 128, 2049, elem)
    q = rng.vec_in(32 * 128, -2.0, 2.0)
    for split_len in (0, 64, 200, 1024, 4096):
        kv.set_tuning(rv.RV_TUNE_DECODE_SPLIT_LEN, split_len)
        for p in (1, 17, 64, 65, 2049):
            outs = {}
            for impl in (0, 3):
                kv.set_tuning(rv.RV_TUNE_DECODE_IMPL, impl)
                out = np.full(q.size, np.nan, np.float32)
                rv.attention_at(q, kv, 0, p, 0.3, None, out)
                outs[impl] = out
            what = f"split {split_len} p {p}"
            gate(outs[3], ref.attention(q, 0, 0.3, positions=p), what=what)
            assert np.array_equal(outs[3].view(np.uint32), outs[0].view(np.uint32)), what
    kv.set_tuning(rv.RV_TUNE_DECODE_IMPL, 0)


def test_config1_decode_step_matches_the_oracle():
    # cached rows 0..511 built by the fused prefill prologue,
    # then the fused decode step at position 512 (prologue + append + decode).
    torch_cuda()
    say("case config 1")
    c = synth.CONFIGS[1]
    kv = rv.KvCache(1, 4, 128, c.capacity, "f32")
    ref = oracle.KvCache(1, 4, 128, c.capacity, oracle.RV_ELEM_F32)
    wq, wk = synth.norm_weight(1, synth.T_QN), synth.norm_weight(1, synth.T_KN)
    q0, k0, v0 = synth.new_rows(1, 512, layer=1)
    out0 = np.zeros_like(q0)
    rv.prefill_chunk(kv, 0, q0, k0, v0, wq, wk, synth.EPS, synth.THETA, 0, synth.SCALE, out0)
    # Oracle: only the prologue and append (its attention over 512 rows is tested elsewhere).
    for r in range(512):
        k = oracle.norm_rope_heads(k0[r], 4, 128, wk, synth.EPS, synth.THETA, r)
        ref.append(0, k, v0[r])
    same = 0
    for pos in (0, 1, 255, 511):
        got, want = kv.k_row(0, pos), ref.read_row(False, 0, pos)
        gate(got, want, rel=2e-7, floor=1e-6, what=f"normed+rotated K row {pos}")
        same += int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
        assert np.array_equal(kv.v_row(0, pos), ref.read_row(True, 0, pos))
    say(f"config 1 prologue: {same} of {4 * 512} K elements bit-identical to the oracle")
    q, k, v = synth.new_rows(1, 1)
    out = np.zeros(q.size, np.float32)
    rv.decode_step(kv, 0, q[0], k[0], v[0], wq, wk, synth.EPS, synth.THETA, 512, synth.SCALE, out)
    want = ref.decode_step(0, q[0], k[0], v[0], wq, wk, synth.EPS, synth.THETA, 512, synth.SCALE)
    e = gate(out, want, what="config 1")
    say(f"config 1 max rel err {e:.3e}")
    assert kv.len(0) == 513


@pytest.mark.parametrize("elem", ["f32", "f16"])
def test_decode_step_rotates_q_and_k_at_the_given_position(elem):
    # forward.rs:2628-2629 rotates q and k at the same rope_pos; the row still
    # lands at the layer's cursor. Head dims 128/256/512 cover one, two and
    # four element pairs per lane in the fused prologue.
    torch_cuda()
    rng = Rng(0x5EED)
    for n_kv, n_q, hd, n_pos, position in ((4, 32, 128, 5, 700), (2, 6, 256, 3, 3), (1, 3, 512, 2, 41)):
        say(f"case decode_step {(n_kv, n_q, hd, n_pos, position)} elem={elem}")
        kv, ref = twin_caches(rng, 1, n_kv, hd, n_pos, elem, cap=n_pos + 1)
        wq, wk = rng.vec_in(hd, 0.9, 1.1), rng.vec_in(hd, 0.9, 1.1)
        q, k, v = rng.vec_in(n_q * hd, -2, 2), rng.vec_in(n_kv * hd, -2, 2), rng.vec_in(n_kv * hd, -2, 2)
        out = np.zeros(q.size, np.float32)
        rv.decode_step(kv, 0, q, k, v, wq, wk, 1e-6, 1e6, position, 0.125, out)
        want = ref.decode_step(0, q, k, v, wq, wk, 1e-6, 1e6, position, 0.125)
        # f16: the new K row may round one ulp apart (f64 sin/cos of two libms).
        f16 = elem == "f16"
        gate(out, want, rel=1e-3 if f16 else FP32_REL, abs_tol=1.5e-3 if f16 else FP32_FLOOR,
             what=f"decode_step hd {hd}")
        got_k, want_k = kv.k_row(0, n_pos), ref.read_row(False, 0, n_pos)
        gate(got_k, want_k, rel=1e-3 if f16 else 2e-7, floor=1e-6, what=f"rotated K row hd {hd}")
        assert np.array_equal(kv.v_row(0, n_pos), ref.read_row(True, 0, n_pos))
        assert kv.len(0) == n_pos + 1


def test_config2_layers_match_the_oracle_at_ctx_4096():
    torch_cuda()
    for layer in (0, 47):
        say(f"case config 2 layer {layer}")
        K, V = synth.cached_kv(2, layer, 4096)
        kv = rv.KvCache(1, 4, 128, 4096, "f32")
        ref = oracle.KvCache(1, 4, 128, 4096, oracle.RV_ELEM_F32)
        kv.append_rows(0, K, V)
        ref.append_rows(0, K, V)
        q = synth.normal(synth.seed(2, synth.T_Q, layer), synth.Q_DIM)
        out = dev(np.zeros(q.size))
        rv.decode_attention(dev(q), kv, 0, synth.SCALE, None, out)
        e = gate(host(out), ref.attention(q, 0, synth.SCALE), what=f"config 2 layer {layer}")
        say(f"config 2 layer {layer} max rel err {e:.3e}")


@pytest.fixture(scope="module")
def config5_oracle():
    """Config 5's cache rows, q, and the oracle's outputs on the f16 cache
    and on the unrounded fp32 rows, computed once."""
    n = 32768
    K, V = synth.cached_kv(5, 0, n)
    q = synth.rope_f64(synth.normal(synth.seed(5, synth.T_Q), synth.Q_DIM), 128, n, synth.THETA)
    ref16 = oracle.KvCache(1, 4, 128, n, oracle.RV_ELEM_F16)
    ref16.append_rows(0, K, V)
    want16 = ref16.attention(q, 0, synth.SCALE)
    del ref16
    ref32 = oracle.KvCache(1, 4, 128, n, oracle.RV_ELEM_F32)
    ref32.append_rows(0, K, V)
    want32 = ref32.attention(q, 0, synth.SCALE)
    return n, K, V, q, want16, want32


@pytest.mark.parametrize("split_len", [0, 1024, 2048, 4096])
def test_config5_long_context_f16_split_k(split_len, config5_oracle):
    # 8-32 KV splits (split_len 4096 / 2048 / 1024 pinned),
    # and the library's own plan (0: 128 splits per kv head), each against
    # the oracle on the same f16 cache and on the unrounded fp32 rows.
    torch_cuda()
    say(f"case config 5 split_len={split_len}")
    n, K, V, q, want16, want32 = config5_oracle
    kv = rv.KvCache(1, 4, 128, n, "f16")
    kv.append_rows(0, K, V)
    kv.set_tuning(rv.RV_TUNE_DECODE_SPLIT_LEN, split_len)
    out = dev(np.full(q.size, np.nan, np.float32))
    rv.decode_attention(dev(q), kv, 0, synth.SCALE, None, out)
    got = host(out)
    e16 = gate(got, want16, what=f"config 5 split {split_len} vs f16 oracle")
    assert_close(got, want32, 1e-3, 1.5e-3, f"config 5 split {split_len} vs fp32 oracle (f16 storage bound)")
    say(f"config 5 split {split_len}: max rel err vs f16 oracle {e16:.3e}; vs fp32 oracle {rel_err(got, want32):.3e}")


def test_outputs_are_convex_combinations_of_v_rows():
    # Size-independent property at a full config size: each output element lies
    # within [min, max] of its kv head's V column, and a constant V is returned.
    torch = torch_cuda()
    say("case convexity")
    n = 4096
    K, V = synth.cached_kv(2, 3, n)
    kv = rv.KvCache(1, 4, 128, n, "f32")
    kv.append_rows(0, K, V)
    q = dev(synth.normal(99, synth.Q_DIM) * 4)
    out = dev(np.zeros(synth.Q_DIM))
    rv.decode_attention(q, kv, 0, synth.SCALE, None, out)
    o = host(out).reshape(4, 8, 128)
    Vh = V.reshape(n, 4, 128)
    lo, hi = Vh.min(axis=0), Vh.max(axis=0)
    assert np.all(o >= lo[:, None, :] - 1e-6) and np.all(o <= hi[:, None, :] + 1e-6)
    kv2 = rv.KvCache(1, 4, 128, n, "f32")
    kv2.append_rows(0, K, np.full_like(V, 0.375))
    rv.decode_attention(q, kv2, 0, synth.SCALE, None, out)
    assert np.allclose(host(out), 0.375, rtol=1e-6, atol=0)
    torch.cuda.synchronize()


@pytest.mark.parametrize("q_scale", [3e4, 1e6, 1e-4])
def test_f16_decode_keeps_fp32_products_at_extreme_q(q_scale):
    # The f16-operand decode splits each head's q into f16 halves after a
    # power-of-two scaling: q far outside f16's range (or deep in its
    # subnormals) must still give the fp32 result on the same f16 cache.
    torch_cuda()
    say(f"case f16 decode q_scale={q_scale}")
    rng = Rng(0xF16)
    kv, ref = twin_caches(rng, 1, 4, 128, 300, "f16")
    q = rng.vec_in(32 * 128, -1.0, 1.0) * np.float32(q_scale)
    scale = 0.0883883 / max(q_scale, 1.0)  # keep the scores in a sane range
    out = np.zeros(q.size, np.float32)
    rv.decode_attention(q, kv, 0, scale, None, out)
    gate(out, ref.attention(q, 0, scale), what=f"f16 decode q x {q_scale}")


@pytest.mark.parametrize("host_ptrs", [False, True])
def test_norm_weight_lengths_are_refused_as_the_oracle_refuses_them(host_ptrs):
    # primitives/norm.rs:72-83 LengthMismatch, q's weight before k's; no row is
    # appended and out is untouched. With host pointers nothing is copied from
    # a short weight (the check runs before any staging).
    torch_cuda()
    n_kv, n_q, hd = 4, 32, 128
    say(f"case norm weight lengths host_ptrs={host_ptrs}")
    rng = Rng(0x11E8)
    w = rng.vec_in(hd, 0.5, 1.5)
    q, k, v = rng.vec_in(n_q * hd, -1.0, 1.0), rng.vec_in(n_kv * hd, -1.0, 1.0), rng.vec_in(n_kv * hd, -1.0, 1.0)
    cases = [(w[:hd - 1], w), (np.concatenate([w, w]), w[:3]), (w, w[:3]), (w, np.concatenate([w, w[:1]]))]
    put = (lambda a: a) if host_ptrs else dev
    for wq, wk in cases:
        kv = rv.KvCache(1, n_kv, hd, 4, "f32")
        ref = oracle.KvCache(1, n_kv, hd, 4, oracle.RV_ELEM_F32)
        with pytest.raises(oracle.OracleError) as e:
            ref.decode_step(0, q, k, v, wq, wk, 1e-6, 1e6, 0, 0.5)
        want = e.value.payload()
        out = np.full(q.size, np.nan, np.float32) if host_ptrs else dev(np.full(q.size, np.nan, np.float32))
        with pytest.raises(rv.RamvampError) as g:
            rv.decode_step(kv, 0, put(q), put(k), put(v), put(wq), put(wk), 1e-6, 1e6, 0, 0.5, out)
        assert g.value.raw == want, (g.value.raw, want)
        with pytest.raises(rv.RamvampError) as g:
            rv.prefill_chunk(kv, 0, put(q.reshape(1, -1)), put(k.reshape(1, -1)), put(v.reshape(1, -1)), put(wq),
                             put(wk), 1e-6, 1e6, 0, 0.5, out.reshape(1, -1) if host_ptrs else out.view(1, -1))
        assert g.value.raw == want, (g.value.raw, want)
        assert kv.len(0) == 0
        assert np.all(np.isnan(out if host_ptrs else host(out)))

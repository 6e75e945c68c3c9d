"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares, and its host-only entry points (no device work) agree with the
oracle. No compute call is made here."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from ramvamp_amd import _lib as L
from ramvamp_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(rv_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(L.LIB_PATH):
        pytest.fail(f"{L.LIB_PATH} not built (run __graft_entry__.build())")
    return L.load()


def test_every_declared_symbol_is_exported_and_typed(lib):
    declared = header_functions()
    assert len(declared) >= 30
    assert set(declared) == set(L.SIGNATURES), set(declared) ^ set(L.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name


def test_library_is_a_gfx950_hip_build():
    data = open(L.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"gfx942" not in data


def test_version_and_status_names(lib):
    assert lib.rv_abi_version() == 1
    names = {c: lib.rv_status_name(c).decode() for c in (0, 1, 2, 3, 4, 5, 6, 7, 16, 17, 18, 19, 20, 21, 24, 25, 32,
                                                            33, 34, 35, 40, 41, 42, 43, 44)}
    assert names[0] == "RV_OK" and names[21] == "RV_ATTN_SCRATCH_TOO_SHORT"
    assert names[44] == "RV_QUANT_UNSUPPORTED_FORMAT"
    assert len(set(names.values())) == len(names)
    assert lib.rv_status_name(999).decode() == "RV_UNKNOWN"


def test_scratch_len_matches_the_reference_carve(lib):
    for args in [(32, 4, 128, 4096), (32, 4, 8, 17), (32, 0, 8, 17), (2 ** 63, 1, 2, 4), (8, 2, 9, 0)]:
        assert lib.rv_scratch_len(*args) == oracle.scratch_len(*args), args
    assert lib.rv_scratch_len(32, 4, 128, 4096) == 33_024


def test_projected_bytes_and_dim_errors_match_the_oracle(lib):
    for dims in [(48, 4, 128, 4096), (1, 1, 1, 1), (3, 2, 9, 13), (0, 4, 128, 8), (1, 0, 128, 8), (2, 2 ** 62, 4, 1),
                 (2, 2 ** 61, 2, 1), (2 ** 40, 2 ** 20, 2 ** 4, 1)]:
        for elem in (1, 2):
            out, err = ctypes.c_uint64(), L.RvError()
            rc = lib.rv_kv_projected_bytes(*dims, elem, ctypes.byref(out), ctypes.byref(err))
            try:
                want = oracle.projected_bytes(*dims, elem)
                assert rc == 0 and out.value == want, dims
            except oracle.OracleError as e:
                assert (rc, err.a, err.b, err.c, err.d, err.what.decode()) == e.payload(), dims
    out, err = ctypes.c_uint64(), L.RvError()
    assert lib.rv_kv_projected_bytes(1, 1, 1, 1, 3, ctypes.byref(out), ctypes.byref(err)) == 35


def test_synthetic_generator_is_deterministic_and_standard_normal():
    a = synth.normal(synth.seed(2, synth.T_KC, 7), 1 << 20)
    b = synth.normal(synth.seed(2, synth.T_KC, 7), 1 << 20)
    c = synth.normal(synth.seed(2, synth.T_KC, 8), 1 << 20)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    # prefix-stable: a shorter draw is a prefix of a longer one
    assert np.array_equal(synth.normal(123, 1001), synth.normal(123, 5000)[:1001])
    w = synth.norm_weight(1, synth.T_QN)
    assert w.shape == (128,) and abs(float(w.mean()) - 1.0) < 0.01


def test_quant_geometry_matches_the_oracle(lib):
    """QuantFormat geometry and row_bytes (quants/mod.rs:75-105) and the
    projection scratch sizes, host-only entry points."""
    for fmt in (1, 2, 3, 4, 5, 0, 6):
        assert lib.rv_quant_block_weights(fmt) == (oracle.quant_block_weights(fmt) if fmt in range(1, 6) else 0)
        assert lib.rv_quant_block_bytes(fmt) == oracle.quant_block_bytes(fmt)
    for fmt in (1, 2, 3, 4, 5):
        for in_dim in (0, 32, 100, 256, 768, 2048, 4096, 4097):
            n, err = ctypes.c_size_t(), L.RvError()
            rc = lib.rv_quant_row_bytes(fmt, in_dim, ctypes.byref(n), ctypes.byref(err))
            try:
                want = oracle.quant_row_bytes(fmt, in_dim)
            except oracle.OracleError as e:
                assert (rc, err.a, err.b, err.c) == e.payload()[:4]
            else:
                assert rc == 0 and n.value == want
    n, err = ctypes.c_size_t(), L.RvError()
    assert lib.rv_quant_row_bytes(9, 256, ctypes.byref(n), ctypes.byref(err)) == 44
    assert lib.rv_attn_in_proj_scratch_bytes(2048) == 16 * ((8 * 292 + 15) // 16) + 64 * 36
    assert lib.rv_attn_out_proj_scratch_bytes(4096) == 16 * 292



def test_mirror_argument_checks_reject_bad_device_tensors():
    # The Python mirror's per-call marshalling: device tensors must be
    # contiguous float32 on the GPU; host arrays go through numpy.
    import numpy as np
    import torch
    from ramvamp_amd import attention as A

    with pytest.raises(TypeError, match="on the GPU"):
        A._Arg(torch.zeros(8, dtype=torch.float32))
    with pytest.raises(TypeError, match="float32"):
        A._Arg(torch.zeros(8, dtype=torch.float64))
    with pytest.raises(TypeError, match="float32"):
        A._Arg(torch.zeros(4, 4, dtype=torch.float32).t())
    a = A._Arg(np.arange(6, dtype=np.float64))  # converted to a float32 copy
    assert a.host and a.n == 6 and a.keep.dtype == np.float32
    with pytest.raises(TypeError, match="read-only"):
        ro = np.zeros(4, np.float32)
        ro.flags.writeable = False
        A._Arg(ro, writable=True)


def test_projected_device_bytes_adds_what_the_device_path_keeps(lib):
    """rv_kv_projected_device_bytes (a fresh cache's rv_kv_device_bytes
    bound): rv_kv_projected_bytes' planes plus the decode workspace, tickets,
    one EXACT staged copy per layer and the (cos, sin) table. Pinned by what
    the header states of each part rather than by restating the sum:
    - it exceeds the planes, and the excess grows by exactly one staged copy
      plus one pair of planes per added layer (the workspace, tickets and
      table do not depend on the layer count);
    - an EXACT staged copy is 17/16 of a layer's f32 planes (17/8 of its f16
      planes): 64-position tiles of two split planes of 2-byte elements plus
      4 KiB of exponents per 64 KiB of f32 K and V;
    - the table is capacity * head_dim * 4 bytes: doubling the capacity of a
      head_dim-128 cache adds 2x the planes, the staged copies and the table,
      and a decode workspace no smaller;
    - a head_dim other than 128 has no staged copy and the 1 MiB workspace."""
    from ctypes import byref, c_uint64

    def proj(L_, H, D, C, elem):
        out, err = c_uint64(), L.RvError()
        rc = lib.rv_kv_projected_device_bytes(L_, H, D, C, elem, byref(out), byref(err))
        assert rc == 0, (rc, err.what)
        return out.value

    def planes(L_, H, D, C, elem):
        out, err = c_uint64(), L.RvError()
        assert lib.rv_kv_projected_bytes(L_, H, D, C, elem, byref(out), byref(err)) == 0
        return out.value

    for elem, ratio in ((L.RV_ELEM_F32, (17, 16)), (L.RV_ELEM_F16, (17, 8))):
        one, two = proj(1, 4, 128, 4096, elem), proj(2, 4, 128, 4096, elem)
        layer_planes = planes(1, 4, 128, 4096, elem)
        staged = (two - one) - layer_planes
        assert staged * ratio[1] == layer_planes * ratio[0], (elem, staged, layer_planes)
        # config 2's cache: 48 layers at 4096 positions, fp32.
        p48 = proj(48, 4, 128, 4096, elem)
        assert p48 == one + 47 * (two - one)
        fixed = one - layer_planes - staged  # workspace + tickets + table
        assert fixed >= 1 << 20 and fixed >= 4096 * 128 * 4
        big = proj(1, 4, 128, 8192, elem)
        assert big - (2 * layer_planes + 2 * staged) >= fixed + 4096 * 128 * 4
    # No staged copy off head_dim 128: the difference per layer is the planes.
    a, b = proj(1, 2, 64, 1000, L.RV_ELEM_F16), proj(3, 2, 64, 1000, L.RV_ELEM_F16)
    assert b - a == 2 * planes(1, 2, 64, 1000, L.RV_ELEM_F16)
    assert a - planes(1, 2, 64, 1000, L.RV_ELEM_F16) >= (1 << 20) + 1000 * 64 * 4
    # Invalid geometries fail as rv_kv_projected_bytes does.
    out, err = c_uint64(), L.RvError()
    assert lib.rv_kv_projected_device_bytes(0, 4, 128, 16, L.RV_ELEM_F16, byref(out), byref(err)) == 1

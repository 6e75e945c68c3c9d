"""Helpers for the GPU parity tests: device placement, tolerance gates, and
building an oracle cache with the same contents as a device cache."""
import sys

import numpy as np
import pytest

import oracle

# fp32 parity gate: max relative error <= 1e-4, judged two ways, both required:
#  - the reference's own elementwise gate, |err| <= 5e-5 or |err|/|ref| <= 1e-4
#    (assert_close at attention.rs:1469);
#  - scale-normalised: max|err| / max|ref| <= 1e-5, so outputs far below the
#    reference gate's 5e-5 absolute term are still held to the output's scale.
# Both the device and the oracle accumulate in f32 in different orders, so
# they differ by a few ulps of the output's magnitude on long sums; that is
# the noise floor these gates sit above.
FP32_REL, FP32_FLOOR, FP32_SCALE = 1e-4, 5e-5, 1e-5


def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(x):
    torch = torch_cuda()
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def host(t):
    torch = torch_cuda()
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def rel_err(got, want, floor=FP32_FLOOR):
    """max |err| / max(|ref|, floor)."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    return float(np.max(np.abs(g - w) / np.maximum(np.abs(w), floor))) if g.size else 0.0


def scaled_err(got, want):
    """max |err| / max |ref|."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    return float(np.max(np.abs(g - w)) / max(float(np.max(np.abs(w))), np.finfo(np.float64).tiny)) if g.size else 0.0


def gate(got, want, rel=FP32_REL, abs_tol=FP32_FLOOR, scale=None, floor=None, what=""):
    """The reference's elementwise gate (|err| <= abs_tol or |err| <= rel*|ref|)
    and the scale-normalised gate (max|err|/max|ref| <= scale, default rel/10)
    must both hold; with `floor`, max|err|/max(|ref|, floor) <= rel instead of
    the latter (for near-bit-exact comparisons). Returns max|err|/max|ref|."""
    got = np.asarray(got)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    g = got.astype(np.float64)
    w = np.asarray(want, np.float64)
    diff = np.abs(g - w)
    ref_ok = (diff <= abs_tol) | (diff <= rel * np.abs(w))
    assert np.all(ref_ok), (f"{what}: reference gate (rel {rel:.0e} / abs {abs_tol:.0e}) fails at "
                            f"{int(np.sum(~ref_ok))} elements, max abs err {float(diff.max()):.3e}")
    if floor is not None:
        e = rel_err(g, w, floor)
        assert e <= rel, f"{what}: max rel err {e:.3e} > {rel:.1e} (floor {floor:.0e})"
        return e
    s = scaled_err(g, w)
    lim = rel / 10 if scale is None else scale
    assert s <= lim, f"{what}: max|err|/max|ref| {s:.3e} > {lim:.1e}"
    return s


def elem_code(elem):
    return oracle.RV_ELEM_F16 if elem == "f16" else oracle.RV_ELEM_F32

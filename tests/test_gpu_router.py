"""GPU parity of the router decision (include/ramvamp_router.h;
model/forward.rs:2658-2705): expert indices and weights bit-identical to
the oracle's, per row, at the model's shape (128 experts over a 2048-wide
row, top 8, with and without renormalization), odd sizes, batches of
prefill rows (including the sizes that group 2 and 4 rows per workgroup,
with a ragged last group), exact ties, and the validation order."""
import numpy as np
import pytest

import oracle
import ramvamp_amd as rv
from gpu_util import say, torch_cuda
from ramvamp_amd import router as R

pytestmark = pytest.mark.gpu


def check(torch, x, router, top_k, norm):
    n_experts = router.shape[0]
    ex, w = R.router_topk(torch.from_numpy(x).cuda(), torch.from_numpy(router).cuda(), top_k, norm)
    torch.cuda.synchronize()
    ex, w = ex.cpu().numpy().view(np.uint32), w.cpu().numpy()
    for r in range(x.shape[0]):
        we, ww = oracle.router_topk(x[r], router, n_experts, top_k, norm)
        assert list(ex[r]) == list(we), f"row {r} experts"
        assert w[r].tobytes() == ww.tobytes(), f"row {r} weights {w[r]} vs {ww}"


@pytest.mark.parametrize("n_rows,hidden,n_experts,top_k", [(1, 2048, 128, 8), (7, 2048, 128, 8), (64, 2048, 128, 8),
                                                           (3, 33, 5, 5), (2, 4096, 257, 3), (513, 2048, 128, 8),
                                                           (1027, 2048, 128, 8), (1030, 100, 300, 4),
                                                           (2, 64, 60, 4), (3, 192, 128, 2), (1, 320, 100, 6),
                                                           (1, 4096, 128, 8)])
@pytest.mark.parametrize("norm", [False, True])
def test_router_is_bit_identical_to_the_oracle(n_rows, hidden, n_experts, top_k, norm):
    torch = torch_cuda()
    say(f"case router rows={n_rows} hidden={hidden} experts={n_experts} top_k={top_k} norm={norm}")
    rng = np.random.default_rng(hidden + n_experts + n_rows)
    x = rng.standard_normal((n_rows, hidden)).astype(np.float32)
    router = (rng.standard_normal((n_experts, hidden)) * 0.03).astype(np.float32)
    check(torch, x, router, top_k, norm)


def test_router_ties_take_the_first_index():
    torch = torch_cuda()
    router = np.zeros((16, 64), np.float32)  # every logit 0: probabilities equal
    x = np.ones((2, 64), np.float32)
    check(torch, x, router, 6, False)
    router = np.tile(np.linspace(-1, 1, 64, dtype=np.float32), (8, 1))  # identical rows: identical logits
    check(torch, x, router, 8, True)


def test_router_validation_order():
    torch = torch_cuda()
    x = torch.ones(1, 8, device="cuda")
    router = torch.ones(4, 8, device="cuda")
    with pytest.raises(rv.RamvampError) as ei:
        R.router_topk(x, router, 0, False)
    assert ei.value.variant == "InvalidTopK" and ei.value.fields["top_k"] == 0
    with pytest.raises(rv.RamvampError) as ei:
        R.router_topk(x, router, 5, False)
    assert ei.value.variant == "InvalidTopK" and ei.value.fields["n_experts"] == 4
    with pytest.raises(rv.RamvampError) as ei:
        R.router_topk(x, torch.ones(4, 7, device="cuda").reshape(4, 7)[:, :7].contiguous(), 2, False)
    assert ei.value.variant in ("LengthMismatch",)

"""iq_gemv_noalloc (the entry point that allocates nothing, scratch in a
static device array) against iq_gemv through the C ABI: the same kernels
on the same inputs give bit-identical outputs, over two calls in a row
whose second is smaller, at widths that use the workspace (2..16-row
activation conversion, split-K partial sums, the 17..32-row GEMM tiles).
It has no counterpart in the reference."""
import numpy as np
import pytest
import torch

from infer_amd import ops
from tests.gpu_util import CANARY, QFix, check_linear, out_buffer, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", [0, 1])
def test_noalloc_matches_iq_gemv(kind):
    rng = np.random.default_rng(4242 + kind)
    # (M, K, N): first call large, second smaller
    for (M1, K1, N1), (M2, K2, N2) in (((16, 18944, 3584), (3, 1536, 700)),
                                       ((32, 8960, 1536), (12, 3584, 512)),
                                       ((9, 3584, 18944), (1, 3584, 3584))):
        for M, K, N in ((M1, K1, N1), (M2, K2, N2)):
            W = QFix(rng, N, K, kind, sd=0.02)
            x = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).cuda()
            ya, yb = out_buffer(M, N), out_buffer(M, N)
            say("noalloc", kind, M, K, N)
            ops.launch_gemv_batched_q(x, W.view, None, M, K, N, ya)
            ops.gemv_noalloc(x, W.view, None, M, K, N, yb)
            torch.cuda.synchronize()
            assert torch.equal(ya, yb), (kind, M, K, N)
            if M * N <= 16 * 4096:
                check_linear(yb, x.cpu().numpy(), W, None, M, f"noalloc kind={kind} M={M} {N}x{K}")


def test_noalloc_rejects_oversize():
    rng = np.random.default_rng(5)
    W = QFix(rng, 16, 32896, 0, sd=0.02)
    x = torch.zeros(1, 32896, device="cuda")
    y = out_buffer(1, 16)
    with pytest.raises(RuntimeError, match="workspace limits"):
        ops.gemv_noalloc(x, W.view, None, 1, 32896, 16, y)
    torch.cuda.synchronize()
    assert torch.all(y == CANARY)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [28, 32])
def test_noalloc_lm_head_wide_rows(kind, M):
    """The 7B lm_head (152064 x 3584) at 28..32 rows through the static
    scratch: the widest call whose K-range partial sums cannot fit the
    scratch (the plan then keeps every range in one workgroup per row
    block), checked against the oracle on sampled rows, then a smaller
    call on the same scratch."""
    from tests.test_gpu_routes import Packed, check_sampled
    rng = np.random.default_rng(152064 + 2 * M + kind)
    N, K = 152064, 3584
    W = Packed(rng, N, K, kind)
    x = rng.standard_normal((M, K), dtype=np.float32)
    y = out_buffer(M, N)
    say("noalloc lm_head", kind, M)
    ops.gemv_noalloc(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, M, rng, f"noalloc lm_head kind={kind} M={M}")
    W2 = Packed(rng, 1536, K, kind)
    x2 = rng.standard_normal((9, K), dtype=np.float32)
    y2 = out_buffer(9, 1536)
    ops.gemv_noalloc(torch.from_numpy(x2).cuda(), W2.view, None, 9, K, 1536, y2)
    torch.cuda.synchronize()
    check_sampled(y2, x2, W2, 9, rng, f"noalloc 1536x3584 kind={kind} M=9")

"""Graph capture of the launchers (the reference captures its decode and
prefill launches in graphs, kernels/batch_gpu.cu:81-85,255-269): after
iq_init_stream, no call allocates, so a call can be captured the first time
it is made.

* the reference's 256-row prefill chunk on 7B down (fp32 activations,
  3584 x 18944: 19.4 MB of prepared operands) captured without being called
  before, replayed several times with eager work in between, every replay
  bit-identical to the eager result and within the oracle's tolerance;
* a 1024-row call (78 MB of operands, one chunk) and a 1100-row call (two
  row chunks) eager, against the oracle on sampled rows;
* a capturing stream without its own workspace is refused (nothing
  enqueued) instead of sharing another stream's buffers."""
import numpy as np
import pytest
import torch

from infer_amd import ops
from tests.gpu_util import out_buffer, say
from tests.test_gpu_routes import Packed, check_sampled

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", [0, 1])
def test_capture_prefill_chunk_without_precall(kind):
    rng = np.random.default_rng(256 + kind)
    T, N, K = 256, 3584, 18944
    W = Packed(rng, N, K, kind)
    x = rng.standard_normal((T, K), dtype=np.float32)
    xd = torch.from_numpy(x).cuda()
    s = torch.cuda.Stream()
    ops.init(0, s)
    torch.cuda.synchronize()
    yg = out_buffer(T, N)
    say("capture prefill chunk", kind)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.launch_gemm_tiled_q(xd, W.view, None, T, K, N, yg, stream=s)
    torch.cuda.synchronize()
    ye = out_buffer(T, N)
    ops.launch_gemm_tiled_q(xd, W.view, None, T, K, N, ye)
    torch.cuda.synchronize()
    check_sampled(ye, x, W, T, rng, f"eager T=256 down kind={kind}")
    other = Packed(rng, 512, 3584, kind)
    for r in range(4):
        yg[: T * N].fill_(0.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ye), f"replay {r} differs from the eager result"
        # eager work on the same buffers between replays
        xo = torch.from_numpy(rng.standard_normal((300, 3584), dtype=np.float32)).cuda()
        yo = torch.empty(300, 512, device="cuda")
        ops.launch_gemm_tiled_q(xo, other.view, None, 300, 3584, 512, yo)
        ops.launch_gemm_tiled_q(xd, W.view, None, T, K, N, yo.new_empty(T * N))
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1024, 1100])
def test_long_prefill_in_row_chunks(T):
    rng = np.random.default_rng(T)
    N, K = 3584, 18944
    W = Packed(rng, N, K, 0)
    x = rng.standard_normal((T, K), dtype=np.float32)
    y = out_buffer(T, N)
    say("long prefill", T)
    ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, T, rng, f"T={T} down int8")


def test_capture_without_workspace_is_refused():
    rng = np.random.default_rng(9)
    W = Packed(rng, 512, 3584, 1)
    x = torch.zeros(4, 3584, device="cuda")
    y = out_buffer(4, 512)
    s = torch.cuda.Stream()  # no iq_init_stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="iq_gemv"):
        with torch.cuda.graph(g, stream=s):
            x.add_(0.0)  # (a non-empty capture)
            ops.launch_gemv_batched_q(x, W.view, None, 4, 3584, 512, y, stream=s)
    torch.cuda.synchronize()

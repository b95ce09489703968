"""GEMV / GEMM / embedding parity through the C ABI against the oracle:
float64 over dequant() (tests/test_ops_gpu.cu:664-692), conditioning-normalised
error <= 5e-6 and max|y-ref|/max|ref| <= 1e-3, canaries past y, ragged shapes."""
import numpy as np
import pytest
import torch

from infer_amd import ops
from oracle import oracle as O
from tests.gpu_util import QFix, bias_of, check_linear, out_buffer, say, CANARY

pytestmark = pytest.mark.gpu

# tests/test_ops_gpu.cu:886-893 shapes (in, out) and T values
REF_SHAPES = [(128, 64), (130, 127), (896, 300), (1536, 65)]


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("T", [1, 5, 32, 70])
@pytest.mark.parametrize("bias", [False, True])
def test_reference_shapes(kind, T, bias):
    rng = np.random.default_rng(20260919 + T + kind)
    for K, N in REF_SHAPES:
        W = QFix(rng, N, K, kind)
        x = rng.standard_normal((T, K), dtype=np.float32)
        bb, bd = bias_of(rng, N) if bias else (None, None)
        y = out_buffer(T, N)
        say("linear ref-shape", kind, T, K, N, bias)
        ops.launch_linear_q(torch.from_numpy(x).cuda(), W.view, bd, T, K, N, y)
        torch.cuda.synchronize()
        check_linear(y, x, W, bb, T, f"kind={kind} T={T} {N}x{K}")


@pytest.mark.parametrize("kind", [0, 1])
def test_tiny_shapes_every_row_count(kind):
    """Matrices smaller than one 16-row tile or one 4-group block (1, 7 and
    33 output rows; 128, 256 and ragged 130 / 640 columns) at every row
    count 1..32 through the reference's linear_b routing (GEMV to 32 rows),
    with a bias: every route's ragged edge, the short 1-row tiles on
    matrices of a tile or two, and K of one group."""
    rng = np.random.default_rng(31337 + kind)
    for N, K in ((1, 128), (7, 256), (33, 130), (33, 640), (17, 384)):
        W = QFix(rng, N, K, kind)
        bb, bd = bias_of(rng, N)
        for M in range(1, 33):
            x = rng.standard_normal((M, K), dtype=np.float32)
            y = out_buffer(M, N)
            say("tiny shapes", kind, N, K, M)
            ops.launch_linear_q(torch.from_numpy(x).cuda(), W.view, bd, M, K, N, y)
            torch.cuda.synchronize()
            check_linear(y, x, W, bb, M, f"tiny kind={kind} {N}x{K} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
def test_tiny_shapes_prefill(kind):
    """The prefill GEMM on matrices smaller than one output tile (1, 7 and
    33 rows; K of one group, ragged 130 and 640) at T = 33, 64, 65, 128,
    129 and 300, fp32 activations through linear_b and bf16 activations
    through iq_gemm_bf16x, with a bias on the fp32 calls."""
    rng = np.random.default_rng(4242 + kind)
    for N, K in ((1, 128), (7, 256), (33, 130), (33, 640)):
        W = QFix(rng, N, K, kind)
        bb, bd = bias_of(rng, N)
        for T in (33, 64, 65, 128, 129, 300):
            x = rng.standard_normal((T, K), dtype=np.float32)
            y = out_buffer(T, N)
            say("tiny prefill", kind, N, K, T)
            ops.launch_linear_q(torch.from_numpy(x).cuda(), W.view, bd, T, K, N, y)
            torch.cuda.synchronize()
            check_linear(y, x, W, bb, T, f"tiny prefill kind={kind} {N}x{K} T={T}")
            xb = O.f32_to_bf16(x)
            y = out_buffer(T, N)
            ops.launch_gemm_bf16x(torch.from_numpy(xb.view(np.int16)).cuda(), W.view, None, T, K, N, y)
            torch.cuda.synchronize()
            check_linear(y, O.bf16_to_f32(xb), W, None, T, f"tiny prefill bf16 kind={kind} {N}x{K} T={T}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 12, 16, 17, 32])
def test_gemv_15b_mlp_shapes(kind, M):
    rng = np.random.default_rng(77 + M)
    for N, K in ((8960, 1536), (1536, 8960)):
        W = QFix(rng, N, K, kind, sd=0.02)
        x = rng.standard_normal((M, K), dtype=np.float32)
        y = out_buffer(M, N)
        say("gemv 1.5B", kind, M, N, K)
        ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
        torch.cuda.synchronize()
        check_linear(y, x, W, None, M, f"gemv kind={kind} M={M} {N}x{K}")


@pytest.mark.parametrize("kind", [0, 1])
def test_gemv_7b_down_and_wide_activations(kind):
    """K = 18944 (split-K path) and activations spanning many decades
    (the per-group power-of-two prescale keeps fp16 in range)."""
    rng = np.random.default_rng(3)
    N, K = 3584, 18944
    W = QFix(rng, N, K, kind, sd=0.02)
    for M in (1, 16):
        x = rng.standard_normal((M, K), dtype=np.float32)
        x *= np.float32(10.0) ** rng.integers(-6, 6, size=(M, K)).astype(np.float32)
        x[0, :128] *= np.float32(1e6)  # beyond fp16 range without prescale
        y = out_buffer(M, N)
        say("gemv 7B down wide", kind, M)
        ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
        torch.cuda.synchronize()
        check_linear(y, x, W, None, M, f"gemv wide kind={kind} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
def test_gemv_deterministic(kind):
    rng = np.random.default_rng(4)
    N, K = 3584, 18944
    W = QFix(rng, N, K, kind, sd=0.02)
    x = torch.from_numpy(rng.standard_normal((4, K), dtype=np.float32)).cuda()
    ys = []
    for _ in range(3):
        y = torch.empty(4, N, device="cuda")
        ops.launch_gemv_batched_q(x, W.view, None, 4, K, N, y)
        ys.append(y)
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2])


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("T", [33, 256, 300])
def test_gemm_fp32(kind, T):
    rng = np.random.default_rng(500 + T)
    for N, K in ((640, 1536), (300, 896), (127, 130)):
        W = QFix(rng, N, K, kind, sd=0.02)
        x = rng.standard_normal((T, K), dtype=np.float32)
        bb, bd = bias_of(rng, N)
        y = out_buffer(T, N)
        say("gemm fp32", kind, T, N, K)
        ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, bd, T, K, N, y)
        torch.cuda.synchronize()
        check_linear(y, x, W, bb, T, f"gemm kind={kind} T={T} {N}x{K}")


@pytest.mark.parametrize("kind", [0, 1])
def test_gemm_fp32_precision(kind):
    """fp32 activations spanning six decades within each row: the fp16
    hi + lo operands (whole groups) and the three bf16 terms (ragged K) keep
    about 22 significant bits, so the error stays below 2^-19 of the
    conditioning sum -- a two-term bf16 split (about 16 bits) would not."""
    rng = np.random.default_rng(77 + kind)
    for T, N, K in ((96, 384, 3584), (520, 256, 1024), (40, 130, 130)):
        W = QFix(rng, N, K, kind, sd=0.02)
        x = (rng.standard_normal((T, K)) * 10.0 ** rng.uniform(-3, 3, (T, K))).astype(np.float32)
        y = out_buffer(T, N)
        say("gemm fp32 precision", kind, T, N, K)
        ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
        torch.cuda.synchronize()
        worst, _ = check_linear(y, x, W, None, T, f"gemm fp32 precision kind={kind} T={T} {N}x{K}")
        assert worst < 2.0 ** -19, (T, N, K, worst)


@pytest.mark.parametrize("kind", [0, 1])
def test_gemm_fp32_nonfinite_row(kind):
    """A row holding inf or NaN makes that row's outputs NaN; the other rows
    are unaffected (fp16 operand path: the row's factor is NaN)."""
    rng = np.random.default_rng(91 + kind)
    T, N, K = 70, 256, 1024
    W = QFix(rng, N, K, kind, sd=0.02)
    x = rng.standard_normal((T, K), dtype=np.float32)
    x[3, 17] = np.inf
    x[50, 900] = np.nan
    y = out_buffer(T, N)
    say("gemm fp32 non-finite", kind)
    ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()[: T * N].reshape(T, N)
    assert np.all(np.isnan(got[3])) and np.all(np.isnan(got[50]))
    keep = [m for m in range(T) if m not in (3, 50)]
    ref, cond = O.linear_dq_f64(x[keep], W.dq, None)
    err = np.abs(got[keep].astype(np.float64) - ref)
    assert float((err / np.maximum(cond, 1e-30)).max()) <= 5e-6


@pytest.mark.parametrize("kind", [0, 1])
def test_gemm_bf16x(kind):
    rng = np.random.default_rng(9)
    # (48, 700, 3584): 64-row tiles with K split over workgroups
    for T, N, K in ((1024, 512, 3584), (200, 384, 18944), (37, 130, 130), (48, 700, 3584)):
        W = QFix(rng, N, K, kind, sd=0.02)
        xb = O.seeded_bf16(rng, (T, K), 1.0)
        x = O.bf16_to_f32(xb)
        y = out_buffer(T, N)
        say("gemm bf16x", kind, T, N, K)
        ops.launch_gemm_bf16x(torch.from_numpy(xb.view(np.int16)).cuda(), W.view, None, T, K, N, y)
        torch.cuda.synchronize()
        check_linear(y, x, W, None, T, f"gemm bf16x kind={kind} T={T} {N}x{K}")


@pytest.mark.parametrize("kind", [0, 1])
def test_embedding_exact(kind):
    rng = np.random.default_rng(8)
    W = QFix(rng, 50, 256, kind)
    ids = np.array([0, 49, 7, 7], np.int64)
    out = torch.full((len(ids) * 256 + 16,), CANARY, device="cuda")
    say("embedding", kind)
    ops.launch_embedding_q(W.view, torch.from_numpy(ids).cuda(), len(ids), 256, out)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    ref = O.embedding(W.q, W.s, W.z, kind, 256, ids)
    assert np.array_equal(o[: ids.size * 256].reshape(len(ids), 256), ref)
    assert np.all(o[ids.size * 256:] == CANARY)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 3])
def test_gemv_multi_matches_oracle(kind, M):
    """q|k|v (and gate|up) in one call: each output equals the oracle."""
    rng = np.random.default_rng(31 + kind + M)
    K = 1536
    Ws = [QFix(rng, N, K, kind, sd=0.02) for N in (1536, 256, 256)]
    x = rng.standard_normal((M, K), dtype=np.float32)
    bb, bd = bias_of(rng, 256)
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("gemv multi", kind, M)
    ops.gemv_prep(torch.from_numpy(x).cuda(), M, K, kind)
    ops.gemv_prepped_multi([W.view for W in Ws], [None, bd, None], M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y) in enumerate(zip(Ws, ys)):
        check_linear(y, x, W, bb if i == 1 else None, M, f"multi[{i}] kind={kind} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 3])
def test_gemv_multi_direct(kind, M):
    """iq_gemv_multi: q|k|v at 1.5B and gate|up at 7B width, one call each."""
    rng = np.random.default_rng(131 + kind + M)
    for K, Ns in ((1536, (1536, 256, 256)), (3584, (18944, 18944))):
        Ws = [QFix(rng, N, K, kind, sd=0.02) for N in Ns]
        x = rng.standard_normal((M, K), dtype=np.float32)
        bb, bd = bias_of(rng, Ns[-1])
        ys = [out_buffer(M, W.rows) for W in Ws]
        say("gemv multi direct", kind, M, K, Ns)
        biases = [None] * (len(Ws) - 1) + [bd]
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], biases, M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y) in enumerate(zip(Ws, ys)):
            check_linear(y, x, W, bb if i == len(Ws) - 1 else None, M, f"multi direct[{i}] kind={kind} M={M} K={K}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [2, 3, 4, 5, 7, 8])
def test_gemv_few_rows_in_the_one_row_kernel(kind, M):
    """2..8 rows through the 1-row kernel (rows packed 4 limbs apart on one
    MFMA operand, two blocks of 4 past 4 rows, long K split into ranges):
    ragged N, a bias, the 7B gate|up width in one call, and an inf in one
    row leaving the other rows exact."""
    rng = np.random.default_rng(151 + kind + M)
    # K = 6144: int8 slices of 8 groups (the 8-group instance at 2..4 rows);
    # K = 18944: K split over several workgroups per tile + range reduction
    for K, Ns in ((3584, (1000, 37)), (3584, (18944, 18944)), (1536, (8960,)), (6144, (700,)), (18944, (3584,))):
        Ws = [QFix(rng, N, K, kind, sd=0.02) for N in Ns]
        x = rng.standard_normal((M, K), dtype=np.float32)
        bb, bd = bias_of(rng, Ns[0])
        ys = [out_buffer(M, W.rows) for W in Ws]
        say("gemv few rows", kind, M, K, Ns)
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], [bd] + [None] * (len(Ws) - 1), M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y) in enumerate(zip(Ws, ys)):
            check_linear(y, x, W, bb if i == 0 else None, M, f"few rows[{i}] kind={kind} M={M} K={K}")
    K, N = 3584, 512
    W = QFix(rng, N, K, kind, sd=0.02)
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[M - 1, 1000] = np.inf
    y = out_buffer(M, N)
    ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()[: M * N].reshape(M, N)
    assert not np.any(np.isfinite(got[M - 1]))
    ref, cond = O.linear_dq_f64(x[: M - 1], W.dq, None)
    err = np.abs(got[: M - 1].astype(np.float64) - ref)
    assert float((err / np.maximum(cond, 1e-30)).max()) <= 5e-6


@pytest.mark.parametrize("kind", [0, 1])
def test_gemv_unaligned_activation_row(kind):
    """1 row whose fp32 activations start 4 bytes past a 16-byte boundary."""
    rng = np.random.default_rng(61 + kind)
    N, K = 1000, 1536
    W = QFix(rng, N, K, kind, sd=0.02)
    x = rng.standard_normal((1, K), dtype=np.float32)
    buf = torch.zeros(K + 4, device="cuda")
    buf[1:K + 1] = torch.from_numpy(x[0]).cuda()
    xv = buf[1:K + 1]
    assert xv.data_ptr() % 16 == 4
    y = out_buffer(1, N)
    say("gemv unaligned x", kind)
    ops.launch_gemv_batched_q(xv, W.view, None, 1, K, N, y)
    torch.cuda.synchronize()
    check_linear(y, x, W, None, 1, f"unaligned x kind={kind}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("K", [3584, 18944])
def test_gemv_prep_keeps_its_input(kind, M, K):
    """A 1..4-row preparation holds the activations of the time of the call:
    overwriting x afterwards does not change what gemv_prepped computes."""
    rng = np.random.default_rng(71 + kind + M)
    N = 512
    W = QFix(rng, N, K, kind, sd=0.02)
    x = rng.standard_normal((M, K), dtype=np.float32)
    xd = torch.from_numpy(x).cuda()
    ops.gemv_prep(xd, M, K, kind)
    xd.fill_(1e30)
    y = out_buffer(M, N)
    say("gemv prep snapshot", kind, M)
    ops.gemv_prepped(W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    check_linear(y, x, W, None, M, f"prep snapshot kind={kind} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 4])
def test_gemv_nonfinite_activation(kind, M):
    """An inf / NaN activation makes every output of its row non-finite (as
    the reference's fp32 sum does); the other rows stay exact."""
    rng = np.random.default_rng(81 + kind + M)
    N, K = 256, 1536
    W = QFix(rng, N, K, kind, sd=0.02)
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[0, 300] = np.inf
    if M > 1:
        x[1, 5] = np.nan
    y = out_buffer(M, N)
    say("gemv nonfinite", kind, M)
    ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()[: M * N].reshape(M, N)
    bad = 2 if M > 1 else 1
    assert not np.any(np.isfinite(got[:bad]))
    if M > bad:
        ref, cond = O.linear_dq_f64(x[bad:], W.dq, None)
        err = np.abs(got[bad:].astype(np.float64) - ref)
        assert float((err / np.maximum(cond, 1e-30)).max()) <= 5e-6


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [2, 16, 17, 32])
def test_gemv_prepared_f16_split_tile_blocks(kind, M):
    """The prepare-once path (iq_gemv_prep + iq_gemv_prepped_multi) at 2..32
    rows runs the f16 hi/lo split kernel for every width: one, two and four
    16-row tiles per workgroup (224, 288 and 4096+ tiles per call), with a
    bias on one matrix and activations spanning several decades."""
    rng = np.random.default_rng(700 + 10 * kind + M)
    for K, Ns in ((3584, (3584,)), (1536, (4096, 256, 256)), (256, (65536,))):
        Ws = [QFix(rng, N, K, kind, sd=0.02) for N in Ns]
        x = rng.standard_normal((M, K), dtype=np.float32)
        x *= np.float32(10.0) ** rng.integers(-3, 3, size=(M, K)).astype(np.float32)
        bb, bd = bias_of(rng, Ns[0])
        ys = [out_buffer(M, W.rows) for W in Ws]
        say("gemv prepared f16 split", kind, M, K, Ns)
        ops.gemv_prep(torch.from_numpy(x).cuda(), M, K, kind)
        ops.gemv_prepped_multi([W.view for W in Ws], [bd] + [None] * (len(Ws) - 1), M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y) in enumerate(zip(Ws, ys)):
            check_linear(y, x, W, bb if i == 0 else None, M, f"prepared[{i}] kind={kind} M={M} K={K}")

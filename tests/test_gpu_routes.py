"""Parity of the kernel instances behind the benchmark's full-size numbers,
through the C ABI, against the oracle's float64 product over dequant()
(tests/test_ops_gpu.cu:664-692 semantics, same tolerances as
tests/gpu_util.check_linear), plus the workspace contract.

The matrices here are packed directly with random codes, scales and zero
points (any bytes are a valid packed matrix, src/quant.h:40-58), so the
full Qwen2.5-7B shapes need no host quantisation; outputs are checked on a
seeded sample of output features, with every row of the activation block.

Routes covered (dispatch in infer_amd/csrc/iq_gemm.hip / iq_gemv.hip):
  * prefill GEMM at T = 1024 on 18944 x 3584: 8 row tiles x 148 column
    tiles >= 2 x CUs, i.e. the 128 x 128 tile instance (NJ = 2, BM = 128),
    and on 3584 x 18944 (config 5's down, K = 18944), bf16 and fp32
    activations, int8 and int4;
  * gate|up (2 x 18944 x 3584) in one iq_gemv_multi call at 9, 12 and 16
    rows (int4 on gemvq: 32-row tiles on the 32 x 32 matrix instruction,
    both terms of all 16 rows in one operand; int8 on gemvr) and at 1 row;
  * the int8 lm_head 152064 x 3584 at 1, 5 and 16 rows, and wide calls
    (>= 4096 tiles) at 5..16 rows (gemvr at 5..6, gemvs at 7..16: operands
    shared through LDS over 8 tiles), both kinds, with ragged row counts and
    biases;
  * 17..32 rows on gemvq's two 16-row blocks (7B gate|up and down, ragged
    matrices, the fp32 GEMM entry);
  * gate|up and down at 5..8 rows and down at 9..16 take gemvr (a K range
    requested at once, the f16 split operands made from x inside the
    kernel), gate|up at 9..16 gemvq, with a non-finite activation in two
    rows;
  * every other 7B decode matrix at 16 rows;
  * every row count where the routing changes, on narrow, wide and long-K
    shapes, and every T where the prefill GEMM's choices change, both
    activation types.
"""
import numpy as np
import pytest
import torch

from infer_amd import ops
from oracle import oracle as O
from tests.gpu_util import CANARY, KGEMV_TOL, MAX_REL, out_buffer, say

pytestmark = pytest.mark.gpu


class Packed:
    """A random packed [rows x cols] matrix (codes, bf16 scales, u8 zeros)
    on the device, with its host copy for sampled dequantisation."""

    def __init__(self, rng, rows, cols, kind):
        G = O.groups(cols)
        self.kind, self.rows, self.cols = kind, rows, cols
        nq = rows * cols // 2 if kind == 1 else rows * cols
        if kind == 1:
            self.q = rng.integers(0, 256, nq, dtype=np.uint8)
            self.z = rng.integers(0, 16, (rows, G), dtype=np.uint8)
        else:
            # int8 codes -127..127 (src/quant.cpp:56-57 never writes -128)
            self.q = rng.integers(-127, 128, nq, dtype=np.int16).astype(np.int8).view(np.uint8)
            self.z = None
        self.s = O.f32_to_bf16(rng.uniform(2e-4, 8e-4, (rows, G)).astype(np.float32))
        self.view = ops.upload_q(kind, rows, cols, self.q, self.s, self.z)

    def dq_rows(self, idx):
        """dequant() of output features idx (src/quant.cpp:86-93)."""
        K = self.cols
        rb = K // 2 if self.kind == 1 else K
        q = self.q.reshape(self.rows, rb)[idx]
        z = None if self.z is None else self.z[idx]
        return O.dequant_matrix(q, self.s[idx], z, self.kind, len(idx), K)


def sample_rows(rng, N, n=192):
    """Sampled output features: both ends, a tile boundary and random ones."""
    idx = set(rng.choice(N, size=min(n, N), replace=False).tolist())
    idx.update([0, 1, 15, 16, N - 1, N - 17, N - 16])
    return np.array(sorted(i for i in idx if 0 <= i < N), np.int64)


def check_sampled(y_dev, x, W, T, rng, what, bias_bits=None):
    N = W.rows
    y = y_dev.detach().cpu().numpy().reshape(-1)
    got = y[: T * N].reshape(T, N)
    assert np.all(y[T * N:] == CANARY), f"{what}: wrote past y"
    idx = sample_rows(rng, N)
    ref, cond = O.linear_dq_f64(x[:T], W.dq_rows(idx), None if bias_bits is None else bias_bits[idx])
    g = got[:, idx].astype(np.float64)
    assert np.all(np.isfinite(g)), what
    err = np.abs(g - ref)
    worst = float((err / np.maximum(cond, 1e-30)).max())
    rel = float(err.max() / max(np.abs(ref).max(), 1e-30))
    say(f"  {what}: cond err {worst:.3g}, max rel {rel:.3g}")
    assert worst <= KGEMV_TOL, f"{what}: conditioning error {worst:.3g}"
    assert rel <= MAX_REL, f"{what}: max rel error {rel:.3g}"


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("xtype", ["bf16", "fp32"])
def test_prefill_gemm_t1024_wide(kind, xtype):
    """Config 5's gate/up shape (T = 1024, 18944 x 3584): the 128 x 128
    output-tile instance, chosen when row tiles x column tiles >= 2 x CUs."""
    rng = np.random.default_rng(1024 + kind + (10 if xtype == "fp32" else 0))
    T, N, K = 1024, 18944, 3584
    W = Packed(rng, N, K, kind)
    y = out_buffer(T, N)
    say("gemm T=1024 wide", kind, xtype)
    if xtype == "bf16":
        xb = O.seeded_bf16(rng, (T, K), 1.0)
        x = O.bf16_to_f32(xb)
        ops.launch_gemm_bf16x(torch.from_numpy(xb.view(np.int16)).cuda(), W.view, None, T, K, N, y)
    else:
        x = rng.standard_normal((T, K), dtype=np.float32)
        ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, T, rng, f"gemm T=1024 {xtype} kind={kind}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("xtype", ["bf16", "fp32"])
def test_prefill_gemm_t1024_down(kind, xtype):
    """Config 5's down shape at its own size: X[1024, 18944] times the
    3584 x 18944 matrix (148 groups per row), the instance the benchmark's
    down figure is measured on."""
    rng = np.random.default_rng(2048 + kind + (10 if xtype == "fp32" else 0))
    T, N, K = 1024, 3584, 18944
    W = Packed(rng, N, K, kind)
    y = out_buffer(T, N)
    say("gemm T=1024 down", kind, xtype)
    if xtype == "bf16":
        xb = O.seeded_bf16(rng, (T, K), 1.0)
        x = O.bf16_to_f32(xb)
        ops.launch_gemm_bf16x(torch.from_numpy(xb.view(np.int16)).cuda(), W.view, None, T, K, N, y)
    else:
        x = rng.standard_normal((T, K), dtype=np.float32)
        ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, T, rng, f"gemm T=1024 down {xtype} kind={kind}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 9, 12, 16])
def test_gate_up_7b_multi(kind, M):
    """gate|up of one 7B layer in one iq_gemv_multi call (2 x 18944 x 3584)."""
    rng = np.random.default_rng(900 + 20 * kind + M)
    K = 3584
    Ws = [Packed(rng, 18944, K, kind) for _ in range(2)]
    x = rng.standard_normal((M, K), dtype=np.float32)
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("gate|up 7B multi", kind, M)
    ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], None, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y) in enumerate(zip(Ws, ys)):
        check_sampled(y, x, W, M, rng, f"gate|up[{i}] kind={kind} M={M}")


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_one_row_two_tiles_per_workgroup(M):
    """int4 at 1..4 rows on a wide call (over 4 workgroups per CU, G = 24: six
    waves of 4 groups): two 16-row tiles per workgroup.  Matrices of 1025
    (ragged), 20, 3 and 1 tiles in one call with biases: tile pairs that
    straddle two matrices, and an odd tile count, so the last workgroup's
    second tile is past every matrix."""
    rng = np.random.default_rng(2525 + M)
    K = 3072
    Ws = [Packed(rng, N, K, 1) for N in (16389, 309, 48, 5)]
    bias_bits = [O.seeded_bf16(rng, (W.rows,), 0.5) for W in Ws]
    bias = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
    x = rng.standard_normal((M, K), dtype=np.float32)
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("two tiles per workgroup", M)
    ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bias, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y, bb) in enumerate(zip(Ws, ys, bias_bits)):
        check_sampled(y, x, W, M, rng, f"two tiles[{i}] M={M}", bias_bits=bb)


@pytest.mark.parametrize("kind", [0, 1])
def test_one_row_short_tiles(kind):
    """1 row on fewer 16-row tiles than CUs: tiles of 8..15 rows, one per
    workgroup.  Ragged matrices in one call with biases (1530 + 250 + 250
    rows, K = 1536: 8-row tiles), 7B down alone (3584 x 18944: 14-row
    tiles) and 1.5B down (1536 x 8960, 70 groups: per-group metadata loads,
    8-row tiles)."""
    rng = np.random.default_rng(1414 + kind)
    for K, Ns in ((1536, (1530, 250, 250)), (18944, (3584,)), (8960, (1536,))):
        Ws = [Packed(rng, N, K, kind) for N in Ns]
        bias_bits = [O.seeded_bf16(rng, (W.rows,), 0.5) for W in Ws]
        bias = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
        x = rng.standard_normal((1, K), dtype=np.float32)
        ys = [out_buffer(1, W.rows) for W in Ws]
        say("1 row, short tiles", kind, K, Ns)
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bias, 1, K, ys)
        torch.cuda.synchronize()
        for i, (W, y, bb) in enumerate(zip(Ws, ys, bias_bits)):
            check_sampled(y, x, W, 1, rng, f"short tiles[{i}] K={K} kind={kind}", bias_bits=bb)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [9, 16])
def test_qkv_7b_multi_gemvh(kind, M):
    """q|k|v of one 7B layer (3584 + 512 + 512 rows x 3584, 288 tiles) in
    one iq_gemv_multi call at 9..16 rows: the preparation launch and gemvh
    on two tiles per workgroup, two groups in flight per wave."""
    rng = np.random.default_rng(4600 + 20 * kind + M)
    K = 3584
    Ws = [Packed(rng, n, K, kind) for n in (3584, 512, 512)]
    x = rng.standard_normal((M, K), dtype=np.float32)
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("q|k|v 7B multi gemvh", kind, M)
    ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], None, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y) in enumerate(zip(Ws, ys)):
        check_sampled(y, x, W, M, rng, f"q|k|v[{i}] kind={kind} M={M}")


@pytest.mark.parametrize("M", [1, 3, 4, 5, 9, 16])
def test_lm_head_int8(M):
    """The int8 lm_head 152064 x 3584 (9504 tiles)."""
    rng = np.random.default_rng(152064 + M)
    N, K = 152064, 3584
    W = Packed(rng, N, K, 0)
    x = rng.standard_normal((M, K), dtype=np.float32)
    y = out_buffer(M, N)
    say("lm_head int8", M)
    ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, M, rng, f"lm_head M={M}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [5, 7, 8, 9, 10, 11, 13, 16])
def test_wide_call_5_to_16_rows(kind, M):
    """Over 4096 16-row tiles (here 65541 rows, the last tile ragged, and a
    second matrix in the same call) at 5..16 rows: the gemvr route on the
    packed hi/lo operands (5..6 rows), the gemvs route on 16-row operand
    blocks (int8 at 7..16) and gemvq straight from x (int4 at 7..16)."""
    rng = np.random.default_rng(4096 + 10 * M + kind)
    K = 1024
    Ws = [Packed(rng, 65541, K, kind), Packed(rng, 300, K, kind)]
    bias_bits = [O.seeded_bf16(rng, (W.rows,), 0.5) for W in Ws]
    bias = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
    x = rng.standard_normal((M, K), dtype=np.float32)
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("wide 9..16 rows", kind, M)
    ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bias, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y, bb) in enumerate(zip(Ws, ys, bias_bits)):
        check_sampled(y, x, W, M, rng, f"wide[{i}] kind={kind} M={M}", bias_bits=bb)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [9, 16])
def test_gemvq_ragged_matrices(kind, M):
    """gemvq (int4; int8 takes gemvr) at 1024..4095 16-row tiles and 9..16
    rows, on matrices whose rows are not a multiple of 32: 20005 + 309 + 48 rows in one call, with
    biases, so the 32-row tiles of the second and third matrix start inside
    the first one's last 16-row tile pair and the split-K partials of each
    land in the 16-row tile order of the reduction."""
    rng = np.random.default_rng(3232 + 10 * M + kind)
    K = 1024
    Ws = [Packed(rng, N, K, kind) for N in (20005, 309, 48)]
    bias_bits = [O.seeded_bf16(rng, (W.rows,), 0.5) for W in Ws]
    bias = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
    x = rng.standard_normal((M, K), dtype=np.float32)
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("gemvq ragged", kind, M)
    ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bias, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y, bb) in enumerate(zip(Ws, ys, bias_bits)):
        check_sampled(y, x, W, M, rng, f"gemvq[{i}] kind={kind} M={M}", bias_bits=bb)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [17, 24, 32])
def test_gemvq_two_row_blocks(kind, M):
    """17..32 rows on gemvq's two 16-row blocks: 7B gate|up (one call),
    down (K = 18944) and q|k|v (a narrow call of three matrices) with
    biases, ragged matrices (20005 + 309 + 48 rows, K = 1024) in one call,
    and the fp32 GEMM entry (iq_gemm) on 7B gate."""
    rng = np.random.default_rng(1732 + 10 * M + kind)
    cases = ((3584, (18944, 18944)), (18944, (3584,)), (3584, (3584, 512, 512)), (1024, (20005, 309, 48)))
    for K, Ns in cases:
        Ws = [Packed(rng, N, K, kind) for N in Ns]
        x = rng.standard_normal((M, K), dtype=np.float32)
        bias_bits = [O.seeded_bf16(rng, (N,), 0.5) for N in Ns]
        bds = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
        ys = [out_buffer(M, W.rows) for W in Ws]
        say("gemvq two blocks", kind, M, K, Ns)
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bds, M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y) in enumerate(zip(Ws, ys)):
            check_sampled(y, x, W, M, rng, f"gemvq M={M} K={K} N={Ns[i]} kind={kind}", bias_bits[i])
    K, N = 3584, 18944
    W = Packed(rng, N, K, kind)
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[M - 1, 77] = np.inf
    y = out_buffer(M, N)
    say("gemvq via iq_gemm", kind, M)
    ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    got = y.detach().cpu().numpy().reshape(-1)[: M * N].reshape(M, N)
    assert not np.any(np.isfinite(got[M - 1])), "finite output in the non-finite row"
    check_sampled(y[: (M - 1) * N].contiguous(), x[: M - 1], W, M - 1, rng, f"iq_gemm M={M} kind={kind}")


@pytest.mark.parametrize("kind", [0, 1])
def test_route_boundaries(kind):
    """Every row count where the GEMV routing changes (1..9, 12, 16, 17,
    24, 31, 32) on three shapes that fall on different sides of the width
    and K thresholds: narrow and ragged (3000 x 2048), wide (20000 x 1024,
    >= 1024 tiles) and long rows (1024 x 16512, G = 129 >= 128), with a
    bias, and 17..32 rows on either side of the 224-tile threshold (3568 and
    3570 x 2048: 223 and 224 tiles), against the oracle."""
    rng = np.random.default_rng(5150 + kind)
    every = (1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 24, 31, 32)
    for N, K, Ms in ((3000, 2048, every), (20000, 1024, every), (1024, 16512, every),
                     (3568, 2048, (17, 32)), (3570, 2048, (17, 32))):
        W = Packed(rng, N, K, kind)
        bb = O.seeded_bf16(rng, (N,), 0.5)
        bd = torch.from_numpy(bb.view(np.int16)).cuda()
        for M in Ms:
            x = rng.standard_normal((M, K), dtype=np.float32)
            y = out_buffer(M, N)
            say("route boundaries", kind, N, K, M)
            ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, bd, M, K, N, y)
            torch.cuda.synchronize()
            check_sampled(y, x, W, M, rng, f"boundaries {N}x{K} M={M} kind={kind}", bias_bits=bb)


@pytest.mark.parametrize("kind", [0, 1])
def test_gemm_t_boundaries(kind):
    """iq_gemm (fp32 activations) and iq_gemm_bf16x across the T where the
    GEMM's choices change (gemvq's row blocks at 17..32 on wide matrices,
    the in-kernel split up to 32, the prepared fp16 operands past it, 64-,
    128- and 256-row tiles, split K): 17, 32, 33, 64, 65, 128, 129, 256,
    257 and 520 rows on a wide (20000 x 1024) and a narrow ragged (3000 x
    2048) matrix, 65..257 on a small one (520 x 3584, under 2^22 weights),
    257 and 600 on a smaller one (250 x 1536, under 2^19), 2048 on a
    narrow one (3000 x 1024: 128-wide tiles by the round count, on 256-row
    tiles for int4 with bf16 activations),
    17..257 on long rows (1024 x 16512), against the oracle."""
    rng = np.random.default_rng(6160 + kind)
    for N, K, Ts in ((20000, 1024, (17, 32, 33, 64, 65, 128, 129, 256, 257, 520)),
                     (3000, 2048, (17, 32, 33, 64, 65, 128, 129, 256, 257, 520)),
                     (520, 3584, (65, 200, 256, 257)),
                     (250, 1536, (257, 600)),
                     (3000, 1024, (2048,)),
                     (1024, 16512, (17, 32, 33, 64, 129, 257))):
        W = Packed(rng, N, K, kind)
        for T in Ts:
            x = rng.standard_normal((T, K), dtype=np.float32)
            say("gemm T boundaries", kind, N, K, T)
            y = out_buffer(T, N)
            ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
            torch.cuda.synchronize()
            check_sampled(y, x, W, T, rng, f"iq_gemm {N}x{K} T={T} kind={kind}")
            xb = O.f32_to_bf16(x)
            y = out_buffer(T, N)
            ops.launch_gemm_bf16x(torch.from_numpy(xb.view(np.int16)).cuda(), W.view, None, T, K, N, y)
            torch.cuda.synchronize()
            check_sampled(y, O.bf16_to_f32(xb), W, T, rng, f"iq_gemm_bf16x {N}x{K} T={T} kind={kind}")


@pytest.mark.parametrize("kind", [0, 1])
def test_gemm_three_k_ranges(kind):
    """Tiles that fill half to two thirds of one round of workgroup slots,
    or one to 2.5 rounds, on rows of >= 24 groups, take three K ranges: 7B
    gate (18944 x 3584) at T = 65, 128 and 256, and a ragged 18000 x 3072
    at T = 100 and 250, both activation types."""
    rng = np.random.default_rng(6565 + kind)
    for N, K, Ts in ((18944, 3584, (65, 128, 256)), (18000, 3072, (100, 250))):
        W = Packed(rng, N, K, kind)
        for T in Ts:
            x = rng.standard_normal((T, K), dtype=np.float32)
            say("gemm three K ranges", kind, N, K, T)
            y = out_buffer(T, N)
            ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, None, T, K, N, y)
            torch.cuda.synchronize()
            check_sampled(y, x, W, T, rng, f"iq_gemm {N}x{K} T={T} kind={kind}")
            xb = O.f32_to_bf16(x)
            y = out_buffer(T, N)
            ops.launch_gemm_bf16x(torch.from_numpy(xb.view(np.int16)).cuda(), W.view, None, T, K, N, y)
            torch.cuda.synchronize()
            check_sampled(y, O.bf16_to_f32(xb), W, T, rng, f"iq_gemm_bf16x {N}x{K} T={T} kind={kind}")


@pytest.mark.parametrize("kind", [0, 1])
def test_random_shapes_across_routes(kind):
    """A seeded sweep over the routing space: 24 random (rows, columns,
    activation rows) with whole-group or ragged K, one to three matrices
    per call below 33 rows (iq_gemv_multi) and the GEMM past it, with
    biases, on sampled output rows against the oracle."""
    rng = np.random.default_rng(8800 + kind)
    for case in range(24):
        G = int(rng.integers(1, 160))
        K = 128 * G if rng.random() < 0.8 else 128 * G + 2 * int(rng.integers(1, 63))
        N = int(rng.integers(1, 40000 if K <= 4096 else 6000))
        M = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 32, 33, 64, 65, 128, 200]))
        if M > 32:
            W = Packed(rng, N, K, kind)
            x = rng.standard_normal((M, K), dtype=np.float32)
            bb = O.seeded_bf16(rng, (N,), 0.5)
            y = out_buffer(M, N)
            say("random shapes", kind, case, N, K, M)
            ops.launch_gemm_tiled_q(torch.from_numpy(x).cuda(), W.view, torch.from_numpy(bb.view(np.int16)).cuda(),
                                    M, K, N, y)
            torch.cuda.synchronize()
            check_sampled(y, x, W, M, rng, f"random gemm {N}x{K} M={M} kind={kind}", bias_bits=bb)
            continue
        n = int(rng.integers(1, 4))
        Ns = [N] + [int(rng.integers(1, 5000)) for _ in range(n - 1)]
        Ws = [Packed(rng, Ni, K, kind) for Ni in Ns]
        bias_bits = [O.seeded_bf16(rng, (Ni,), 0.5) for Ni in Ns]
        bias = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
        x = rng.standard_normal((M, K), dtype=np.float32)
        ys = [out_buffer(M, Ni) for Ni in Ns]
        say("random shapes", kind, case, Ns, K, M)
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bias, M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y, bb) in enumerate(zip(Ws, ys, bias_bits)):
            check_sampled(y, x, W, M, rng, f"random {Ns[i]}x{K} M={M} kind={kind} [{i}]", bias_bits=bb)


def test_gemvq_looped_k_ranges():
    """gemvq where one K range per workgroup would need more partial sums
    than the workspace holds, so each workgroup loops over several ranges:
    the int8 lm_head at 32 rows (per-stream workspace) and int4 7B gate at
    32 rows through iq_gemv_noalloc (the static array's smaller capacity)."""
    rng = np.random.default_rng(3232032)
    M, K = 32, 3584
    W = Packed(rng, 152064, K, 0)
    x = rng.standard_normal((M, K), dtype=np.float32)
    y = out_buffer(M, W.rows)
    say("gemvq looped: lm_head int8", M)
    ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, W.rows, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, M, rng, "looped lm_head int8 M=32")
    del W
    W = Packed(rng, 18944, K, 1)
    y = out_buffer(M, W.rows)
    say("gemvq looped: noalloc int4 gate", M)
    ops.gemv_noalloc(torch.from_numpy(x).cuda(), W.view, None, M, K, W.rows, y)
    torch.cuda.synchronize()
    check_sampled(y, x, W, M, rng, "looped noalloc int4 gate M=32")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [6, 12])
def test_in_kernel_operands_unaligned_x(kind, M):
    """gemvr (6 rows) and gemvq (12 rows), which read fp32 x themselves, on
    an activation block that starts 4 bytes past a 16-byte boundary (7B
    gate|up in one call)."""
    rng = np.random.default_rng(4444 + 10 * M + kind)
    K = 3584
    Ws = [Packed(rng, 18944, K, kind) for _ in range(2)]
    x = rng.standard_normal((M, K), dtype=np.float32)
    buf = torch.zeros(M * K + 4, dtype=torch.float32, device="cuda")
    xd = buf[1:1 + M * K]
    xd.copy_(torch.from_numpy(x.reshape(-1)).cuda())
    assert xd.data_ptr() % 16 == 4
    ys = [out_buffer(M, W.rows) for W in Ws]
    say("in-kernel operands, unaligned x", kind, M)
    ops.gemv_multi(xd, [W.view for W in Ws], None, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y) in enumerate(zip(Ws, ys)):
        check_sampled(y, x, W, M, rng, f"unaligned x [{i}] kind={kind} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [6, 12])
def test_gemvr_nonfinite_rows(kind, M):
    """gemvr (7B gate|up and down shapes at 6 and 12 rows): an inf in row 0
    and a NaN in row 1 make every output of those rows non-finite; the
    other rows match the oracle."""
    rng = np.random.default_rng(7100 + 10 * M + kind)
    for K, Ns in ((3584, (18944, 18944)), (18944, (3584,))):
        Ws = [Packed(rng, N, K, kind) for N in Ns]
        x = rng.standard_normal((M, K), dtype=np.float32)
        x[0, K - 3] = np.inf
        x[1, 200] = np.nan
        ys = [out_buffer(M, W.rows) for W in Ws]
        say("gemvr non-finite rows", kind, M, K, Ns)
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], None, M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y) in enumerate(zip(Ws, ys)):
            got = y.detach().cpu().numpy().reshape(-1)[: M * W.rows].reshape(M, W.rows)
            assert not np.any(np.isfinite(got[:2])), f"gemvr[{i}] K={K}: finite output in a non-finite row"
            check_sampled(y[2 * W.rows:], x[2:], W, M - 2, rng,
                          f"gemvr[{i}] K={K} kind={kind} M={M} rows 2..")


@pytest.mark.parametrize("kind", [0, 1])
def test_decode_set_7b_16_rows(kind):
    """The remaining 7B decode calls at 16 rows: q|k|v (one call, biases),
    o, and down (K = 18944)."""
    rng = np.random.default_rng(716 + kind)
    M = 16
    for K, Ns in ((3584, (3584, 512, 512)), (3584, (3584,)), (18944, (3584,))):
        Ws = [Packed(rng, N, K, kind) for N in Ns]
        x = rng.standard_normal((M, K), dtype=np.float32)
        bias_bits = [O.seeded_bf16(rng, (N,), 0.5) for N in Ns]
        bds = [torch.from_numpy(b.view(np.int16)).cuda() for b in bias_bits]
        ys = [out_buffer(M, W.rows) for W in Ws]
        say("7B decode set 16 rows", kind, K, Ns)
        ops.gemv_multi(torch.from_numpy(x).cuda(), [W.view for W in Ws], bds, M, K, ys)
        torch.cuda.synchronize()
        for i, (W, y) in enumerate(zip(Ws, ys)):
            check_sampled(y, x, W, M, rng, f"7B K={K} N={Ns[i]} kind={kind}", bias_bits[i])


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [8, 16])
def test_direct_call_never_leaves_a_stale_preparation(kind, M):
    """After gemv_prep(x1), a direct GEMV on x2 either leaves the preparation
    intact (8 rows on a narrow matrix run in the 1-row kernel, which reads x2
    itself) or overwrites its buffers, in which case iq_gemv_prepped must
    fail with IQ_ESHAPE (16 rows: the conversion launch reuses them).  It
    never multiplies x2 in place of x1.  A fresh preparation works again."""
    rng = np.random.default_rng(55 + kind + M)
    K, N = 3584, 3584
    W = Packed(rng, N, K, kind)
    x1 = rng.standard_normal((M, K), dtype=np.float32)
    x2 = rng.standard_normal((M, K), dtype=np.float32)
    y = out_buffer(M, N)
    say("prep invalidation", kind, M)
    ops.gemv_prep(torch.from_numpy(x1).cuda(), M, K, kind)
    ops.gemv_multi(torch.from_numpy(x2).cuda(), [W.view], None, M, K, [y])
    if M == 16:
        with pytest.raises(RuntimeError, match="shape"):
            ops.gemv_prepped(W.view, None, M, K, N, y)
        ops.gemv_prep(torch.from_numpy(x1).cuda(), M, K, kind)
    y = out_buffer(M, N)
    ops.gemv_prepped(W.view, None, M, K, N, y)
    torch.cuda.synchronize()
    check_sampled(y, x1, W, M, rng, f"prepared x1 kind={kind} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
def test_two_streams_have_separate_workspaces(kind):
    """Preparations on two streams do not disturb each other: each stream's
    iq_gemv_prepped multiplies that stream's activations."""
    rng = np.random.default_rng(77 + kind)
    M, K, N = 12, 3584, 4096
    W = Packed(rng, N, K, kind)
    xs = [rng.standard_normal((M, K), dtype=np.float32) for _ in range(2)]
    xd = [torch.from_numpy(x).cuda() for x in xs]
    ys = [out_buffer(M, N) for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        ops.init(0, s)
    torch.cuda.synchronize()
    say("two streams", kind)
    ops.gemv_prep(xd[0], M, K, kind, stream=streams[0])
    ops.gemv_prep(xd[1], M, K, kind, stream=streams[1])
    ops.gemv_prepped(W.view, None, M, K, N, ys[1], stream=streams[1])
    ops.gemv_prepped(W.view, None, M, K, N, ys[0], stream=streams[0])
    torch.cuda.synchronize()
    for i in range(2):
        check_sampled(ys[i], xs[i], W, M, rng, f"stream {i} kind={kind}")

"""Outlier activation channels through every activation format of the GEMV.

LLM residual streams and MLP inputs carry a few "massive" channels, 10^3 to
10^5 x the typical magnitude.  Here every 128-column group holds one such
channel (at a random column of the group), and a block of output rows has
weight 0 on it (int8 code 0, int4 code = the group's zero point), so for
those rows the product is made entirely of the typical values while each
group's fixed-point scale is set by the outlier.  The check is the
reference's: |y - ref| <= 5e-6 sum |w x| (tests/test_ops_gpu.cu:199-206),
against the oracle's float64 product over dequant(), on every zero-weight
row and a sample of the others.

Covered: the 1-row kernel (1 row; 2..4 rows with and without the K split;
5..8 rows), the prepared byte-limb kernels (gemvt, gemvb on ragged K), the
f16 split kernels (gemvh, gemvr, gemvq), iq_gemv_multi, iq_gemv_prep /
iq_gemv_prepped, iq_gemv_noalloc and a chain stage (plain and RMSNorm
inputs)."""
import numpy as np
import pytest
import torch

from infer_amd import chain as C
from infer_amd import ops
from oracle import oracle as O
from tests.gpu_util import CANARY, KGEMV_TOL, MAX_REL, out_buffer, say

pytestmark = pytest.mark.gpu

NZERO = 24  # output rows [0, NZERO) have weight 0 on every outlier channel


class OutlierMat:
    """Oracle-quantised seeded weights whose first NZERO rows dequantise to
    exactly 0 on the outlier column of every group."""

    def __init__(self, rng, rows, cols, kind, ocol):
        self.kind, self.rows, self.cols = kind, rows, cols
        G = O.groups(cols)
        w = O.seeded_bf16(rng, (rows, cols), 0.02)
        q, s, z = O.quantize(w, kind)
        q = q.copy()
        cols_o = np.arange(G) * 128 + ocol
        cols_o = cols_o[cols_o < cols]
        if kind == 1:
            qb = q.reshape(rows, cols // 2)
            for r in range(NZERO):
                for c in cols_o:
                    b, zp = qb[r, c // 2], int(z[r, c // 128])
                    qb[r, c // 2] = (b & 0xF0) | zp if c % 2 == 0 else (b & 0x0F) | (zp << 4)
        else:
            q.reshape(rows, cols)[:NZERO, cols_o] = 0
        self.q, self.s, self.z = q, s, z
        self.view = ops.upload_q(kind, rows, cols, q, s, z)

    def dq_rows(self, idx):
        rb = self.cols // 2 if self.kind == 1 else self.cols
        q = self.q.reshape(self.rows, rb)[idx]
        z = None if self.z is None else self.z[idx]
        return O.dequant_matrix(q, self.s[idx], z, self.kind, len(idx), self.cols)


def outlier_x(rng, M, K, ocol, mag):
    x = rng.standard_normal((M, K), dtype=np.float32)
    cols = np.arange(0, K, 128) + ocol
    cols = cols[cols < K]
    sign = np.where(rng.random((M, len(cols))) < 0.5, -1.0, 1.0).astype(np.float32)
    x[:, cols] = np.float32(mag) * sign * (1.0 + 0.25 * rng.random((M, len(cols)), dtype=np.float32))
    return x


def rows_to_check(rng, N):
    idx = set(range(NZERO)) | set(rng.choice(N, size=min(64, N), replace=False).tolist()) | {N - 1}
    return np.array(sorted(idx), np.int64)


def check(y_dev, x, W, M, rng, what):
    N = W.rows
    y = y_dev.detach().cpu().numpy().reshape(-1)
    assert np.all(y[M * N:] == CANARY), f"{what}: wrote past y"
    got = y[: M * N].reshape(M, N)
    idx = rows_to_check(rng, N)
    ref, cond = O.linear_dq_f64(x[:M], W.dq_rows(idx))
    g = got[:, idx].astype(np.float64)
    assert np.all(np.isfinite(g)), what
    err = np.abs(g - ref)
    worst = float((err / np.maximum(cond, 1e-30)).max())
    zero_rows = float((err[:, :NZERO] / np.maximum(cond[:, :NZERO], 1e-30)).max())
    rel = float(err.max() / max(np.abs(ref).max(), 1e-30))
    say(f"  {what}: cond err {worst:.3g} (zero-weight rows {zero_rows:.3g}), max rel {rel:.3g}")
    assert worst <= KGEMV_TOL, f"{what}: conditioning error {worst:.3g}"
    assert rel <= MAX_REL, f"{what}: max rel error {rel:.3g}"


# (rows, cols): a narrow tile count (1-row kernel at 1..8 rows), a wide
# one (gemvt / gemvq / gemvr territory), long K (the 1-row kernel's 148-group
# row, the 2..4-row K split) and ragged K (gemvb)
SHAPES = [(512, 3584), (18944, 3584), (256, 18944), (384, 1000)]


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 12, 16, 32])
def test_gemv_outlier_channels(kind, shape, M):
    N, K = shape
    if kind == 1 and K % 2:
        pytest.skip("int4 needs an even K")
    rng = np.random.default_rng(31 * M + 7 * kind + N + K)
    ocol = int(rng.integers(0, 128))
    W = OutlierMat(rng, N, K, kind, ocol)
    for mag in (1e3, 1e4, 1e5):
        x = outlier_x(rng, M, K, ocol, mag)
        y = out_buffer(M, N)
        say("gemv outliers", kind, N, K, M, mag)
        ops.launch_gemv_batched_q(torch.from_numpy(x).cuda(), W.view, None, M, K, N, y)
        torch.cuda.synchronize()
        check(y, x, W, M, rng, f"kind={kind} {N}x{K} M={M} outlier {mag:g}")


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_multi_prepped_noalloc_outliers(kind, M):
    """q|k|v-shaped iq_gemv_multi, iq_gemv_prep + iq_gemv_prepped_multi and
    iq_gemv_noalloc on the same outlier activations."""
    rng = np.random.default_rng(500 + 10 * kind + M)
    K = 3584
    ocol = int(rng.integers(0, 128))
    Ws = [OutlierMat(rng, n, K, kind, ocol) for n in (3584, 512, 512)]
    x = outlier_x(rng, M, K, ocol, 1e5)
    xd = torch.from_numpy(x).cuda()
    say("multi / prepped / noalloc outliers", kind, M)
    ys = [out_buffer(M, W.rows) for W in Ws]
    ops.gemv_multi(xd, [W.view for W in Ws], None, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y) in enumerate(zip(Ws, ys)):
        check(y, x, W, M, rng, f"multi[{i}] kind={kind} M={M}")
    ys = [out_buffer(M, W.rows) for W in Ws]
    ops.gemv_prep(xd, M, K, kind)
    ops.gemv_prepped_multi([W.view for W in Ws], None, M, K, ys)
    torch.cuda.synchronize()
    for i, (W, y) in enumerate(zip(Ws, ys)):
        check(y, x, W, M, rng, f"prepped[{i}] kind={kind} M={M}")
    y = out_buffer(M, Ws[0].rows)
    ops.gemv_noalloc(xd, Ws[0].view, None, M, K, Ws[0].rows, y)
    torch.cuda.synchronize()
    check(y, x, Ws[0], M, rng, f"noalloc kind={kind} M={M}")


@pytest.mark.parametrize("kind", [0, 1])
def test_chain_stage_outliers(kind):
    """One chain stage with a plain input and one with an RMSNorm input
    (the norm weights 1.0, so the normalised vector keeps the outliers)."""
    rng = np.random.default_rng(77 + kind)
    K, N = 3584, 4096
    ocol = int(rng.integers(0, 128))
    W = OutlierMat(rng, N, K, kind, ocol)
    x = outlier_x(rng, 1, K, ocol, 1e5)[0]
    xd = torch.from_numpy(x).cuda()
    ones = torch.from_numpy(np.full(K, 0x3F80, np.uint16).view(np.int16)).cuda()
    for in_op in (C.IN_PLAIN, C.IN_RMSNORM):
        y = out_buffer(1, N)
        say("chain stage outliers", kind, in_op)
        ch = C.Chain([C.Stage([W.view], xd, [y], in_op, C.OUT_STORE, norm=ones if in_op else None, eps=1e-6)])
        ch.run()
        torch.cuda.synchronize()
        ch.close()
        xin = x.astype(np.float64)
        if in_op == C.IN_RMSNORM:
            xin = O.rmsnorm_f64(xin, np.full(K, 0x3F80, np.uint16), 1e-6)
        check(y, xin[None, :], W, 1, rng, f"chain stage kind={kind} in_op={in_op}")

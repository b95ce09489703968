"""Helpers shared by the GPU parity tests (seeded inputs, oracle references)."""
import sys

import numpy as np
import torch

from infer_amd import ops
from oracle import oracle as O

CANARY = -12345.5  # tests/test_ops_gpu.cu:131-132
KGEMV_TOL = 5e-6   # tests/test_ops_gpu.cu:206
MAX_REL = 1e-3     # max |y - ref| / max |ref|


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class QFix:
    """tests/test_ops_gpu.cu:641-662: a matrix quantised by the (oracle)
    quantiser, uploaded, plus its dequantised host copy."""

    def __init__(self, rng, rows, cols, kind, sd=0.05):
        self.kind = kind
        self.rows, self.cols = rows, cols
        self.w = O.seeded_bf16(rng, (rows, cols), sd)
        self.q, self.s, self.z = O.quantize(self.w, kind)
        self.view = ops.upload_q(kind, rows, cols, self.q, self.s, self.z)
        self._dq = None

    @property
    def dq(self):
        if self._dq is None:
            self._dq = O.dequant_matrix(self.q, self.s, self.z, self.kind, self.rows, self.cols)
        return self._dq


def check_linear(y_dev, x, W, bias_bits, T, what):
    """Reference check of a [T, out] result against float64 over dequant()."""
    y = y_dev.detach().cpu().numpy().reshape(-1)
    N = W.rows
    got = y[: T * N].reshape(T, N)
    ref, cond = O.linear_dq_f64(x[:T], W.dq, bias_bits)
    err = np.abs(got.astype(np.float64) - ref)
    worst_cond = float((err / np.maximum(cond, 1e-30)).max())
    max_rel = float(err.max() / max(np.abs(ref).max(), 1e-30))
    assert np.all(np.isfinite(got)), what
    assert worst_cond <= KGEMV_TOL, f"{what}: conditioning error {worst_cond:.3g}"
    assert max_rel <= MAX_REL, f"{what}: max rel error {max_rel:.3g}"
    tail = y[T * N:]
    assert np.all(tail == CANARY), f"{what}: wrote past y"
    return worst_cond, max_rel


def out_buffer(T, N, extra_rows=0):
    n = (T + extra_rows) * N + 16
    return torch.full((n,), CANARY, dtype=torch.float32, device="cuda")


def bias_of(rng, N):
    bits = O.seeded_bf16(rng, (N,), 0.5)
    return bits, torch.from_numpy(bits.view(np.int16)).cuda()

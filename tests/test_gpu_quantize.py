"""On-device quantize + pack (iq_quantize) is bit-exact to the reference's
llm::quantize (src/quant.cpp:34-84): against the fixtures written by the
reference's own compiled quantiser, and against the pinned oracle on random
and full Qwen2.5-7B shapes."""
import os

import numpy as np
import pytest
import torch

from infer_amd import ops
from oracle import oracle as O
from tests.gpu_util import say

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


def gpu_quantize(w_bits, kind):
    rows, cols = w_bits.shape
    if isinstance(w_bits, torch.Tensor):
        w = w_bits.cuda()
    else:
        w = torch.from_numpy(np.ascontiguousarray(w_bits).view(np.int16)).cuda()
    v = ops.quantize(w, kind)
    torch.cuda.synchronize()
    q = v.q.cpu().numpy()
    s = v.scales.cpu().numpy().view(np.uint16).reshape(rows, -1)
    z = v.zeros.cpu().numpy().reshape(rows, -1) if kind == 1 else None
    return q, s, z


def test_quantize_matches_reference_fixtures():
    g = np.load(GOLD, allow_pickle=False)
    keys = sorted({k.rsplit("_", 1)[0] for k in g.files})
    for key in keys:
        kind = 0 if key.startswith("int8") else 1
        say("quantize fixture", key)
        q, s, z = gpu_quantize(g[key + "_w"], kind)
        assert np.array_equal(q, g[key + "_q"]), key
        assert np.array_equal(s, g[key + "_s"]), key
        if kind == 1:
            assert np.array_equal(z, g[key + "_z"]), key


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("shape", [(1, 2), (3, 130), (7, 254), (64, 1536), (33, 8960), (5, 1000)])
def test_quantize_random_vs_oracle(kind, shape):
    rng = np.random.default_rng(100 + shape[1] + kind)
    w = O.seeded_bf16(rng, shape, 0.05)
    # sprinkle exact-tie and zero groups
    w[0, : min(shape[1], 128)] = O.f32_to_bf16(np.zeros(min(shape[1], 128), np.float32))
    say("quantize random", kind, shape)
    q, s, z = gpu_quantize(w, kind)
    rq, rs, rz = O.quantize(w, kind)
    assert np.array_equal(q, rq)
    assert np.array_equal(s, rs)
    if kind == 1:
        assert np.array_equal(z, rz)


@pytest.mark.parametrize("kind", [0, 1])
def test_quantize_7b_shapes_bit_exact(kind):
    """Full 7B matrices: gate/up 18944x3584 and down 3584x18944, plus q/k."""
    for i, (rows, cols) in enumerate([(18944, 3584), (3584, 18944), (512, 3584)]):
        gen = torch.Generator(device="cuda").manual_seed(1234 + i)
        w = (torch.randn(rows, cols, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
        say("quantize 7B", kind, rows, cols)
        q, s, z = gpu_quantize(w.view(torch.int16), kind)
        wb = w.view(torch.int16).cpu().numpy().view(np.uint16)
        rq, rs, rz = O.quantize(wb, kind)
        assert np.array_equal(s, rs)
        assert np.array_equal(q, rq)
        if kind == 1:
            assert np.array_equal(z, rz)


def _tie_rows(kind):
    """Groups built on exact half-integer quotients w / s = c + 1/2 (the
    round-half-even cases of lrint), over scales from 2^-133 (bf16 subnormal)
    to 2^100, plus every bf16 bit pattern (NaN, inf, subnormals) in groups."""
    groups = []
    for e in list(range(-140, -120)) + list(range(-80, -60, 3)) + [-20, -7, 0, 3, 50, 100]:
        p2 = np.float32(2.0) ** np.float32(e) if e > -127 else np.float32(np.ldexp(1.0, e))
        if kind == 0:
            c = np.arange(-127, 1, dtype=np.float32)  # 128 values: ties c + 1/2 and the max 127
            vals = (c + np.float32(0.5)) * p2
            vals[0] = np.float32(127.0) * p2
        else:
            k = np.arange(-14, 114, dtype=np.float32)  # (k / 2) s with range 15 s, zero point ~7
            vals = (k / np.float32(2.0) - np.float32(7.0)) * p2
            vals[0], vals[1] = np.float32(-7.5) * p2, np.float32(7.5) * p2
        groups.append(O.f32_to_bf16(vals.astype(np.float32)))
    rng = np.random.default_rng(7)
    allbits = np.arange(65536, dtype=np.uint16)
    groups += list(allbits.reshape(-1, 128))
    groups += list(rng.permutation(allbits).reshape(-1, 128))
    while len(groups) % 4:
        groups.append(np.zeros(128, np.uint16))
    return np.stack(groups).reshape(-1, 128 * 4)  # rows of four groups


@pytest.mark.parametrize("kind", [0, 1])
def test_quantize_ties_and_extreme_scales(kind):
    w = _tie_rows(kind)
    say("quantize ties/extremes", kind, w.shape)
    q, s, z = gpu_quantize(w, kind)
    rq, rs, rz = O.quantize(w, kind)
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)
    if kind == 1:
        assert np.array_equal(z, rz)


@pytest.mark.parametrize("kind", [0, 1])
def test_quantize_nan_in_finite_groups_and_mixed_waves(kind):
    """NaN values inside otherwise finite groups (the reference skips them
    in the group statistics and codes them 0), in waves whose other groups
    are ordinary, next to waves holding an infinite value or a tiny scale
    (which take the general rounding path for the whole wave)."""
    rng = np.random.default_rng(31 + kind)
    rows, cols = 64, 1024
    w = O.seeded_bf16(rng, (rows, cols), 0.05)
    nan = np.uint16(0x7FC0)
    for r in range(0, rows, 3):
        w[r, rng.integers(0, cols, 5)] = nan
    w[5, 700] = np.uint16(0x7F80)            # +inf
    w[9, 130:258] = O.f32_to_bf16(np.full(128, 1e-30, np.float32))  # tiny scale group
    w[9, 200] = nan
    say("quantize NaN groups", kind)
    q, s, z = gpu_quantize(w, kind)
    rq, rs, rz = O.quantize(w, kind)
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)
    if kind == 1:
        assert np.array_equal(z, rz)

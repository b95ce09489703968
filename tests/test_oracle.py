"""Pins the CPU oracle (oracle/iq_oracle.c) before anything is checked
against it.

- quantize/dequant: bit-exact against fixtures written by the reference's
  own compiled src/quant.cpp (tests/golden/gen_golden.py), plus closed-form
  invariants and brute-force cases a plausible slip would break.
- bf16: the exhaustive round trip and spot values of the reference's
  tests/test_f16.cpp, and an independent numpy restatement.
- linear: against an independent numpy float64 matmul on dequantised weights
  (tolerance kGemvTol = 5e-6 of the conditioning, tests/test_ops_gpu.cu:199-206).
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def cases(g):
    return sorted({k.rsplit("_", 1)[0] for k in g.files})


def test_quantize_matches_reference_fixtures(gold):
    n = 0
    for key in cases(gold):
        kind = 0 if key.startswith("int8") else 1
        w = gold[key + "_w"]
        q, s, z = O.quantize(w, kind)
        assert np.array_equal(q, gold[key + "_q"]), key
        assert np.array_equal(s, gold[key + "_s"]), key
        if kind == 1:
            assert np.array_equal(z, gold[key + "_z"]), key
        if key + "_dq" in gold.files:
            dq = O.dequant_matrix(q, s, z, kind, *w.shape)
            assert np.array_equal(dq.view(np.uint32), gold[key + "_dq"].view(np.uint32)), key
        n += 1
    assert n >= 20


def test_bf16_exhaustive_roundtrip():
    # tests/test_f16.cpp:45-55: every bf16 widens and re-rounds to itself (NaN stays NaN)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_to_f32(h)
    back = O.f32_to_bf16(f)
    nan = ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)
    assert np.array_equal(back[~nan], h[~nan])
    assert np.all(np.isnan(O.bf16_to_f32(back[nan])))
    L = O.lib()
    for v in (1.0, -0.0, 3.14159, 1e38, 1.00390625, 1.01171875, 2.0 ** -130, float("inf")):
        assert L.iqo_f32_to_bf16(v) == int(O.f32_to_bf16(np.float32(v)))
    # tests/test_f16.cpp:84-90 spot values
    assert L.iqo_bf16_to_f32(0x3F80) == 1.0
    assert L.iqo_f32_to_bf16(-0.0) == 0x8000
    assert not np.isinf(L.iqo_bf16_to_f32(L.iqo_f32_to_bf16(1e38)))
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1.0 (even)
    assert L.iqo_f32_to_bf16(1.00390625) == 0x3F80
    assert L.iqo_f32_to_bf16(1.01171875) == 0x3F82  # halfway 0x3F81/0x3F82 -> even 0x3F82


def test_bf16_random_vs_numpy():
    rng = np.random.default_rng(3)
    u = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    L = O.lib()
    vec = O.f32_to_bf16(f)
    idx = rng.integers(0, len(f), 2000)
    for i in idx:
        assert L.iqo_f32_to_bf16(float(f[i])) == int(vec[i]) or np.isnan(f[i])


def brute_quant_group(vals, kind):
    """Textbook restatement for one group, straight from the formulas of
    src/quant.h:5-10 with the stored-scale rule of src/quant.cpp:53-57."""
    vals = np.asarray(vals, np.float32)
    if kind == 0:
        amax = np.float32(np.max(np.abs(vals))) if len(vals) else np.float32(0)
        s = O.bf16_to_f32(O.f32_to_bf16(np.float32(amax / np.float32(127.0)) if amax > 0 else np.float32(1))).item()
        s = np.float32(s)
        q = np.clip(np.rint(vals / s), -127, 127).astype(int)
        return s, q, 0
    lo = min(np.float32(0), np.min(vals))
    hi = max(np.float32(0), np.max(vals))
    s = O.bf16_to_f32(O.f32_to_bf16(np.float32((hi - lo) / np.float32(15.0)) if hi > lo else np.float32(1))).item()
    s = np.float32(s)
    z = int(np.clip(np.rint(np.float32(-lo) / s), 0, 15).item())
    q = np.clip(np.rint(vals / s).astype(int) + z, 0, 15)
    return s, q, z


@pytest.mark.parametrize("kind", [0, 1])
def test_quantize_brute_force(kind):
    rng = np.random.default_rng(7 + kind)
    for cols in (2, 6, 128, 130, 258):
        w = O.seeded_bf16(rng, (3, cols), 0.05)
        q, s, z = O.quantize(w, kind)
        wf = O.bf16_to_f32(w)
        G = O.groups(cols)
        for r in range(3):
            for g in range(G):
                c0, c1 = g * 128, min(cols, g * 128 + 128)
                sb, qb, zb = brute_quant_group(wf[r, c0:c1], kind)
                assert O.bf16_to_f32(s[r, g]) == sb
                if kind == 0:
                    got = q.reshape(3, cols)[r, c0:c1].view(np.int8).astype(int)
                else:
                    assert z[r, g] == zb
                    flat = np.arange(r * cols + c0, r * cols + c1)
                    byte = q[flat // 2]
                    got = np.where(flat % 2 == 0, byte & 15, byte >> 4).astype(int)
                assert np.array_equal(got, qb), (cols, r, g)


def test_quantize_invariants(gold):
    for key in cases(gold):
        kind = 0 if key.startswith("int8") else 1
        w = gold[key + "_w"]
        q, s, z = O.quantize(w, kind)
        wf = O.bf16_to_f32(w)
        rows, cols = w.shape
        if kind == 0:
            assert q.view(np.int8).min() >= -127  # -128 is never produced
        else:
            assert z.max() <= 15
        # all-zero groups: scale 1.0 (0x3F80), codes 0 / z 0
        for r in range(rows):
            for g in range(O.groups(cols)):
                seg = wf[r, g * 128:(g + 1) * 128]
                if np.all(seg == 0):
                    assert s[r, g] == 0x3F80
                    if kind == 1:
                        assert z[r, g] == 0


def test_quantize_errors():
    w = np.zeros((2, 3), np.uint16)
    with pytest.raises(ValueError):
        O.quantize(w, 1)  # int4 with odd cols (src/quant.cpp:36)


def test_int4_nibble_ramp(gold):
    # tests/test_quant.cpp:55-64: values on half-steps of s = 1 land where dequant reads them
    w = gold["int4_ramp_w"]
    q, s, z = O.quantize(w, 1)
    dq = O.dequant_matrix(q, s, z, 1, 2, 128)
    want = (np.arange(128) % 16) - 7.5
    assert np.all(np.abs(dq[0] - want) <= 0.51)


@pytest.mark.parametrize("kind", [0, 1])
def test_dequant_closed_form(kind):
    rng = np.random.default_rng(11)
    rows, cols = 5, 260
    w = O.seeded_bf16(rng, (rows, cols), 0.05)
    q, s, z = O.quantize(w, kind)
    dq = O.dequant_matrix(q, s, z, kind, rows, cols)
    sc = np.repeat(O.bf16_to_f32(s), 128, axis=1)[:, :cols]
    if kind == 0:
        codes = q.view(np.int8).reshape(rows, cols).astype(np.float32)
    else:
        flat = np.arange(rows * cols)
        nib = np.where(flat % 2 == 0, q[flat // 2] & 15, q[flat // 2] >> 4).reshape(rows, cols)
        codes = (nib.astype(np.int32) - np.repeat(z, 128, axis=1)[:, :cols]).astype(np.float32)
    assert np.array_equal(dq, (sc * codes).astype(np.float32))
    # round-trip error bound of tests/test_quant.cpp:45-47
    wf = O.bf16_to_f32(w)
    bound = 0.5 / 127 + 0.004 if kind == 0 else 0.5 / 15 * 2 + 0.01
    for r in range(rows):
        for g in range(O.groups(cols)):
            seg = slice(g * 128, min(cols, g * 128 + 128))
            amax = np.abs(wf[r, seg]).max()
            assert np.abs(wf[r, seg] - dq[r, seg]).max() <= bound * amax + 1e-30


@pytest.mark.parametrize("kind", [0, 1])
def test_linear_vs_numpy_f64(kind):
    rng = np.random.default_rng(5)
    for T, K, N, bias in ((1, 1536, 64, False), (5, 130, 127, True), (3, 896, 33, True)):
        w = O.seeded_bf16(rng, (N, K), 0.02)
        q, s, z = O.quantize(w, kind)
        x = rng.standard_normal((T, K), dtype=np.float32)
        b = O.seeded_bf16(rng, (N,), 0.5) if bias else None
        y32 = O.linear_q_f32(x, q, s, z, kind, b, N)
        y64, c64 = O.linear_q_f64(x, q, s, z, kind, b, N)
        dq = O.dequant_matrix(q, s, z, kind, N, K)
        yn, cn = O.linear_dq_f64(x, dq, b)
        assert np.allclose(y64, yn, rtol=0, atol=1e-12 * cn.max())
        assert np.allclose(c64, cn, rtol=1e-12)
        assert np.all(np.abs(y32 - yn) <= 5e-6 * cn)


def test_linear_detects_transposed_or_dropped_term():
    rng = np.random.default_rng(9)
    K, N = 256, 16
    w = O.seeded_bf16(rng, (N, K), 0.02)
    q, s, z = O.quantize(w, 0)
    x = rng.standard_normal((1, K), dtype=np.float32)
    dq = O.dequant_matrix(q, s, z, 0, N, K)
    y = O.linear_q_f32(x, q, s, z, 0, None, N)
    _, c = O.linear_dq_f64(x, dq)
    dropped = x[:, :-1].astype(np.float64) @ dq[:, :-1].T      # last term dropped
    transposed = x.astype(np.float64) @ dq[::-1].T               # output rows reversed
    assert np.any(np.abs(y - dropped) > 5e-6 * c)
    assert np.any(np.abs(y - transposed) > 5e-6 * c)


def test_embedding_is_dequant():
    rng = np.random.default_rng(2)
    for kind in (0, 1):
        w = O.seeded_bf16(rng, (50, 256), 0.05)
        q, s, z = O.quantize(w, kind)
        ids = np.array([0, 49, 7, 7])
        out = O.embedding(q, s, z, kind, 256, ids)
        dq = O.dequant_matrix(q, s, z, kind, 50, 256)
        assert np.array_equal(out, dq[ids])

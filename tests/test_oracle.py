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


# ---------------------------------------------------------------- decode step pieces
ONE_BF16 = np.uint16(0x3F80)


def test_rmsnorm_closed_forms():
    """src/forward.cpp:21-31 pinned by closed forms: [3, 4] has mean square
    12.5; a constant vector maps to its sign (eps = 0); scale invariance;
    the weight multiplies elementwise.  A 'sum instead of mean' or a dropped
    weight fails one of these."""
    w = np.full(2, ONE_BF16)
    y = O.rmsnorm_f64(np.array([3.0, 4.0]), w, 0.0)
    assert np.allclose(y, np.array([3.0, 4.0]) / np.sqrt(12.5), rtol=1e-15)
    c = np.full(64, -2.5)
    assert np.allclose(O.rmsnorm_f64(c, np.full(64, ONE_BF16), 0.0), -1.0, rtol=1e-15)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(256)
    wb = O.f32_to_bf16(rng.uniform(0.5, 1.5, 256).astype(np.float32))
    a = O.rmsnorm_f64(x, wb, 0.0)
    assert np.allclose(O.rmsnorm_f64(x * 1e3, wb, 0.0), a, rtol=1e-12)
    assert np.allclose(a / O.bf16_to_f32(wb), O.rmsnorm_f64(x, np.full(256, ONE_BF16), 0.0), rtol=1e-12)
    # eps enters inside the root: x = [1] * 4, eps = 3 -> 1 / 2
    assert np.allclose(O.rmsnorm_f64(np.ones(4), np.full(4, ONE_BF16), 3.0), 0.5, rtol=1e-15)


def test_silu_closed_forms():
    """src/forward_internal.h:41-42: silu(0) = 0, silu(z) - silu(-z) = z,
    silu(1) = 1 / (1 + e^-1), silu(z) -> z for large z."""
    z = np.linspace(-8, 8, 33)
    assert O.silu_f64(0.0) == 0.0
    assert np.allclose(O.silu_f64(z) - O.silu_f64(-z), z, rtol=1e-14, atol=1e-14)
    assert abs(O.silu_f64(1.0) - 0.7310585786300049) < 1e-15
    assert abs(O.silu_f64(40.0) - 40.0) < 1e-12


def test_single_key_attention_is_the_value_row():
    """Brute force: scaled dot-product attention with one cached key (any q,
    k) and GQA head sharing gives each query head its kv head's value row."""
    rng = np.random.default_rng(2)
    nh, nkv, hd = 8, 2, 16
    q = rng.standard_normal((nh, hd))
    k = rng.standard_normal((nkv, hd))
    v = rng.standard_normal((nkv, hd))
    out = np.zeros((nh, hd))
    for h in range(nh):
        kv = h // (nh // nkv)
        s = np.array([q[h] @ k[kv] / np.sqrt(hd)])
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p[0] * v[kv]
    assert np.allclose(O.attention_single_key(v.reshape(-1), nh, nkv, hd), out.reshape(-1), rtol=1e-15)


def _tiny_decode_model(rng, zero_o_down=False):
    H, I, nh, nkv, hd, V = 32, 48, 4, 2, 8, 20
    cfg = dict(hidden=H, inter=I, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V, layers=2, eps=1e-6)
    bf = lambda n: O.f32_to_bf16(rng.uniform(0.5, 1.5, n).astype(np.float32))
    layers = []
    for _ in range(2):
        Lw = {"q": rng.standard_normal((nh * hd, H)), "k": rng.standard_normal((nkv * hd, H)),
              "v": rng.standard_normal((nkv * hd, H)), "o": rng.standard_normal((H, nh * hd)),
              "gate": rng.standard_normal((I, H)), "up": rng.standard_normal((I, H)),
              "down": rng.standard_normal((H, I)), "input_ln": bf(H), "post_ln": bf(H)}
        if zero_o_down:
            Lw["o"] = np.zeros_like(Lw["o"])
            Lw["down"] = np.zeros_like(Lw["down"])
        layers.append(Lw)
    return dict(cfg=cfg, embed_dq=rng.standard_normal((V, H)), head_dq=rng.standard_normal((V, H)),
                final_norm=bf(H), layers=layers)


def test_decode_wiring_invariants():
    """The residual stream of src/forward.cpp:200-246: with o and down zero
    the hidden state stays the embedding row through every layer and the
    logits are head . rmsnorm(embedding); q/k/v read rmsnorm(h, input_ln);
    h1 = h + o . attn; h2 = h1 + down . act."""
    rng = np.random.default_rng(3)
    m = _tiny_decode_model(rng, zero_o_down=True)
    r = O.decode_first_token_f64(m, 5)
    for Lr in r["layers"]:
        assert np.array_equal(Lr["h2"], m["embed_dq"][5])
    assert np.allclose(r["logits"], m["head_dq"] @ O.rmsnorm_f64(m["embed_dq"][5], m["final_norm"], 1e-6))
    m = _tiny_decode_model(rng)
    r = O.decode_first_token_f64(m, 3)
    L0, W0 = r["layers"][0], m["layers"][0]
    n = O.rmsnorm_f64(m["embed_dq"][3], W0["input_ln"], 1e-6)
    assert np.allclose(L0["q"], W0["q"] @ n) and np.allclose(L0["v"], W0["v"] @ n)
    ctx = O.attention_single_key(L0["v"], 4, 2, 8)
    assert np.allclose(L0["h1"], m["embed_dq"][3] + W0["o"] @ ctx)
    n2 = O.rmsnorm_f64(L0["h1"], W0["post_ln"], 1e-6)
    assert np.allclose(L0["act"], O.silu_f64(W0["gate"] @ n2) * (W0["up"] @ n2))
    assert np.allclose(L0["h2"], L0["h1"] + W0["down"] @ L0["act"])
    assert np.array_equal(r["layers"][1]["h"], L0["h2"])

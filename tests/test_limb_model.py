"""CPU model of the GEMV's activation format (infer_amd/csrc/iq_limbs.h),
in numpy: per (row, 128-column group) 2^k with max|x| 2^k in
[2^30 * 0xFEFEFE / 2^24, 0x7F7F7F7F], X = rint(x 2^k) as four balanced byte limbs, exact
integer sums of codes times limbs, and the group's value
fp32(2^16 (256 t0 + t1) + (256 t2 + t3)) * s * 2^-k accumulated in fp32.

Checks, against float64 over dequant() (the oracle's reference product):
* the limbs reassemble X exactly and stay in [-128, 127];
* one outlier channel per group at 10^3..10^5 x the typical value, with
  output rows whose weight on it is 0, stays within the reference's
  5e-6 of the conditioning sum |w x| (tests/test_ops_gpu.cu:199-206, kGemvTol);
* the three-limb form this replaced (22 bits) fails that bound at 10^4,
  so the check separates the two.
The GPU tests (tests/test_gpu_outliers.py) hold the kernels to the same
bound on every route."""
import numpy as np

from oracle import oracle as O

TOL = 5e-6
MAXV = 0x7F7F7F7F  # 127 * (2^24 + 2^16 + 2^8 + 1)


def group_scale_exp(amax, bits):
    """k of the kernel: the largest power with amax 2^k <= the limb range
    (bits = 31: four limbs, 0x7F7F7F7F; bits = 22: the old three limbs)."""
    mant, e = np.frexp(amax)
    if bits == 31:
        k = 31 - e
        return np.where(mant * 2.0 ** 24 > 16711422.0, k - 1, k)
    return 22 - e


def to_fixed(xg, bits):
    amax = np.abs(xg).max(-1, keepdims=True)
    amax = np.where(amax > 0, amax, 1.0)
    k = group_scale_exp(amax, bits)
    X = np.rint(xg * 2.0 ** k)
    return X, k


def limbs(X):
    U = (X.astype(np.int64) + 0x80808080) & 0xFFFFFFFF
    return [((U >> (24 - 8 * L)) & 0xFF) - 128 for L in range(4)]


def gemv_model(x, q, s, z, kind, rows, cols, bits=31):
    """y[m, n] with the kernels' arithmetic (exact integer group sums, fp32
    combination and accumulation)."""
    G = cols // 128
    codes = O.dequant_matrix(q, np.ones_like(s) * 0x3F80, None if z is None else np.zeros_like(z), kind, rows, cols)
    codes = np.rint(codes).astype(np.int64).reshape(rows, G, 128)  # stored codes (int4: the nibble)
    zz = np.zeros((rows, G), np.int64) if z is None else z.astype(np.int64)
    sc = O.bf16_to_f32(s).reshape(rows, G).astype(np.float32)
    M = x.shape[0]
    y = np.zeros((M, rows), np.float32)
    for m in range(M):
        X, k = to_fixed(x[m].astype(np.float64).reshape(G, 128), bits)
        for g in range(G):
            t = codes[:, g, :] @ X[g]  # exact: |sum| < 2^53
            sx = X[g].sum()
            tq = t - zz[:, g] * sx
            v = np.float32(tq)  # one rounding of the group's exact value
            f = np.float32(2.0 ** -float(k[g, 0]))
            y[m] = np.float32(y[m] + v * (sc[:, g] * f))
    return y


def outlier_case(rng, kind, mag, rows=96, cols=1024):
    G = cols // 128
    w = O.seeded_bf16(rng, (rows, cols), 0.02)
    q, s, z = O.quantize(w, kind)
    q = q.copy()
    ocol = int(rng.integers(0, 128))
    cols_o = np.arange(G) * 128 + ocol
    if kind == 1:
        qb = q.reshape(rows, cols // 2)
        for r in range(rows // 2):
            for c in cols_o:
                b, zp = qb[r, c // 2], int(z[r, c // 128])
                qb[r, c // 2] = (b & 0xF0) | zp if c % 2 == 0 else (b & 0x0F) | (zp << 4)
    else:
        q.reshape(rows, cols)[: rows // 2, cols_o] = 0
    x = rng.standard_normal((2, cols)).astype(np.float32)
    x[:, cols_o] = np.float32(mag)
    return x, q, s, z


def worst(x, q, s, z, kind, rows, cols, bits):
    dq = O.dequant_matrix(q, s, z, kind, rows, cols)
    ref, cond = O.linear_dq_f64(x, dq)
    got = gemv_model(x, q, s, z, kind, rows, cols, bits)
    return float((np.abs(got - ref) / np.maximum(cond, 1e-30)).max())


def test_limbs_reassemble_exactly():
    rng = np.random.default_rng(0)
    X = rng.integers(-MAXV, MAXV + 1, 20000, dtype=np.int64)
    X[:4] = [MAXV, -MAXV, 0, -1]
    L = limbs(X)
    assert all(((l >= -128) & (l <= 127)).all() for l in L)
    back = (L[0] << 24) + (L[1] << 16) + (L[2] << 8) + L[3]
    assert np.array_equal(back, X)


def test_scale_keeps_the_group_inside_the_limb_range():
    rng = np.random.default_rng(1)
    xg = (rng.standard_normal((5000, 128)) * 10.0 ** rng.integers(-30, 30, (5000, 1))).astype(np.float32)
    X, k = to_fixed(xg.astype(np.float64), 31)
    assert np.abs(X).max() <= MAXV
    # at least 2^30 * 0xFEFEFE / 2^24: the step down to k - 1 only happens
    # when the mantissa would overflow the limb range
    assert (np.abs(X).max(-1) >= np.floor(2.0 ** 6 * 16711422.0)).all()


def test_outlier_channels_within_the_reference_bound():
    rng = np.random.default_rng(2)
    for kind in (0, 1):
        for mag in (1e3, 1e4, 1e5):
            x, q, s, z = outlier_case(rng, kind, mag)
            e = worst(x, q, s, z, kind, 96, 1024, 31)
            assert e <= TOL, (kind, mag, e)


def test_three_limb_form_fails_the_bound():
    rng = np.random.default_rng(3)
    x, q, s, z = outlier_case(rng, 0, 1e4)
    assert worst(x, q, s, z, 0, 96, 1024, 22) > TOL

"""Writes the golden quantisation fixtures from the reference's OWN compiled
quantiser (oracle/_ref/libref.so, built by `make -C oracle ref` from
/root/reference/src/quant.cpp).  Run in the build container only:

    make -C oracle ref && python tests/golden/gen_golden.py

Output: tests/golden/quant_golden.npz (inputs as bf16 bits, the reference's
codes / scales / zeros and dequantised values) and tests/golden/ref_small.llmq
(a container written by the reference's QuantWriter, src/quant.cpp:106-134).
Cases follow tests/test_quant.cpp:27-64 (rows 37, cols 128/130/896/1536,
N(0,0.05) bf16, the int4 half-step ramp) plus model-width rows and
adversarial groups (zero, one-signed, spike, exact ties, denormals, huge).
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle.oracle import REF_PATH, f32_to_bf16, groups  # noqa: E402


def ref_lib():
    L = ctypes.CDLL(REF_PATH, mode=os.RTLD_NOW)
    P = ctypes.c_void_p
    L.ref_quantize.argtypes = [P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, P, P, P]
    L.ref_quantize.restype = ctypes.c_int
    L.ref_dequant_matrix.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, P]
    L.ref_llmq_write.argtypes = [ctypes.c_char_p, ctypes.c_char_p, P, P, P, ctypes.c_int,
                                 ctypes.c_int64, ctypes.c_int64]
    L.ref_llmq_write.restype = ctypes.c_int
    return L


def p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def ref_quantize(L, w, kind):
    rows, cols = w.shape
    G = groups(cols)
    q = np.zeros(rows * cols // 2 if kind == 1 else rows * cols, np.uint8)
    s = np.zeros(rows * G, np.uint16)
    z = np.zeros(rows * G, np.uint8)
    rc = L.ref_quantize(p(np.ascontiguousarray(w)), rows, cols, kind, p(q), p(s), p(z))
    assert rc == 0
    dq = np.zeros((rows, cols), np.float32)
    L.ref_dequant_matrix(p(q), p(s), p(z), kind, rows, cols, p(dq))
    return q, s.reshape(rows, G), z.reshape(rows, G), dq


def adversarial(cols):
    """One row per pathological group pattern, each over `cols` columns."""
    rows = []
    f = np.float32
    rows.append(np.zeros(cols, f))                                   # all zero
    rows.append(np.abs(np.linspace(0.01, 0.3, cols, dtype=f)))       # all positive
    rows.append(-np.abs(np.linspace(0.01, 0.3, cols, dtype=f)))      # all negative
    spike = np.full(cols, 1e-3, f); spike[::97] = 5.0; rows.append(spike)  # single spike per group
    # int8 exact ties: amax 127 -> s = 1, values k + 0.5 exactly
    tie = (np.arange(cols, dtype=f) % 254) - 126.5; tie[::128] = 127.0; rows.append(tie)
    # int4 ties: range [-7.5, 7.5] -> s = 1, z = lrint(7.5) = 8 (even), values on half steps
    rows.append(((np.arange(cols) % 16).astype(f) - 7.5))
    rows.append(np.full(cols, 1e-40, f))                              # denormals
    big = np.full(cols, 1e38, f); big[1::2] = -3e38; rows.append(big)  # near fp32 max
    rows.append(np.where(np.arange(cols) % 2 == 0, -0.0, 0.0).astype(f))  # signed zeros
    mixed = np.linspace(-1.0, 1.0, cols, dtype=f) ** 3; rows.append(mixed)
    return f32_to_bf16(np.stack(rows))


def main():
    L = ref_lib()
    out = {}
    rng = np.random.default_rng(10)
    shapes = [(37, 128), (37, 130), (37, 896), (37, 1536), (8, 256), (5, 1536), (3, 8960), (2, 18944)]
    for kind, kn in ((0, "int8"), (1, "int4")):
        for rows, cols in shapes:
            w = f32_to_bf16(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05))
            q, s, z, dq = ref_quantize(L, w, kind)
            key = f"{kn}_{rows}x{cols}"
            out[key + "_w"] = w
            out[key + "_q"] = q
            out[key + "_s"] = s
            if kind == 1:
                out[key + "_z"] = z
            if rows * cols <= 37 * 1536:
                out[key + "_dq"] = dq
        for cols in (128, 130, 256):
            w = adversarial(cols)
            q, s, z, dq = ref_quantize(L, w, kind)
            key = f"{kn}_adv{cols}"
            out[key + "_w"] = w
            out[key + "_q"] = q
            out[key + "_s"] = s
            if kind == 1:
                out[key + "_z"] = z
            out[key + "_dq"] = dq
    # tests/test_quant.cpp:55-64 int4 ramp (2 x 128, values (i%16) - 7.5)
    ramp = f32_to_bf16(((np.arange(256) % 16).astype(np.float32) - 7.5).reshape(2, 128))
    q, s, z, dq = ref_quantize(L, ramp, 1)
    out.update(int4_ramp_w=ramp, int4_ramp_q=q, int4_ramp_s=s, int4_ramp_z=z, int4_ramp_dq=dq)
    np.savez_compressed(os.path.join(HERE, "quant_golden.npz"), **out)

    # container fixture: one int4 and one int8 matrix via the reference writer
    w = f32_to_bf16(rng.standard_normal((8, 256), dtype=np.float32) * np.float32(0.1))
    q, s, z, _ = ref_quantize(L, w, 1)
    path = os.path.join(HERE, "ref_small_int4.llmq")
    assert L.ref_llmq_write(path.encode(), b"m", p(q), p(s), p(z), 1, 8, 256) == 0
    np.savez_compressed(os.path.join(HERE, "ref_small_int4.npz"), w=w, q=q, s=s, z=z)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()

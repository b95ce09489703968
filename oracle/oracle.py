"""numpy/ctypes front-end of oracle/iq_oracle.c (test infrastructure only).

Each wrapper names the reference function it restates; the C file carries the
file:line citations.  Kind codes: 0 = int8, 1 = int4 (kernels/ops/ops.cuh:165).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")
GROUP = 128

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.iqo_quantize.argtypes = [P, i64, i64, ctypes.c_int, P, P, P, P]
        L.iqo_quantize.restype = ctypes.c_int
        L.iqo_dequant_matrix.argtypes = [P, P, P, ctypes.c_int, i64, i64, P]
        L.iqo_linear_q_f32.argtypes = [P, P, P, P, ctypes.c_int, P, i64, i64, i64, P]
        L.iqo_linear_q_f64.argtypes = [P, P, P, P, ctypes.c_int, P, i64, i64, i64, P, P]
        L.iqo_embedding.argtypes = [P, P, P, ctypes.c_int, i64, P, i64, P]
        L.iqo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.iqo_f32_to_bf16.restype = ctypes.c_uint16
        L.iqo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.iqo_bf16_to_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def groups(cols):
    return (cols + GROUP - 1) // GROUP


def f32_to_bf16(a):
    """src/f16.h:41-51 vectorised in numpy (RNE, NaN kept quiet).  Pinned
    against the scalar C restatement in tests/test_oracle.py."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize(w_bf16, kind):
    """llm::quantize (src/quant.cpp:34-84) -> (q, scales, zeros|None)."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    rows, cols = w.shape
    G = groups(cols)
    q = np.zeros(rows * cols // 2 if kind == 1 else rows * cols, np.uint8)
    s = np.zeros(rows * G, np.uint16)
    z = np.zeros(rows * G, np.uint8) if kind == 1 else None
    buf = np.zeros(max(cols, 1), np.float32)
    rc = lib().iqo_quantize(_p(w), rows, cols, kind, _p(q), _p(s), _p(z), _p(buf))
    if rc != 0:
        raise ValueError("quantize: kind" if rc == -1 else "quantize: int4 needs even cols")
    return q, s.reshape(rows, G), (z.reshape(rows, G) if z is not None else None)


def dequant_matrix(q, scales, zeros, kind, rows, cols):
    """llm::dequant (src/quant.cpp:86-93) for every element."""
    out = np.zeros((rows, cols), np.float32)
    lib().iqo_dequant_matrix(_p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(scales)),
                             _p(None if zeros is None else np.ascontiguousarray(zeros)),
                             kind, rows, cols, _p(out))
    return out


def linear_q_f32(x, q, scales, zeros, kind, bias, out_features):
    """src/forward.cpp:35-47 on dequantised weights (sequential fp32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    y = np.zeros((T, out_features), np.float32)
    lib().iqo_linear_q_f32(_p(x), _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(scales)),
                           _p(None if zeros is None else np.ascontiguousarray(zeros)), kind,
                           _p(None if bias is None else np.ascontiguousarray(bias, dtype=np.uint16)),
                           T, K, out_features, _p(y))
    return y


def linear_q_f64(x, q, scales, zeros, kind, bias, out_features):
    """tests/test_ops_gpu.cu:676-687: double reference y and conditioning."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    y = np.zeros((T, out_features), np.float64)
    c = np.zeros((T, out_features), np.float64)
    lib().iqo_linear_q_f64(_p(x), _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(scales)),
                           _p(None if zeros is None else np.ascontiguousarray(zeros)), kind,
                           _p(None if bias is None else np.ascontiguousarray(bias, dtype=np.uint16)),
                           T, K, out_features, _p(y), _p(c))
    return y, c


def linear_dq_f64(x, wdq, bias_bf16=None):
    """Fast double reference for large shapes: x(f64) @ dequant(W)(f64)^T
    plus conditioning |x| @ |W|^T (+|b|).  Same quantities as linear_q_f64."""
    xd = np.asarray(x, np.float64)
    wd = np.asarray(wdq, np.float64)
    y = xd @ wd.T
    c = np.abs(xd) @ np.abs(wd).T
    if bias_bf16 is not None:
        b = bf16_to_f32(bias_bf16).astype(np.float64)
        y = y + b
        c = c + np.abs(b)
    return y, c


def embedding(q, scales, zeros, kind, H, ids):
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    out = np.zeros((len(ids), H), np.float32)
    lib().iqo_embedding(_p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(scales)),
                        _p(None if zeros is None else np.ascontiguousarray(zeros)), kind, H,
                        _p(ids), len(ids), _p(out))
    return out


def seeded_bf16(rng, shape, sd):
    """Synthetic weights: fp32 ~N(0, sd) rounded RNE to bf16 (src/f16.h:41-51),
    the form llm::quantize consumes (src/quant.h:61)."""
    return f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(sd))


# ---------------------------------------------------------------- decode step
# The reference's CPU forward (src/forward.cpp:160-262) for one token at
# position 0, on dequantised weights, in float64 (the truth the fp32 GPU
# chain is compared with).  Pieces: rmsnorm (src/forward.cpp:21-31), linear
# (:35-47), silu (src/forward_internal.h:41-42), attention over one cached
# key (softmax weight 1: every query head takes its kv head's value row).

def rmsnorm_f64(x, w_bf16, eps):
    """src/forward.cpp:21-31: x / sqrt(mean(x^2) + eps) * w."""
    x = np.asarray(x, np.float64)
    scale = 1.0 / np.sqrt(np.mean(x * x) + float(eps))
    return x * scale * bf16_to_f32(w_bf16).astype(np.float64)


def silu_f64(z):
    """src/forward_internal.h:41-42: z / (1 + exp(-z))."""
    z = np.asarray(z, np.float64)
    return z / (1.0 + np.exp(-z))


def attention_single_key(v, n_heads, n_kv_heads, head_dim):
    """Attention output of a sequence of one token (src/forward.cpp
    attention() with T = 1): softmax over one score is 1, so query head h
    gets value row h // (n_heads / n_kv_heads)."""
    v = np.asarray(v).reshape(n_kv_heads, head_dim)
    grp = n_heads // n_kv_heads
    return np.repeat(v, grp, axis=0).reshape(-1)


def decode_first_token_f64(model, token):
    """Every intermediate of the forward of `token` at position 0.  model:
    cfg dict (hidden, heads, kv_heads, head_dim, eps), embed_dq [V, H],
    head_dq, final_norm (bf16 bits), layers: dicts of dequantised q, k, v,
    o, gate, up, down (float arrays [out, in]), bf16 bits input_ln, post_ln,
    optional q_b, k_b, v_b."""
    c = model["cfg"]
    h = np.asarray(model["embed_dq"][token], np.float64)
    out = {"h0": h, "layers": []}
    for Lw in model["layers"]:
        n = rmsnorm_f64(h, Lw["input_ln"], c["eps"])
        r = {"h": h}
        for name in ("q", "k", "v"):
            y = np.asarray(Lw[name], np.float64) @ n
            if Lw.get(name + "_b") is not None:
                y = y + bf16_to_f32(Lw[name + "_b"]).astype(np.float64)
            r[name] = y
        ctx = attention_single_key(r["v"], c["heads"], c["kv_heads"], c["head_dim"])
        h1 = h + np.asarray(Lw["o"], np.float64) @ ctx
        n2 = rmsnorm_f64(h1, Lw["post_ln"], c["eps"])
        act = silu_f64(np.asarray(Lw["gate"], np.float64) @ n2) * (np.asarray(Lw["up"], np.float64) @ n2)
        h2 = h1 + np.asarray(Lw["down"], np.float64) @ act
        r.update(h1=h1, act=act, h2=h2)
        out["layers"].append(r)
        h = h2
    out["logits"] = np.asarray(model["head_dq"], np.float64) @ rmsnorm_f64(h, model["final_norm"], c["eps"])
    return out

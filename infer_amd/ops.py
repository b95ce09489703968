"""Python mirror of the reference's quantised-op interface, over libiq.so.

Mirrors, with the same names, argument meaning and order:
  QuantKind, QuantView            kernels/ops/ops.cuh:165-172
  launch_gemv_batched_q           kernels/ops/ops.cuh:173-174
  launch_gemm_tiled_q             kernels/ops/ops.cuh:175-176
  launch_embedding_q              kernels/ops/ops.cuh:177-178
  linear_b (quantised branch)     kernels/batch_gpu.cu:137-147
  quantize                        src/quant.h:61 (on the device here)
  upload_q                        kernels/model_gpu_internal.cuh:67-83

Every call goes through the C ABI of include/iq.h (ctypes); torch is used
only for device memory and the current stream.  Launches are asynchronous
on torch's current stream, like the reference's (ops.cuh:3-7).  Where the
reference would fail later inside CUDA_CHECK (exit(1)), these wrappers raise
RuntimeError with the library's message at the call.  There is no CPU
fallback: without libiq.so every entry point raises.
"""
import ctypes
import enum
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libiq.so")
GROUP = 128

_lib = None


class IqView(ctypes.Structure):
    """iq_view / gpu::QuantView (kernels/ops/ops.cuh:166-172)."""
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("q", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("zeros", ctypes.c_void_p),
    ]


class IqStage(ctypes.Structure):
    """iq_stage (include/iq.h): one stage of a chain."""
    _fields_ = [
        ("in_op", ctypes.c_int32),
        ("out_op", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("gqa_head_dim", ctypes.c_int32),
        ("gqa_group", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("x", ctypes.c_void_p),
        ("norm", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
        ("W", IqView * 3),
        ("bias", ctypes.c_void_p * 3),
        ("y", ctypes.c_void_p * 3),
        ("rows", ctypes.c_int32),
    ]


# Every function include/iq.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_VP = ctypes.POINTER(IqView)
SIGNATURES = {
    "iq_gemv": ([_P, _VP, _P, ctypes.c_int, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_gemv_noalloc": ([_P, _VP, _P, ctypes.c_int, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_gemv_prep": ([_P, ctypes.c_int, _I64, ctypes.c_int, _P], ctypes.c_int),
    "iq_gemv_prepped": ([_VP, _P, ctypes.c_int, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_gemv_prepped_multi": ([_P, ctypes.c_int, _P, ctypes.c_int, _I64, _P, _P], ctypes.c_int),
    "iq_gemv_multi": ([_P, _P, ctypes.c_int, _P, ctypes.c_int, _I64, _P, _P], ctypes.c_int),
    "iq_gemm": ([_P, _VP, _P, _I64, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_gemm_bf16x": ([_P, _VP, _P, _I64, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_linear": ([_P, _VP, _P, _I64, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_embedding": ([_VP, _P, _I64, _I64, _P, _P], ctypes.c_int),
    "iq_quantize": ([_P, _I64, _I64, ctypes.c_int, _P, _P, _P, _P], ctypes.c_int),
    "iq_chain_create": ([ctypes.POINTER(IqStage), ctypes.c_int, ctypes.POINTER(_P)], ctypes.c_int),
    "iq_chain_run": ([_P, _P], ctypes.c_int),
    "iq_chain_destroy": ([_P], None),
    "iq_init": ([ctypes.c_int], ctypes.c_int),
    "iq_init_stream": ([ctypes.c_int, _P], ctypes.c_int),
    "iq_error_string": ([ctypes.c_int], ctypes.c_char_p),
    "iq_version": ([], ctypes.c_char_p),
}


def lib():
    """Loads libiq.so (built by infer_amd.build).  Raises when it is missing:
    the quantised path has no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m infer_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def _check(rc, what):
    if rc != 0:
        msg = lib().iq_error_string(rc).decode()
        raise RuntimeError(f"{what}: {msg} (code {rc})")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class QuantKind(enum.IntEnum):
    """gpu::QuantKind (kernels/ops/ops.cuh:165)."""
    kInt8 = 0
    kInt4 = 1


def groups_of(cols):
    return (cols + GROUP - 1) // GROUP


class QuantView:
    """A quantised [rows x cols] matrix resident on the device (the packed
    layout of src/quant.h:34-58).  Owns its tensors (the reference's DevTensor
    owns q/scales/zeros and hands out the POD QuantView)."""

    def __init__(self, kind, rows, cols, q, scales, zeros=None):
        self.kind = QuantKind(kind)
        self.rows = int(rows)
        self.cols = int(cols)
        self.groups = groups_of(self.cols)
        self.q = q
        self.scales = scales
        self.zeros = zeros
        self._c = IqView(int(self.kind), self.rows, self.cols, self.groups,
                         q.data_ptr(), scales.data_ptr(),
                         zeros.data_ptr() if zeros is not None else None)

    @property
    def c(self):
        return ctypes.byref(self._c)

    def q_bytes(self):
        return self.rows * self.cols // 2 if self.kind == QuantKind.kInt4 else self.rows * self.cols

    def nbytes(self):
        """Packed bytes: codes + bf16 scales (+ u8 zeros)."""
        n = self.q_bytes() + 2 * self.rows * self.groups
        if self.kind == QuantKind.kInt4:
            n += self.rows * self.groups
        return n


def alloc_quant(kind, rows, cols, device="cuda"):
    kind = QuantKind(kind)
    G = groups_of(cols)
    nq = rows * cols // 2 if kind == QuantKind.kInt4 else rows * cols
    q = torch.empty(nq, dtype=torch.uint8, device=device)
    s = torch.empty(rows * G, dtype=torch.int16, device=device)
    z = torch.empty(rows * G, dtype=torch.uint8, device=device) if kind == QuantKind.kInt4 else None
    return QuantView(kind, rows, cols, q, s, z)


def quantize(w_bf16, kind, out=None, stream=None):
    """llm::quantize (src/quant.cpp:34-84) on the device: w_bf16 is a
    [rows, cols] torch.bfloat16 (or int16 bf16-bit) CUDA tensor.  Returns a
    QuantView (allocated unless `out` is given)."""
    if w_bf16.dim() != 2:
        raise ValueError("quantize: expected a 2-D weight")
    rows, cols = w_bf16.shape
    kind = QuantKind(kind)
    if kind == QuantKind.kInt4 and cols % 2:
        raise ValueError("quantize: int4 needs even cols")
    w = w_bf16.contiguous()
    if out is None:
        out = alloc_quant(kind, rows, cols, device=w.device)
    rc = lib().iq_quantize(_ptr(w), rows, cols, int(kind), _ptr(out.q), _ptr(out.scales),
                           _ptr(out.zeros), _stream(stream))
    _check(rc, "iq_quantize")
    return out


def upload_q(kind, rows, cols, q, scales, zeros=None, device="cuda"):
    """DevTensor::upload_q (kernels/model_gpu_internal.cuh:67-83): numpy
    arrays of the packed layout (q u8, scales u16 bf16 bits, zeros u8) ->
    device QuantView."""
    import numpy as np

    def dev(a, npdt, tdt):
        return torch.from_numpy(np.ascontiguousarray(a).reshape(-1).view(npdt)).to(device)

    qd = dev(q, np.uint8, torch.uint8)
    sd = dev(scales, np.int16, torch.int16)
    zd = dev(zeros, np.uint8, torch.uint8) if zeros is not None else None
    return QuantView(kind, rows, cols, qd, sd, zd)


def _bias_ptr(bias):
    if bias is None:
        return None
    if bias.dtype not in (torch.bfloat16, torch.int16):
        raise TypeError("bias must be bf16 (torch.bfloat16 or int16 bits)")
    return _ptr(bias)


def launch_gemv_batched_q(x, W, bias, B, in_, out, y, stream=None):
    """y[b, o] = sum_c dequant(W, o, c) x[b, c] (+ bias[o]) for b < B <= 32."""
    rc = lib().iq_gemv(_ptr(x), W.c, _bias_ptr(bias), int(B), int(in_), int(out), _ptr(y), _stream(stream))
    _check(rc, "iq_gemv")


def gemv_noalloc(x, W, bias, B, in_, out, y, stream=None):
    """launch_gemv_batched_q on the library's static scratch (no allocation;
    in <= 32768; calls that overlap on one device race)."""
    rc = lib().iq_gemv_noalloc(_ptr(x), W.c, _bias_ptr(bias), int(B), int(in_), int(out), _ptr(y), _stream(stream))
    _check(rc, "iq_gemv_noalloc")


def gemv_prep(x, B, in_, kind, stream=None):
    """Prepare activations x [B, in] once for several GEMVs of one kind."""
    rc = lib().iq_gemv_prep(_ptr(x), int(B), int(in_), int(kind), _stream(stream))
    _check(rc, "iq_gemv_prep")


def gemv_prepped(W, bias, B, in_, out, y, stream=None):
    """GEMV of W on the activations of the last gemv_prep."""
    rc = lib().iq_gemv_prepped(W.c, _bias_ptr(bias), int(B), int(in_), int(out), _ptr(y), _stream(stream))
    _check(rc, "iq_gemv_prepped")


def gemv_prepped_multi(Ws, biases, B, in_, ys, stream=None):
    """Several matrices (same kind and width) on the last gemv_prep's
    activations in one call: ys[i] = x @ dequant(Ws[i])^T (+ biases[i])."""
    n = len(Ws)
    views = (ctypes.c_void_p * n)(*[ctypes.addressof(W._c) for W in Ws])
    bs = (ctypes.c_void_p * n)(*[(b.data_ptr() if b is not None else None) for b in (biases or [None] * n)])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    rc = lib().iq_gemv_prepped_multi(views, n, bs, int(B), int(in_), yp, _stream(stream))
    _check(rc, "iq_gemv_prepped_multi")


def gemv_multi(x, Ws, biases, B, in_, ys, stream=None):
    """Several matrices (same kind and width) sharing the activations
    x [B, in]: ys[i] = x @ dequant(Ws[i])^T (+ biases[i]); one launch at B = 1."""
    n = len(Ws)
    views = (ctypes.c_void_p * n)(*[ctypes.addressof(W._c) for W in Ws])
    bs = (ctypes.c_void_p * n)(*[(b.data_ptr() if b is not None else None) for b in (biases or [None] * n)])
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    rc = lib().iq_gemv_multi(_ptr(x), views, n, bs, int(B), int(in_), yp, _stream(stream))
    _check(rc, "iq_gemv_multi")


def launch_gemm_tiled_q(x, W, bias, T, in_, out, y, stream=None):
    """Same contract for any T (the prefill GEMM), fp32 activations."""
    rc = lib().iq_gemm(_ptr(x), W.c, _bias_ptr(bias), int(T), int(in_), int(out), _ptr(y), _stream(stream))
    _check(rc, "iq_gemm")


def launch_gemm_bf16x(x_bf16, W, bias, T, in_, out, y, stream=None):
    """Prefill GEMM with bf16 activations (fp32 output)."""
    rc = lib().iq_gemm_bf16x(_ptr(x_bf16), W.c, _bias_ptr(bias), int(T), int(in_), int(out), _ptr(y),
                             _stream(stream))
    _check(rc, "iq_gemm_bf16x")


def launch_linear_q(x, W, bias, T, in_, out, y, stream=None):
    """GpuBatch::Impl::linear_b quantised branch (kernels/batch_gpu.cu:137-147)."""
    rc = lib().iq_linear(_ptr(x), W.c, _bias_ptr(bias), int(T), int(in_), int(out), _ptr(y), _stream(stream))
    _check(rc, "iq_linear")


def launch_embedding_q(table, ids, T, H, out, stream=None):
    """out[t, i] = dequant(table, ids[t], i)."""
    rc = lib().iq_embedding(table.c, _ptr(ids), int(T), int(H), _ptr(out), _stream(stream))
    _check(rc, "iq_embedding")


def linear(x, W, bias=None, stream=None):
    """Allocating convenience: y = x @ dequant(W)^T (+ bias), x [T, in] fp32."""
    T, K = x.shape
    y = torch.empty(T, W.rows, dtype=torch.float32, device=x.device)
    launch_linear_q(x.contiguous(), W, bias, T, K, W.rows, y, stream)
    return y


def init(device=0, stream=None):
    """Reserve the workspace of (device, stream) before a graph capture."""
    if stream is None:
        _check(lib().iq_init(int(device)), "iq_init")
    else:
        _check(lib().iq_init_stream(int(device), ctypes.c_void_p(stream.cuda_stream)), "iq_init_stream")

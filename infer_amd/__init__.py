"""infer_amd -- MI355X (gfx950) quantized-weight matrix path.

HIP kernels and a C ABI in libiq.so (include/iq.h); `infer_amd.ops` is the
Python mirror of the reference's launcher interface over that ABI.
"""
from .ops import (  # noqa: F401
    QuantKind,
    QuantView,
    alloc_quant,
    launch_embedding_q,
    launch_gemm_bf16x,
    launch_gemm_tiled_q,
    launch_gemv_batched_q,
    launch_linear_q,
    lib,
    linear,
    quantize,
    upload_q,
)

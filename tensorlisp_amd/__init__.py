"""tensorlisp_amd: MI355X (gfx950) executor for tensorlisp's quantized hot path.

GGML_OP_MUL_MAT over Q8_0 / Q4_0 / Q4_K weights (decode GEMV and prefill GEMM)
and paged-attention decode over an f16 block-table KV cache, as hand-written
HIP kernels behind the C ABI in include/tlhip.h. ``tensorlisp_amd.native``
binds that ABI; the library is built by ``tensorlisp_amd.build``.
"""

__all__ = ["native", "build"]

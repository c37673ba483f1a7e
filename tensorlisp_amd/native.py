"""Python binding of the gfx950 executor's C ABI (``include/tlhip.h``).

This mirrors, for tests and the benchmark, what a ``native-hip`` Rust binding
would do: build the 456-byte op descriptor of a ggml node (the ``struct Op``
of crates/kernels/src/cuda/native/common.cuh:14-26, packed like OpBlob in
crates/kernels/src/cuda/lower.rs:67-99) and call the library on a stream.
PyTorch only supplies device memory and the current stream.

The library must be built (``python -m tensorlisp_amd.build``); importing this
module without it raises, there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libtlhip.so"

# ggml type numbers (vendor/ggml/include/ggml.h:390-405)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 15, 30
Q4_1, Q5_0, Q5_1, Q8_1 = 3, 6, 7, 9
Q2_K, Q3_K = 10, 11
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292),
         Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_1: (32, 36), F32: (1, 4), F16: (1, 2), BF16: (1, 2),
         Q2_K: (256, 84), Q3_K: (256, 110)}
# ggml's vec_dot_type: what src1 is converted to (float weights: their own type)
VEC_DOT_TYPE = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K, Q4_1: Q8_1, Q5_0: Q8_0, Q5_1: Q8_1,
                F32: F32, F16: F16, BF16: BF16, Q2_K: Q8_K, Q3_K: Q8_K}
TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K",
              BF16: "bf16", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q8_1: "q8_1", Q2_K: "q2_K", Q3_K: "q3_K"}
TYPES_BY_NAME = {v: k for k, v in TYPE_NAMES.items()}

STATUS = {0: "OK", 1: "NO_DEVICE", 2: "UNSUPPORTED", 3: "INVALID", 4: "ALLOC", 5: "EXECUTION"}

# Every symbol include/tlhip.h declares.
EXPORTS = (
    "tlh_last_error", "tlh_status_name", "tlh_version", "tlh_device_count", "tlh_device_open", "tlh_alloc",
    "tlh_free", "tlh_h2d", "tlh_d2h", "tlh_stream_sync", "tlh_mul_mat_scratch_bytes", "tlh_mul_mat",
    "tlh_mul_mat_noalloc", "tlh_mul_mat_quantize", "tlh_mul_mat_compute", "tlh_mul_mat_id_scratch_bytes", "tlh_mul_mat_id",
    "tlh_quantize_act", "tlh_dequantize", "tlh_flash_attn_ext_scratch_bytes", "tlh_flash_attn_ext",
    "tlh_paged_attention_scratch_bytes", "tlh_paged_attention", "tlh_reshape_and_cache",
    "tlh_core_check", "tlh_core", "tlh_program_compile", "tlh_program_destroy", "tlh_copy", "tlh_memset",
    "tlh_read_floor",
    "tlh_program_input",
    "tlh_program_tensor", "tlh_program_run", "tlh_program_stats", "tlh_program_profile", "tlh_program_trace",
    "tlh_program_plan",
    "tlh_gguf_open", "tlh_gguf_close", "tlh_gguf_counts", "tlh_gguf_tensor", "tlh_gguf_find_tensor",
    "tlh_gguf_find_key", "tlh_gguf_key", "tlh_gguf_value", "tlh_gguf_string", "tlh_gguf_layout", "tlh_gguf_upload",
)


class TlhError(RuntimeError):
    """A failed call: .status is the tlh_status name (mirrors tensorlisp_kernels::Error)."""

    def __init__(self, status: int, msg: str):
        self.status = STATUS.get(status, str(status))
        super().__init__(f"{self.status}: {msg}")


class TlhTensor(C.Structure):
    _fields_ = [("ne", C.c_int64 * 4), ("nb", C.c_int64 * 4), ("ty", C.c_int32), ("pad_", C.c_int32)]


class TlhOp(C.Structure):
    _fields_ = [("t", TlhTensor * 5), ("x", C.c_int64 * 12)]


class TlhDeviceProps(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 32), ("compute_units", C.c_int),
                ("wave_size", C.c_int), ("lds_bytes", C.c_int), ("clock_khz", C.c_int), ("hbm_bytes", C.c_int64)]


class TlhPagedArgs(C.Structure):
    _fields_ = [("out", C.c_void_p), ("q", C.c_void_p), ("k_cache", C.c_void_p), ("v_cache", C.c_void_p),
                ("block_tables", C.c_void_p), ("context_lens", C.c_void_p), ("num_seqs", C.c_int32),
                ("num_heads", C.c_int32), ("num_kv_heads", C.c_int32), ("head_size", C.c_int32),
                ("block_size", C.c_int32), ("max_blocks_per_seq", C.c_int32), ("max_context_len", C.c_int32),
                ("scale", C.c_float)]


assert C.sizeof(TlhOp) == 456, C.sizeof(TlhOp)


def load_library(path: Path = LIB_PATH) -> C.CDLL:
    if not path.exists():
        raise ImportError(f"{path} is missing: build it with `python -m tensorlisp_amd.build` (no fallback exists)")
    L = C.CDLL(str(path))
    vp, i64, st = C.c_void_p, C.c_int64, C.c_int
    L.tlh_last_error.restype = C.c_char_p
    L.tlh_status_name.restype = C.c_char_p
    L.tlh_status_name.argtypes = [C.c_int]
    L.tlh_version.restype = C.c_char_p
    L.tlh_device_count.argtypes = [C.POINTER(C.c_int)]
    L.tlh_device_open.argtypes = [C.c_int, C.POINTER(TlhDeviceProps)]
    L.tlh_alloc.argtypes = [C.c_size_t, C.POINTER(C.c_void_p)]
    L.tlh_free.argtypes = [vp]
    L.tlh_h2d.argtypes = [vp, vp, C.c_size_t]
    L.tlh_d2h.argtypes = [vp, vp, C.c_size_t]
    L.tlh_stream_sync.argtypes = [vp]
    L.tlh_mul_mat_scratch_bytes.argtypes = [C.POINTER(TlhOp), C.POINTER(C.c_size_t)]
    L.tlh_mul_mat.argtypes = [C.POINTER(TlhOp), vp, vp, vp, vp, C.c_size_t, vp]
    L.tlh_mul_mat_noalloc.argtypes = [C.POINTER(TlhOp), vp, vp, vp, vp]
    L.tlh_mul_mat_quantize.argtypes = [C.POINTER(TlhOp), vp, vp, C.c_size_t, vp]
    L.tlh_mul_mat_compute.argtypes = [C.POINTER(TlhOp), vp, vp, C.c_size_t, vp, vp]
    L.tlh_mul_mat_id_scratch_bytes.argtypes = [C.POINTER(TlhOp), C.POINTER(C.c_size_t)]
    L.tlh_mul_mat_id.argtypes = [C.POINTER(TlhOp), vp, vp, vp, vp, vp, C.c_size_t, vp]
    L.tlh_quantize_act.argtypes = [C.c_int, vp, i64, i64, i64, vp, vp]
    L.tlh_dequantize.argtypes = [C.c_int, vp, i64, i64, i64, vp, vp]
    L.tlh_flash_attn_ext_scratch_bytes.argtypes = [C.POINTER(TlhOp), C.POINTER(C.c_size_t)]
    L.tlh_flash_attn_ext.argtypes = [C.POINTER(TlhOp), vp, vp, vp, vp, vp, vp, C.c_size_t, vp]
    L.tlh_paged_attention_scratch_bytes.argtypes = [C.POINTER(TlhPagedArgs), C.POINTER(C.c_size_t)]
    L.tlh_paged_attention.argtypes = [C.POINTER(TlhPagedArgs), vp, C.c_size_t, vp]
    L.tlh_reshape_and_cache.argtypes = [vp, vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int64, vp]
    L.tlh_core_check.argtypes = [C.c_int, C.POINTER(TlhOp), C.c_int, C.c_int]
    L.tlh_core.argtypes = [C.c_int, C.POINTER(TlhOp), vp, vp, vp, vp, vp]
    i32p, i64p = C.POINTER(C.c_int32), C.POINTER(C.c_int64)
    L.tlh_program_compile.argtypes = [vp, C.c_int32, i32p, C.c_int32, i32p, C.c_int32, C.POINTER(C.c_void_p),
                                      C.c_int32, i64p, C.c_int32, C.POINTER(C.c_void_p)]
    L.tlh_program_destroy.argtypes = [vp]
    L.tlh_copy.argtypes = [vp, vp, C.c_size_t, vp]
    L.tlh_memset.argtypes = [vp, C.c_int, C.c_size_t, vp]
    L.tlh_read_floor.argtypes = [vp, C.c_size_t, C.c_int32, C.c_int32, vp]
    L.tlh_program_input.argtypes = [vp, C.c_int32, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    L.tlh_program_tensor.argtypes = [vp, C.c_int32, vp, C.POINTER(C.c_void_p)]
    L.tlh_program_run.argtypes = [vp, vp, vp, C.c_int32]
    L.tlh_program_stats.argtypes = [vp, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t), C.POINTER(C.c_int32)]
    L.tlh_program_profile.argtypes = [vp, vp, vp, C.POINTER(C.c_float), C.c_int32]
    L.tlh_program_trace.argtypes = [vp, vp, vp, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]
    L.tlh_program_plan.argtypes = [vp, C.c_int32, i32p, C.c_int32, i32p, C.c_int32, i64p, i64p,
                                   C.POINTER(C.c_size_t)]
    u64p, cpp = C.POINTER(C.c_uint64), C.POINTER(C.c_char_p)
    L.tlh_gguf_open.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
    L.tlh_gguf_close.argtypes = [vp]
    L.tlh_gguf_counts.argtypes = [vp, C.POINTER(C.c_uint32), i64p, i64p, u64p, u64p]
    L.tlh_gguf_tensor.argtypes = [vp, C.c_int64, vp]
    L.tlh_gguf_find_tensor.argtypes = [vp, C.c_char_p, i64p]
    L.tlh_gguf_find_key.argtypes = [vp, C.c_char_p, i64p]
    L.tlh_gguf_key.argtypes = [vp, C.c_int64, cpp, C.POINTER(C.c_int32), C.POINTER(C.c_int32), u64p]
    L.tlh_gguf_value.argtypes = [vp, C.c_int64, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    L.tlh_gguf_string.argtypes = [vp, C.c_int64, C.c_uint64, cpp, u64p]
    L.tlh_gguf_layout.argtypes = [vp, u64p, u64p]
    L.tlh_gguf_upload.argtypes = [vp, vp, u64p, vp]
    for name in EXPORTS:
        if name not in ("tlh_last_error", "tlh_status_name", "tlh_version"):
            getattr(L, name).restype = st
    return L


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise TlhError(status, lib().tlh_last_error().decode())


def row_bytes(t: int, k: int) -> int:
    be, bb = BLOCK[t]
    if k % be:
        raise ValueError(f"k={k} is not a multiple of the {TYPE_NAMES[t]} block ({be})")
    return k // be * bb


def ggml_tensor(ty: int, ne, nb=None) -> TlhTensor:
    """A ggml-style tensor descriptor; nb defaults to the contiguous strides of `ty`."""
    ne = list(ne) + [1] * (4 - len(ne))
    t = TlhTensor()
    if nb is None:
        if ty in BLOCK:
            be, bb = BLOCK[ty]
            nb0, nb1 = bb, ne[0] // be * bb
        else:
            nb0 = {F32: 4, F16: 2, 26: 4, 27: 8}[ty]  # f32, f16, i32, i64
            nb1 = nb0 * ne[0]
        nb = [nb0, nb1, nb1 * ne[1], nb1 * ne[1] * ne[2]]
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    t.ty = int(ty)
    return t


def mul_mat_op(wtype: int, M: int, K: int, N: int, ne2: int = 1, ne3: int = 1, w_ne2: int = 1,
               w_ne3: int = 1, x_nb=None, w_nb=None, d_nb=None, xtype: int = F32) -> TlhOp:
    """The MUL_MAT descriptor of Ctx::mul_mat (lower.rs:543-571): t0 weights [K, M], t1 [K, N] (f32, or the
    f16 / bf16 of f16 / bf16 weights), t4 f32 [M, N]."""
    op = TlhOp()
    op.t[0] = ggml_tensor(wtype, [K, M, w_ne2, w_ne3], w_nb)
    op.t[1] = ggml_tensor(xtype, [K, N, ne2, ne3], x_nb)
    op.t[4] = ggml_tensor(F32, [M, N, ne2, ne3], d_nb)
    op.x[0] = ne2 // w_ne2
    op.x[1] = ne3 // w_ne3
    return op


def _stream(stream):
    import torch

    if stream is None:
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return C.c_void_p(getattr(stream, "cuda_stream", stream))


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def device_props(ordinal: int = 0) -> dict:
    p = TlhDeviceProps()
    check(lib().tlh_device_open(ordinal, C.byref(p)))
    return {"name": p.name.decode(), "arch": p.arch.decode(), "compute_units": p.compute_units,
            "wave_size": p.wave_size, "lds_bytes": p.lds_bytes, "clock_khz": p.clock_khz, "hbm_bytes": p.hbm_bytes}


def device_count() -> int:
    n = C.c_int()
    check(lib().tlh_device_count(C.byref(n)))
    return n.value


def mul_mat_scratch_bytes(op: TlhOp) -> int:
    n = C.c_size_t()
    check(lib().tlh_mul_mat_scratch_bytes(C.byref(op), C.byref(n)))
    return n.value


class MulMat:
    """One GGML_OP_MUL_MAT node with its scratch, launched many times (what a lowered
    Dispatch is in crates/kernels/src/cuda/exec.rs:186-225)."""

    def __init__(self, wtype: int, M: int, K: int, N: int, device="cuda", op: TlhOp = None):
        import torch

        self.wtype, self.M, self.K, self.N = wtype, M, K, N
        self.op = mul_mat_op(wtype, M, K, N) if op is None else op
        self.scratch_bytes = mul_mat_scratch_bytes(self.op)
        self.scratch = torch.empty(max(self.scratch_bytes, 256) + 256, dtype=torch.uint8, device=device)
        off = (-self.scratch.data_ptr()) % 256
        self.scratch_ptr = C.c_void_p(self.scratch.data_ptr() + off)

    def __call__(self, w, x, y, stream=None):
        check(lib().tlh_mul_mat(C.byref(self.op), _ptr(w), _ptr(x), _ptr(y), self.scratch_ptr,
                                self.scratch_bytes, _stream(stream)))
        return y

    def quantize(self, x, stream=None):
        """Phase 1 only: x -> the node's scratch."""
        check(lib().tlh_mul_mat_quantize(C.byref(self.op), _ptr(x), self.scratch_ptr, self.scratch_bytes,
                                         _stream(stream)))

    def compute(self, w, y, stream=None):
        """Phase 2 only: the products from the scratch the last quantize() filled."""
        check(lib().tlh_mul_mat_compute(C.byref(self.op), _ptr(w), self.scratch_ptr, self.scratch_bytes, _ptr(y),
                                        _stream(stream)))
        return y


def mul_mat(wtype: int, w, M: int, K: int, x, stream=None):
    """y [N, M] f32 = x [N, K] @ dequant(W [M rows of K])^T, computed as ggml's CPU mul_mat does."""
    import torch

    x = x.contiguous()
    N = x.shape[0]
    y = torch.empty((N, M), dtype=torch.float32, device=x.device)
    MulMat(wtype, M, K, N, device=x.device)(w, x, y, stream)
    return y


def mul_mat_views(w, x, out=None, stream=None, split: bool = False):
    """ggml_mul_mat on torch views of float weights: w (w3, w2, M, K) f32 / f16 /
    bf16, x (n3, n2, N, K) f32 or w's dtype, out (n3, n2, N, M) f32 (ggml's ne
    reversed; fewer leading dims are 1). Any element-aligned strides with K
    contiguous; w's batch dims broadcast over x's (r2 = n2 / w2, r3 = n3 / w3).
    split: src1's conversion and the products as two launches
    (tlh_mul_mat_quantize + tlh_mul_mat_compute) instead of one."""
    import torch

    wt, xt = _ggml_type(w), _ggml_type(x)
    lead = lambda t: [1] * (4 - t.dim()) + list(t.shape[:-2])  # noqa: E731
    n3, n2 = lead(x)[-2:]
    if out is None:
        out = torch.empty((n3, n2, x.shape[-2], w.shape[-2]), dtype=torch.float32, device=x.device)
    op = TlhOp()
    op.t[0], op.t[1], op.t[4] = tensor_desc(w, wt), tensor_desc(x, xt), tensor_desc(out, F32)
    w3, w2 = lead(w)[-2:]
    op.x[0], op.x[1] = n2 // max(w2, 1), n3 // max(w3, 1)
    mm = MulMat(wt, w.shape[-2], w.shape[-1], x.shape[-2], device=x.device, op=op)
    if split:
        mm.quantize(x, stream)
        mm.compute(w, out, stream)
    else:
        mm(w, x, out, stream)
    return out


def quantize_act(wtype: int, x, stream=None):
    """x [rows, k] f32 -> uint8 [rows, row_bytes(vec_dot_type, k)] in ggml's block layout."""
    import torch

    rows, k = x.shape
    assert x.dtype == torch.float32 and x.stride(1) == 1
    out = torch.empty((rows, row_bytes(VEC_DOT_TYPE[wtype], k)), dtype=torch.uint8, device=x.device)
    check(lib().tlh_quantize_act(wtype, _ptr(x), k, rows, x.stride(0) * 4, _ptr(out), _stream(stream)))
    return out


def memset(t, value: int, nbytes: int = None, offset: int = 0, stream=None) -> None:
    """Fill `nbytes` bytes of device tensor t (from byte `offset`; all of it by
    default) with the low 8 bits of value, on `stream` (tlh_memset)."""
    n = t.numel() * t.element_size() - offset if nbytes is None else nbytes
    check(lib().tlh_memset(C.c_void_p(t.data_ptr() + offset), int(value), n, _stream(stream)))


def dequantize(wtype: int, w, k: int, stream=None):
    """uint8 [rows, row_bytes] -> f32 [rows, k]."""
    import torch

    rows = w.shape[0]
    y = torch.empty((rows, k), dtype=torch.float32, device=w.device)
    check(lib().tlh_dequantize(wtype, _ptr(w), k, rows, w.stride(0), _ptr(y), _stream(stream)))
    return y


def _f32_bits(x: float) -> int:
    """A float op parameter as OpBlob::float stores it (lower.rs:96-98): the f32
    bit pattern, sign-extended to 64 bits."""
    import struct

    return struct.unpack("<i", struct.pack("<f", x))[0]


def flash_attn_params(n_head: int, scale: float, max_bias: float = 0.0, softcap: float = 0.0):
    """(scale, max_bias, m0, m1, n_head_log2, softcap) as Ctx::flash_attn_ext derives
    them (lower.rs:604-620), in f32 arithmetic."""
    import numpy as np

    f = np.float32
    scale, max_bias, softcap = f(scale), f(max_bias), f(softcap)
    if softcap != 0:
        scale = f(scale / softcap)
    nhl2 = 1 << int(np.floor(np.log2(f(n_head))))
    m0 = f(np.power(f(2.0), f(-max_bias / f(nhl2))))
    m1 = f(np.power(f(2.0), f(-(max_bias / f(2.0)) / f(nhl2))))
    return float(scale), float(max_bias), float(m0), float(m1), nhl2, float(softcap)


def _ggml_type(t) -> int:
    import torch

    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}.get(t.dtype, -1)


def tensor_desc(t, ty: int) -> TlhTensor:
    """The ggml descriptor of a torch tensor whose shape is ggml's ne reversed
    (torch (n3, n2, n1, n0) <-> ggml [n0, n1, n2, n3]); strides follow the view."""
    shape = list(t.shape)[::-1] + [1] * (4 - t.dim())
    if t.numel() == 0:  # an empty view's strides are arbitrary: use ggml's contiguous ones
        strides = [t.element_size()]
        for i in range(1, 4):
            strides.append(strides[-1] * max(shape[i - 1], 1))
        return ggml_tensor(ty, shape, strides)
    strides = [s * t.element_size() for s in list(t.stride())[::-1]]
    for i in range(t.dim(), 4):
        strides.append(strides[-1] * shape[i - 1] if strides else t.element_size())
    return ggml_tensor(ty, shape, strides)


def flash_attn_op(q, k, v, mask, dst, scale: float, max_bias: float = 0.0, softcap: float = 0.0) -> TlhOp:
    """The FLASH_ATTN_EXT descriptor Ctx::flash_attn_ext packs (lower.rs:611-621):
    t0 q, t1 k, t2 v, t3 mask (zeros when absent), t4 dst; x0..x5 the parameters."""
    op = TlhOp()
    op.t[0] = tensor_desc(q, _ggml_type(q))
    op.t[1] = tensor_desc(k, _ggml_type(k))
    op.t[2] = tensor_desc(v, _ggml_type(v))
    if mask is not None:
        op.t[3] = tensor_desc(mask, _ggml_type(mask))
    op.t[4] = tensor_desc(dst, _ggml_type(dst))
    sc, mb, m0, m1, nhl2, cap = flash_attn_params(int(op.t[0].ne[2]), scale, max_bias, softcap)
    op.x[0], op.x[1], op.x[2], op.x[3] = _f32_bits(sc), _f32_bits(mb), _f32_bits(m0), _f32_bits(m1)
    op.x[4] = nhl2
    op.x[5] = _f32_bits(cap)
    return op


def flash_attn_scratch_bytes(op: TlhOp) -> int:
    n = C.c_size_t()
    check(lib().tlh_flash_attn_ext_scratch_bytes(C.byref(op), C.byref(n)))
    return n.value


class FlashAttnExt:
    """One GGML_OP_FLASH_ATTN_EXT node with its split-key scratch. Tensors are torch
    views whose shapes are ggml's ne reversed: q f32 (nb, nh, nq, D), k f16
    (nbk, nhkv, L, D), v f16 (nbk, nhkv, L, DV), mask f16 (mne3, mne2, >= nq, >= L)
    or None, dst f32 (nb, nq, nh, DV)."""

    def __init__(self, q, k, v, mask, dst, scale: float, max_bias: float = 0.0, softcap: float = 0.0):
        import torch

        self.op = flash_attn_op(q, k, v, mask, dst, scale, max_bias, softcap)
        self.scratch_bytes = flash_attn_scratch_bytes(self.op)
        self.scratch = torch.empty(max(self.scratch_bytes, 4), dtype=torch.uint8, device=q.device)

    def __call__(self, q, k, v, mask, dst, stream=None):
        check(lib().tlh_flash_attn_ext(C.byref(self.op), _ptr(q), _ptr(k), _ptr(v),
                                       _ptr(mask) if mask is not None else None, _ptr(dst), _ptr(self.scratch),
                                       self.scratch_bytes, _stream(stream)))
        return dst


def flash_attn_ext(q, k, v, mask=None, scale: float = 1.0, max_bias: float = 0.0, softcap: float = 0.0,
                   stream=None):
    """ggml_flash_attn_ext(q, k, v, mask, scale, max_bias, softcap) on torch views
    (shapes as in FlashAttnExt) -> dst f32 (nb, nq, nh, DV), ggml [DV, nh, nq, nb]."""
    import torch

    nb, nh, nq, _ = q.shape
    dst = torch.empty((nb, nq, nh, v.shape[-1]), dtype=torch.float32, device=q.device)
    return FlashAttnExt(q, k, v, mask, dst, scale, max_bias, softcap)(q, k, v, mask, dst, stream)


class PagedAttention:
    """The `paged-attention` node (crates/tensorlisp/src/scheme/core.ss:251-258) with its scratch."""

    def __init__(self, num_seqs, num_heads, num_kv_heads, head_size, block_size, max_blocks_per_seq,
                 max_context_len, scale, device="cuda"):
        import torch

        self.args = TlhPagedArgs()
        a = self.args
        a.num_seqs, a.num_heads, a.num_kv_heads = num_seqs, num_heads, num_kv_heads
        a.head_size, a.block_size = head_size, block_size
        a.max_blocks_per_seq, a.max_context_len, a.scale = max_blocks_per_seq, max_context_len, scale
        n = C.c_size_t()
        check(lib().tlh_paged_attention_scratch_bytes(C.byref(a), C.byref(n)))
        self.scratch_bytes = n.value
        self.scratch = torch.empty(max(n.value, 4), dtype=torch.uint8, device=device)

    def __call__(self, out, q, k_cache, v_cache, block_tables, context_lens, stream=None):
        a = self.args
        a.out, a.q, a.k_cache, a.v_cache = out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()
        a.block_tables, a.context_lens = block_tables.data_ptr(), context_lens.data_ptr()
        check(lib().tlh_paged_attention(C.byref(a), _ptr(self.scratch), self.scratch_bytes, _stream(stream)))
        return out


def paged_attention(q, k_cache, v_cache, block_tables, context_lens, block_size, max_context_len, scale,
                    num_kv_heads, stream=None):
    """q f16 [seqs, heads, hs] -> out f16 [seqs, heads, hs] (vLLM cache layouts)."""
    import torch

    seqs, heads, hs = q.shape
    out = torch.empty_like(q)
    pa = PagedAttention(seqs, heads, num_kv_heads, hs, block_size, block_tables.shape[1], max_context_len, scale,
                        device=q.device)
    return pa(out, q.contiguous(), k_cache, v_cache, block_tables.contiguous(), context_lens.contiguous(), stream)


def reshape_and_cache(key, value, k_cache, v_cache, slots, num_kv_heads, block_size, stream=None):
    """key/value f16 [tokens, kv_heads*hs] scattered into the caches; slots i64 [tokens] (negative = skip;
    at or past the pools' end = dropped)."""
    tokens = key.shape[0]
    hs = key.shape[1] // num_kv_heads
    num_blocks = min(k_cache.numel(), v_cache.numel()) // (num_kv_heads * hs * block_size)
    check(lib().tlh_reshape_and_cache(_ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slots), tokens,
                                      num_kv_heads, hs, block_size, num_blocks, _stream(stream)))


# ------------------------------------------------------------------ core ops
# The ops around MUL_MAT and attention in a decoder step, packed as the
# reference's lowering packs them for its core kernels
# (crates/kernels/src/cuda/lower.rs:175-500) and run by tlh_core.
(CORE_BIN, CORE_UNARY, CORE_NORM, CORE_GET_ROWS, CORE_SET_ROWS, CORE_CPY, CORE_ROPE, CORE_SOFT_MAX, CORE_ARGMAX,
 CORE_GLU) = range(1, 11)
I32, I64 = 26, 27
# ggml_unary_op codes (ggml.h) and the lowering's extra element-wise codes
UNARY = {"abs": 0, "sgn": 1, "neg": 2, "step": 3, "tanh": 4, "elu": 5, "relu": 6, "sigmoid": 7, "gelu": 8,
         "gelu_quick": 9, "silu": 10, "hardswish": 11, "hardsigmoid": 12, "exp": 13, "expm1": 14, "softplus": 15,
         "gelu_erf": 16, "floor": 18, "ceil": 19, "round": 20, "trunc": 21, "scale": 100, "fill": 101,
         "clamp": 102, "leaky_relu": 103, "sqr": 104, "sqrt": 105, "sin": 106, "cos": 107, "log": 108}
# ggml_glu_op codes (ggml.h:623-630); swiglu_oai is not supported
GLU = {"reglu": 0, "geglu": 1, "swiglu": 2, "geglu_erf": 4, "geglu_quick": 5}

_libm = None


def _f32_fn(name: str):
    """The C library's single-precision `name` (powf, logf, ...): the host-side
    parameters below are derived with the same f32 functions the CPU backend
    and the reference's lowering call, so they match bit for bit."""
    global _libm
    if _libm is None:
        _libm = C.CDLL("libm.so.6")
    f = getattr(_libm, name)
    f.restype = C.c_float
    f.argtypes = [C.c_float] * (2 if name == "powf" else 1)
    return f


def _f32(x) -> float:
    import struct

    return struct.unpack("<f", struct.pack("<f", x))[0]


def core_type(t) -> int:
    import torch

    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int32: I32,
            torch.int64: I64}.get(t.dtype, -1)


def quant_desc(t, wtype: int, k: int) -> TlhTensor:
    """The ggml descriptor of quantized rows held as a uint8 torch tensor of shape
    (..., rows, row_bytes): ne [k, rows, ...], nb from the tensor's byte strides."""
    rb = row_bytes(wtype, k)
    if t.shape[-1] != rb or t.stride(-1) != 1:
        raise ValueError(f"rows must be {rb} contiguous bytes for {TYPE_NAMES[wtype]} k={k}")
    lead = list(t.shape[:-1])[::-1] + [1] * (4 - t.dim())
    nbs = [s for s in list(t.stride()[:-1])[::-1]]
    while len(nbs) < 3:
        nbs.append(nbs[-1] * lead[len(nbs) - 1] if nbs else rb)
    return ggml_tensor(wtype, [k] + lead[:3], [BLOCK[wtype][1]] + nbs[:3])


def core_op(srcs, dst, x=()) -> TlhOp:
    """t[0..2] = the sources (torch tensors, TlhTensor descriptors or None),
    t[4] = dst, x[] = the op's parameters."""
    op = TlhOp()
    for i, t in enumerate(srcs):
        if t is None:
            continue
        op.t[i] = t if isinstance(t, TlhTensor) else tensor_desc(t, core_type(t))
    op.t[4] = dst if isinstance(dst, TlhTensor) else tensor_desc(dst, core_type(dst))
    for i, v in enumerate(x):
        op.x[i] = v
    return op


class CoreOp:
    """One core node, validated once (tlh_core_check) and run on each call."""

    def __init__(self, kind: int, op: TlhOp, has_src1: bool, has_src2: bool):
        self.kind, self.op = kind, op
        check(lib().tlh_core_check(kind, C.byref(op), int(has_src1), int(has_src2)))

    def __call__(self, src0, src1, src2, dst, stream=None):
        p = lambda t: _ptr(t) if t is not None else None  # noqa: E731
        check(lib().tlh_core(self.kind, C.byref(self.op), p(src0), p(src1), p(src2), _ptr(dst), _stream(stream)))
        return dst


def _run(kind, srcs, dst, x=(), descs=None, stream=None):
    op = core_op(descs if descs is not None else srcs, dst, x)
    s = list(srcs) + [None] * (3 - len(srcs))
    return CoreOp(kind, op, s[1] is not None, s[2] is not None)(s[0], s[1], s[2], dst, stream)


def _out(like, out, dtype=None):
    import torch

    return out if out is not None else torch.empty(like.shape, dtype=dtype or like.dtype, device=like.device)


def binary(code: int, a, b, out=None, stream=None):
    """ADD/SUB/MUL/DIV (code 0..3) with b repeated to a's shape (lower.rs:219-248)."""
    return _run(CORE_BIN, [a, b], _out(a, out), (code,), stream=stream)


def add(a, b, out=None, stream=None):
    return binary(0, a, b, out, stream)


def mul(a, b, out=None, stream=None):
    return binary(2, a, b, out, stream)


def unary(op, a, p1: float = 0.0, p2: float = 0.0, out=None, stream=None):
    """A ggml unary op or the lowering's element-wise extras (lower.rs:250-290),
    by name or code: scale (p1 s, p2 b), fill (p1), clamp (p1 min, p2 max),
    leaky_relu (p1 slope)."""
    code = UNARY[op] if isinstance(op, str) else int(op)
    return _run(CORE_UNARY, [a], _out(a, out), (code, _f32_bits(p1), _f32_bits(p2)), stream=stream)


def norm(a, eps: float, rms: bool = False, out=None, stream=None):
    """ggml_norm / ggml_rms_norm over ne0 (lower.rs:292-312)."""
    return _run(CORE_NORM, [a], _out(a, out), (int(rms), _f32_bits(eps)), stream=stream)


def rms_norm(a, eps: float, out=None, stream=None):
    return norm(a, eps, True, out, stream)


def get_rows(a, idx, wtype: int = None, k: int = None, out=None, stream=None):
    """ggml_get_rows: out (i3, i2, i1) row = a's row idx[i3, i2, i1] of plane
    (i2, i3). `a` is f32/f16, or quantized rows (uint8, (..., rows, row_bytes))
    with `wtype` and their element count `k`. out is f32 (..., n_idx, ne0)."""
    import torch

    ad = quant_desc(a, wtype, k) if wtype is not None else tensor_desc(a, core_type(a))
    ne0 = k if wtype is not None else a.shape[-1]
    if out is None:
        out = torch.empty(tuple(idx.shape) + (ne0,), dtype=torch.float32, device=idx.device)
    return _run(CORE_GET_ROWS, [a, idx], out, descs=[ad, idx], stream=stream)


def set_rows(dst, src, idx, stream=None):
    """ggml_set_rows: src row (i3, i2, i1) to dst row idx[i3 % n2, i2 % n1, i1]."""
    return _run(CORE_SET_ROWS, [src, idx], dst, stream=stream)


def cpy(src, dst, wtype: int = None, k: int = None, stream=None):
    """ggml_cpy / ggml_cont / ggml_dup: element i of src (row-major over ggml's
    ne) to element i of dst, converted to dst's type."""
    sd = quant_desc(src, wtype, k) if wtype is not None else tensor_desc(src, core_type(src))
    return _run(CORE_CPY, [src], dst, descs=[sd], stream=stream)


def rope_params(n_dims: int, mode: int, n_ctx_orig: int, freq_base: float, freq_scale: float, ext_factor: float,
                attn_factor: float, beta_fast: float, beta_slow: float, has_ff: bool):
    """x[] of Ctx::rope (lower.rs:422-466): the YaRN corr dims of
    ggml_rope_yarn_corr_dims (ggml.c:4369-4381) and theta_scale =
    freq_base^(-2/n_dims), all in f32."""
    import numpy as np

    powf, logf = _f32_fn("powf"), _f32_fn("logf")
    f = np.float32
    with np.errstate(all="ignore"):  # beta 0 or n_ctx_orig 0 give inf / nan, as in C
        def corr(beta):
            ratio = f(n_ctx_orig) / (f(beta) * f(2.0) * f(np.pi))
            return f(f(n_dims) * f(logf(float(ratio)))) / f(f(2.0) * f(logf(freq_base)))

        start, end = np.floor(corr(beta_fast)), np.ceil(corr(beta_slow))
    c0 = 0.0 if 0.0 > start else float(start)  # MAX(0, start) and MIN(n_dims - 1, end) of ggml.c
    c1 = float(n_dims - 1) if n_dims - 1 < end else float(end)
    ts = powf(freq_base, _f32(-2.0 / n_dims))
    return (n_dims, mode, _f32_bits(freq_scale), _f32_bits(ext_factor), _f32_bits(attn_factor), _f32_bits(ts),
            _f32_bits(c0), _f32_bits(c1), int(has_ff))


def rope(a, pos, n_dims: int, mode: int = 0, n_ctx_orig: int = 0, freq_base: float = 10000.0,
         freq_scale: float = 1.0, ext_factor: float = 0.0, attn_factor: float = 1.0, beta_fast: float = 32.0,
         beta_slow: float = 1.0, freq_factors=None, out=None, stream=None):
    """ggml_rope_ext on a (ggml [ne0, heads, tokens, ne3]) with i32 positions [tokens]."""
    x = rope_params(n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor, beta_fast,
                    beta_slow, freq_factors is not None)
    return _run(CORE_ROPE, [a, pos, freq_factors], _out(a, out), x, stream=stream)


def soft_max_params(n_head: int, scale: float, max_bias: float):
    """x[] of Ctx::soft_max (lower.rs:314-341): scale, max_bias, m0, m1, n_head_log2."""
    import math

    powf = _f32_fn("powf")
    nhl2 = 1 << int(math.floor(math.log2(n_head))) if n_head > 0 else 1
    m0 = powf(2.0, _f32(_f32(-max_bias) / nhl2))
    m1 = powf(2.0, _f32(_f32(-_f32(max_bias / 2.0)) / nhl2))
    return (_f32_bits(scale), _f32_bits(max_bias), _f32_bits(m0), _f32_bits(m1), nhl2)


def soft_max(a, mask=None, scale: float = 1.0, max_bias: float = 0.0, out=None, stream=None):
    """ggml_soft_max_ext over ne0 of f32 a, with an optional f16/f32 mask
    (ggml [ne0, >= rows, broadcast over heads / batches])."""
    n_head = a.shape[-3] if a.dim() >= 3 else 1
    return _run(CORE_SOFT_MAX, [a, mask], _out(a, out), soft_max_params(n_head, scale, max_bias), stream=stream)


def argmax(a, out=None, stream=None):
    """ggml_argmax of f32 a (rows, n) -> i32 (rows,): the last index of each row's maximum."""
    import torch

    if out is None:
        out = torch.empty((a.shape[0],), dtype=torch.int32, device=a.device)
    return _run(CORE_ARGMAX, [a], out, stream=stream)


def glu(op, a, b=None, swapped: bool = False, out=None, stream=None):
    """GGML_OP_GLU on f32 rows: act(x) * g with x, g = a, b (ggml_glu_split) or
    the two halves of a's rows (ggml_glu; x first unless swapped)."""
    import torch

    code = GLU[op] if isinstance(op, str) else int(op)
    if out is None:
        shape = tuple(a.shape) if b is not None else tuple(a.shape[:-1]) + (a.shape[-1] // 2,)
        out = torch.empty(shape, dtype=torch.float32, device=a.device)
    return _run(CORE_GLU, [a, b], out, (code, int(swapped)), stream=stream)

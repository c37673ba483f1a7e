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
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 14, 15
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}
VEC_DOT_TYPE = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K}
TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q6_K: "q6_K", Q8_K: "q8_K"}
TYPES_BY_NAME = {v: k for k, v in TYPE_NAMES.items()}

STATUS = {0: "OK", 1: "NO_DEVICE", 2: "UNSUPPORTED", 3: "INVALID", 4: "ALLOC", 5: "EXECUTION"}

# Every symbol include/tlhip.h declares.
EXPORTS = (
    "tlh_last_error", "tlh_status_name", "tlh_version", "tlh_device_count", "tlh_device_open", "tlh_alloc",
    "tlh_free", "tlh_h2d", "tlh_d2h", "tlh_stream_sync", "tlh_mul_mat_scratch_bytes", "tlh_mul_mat",
    "tlh_mul_mat_quantize", "tlh_mul_mat_compute",
    "tlh_quantize_act", "tlh_dequantize", "tlh_flash_attn_ext_scratch_bytes", "tlh_flash_attn_ext",
    "tlh_paged_attention_scratch_bytes", "tlh_paged_attention", "tlh_reshape_and_cache",
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
    L.tlh_mul_mat_quantize.argtypes = [C.POINTER(TlhOp), vp, vp, C.c_size_t, vp]
    L.tlh_mul_mat_compute.argtypes = [C.POINTER(TlhOp), vp, vp, C.c_size_t, vp, vp]
    L.tlh_quantize_act.argtypes = [C.c_int, vp, i64, i64, i64, vp, vp]
    L.tlh_dequantize.argtypes = [C.c_int, vp, i64, i64, i64, vp, vp]
    L.tlh_flash_attn_ext_scratch_bytes.argtypes = [C.POINTER(TlhOp), C.POINTER(C.c_size_t)]
    L.tlh_flash_attn_ext.argtypes = [C.POINTER(TlhOp), vp, vp, vp, vp, vp, vp, C.c_size_t, vp]
    L.tlh_paged_attention_scratch_bytes.argtypes = [C.POINTER(TlhPagedArgs), C.POINTER(C.c_size_t)]
    L.tlh_paged_attention.argtypes = [C.POINTER(TlhPagedArgs), vp, C.c_size_t, vp]
    L.tlh_reshape_and_cache.argtypes = [vp, vp, vp, vp, vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, vp]
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
            nb0 = 4 if ty == F32 else 2
            nb1 = nb0 * ne[0]
        nb = [nb0, nb1, nb1 * ne[1], nb1 * ne[1] * ne[2]]
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    t.ty = int(ty)
    return t


def mul_mat_op(wtype: int, M: int, K: int, N: int, ne2: int = 1, ne3: int = 1, w_ne2: int = 1,
               w_ne3: int = 1, x_nb=None, w_nb=None, d_nb=None) -> TlhOp:
    """The MUL_MAT descriptor of Ctx::mul_mat (lower.rs:543-571): t0 weights [K, M], t1 f32 [K, N], t4 f32 [M, N]."""
    op = TlhOp()
    op.t[0] = ggml_tensor(wtype, [K, M, w_ne2, w_ne3], w_nb)
    op.t[1] = ggml_tensor(F32, [K, N, ne2, ne3], x_nb)
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

    def __init__(self, wtype: int, M: int, K: int, N: int, device="cuda"):
        import torch

        self.wtype, self.M, self.K, self.N = wtype, M, K, N
        self.op = mul_mat_op(wtype, M, K, N)
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


def quantize_act(wtype: int, x, stream=None):
    """x [rows, k] f32 -> uint8 [rows, row_bytes(vec_dot_type, k)] in ggml's block layout."""
    import torch

    rows, k = x.shape
    assert x.dtype == torch.float32 and x.stride(1) == 1
    out = torch.empty((rows, row_bytes(VEC_DOT_TYPE[wtype], k)), dtype=torch.uint8, device=x.device)
    check(lib().tlh_quantize_act(wtype, _ptr(x), k, rows, x.stride(0) * 4, _ptr(out), _stream(stream)))
    return out


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

    return {torch.float32: F32, torch.float16: F16}.get(t.dtype, -1)


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
    """key/value f16 [tokens, kv_heads*hs] scattered into the caches; slots i64 [tokens] (negative = skip)."""
    tokens = key.shape[0]
    hs = key.shape[1] // num_kv_heads
    check(lib().tlh_reshape_and_cache(_ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slots), tokens,
                                      num_kv_heads, hs, block_size, _stream(stream)))

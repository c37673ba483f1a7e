"""ctypes loaders for the two CPU checkers (test infrastructure only).

* ``Oracle`` wraps ``oracle/liboracle.so``: our C restatement of ggml's
  quantized MUL_MAT arithmetic and of vLLM-style paged attention.
* ``Ref`` wraps ``oracle/_ref/libggml_ref.so``: the reference's own ggml CPU
  backend compiled in place from /root/reference (crates/ggml-sys/build.rs:357-418
  file list and defines) plus the one-op graph harness ``oracle/ref_graph.c``.
  It is absent where it was not built; tests that need it skip then.

Both are checkers: the product library never loads either.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libggml_ref.so"

# ggml type numbers (vendor/ggml/include/ggml.h:390-405)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 15, 30
Q4_1, Q5_0, Q5_1, Q8_1 = 3, 6, 7, 9
Q2_K, Q3_K = 10, 11
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292),
         Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_1: (32, 36), Q2_K: (256, 84), Q3_K: (256, 110)}
VEC_DOT_TYPE = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K, Q4_1: Q8_1, Q5_0: Q8_0, Q5_1: Q8_1,
                Q2_K: Q8_K, Q3_K: Q8_K}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K", F32: "f32", F16: "f16",
         BF16: "bf16", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q8_1: "q8_1", Q2_K: "q2_K", Q3_K: "q3_K"}


FLOAT_BYTES = {F32: 4, F16: 2, BF16: 2}  # element sizes of the float weight types


def row_bytes(t: int, k: int) -> int:
    if t in FLOAT_BYTES:
        return k * FLOAT_BYTES[t]
    be, bb = BLOCK[t]
    assert k % be == 0, (t, k)
    return k // be * bb


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ne(a: np.ndarray) -> np.ndarray:
    """ggml ne of an array whose shape is ne reversed."""
    return np.array(list(a.shape)[::-1] + [1] * (4 - a.ndim), np.int64)


def _nb(a: np.ndarray) -> np.ndarray:
    """ggml byte strides of such an array."""
    st = list(a.strides)[::-1]
    while len(st) < 4:
        st.append(st[-1] * a.shape[0] if st else a.itemsize)
    return np.array(st, np.int64)


def _i64p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int64))


I32, I64 = 26, 27
NP_OF = {F32: np.float32, F16: np.uint16, BF16: np.uint16, I32: np.int32, I64: np.int64}


class TlqT(C.Structure):
    """tlq_t of oracle/tlq_oracle.h: a ggml tensor view over caller memory."""
    _fields_ = [("data", C.c_void_p), ("ne", C.c_int64 * 4), ("nb", C.c_int64 * 4), ("ty", C.c_int)]


def tlq_t(a: np.ndarray, ty: int, k: int = None) -> TlqT:
    """The view of numpy array `a` (shape = ggml ne reversed, any strides) as
    ggml type `ty`; quantized rows are uint8 (..., rows, row_bytes) with `k`
    elements per row."""
    t = TlqT()
    t.data = a.ctypes.data
    if ty in BLOCK:
        assert a.dtype == np.uint8 and a.shape[-1] == row_bytes(ty, k) and a.strides[-1] == 1
        lead = list(a.shape[:-1])[::-1]
        st = list(a.strides[:-1])[::-1]
        while len(lead) < 3:
            st.append(st[-1] * lead[-1] if st else a.shape[-1])
            lead.append(1)
        ne, nb = [k] + lead[:3], [BLOCK[ty][1]] + st[:3]
    else:
        assert a.dtype == NP_OF[ty], (a.dtype, ty)
        ne, nb = list(_ne(a)), list(_nb(a))
    for i in range(4):
        t.ne[i], t.nb[i] = int(ne[i]), int(nb[i])
    t.ty = ty
    return t


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built: run `make -C oracle oracle` or __graft_entry__.build()")
        L = self.lib = C.CDLL(str(path))
        vp, i64 = C.c_void_p, C.c_int64
        for name in ("tlq_quantize_row_q4_0", "tlq_quantize_row_q4_K", "tlq_quantize_row_q8_0",
                     "tlq_quantize_row_q8_K", "tlq_dequantize_row_q4_0", "tlq_dequantize_row_q8_0",
                     "tlq_dequantize_row_q4_K", "tlq_dequantize_row_q5_K", "tlq_dequantize_row_q6_K",
                     "tlq_dequantize_row_q8_K", "tlq_quantize_row_q8_1", "tlq_dequantize_row_q4_1",
                     "tlq_dequantize_row_q5_0", "tlq_dequantize_row_q5_1", "tlq_dequantize_row_q2_K",
                     "tlq_dequantize_row_q3_K"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        for name in ("tlq_vec_dot_q4_0_q8_0", "tlq_vec_dot_q8_0_q8_0", "tlq_vec_dot_q4_K_q8_K",
                     "tlq_vec_dot_q5_K_q8_K", "tlq_vec_dot_q6_K_q8_K", "tlq_vec_dot_q4_1_q8_1",
                     "tlq_vec_dot_q5_0_q8_0", "tlq_vec_dot_q5_1_q8_1", "tlq_vec_dot_q2_K_q8_K",
                     "tlq_vec_dot_q3_K_q8_K"):
            getattr(L, name).argtypes = [i64, vp, vp]
            getattr(L, name).restype = C.c_float
        L.tlq_fp16_to_fp32_row.argtypes = [vp, vp, i64]
        L.tlq_fp32_to_fp16_row.argtypes = [vp, vp, i64]
        L.tlq_bf16_to_fp32.argtypes = [C.c_uint16]
        L.tlq_bf16_to_fp32.restype = C.c_float
        L.tlq_fp32_to_bf16.argtypes = [C.c_float]
        L.tlq_fp32_to_bf16.restype = C.c_uint16
        for name in ("tlq_vec_dot_f32", "tlq_vec_dot_f16", "tlq_vec_dot_bf16"):
            getattr(L, name).argtypes = [i64, vp, vp]
            getattr(L, name).restype = C.c_float
        L.tlq_block_ints_q4_K.argtypes = [vp, vp, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]
        L.tlq_mul_mat.argtypes = [C.c_int, vp, i64, i64, vp, i64, vp, C.c_int]
        L.tlq_mul_mat.restype = C.c_int
        L.tlq_paged_attention.argtypes = [vp, vp, vp, vp, C.c_int, C.c_float, vp, vp, C.c_int, C.c_int, C.c_int,
                                          C.c_int, C.c_int]
        L.tlq_paged_attention.restype = C.c_int
        L.tlq_reshape_and_cache.argtypes = [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int]
        arr4 = C.POINTER(C.c_int64)
        L.tlq_flash_attn_ext.argtypes = [vp, arr4, arr4, vp, arr4, arr4, vp, arr4, arr4, vp, arr4, arr4, vp, arr4,
                                         C.c_float, C.c_float, C.c_float, C.c_int]
        L.tlq_flash_attn_ext.restype = C.c_int
        tp = C.POINTER(TlqT)
        L.tlq_core_bin.argtypes = [C.c_int, tp, tp, tp]
        L.tlq_core_unary.argtypes = [C.c_int, C.c_float, C.c_float, tp, tp]
        L.tlq_core_norm.argtypes = [C.c_int, C.c_float, tp, tp]
        L.tlq_core_get_rows.argtypes = [tp, tp, tp]
        L.tlq_core_set_rows.argtypes = [tp, tp, tp]
        L.tlq_core_cpy.argtypes = [tp, tp]
        L.tlq_core_rope.argtypes = [C.c_int, C.c_int, C.c_int] + [C.c_float] * 6 + [tp, vp, vp, tp]
        L.tlq_core_soft_max.argtypes = [C.c_float, C.c_float, tp, tp, tp]
        L.tlq_core_argmax.argtypes = [tp, vp]
        L.tlq_core_glu.argtypes = [C.c_int, C.c_int, tp, tp, tp]
        L.tlq_gather_kv.argtypes = [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp]

    # -- fp16
    def f16_to_f32(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.tlq_fp16_to_fp32_row(_p(h), _p(out), h.size)
        return out

    def f32_to_f16(self, f) -> np.ndarray:
        f = _f32(f)
        out = np.empty(f.shape, np.uint16)
        self.lib.tlq_fp32_to_fp16_row(_p(f), _p(out), f.size)
        return out

    # -- bf16 (element by element through the C functions: small arrays only)
    def f32_to_bf16(self, f) -> np.ndarray:
        f = _f32(f)
        return np.array([self.lib.tlq_fp32_to_bf16(float(v)) for v in f.reshape(-1)], np.uint16).reshape(f.shape)

    def bf16_to_f32(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        return np.array([self.lib.tlq_bf16_to_fp32(int(v)) for v in h.reshape(-1)], np.float32).reshape(h.shape)

    # -- quantizers: x [rows, k] f32 -> uint8 [rows, row_bytes]
    def quantize(self, t: int, x) -> np.ndarray:
        x = _f32(np.atleast_2d(x))
        rows, k = x.shape
        out = np.zeros((rows, row_bytes(t, k)), np.uint8)
        fn = {Q4_0: self.lib.tlq_quantize_row_q4_0, Q4_K: self.lib.tlq_quantize_row_q4_K,
              Q8_0: self.lib.tlq_quantize_row_q8_0, Q8_K: self.lib.tlq_quantize_row_q8_K,
              Q8_1: self.lib.tlq_quantize_row_q8_1}[t]
        fn(_p(x), _p(out), rows * k)
        return out

    def quantize_act(self, wtype: int, x) -> np.ndarray:
        return self.quantize(VEC_DOT_TYPE[wtype], x)

    def dequantize(self, t: int, q, k: int) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.uint8)
        rows = q.size // row_bytes(t, k)
        out = np.empty((rows, k), np.float32)
        fn = {Q4_0: self.lib.tlq_dequantize_row_q4_0, Q8_0: self.lib.tlq_dequantize_row_q8_0,
              Q4_K: self.lib.tlq_dequantize_row_q4_K, Q5_K: self.lib.tlq_dequantize_row_q5_K,
              Q6_K: self.lib.tlq_dequantize_row_q6_K,
              Q8_K: self.lib.tlq_dequantize_row_q8_K, Q4_1: self.lib.tlq_dequantize_row_q4_1,
              Q5_0: self.lib.tlq_dequantize_row_q5_0, Q5_1: self.lib.tlq_dequantize_row_q5_1,
              Q2_K: self.lib.tlq_dequantize_row_q2_K, Q3_K: self.lib.tlq_dequantize_row_q3_K}[t]
        fn(_p(q), _p(out), rows * k)
        return out

    def vec_dot(self, wtype: int, k: int, xrow, yrow) -> float:
        xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
        yrow = np.ascontiguousarray(yrow, dtype=np.uint8)
        fn = {Q4_0: self.lib.tlq_vec_dot_q4_0_q8_0, Q8_0: self.lib.tlq_vec_dot_q8_0_q8_0,
              Q4_K: self.lib.tlq_vec_dot_q4_K_q8_K, Q5_K: self.lib.tlq_vec_dot_q5_K_q8_K,
              Q6_K: self.lib.tlq_vec_dot_q6_K_q8_K, Q4_1: self.lib.tlq_vec_dot_q4_1_q8_1,
              Q5_0: self.lib.tlq_vec_dot_q5_0_q8_0, Q5_1: self.lib.tlq_vec_dot_q5_1_q8_1,
              Q2_K: self.lib.tlq_vec_dot_q2_K_q8_K, Q3_K: self.lib.tlq_vec_dot_q3_K_q8_K}[wtype]
        return float(fn(k, _p(xrow), _p(yrow)))

    def block_ints_q4_K(self, xblock, yblock):
        a, b = C.c_int32(), C.c_int32()
        xb = np.ascontiguousarray(xblock, dtype=np.uint8)
        yb = np.ascontiguousarray(yblock, dtype=np.uint8)
        self.lib.tlq_block_ints_q4_K(_p(xb), _p(yb), C.byref(a), C.byref(b))
        return a.value, b.value

    def mul_mat(self, wtype: int, w, M: int, K: int, x, nthreads: int = 8) -> np.ndarray:
        """x [N, K] f32 -> y [N, M] f32 (ggml dst layout ne0 = M). w: block bytes, or
        the f32 / f16 (uint16 bits) / bf16 (uint16 bits) rows of float weights."""
        w = np.ascontiguousarray(w).view(np.uint8)
        x = _f32(np.atleast_2d(x))
        N = x.shape[0]
        y = np.empty((N, M), np.float32)
        rc = self.lib.tlq_mul_mat(wtype, _p(w), M, K, _p(x), N, _p(y), nthreads)
        assert rc == 0, rc
        return y

    def paged_attention(self, q, k_cache, v_cache, num_kv_heads, scale, block_tables, context_lens, block_size):
        q = np.ascontiguousarray(q, dtype=np.uint16)
        seqs, heads, hs = q.shape
        bt = np.ascontiguousarray(block_tables, dtype=np.int32)
        lens = np.ascontiguousarray(context_lens, dtype=np.int32)
        out = np.zeros_like(q)
        rc = self.lib.tlq_paged_attention(_p(out), _p(q), _p(np.ascontiguousarray(k_cache)),
                                          _p(np.ascontiguousarray(v_cache)), num_kv_heads, float(scale), _p(bt),
                                          _p(lens), bt.shape[1], seqs, heads, hs, block_size)
        assert rc == 0, rc
        return out

    def flash_attn_ext(self, q, k, v, mask=None, scale=1.0, max_bias=0.0, softcap=0.0,
                       nthreads: int = 8) -> np.ndarray:
        """GGML_OP_FLASH_ATTN_EXT on numpy arrays whose shapes are ggml's ne reversed
        (any strides): q f32 (nb, nh, nq, D), k/v f16 bits (nb, nhkv, L, D|DV),
        mask f16 bits (mne3, mne2, >= nq, >= L) or None -> f32 (nb, nq, nh, DV).
        nthreads matters only on the backend's split-KV decode path."""
        nb, nh, nq, _ = q.shape
        DV = v.shape[-1]
        out = np.zeros((nb, nq, nh, DV), np.float32)
        zero = np.zeros(4, np.int64)
        args = []
        for a, dt in ((q, np.float32), (k, np.uint16), (v, np.uint16), (mask, np.uint16)):
            if a is None:
                args += [None, _i64p(zero), _i64p(zero)]
                continue
            assert a.dtype == dt, (a.dtype, dt)
            args += [_p(a), _i64p(_ne(a)), _i64p(_nb(a))]
        rc = self.lib.tlq_flash_attn_ext(*args, _p(out), _i64p(_nb(out)), float(scale), float(max_bias),
                                         float(softcap), nthreads)
        assert rc == 0, rc
        return out

    # ----------------------------------------------------------- core ops
    # numpy arrays shaped as ggml's ne reversed: f32 float32, f16 uint16 bits,
    # i32/i64 indices; the destination type is F32 unless given.
    def core_bin(self, code: int, a, ta: int, b, tb: int, td: int = F32) -> np.ndarray:
        d = np.zeros(a.shape, NP_OF[td])
        self.lib.tlq_core_bin(code, C.byref(tlq_t(a, ta)), C.byref(tlq_t(b, tb)), C.byref(tlq_t(d, td)))
        return d

    def core_unary(self, code: int, a, ta: int, p1: float = 0.0, p2: float = 0.0, td: int = F32) -> np.ndarray:
        d = np.zeros(a.shape, NP_OF[td])
        self.lib.tlq_core_unary(code, p1, p2, C.byref(tlq_t(a, ta)), C.byref(tlq_t(d, td)))
        return d

    def core_norm(self, rms: bool, eps: float, a) -> np.ndarray:
        d = np.zeros(a.shape, np.float32)
        self.lib.tlq_core_norm(int(rms), eps, C.byref(tlq_t(a, F32)), C.byref(tlq_t(d, F32)))
        return d

    def core_get_rows(self, a, ta: int, idx, ti: int, k: int = None, td: int = F32) -> np.ndarray:
        ne0 = k if ta in BLOCK else a.shape[-1]
        d = np.zeros(tuple(idx.shape) + (ne0,), NP_OF[td])
        self.lib.tlq_core_get_rows(C.byref(tlq_t(a, ta, k)), C.byref(tlq_t(idx, ti)), C.byref(tlq_t(d, td)))
        return d

    def core_set_rows(self, dst, td: int, src, ts: int, idx, ti: int) -> np.ndarray:
        d = np.array(dst, copy=True)
        self.lib.tlq_core_set_rows(C.byref(tlq_t(src, ts)), C.byref(tlq_t(idx, ti)), C.byref(tlq_t(d, td)))
        return d

    def core_cpy(self, a, ta: int, shape, td: int, k: int = None) -> np.ndarray:
        d = np.zeros(shape, NP_OF[td])
        self.lib.tlq_core_cpy(C.byref(tlq_t(a, ta, k)), C.byref(tlq_t(d, td)))
        return d

    def core_rope(self, a, ta: int, pos, n_dims: int, mode: int, n_ctx_orig: int, freq_base: float,
                  freq_scale: float, ext_factor: float, attn_factor: float, beta_fast: float, beta_slow: float,
                  ff=None) -> np.ndarray:
        d = np.zeros(a.shape, NP_OF[ta])
        pos = np.ascontiguousarray(pos, np.int32)
        ffp = None
        if ff is not None:
            ff = np.ascontiguousarray(ff, np.float32)
            ffp = _p(ff)
        self.lib.tlq_core_rope(mode, n_dims, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor, beta_fast,
                               beta_slow, C.byref(tlq_t(a, ta)), _p(pos), ffp, C.byref(tlq_t(d, ta)))
        return d

    def core_soft_max(self, a, scale: float, max_bias: float, mask=None, tm: int = F16) -> np.ndarray:
        d = np.zeros(a.shape, np.float32)
        m = C.byref(tlq_t(mask, tm)) if mask is not None else None
        self.lib.tlq_core_soft_max(scale, max_bias, C.byref(tlq_t(a, F32)), m, C.byref(tlq_t(d, F32)))
        return d

    def core_glu(self, code: int, swapped: bool, a, b=None) -> np.ndarray:
        shape = a.shape if b is not None else a.shape[:-1] + (a.shape[-1] // 2,)
        d = np.zeros(shape, np.float32)
        bp = C.byref(tlq_t(b, F32)) if b is not None else None
        self.lib.tlq_core_glu(code, int(swapped), C.byref(tlq_t(a, F32)), bp, C.byref(tlq_t(d, F32)))
        return d

    def core_argmax(self, a) -> np.ndarray:
        out = np.zeros(a.shape[0], np.int32)
        self.lib.tlq_core_argmax(C.byref(tlq_t(a, F32)), _p(out))
        return out

    def reshape_and_cache(self, key, value, k_cache, v_cache, slots, num_kv_heads, head_size, block_size):
        key = np.ascontiguousarray(key, dtype=np.uint16)
        value = np.ascontiguousarray(value, dtype=np.uint16)
        slots = np.ascontiguousarray(slots, dtype=np.int64)
        assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
        self.lib.tlq_reshape_and_cache(_p(key), _p(value), _p(k_cache), _p(v_cache), _p(slots), slots.size,
                                       num_kv_heads, head_size, block_size)

    def gather_kv(self, k_cache, v_cache, block_table, L, num_kv_heads, head_size, block_size):
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        k = np.empty((num_kv_heads, L, head_size), np.uint16)
        v = np.empty_like(k)
        self.lib.tlq_gather_kv(_p(np.ascontiguousarray(k_cache)), _p(np.ascontiguousarray(v_cache)), _p(bt), L,
                               num_kv_heads, head_size, block_size, _p(k), _p(v))
        return k, v


class Ref:
    """The reference's compiled ggml CPU code (oracle/_ref)."""

    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (needs /root/reference): run `make -C oracle ref`")
        L = self.lib = C.CDLL(str(path))
        vp, i64 = C.c_void_p, C.c_int64
        for name in ("quantize_row_q8_0", "quantize_row_q8_K", "quantize_row_q8_0_ref", "quantize_row_q8_K_ref",
                     "quantize_row_q4_0_ref", "quantize_row_q4_K_ref", "dequantize_row_q4_0",
                     "dequantize_row_q8_0", "dequantize_row_q4_K", "dequantize_row_q5_K", "dequantize_row_q6_K",
                     "quantize_row_q8_1", "dequantize_row_q4_1", "dequantize_row_q5_0", "dequantize_row_q5_1",
                     "dequantize_row_q2_K", "dequantize_row_q3_K"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        for name in ("ggml_vec_dot_q4_0_q8_0", "ggml_vec_dot_q8_0_q8_0", "ggml_vec_dot_q4_K_q8_K",
                     "ggml_vec_dot_q5_K_q8_K", "ggml_vec_dot_q6_K_q8_K", "ggml_vec_dot_q4_1_q8_1",
                     "ggml_vec_dot_q5_0_q8_0", "ggml_vec_dot_q5_1_q8_1", "ggml_vec_dot_q2_K_q8_K",
                     "ggml_vec_dot_q3_K_q8_K"):
            getattr(L, name).argtypes = [C.c_int, C.POINTER(C.c_float), C.c_size_t, vp, C.c_size_t, vp, C.c_size_t,
                                         C.c_int]
            getattr(L, name).restype = None
        L.ggml_quantize_chunk.argtypes = [C.c_int, vp, vp, i64, i64, i64, vp]
        L.ggml_quantize_chunk.restype = C.c_size_t
        L.ggml_fp16_to_fp32_row.argtypes = [vp, vp, i64]
        L.ggml_fp32_to_fp16_row.argtypes = [vp, vp, i64]
        L.ref_mul_mat.argtypes = [C.c_int, vp, i64, i64, vp, i64, vp, C.c_int, C.c_int, C.POINTER(C.c_double)]
        L.ref_mul_mat.restype = C.c_int
        L.ref_flash_attn.argtypes = [vp, vp, vp, i64, i64, i64, i64, C.c_float, vp, C.c_int, C.c_int,
                                     C.POINTER(C.c_double)]
        L.ref_flash_attn.restype = C.c_int
        L.ref_flash_attn_ext.argtypes = [vp, vp, vp, vp] + [i64] * 11 + [C.c_float] * 3 + [
            vp, C.c_int, C.c_int, C.POINTER(C.c_double)]
        L.ref_flash_attn_ext.restype = C.c_int
        L.ref_core.argtypes = [C.c_int, vp, vp, vp, vp, vp, C.c_int]
        L.ref_ir_run.argtypes = [vp, C.c_int, vp, C.c_int, vp, vp, vp, vp, vp, C.c_int, C.c_int]
        L.ref_gguf_open.argtypes, L.ref_gguf_open.restype = [C.c_char_p], vp
        L.ref_gguf_close.argtypes = [vp]
        L.ref_gguf_info.argtypes = [vp] + [C.POINTER(C.c_int64)] * 2 + [C.POINTER(C.c_size_t)] * 2 + [
            C.POINTER(C.c_uint32)]
        L.ref_gguf_tensor.argtypes = [vp, C.c_int64, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int64),
                                      C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        L.ref_gguf_key.argtypes = [vp, C.c_int64, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_size_t)]
        L.ref_gguf_key.restype = C.c_char_p
        L.ref_gguf_data.argtypes, L.ref_gguf_data.restype = [vp, C.c_int64], vp
        L.ref_gguf_str.argtypes, L.ref_gguf_str.restype = [vp, C.c_int64, C.c_int64], C.c_char_p
        L.ref_gguf_write_sample.argtypes = [C.c_char_p, C.c_uint32]
        L.ggml_cpu_init.argtypes = []
        L.ggml_cpu_init()

    def f16_to_f32(self, h) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.ggml_fp16_to_fp32_row(_p(h), _p(out), h.size)
        return out

    def f32_to_f16(self, f) -> np.ndarray:
        f = _f32(f)
        out = np.empty(f.shape, np.uint16)
        self.lib.ggml_fp32_to_fp16_row(_p(f), _p(out), f.size)
        return out

    def quantize_weights(self, t: int, x) -> np.ndarray:
        """ggml_quantize_chunk(type, ..., imatrix=NULL): the path of DType::from_f32 (dtype.rs:98-124)."""
        x = _f32(np.atleast_2d(x))
        rows, k = x.shape
        out = np.zeros((rows, row_bytes(t, k)), np.uint8)
        self.lib.ggml_quantize_chunk(t, _p(x), _p(out), 0, rows, k, None)
        return out

    def quantize_act(self, wtype: int, x) -> np.ndarray:
        """The x86 from_float entry the CPU mul_mat calls for src1 rows."""
        x = _f32(np.atleast_2d(x))
        rows, k = x.shape
        t = VEC_DOT_TYPE[wtype]
        out = np.zeros((rows, row_bytes(t, k)), np.uint8)
        fn = {Q8_0: self.lib.quantize_row_q8_0, Q8_K: self.lib.quantize_row_q8_K, Q8_1: self.lib.quantize_row_q8_1}[t]
        for r in range(rows):
            fn(_p(x[r]), out[r].ctypes.data_as(C.c_void_p), k)
        return out

    def dequantize(self, t: int, q, k: int) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.uint8)
        rows = q.size // row_bytes(t, k)
        out = np.empty((rows, k), np.float32)
        fn = {Q4_0: self.lib.dequantize_row_q4_0, Q8_0: self.lib.dequantize_row_q8_0,
              Q4_K: self.lib.dequantize_row_q4_K, Q5_K: self.lib.dequantize_row_q5_K,
              Q6_K: self.lib.dequantize_row_q6_K, Q4_1: self.lib.dequantize_row_q4_1,
              Q5_0: self.lib.dequantize_row_q5_0, Q5_1: self.lib.dequantize_row_q5_1,
              Q2_K: self.lib.dequantize_row_q2_K, Q3_K: self.lib.dequantize_row_q3_K}[t]
        fn(_p(q), _p(out), rows * k)
        return out

    def vec_dot(self, wtype: int, k: int, xrow, yrow) -> float:
        xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
        yrow = np.ascontiguousarray(yrow, dtype=np.uint8)
        s = C.c_float()
        fn = {Q4_0: self.lib.ggml_vec_dot_q4_0_q8_0, Q8_0: self.lib.ggml_vec_dot_q8_0_q8_0,
              Q4_K: self.lib.ggml_vec_dot_q4_K_q8_K, Q5_K: self.lib.ggml_vec_dot_q5_K_q8_K,
              Q6_K: self.lib.ggml_vec_dot_q6_K_q8_K, Q4_1: self.lib.ggml_vec_dot_q4_1_q8_1,
              Q5_0: self.lib.ggml_vec_dot_q5_0_q8_0, Q5_1: self.lib.ggml_vec_dot_q5_1_q8_1,
              Q2_K: self.lib.ggml_vec_dot_q2_K_q8_K, Q3_K: self.lib.ggml_vec_dot_q3_K_q8_K}[wtype]
        fn(k, C.byref(s), 0, _p(xrow), 0, _p(yrow), 0, 1)
        return float(s.value)

    def mul_mat(self, wtype: int, w, M: int, K: int, x, nthreads: int = 8, reps: int = 1):
        """One GGML_OP_MUL_MAT on the CPU backend. Returns (y [N, M], seconds for `reps` runs)."""
        w = np.ascontiguousarray(w).view(np.uint8)
        x = _f32(np.atleast_2d(x))
        N = x.shape[0]
        y = np.empty((N, M), np.float32)
        secs = C.c_double()
        rc = self.lib.ref_mul_mat(wtype, _p(w), M, K, _p(x), N, _p(y), nthreads, reps, C.byref(secs))
        assert rc == 0, rc
        return y, secs.value

    def flash_attn(self, q, k, v, scale, nthreads: int = 8, reps: int = 1):
        """q f32 [H, D], k/v f16 bits [Hkv, L, D] -> (out f32 [H, D], seconds)."""
        q = _f32(q)
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        H, D = q.shape
        Hkv, L, _ = k.shape
        out = np.empty((H, D), np.float32)
        secs = C.c_double()
        rc = self.lib.ref_flash_attn(_p(q), _p(k), _p(v), D, L, H, Hkv, float(scale), _p(out), nthreads, reps,
                                     C.byref(secs))
        assert rc == 0, rc
        return out, secs.value

    def flash_attn_ext(self, q, k, v, mask=None, scale=1.0, max_bias=0.0, softcap=0.0, nthreads: int = 8,
                       reps: int = 1):
        """ggml_flash_attn_ext on the CPU backend, contiguous inputs shaped as in
        Oracle.flash_attn_ext. Returns (out f32 (nb, nq, nh, DV), seconds)."""
        q = _f32(q)
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        nb, nh, nq, D = q.shape
        _, nhkv, L, DV = v.shape
        out = np.empty((nb, nq, nh, DV), np.float32)
        if mask is not None:
            mask = np.ascontiguousarray(mask, dtype=np.uint16)
            mne3, mne2, nqm, Lm = mask.shape
        else:
            mne3 = mne2 = nqm = Lm = 0
        secs = C.c_double()
        rc = self.lib.ref_flash_attn_ext(_p(q), _p(k), _p(v), _p(mask) if mask is not None else None, D, DV, nq, nh,
                                         nb, L, nhkv, Lm, nqm, mne2, mne3, float(scale), float(max_bias),
                                         float(softcap), _p(out), nthreads, reps, C.byref(secs))
        assert rc == 0, rc
        return out, secs.value


    def core(self, kind: int, srcs, dst, td: int, ip=(), fp=(), nthreads: int = 4) -> np.ndarray:
        """One core op on the CPU backend (ref_core in oracle/ref_graph.c).
        srcs: up to three (array, ggml type[, k]) or None, contiguous; dst an
        array (its contents are the rows SET_ROWS leaves) of type td."""
        ty = np.zeros(4, np.int32)
        ne = np.zeros(16, np.int64)
        ptrs = (C.c_void_p * 4)()
        keep = []
        for i, src in enumerate(list(srcs) + [None] * (3 - len(srcs))):
            if src is None:
                continue
            a, t = np.ascontiguousarray(src[0]), src[1]
            keep.append(a)
            ty[i] = t
            if t in BLOCK:
                k = src[2]
                lead = list(a.shape[:-1])[::-1] + [1] * (4 - a.ndim)
                ne[4 * i:4 * i + 4] = [k] + lead[:3]
            else:
                ne[4 * i:4 * i + 4] = _ne(a)
            ptrs[i] = a.ctypes.data
        assert dst.flags.c_contiguous
        ty[3] = td
        ne[12:16] = _ne(dst)
        ptrs[3] = dst.ctypes.data
        ipa = np.zeros(16, np.int32)
        ipa[:len(ip)] = ip
        fpa = np.zeros(16, np.float32)
        fpa[:len(fp)] = fp
        rc = self.lib.ref_core(kind, _p(ty), _p(ne), C.cast(ptrs, C.c_void_p), _p(ipa), _p(fpa), nthreads)
        assert rc == 0, rc
        return dst


    def ir_run(self, builder, weights, states, inputs, outs, nthreads: int = 8):
        """Runs a tensorlisp_amd.graph.Builder graph through ggml (ref_ir_run in
        oracle/ref_graph.c): weights / states / inputs are contiguous numpy arrays
        by storage index (states are updated in place); `outs` are (tensor,
        numpy dtype); returns their values. Fails if ggml shapes any tensor
        differently from the builder."""
        recs = builder.records()
        nodes = np.array(builder.nodes, np.int32)
        arrs = [np.ascontiguousarray(a) for a in weights] + list(inputs)
        for a in states:
            assert a.flags.c_contiguous
        ptrs = lambda xs: (C.c_void_p * max(len(xs), 1))(*[x.ctypes.data for x in xs])  # noqa: E731
        inputs = [np.ascontiguousarray(a) for a in inputs]
        res = [np.empty(t.ne[::-1], dt) for t, dt in outs]
        ids = np.array([t.id for t, _ in outs], np.int32)
        rc = self.lib.ref_ir_run(C.cast(recs, C.c_void_p), len(builder.t), _p(nodes), len(nodes),
                                 C.cast(ptrs(arrs[:len(weights)]), C.c_void_p), C.cast(ptrs(states), C.c_void_p),
                                 C.cast(ptrs(inputs), C.c_void_p), _p(ids), C.cast(ptrs(res), C.c_void_p), len(res),
                                 nthreads)
        assert rc == 0, (rc, builder.t[-rc % 1000].op if rc < -999 else "")
        return res


    def gguf_describe(self, path):
        """A GGUF file as ggml's reader sees it: None if it refuses the file, else
        dict(version, alignment, data_offset, tensors [(name, type, ne, offset,
        bytes)], kv {key: (gguf type, value)})."""
        L = self.lib
        h = L.ref_gguf_open(str(path).encode())
        if not h:
            return None
        try:
            nt, nk, al, do, ver = C.c_int64(), C.c_int64(), C.c_size_t(), C.c_size_t(), C.c_uint32()
            L.ref_gguf_info(h, C.byref(nt), C.byref(nk), C.byref(al), C.byref(do), C.byref(ver))
            tensors = []
            for i in range(nt.value):
                name = C.create_string_buffer(64)
                ty, ne, off, nb = C.c_int(), (C.c_int64 * 4)(), C.c_size_t(), C.c_size_t()
                L.ref_gguf_tensor(h, i, name, C.byref(ty), ne, C.byref(off), C.byref(nb))
                tensors.append((name.value.decode(), ty.value, list(ne), off.value, nb.value))
            kv = {}
            sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
            npt = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
                   7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}
            for i in range(nk.value):
                ty, aty, n = C.c_int(), C.c_int(), C.c_size_t()
                key = L.ref_gguf_key(h, i, C.byref(ty), C.byref(aty), C.byref(n)).decode()
                t = ty.value
                if t == 8 or (t == 9 and aty.value == 8):
                    vals = [L.ref_gguf_str(h, i, j).decode("utf-8", "replace") for j in range(n.value)]
                    kv[key] = (t, vals[0] if t == 8 else vals)
                else:
                    et = aty.value if t == 9 else t
                    raw = np.frombuffer(C.string_at(L.ref_gguf_data(h, i), n.value * sizes[et]), npt[et])
                    kv[key] = (t, raw.copy() if t == 9 else raw[0].item())
            return dict(version=ver.value, alignment=al.value, data_offset=do.value, tensors=tensors, kv=kv)
        finally:
            L.ref_gguf_close(h)

    def gguf_write_sample(self, path, alignment: int = 0):
        assert self.lib.ref_gguf_write_sample(str(path).encode(), alignment) == 0


def flash_attn_f64(q, k, v, mask=None, scale=1.0, max_bias=0.0, softcap=0.0) -> np.ndarray:
    """FLASH_ATTN_EXT in float64 on exactly the f16 inputs (q rounded to f16 first,
    as the CPU backend does for f16 keys): the mathematical value every
    implementation approximates. Shapes as in Oracle.flash_attn_ext."""
    nb, nh, nq, D = q.shape
    _, nhkv, L, DV = v.shape
    q16 = np.asarray(q, np.float32).astype(np.float16).astype(np.float64)
    kk = np.asarray(k).view(np.float16).astype(np.float64)
    vv = np.asarray(v).view(np.float16).astype(np.float64)
    sc = np.float32(scale)
    if softcap != 0:
        sc = np.float32(sc / np.float32(softcap))
    nhl2 = 1 << int(np.floor(np.log2(nh)))
    m0 = 2.0 ** (-max_bias / nhl2)
    m1 = 2.0 ** (-(max_bias / 2.0) / nhl2)
    out = np.zeros((nb, nq, nh, DV), np.float64)
    for b in range(nb):
        for h in range(nh):
            hk = h // (nh // nhkv)
            bk = b // (nb // k.shape[0])
            s = (q16[b, h] @ kk[bk, hk].T) * float(sc)  # (nq, L)
            if softcap != 0:
                s = softcap * np.tanh(s)
            if mask is not None:
                slope = 1.0 if max_bias <= 0 else (m0 ** (h + 1) if h < nhl2 else m1 ** (2 * (h - nhl2) + 1))
                mv = np.asarray(mask).view(np.float16)[b % mask.shape[0], h % mask.shape[1], :nq, :L]
                mv = mv.astype(np.float64) * slope
                s = np.where(np.isneginf(mv), -np.inf, s + mv)
            m = s.max(axis=1, keepdims=True)
            live = np.isfinite(m)
            e = np.where(live, np.exp(s - np.where(live, m, 0.0)), 0.0)
            den = e.sum(axis=1, keepdims=True)
            out[b, :, h] = np.where(den > 0, (e @ vv[bk, hk]) / np.where(den > 0, den, 1.0), 0.0)
    return out


# FLASH_ATTN_EXT cases of the reference's own tests (crates/tensorlisp/tests/native.rs:156-345)
# plus ALiBi: (name, nb, nh, nhkv, nq, L, D, DV, mask kind, max_bias, softcap).
# Mask kinds build the f16 padding masks those tests use ([L, nq, 1, nb]: 0 or -inf):
#   "flash"  native.rs:175-181  batch 0 masks keys >= 3L/4, batch 1 keys >= 5
#   "split"  native.rs:202-208  batch 0 keeps keys < v0, batch 1 keys < v1 (v0, v1 in the name)
#   "holes"  native.rs:290-293  keys < 3L/4 with j % 3 != 1
#   "many"   native.rs:336-344  batch 0 masks the first L/4 and [L/2, L/2 + 7), batch 1 keys >= 3
#   "bias"   finite position biases -0.05 * |distance| (what ALiBi slopes scale) and
#            -inf on every fifth key
#   "none"   no mask
FA_CASES = (
    [(f"flash-{nq}-{nk}-{m}", 2, 4, 2, nq, nk, 64, 64, m, 0.0, 0.0)
     for nq, nk in ((5, 6), (40, 70), (40, 64), (3, 100), (1, 1000), (1, 777)) for m in ("flash", "none")]
    + [(f"split-{nk}-{v0}-{v1}", 2, 4, 2, 1, nk, 64, 64, "split", 0.0, 0.0)
       for nk, v0, v1 in ((300, 300, 300), (1000, 750, 5), (512, 129, 128), (777, 1, 777))]
    + [(f"hs-{hs}-{nq}-{nk}", 1, 4, 1, nq, nk, hs, hs, "holes", 0.0, 0.0)
       for hs, nq, nk in ((128, 1, 300), (256, 1, 1000), (256, 1, 100), (256, 5, 60), (256, 40, 70))]
    + [(f"many-{hs}-{nq}-{nk}", 2, 4, 2, nq, nk, hs, hs, "many", 0.0, sc)
       for hs, nq, nk, sc in ((72, 16, 1, 0.0), (72, 17, 17, 0.0), (72, 100, 300, 0.0), (80, 33, 129, 0.0),
                              (64, 130, 70, 30.0), (96, 20, 5000, 0.0), (112, 50, 33, 0.0), (128, 64, 256, 20.0))]
    + [("alibi-6-2", 1, 6, 2, 3, 90, 64, 64, "bias", 8.0, 0.0),
       ("alibi-12-4", 2, 12, 4, 2, 40, 128, 128, "bias", 4.0, 10.0),
       ("dv-192-128", 1, 8, 2, 4, 50, 192, 128, "holes", 0.0, 0.0)]
)


def fa_mask(kind: str, nb: int, nq: int, L: int):
    """f16 bits (nb, 1, nq, L) of a padding mask, or None."""
    if kind == "none":
        return None
    if kind == "bias":
        iq = np.arange(nq)[:, None] + (L - nq)
        j = np.arange(L)[None, :]
        m = np.where(j % 5 == 4, -np.inf, -0.05 * np.abs(j - iq)).astype(np.float32)
        m = m[None, None] + np.float32(0.25) * np.arange(nb, dtype=np.float32)[:, None, None, None]
        return np.ascontiguousarray(m.astype(np.float16)).view(np.uint16)
    valid = np.ones((nb, L), bool)
    if kind == "flash":
        valid[0, L * 3 // 4:] = False
        valid[1, 5:] = False
    elif kind.startswith("split"):
        v0, v1 = (int(t) for t in kind.split(":")[1:])
        valid[:] = False
        valid[0, :v0] = True
        valid[1, :v1] = True
    elif kind == "holes":
        j = np.arange(L)
        valid[:] = (j < L * 3 // 4) & (j % 3 != 1)
    elif kind == "many":
        valid[0, :L // 4] = False
        valid[1, 3:] = False
        valid[0, L // 2:min(L // 2 + 7, L)] = False
    else:
        raise ValueError(kind)
    m = np.where(valid, np.float32(0.0), np.float32(-np.inf)).astype(np.float16)
    return np.ascontiguousarray(np.broadcast_to(m[:, None, None, :], (nb, 1, nq, L))).view(np.uint16)


def fa_case_inputs(case, seed: int):
    """(q, k, v, mask, scale, max_bias, softcap) of one FA_CASES entry: q f32 and K/V
    f16 bits from tensorlisp_amd.synth normal draws seeded by `seed`."""
    import sys

    sys.path.insert(0, str(ROOT))
    from tensorlisp_amd import synth

    name, nb, nh, nhkv, nq, L, D, DV, mkind, max_bias, softcap = case
    if mkind == "split":
        _, nk, v0, v1 = name.split("-")
        mkind = f"split:{v0}:{v1}"
    q = synth.normal(seed, (nb, nh, nq, D))
    k = synth.f16_bits(synth.normal(seed + 1, (nb, nhkv, L, D)))
    v = synth.f16_bits(synth.normal(seed + 2, (nb, nhkv, L, DV)))
    return q, k, v, fa_mask(mkind, nb, nq, L), 1.0 / np.sqrt(D), max_bias, softcap


_oracle = None
_ref = None


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def ref():
    """The compiled reference, or None where it was not built."""
    global _ref
    if _ref is None and REF_SO.exists():
        _ref = Ref()
    return _ref


# x86-64 micro-architecture levels of the fast reference builds (oracle/Makefile
# ref_fast) and the /proc/cpuinfo flags each needs
ISA_LEVELS = (("v4", ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl", "avx2", "fma", "f16c", "bmi2")),
              ("v3", ("avx2", "fma", "f16c", "bmi1", "bmi2", "movbe", "abm")))
_ref_fast = None


def ref_fast():
    """(Ref, level) for the fastest ISA build of the reference this host can
    run (x86-64-v4, else v3), or (None, None): ggml's SIMD paths, a labelled
    speed baseline only -- parity is defined by the no -march build."""
    global _ref_fast
    if _ref_fast is None:
        _ref_fast = (None, None)
        try:
            flags = set()
            for ln in Path("/proc/cpuinfo").read_text().splitlines():
                if ln.startswith("flags"):
                    flags = set(ln.split(":", 1)[1].split())
                    break
        except OSError:
            flags = set()
        for level, need in ISA_LEVELS:
            so = REF_SO.parent / level / REF_SO.name
            if so.exists() and all(f in flags for f in need):
                _ref_fast = (Ref(so), level)
                break
    return _ref_fast


def fp16_probe_values() -> np.ndarray:
    """f32 inputs that pin an f32 -> f16 conversion: every midpoint between adjacent
    finite halves and its two f32 neighbours, a random sample over all exponents,
    and the overflow / underflow edges."""
    import sys

    sys.path.insert(0, str(ROOT))
    from tensorlisp_amd import synth

    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float64)
    hv = np.unique(h[np.isfinite(h)])
    mids = ((hv[1:] + hv[:-1]) / 2).astype(np.float32)
    rnd = synth.normal(7, (1 << 14,)) * np.float32(2.0) ** synth.integers(8, -30, 17, 1 << 14).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504, 65519.996, 65520, -65520, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                      np.inf, -np.inf], np.float32)
    return np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                           rnd, edges]).astype(np.float32)


def xorshift_noise(shape, seed: int) -> np.ndarray:
    """The reference tests' input generator (crates/tensorlisp/tests/native.rs:10-18):
    xorshift64 seeded with seed * 0x9e3779b97f4a7c15 | 1, values in [-1, 1)."""
    n = int(np.prod(shape))
    state = np.uint64((seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF) | np.uint64(1)
    out = np.empty(n, np.float32)
    s = int(state)
    mask = 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        out[i] = np.float32((s >> 40) / float(1 << 23) - 1.0)
    return out.reshape(shape)


# ------------------------------------------------------------------ core ops
CORE_KINDS = {"bin": 1, "unary": 2, "norm": 3, "get_rows": 4, "set_rows": 5, "cpy": 6, "rope": 7, "soft_max": 8,
              "argmax": 9, "glu": 10}
# ggml_unary_op codes (ggml.h:596-619) and the lowering's element-wise extras
UNARY_CODES = [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 18, 19, 20, 21, 100, 101, 102, 103, 104,
               105, 106, 107, 108]
# the CPU's x86-64 build evaluates exp in soft_max and silu with a polynomial
# (vec.h:1278-1316); the oracle and the GPU call expf, a few ulp away
CORE_INEXACT_UNARY = {10}
ROPE_ARGS = ("n_dims", "mode", "n_ctx_orig", "freq_base", "freq_scale", "ext_factor", "attn_factor", "beta_fast",
             "beta_slow")


def _special_row() -> np.ndarray:
    return np.array([0.0, -0.0, 10.0, -10.0, 9.99, -9.99, 20.0, 20.5, -20.0, 1e-3, -1e-3, 80.0, -80.0, 100.0,
                     -100.0, 0.5, -0.5, 1.5, 2.5, -2.5, 3.0, -3.0, 6.0, 1e-30, -1e-30, 60000.0, -60000.0],
                    np.float32)


def core_cases():
    """The core-op cases pinned against the reference's CPU backend: the
    shapes and inputs of the reference's own tests
    (crates/tensorlisp/tests/native.rs:109-154 elementwise/norms, 252-281 rope
    and argmax, 416-435 argmax of long rows, 437-469 set_rows, 471-498 norm
    and rope chains) and decoder-sized ones (rows of 4096, 32 heads of 128,
    a 32000-entry vocabulary). Inputs are regenerated from seeds; the golden
    file keeps the reference's outputs. Each case: name, kind, srcs [(array,
    ggml type[, k])], dst (shape, type), ip / fp (ref_core's arguments), init
    (SET_ROWS' destination before the op), perm (CPY of a permuted view),
    exact (bit-equal to the reference)."""
    from tensorlisp_amd import synth

    f16 = lambda a: synth.f16_bits(np.asarray(a, np.float32))  # noqa: E731
    cases = []

    def add(name, kind, srcs, dst, ip=(), fp=(), init=None, perm=None, exact=True):
        cases.append(dict(name=name, kind=CORE_KINDS[kind], srcs=srcs, dst=dst, ip=tuple(ip), fp=tuple(fp),
                          init=init, perm=perm, exact=exact))

    # native.rs elementwise_norms_and_reductions
    x = xorshift_noise([5, 8], 5) * np.float32(3.0)
    y = xorshift_noise([5, 8], 6)
    add("t_rms", "norm", [(x, F32)], ((5, 8), F32), (1,), (1e-6,))
    add("t_norm", "norm", [(x, F32)], ((5, 8), F32), (0,), (1e-6,))
    for nm, code in (("gelu", 8), ("gelu_erf", 16), ("relu", 6), ("silu", 10), ("sqr", 104), ("exp", 13),
                     ("sin", 106)):
        add(f"t_{nm}", "unary", [(x, F32)], ((5, 8), F32), (code,), exact=code not in CORE_INEXACT_UNARY)
    add("t_cos_y", "unary", [(y, F32)], ((5, 8), F32), (107,))
    add("t_bias", "unary", [(x, F32)], ((5, 8), F32), (100,), (0.5, 3.0))
    add("t_scale_bias_exp", "unary", [(np.exp(y).astype(np.float32), F32)], ((5, 8), F32), (100,), (1.0, 2.0))
    for nm, code in (("add", 0), ("sub", 1), ("mul", 2), ("div", 3)):
        add(f"t_{nm}", "bin", [(x, F32), (y + np.float32(1.5), F32)], ((5, 8), F32), (code,))
    # embedding: an f16 table [4, 10] read at ids [[1,7,3],[0,9,9]], flattened
    table = f16(xorshift_noise([10, 4], 4))
    add("t_embed", "get_rows", [(table, F16), (np.array([1, 7, 3, 0, 9, 9], np.int32), I32)], ((6, 4), F32))
    # rope_pooling_depthwise_argmax: neox base 100 scale 0.5 and the normal rope_ext
    rx = xorshift_noise([3, 2, 8], 4)
    pos = np.array([0, 3, 7], np.int32)
    add("t_rope_neox", "rope", [(rx, F32), (pos, I32)], ((3, 2, 8), F32), (8, 2, 0), (100.0, 0.5, 0.0, 1.0, 0.0, 0.0))
    add("t_rope_norm", "rope", [(rx, F32), (pos, I32)], ((3, 2, 8), F32), (8, 0, 0), (100.0, 1.0, 0.0, 1.0, 0.0, 0.0))
    ax = xorshift_noise([2, 3, 7, 9], 5).reshape(42, 9)
    add("t_argmax_pool", "argmax", [(ax, F32)], ((42,), I32))
    # argmax_of_long_rows (the 262144 case is in the GPU tests only)
    for n in (100, 16384, 20000):
        a = xorshift_noise([3, n], 5)
        for j in (n // 3, n // 2 + 1, n - 1):
            a[0, j] = 5.0
        a[1, n - 1] = 9.0
        add(f"t_argmax_{n}", "argmax", [(a, F32)], ((3,), I32))
    # state_and_set_rows_persist_between_runs: a [2] row into row `at` of [2, 3]
    for step, at in enumerate((0, 2, 1, 2)):
        x1 = xorshift_noise([1, 4], 20 + step)[:, :2].copy()
        for ty, npty in ((F32, np.float32), (F16, np.uint16)):
            init = np.zeros((3, 2), npty)
            add(f"t_set_rows_{TYPE_SUFFIX[ty]}_{step}", "set_rows", [(x1, F32), (np.array([at], np.int32), I32)],
                ((3, 2), ty), init=init)
    # norm_weight_rope_chains_match_unfused
    cx = xorshift_noise([5, 2, 64], 13)
    cpos = np.array([0, 1, 5, 6, 31], np.int32)
    add("t_chain_rms", "norm", [(cx, F32)], ((5, 2, 64), F32), (1,), (1e-6,))
    add("t_chain_mulw", "bin", [(cx, F32), (xorshift_noise([64], 11), F32)], ((5, 2, 64), F32), (2,))
    add("t_chain_rope_neox", "rope", [(cx, F32), (cpos, I32)], ((5, 2, 64), F32), (64, 2, 0),
        (1000.0, 1.0, 0.0, 1.0, 0.0, 0.0))
    add("t_chain_rope_norm", "rope", [(cx, F32), (cpos, I32)], ((5, 2, 64), F32), (64, 0, 0),
        (1000.0, 1.0, 0.0, 1.0, 0.0, 0.0))

    # every unary op over random values and the special ones
    u = np.concatenate([synth.normal(201, (3 * 256,)) * np.float32(4.0), _special_row()]).reshape(1, -1)
    for code in UNARY_CODES:
        src = np.abs(u) + np.float32(0.1) if code in (105, 108) else u
        p = (-1.5, 2.0) if code == 102 else (0.7, -0.3)
        add(f"u_{code}", "unary", [(src, F32)], (src.shape, F32), (code,), p, exact=code not in CORE_INEXACT_UNARY)
    uh = f16(u)
    add("u_f16_gelu", "unary", [(uh, F16)], (u.shape, F16), (8,))

    # decoder-sized (llama-7B shapes: 2 tokens, 4096 wide, 32 heads of 128)
    h = synth.normal(211, (2, 4096))
    add("d_rms", "norm", [(h, F32)], ((2, 4096), F32), (1,), (1e-5,))
    add("d_norm", "norm", [(h + np.float32(0.3), F32)], ((2, 4096), F32), (0,), (1e-5,))
    add("d_mul_w", "bin", [(h, F32), (synth.normal(212, (4096,)), F32)], ((2, 4096), F32), (2,))
    add("d_add", "bin", [(h, F32), (synth.normal(213, (2, 4096)), F32)], ((2, 4096), F32), (0,))
    add("d_silu", "unary", [(h, F32)], ((2, 4096), F32), (10,), exact=False)
    qh = synth.normal(214, (2, 32, 128))
    dpos = np.array([37, 4095], np.int32)
    add("d_rope_neox", "rope", [(qh, F32), (dpos, I32)], ((2, 32, 128), F32), (128, 2, 4096),
        (10000.0, 1.0, 0.0, 1.0, 32.0, 1.0))
    add("d_rope_norm", "rope", [(qh, F32), (dpos, I32)], ((2, 32, 128), F32), (128, 0, 4096),
        (500000.0, 1.0, 0.0, 1.0, 32.0, 1.0))
    ff = (np.float32(1.0) + np.abs(synth.normal(215, (64,)))).astype(np.float32)
    ypos = np.array([5, 30000], np.int32)
    add("d_rope_yarn_ff", "rope", [(qh, F32), (ypos, I32), (ff, F32)], ((2, 32, 128), F32), (96, 2, 4096),
        (10000.0, 0.25, 1.0, 1.0, 32.0, 1.0))
    add("d_rope_f16", "rope", [(f16(qh), F16), (dpos, I32)], ((2, 32, 128), F16), (128, 2, 4096),
        (10000.0, 1.0, 0.0, 1.0, 32.0, 1.0))
    s = synth.normal(216, (1, 32, 2, 300)) * np.float32(3.0)
    m = np.where(synth.uniform(217, 8 * 300).reshape(1, 1, 8, 300) < 0.25, -np.inf, 0.0).astype(np.float32)
    add("d_soft_max_f16mask", "soft_max", [(s, F32), (f16(m), F16)], (s.shape, F32), (), (0.088388, 0.0),
        exact=False)
    mb = (m + synth.normal(218, (1, 1, 8, 300))).astype(np.float32)
    add("d_soft_max_alibi", "soft_max", [(s, F32), (mb, F32)], (s.shape, F32), (), (0.125, 8.0), exact=False)
    add("d_soft_max_plain", "soft_max", [(s, F32)], (s.shape, F32), (), (1.0, 0.0), exact=False)
    for t in (F32, F16, Q4_0, Q8_0, Q4_K, Q6_K):
        K = 512
        if t == F32:
            tab = synth.normal(220, (64, K))
            src = (tab, t)
        elif t == F16:
            src = (f16(synth.normal(220, (64, K))), t)
        else:
            src = (synth.random_blocks(t, 221 + t, 64, K), t, K)
        ids = np.array([3, 63, 0, 17, 17, 42, 8], np.int32)
        add(f"d_get_rows_{TYPE_SUFFIX[t]}", "get_rows", [src, (ids, I32)], ((7, K), F32))
    kv = synth.normal(222, (5, 512))
    slots = np.array([9, 0, 63, 31, 32], np.int64)
    add("d_set_rows_kv_f16", "set_rows", [(kv, F32), (slots, I64)], ((64, 512), F16),
        init=f16(synth.normal(223, (64, 512))))
    add("d_set_rows_kv_f32", "set_rows", [(kv, F32), (slots.astype(np.int32), I32)], ((64, 512), F32),
        init=synth.normal(224, (64, 512)))
    add("d_cpy_f16", "cpy", [(h, F32)], ((2, 4096), F16))
    add("d_cpy_f16_f32", "cpy", [(f16(h), F16)], ((2, 4096), F32))
    add("d_cpy_perm", "cpy", [(qh, F32)], ((32, 2, 128), F32), perm=(0, 2, 1, 3))
    add("d_cpy_reshape", "cpy", [(qh, F32)], ((16, 4, 128), F32))
    add("d_cpy_q8_0", "cpy", [(synth.random_blocks(Q8_0, 225, 6, 512), Q8_0, 512)], ((6, 512), F32))
    gx = synth.normal(227, (2, 2 * 1376)) * np.float32(3.0)
    gx[0, :27] = _special_row()[:27] / np.float32(1000.0) * np.float32(400.0)
    for code, nm in ((0, "reglu"), (1, "geglu"), (2, "swiglu"), (4, "geglu_erf"), (5, "geglu_quick")):
        add(f"d_glu_{nm}", "glu", [(gx, F32)], ((2, 1376), F32), (code, 0), exact=code != 2)
    add("d_glu_swiglu_swapped", "glu", [(gx, F32)], ((2, 1376), F32), (2, 1), exact=False)
    add("d_glu_geglu_split", "glu", [(gx[:, :1376].copy(), F32), (gx[:, 1376:].copy(), F32)], ((2, 1376), F32),
        (1, 0))
    add("d_glu_swiglu_split", "glu", [(gx[:, :1376].copy(), F32), (gx[:, 1376:].copy(), F32)], ((2, 1376), F32),
        (2, 0), exact=False)
    logits = synth.normal(226, (4, 32000))
    logits[1, 7] = logits[1, 31999] = logits[1].max() + np.float32(1.0)
    logits[2, :] = np.float32(0.25)
    add("d_argmax", "argmax", [(logits, F32)], ((4,), I32))
    return cases


TYPE_SUFFIX = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K"}


def core_ref(r, case) -> np.ndarray:
    """The reference's CPU backend on a case (Ref.core)."""
    shape, td = case["dst"]
    dst = np.array(case["init"], copy=True) if case["init"] is not None else np.zeros(shape, NP_OF[td])
    ip = case["ip"]
    if case["kind"] == CORE_KINDS["cpy"] and case["perm"] is not None:
        ip = tuple(case["perm"]) + (1,)
    return r.core(case["kind"], case["srcs"], dst, td, ip=ip, fp=case["fp"])


def core_oracle(o, case) -> np.ndarray:
    """Our C restatement on a case."""
    k, srcs = case["kind"], case["srcs"]
    shape, td = case["dst"]
    ip, fp = case["ip"], case["fp"]
    a = srcs[0]
    if k == CORE_KINDS["bin"]:
        return o.core_bin(ip[0], a[0], a[1], srcs[1][0], srcs[1][1], td)
    if k == CORE_KINDS["unary"]:
        p = tuple(fp) + (0.0, 0.0)
        return o.core_unary(ip[0], a[0], a[1], p[0], p[1], td)
    if k == CORE_KINDS["norm"]:
        return o.core_norm(bool(ip[0]), fp[0], a[0])
    if k == CORE_KINDS["get_rows"]:
        return o.core_get_rows(a[0], a[1], srcs[1][0], srcs[1][1], k=a[2] if len(a) > 2 else None, td=td)
    if k == CORE_KINDS["set_rows"]:
        return o.core_set_rows(case["init"], td, a[0], a[1], srcs[1][0], srcs[1][1])
    if k == CORE_KINDS["cpy"]:
        src = a[0]
        if case["perm"] is not None:
            src = core_perm_view(src, case["perm"])
        return o.core_cpy(src, a[1], shape, td, k=a[2] if len(a) > 2 else None)
    if k == CORE_KINDS["rope"]:
        ff = srcs[2][0] if len(srcs) > 2 else None
        return o.core_rope(a[0], a[1], srcs[1][0], ip[0], ip[1], ip[2], *fp, ff=ff)
    if k == CORE_KINDS["soft_max"]:
        m = srcs[1] if len(srcs) > 1 else None
        return o.core_soft_max(a[0], fp[0], fp[1], m[0] if m else None, m[1] if m else F16)
    if k == CORE_KINDS["argmax"]:
        return o.core_argmax(a[0])
    if k == CORE_KINDS["glu"]:
        return o.core_glu(ip[0], bool(ip[1]), a[0], srcs[1][0] if len(srcs) > 1 else None)
    raise ValueError(k)


def core_perm_view(a: np.ndarray, perm):
    """ggml_permute(a, *perm) as a numpy view (a's shape is ggml's ne reversed):
    ggml axis i of a becomes axis perm[i] of the view."""
    nd = a.ndim
    ax = [0] * 4
    for i in range(4):
        ax[perm[i]] = i
    # numpy axis j <-> ggml axis nd - 1 - j; pad a to 4 dims first
    a4 = a.reshape((1,) * (4 - nd) + a.shape)
    v = a4.transpose([3 - ax[3 - j] for j in range(4)])
    assert all(s == 1 for s in v.shape[:4 - nd]), "the permutation must keep the padding axes"
    return v[(0,) * (4 - nd)]


# ------------------------------------------------------------ decoder steps
def decoder_tiny_config():
    from tensorlisp_amd import graph as G

    return G.DecoderConfig(n_embd=256, n_head=4, n_head_kv=2, n_ff=512, n_layer=2, n_vocab=1000, n_ctx=64)


def decoder_weights(c, seed=100):
    """Host weights for a decoder config: structurally valid random blocks and
    norm weights near one (synth, seeded by weight index)."""
    from tensorlisp_amd import native as N
    from tensorlisp_amd import synth

    out = []
    for i, (_, ty, ne) in enumerate(c.weight_shapes()):
        if ty == N.F32:
            out.append((1.0 + 0.1 * synth.normal(seed + i, (ne[0],))).astype(np.float32))
        else:
            out.append(synth.random_blocks(ty, seed + i, ne[1], ne[0], 0.05))
    return out


# (tokens, first position, attended cache rows, logits of every token?): a
# 5-token prompt, then three single-token steps, then a 3-token chunk
DECODER_STEPS = [([1, 7, 3, 999, 0], 0, 8, False), ([42], 5, 8, False), ([17], 6, 8, False), ([500], 7, 8, False),
                 ([3, 4, 5], 8, 16, True)]


def decoder_lowk_config():
    """The tiny decoder with the matrix types of a Q2_K model file: q2_K token
    embedding and attention / FFN matrices, q3_K value and down projections and
    lm_head (llama.cpp's Q2_K mix keeps those a step higher)."""
    from tensorlisp_amd import graph as G

    types = {f"l{i}.{n}": Q3_K for i in range(2) for n in ("wv", "w_down")}
    return G.DecoderConfig(n_embd=256, n_head=4, n_head_kv=2, n_ff=512, n_layer=2, n_vocab=1000, n_ctx=64,
                           wtype=Q2_K, embd_type=Q2_K, out_type=Q3_K, types=types)


# DECODER_STEPS plus a 20-token chunk (more than 16 columns: the few-column
# kernel's 16-column slabs)
LOWK_STEPS = DECODER_STEPS + [(list(range(100, 120)), 11, 32, False)]


def decoder_step_inputs(step):
    from tensorlisp_amd import graph as G

    toks, p0, n_kv, _ = step
    pos = np.arange(len(toks), dtype=np.int32) + p0
    return [np.array(toks, np.int32), pos, pos.astype(np.int64), G.causal_mask(pos, n_kv)]


def decoder_ref_run(r, c, weights, steps=DECODER_STEPS, f32_values=False):
    """`steps` through the reference CPU backend; returns (logits per step,
    argmax per step, final caches). f32_values: attention reads the cached
    values through an f32 cast (P.V accumulated in f32)."""
    from tensorlisp_amd import graph as G

    states = [np.zeros((c.n_ctx, c.n_embd_kv), np.uint16) for _ in range(2 * c.n_layer)]
    logits, ams = [], []
    for step in steps:
        st = G.decoder_step(c, len(step[0]), step[2], last_only=not step[3], f32_values=f32_values)
        lg, am = r.ir_run(st.builder, weights, states, decoder_step_inputs(step),
                          [(st.logits, np.float32), (st.argmax, np.int32)])
        logits.append(lg.reshape(-1, c.n_vocab))
        ams.append(am.reshape(-1))
    return logits, ams, states


# --------------------------------------------------- 8B-shaped decoder slice
def decoder_8b_slice_config():
    """BASELINE configs[4]'s Llama-style 8B decoder at its own shapes (hidden
    4096, 32 / 8 heads of 128, SwiGLU FFN 14336, vocab 128256, RoPE theta
    500000, every matrix q4_K including the token embedding and lm_head) cut to
    its first two layers, with a 1024-row cache."""
    from tensorlisp_amd import graph as G

    return G.DecoderConfig(n_layer=2, n_ctx=1024, wtype=Q4_K, embd_type=Q4_K, out_type=Q4_K)


def decoder_8b_weights(c, seed=300):
    """Random-init weights for an 8B-shaped config: q4_K blocks that behave like
    quantized zero-mean N(0, 0.02) weights (synth.q4_K_model_blocks), f32 norm
    weights near one."""
    from tensorlisp_amd import native as N
    from tensorlisp_amd import synth

    return [decoder_8b_weight(c, i, seed) for i in range(len(c.weight_shapes()))]


def decoder_8b_weight(c, i, seed=300):
    """Weight i of decoder_8b_weights alone."""
    from tensorlisp_amd import native as N
    from tensorlisp_amd import synth

    _, ty, ne = c.weight_shapes()[i]
    if ty == N.F32:
        return (1.0 + 0.1 * synth.normal(seed + i, (ne[0],))).astype(np.float32)
    return synth.q4_K_model_blocks(seed + i, ne[1], ne[0], 0.02)


# (tokens, first position, attended cache rows, logits of every token?): a
# 6-token prompt, three single-token steps (the last over a 768-row cache view,
# the bench's padded decode view, which splits the attention into partitions),
# then a 3-token chunk with every token's logits
DECODER_8B_STEPS = [([128000, 791, 3938, 315, 279, 1917], 0, 8, False), ([374], 6, 8, False),
                    ([264], 7, 16, False), ([128255], 8, 768, False), ([0, 65535, 100000], 9, 16, True)]


def decoder_8b_ref_run(r, c, weights, steps=DECODER_8B_STEPS, f32_values=False):
    """`steps` of the 8B slice through the reference CPU backend (one dense
    cache); returns (logits per step, argmax per step, final caches). With
    f32_values the attention reads the cached values through an f32 cast, so
    the CPU accumulates P.V in f32 instead of f16 (same model, same values)."""
    from tensorlisp_amd import graph as G

    states = [np.zeros((c.n_ctx, c.n_embd_kv), np.uint16) for _ in range(2 * c.n_layer)]
    logits, ams, taps = [], [], []
    for step in steps:
        st = G.decoder_step(c, len(step[0]), step[2], last_only=not step[3], f32_values=f32_values)
        res = r.ir_run(st.builder, weights, states, decoder_step_inputs(step),
                       [(st.logits, np.float32), (st.argmax, np.int32)] + [(t, np.float32) for t in st.taps])
        logits.append(res[0].reshape(-1, c.n_vocab))
        ams.append(res[1].reshape(-1))
        taps.append([x.reshape(len(step[0]), c.n_embd) for x in res[2:]])
    return logits, ams, states, taps


def decoder_8b_layer_ref(r, c, weights, caches, step, layer, x, f32_values):
    """Layer `layer` alone (graph.decoder_layer_step) on the reference CPU backend
    for decode step `step`, fed the residual stream x [T, n_embd], over dense
    caches holding `caches` (rows past the step's first position are masked or
    overwritten); returns the layer's output [T, n_embd]."""
    from tensorlisp_amd import graph as G

    toks, p0, n_kv, _ = step
    T_ = len(toks)
    states = [np.zeros((c.n_ctx, c.n_embd_kv), np.uint16) for _ in range(2 * c.n_layer)]
    for s, cache in zip(states, caches):
        s[:len(cache)] = cache
    ls = G.decoder_layer_step(c, layer, T_, n_kv, f32_values)
    pos = np.arange(T_, dtype=np.int32) + p0
    (out,) = r.ir_run(ls.builder, weights, states, [np.ascontiguousarray(x, np.float32), pos, pos.astype(np.int64),
                                                    G.causal_mask(pos, n_kv)], [(ls.out, np.float32)])
    return out.reshape(T_, c.n_embd)


# configs[4]'s own run shape on the 8B slice: a 512-token prompt, a 64-token
# chunk, then two single-token steps attending a padded 584-row view (tokens
# uniform over the vocabulary); the paged form of the same prompt decodes two
# other tokens at positions 512 and 513
def prefill_8b_tokens():
    from tensorlisp_amd import synth

    t = synth.integers(340, 0, 128255, 512 + 64 + 4).astype(np.int64)
    return [int(x) for x in t[:512]], [int(x) for x in t[512:576]], [int(x) for x in t[576:]]


def prefill_8b_steps():
    """(tokens, first position, attended cache rows, logits of every token?) of
    the dense run."""
    prompt, chunk, dec = prefill_8b_tokens()
    return [(prompt, 0, 512, False), (chunk, 512, 576, False), ([dec[0]], 576, 584, False),
            ([dec[1]], 577, 584, False)]


def prefill_8b_paged_steps():
    """The paged run's decode steps after the 512-token prompt, as dense steps
    (each attends exactly the rows it has)."""
    prompt, _, dec = prefill_8b_tokens()
    return [([dec[2]], 512, 513, False), ([dec[3]], 513, 514, False)]


# rows of the 512-token prompt's last residual stream kept in the fixture
PREFILL_8B_SAMPLE = np.concatenate([np.arange(0, 512, 16), [511]])


def decoder_8b_run_states(r, c, weights, steps, states, f32_values):
    """`steps` through the reference CPU backend from the dense caches `states`
    (updated in place); per step the logits and the residual stream after the
    embedding and each layer."""
    from tensorlisp_amd import graph as G

    logits, taps = [], []
    for step in steps:
        st = G.decoder_step(c, len(step[0]), step[2], last_only=not step[3], f32_values=f32_values)
        res = r.ir_run(st.builder, weights, states, decoder_step_inputs(step),
                       [(st.logits, np.float32)] + [(t, np.float32) for t in st.taps])
        logits.append(res[0].reshape(-1, c.n_vocab))
        taps.append([x.reshape(len(step[0]), c.n_embd) for x in res[1:]])
    return logits, taps


def embed_rows(c, weights, tokens):
    """The token embedding rows (GET_ROWS of the q4_K table, which the CPU
    backend forms with dequantize_row_q4_K) through the oracle's dequantizer,
    which the quant fixtures pin bit for bit to the reference's."""
    rb = row_bytes(Q4_K, c.n_embd)
    tab = weights[0].reshape(c.n_vocab, rb)
    return oracle().dequantize(Q4_K, np.ascontiguousarray(tab[np.asarray(tokens)]), c.n_embd).reshape(-1, c.n_embd)


# 16 sequences of the 8B slice for a batched paged decode: prompts of 1..16
# tokens, then two decode tokens each
def paged_8b_seqs():
    from tensorlisp_amd import synth

    toks = synth.integers(330, 0, 128255, 16 * 18).astype(np.int64).reshape(16, 18)
    return [([int(t) for t in toks[s, :s + 1]], [int(toks[s, 16]), int(toks[s, 17])]) for s in range(16)]


def paged_8b_ref(r, c, weights, top=8):
    """Each paged_8b_seqs sequence alone through the reference CPU backend with the
    dense-cache step, with its attention's P.V accumulated in f32 and, again, in
    f16 (the backend's default). For the prompt and each decode step ([3, S]):
    the argmax and the `top` largest logits of the f32 run (indices and values,
    [3, S, top]), and the largest |difference| between the two runs' logits
    (how far the backend's own accumulation choice moves them)."""
    from tensorlisp_amd import graph as G

    seqs = paged_8b_seqs()
    am = np.zeros((3, len(seqs)), np.int32)
    ti = np.zeros((3, len(seqs), top), np.int32)
    tv = np.zeros((3, len(seqs), top), np.float32)
    spread = np.zeros((3, len(seqs)), np.float32)
    for s, (prompt, dec) in enumerate(seqs):
        rows = {}
        for f32v in (True, False):
            states = [np.zeros((c.n_ctx, c.n_embd_kv), np.uint16) for _ in range(2 * c.n_layer)]
            todo = [(prompt, 0)] + [([t], len(prompt) + j) for j, t in enumerate(dec)]
            for k, (toks, p0) in enumerate(todo):
                n_kv = p0 + len(toks)
                st = G.decoder_step(c, len(toks), n_kv, f32_values=f32v)
                lg, a = r.ir_run(st.builder, weights, states, decoder_step_inputs((toks, p0, n_kv, False)),
                                 [(st.logits, np.float32), (st.argmax, np.int32)])
                rows[(f32v, k)] = lg.reshape(-1)
                if f32v:
                    am[k, s] = a.reshape(-1)[0]
        for k in range(3):
            lg = rows[(True, k)]
            idx = np.argsort(-lg, kind="stable")[:top]
            ti[k, s], tv[k, s] = idx, lg[idx]
            spread[k, s] = np.abs(lg - rows[(False, k)]).max()
    return am, ti, tv, spread


# ------------------------------------------------------- paged decoder steps
# Three sequences (prompt tokens, then three decode tokens fed one per step),
# block tables into a 16-block pool of 16-row blocks.
PAGED_SEQS = [([1, 7, 3, 999, 0], [42, 17, 500]), ([5, 6, 7, 8, 9, 10, 11, 12, 13], [1, 2, 3]),
              ([250, 251, 252], [9, 99, 999])]
PAGED_TABLES = [[7, 2, 11, 0], [3, 15, 8, 5], [12, 1, 9, 14]]


def paged_ref_run(r, c, weights):
    """Each PAGED_SEQS sequence alone through the reference CPU backend with the
    dense-cache decoder step (decoder_step): the prompt as one step, then one
    step per decode token. Returns (prompt logits [S, vocab], decode logits
    [steps, S, vocab]) and their argmax."""
    from tensorlisp_amd import graph as G

    S, steps = len(PAGED_SEQS), len(PAGED_SEQS[0][1])
    pl = np.zeros((S, c.n_vocab), np.float32)
    dl = np.zeros((steps, S, c.n_vocab), np.float32)
    pa = np.zeros(S, np.int32)
    da = np.zeros((steps, S), np.int32)
    for s, (prompt, dec) in enumerate(PAGED_SEQS):
        states = [np.zeros((c.n_ctx, c.n_embd_kv), np.uint16) for _ in range(2 * c.n_layer)]
        todo = [(prompt, 0)] + [([t], len(prompt) + j) for j, t in enumerate(dec)]
        for k, (toks, p0) in enumerate(todo):
            n_kv = p0 + len(toks)
            st = G.decoder_step(c, len(toks), n_kv)
            lg, am = r.ir_run(st.builder, weights, states, decoder_step_inputs((toks, p0, n_kv, False)),
                              [(st.logits, np.float32), (st.argmax, np.int32)])
            if k == 0:
                pl[s], pa[s] = lg.reshape(-1), am.reshape(-1)[0]
            else:
                dl[k - 1, s], da[k - 1, s] = lg.reshape(-1), am.reshape(-1)[0]
    return pl, pa, dl, da


# ------------------------------------------------------------- MUL_MAT_ID
# (name, weight type, K, M, n_as, n_used, n_b1, n_tokens, seed): decode-sized
# (one token, 2 of 6 experts), a token batch with broadcast src1 (n_b1 = 1),
# K chunks (K > 4096), every weight type, repeated experts within a token.
MMID_CASES = [
    ("q4_K_b2_t3", Q4_K, 512, 96, 8, 2, 2, 3, 1),
    ("q8_0_bcast_t5", Q8_0, 256, 64, 4, 4, 1, 5, 2),
    ("q6_K_decode", Q6_K, 1024, 40, 6, 2, 1, 1, 3),
    ("q4_0_kchunks", Q4_0, 4608, 33, 3, 3, 3, 2, 4),
    ("q5_K_t17_repeats", Q5_K, 256, 17, 5, 2, 2, 17, 5),
]


def mmid_case(case):
    """(builder, output tensor, host weights [as], inputs [b, ids]) of a MUL_MAT_ID case."""
    from tensorlisp_amd import graph as G
    from tensorlisp_amd import synth

    name, t, K, M, n_as, n_used, n_b1, n_tok, seed = case
    b = G.Builder()
    w = b.weight(t, [K, M, n_as], "experts")
    x = b.input(F32, [K, n_b1, n_tok], "b")
    ids = b.input(I32, [n_used, n_tok], "ids")
    y = b.mul_mat_id(w, x, ids)
    b.expand(y)
    wh = synth.random_blocks(t, 900 + seed, n_as * M, K)
    xh = synth.normal(910 + seed, (n_tok, n_b1, K))
    if name.endswith("repeats"):
        idh = (synth.integers(920 + seed, 0, n_as - 1, n_tok * n_used)).astype(np.int32).reshape(n_tok, n_used)
    else:
        rng = np.random.default_rng(930 + seed)
        idh = np.stack([rng.permutation(n_as)[:n_used] for _ in range(n_tok)]).astype(np.int32)
    return b, y, [wh], [xh, idh]


# ------------------------------------------------------------ attn:sdpa graphs
# (head dim, queries, keys, heads, kv heads, K/V type, causal mask): decode and
# prefill shapes, grouped and plain heads, an f16 cache and f32 projections
SDPA_CASES = ((64, 7, 7, 4, 2, F16, True), (128, 1, 33, 8, 2, F16, False), (64, 5, 12, 4, 4, F32, True),
              (128, 20, 40, 8, 8, BF16, True))


def sdpa_graph(hd, lq, lk, heads, kvh, kvt, masked):
    """attn:sdpa's non-flash branch (crates/tensorlisp/src/scheme/stdlib/attn.ss:75-90)
    on split heads (attn.ss:55-60): q [hd, heads, lq] f32 and k, v [hd, kvh, lk] of
    `kvt` permuted to [hd, L, heads]; probs = soft_max_ext(mul_mat(cont k, cont q),
    mask, 1/sqrt(hd)); out = mul_mat(cont(permute(v, 1, 0, 2, 3)), probs), heads
    merged back to [hd * heads, lq]. Returns (builder, output, (q, k, v, mask)).
    Both MUL_MATs have float weights: the f16 / bf16 / f32 keys and values."""
    from tensorlisp_amd import graph as G

    b = G.Builder()
    q = b.input(F32, [hd, heads, lq])
    k = b.input(kvt, [hd, kvh, lk])
    v = b.input(kvt, [hd, kvh, lk])
    m = b.input(F16, [lk, lq]) if masked else None
    qh, kh, vh = (b.permute(t, 0, 2, 1, 3) for t in (q, k, v))
    kq = b.mul_mat(b.cont(kh), b.cont(qh))  # [lk, lq, heads]
    probs = b.soft_max_ext(kq, m, float(np.float32(1.0) / np.sqrt(np.float32(hd))), 0.0)
    out = b.mul_mat(b.cont(b.permute(vh, 1, 0, 2, 3)), probs)  # [hd, lq, heads]
    merged = b.reshape(b.cont(b.permute(out, 0, 2, 1, 3)), hd * heads, lq)
    b.expand(merged)
    return b, merged, (q, k, v, m)


def sdpa_inputs(case, seed: int):
    """numpy inputs of an SDPA_CASES graph (ggml ne reversed; f16 / bf16 as uint16
    bits): q, k, v and, when masked, the causal f16 mask (key j of query i is
    visible while j <= i + lk - lq)."""
    from tensorlisp_amd import synth

    hd, lq, lk, heads, kvh, kvt, masked = case
    q = synth.normal(seed, (lq, heads, hd))
    kv = [synth.normal(seed + i, (lk, kvh, hd)) for i in (1, 2)]
    if kvt == F16:
        kv = [a.astype(np.float16).view(np.uint16) for a in kv]
    elif kvt == BF16:
        kv = [((a.view(np.uint32) + 0x7FFF + ((a.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16) for a in kv]
    ins = [q] + kv
    if masked:
        i, j = np.arange(lq)[:, None], np.arange(lk)[None, :]
        ins.append(np.where(j <= i + lk - lq, 0.0, -np.inf).astype(np.float16).view(np.uint16))
    return ins

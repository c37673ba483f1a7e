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
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 14, 15
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}
VEC_DOT_TYPE = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q6_K: "q6_K", Q8_K: "q8_K"}


def row_bytes(t: int, k: int) -> int:
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


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built: run `make -C oracle oracle` or __graft_entry__.build()")
        L = self.lib = C.CDLL(str(path))
        vp, i64 = C.c_void_p, C.c_int64
        for name in ("tlq_quantize_row_q4_0", "tlq_quantize_row_q4_K", "tlq_quantize_row_q8_0",
                     "tlq_quantize_row_q8_K", "tlq_dequantize_row_q4_0", "tlq_dequantize_row_q8_0",
                     "tlq_dequantize_row_q4_K", "tlq_dequantize_row_q6_K", "tlq_dequantize_row_q8_K"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        for name in ("tlq_vec_dot_q4_0_q8_0", "tlq_vec_dot_q8_0_q8_0", "tlq_vec_dot_q4_K_q8_K",
                     "tlq_vec_dot_q6_K_q8_K"):
            getattr(L, name).argtypes = [i64, vp, vp]
            getattr(L, name).restype = C.c_float
        L.tlq_fp16_to_fp32_row.argtypes = [vp, vp, i64]
        L.tlq_fp32_to_fp16_row.argtypes = [vp, vp, i64]
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

    # -- quantizers: x [rows, k] f32 -> uint8 [rows, row_bytes]
    def quantize(self, t: int, x) -> np.ndarray:
        x = _f32(np.atleast_2d(x))
        rows, k = x.shape
        out = np.zeros((rows, row_bytes(t, k)), np.uint8)
        fn = {Q4_0: self.lib.tlq_quantize_row_q4_0, Q4_K: self.lib.tlq_quantize_row_q4_K,
              Q8_0: self.lib.tlq_quantize_row_q8_0, Q8_K: self.lib.tlq_quantize_row_q8_K}[t]
        fn(_p(x), _p(out), rows * k)
        return out

    def quantize_act(self, wtype: int, x) -> np.ndarray:
        return self.quantize(VEC_DOT_TYPE[wtype], x)

    def dequantize(self, t: int, q, k: int) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.uint8)
        rows = q.size // row_bytes(t, k)
        out = np.empty((rows, k), np.float32)
        fn = {Q4_0: self.lib.tlq_dequantize_row_q4_0, Q8_0: self.lib.tlq_dequantize_row_q8_0,
              Q4_K: self.lib.tlq_dequantize_row_q4_K, Q6_K: self.lib.tlq_dequantize_row_q6_K,
              Q8_K: self.lib.tlq_dequantize_row_q8_K}[t]
        fn(_p(q), _p(out), rows * k)
        return out

    def vec_dot(self, wtype: int, k: int, xrow, yrow) -> float:
        xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
        yrow = np.ascontiguousarray(yrow, dtype=np.uint8)
        fn = {Q4_0: self.lib.tlq_vec_dot_q4_0_q8_0, Q8_0: self.lib.tlq_vec_dot_q8_0_q8_0,
              Q4_K: self.lib.tlq_vec_dot_q4_K_q8_K, Q6_K: self.lib.tlq_vec_dot_q6_K_q8_K}[wtype]
        return float(fn(k, _p(xrow), _p(yrow)))

    def block_ints_q4_K(self, xblock, yblock):
        a, b = C.c_int32(), C.c_int32()
        xb = np.ascontiguousarray(xblock, dtype=np.uint8)
        yb = np.ascontiguousarray(yblock, dtype=np.uint8)
        self.lib.tlq_block_ints_q4_K(_p(xb), _p(yb), C.byref(a), C.byref(b))
        return a.value, b.value

    def mul_mat(self, wtype: int, w, M: int, K: int, x, nthreads: int = 8) -> np.ndarray:
        """x [N, K] f32 -> y [N, M] f32 (ggml dst layout ne0 = M)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
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
                     "dequantize_row_q8_0", "dequantize_row_q4_K", "dequantize_row_q6_K"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        for name in ("ggml_vec_dot_q4_0_q8_0", "ggml_vec_dot_q8_0_q8_0", "ggml_vec_dot_q4_K_q8_K",
                     "ggml_vec_dot_q6_K_q8_K"):
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
        fn = self.lib.quantize_row_q8_0 if t == Q8_0 else self.lib.quantize_row_q8_K
        for r in range(rows):
            fn(_p(x[r]), out[r].ctypes.data_as(C.c_void_p), k)
        return out

    def dequantize(self, t: int, q, k: int) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.uint8)
        rows = q.size // row_bytes(t, k)
        out = np.empty((rows, k), np.float32)
        fn = {Q4_0: self.lib.dequantize_row_q4_0, Q8_0: self.lib.dequantize_row_q8_0,
              Q4_K: self.lib.dequantize_row_q4_K, Q6_K: self.lib.dequantize_row_q6_K}[t]
        fn(_p(q), _p(out), rows * k)
        return out

    def vec_dot(self, wtype: int, k: int, xrow, yrow) -> float:
        xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
        yrow = np.ascontiguousarray(yrow, dtype=np.uint8)
        s = C.c_float()
        fn = {Q4_0: self.lib.ggml_vec_dot_q4_0_q8_0, Q8_0: self.lib.ggml_vec_dot_q8_0_q8_0,
              Q4_K: self.lib.ggml_vec_dot_q4_K_q8_K, Q6_K: self.lib.ggml_vec_dot_q6_K_q8_K}[wtype]
        fn(k, C.byref(s), 0, _p(xrow), 0, _p(yrow), 0, 1)
        return float(s.value)

    def mul_mat(self, wtype: int, w, M: int, K: int, x, nthreads: int = 8, reps: int = 1):
        """One GGML_OP_MUL_MAT on the CPU backend. Returns (y [N, M], seconds for `reps` runs)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
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

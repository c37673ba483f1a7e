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
F32, F16, Q4_0, Q8_0, Q4_K, Q8_K = 0, 1, 2, 8, 12, 15
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q8_K: (256, 292)}
VEC_DOT_TYPE = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_K", Q8_K: "q8_K"}


def row_bytes(t: int, k: int) -> int:
    be, bb = BLOCK[t]
    assert k % be == 0, (t, k)
    return k // be * bb


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built: run `make -C oracle oracle` or __graft_entry__.build()")
        L = self.lib = C.CDLL(str(path))
        vp, i64 = C.c_void_p, C.c_int64
        for name in ("tlq_quantize_row_q4_0", "tlq_quantize_row_q4_K", "tlq_quantize_row_q8_0",
                     "tlq_quantize_row_q8_K", "tlq_dequantize_row_q4_0", "tlq_dequantize_row_q8_0",
                     "tlq_dequantize_row_q4_K", "tlq_dequantize_row_q8_K"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        for name in ("tlq_vec_dot_q4_0_q8_0", "tlq_vec_dot_q8_0_q8_0", "tlq_vec_dot_q4_K_q8_K"):
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
              Q4_K: self.lib.tlq_dequantize_row_q4_K, Q8_K: self.lib.tlq_dequantize_row_q8_K}[t]
        fn(_p(q), _p(out), rows * k)
        return out

    def vec_dot(self, wtype: int, k: int, xrow, yrow) -> float:
        xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
        yrow = np.ascontiguousarray(yrow, dtype=np.uint8)
        fn = {Q4_0: self.lib.tlq_vec_dot_q4_0_q8_0, Q8_0: self.lib.tlq_vec_dot_q8_0_q8_0,
              Q4_K: self.lib.tlq_vec_dot_q4_K_q8_K}[wtype]
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
                     "dequantize_row_q8_0", "dequantize_row_q4_K"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        for name in ("ggml_vec_dot_q4_0_q8_0", "ggml_vec_dot_q8_0_q8_0", "ggml_vec_dot_q4_K_q8_K"):
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
              Q4_K: self.lib.dequantize_row_q4_K}[t]
        fn(_p(q), _p(out), rows * k)
        return out

    def vec_dot(self, wtype: int, k: int, xrow, yrow) -> float:
        xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
        yrow = np.ascontiguousarray(yrow, dtype=np.uint8)
        s = C.c_float()
        fn = {Q4_0: self.lib.ggml_vec_dot_q4_0_q8_0, Q8_0: self.lib.ggml_vec_dot_q8_0_q8_0,
              Q4_K: self.lib.ggml_vec_dot_q4_K_q8_K}[wtype]
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

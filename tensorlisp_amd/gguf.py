"""GGUF models for the executor: reading (tlh_gguf_*), loading onto the GPU, and
a writer for making model files.

``GgufFile`` mirrors the reader the reference uses (crates/tensorlisp/src/gguf.rs:79-320
over ggml's gguf.cpp): metadata with GGUF types, tensor infos, data offsets.
``GgufFile.load`` places every tensor 256-byte aligned in one device buffer and
copies the file's data there, as the reference's Native::load does for its
native executors (crates/tensorlisp/src/native_cuda.rs:44-82).
``decoder_config`` / ``decoder_weights`` map a llama-architecture file (the
llama.* keys and blk.N.* tensor names of llama.cpp's GGUF convention) onto
``graph.DecoderConfig`` and its weight order. ``GgufWriter`` writes version-3
files with the same layout rules (the reference's own writer is
crates/tensorlisp/src/gguf.rs:336-500).
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from . import native as N

# gguf_type (vendor/ggml/include/gguf.h)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32, F32: np.float32,
       BOOL: np.bool_, U64: np.uint64, I64: np.int64, F64: np.float64}


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("ty", C.c_int32), ("n_dims", C.c_int32), ("ne", C.c_int64 * 4),
                ("offset", C.c_uint64), ("bytes", C.c_uint64)]


class GgufFile:
    """An opened GGUF file: metadata and tensor infos (no tensor data read yet)."""

    def __init__(self, path):
        L = N.lib()
        self.path = str(path)
        self._h = C.c_void_p()
        N.check(L.tlh_gguf_open(self.path.encode(), C.byref(self._h)))
        v, nt, nk, al, do = C.c_uint32(), C.c_int64(), C.c_int64(), C.c_uint64(), C.c_uint64()
        N.check(L.tlh_gguf_counts(self._h, C.byref(v), C.byref(nt), C.byref(nk), C.byref(al), C.byref(do)))
        self.version, self.alignment, self.data_offset = v.value, al.value, do.value
        self.tensors = []
        for i in range(nt.value):
            ti = TensorInfo()
            N.check(L.tlh_gguf_tensor(self._h, i, C.byref(ti)))
            self.tensors.append({"name": ti.name.decode(), "type": ti.ty, "n_dims": ti.n_dims,
                                 "ne": list(ti.ne), "offset": ti.offset, "bytes": ti.bytes})
        self.kv = {}
        for i in range(nk.value):
            key, ty, aty, n = C.c_char_p(), C.c_int32(), C.c_int32(), C.c_uint64()
            N.check(L.tlh_gguf_key(self._h, i, C.byref(key), C.byref(ty), C.byref(aty), C.byref(n)))
            self.kv[key.value.decode()] = (ty.value, self._value(i, ty.value, aty.value, n.value))

    def _value(self, i, ty, aty, n):
        L = N.lib()
        if ty == STRING or (ty == ARRAY and aty == STRING):
            out = []
            for j in range(n):
                s, ln = C.c_char_p(), C.c_uint64()
                N.check(L.tlh_gguf_string(self._h, i, j, C.byref(s), C.byref(ln)))
                out.append(C.string_at(s, ln.value).decode("utf-8", "replace"))
            return out[0] if ty == STRING else out
        p, nb = C.c_void_p(), C.c_size_t()
        N.check(L.tlh_gguf_value(self._h, i, C.byref(p), C.byref(nb)))
        raw = np.frombuffer(C.string_at(p, nb.value), dtype=_NP[aty if ty == ARRAY else ty])
        return raw.copy() if ty == ARRAY else raw[0].item()

    def close(self):
        if self._h and self._h.value:
            N.lib().tlh_gguf_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        if N is not None and N._lib is not None:
            self.close()

    def get(self, key, default=None):
        return self.kv[key][1] if key in self.kv else default

    def tensor(self, name):
        for t in self.tensors:
            if t["name"] == name:
                return t
        return None

    def read(self, name) -> np.ndarray:
        """A tensor's bytes from the file (host), as uint8 [rows, row bytes]."""
        t = self.tensor(name)
        with open(self.path, "rb") as f:
            f.seek(self.data_offset + t["offset"])
            b = np.frombuffer(f.read(t["bytes"]), np.uint8)
        rows = t["ne"][1] * t["ne"][2] * t["ne"][3]
        return b.reshape(rows, -1) if rows else b

    def load(self, stream=None):
        """Every tensor onto the current GPU: (one uint8 device buffer, {name: its
        bytes as a uint8 view [rows, row bytes]})."""
        import torch

        L = N.lib()
        n = len(self.tensors)
        offs = (C.c_uint64 * max(n, 1))()
        total = C.c_uint64()
        N.check(L.tlh_gguf_layout(self._h, offs, C.byref(total)))
        buf = torch.empty(max(total.value, 256), dtype=torch.uint8, device="cuda")
        N.check(L.tlh_gguf_upload(self._h, C.c_void_p(buf.data_ptr()), offs, N._stream(stream)))
        views = {}
        for t, o in zip(self.tensors, offs):
            rows = t["ne"][1] * t["ne"][2] * t["ne"][3]
            v = buf[o:o + t["bytes"]]
            views[t["name"]] = v.view(rows, -1) if rows else v
        return buf, views


# ---------------------------------------------------------------- llama models
LLAMA_NAMES = {"attn_norm": "attn_norm", "wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
               "ffn_norm": "ffn_norm", "w_gate": "ffn_gate", "w_up": "ffn_up", "w_down": "ffn_down"}


def gguf_name(ours: str) -> str:
    """graph.DecoderConfig weight name -> llama.cpp GGUF tensor name."""
    if ours == "tok_embd":
        return "token_embd.weight"
    if ours == "out_norm":
        return "output_norm.weight"
    if ours == "output":
        return "output.weight"
    layer, part = ours.split(".", 1)
    return f"blk.{int(layer[1:])}.{LLAMA_NAMES[part]}.weight"


def decoder_config(g: GgufFile, n_ctx: int = None):
    """graph.DecoderConfig from a llama-architecture file's llama.* keys, with
    each weight's type as the file stores it."""
    from .graph import DecoderConfig

    arch = g.get("general.architecture", "llama")
    k = lambda name, d=None: g.get(f"{arch}.{name}", d)  # noqa: E731
    emb = g.tensor("token_embd.weight")
    c = DecoderConfig(n_embd=int(k("embedding_length")), n_head=int(k("attention.head_count")),
                      n_head_kv=int(k("attention.head_count_kv", k("attention.head_count"))),
                      n_ff=int(k("feed_forward_length")), n_layer=int(k("block_count")),
                      n_vocab=int(emb["ne"][1]), n_ctx=int(n_ctx or k("context_length", 4096)),
                      rope_base=float(k("rope.freq_base", 10000.0)),
                      eps=float(k("attention.layer_norm_rms_epsilon", 1e-5)))
    types = {}
    for name, _, _ in c.weight_shapes():
        t = g.tensor(gguf_name(name)) or (g.tensor("token_embd.weight") if name == "output" else None)
        if t is None:
            raise ValueError(f"{g.path}: no tensor {gguf_name(name)}")
        types[name] = t["type"]
    c.types = types
    return c


def decoder_weights(c, views):
    """The device weights in graph.DecoderConfig.weight_shapes order (an absent
    output.weight is the token embedding, as llama.cpp ties them)."""
    out = []
    for name, _, _ in c.weight_shapes():
        v = views.get(gguf_name(name))
        if v is None and name == "output":
            v = views["token_embd.weight"]
        out.append(v)
    return out


# ---------------------------------------------------------------- writer
class GgufWriter:
    """Writes a version-3 GGUF file: typed key-value pairs, then tensor infos,
    then the tensor data, each tensor at the next multiple of the alignment."""

    def __init__(self, alignment: int = 32):
        self.kv = []
        self.tensors = []
        self.alignment = alignment
        if alignment != 32:
            self.add("general.alignment", U32, alignment)

    def add(self, key: str, ty: int, value, arr_type: int = None):
        self.kv.append((key, ty, value, arr_type))

    def add_tensor(self, name: str, ty: int, ne, data: bytes):
        self.tensors.append((name, ty, list(ne), bytes(data)))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def _scalar(self, ty, v) -> bytes:
        return np.array([v], dtype=_NP[ty]).tobytes()

    def write(self, path) -> None:
        out = bytearray(b"GGUF" + struct.pack("<IqQ", 3, len(self.tensors), len(self.kv)))
        for key, ty, v, aty in self.kv:
            out += self._str(key) + struct.pack("<i", ty)
            if ty == STRING:
                out += self._str(v)
            elif ty == ARRAY:
                out += struct.pack("<iQ", aty, len(v))
                out += b"".join(self._str(x) for x in v) if aty == STRING else np.asarray(v, _NP[aty]).tobytes()
            else:
                out += self._scalar(ty, v)
        off = 0
        for name, ty, ne, data in self.tensors:
            out += self._str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}q", *ne)
            out += struct.pack("<iQ", ty, off)
            off += (len(data) + self.alignment - 1) // self.alignment * self.alignment
        out += b"\0" * (-len(out) % self.alignment)
        for name, ty, ne, data in self.tensors:
            out += data + b"\0" * (-len(data) % self.alignment)
        with open(path, "wb") as f:
            f.write(out)


def write_llama(path, c, weights, alignment: int = 32) -> None:
    """A llama-architecture GGUF of decoder config c with host weights in
    c.weight_shapes() order (numpy: f32 arrays, or quantized uint8 rows)."""
    w = GgufWriter(alignment)
    w.add("general.architecture", STRING, "llama")
    for key, ty, val in (("embedding_length", U32, c.n_embd), ("attention.head_count", U32, c.n_head),
                         ("attention.head_count_kv", U32, c.n_head_kv), ("feed_forward_length", U32, c.n_ff),
                         ("block_count", U32, c.n_layer), ("context_length", U32, c.n_ctx),
                         ("rope.freq_base", F32, c.rope_base), ("attention.layer_norm_rms_epsilon", F32, c.eps)):
        w.add(f"llama.{key}", ty, val)
    for (name, ty, ne), data in zip(c.weight_shapes(), weights):
        w.add_tensor(gguf_name(name), ty, ne, np.ascontiguousarray(data).tobytes())
    w.write(path)

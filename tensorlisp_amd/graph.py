"""Graphs for the executor (tlh_program_*): a ggml-style builder and a compiled program.

The reference's Scheme programs build ggml graphs and its native executor
takes them over as IR (crates/kernels/src/graph.rs:72-229, converted by
native_ir.rs lower_graph). There is no ggml in the product path here, so
``Builder`` forms that IR directly, with the shape and stride rules of the
ggml constructors it mirrors (vendor/ggml/src/ggml.c: ggml_new_tensor_impl,
ggml_view_impl, ggml_reshape_*, ggml_permute, ggml_cont, ggml_cpy, ggml_mul_mat,
ggml_add/mul, ggml_rms_norm, ggml_rope_ext, ggml_soft_max_ext,
ggml_flash_attn_ext, ggml_get_rows, ggml_set_rows, ggml_glu, ggml_argmax), so a
graph built here is the graph ggml would build from the same calls. Each
method cites nothing further: the ne/nb rule is the constructor's.

``Program`` compiles an IR with weights bound and replays it
(tlh_program_compile / run), eagerly or as one captured hipGraph.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass, field

from . import native as N

STORE_TEMP, STORE_WEIGHT, STORE_STATE, STORE_INPUT = 0, 1, 2, 3
ELEM = {N.F32: 4, N.F16: 2, N.BF16: 2, N.I32: 4, N.I64: 8}


class TlhIrTensor(C.Structure):
    _fields_ = [("op", C.c_char * 24), ("ty", C.c_int32), ("storage", C.c_int32), ("storage_index", C.c_int32),
                ("view_src", C.c_int32), ("view_offs", C.c_int64), ("ne", C.c_int64 * 4), ("nb", C.c_int64 * 4),
                ("op_params", C.c_int32 * 16), ("src", C.c_int32 * 10)]


def _bits(f: float) -> int:
    return struct.unpack("<i", struct.pack("<f", f))[0]


def row_bytes(ty: int, ne0: int) -> int:
    if ty in N.BLOCK:
        be, bb = N.BLOCK[ty]
        return ne0 // be * bb
    return ne0 * ELEM[ty]


def contiguous_nb(ty: int, ne) -> list:
    nb0 = N.BLOCK[ty][1] if ty in N.BLOCK else ELEM[ty]
    nb = [nb0, row_bytes(ty, ne[0])]
    nb.append(nb[1] * ne[1])
    nb.append(nb[2] * ne[2])
    return nb


@dataclass
class T:
    """One IR tensor (ggml_tensor's fields the executor reads)."""
    id: int
    ty: int
    ne: list
    nb: list
    op: str = "NONE"
    params: list = field(default_factory=lambda: [0] * 16)
    src: list = field(default_factory=list)
    view_src: int = -1
    view_offs: int = 0
    storage: int = STORE_TEMP
    index: int = 0
    name: str = ""

    def nelements(self) -> int:
        return self.ne[0] * self.ne[1] * self.ne[2] * self.ne[3]

    def is_contiguous(self) -> bool:
        return self.nb == contiguous_nb(self.ty, self.ne) or self.nelements() == 0


class Builder:
    """Builds the IR of one graph; `expand` appends a result and what it needs in
    ggml_build_forward_expand's order (sources first, each node once)."""

    def __init__(self):
        self.t: list[T] = []
        self.nodes: list[int] = []
        self._visited: set[int] = set()
        self.n_weights = self.n_states = self.n_inputs = 0

    # -------------------------------------------------------------- leaves
    def _new(self, ty, ne, op="NONE", src=(), params=None, view_of: T = None, offs: int = 0, nb=None, **kw) -> T:
        ne = [int(x) for x in ne] + [1] * (4 - len(ne))
        t = T(len(self.t), ty, ne, list(nb) if nb is not None else contiguous_nb(ty, ne), op,
              (list(params) + [0] * 16)[:16] if params else [0] * 16, [s.id for s in src], **kw)
        if view_of is not None:  # ggml_new_tensor_impl: views alias the root at an accumulated offset
            root = view_of if view_of.view_src < 0 else self.t[view_of.view_src]
            t.view_src = root.id
            t.view_offs = (view_of.view_offs if view_of.view_src >= 0 else 0) + offs
        self.t.append(t)
        return t

    def weight(self, ty, ne, name="") -> T:
        t = self._new(ty, ne, storage=STORE_WEIGHT, index=self.n_weights, name=name)
        self.n_weights += 1
        return t

    def state(self, ty, ne, name="") -> T:
        t = self._new(ty, ne, storage=STORE_STATE, index=self.n_states, name=name)
        self.n_states += 1
        return t

    def input(self, ty, ne, name="") -> T:
        t = self._new(ty, ne, storage=STORE_INPUT, index=self.n_inputs, name=name)
        self.n_inputs += 1
        return t

    # --------------------------------------------------------------- views
    def view(self, a: T, ne, nb=None, offset: int = 0) -> T:
        """ggml_view_1d..4d: nb1..nb3 given (nb0 = the type's size), offset in bytes."""
        ne = list(ne) + [1] * (4 - len(ne))
        full = contiguous_nb(a.ty, ne)
        if nb is not None:
            full = [full[0]] + list(nb) + full[1 + len(nb):]
            for i in range(len(nb) + 1, 4):  # ggml_view_Nd leaves higher strides as ne products
                full[i] = full[i - 1] * ne[i - 1]
        return self._new(a.ty, ne, "VIEW", [a], [offset & 0xFFFFFFFF, offset >> 32], view_of=a, offs=offset, nb=full)

    def reshape(self, a: T, *ne) -> T:
        assert a.is_contiguous(), "ggml_reshape needs a contiguous tensor"
        ne = list(ne) + [1] * (4 - len(ne))
        assert ne[0] * ne[1] * ne[2] * ne[3] == a.nelements()
        return self._new(a.ty, ne, "RESHAPE", [a], view_of=a)

    def permute(self, a: T, a0, a1, a2, a3) -> T:
        ne, nb = [0] * 4, [0] * 4
        for i, ax in enumerate((a0, a1, a2, a3)):
            ne[ax], nb[ax] = a.ne[i], a.nb[i]
        return self._new(a.ty, ne, "PERMUTE", [a], [a0, a1, a2, a3], view_of=a, nb=nb)

    def transpose(self, a: T) -> T:
        t = self.permute(a, 1, 0, 2, 3)
        t.op, t.params = "TRANSPOSE", [0] * 16
        return t

    # ----------------------------------------------------------------- ops
    def _dup(self, a: T, op, src, params=None) -> T:
        return self._new(a.ty, a.ne, op, src, params)

    def mul_mat(self, a: T, b: T) -> T:
        assert a.ne[0] == b.ne[0] and b.ne[2] % a.ne[2] == 0 and b.ne[3] % a.ne[3] == 0
        return self._new(N.F32, [a.ne[1], b.ne[1], b.ne[2], b.ne[3]], "MUL_MAT", [a, b])

    def mul_mat_id(self, a: T, b: T, ids: T) -> T:
        """ggml_mul_mat_id: experts a [K, M, n_as], b [K, n_b1, n_tokens], ids i32
        [n_used, n_tokens] -> f32 [M, n_used, n_tokens] (ggml.c:3329-3353)."""
        assert ids.ty == N.I32 and ids.ne[1] == b.ne[2] and a.ne[0] == b.ne[0] and ids.ne[0] % b.ne[1] == 0
        return self._new(N.F32, [a.ne[1], ids.ne[0], b.ne[2], 1], "MUL_MAT_ID", [a, b, ids])

    def add(self, a, b):
        return self._dup(a, "ADD", [a, b])

    def add_inplace(self, a, b):
        """ggml_add_inplace: the sum is written over a (the result is a view of a)."""
        return self._new(a.ty, a.ne, "ADD", [a, b], view_of=a, nb=a.nb)

    def sub(self, a, b):
        return self._dup(a, "SUB", [a, b])

    def mul(self, a, b):
        return self._dup(a, "MUL", [a, b])

    def div(self, a, b):
        return self._dup(a, "DIV", [a, b])

    def rms_norm(self, a, eps):
        return self._dup(a, "RMS_NORM", [a], [_bits(eps)])

    def norm(self, a, eps):
        return self._dup(a, "NORM", [a], [_bits(eps)])

    def unary(self, a, name: str):
        return self._dup(a, "UNARY", [a], [N.UNARY[name]])

    def silu(self, a):
        return self.unary(a, "silu")

    def scale(self, a, s, b=0.0):
        return self._dup(a, "SCALE", [a], [_bits(s), _bits(b)])

    def cont(self, a):
        return self._new(a.ty, a.ne, "CONT", [a])

    def cpy(self, a: T, b: T) -> T:
        assert a.nelements() == b.nelements()
        return self._new(b.ty, b.ne, "CPY", [a, b], view_of=b, nb=b.nb)

    def get_rows(self, a: T, b: T) -> T:
        assert a.ne[2] == b.ne[1] and a.ne[3] == b.ne[2] and b.ne[3] == 1 and b.ty == N.I32
        return self._new(N.F32, [a.ne[0], b.ne[0], b.ne[1], b.ne[2]], "GET_ROWS", [a, b])

    def set_rows(self, a: T, b: T, c: T) -> T:
        """Rows of b to rows c of a (the result is a view of a)."""
        return self._new(a.ty, a.ne, "SET_ROWS", [b, c], view_of=a, nb=a.nb)

    def rope_ext(self, a: T, pos: T, ff, n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor,
                 beta_fast, beta_slow) -> T:
        p = [0, n_dims, mode, 0, n_ctx_orig] + [_bits(x) for x in (freq_base, freq_scale, ext_factor, attn_factor,
                                                                     beta_fast, beta_slow)]
        return self._dup(a, "ROPE", [a, pos] + ([ff] if ff is not None else []), p)

    def soft_max_ext(self, a: T, mask, scale, max_bias) -> T:
        return self._dup(a, "SOFT_MAX", [a] + ([mask] if mask is not None else []), [_bits(scale), _bits(max_bias)])

    def flash_attn_ext(self, q: T, k: T, v: T, mask, scale, max_bias=0.0, softcap=0.0) -> T:
        return self._new(N.F32, [v.ne[0], q.ne[2], q.ne[1], q.ne[3]], "FLASH_ATTN_EXT",
                         [q, k, v] + ([mask] if mask is not None else []),
                         [_bits(scale), _bits(max_bias), _bits(softcap)])

    def glu_split(self, a: T, b: T, name: str) -> T:
        return self._new(a.ty, a.ne, "GLU", [a, b], [N.GLU[name], 0])

    def argmax(self, a: T) -> T:
        return self._new(N.I32, [a.ne[1]], "ARGMAX", [a])

    def cast(self, a: T, ty: int) -> T:
        """ggml_cast: a copied into a new tensor of type ty."""
        return self.cpy(a, self._new(ty, a.ne))

    # --------------------------------------------------- paged attention nodes
    # ggml CUSTOM nodes that nothing computes on ggml; the executor reads the
    # kernel's parameters from userdata (crates/tensorlisp/src/scheme/core.ss:215-272).
    def _custom(self, ty, ne, userdata: int, src) -> T:
        p = [0] * 16
        lo, hi = userdata & 0xFFFFFFFF, userdata >> 32
        p[4], p[5] = (lo ^ 0x80000000) - 0x80000000, (hi ^ 0x80000000) - 0x80000000
        return self._new(ty, ne, "CUSTOM", src, p)

    def paged_attention(self, q: T, kc: T, vc: T, tables: T, lens: T, block_size: int, max_ctx: int, scale: float,
                        kv_heads: int = 1) -> T:
        """One query per sequence: q f16 [hs, heads, seqs] (contiguous), block tables
        i32 [max_blocks, seqs], context lengths i32 [seqs] -> f16 [hs, heads, seqs]
        (core.ss:247-258)."""
        return self._custom(N.F16, [q.ne[0], q.ne[1], q.ne[2], 1],
                            paged_userdata(1, kv_heads, block_size, max_ctx, scale), [q, kc, vc, tables, lens])

    def paged_cache_write(self, k: T, v: T, kc: T, vc: T, slots: T, block_size: int, kv_heads: int = 1) -> T:
        """key and value f16 [hs * kv_heads, tokens] into the pools at the slots (i32
        [2 * tokens], one little-endian i64 per token; negative skips), core.ss:260-272.
        Expand the result before the attention that reads the pools."""
        return self._custom(N.F16, [1, 1, 1, 1], paged_userdata(2, kv_heads, block_size, 1, 1.0), [k, v, kc, vc, slots])

    # ------------------------------------------------------------- ordering
    def expand(self, t: T) -> None:
        """ggml_build_forward_expand: sources first (in slot order), then t; leaves
        (op NONE) are not nodes."""
        stack = [(t.id, False)]
        while stack:
            i, done = stack.pop()
            if done:
                if i not in self._visited:
                    self._visited.add(i)
                    if self.t[i].op != "NONE":
                        self.nodes.append(i)
                continue
            if i in self._visited:
                continue
            stack.append((i, True))
            for s in reversed(self.t[i].src):
                if s not in self._visited:
                    stack.append((s, False))

    def records(self):
        arr = (TlhIrTensor * len(self.t))()
        for t, r in zip(self.t, arr):
            r.op = t.op.encode()
            r.ty, r.storage, r.storage_index = t.ty, t.storage, t.index
            r.view_src, r.view_offs = t.view_src, t.view_offs
            for i in range(4):
                r.ne[i], r.nb[i] = t.ne[i], t.nb[i]
            for i in range(16):
                r.op_params[i] = t.params[i]
            for i in range(10):
                r.src[i] = t.src[i] if i < len(t.src) else -1
        return arr


def paged_userdata(kind: int, kv_heads: int, block_size: int, max_ctx: int, scale: float) -> int:
    """The u64 a paged CUSTOM node carries (core.ss:240-245): low to high bits kind
    (4), kv heads (4), block size (8), max context (16), scale (f32 bits)."""
    if not 0 < kv_heads < 16:
        raise ValueError(f"kv-heads must be 1..15: {kv_heads}")
    if block_size not in (8, 16, 32):
        raise ValueError(f"block-size must be 8, 16 or 32: {block_size}")
    if not 0 < max_ctx < 65536:
        raise ValueError(f"max-context must be 1..65535: {max_ctx}")
    return kind + kv_heads * 16 + block_size * 256 + max_ctx * 65536 + ((_bits(scale) & 0xFFFFFFFF) << 32)


def _i32_array(xs):
    return (C.c_int32 * max(len(xs), 1))(*xs)


def plan(b: Builder, keep) -> tuple:
    """The executor's memory plan without a device: (arena offset per tensor,
    scratch offset per node position, arena bytes)."""
    L = N.lib()
    recs = b.records()
    offs = (C.c_int64 * len(b.t))()
    scr = (C.c_int64 * max(len(b.nodes), 1))()
    size = C.c_size_t()
    N.check(L.tlh_program_plan(recs, len(b.t), _i32_array(b.nodes), len(b.nodes), _i32_array([k.id for k in keep]),
                               len(keep), offs, scr, C.byref(size)))
    return list(offs), list(scr)[:len(b.nodes)], size.value


class Program:
    """A compiled graph with weights bound (device tensors in weight-index order)
    and state tensors at byte offsets of a state buffer given per run."""

    def __init__(self, b: Builder, keep, weights, state_offsets=()):
        self.builder = b
        self._weights = list(weights)  # keeps the memory alive
        L = N.lib()
        recs = b.records()
        wp = (C.c_void_p * max(len(weights), 1))(*[w.data_ptr() for w in weights])
        so = (C.c_int64 * max(len(state_offsets), 1))(*state_offsets)
        self.ptr = C.c_void_p()
        N.check(L.tlh_program_compile(recs, len(b.t), _i32_array(b.nodes), len(b.nodes),
                                      _i32_array([k.id for k in keep]), len(keep), wp, len(weights), so,
                                      len(state_offsets), C.byref(self.ptr)))

    def __del__(self):
        ptr = getattr(self, "ptr", None)
        if ptr is not None and ptr.value and N is not None and N._lib is not None:
            N._lib.tlh_program_destroy(ptr)
            self.ptr = C.c_void_p()

    def input(self, i: int):
        p, n = C.c_void_p(), C.c_size_t()
        N.check(N.lib().tlh_program_input(self.ptr, i, C.byref(p), C.byref(n)))
        return p.value, n.value

    def tensor_ptr(self, t: T, state=None) -> int:
        p = C.c_void_p()
        N.check(N.lib().tlh_program_tensor(self.ptr, t.id, C.c_void_p(state.data_ptr() if state is not None else None),
                                           C.byref(p)))
        return p.value

    @staticmethod
    def _order(tensor, stream) -> None:
        """Orders `stream` after the current stream (which made `tensor` or last used
        its memory) and tells the caching allocator that `stream` uses `tensor`, so
        the block is not handed out again before `stream`'s copy has run."""
        import torch

        if stream is None or not isinstance(stream, torch.cuda.Stream):
            return
        cur = torch.cuda.current_stream(tensor.device)
        if stream != cur:
            stream.wait_stream(cur)
            tensor.record_stream(stream)

    def write_input(self, i: int, src, stream=None) -> None:
        """Copies a contiguous torch device tensor into graph input i (stream-ordered)."""
        ptr, n = self.input(i)
        assert src.is_contiguous() and src.numel() * src.element_size() == n, (i, n)
        self._order(src, stream)
        N.check(N.lib().tlh_copy(C.c_void_p(ptr), C.c_void_p(src.data_ptr()), n, N._stream(stream)))

    def read(self, t: T, dtype, state=None, stream=None):
        """A copy of tensor t (contiguous bytes) as a torch tensor shaped as ggml's ne reversed."""
        import torch

        out = torch.empty(list(t.ne[::-1]), dtype=dtype, device="cuda")
        n = out.numel() * out.element_size()
        self._order(out, stream)
        N.check(N.lib().tlh_copy(C.c_void_p(out.data_ptr()), C.c_void_p(self.tensor_ptr(t, state)), n,
                                 N._stream(stream)))
        return out

    def run(self, state=None, stream=None, graph: bool = False) -> None:
        st = C.c_void_p(state.data_ptr() if state is not None else None)
        if state is not None:
            self._order(state, stream)
        N.check(N.lib().tlh_program_run(self.ptr, st, N._stream(stream), int(graph)))

    def stats(self):
        a, io, n = C.c_size_t(), C.c_size_t(), C.c_int32()
        N.check(N.lib().tlh_program_stats(self.ptr, C.byref(a), C.byref(io), C.byref(n)))
        return {"arena_bytes": a.value, "io_bytes": io.value, "launches": n.value}

    def trace(self, state=None, stream=None):
        """One eager run that records the kernels each dispatch launched:
        a list of (ggml op of the dispatch's first node, [launch labels])."""
        st = C.c_void_p(state.data_ptr() if state is not None else None)
        if state is not None:
            self._order(state, stream)
        need, cap = C.c_size_t(), 1 << 20
        buf = C.create_string_buffer(cap)
        N.check(N.lib().tlh_program_trace(self.ptr, st, N._stream(stream), buf, cap, C.byref(need)))
        if need.value > cap:  # not run again: a second run would repeat the program's writes
            raise RuntimeError(f"trace text of {need.value} bytes exceeds {cap}")
        out = []
        for line in buf.value.decode().splitlines():
            _, op, labels = line.split("\t")
            out.append((op, labels.split(",") if labels else []))
        return out

    def profile(self, state=None, stream=None):
        """Per-dispatch GPU milliseconds of one eager run (synchronous)."""
        n = self.stats()["launches"]
        ms = (C.c_float * max(n, 1))()
        st = C.c_void_p(state.data_ptr() if state is not None else None)
        if state is not None:
            self._order(state, stream)
        N.check(N.lib().tlh_program_profile(self.ptr, st, N._stream(stream), ms, n))
        return list(ms[:n])



# ----------------------------------------------------------- decoder step
@dataclass
class DecoderConfig:
    """A llama-style decoder's shapes and types (the defaults are Llama-3-8B's
    with Q4_K_M-style weight types)."""
    n_embd: int = 4096
    n_head: int = 32
    n_head_kv: int = 8
    n_ff: int = 14336
    n_layer: int = 32
    n_vocab: int = 128256
    n_ctx: int = 4096
    rope_base: float = 500000.0
    rope_mode: int = 0
    eps: float = 1e-5
    wtype: int = N.Q4_K       # attention and FFN matrices
    embd_type: int = N.Q4_K   # token embedding (read with GET_ROWS)
    out_type: int = N.Q6_K    # lm_head
    types: dict = None        # per-weight types (a GGUF file's), overriding the three above

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    @property
    def n_embd_kv(self) -> int:
        return self.head_dim * self.n_head_kv

    def weight_shapes(self):
        """(name, ggml type, ne) in weight-index order."""
        c = self
        out = [("tok_embd", c.embd_type, [c.n_embd, c.n_vocab])]
        for i in range(c.n_layer):
            out += [(f"l{i}.attn_norm", N.F32, [c.n_embd]), (f"l{i}.wq", c.wtype, [c.n_embd, c.n_embd]),
                    (f"l{i}.wk", c.wtype, [c.n_embd, c.n_embd_kv]), (f"l{i}.wv", c.wtype, [c.n_embd, c.n_embd_kv]),
                    (f"l{i}.wo", c.wtype, [c.n_embd, c.n_embd]), (f"l{i}.ffn_norm", N.F32, [c.n_embd]),
                    (f"l{i}.w_gate", c.wtype, [c.n_embd, c.n_ff]), (f"l{i}.w_up", c.wtype, [c.n_embd, c.n_ff]),
                    (f"l{i}.w_down", c.wtype, [c.n_ff, c.n_embd])]
        out += [("out_norm", N.F32, [c.n_embd]), ("output", c.out_type, [c.n_embd, c.n_vocab])]
        if c.types:
            out = [(name, c.types.get(name, ty), ne) for name, ty, ne in out]
        return out

    def state_bytes(self):
        """Byte offsets of the per-layer K and V caches (f16 [n_embd_kv, n_ctx]) in one state buffer."""
        per = self.n_embd_kv * self.n_ctx * 2
        return [i * per for i in range(2 * self.n_layer)], 2 * self.n_layer * per


@dataclass
class DecoderStep:
    builder: Builder
    tokens: T
    pos: T
    slots: T
    mask: T
    logits: T
    argmax: T
    keep: list
    taps: list = None  # residual stream after the embedding and after each layer


def _layer(b: Builder, c: DecoderConfig, W, x: T, pos: T, T_: int, attend, i: int) -> T:
    """Layer i of llm_build_llama: attention block and SwiGLU FFN, each with its
    RMS_NORM x weight and residual ADD. attend(i, q, k, v) gets the roped q [hd,
    heads, T] and k [hd, kv_heads, T] and v [n_embd_kv, T] (f32) and returns the
    attention output [n_embd, T] (f32)."""
    hd = c.head_dim
    cur = b.mul(b.rms_norm(x, c.eps), W[f"l{i}.attn_norm"])
    q = b.reshape(b.mul_mat(W[f"l{i}.wq"], cur), hd, c.n_head, T_)
    k = b.reshape(b.mul_mat(W[f"l{i}.wk"], cur), hd, c.n_head_kv, T_)
    v = b.mul_mat(W[f"l{i}.wv"], cur)
    q = b.rope_ext(q, pos, None, hd, c.rope_mode, c.n_ctx, c.rope_base, 1.0, 0.0, 1.0, 32.0, 1.0)
    k = b.rope_ext(k, pos, None, hd, c.rope_mode, c.n_ctx, c.rope_base, 1.0, 0.0, 1.0, 32.0, 1.0)
    att = attend(i, q, k, v)
    x = b.add(b.mul_mat(W[f"l{i}.wo"], att), x)
    cur = b.mul(b.rms_norm(x, c.eps), W[f"l{i}.ffn_norm"])
    h = b.glu_split(b.mul_mat(W[f"l{i}.w_gate"], cur), b.mul_mat(W[f"l{i}.w_up"], cur), "swiglu")
    return b.add(b.mul_mat(W[f"l{i}.w_down"], h), x)


def _head(b: Builder, c: DecoderConfig, W, x: T, T_: int, last_only: bool):
    """Final RMS_NORM x weight, lm_head MUL_MAT and ARGMAX (of the last token, or every token)."""
    if last_only and T_ > 1:
        x = b.view(x, [c.n_embd, 1], [x.nb[1]], (T_ - 1) * x.nb[1])
    cur = b.mul(b.rms_norm(x, c.eps), W["out_norm"])
    logits = b.mul_mat(W["output"], cur)
    am = b.argmax(logits)
    b.expand(logits)
    b.expand(am)
    return logits, am


def _decoder_body(b: Builder, c: DecoderConfig, W, tokens: T, pos: T, T_: int, attend, last_only: bool,
                  taps: list = None):
    """Token embedding (GET_ROWS), the layers and the head. `taps` (a list)
    receives the residual stream after the embedding and after each layer."""
    x = b.get_rows(W["tok_embd"], tokens)
    if taps is not None:
        taps.append(x)
    for i in range(c.n_layer):
        x = _layer(b, c, W, x, pos, T_, attend, i)
        if taps is not None:
            taps.append(x)
    return _head(b, c, W, x, T_, last_only)


def _dense_attend(b: Builder, c: DecoderConfig, caches, slots: T, mask: T, T_: int, n_kv: int, f32_values: bool):
    hd = c.head_dim
    scale = 1.0 / float(hd) ** 0.5

    def attend(i, q, k, v):
        kc, vc = caches[i]
        b.expand(b.set_rows(kc, b.reshape(k, c.n_embd_kv, T_), slots))
        b.expand(b.set_rows(vc, v, slots))
        row = c.n_embd_kv * 2
        K = b.permute(b.view(kc, [hd, c.n_head_kv, n_kv], [hd * 2, row], 0), 0, 2, 1, 3)
        V = b.permute(b.view(vc, [hd, c.n_head_kv, n_kv], [hd * 2, row], 0), 0, 2, 1, 3)
        if f32_values:
            V = b.cast(V, N.F32)
        Q = b.permute(q, 0, 2, 1, 3)
        return b.reshape(b.flash_attn_ext(Q, K, V, mask, scale), c.n_embd, T_)

    return attend


def _dense_caches(b: Builder, c: DecoderConfig):
    return [(b.state(N.F16, [c.n_embd_kv, c.n_ctx], f"k{i}"), b.state(N.F16, [c.n_embd_kv, c.n_ctx], f"v{i}"))
            for i in range(c.n_layer)]


@dataclass
class LayerStep:
    """One layer (or the head) as a graph of its own, fed the residual stream."""
    builder: Builder
    x: T        # input 0: residual stream f32 [n_embd, T]
    out: T      # the layer's residual output, or the logits of the head
    argmax: T   # the head's argmax (None for a layer)
    keep: list


def decoder_layer_step(c: DecoderConfig, layer: int, n_tokens: int, n_kv: int, f32_values: bool = False) -> LayerStep:
    """Layer `layer` of decoder_step alone, over the same weights and dense
    caches: inputs 0 x f32 [n_embd, T], 1 positions i32 [T], 2 cache rows i64
    [T], 3 mask f16 [n_kv, T]; output the residual stream after the layer."""
    b = Builder()
    W = {name: b.weight(ty, ne, name) for name, ty, ne in c.weight_shapes()}
    caches = _dense_caches(b, c)
    T_ = n_tokens
    x = b.input(N.F32, [c.n_embd, T_], "x")
    pos = b.input(N.I32, [T_], "pos")
    slots = b.input(N.I64, [T_], "slots")
    mask = b.input(N.F16, [n_kv, T_], "mask")
    out = _layer(b, c, W, x, pos, T_, _dense_attend(b, c, caches, slots, mask, T_, n_kv, f32_values), layer)
    b.expand(out)
    return LayerStep(b, x, out, None, [out])


def decoder_head_step(c: DecoderConfig, n_tokens: int, last_only: bool = True) -> LayerStep:
    """The decoder's head alone: input 0 x f32 [n_embd, T]; logits and argmax."""
    b = Builder()
    W = {name: b.weight(ty, ne, name) for name, ty, ne in c.weight_shapes()}
    x = b.input(N.F32, [c.n_embd, n_tokens], "x")
    logits, am = _head(b, c, W, x, n_tokens, last_only)
    return LayerStep(b, x, logits, am, [logits, am])


def decoder_step(c: DecoderConfig, n_tokens: int, n_kv: int, last_only: bool = True,
                 f32_values: bool = False) -> DecoderStep:
    """One forward step of `n_tokens` new tokens over a cache whose first `n_kv`
    rows are attended (llama.cpp's llm_build_llama with the flash-attention
    path): inputs 0 tokens i32 [T], 1 positions i32 [T], 2 cache rows i64 [T],
    3 mask f16 [n_kv, T]; logits of the last token (or of every token), and
    their argmax. f32_values: the attention reads the cached values through an
    f16 -> f32 cast (the same values; ggml's CPU backend then accumulates P.V in
    f32 rather than f16)."""
    b = Builder()
    W = {name: b.weight(ty, ne, name) for name, ty, ne in c.weight_shapes()}
    caches = _dense_caches(b, c)
    T_ = n_tokens
    tokens = b.input(N.I32, [T_], "tokens")
    pos = b.input(N.I32, [T_], "pos")
    slots = b.input(N.I64, [T_], "slots")
    mask = b.input(N.F16, [n_kv, T_], "mask")
    taps = []
    logits, am = _decoder_body(b, c, W, tokens, pos, T_, _dense_attend(b, c, caches, slots, mask, T_, n_kv, f32_values),
                               last_only, taps)
    return DecoderStep(b, tokens, pos, slots, mask, logits, am, [logits, am], taps)


@dataclass
class PagedConfig:
    """A paged KV pool per layer: `n_blocks` blocks of `block_size` token rows in
    vLLM's layouts (keys [blocks, kv_heads, hs/8, block_size, 8], values
    [blocks, kv_heads, hs, block_size], f16) and `max_blocks` block-table
    entries per sequence (context at most block_size * max_blocks < 65536)."""
    block_size: int = 16
    n_blocks: int = 4096
    max_blocks: int = 256

    @property
    def max_ctx(self) -> int:
        return min(self.block_size * self.max_blocks, 65535)

    def pool_bytes(self, c: DecoderConfig) -> int:
        return self.n_blocks * c.n_head_kv * c.head_dim * self.block_size * 2

    def state_bytes(self, c: DecoderConfig):
        """Byte offsets of the per-layer key and value pools in one state buffer."""
        per = self.pool_bytes(c)
        return [i * per for i in range(2 * c.n_layer)], 2 * c.n_layer * per


@dataclass
class PagedStep:
    builder: Builder
    tokens: T
    pos: T
    slots: T
    mask: T        # prefill only
    tables: T      # decode only
    lens: T        # decode only
    logits: T
    argmax: T
    keep: list


def _paged_pools(b: Builder, c: DecoderConfig, pc: PagedConfig):
    n = pc.n_blocks * c.n_head_kv * c.head_dim * pc.block_size
    return [(b.state(N.F16, [n], f"kpool{i}"), b.state(N.F16, [n], f"vpool{i}")) for i in range(c.n_layer)]


def decoder_prefill_paged(c: DecoderConfig, pc: PagedConfig, n_tokens: int) -> PagedStep:
    """A new sequence's prompt of `n_tokens` tokens: keys and values go to the
    pools through paged-cache-write and the prompt attends to its own keys with
    FLASH_ATTN_EXT and a causal mask. Inputs 0 tokens i32 [T], 1 positions i32
    [T], 2 slots i32 [2T] (one i64 per token), 3 mask f16 [T, T]; logits and
    argmax of the last token."""
    b = Builder()
    W = {name: b.weight(ty, ne, name) for name, ty, ne in c.weight_shapes()}
    pools = _paged_pools(b, c, pc)
    T_, hd = n_tokens, c.head_dim
    tokens = b.input(N.I32, [T_], "tokens")
    pos = b.input(N.I32, [T_], "pos")
    slots = b.input(N.I32, [2 * T_], "slots")
    mask = b.input(N.F16, [T_, T_], "mask")
    scale = 1.0 / float(hd) ** 0.5

    def attend(i, q, k, v):
        kc, vc = pools[i]
        k16 = b.cast(b.reshape(k, c.n_embd_kv, T_), N.F16)
        v16 = b.cast(v, N.F16)
        b.expand(b.paged_cache_write(k16, v16, kc, vc, slots, pc.block_size, c.n_head_kv))
        K = b.permute(b.reshape(k16, hd, c.n_head_kv, T_), 0, 2, 1, 3)
        V = b.permute(b.reshape(v16, hd, c.n_head_kv, T_), 0, 2, 1, 3)
        Q = b.permute(q, 0, 2, 1, 3)
        return b.reshape(b.flash_attn_ext(Q, K, V, mask, scale), c.n_embd, T_)

    logits, am = _decoder_body(b, c, W, tokens, pos, T_, attend, True)
    return PagedStep(b, tokens, pos, slots, mask, None, None, logits, am, [logits, am])


def decoder_decode_paged(c: DecoderConfig, pc: PagedConfig, n_seqs: int) -> PagedStep:
    """One decode step of `n_seqs` sequences, one token each, over the paged
    pools (the `paged-attention` node, vLLM's decode kernel). Inputs 0 tokens
    i32 [S], 1 positions i32 [S], 2 slots i32 [2S], 3 block tables i32
    [max_blocks, S], 4 context lengths i32 [S] (including the new token);
    logits [vocab, S] and their argmax [S]."""
    b = Builder()
    W = {name: b.weight(ty, ne, name) for name, ty, ne in c.weight_shapes()}
    pools = _paged_pools(b, c, pc)
    S = n_seqs
    tokens = b.input(N.I32, [S], "tokens")
    pos = b.input(N.I32, [S], "pos")
    slots = b.input(N.I32, [2 * S], "slots")
    tables = b.input(N.I32, [pc.max_blocks, S], "tables")
    lens = b.input(N.I32, [S], "lens")
    attend = _paged_attend(b, c, pc, pools, slots, tables, lens, S)
    logits, am = _decoder_body(b, c, W, tokens, pos, S, attend, False)
    return PagedStep(b, tokens, pos, slots, None, tables, lens, logits, am, [logits, am])


def _paged_attend(b: Builder, c: DecoderConfig, pc: PagedConfig, pools, slots: T, tables: T, lens: T, S: int):
    scale = 1.0 / float(c.head_dim) ** 0.5

    def attend(i, q, k, v):
        kc, vc = pools[i]
        q16 = b.cast(q, N.F16)
        b.expand(q16)  # ahead of the cache write, next to K's rope (one launch for both)
        k16 = b.cast(b.reshape(k, c.n_embd_kv, S), N.F16)
        v16 = b.cast(v, N.F16)
        b.expand(b.paged_cache_write(k16, v16, kc, vc, slots, pc.block_size, c.n_head_kv))
        att = b.paged_attention(q16, kc, vc, tables, lens, pc.block_size, pc.max_ctx, scale, c.n_head_kv)
        return b.cast(b.reshape(att, c.n_embd, S), N.F32)

    return attend


def decoder_layer_decode_paged(c: DecoderConfig, pc: PagedConfig, layer: int, n_seqs: int) -> LayerStep:
    """Layer `layer` of decoder_decode_paged alone: inputs 0 x f32 [n_embd, S],
    1 positions i32 [S], 2 slots i32 [2S], 3 block tables i32 [max_blocks, S],
    4 context lengths i32 [S]; output the residual stream after the layer."""
    b = Builder()
    W = {name: b.weight(ty, ne, name) for name, ty, ne in c.weight_shapes()}
    pools = _paged_pools(b, c, pc)
    S = n_seqs
    x = b.input(N.F32, [c.n_embd, S], "x")
    pos = b.input(N.I32, [S], "pos")
    slots = b.input(N.I32, [2 * S], "slots")
    tables = b.input(N.I32, [pc.max_blocks, S], "tables")
    lens = b.input(N.I32, [S], "lens")
    out = _layer(b, c, W, x, pos, S, _paged_attend(b, c, pc, pools, slots, tables, lens, S), layer)
    b.expand(out)
    return LayerStep(b, x, out, None, [out])


def paged_slots(table, positions, block_size: int):
    """i32 [2T] slot words (one little-endian i64 per token) for token positions of
    one sequence whose block table is `table` (numpy)."""
    import numpy as np

    pos = np.asarray(positions, np.int64)
    tab = np.asarray(table, np.int64)
    return (tab[pos // block_size] * block_size + pos % block_size).astype(np.int64).view(np.int32)


def causal_mask(positions, n_kv: int):
    """f16 bits [T, n_kv] (numpy): 0 where cache row j <= the token's position, -inf elsewhere."""
    import numpy as np

    pos = np.asarray(positions).reshape(-1, 1)
    m = np.where(np.arange(n_kv).reshape(1, -1) <= pos, 0.0, -np.inf).astype(np.float16)
    return m.view(np.uint16)

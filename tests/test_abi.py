"""The C ABI (include/tlhip.h) without touching a GPU: the library loads, exports
every declared symbol, and validates descriptors the way Ctx::mul_mat
(crates/kernels/src/cuda/lower.rs:543-571) and PagedGeometry::prepare
(crates/kernels/src/cuda/paged_attn.rs:223-250) refuse them: unsupported types
and shapes are named errors, not crashes (the reference's
native.rs:241-250 "unsupported op reported by name")."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from tensorlisp_amd import native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "tlhip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tlh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    decl = declared_functions()
    assert decl, "no declarations parsed"
    missing = [f for f in decl if not hasattr(lib, f)]
    assert not missing, missing
    assert sorted(N.EXPORTS) == decl


def test_integration_binding_lists_every_declaration():
    """The reference-side FFI block a maintainer would add (INTEGRATION.md's
    `extern "C"` block) names every function the header declares, once."""
    text = (HEADER.parents[1] / "INTEGRATION.md").read_text()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    bound = re.findall(r"pub fn (tlh_[a-z0-9_]+)\(", block)
    assert len(bound) == len(set(bound)), sorted(f for f in bound if bound.count(f) > 1)
    assert sorted(bound) == declared_functions()


def test_descriptor_layout():
    assert C.sizeof(N.TlhTensor) == 72
    assert C.sizeof(N.TlhOp) == 5 * 72 + 12 * 8  # OP_BYTES of lower.rs:67
    assert N.TlhOp.x.offset == 360


def test_version_and_device_count_without_gpu():
    assert N.lib().tlh_version().decode().startswith("tlhip")
    assert N.device_count() >= 0


def _status(fn, *args):
    st = fn(*args)
    return N.STATUS[st], N.lib().tlh_last_error().decode()


def scratch_status(op):
    n = C.c_size_t()
    st, msg = _status(N.lib().tlh_mul_mat_scratch_bytes, C.byref(op), C.byref(n))
    return st, msg, n.value


@pytest.mark.parametrize("wt", [N.Q4_0, N.Q8_0, N.Q4_K])
@pytest.mark.parametrize("n", [1, 8, 9, 512])
def test_mul_mat_scratch_sizes(wt, n):
    K, M = 4096, 1024
    st, msg, nbytes = scratch_status(N.mul_mat_op(wt, M, K, n))
    assert st == "OK", msg
    # codes + f32 scales + per-block sums, each region 256-byte aligned
    at = N.VEC_DOT_TYPE[wt]
    be = N.BLOCK[at][0]
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    sums = n * (K // 16) * 2 if at == N.Q8_K else n * (K // 32) * 4
    # q4_K GEMM launches also stage the codes and the bsums as f16
    f16_codes = al(n * K * 2) + n * (K // 16) * 2 if wt == N.Q4_K and n > 16 else 0
    # a GEMM of fewer 128 x 128 tiles than CUs (256) splits K into up to 512 / tiles
    # chunks of at least 4 x 256 elements (at most 16) with f32 partials [chunk][N][M]
    tiles = -(-n // 128) * -(-M // 128)
    ks = 1 if n <= 16 or tiles >= 256 else max(1, min(-(-512 // tiles), K // 256 // 4, 16))
    parts = al(ks * n * M * 4) if ks > 1 else 0
    assert nbytes == al(al(al(al(n * K) + n * (K // be) * 4) + sums) + f16_codes) + parts


@pytest.mark.parametrize("wt", [N.Q4_0, N.Q8_0, N.Q4_K])
@pytest.mark.parametrize("n,K,parts", [(1, 14336, 0), (8, 4096, 0), (8, 14336, 4), (16, 8192, 2), (1, 16640, 5)])
def test_mul_mat_scratch_has_mfma_partials_for_long_K(wt, n, K, parts):
    """The few-column MFMA kernel (N <= 16 outside the register GEMV) with K above 4096
    keeps per-chunk partial sums [chunks][batches][N][M] after the activations. q4_0 at
    N <= 2 reserves them as well: with weights that are not 4-byte aligned (which only
    the pointers tell) it takes the MFMA kernel instead of the register GEMV."""
    M = 1000
    if K % 256:
        pytest.skip("K multiple of 256 here")
    if wt == N.Q4_0 and n <= 2:
        parts = -(-(K // 256) // 16) if K > 4096 else 0  # 16 units of 256 a chunk
    st, msg, nbytes = scratch_status(N.mul_mat_op(wt, M, K, n))
    assert st == "OK", msg
    at = N.VEC_DOT_TYPE[wt]
    be = N.BLOCK[at][0]
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    sums = n * (K // 16) * 2 if at == N.Q8_K else n * (K // 32) * 4
    act = al(al(al(al(n * K) + n * (K // be) * 4) + sums))
    assert nbytes == act + al(parts * n * M * 4)


def test_mul_mat_unsupported_weight_type_is_named():
    """A weight type the reference's lowering refuses too (quant_ok,
    crates/kernels/src/cuda/lower.rs:117-119, admits 2, 3, 6, 7, 8, 10..14 and
    the float types): iq2_xxs (16)."""
    op = N.mul_mat_op(N.Q4_0, 64, 256, 1)
    op.t[0].ty = 16
    st, msg, _ = scratch_status(op)
    assert st == "UNSUPPORTED" and "type 16" in msg


def test_mul_mat_admits_the_reference_lowering_types():
    """Every quantized type quant_ok admits (lower.rs:117-119) sizes its scratch."""
    for t in (N.Q4_0, N.Q4_1, N.Q5_0, N.Q5_1, N.Q8_0, N.Q2_K, N.Q3_K, N.Q4_K, N.Q5_K, N.Q6_K):
        st, msg, _ = scratch_status(N.mul_mat_op(t, 64, 512, 3))
        assert st == "OK", (t, msg)


def test_mul_mat_rejects_bad_shapes_and_layouts():
    op = N.mul_mat_op(N.Q4_K, 64, 512, 2)
    op.t[1].ne[0] = 256  # K mismatch
    assert scratch_status(op)[0] == "UNSUPPORTED"
    op = N.mul_mat_op(N.Q4_K, 64, 320, 2)  # K not a multiple of 256
    st, msg, _ = scratch_status(op)
    assert st == "UNSUPPORTED" and "multiple" in msg
    op = N.mul_mat_op(N.Q8_0, 64, 256, 2)
    op.t[1].ty = N.F16
    assert scratch_status(op)[0] == "UNSUPPORTED"
    op = N.mul_mat_op(N.Q8_0, 64, 256, 2)
    op.t[0].nb[0] = 17  # permuted src0
    assert scratch_status(op)[0] == "UNSUPPORTED"
    op = N.mul_mat_op(N.Q8_0, 64, 256, 4, ne2=3, w_ne2=2)  # 3 % 2 != 0
    assert scratch_status(op)[0] == "UNSUPPORTED"
    op = N.mul_mat_op(N.Q8_0, 64, 256, 4, ne2=4, w_ne2=2)
    op.x[0] = 3  # disagrees with ne12 / ne02 = 2
    assert scratch_status(op)[0] == "INVALID"


def test_mul_mat_null_pointers_are_invalid_not_crashes():
    op = N.mul_mat_op(N.Q8_0, 64, 256, 1)
    st, msg = _status(N.lib().tlh_mul_mat, C.byref(op), None, None, None, None, 0, None)
    assert st == "INVALID", msg


def test_quantize_and_dequantize_validation():
    L = N.lib()
    st, msg = _status(L.tlh_quantize_act, 16, None, 256, 1, 1024, None, None)  # iq2_xxs
    assert st == "UNSUPPORTED"
    st, msg = _status(L.tlh_dequantize, 16, None, 256, 1, 66, None, None)
    assert st == "UNSUPPORTED"
    st, msg = _status(L.tlh_quantize_act, N.Q4_K, None, 300, 1, 1200, None, None)
    assert st == "INVALID" and "multiple" in msg
    st, msg = _status(L.tlh_dequantize, N.Q4_0, None, 33, 1, 18, None, None)
    assert st == "INVALID"


def paged_args(**kw):
    a = N.TlhPagedArgs()
    a.num_seqs, a.num_heads, a.num_kv_heads, a.head_size = 32, 32, 8, 128
    a.block_size, a.max_blocks_per_seq, a.max_context_len, a.scale = 16, 512, 8192, 128 ** -0.5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,status", [
    ({}, "OK"),
    ({"head_size": 100}, "INVALID"),
    ({"block_size": 64}, "INVALID"),
    ({"num_kv_heads": 3}, "INVALID"),
    ({"max_blocks_per_seq": 10}, "INVALID"),
])
def test_paged_attention_geometry_validation(kw, status):
    n = C.c_size_t()
    st, msg = _status(N.lib().tlh_paged_attention_scratch_bytes, C.byref(paged_args(**kw)), C.byref(n))
    assert st == status, msg
    if status == "OK":  # partials [seqs][heads][ceil(max_ctx / 256)][head_size + 2] f32, plus the
        # bounded room of 64-token partitions (510 x group size rows)
        assert n.value == 32 * 32 * (8192 // 256) * (128 + 2) * 4 + min(32 * 32 * (8192 // 64), 510 * 4) * 130 * 4


def test_paged_attention_scratch_grows_with_batch_and_context():
    """The scratch size never shrinks as num_seqs or max_context_len grow, so one
    buffer sized for the largest call serves every smaller one; and it holds the
    partials of the partition length the launch picks: 512 tokens when
    sequences x kv heads x 512-token partitions reach 512 workgroups, else 256
    when 128-token ones would reach 256, else 64."""
    def need(seqs, ctx, kvh=8, heads=32):
        parts = lambda p: -(-ctx // p)  # noqa: E731
        part = 512 if seqs * kvh * parts(512) >= 512 else (256 if seqs * kvh * parts(128) >= 256 else 64)
        return seqs * heads * parts(part) * 130 * 4
    def size(seqs, ctx):
        n = C.c_size_t()
        a = paged_args(num_seqs=seqs, max_context_len=ctx, max_blocks_per_seq=(ctx + 15) // 16)
        st, msg = _status(N.lib().tlh_paged_attention_scratch_bytes, C.byref(a), C.byref(n))
        assert st == "OK", msg
        return n.value
    for ctx in (1, 255, 256, 257, 4096, 8192, 8193):
        sizes = [size(s, ctx) for s in range(1, 40)]
        assert sizes == sorted(sizes), ctx
        assert all(sz >= need(s, ctx) for s, sz in zip(range(1, 40), sizes)), ctx
    for s in (1, 3, 4, 32):
        sizes = [size(s, c) for c in range(1, 9000, 97)]
        assert sizes == sorted(sizes), s
        assert all(sz >= need(s, c) for c, sz in zip(range(1, 9000, 97), sizes)), s


def _fa_op(nb=2, nh=8, nhkv=2, nq=1, L=1000, D=128, DV=None, kdt="f16", mask=True, **kw):
    import torch

    DV = D if DV is None else DV
    dt = {"f16": torch.float16, "f32": torch.float32}[kdt]
    q = torch.zeros((nb, nh, nq, D))
    k = torch.zeros((nb, nhkv, L, D), dtype=dt)
    v = torch.zeros((nb, nhkv, L, DV), dtype=dt)
    m = torch.zeros((nb, 1, nq, L), dtype=torch.float16) if mask else None
    d = torch.zeros((nb, nq, nh, DV))
    return N.flash_attn_op(q, k, v, m, d, 0.1, **kw)


def fa_scratch_status(op):
    n = C.c_size_t()
    st, msg = _status(N.lib().tlh_flash_attn_ext_scratch_bytes, C.byref(op), C.byref(n))
    return st, msg, n.value


def test_flash_attn_op_packs_the_lowering_parameters():
    """x0..x5 as Ctx::flash_attn_ext packs them (lower.rs:604-620): scale divided by
    softcap, n_head_log2 = 8 for 12 heads, m0 = 2^(-8/8), m1 = 2^(-4/8)."""
    import struct

    op = _fa_op(nh=12, nhkv=4, softcap=20.0, max_bias=8.0)
    f = [struct.unpack("<f", struct.pack("<i", op.x[i]))[0] for i in (0, 1, 2, 3, 5)]
    assert f[0] == pytest.approx(0.1 / 20.0, rel=1e-6) and f[1] == 8.0 and f[4] == 20.0
    assert op.x[4] == 8 and f[2] == pytest.approx(0.5, rel=1e-6) and f[3] == pytest.approx(2 ** -0.5, rel=1e-6)
    assert list(op.t[3].ne) == [1000, 1, 1, 2] and op.t[3].ty == N.F16
    assert list(op.t[4].ne) == [128, 12, 1, 2]


def test_flash_attn_scratch_sizes():
    """Partials [nb][nh][nq][P][DV + 2] f32 when the keys are split (rounded up to
    256 bytes); nothing for the mask, which the kernel scans itself."""
    st, msg, n = fa_scratch_status(_fa_op(nb=32, nh=32, nhkv=8, L=4096, mask=False))
    assert st == "OK", msg
    assert n == 32 * 32 * 4 * (128 + 2) * 4  # the bench shape: 4 partitions of 1024 keys
    st, msg, n = fa_scratch_status(_fa_op(L=100, mask=False))
    assert st == "OK" and n == 0  # too short to split, no mask
    st, msg, n = fa_scratch_status(_fa_op(L=100, nq=3))
    assert st == "OK" and n == 0  # too short to split; the kernel scans the mask itself
    st, msg, n = fa_scratch_status(_fa_op(nb=1, nh=8, nhkv=8, nq=3, L=5000, D=64, mask=False))
    assert st == "OK" and n > 0 and n % 256 == 0


@pytest.mark.parametrize("kw,status,text", [
    ({"kdt": "f32"}, "UNSUPPORTED", "K/V of type f32"),
    ({"D": 48}, "UNSUPPORTED", "head sizes"),
    ({"D": 128, "DV": 64}, "UNSUPPORTED", "head sizes"),
    ({"D": 576, "DV": 512}, "UNSUPPORTED", "head sizes"),
    ({"nhkv": 3}, "UNSUPPORTED", "inconsistent"),
    ({"D": 192, "DV": 128}, "OK", ""),
    ({"D": 72}, "OK", ""),
])
def test_flash_attn_validation(kw, status, text):
    st, msg, _ = fa_scratch_status(_fa_op(**kw))
    assert st == status, msg
    assert text in msg


def test_no_device_is_reported_not_fatal():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(N.TlhError) as e:
        N.device_props(0)
    assert e.value.status == "NO_DEVICE"


# ------------------------------------------------------------------ core ops
def _core(kind, srcs, dst, x=(), has1=None, has2=None):
    op = N.core_op(srcs, dst, x)
    has1 = len(srcs) > 1 and srcs[1] is not None if has1 is None else has1
    has2 = len(srcs) > 2 and srcs[2] is not None if has2 is None else has2
    return _status(N.lib().tlh_core_check, kind, C.byref(op), int(has1), int(has2))


def test_core_params_pack_as_the_lowering_does():
    """Ctx::rope (lower.rs:422-466) and Ctx::soft_max (:314-341): theta_scale =
    freq_base^(-2/n_dims), YaRN corr dims from ggml_rope_yarn_corr_dims (for
    n_dims 128, n_ctx_orig 4096, base 10000, beta 32/1: [20, 46]); ALiBi m0/m1
    for 12 heads and max_bias 8: n_head_log2 8, m0 = 2^-1, m1 = 2^-0.5."""
    import struct

    f = lambda b: struct.unpack("<f", struct.pack("<i", b))[0]  # noqa: E731
    x = N.rope_params(128, 2, 4096, 10000.0, 1.0, 1.0, 1.0, 32.0, 1.0, False)
    assert x[0] == 128 and x[1] == 2 and x[8] == 0
    assert f(x[5]) == pytest.approx(10000.0 ** (-2 / 128), rel=1e-7)
    assert (f(x[6]), f(x[7])) == (20.0, 46.0)
    sm = N.soft_max_params(12, 0.125, 8.0)
    assert f(sm[0]) == 0.125 and f(sm[1]) == 8.0 and sm[4] == 8
    assert f(sm[2]) == 0.5 and f(sm[3]) == pytest.approx(2 ** -0.5, rel=1e-7)


def test_core_validation():
    """What tlh_core_check accepts and refuses, by kind, without a GPU."""
    f32 = lambda *ne: N.ggml_tensor(N.F32, ne)  # noqa: E731
    f16 = lambda *ne: N.ggml_tensor(N.F16, ne)  # noqa: E731
    i32 = lambda *ne: N.ggml_tensor(N.I32, ne)  # noqa: E731
    ok = [
        (N.CORE_BIN, [f32(64, 5), f32(64, 1)], f32(64, 5), (0,)),
        (N.CORE_BIN, [f16(64, 5), f32(64, 5)], f16(64, 5), (3,)),
        (N.CORE_UNARY, [f32(9, 2)], f32(9, 2), (10,)),
        (N.CORE_UNARY, [f16(9, 2)], f32(9, 2), (108,)),
        (N.CORE_NORM, [f32(4096, 2)], f32(4096, 2), (1,)),
        (N.CORE_GET_ROWS, [N.ggml_tensor(N.Q4_K, [512, 40]), i32(7)], f32(512, 7), ()),
        (N.CORE_SET_ROWS, [f32(512, 5), i32(5)], f16(512, 64), ()),
        (N.CORE_CPY, [f32(128, 32, 2)], f16(4096, 2), ()),
        (N.CORE_ROPE, [f32(128, 32, 2), i32(2)], f32(128, 32, 2), (128, 2)),
        (N.CORE_SOFT_MAX, [f32(300, 5, 32), f16(300, 8)], f32(300, 5, 32), ()),
        (N.CORE_ARGMAX, [f32(32000, 4)], N.ggml_tensor(N.I32, [4]), ()),
        (N.CORE_GLU, [f32(2752, 2)], f32(1376, 2), (2, 0)),
        (N.CORE_GLU, [f32(1376, 2), f32(1376, 2)], f32(1376, 2), (1, 0)),
    ]
    for kind, srcs, dst, x in ok:
        st, msg = _core(kind, srcs, dst, x)
        assert st == "OK", (kind, msg)
    bad = [
        (N.CORE_BIN, [f32(64, 5), f32(64, 2)], f32(64, 5), (0,), "UNSUPPORTED", "repeat"),
        (N.CORE_BIN, [f32(64, 5), f32(64, 5)], f32(64, 5), (4,), "INVALID", "BIN code"),
        (N.CORE_UNARY, [f32(9, 2)], f32(9, 2), (17,), "UNSUPPORTED", "unary op 17"),
        (N.CORE_NORM, [f16(64, 2)], f32(64, 2), (1,), "UNSUPPORTED", "NORM"),
        (N.CORE_GET_ROWS, [N.ggml_tensor(16, [512, 40], [66, 132, 5280, 5280]), i32(7)], f32(512, 7), (),
         "UNSUPPORTED", "GET_ROWS"),
        (N.CORE_GET_ROWS, [f32(512, 40), i32(7)], f32(512, 6), (), "UNSUPPORTED", "shapes"),
        (N.CORE_SET_ROWS, [f32(512, 5), i32(4)], f32(512, 64), (), "UNSUPPORTED", "shapes"),
        (N.CORE_CPY, [f32(128, 32)], f32(128, 31), (), "UNSUPPORTED", "element counts"),
        (N.CORE_ROPE, [f32(128, 32, 2), i32(2)], f32(128, 32, 2), (128, 1), "UNSUPPORTED", "modes"),
        (N.CORE_ROPE, [f32(128, 32, 2), i32(3)], f32(128, 32, 2), (128, 2), "UNSUPPORTED", "position"),
        (N.CORE_ROPE, [f32(128, 32, 2), i32(2)], f32(128, 32, 2), (130, 2), "INVALID", "n_dims"),
        (N.CORE_SOFT_MAX, [f32(300, 5), f16(299, 5)], f32(300, 5), (), "UNSUPPORTED", "mask"),
        (N.CORE_ARGMAX, [f32(100, 4, 2)], N.ggml_tensor(N.I32, [4]), (), "UNSUPPORTED", "2-D"),
        (N.CORE_GLU, [f32(2752, 2)], f32(1375, 2), (2, 0), "UNSUPPORTED", "shapes"),
        (N.CORE_GLU, [f32(2752, 2)], f32(1376, 2), (3, 0), "UNSUPPORTED", "glu op 3"),
        (99, [f32(4)], f32(4), (), "INVALID", "unknown kind"),
    ]
    for kind, srcs, dst, x, status, text in bad:
        st, msg = _core(kind, srcs, dst, x)
        assert st == status and text in msg, (kind, st, msg)
    st, msg = _core(N.CORE_ROPE, [f32(128, 32, 2), i32(2)], f32(128, 32, 2), (128, 2, 0, 0, 0, 0, 0, 0, 1))
    assert st == "UNSUPPORTED" and "frequency factors" in msg


def _mmid_op(wt=N.Q4_K, K=512, M=64, n_as=8, n_used=2, n_b1=2, n_tok=3, ids_ty=26):
    op = N.TlhOp()
    be, bb = N.BLOCK.get(wt, (256, 110))  # q3_K, unsupported: 110-byte super-blocks
    rb = K // be * bb

    def t(slot, ty, ne, nb):
        op.t[slot].ty = ty
        for i in range(4):
            op.t[slot].ne[i], op.t[slot].nb[i] = ne[i], nb[i]
    t(0, wt, [K, M, n_as, 1], [bb, rb, rb * M, rb * M * n_as])
    t(1, N.F32, [K, n_b1, n_tok, 1], [4, 4 * K, 4 * K * n_b1, 4 * K * n_b1 * n_tok])
    t(2, ids_ty, [n_used, n_tok, 1, 1], [4, 4 * n_used, 4 * n_used * n_tok, 4 * n_used * n_tok])
    t(4, N.F32, [M, n_used, n_tok, 1], [4, 4 * M, 4 * M * n_used, 4 * M * n_used * n_tok])
    return op


def test_mul_mat_id_scratch_and_validation():
    """Scratch = src1 quantized once (n_b1 x n_tokens rows) + K-chunk partials per
    (expert, token) pair; ggml_mul_mat_id's shape asserts (ggml.c:3334-3342) are
    refusals."""
    n = C.c_size_t()
    L = N.lib()
    st, msg = _status(L.tlh_mul_mat_id_scratch_bytes, C.byref(_mmid_op()), C.byref(n))
    assert st == "OK", msg
    al = lambda v: (v + 255) // 256 * 256  # noqa: E731
    rows, K = 2 * 3, 512
    assert n.value == al(al(al(al(rows * K) + rows * (K // 256) * 4) + rows * (K // 16) * 2))
    for kw in ({"n_b1": 3}, {"ids_ty": N.F32}, {"wt": 16}):
        st, msg = _status(L.tlh_mul_mat_id_scratch_bytes, C.byref(_mmid_op(**kw)), C.byref(n))
        assert st == "UNSUPPORTED", (kw, msg)
    op = _mmid_op()
    st, msg = _status(L.tlh_mul_mat_id, C.byref(op), None, None, None, None, None, 0, None)
    assert st == "INVALID", msg

"""GPU parity: GGML_OP_MUL_MAT with f32 / f16 / bf16 weights (mm_float.hip) through
the C ABI, against the ggml CPU backend's results (mul_mat_float.npz, written by
the reference's compiled ggml) and the oracle (tlq_mul_mat's float path, pinned
bit-exact to that backend in test_oracle.py).

What the CPU computes: src1 converted to the weight type (f16 / bf16 round to
nearest even; f32 and already-converted src1 as they are), then each output the
dot product of a weight row and a converted src1 row. Every product is exact in
f32 on both sides; only the order of the f32 sums differs. Tolerances: the
north star's 1e-3 relative / 1e-4 absolute against the CPU backend, and a
tighter bound against the oracle -- |got - want| <= 1e-6 * sum_k |w_k x_k| --
that a src1 left unconverted (about 5e-4 relative per f16 product, about 4e-3
per bf16 product) or a dropped term fails.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import BF16, F16, F32, SDPA_CASES, oracle, ref, sdpa_graph, sdpa_inputs, xorshift_noise
from tensorlisp_amd import native as N
from tensorlisp_amd import synth

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-3, 1e-4
FLOATS = ((F32, "f32"), (F16, "f16"), (BF16, "bf16"))


def gold():
    return np.load(GOLD / "mul_mat_float.npz")


def torch_of(bits_or_f32, t):
    """A device tensor of type t from f32 values or uint16 bits."""
    import torch

    a = np.ascontiguousarray(bits_or_f32)
    if t == F32:
        return torch.from_numpy(a.astype(np.float32)).cuda()
    dt = torch.float16 if t == F16 else torch.bfloat16
    return torch.from_numpy(a.view(np.int16)).cuda().view(dt)


def wbits(w_f32, t):
    """f32 weights as the stored rows of type t (f32 values or uint16 bits)."""
    import torch

    if t == F32:
        return np.ascontiguousarray(w_f32, np.float32)
    dt = torch.float16 if t == F16 else torch.bfloat16
    return torch.from_numpy(np.ascontiguousarray(w_f32, np.float32)).to(dt).view(torch.int16).numpy().view(np.uint16)


def as_f32(bits, t):
    import torch

    if t == F32:
        return np.asarray(bits, np.float32)
    dt = torch.float16 if t == F16 else torch.bfloat16
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dt).to(torch.float32).numpy()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def close(got, want, what=""):
    err = np.abs(got - want)
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tol, max err {err.max():.3e}"


def tight(got, want, wd, xd, what=""):
    """|got - want| <= 1e-6 * sum_k |w x| for y [N, M] = xd [N, K] . wd [M, K]^T."""
    scale = np.abs(xd).astype(np.float64) @ np.abs(wd).astype(np.float64).T
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= 1e-6 * scale + 1e-30).all(), f"{what}: max err / scale {(err / (scale + 1e-30)).max():.3e}"


@pytest.mark.parametrize("t,name", FLOATS, ids=[n for _, n in FLOATS])
def test_reference_cases_golden(gpu, t, name):
    """crates/tensorlisp/tests/native.rs:73-107 (f32, f16, bf16 among its types):
    96 x 256 noise weights, n in 1,3,5,8,9,40, one launch and the split
    conversion + products; then K = 100 (element-wise path)."""
    g = gold()
    w = torch_of(g[f"{name}_w"].view(np.float32 if t == F32 else np.uint16), t)
    for n in g["ns"]:
        x = xorshift_noise((int(n), 256), 10 + int(n))
        for split in (False, True):
            y = host(N.mul_mat_views(w, torch_of(x, F32), split=split))[0, 0]
            close(y, g[f"{name}_y{n}"], f"{name} n={n} split={split}")
    w100 = torch_of(g[f"k100_{name}_w"].view(np.float32 if t == F32 else np.uint16), t)
    for split in (False, True):
        y = host(N.mul_mat_views(w100, torch_of(g["k100_x"], F32), split=split))[0, 0]
        close(y, g[f"k100_{name}_y"], f"{name} K=100 split={split}")


@pytest.mark.parametrize("t,name", [(F16, "f16"), (BF16, "bf16")], ids=["f16", "bf16"])
def test_src1_of_the_weight_type_golden(gpu, t, name):
    """src1 already f16 / bf16 (ggml_mul_mat of two f16 tensors): read as it is."""
    g = gold()
    w = torch_of(g[f"{name}_w"].view(np.uint16), t)
    for n in (1, 9):
        x = torch_of(g[f"{name}_x{n}_same"], t)
        for split in (False, True):
            y = host(N.mul_mat_views(w, x, split=split))[0, 0]
            close(y, g[f"{name}_y{n}_same"], f"{name} n={n} split={split}")


@pytest.mark.parametrize("M,K,n", [(4096, 4096, 1), (1000, 4096, 7), (512, 1000, 40), (300, 136, 64)])
@pytest.mark.parametrize("t,name", FLOATS, ids=[n for _, n in FLOATS])
def test_against_oracle(gpu, t, name, M, K, n):
    """Decode (n = 1), few columns and prefill-like widths against the oracle,
    to the tight bound; K = 1000 and 136 end in a partial 512-element step."""
    o = oracle()
    wb = wbits(synth.normal(500 + K + n, (M, K)), t)
    x = synth.normal(600 + n, (n, K)) * 2
    y = host(N.mul_mat_views(torch_of(wb, t), torch_of(x, F32)))[0, 0]
    want = o.mul_mat(t, wb, M, K, x)
    xd = as_f32(wbits(x, t), t)
    tight(y, want.astype(np.float64), as_f32(wb, t), xd, f"{name} {M}x{K} n={n}")
    close(y, want, name)


@pytest.mark.parametrize("t,name", FLOATS, ids=[n for _, n in FLOATS])
def test_split_is_bit_identical_when_both_read_aligned_rows(gpu, t, name):
    """The split form converts src1 into scratch rows of the weight type; the one
    launch converts as it loads. Same products, same order: identical bits."""
    wb = wbits(synth.normal(71, (200, 512)), t)
    x = torch_of(synth.normal(72, (13, 512)), F32)
    w = torch_of(wb, t)
    a = host(N.mul_mat_views(w, x))
    b = host(N.mul_mat_views(w, x, split=True))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("t,name", FLOATS, ids=[n for _, n in FLOATS])
def test_batch_broadcast_and_strided_views(gpu, t, name):
    """ggml_mul_mat's broadcast (weights [K, M, 2, 1] over src1 [K, N, 4, 3]:
    r2 = 2, r3 = 3) on permuted, padded views of both operands and a strided dst;
    each batch slice against the oracle on that slice."""
    import torch

    o = oracle()
    K, M, Nc = 72, 50, 6
    # weights stored [2][M][K + 8] (rows padded: nb1 = (K + 8) * es), viewed [2, M, K]
    wfull = synth.normal(81, (2, M, K + 8))
    wb = wbits(wfull, t)
    w = torch_of(wb, t)[:, :, :K].unsqueeze(0)  # (1, 2, M, K)
    # src1 stored [N][3][4][K] and permuted to (3, 4, N, K)
    xs = synth.normal(82, (Nc, 3, 4, K))
    x = torch_of(xs, F32).permute(1, 2, 0, 3)
    out_store = torch.full((3, 4, Nc, M + 5), 7.0, device="cuda")
    out = out_store[:, :, :, :M]
    N.mul_mat_views(w, x, out=out)
    got = host(out_store)
    for i3 in range(3):
        for i2 in range(4):
            wsl = np.ascontiguousarray(wb[i2 // 2, :, :K])
            want = o.mul_mat(t, wsl, M, K, np.ascontiguousarray(xs[:, i3, i2, :]))
            close(got[i3, i2, :, :M], want, f"{name} slice {i3},{i2}")
    assert (got[:, :, :, M:] == 7.0).all()  # the padding is not written


@pytest.mark.parametrize("t,name", [(F16, "f16"), (BF16, "bf16")], ids=["f16", "bf16"])
def test_unaligned_rows_take_the_element_path(gpu, t, name):
    """Rows at an odd element offset (2-byte aligned only) and K = 130: the
    element-wise loop, against the oracle to the tight bound."""
    o = oracle()
    M, K, n = 70, 130, 5
    wb = wbits(synth.normal(91, (M, K + 1)), t)
    w = torch_of(wb, t)[:, 1:]  # starts 2 bytes into a row
    x = synth.normal(92, (n, K))
    y = host(N.mul_mat_views(w, torch_of(x, F32)))[0, 0]
    wsl = np.ascontiguousarray(wb[:, 1:])
    want = o.mul_mat(t, wsl, M, K, x)
    tight(y, want.astype(np.float64), as_f32(wsl, t), as_f32(wbits(x, t), t), name)


def test_refusals(gpu):
    """f32 weights take only f32 src1; f16 weights take f32 or f16 (not bf16);
    rows must be contiguous along K."""
    import torch

    w16 = torch.zeros((8, 64), dtype=torch.float16, device="cuda")
    w32 = torch.zeros((8, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(N.TlhError):
        N.mul_mat_views(w32, torch.zeros((2, 64), dtype=torch.float16, device="cuda"))
    with pytest.raises(N.TlhError):
        N.mul_mat_views(w16, torch.zeros((2, 64), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(N.TlhError):
        N.mul_mat_views(w16, torch.zeros((64, 2), dtype=torch.float32, device="cuda").t())


@pytest.mark.parametrize("i", range(len(SDPA_CASES)))
def test_sdpa_graph_through_the_executor(gpu, i):
    """attn:sdpa's non-flash branch (attn.ss:75-90) as a graph: MUL_MAT of the
    f16 / f32 / bf16 keys with the f32 queries, SOFT_MAX_EXT with a causal mask,
    MUL_MAT of the transposed values with the probabilities, heads merged; against
    the CPU backend running the same graph (mul_mat_float.npz; live through
    oracle/_ref where it is built)."""
    import torch

    from tensorlisp_amd import graph as G

    case = SDPA_CASES[i]
    b, merged, _ = sdpa_graph(*case)
    ins = sdpa_inputs(case, 300 + 10 * i)
    prog = G.Program(b, [merged], [])
    for j, a in enumerate(ins):
        src = torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
        prog.write_input(j, src)
    prog.run()
    got = host(prog.read(merged, torch.float32)).reshape(gold()[f"sdpa{i}"].shape)
    close(got, gold()[f"sdpa{i}"], f"sdpa case {case}")
    r = ref()
    if r is not None:
        close(got, r.ir_run(b, [], [], ins, [(merged, np.float32)])[0], "live")


def test_bf16_get_rows_and_cpy(gpu):
    """bf16 tables through GET_ROWS (to f32) and CPY (f32 -> bf16, bf16 -> f32 /
    f16), against the oracle: bit-exact (conversions only)."""
    import torch

    o = oracle()
    table = wbits(synth.normal(95, (2, 3, 40, 96)), BF16)  # (i3, i2, rows, ne0)
    idx = synth.integers(96, 0, 39, 2 * 3 * 5).astype(np.int32).reshape(2, 3, 5)
    got = host(N.get_rows(torch_of(table, BF16), torch.from_numpy(idx).cuda()))
    want = o.core_get_rows(table, BF16, idx, 26)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    f = synth.normal(97, (6, 128)) * 100
    f[0, :4] = [np.inf, -np.inf, 0.0, -0.0]
    dst = torch.empty((6, 128), dtype=torch.bfloat16, device="cuda")
    N.cpy(torch_of(f, F32), dst)
    got = host(dst.view(torch.int16)).view(np.uint16)
    assert np.array_equal(got, o.core_cpy(f, F32, (6, 128), BF16))
    assert np.array_equal(got, o.f32_to_bf16(f))
    back = torch.empty((6, 128), dtype=torch.float32, device="cuda")
    N.cpy(dst, back)
    assert np.array_equal(host(back).view(np.uint32), o.core_cpy(got, BF16, (6, 128), F32).view(np.uint32))
    h = torch.empty((6, 128), dtype=torch.float16, device="cuda")
    N.cpy(dst, h)
    assert np.array_equal(host(h.view(torch.int16)).view(np.uint16), o.core_cpy(got, BF16, (6, 128), F16))

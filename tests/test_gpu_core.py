"""GPU parity: the core ops of a decoder step through the C ABI (tlh_core).

Every case of refs.core_cases() (the shapes and inputs of the reference's own
tests, crates/tensorlisp/tests/native.rs:109-498, and decoder-sized ones) runs
on the GPU and is compared with the reference CPU backend's output kept in
tests/golden/core.npz:
  * bit-exact for BIN, GET_ROWS (every weight type), SET_ROWS, CPY, ARGMAX, the
    unary ops without a transcendental function and REGLU;
  * NORM / RMS_NORM within 1e-6 relative (both sum in double; only the order of
    the double additions differs);
  * ops through expf / tanhf / sinf / cosf / logf / erff (the GPU's libm, the
    CPU's glibc or its polynomial exp): 4e-6 relative + 1e-6 absolute;
  * GELU-family values go through f16 like the CPU's tables, so a last-bit
    difference before the rounding may move one f16 ulp: 1e-3 relative; f16
    outputs of RoPE likewise.
Then the edges: 262144-long argmax rows with repeated maxima (native.rs:416-435),
more than 65535 rows, empty tensors, strided views (rows of a fused QKV buffer,
a transposed operand), indices outside the table, fully masked softmax rows.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import (CORE_KINDS, F16, F32, I32, I64, NP_OF, core_cases, core_perm_view, oracle, xorshift_noise)
from tensorlisp_amd import native as N

pytestmark = pytest.mark.gpu
CASES = core_cases()
EXACT_UNARY = {0, 1, 2, 3, 6, 11, 12, 18, 19, 20, 21, 100, 101, 102, 103, 104, 105}
F16_ROUNDED_UNARY = {8, 9}
EXACT_KINDS = {CORE_KINDS[k] for k in ("bin", "get_rows", "set_rows", "cpy", "argmax")}


def gold():
    return np.load(Path(__file__).resolve().parent / "golden" / "core.npz")


def dev(a):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    return torch.from_numpy(a).cuda()


def host(t):
    import torch

    if t.dtype == torch.float16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def empty(shape, ty):
    import torch

    dt = {F32: torch.float32, F16: torch.float16, I32: torch.int32, I64: torch.int64}[ty]
    return torch.empty(shape, dtype=dt, device="cuda")


def run_case(case):
    """The case through the product path (tensorlisp_amd.native -> tlh_core)."""
    import torch

    k, srcs, ip, fp = case["kind"], case["srcs"], case["ip"], case["fp"]
    shape, td = case["dst"]
    a = srcs[0]
    wt = a[1] if a[1] not in (F32, F16) else None
    kk = a[2] if len(a) > 2 else None
    A = dev(a[0])
    out = empty(shape, td)
    if k == CORE_KINDS["bin"]:
        N.binary(ip[0], A, dev(srcs[1][0]), out=out)
    elif k == CORE_KINDS["unary"]:
        p = tuple(fp) + (0.0, 0.0)
        N.unary(ip[0], A, p[0], p[1], out=out)
    elif k == CORE_KINDS["norm"]:
        N.norm(A, fp[0], rms=bool(ip[0]), out=out)
    elif k == CORE_KINDS["get_rows"]:
        N.get_rows(A, dev(srcs[1][0]), wtype=wt, k=kk, out=out)
    elif k == CORE_KINDS["set_rows"]:
        out = dev(case["init"])
        N.set_rows(out, A, dev(srcs[1][0]))
    elif k == CORE_KINDS["cpy"]:
        src = A
        if case["perm"] is not None:  # ggml_permute's view of the base, in torch
            v = core_perm_view(np.ascontiguousarray(a[0]), case["perm"])
            src = torch.as_strided(A, v.shape, [st // v.itemsize for st in v.strides])
        N.cpy(src, out, wtype=wt, k=kk)
    elif k == CORE_KINDS["rope"]:
        ff = dev(srcs[2][0]) if len(srcs) > 2 else None
        N.rope(A, dev(srcs[1][0]), ip[0], ip[1], ip[2], *fp, freq_factors=ff, out=out)
    elif k == CORE_KINDS["soft_max"]:
        m = dev(srcs[1][0]) if len(srcs) > 1 else None
        N.soft_max(A, m, fp[0], fp[1], out=out)
    elif k == CORE_KINDS["argmax"]:
        N.argmax(A, out=out)
    elif k == CORE_KINDS["glu"]:
        N.glu(ip[0], A, dev(srcs[1][0]) if len(srcs) > 1 else None, bool(ip[1]), out=out)
    else:
        raise ValueError(k)
    torch.cuda.synchronize()
    return host(out)


def tolerance(case):
    """None for bit-exact, else (relative, absolute) per element."""
    k, td = case["kind"], case["dst"][1]
    code = case["ip"][0] if case["ip"] else None
    if k in EXACT_KINDS:
        return None
    if k == CORE_KINDS["unary"]:
        if code in EXACT_UNARY:
            return None
        return (1e-3, 1e-6) if code in F16_ROUNDED_UNARY or td == F16 else (4e-6, 1e-6)
    if k == CORE_KINDS["glu"]:
        return None if code == 0 else (1e-3, 1e-6) if code in (1, 5) else (4e-6, 1e-6)
    if k == CORE_KINDS["norm"]:
        return (1e-6, 1e-7)
    if k == CORE_KINDS["rope"]:
        return (1e-3, 1e-6) if td == F16 else (4e-6, 1e-6)
    return (4e-6, 1e-9)  # soft_max


def compare(got, want, tol, what):
    assert got.shape == want.shape and got.dtype == want.dtype, (what, got.shape, want.shape)
    if tol is None:
        bad = ~((got == want) | (np.isnan(got.astype(np.float64)) & np.isnan(want.astype(np.float64))))
        assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} differ, first at {np.argwhere(bad)[0]}: " \
                              f"{got[tuple(np.argwhere(bad)[0])]} != {want[tuple(np.argwhere(bad)[0])]}"
        return
    o = oracle()
    g = o.f16_to_f32(got).astype(np.float64) if got.dtype == np.uint16 else got.astype(np.float64)
    w = o.f16_to_f32(want).astype(np.float64) if want.dtype == np.uint16 else want.astype(np.float64)
    with np.errstate(invalid="ignore"):
        ok = (g == w) | (np.abs(g - w) <= tol[0] * np.abs(w) + tol[1]) | (np.isnan(g) & np.isnan(w))
    assert ok.all(), f"{what}: max err {np.nanmax(np.abs(g - w))}, {int((~ok).sum())} outside {tol}"


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_core_case_matches_reference(gpu, case):
    print(f"[core] {case['name']}", flush=True)
    compare(run_case(case), gold()[case["name"]], tolerance(case), case["name"])


def test_argmax_long_rows(gpu):
    """native.rs:416-435: rows of 100 .. 262144 with the maximum repeated in three
    chunks, in the last element, or noise; ggml's CPU backend (and so this
    kernel) returns the last index among equal maxima."""
    import torch

    o = oracle()
    for n in (100, 16384, 20000, 262144):
        x = xorshift_noise([3, n], 5)
        for j in (n // 3, n // 2 + 1, n - 1):
            x[0, j] = 5.0
        x[1, n - 1] = 9.0
        got = N.argmax(dev(x))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(got), o.core_argmax(x))
        assert host(got)[0] == n - 1


def test_many_rows_and_empty(gpu):
    """More rows than one grid dimension holds (65535), and tensors with no
    elements (no launch, no error)."""
    import torch

    rng = np.random.default_rng(3)
    a = rng.standard_normal((70001, 8)).astype(np.float32)
    b = rng.standard_normal((1, 8)).astype(np.float32)
    got = N.add(dev(a), dev(b))
    n = N.rms_norm(dev(a), 1e-6)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), a + b)
    want = oracle().core_norm(True, 1e-6, a)
    np.testing.assert_allclose(host(n), want, rtol=1e-6, atol=1e-7)
    z = torch.empty((0, 16), dtype=torch.float32, device="cuda")
    for f in (lambda: N.add(z, z[:, :1]), lambda: N.rms_norm(z, 1e-6), lambda: N.unary("silu", z),
              lambda: N.soft_max(z), lambda: N.argmax(z)):
        r = f()
        torch.cuda.synchronize()
        assert r.numel() == 0


def test_strided_views(gpu):
    """Views as ggml hands them over: RoPE on the Q part of a fused QKV buffer
    (row stride wider than the row), RMS_NORM on padded rows, ADD with a
    transposed operand, CPY of a permuted view to f16 (ggml_cont + cast)."""
    import torch

    o = oracle()
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((3, 3 * 4 * 64)).astype(np.float32)  # tokens x (q | k | v), 4 heads of 64
    Q = dev(qkv)
    qv = Q[:, :256].view(3, 4, 64)  # ggml [64, 4, 3], nb1 = 256 B, nb2 = 3072 B
    pos = np.array([3, 9, 2000], np.int32)
    got = N.rope(qv, dev(pos), 64, 2, 0, 10000.0)
    want = o.core_rope(qkv[:, :256].reshape(3, 4, 64), F32, pos, 64, 2, 0, 10000.0, 1.0, 0.0, 1.0, 32.0, 1.0)
    torch.cuda.synchronize()
    compare(host(got), want, (4e-6, 1e-6), "rope view")
    padded = rng.standard_normal((5, 300)).astype(np.float32)
    got = N.rms_norm(dev(padded)[:, :257], 1e-5)
    torch.cuda.synchronize()
    compare(host(got), o.core_norm(True, 1e-5, np.ascontiguousarray(padded[:, :257])), (1e-6, 1e-7), "norm view")
    x = rng.standard_normal((6, 40)).astype(np.float32)
    y = rng.standard_normal((40, 6)).astype(np.float32)
    got = N.add(dev(x), dev(y).t())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), x + y.T)
    t = rng.standard_normal((2, 8, 32)).astype(np.float32)
    src = dev(t).permute(1, 0, 2)
    out = empty((8, 2, 32), F16)
    N.cpy(src, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(out), o.core_cpy(t.transpose(1, 0, 2), F32, (8, 2, 32), F16))


def test_index_and_mask_edges(gpu):
    """GET_ROWS indices outside the table read its nearest row, SET_ROWS indices
    outside the destination write nothing (ggml asserts in both cases), and a
    softmax row whose every entry is masked gives zeros."""
    import torch

    rng = np.random.default_rng(9)
    tab = rng.standard_normal((10, 16)).astype(np.float32)
    got = N.get_rows(dev(tab), dev(np.array([-1, 100, 4], np.int32)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), tab[[0, 9, 4]])
    dst = dev(np.zeros((4, 16), np.float32))
    N.set_rows(dst, dev(tab[:3]), dev(np.array([-2, 2, 4], np.int64)))
    torch.cuda.synchronize()
    want = np.zeros((4, 16), np.float32)
    want[2] = tab[1]
    np.testing.assert_array_equal(host(dst), want)
    s = rng.standard_normal((1, 1, 2, 8)).astype(np.float32)
    m = np.zeros((1, 1, 2, 8), np.float32)
    m[0, 0, 1] = -np.inf
    got = host(N.soft_max(dev(s), dev(m)))
    assert np.all(got[0, 0, 1] == 0)
    np.testing.assert_allclose(got[0, 0, 0].sum(), 1.0, rtol=1e-6)


def test_refusals(gpu):
    """Configurations the kernels do not take fail with the library's error, before
    any launch."""
    import torch

    a = torch.zeros((4, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(N.TlhError, match="NORM"):
        N.rms_norm(a, 1e-6)
    with pytest.raises(N.TlhError, match="SOFT_MAX"):
        N.soft_max(a)
    x = torch.zeros((4, 7), dtype=torch.float32, device="cuda")
    with pytest.raises(N.TlhError, match="GLU"):
        N.glu("swiglu", x, out=torch.empty((4, 3), device="cuda"))
    with pytest.raises(N.TlhError, match="glu op"):
        N.glu(3, torch.zeros((4, 8), device="cuda"))
    with pytest.raises(N.TlhError, match="ROPE"):
        N.rope(torch.zeros((2, 4, 8), device="cuda"), torch.zeros(2, dtype=torch.int32, device="cuda"), 8, 1)
    with pytest.raises(N.TlhError, match="BIN"):
        N.add(x, torch.zeros((4, 3), device="cuda"))


def test_get_rows_q5_K_table(gpu):
    """GET_ROWS from q5_K rows (the token embedding of Q5_K_M files) equals the
    reference's dequantize_row_q5_K of the picked rows bit for bit (q5_K.npz)."""
    import torch

    from refs import Q5_K

    g = np.load(Path(__file__).resolve().parent / "golden" / "q5_K.npz")
    w, deq = g["rand_w"], g["rand_deq"]  # 40 rows of 1024
    idx = np.array([3, 39, 0, 17, 17, 22], np.int32)
    out = N.get_rows(torch.from_numpy(np.ascontiguousarray(w)).cuda(), torch.from_numpy(idx).cuda(), Q5_K, 1024)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(len(idx), 1024)
    assert np.array_equal(got.view(np.uint32), deq[idx].view(np.uint32))

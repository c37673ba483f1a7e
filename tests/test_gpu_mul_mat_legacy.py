"""GPU parity: q4_1, q5_0 and q5_1 weights (the reference test's other 32-element
types, crates/tensorlisp/tests/native.rs:84) through the C ABI -- MUL_MAT at
decode (register GEMV, N <= 2), few columns (int8 MFMA, N 3..16) and prefill
widths (16-column slabs), MUL_MAT_ID, the q8_1 activation quantizer,
dequantize and GET_ROWS -- against the CPU backend's outputs
(legacy_quants.npz) and the oracle (pinned bit-exact to that backend in
test_oracle.py).

Bars: block sums are exact integers, so MUL_MAT differs from the CPU only by
the order of its f32 sums: |got - want| <= 1e-4 + 1e-3 |want| (the north
star's tolerance). The quantizer, dequantizer and GET_ROWS are bit-exact.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import NAMES, Q4_1, Q5_0, Q5_1, oracle, xorshift_noise
from tensorlisp_amd import native as N
from tensorlisp_amd import synth

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-3, 1e-4
LEGACY = ((Q4_1, 111), (Q5_0, 121), (Q5_1, 131))
IDS = [NAMES[t] for t, _ in LEGACY]


def gold():
    return np.load(GOLD / "legacy_quants.npz")


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def close(got, want, what=""):
    err = np.abs(got - want)
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tol, max err {err.max():.3e}"


@pytest.mark.parametrize("t,seed", LEGACY, ids=IDS)
def test_reference_cases_golden(gpu, t, seed):
    """native.rs:73-107: the 96 x 256 noise matrix quantized by ggml, n in
    1,3,5,8,9,40 (register GEMV, MFMA few-column kernel, 16-column slabs), and
    random blocks at K = 1024."""
    g = gold()
    name = NAMES[t]
    w = dev(g[f"{name}_w"])
    for n in g["ns"]:
        print(f"[legacy] {name} n={n}", flush=True)
        y = host(N.mul_mat(t, w, 96, 256, dev(xorshift_noise((int(n), 256), 10 + int(n)))))
        close(y, g[f"{name}_y{n}"], f"{name} n={n}")
    y = host(N.mul_mat(t, dev(g[f"{name}_rand_w"]), 40, 1024, dev(synth.normal(seed + 1, (3, 1024)))))
    close(y, g[f"{name}_rand_y"], f"{name} random blocks")


@pytest.mark.parametrize("M,K,n", [(4096, 4096, 1), (4096, 4096, 2), (1000, 14336, 1), (512, 4160, 5),
                                   (300, 96, 7), (700, 14336, 5), (256, 4096, 40)])
@pytest.mark.parametrize("t,seed", LEGACY, ids=IDS)
def test_against_oracle(gpu, t, seed, M, K, n):
    """Larger shapes against the oracle: K = 14336 (register GEMV with K split
    over waves; MFMA K chunks with partials), K = 4160 and 96 (a unit of 8
    blocks that ends early: unstaged loads), N = 40 slabs."""
    print(f"[legacy] {NAMES[t]} M={M} K={K} n={n}", flush=True)
    w = synth.random_blocks(t, seed + K + n, M, K)
    x = synth.normal(seed + 3 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    close(y, oracle().mul_mat(t, w, M, K, x), f"{NAMES[t]} {M}x{K} n={n}")


@pytest.mark.parametrize("t,seed", LEGACY, ids=IDS)
@pytest.mark.parametrize("n", [1, 2, 6])
def test_split_matches_one_launch(gpu, t, seed, n):
    """tlh_mul_mat_quantize + _compute (src1 through the q8_0 / q8_1 scratch) and
    the one-launch form (N <= 2: the GEMV quantizes src1 itself in LDS) give
    identical bits: the in-kernel quantizer writes what the quantize launch writes."""
    M, K = 520, 2048
    mm = N.MulMat(t, M, K, n)
    w = dev(synth.random_blocks(t, seed + 40, M, K))
    x = dev(synth.normal(seed + 41, (n, K)))
    import torch

    a = torch.empty((n, M), dtype=torch.float32, device="cuda")
    b = torch.empty((n, M), dtype=torch.float32, device="cuda")
    mm(w, x, a)
    mm.quantize(x)
    mm.compute(w, b)
    assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32))


def test_q8_1_quantizer_golden(gpu):
    """tlh_quantize_act for q4_1 / q5_1 weights writes ggml's block_q8_1 bytes
    (d, s, codes) exactly as quantize_row_q8_1 does, edge rows included."""
    g = gold()
    for t in (Q4_1, Q5_1):
        got = host(N.quantize_act(t, dev(g["act_x"])))
        assert np.array_equal(got, g["q8_1"])


@pytest.mark.parametrize("t,seed", LEGACY, ids=IDS)
def test_dequantize_and_get_rows(gpu, t, seed):
    """dequantize_row_* and GET_ROWS of these rows: bit-exact."""
    g = gold()
    name = NAMES[t]
    got = host(N.dequantize(t, dev(g[f"{name}_w"]), 256))
    assert np.array_equal(got.view(np.uint32), g[f"{name}_deq"].view(np.uint32))
    rw = g[f"{name}_rand_w"]
    got = host(N.dequantize(t, dev(rw[:8]), 1024))
    assert np.array_equal(got.view(np.uint32), g[f"{name}_rand_deq8"].view(np.uint32))
    idx = np.array([[3, 0, 39, 3, 17]], np.int32)
    rows = host(N.get_rows(dev(rw), dev(idx), wtype=t, k=1024))
    want = oracle().core_get_rows(rw, t, idx, 26, k=1024)
    assert np.array_equal(rows.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,seed", LEGACY, ids=IDS)
def test_mul_mat_id(gpu, t, seed):
    """MUL_MAT_ID over q4_1 / q5_0 / q5_1 experts (broadcast src1, K of two
    chunks): column (e, t) is the oracle's MUL_MAT of expert ids[t][e] with
    src1 row (e % n_b1, t)."""
    import torch

    from refs import F32, I32
    from tensorlisp_amd import graph as G

    K, M, n_as, n_used, n_b1, n_tok = 4608, 40, 4, 2, 1, 3
    b = G.Builder()
    wt = b.weight(t, [K, M, n_as], "experts")
    x = b.input(F32, [K, n_b1, n_tok], "b")
    ids = b.input(I32, [n_used, n_tok], "ids")
    y = b.mul_mat_id(wt, x, ids)
    b.expand(y)
    wh = synth.random_blocks(t, seed + 50, n_as * M, K)
    xh = synth.normal(seed + 51, (n_tok, n_b1, K))
    idh = np.array([[2, 0], [1, 3], [3, 2]], np.int32)
    prog = G.Program(b, [y], [dev(wh)])
    prog.write_input(0, dev(xh))
    prog.write_input(1, dev(idh))
    prog.run()
    got = host(prog.read(y, torch.float32)).reshape(n_tok, n_used, M)
    o = oracle()
    for tk in range(n_tok):
        for e in range(n_used):
            ex = int(idh[tk, e])
            want = o.mul_mat(t, wh[ex * M:(ex + 1) * M], M, K, xh[tk, e % n_b1][None])
            close(got[tk, e][None], want, f"{NAMES[t]} token {tk} slot {e}")

"""GPU parity: GGML_OP_MUL_MAT (decode GEMV N <= 16, prefill GEMM N > 16) through the C ABI
against the ggml CPU backend's results (golden vectors) and the oracle.

Tolerance: f32 outputs within 1e-3 relative / 1e-4 absolute,
elementwise |got - want| <= 1e-4 + 1e-3 * |want|. The integer block sums are exact;
only the f32 accumulation order differs from the CPU's sequential loop.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, oracle
from tensorlisp_amd import native as N
from tensorlisp_amd import synth

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-3, 1e-4
WTYPES = (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K)
GOLD_TYPES = (Q4_0, Q8_0, Q4_K)  # mul_mat.npz; q6_K has q6_K.npz


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


@pytest.mark.parametrize("t", GOLD_TYPES, ids=[NAMES[t] for t in GOLD_TYPES])
def test_reference_cases_golden(gpu, t):
    """crates/tensorlisp/tests/native.rs:73-107 shapes: 96 x 256, N in 1,3,5,8,9,40."""
    g = np.load(GOLD / "mul_mat.npz")
    w = dev(g[f"{NAMES[t]}_w"])
    for n in g["ns"]:
        y = host(N.mul_mat(t, w, 96, 256, dev(g[f"x{n}"])))
        close(y, g[f"{NAMES[t]}_y{n}"], f"{NAMES[t]} n={n}")


@pytest.mark.parametrize("t,xseed", [(Q6_K, 62), (Q5_K, 72)], ids=["q6_K", "q5_K"])
def test_kquant_reference_cases_golden(gpu, t, xseed):
    """q6_K / q5_K weights from ggml_quantize_chunk on the reference test's 96 x 256
    matrix and structurally random blocks: the CPU backend's outputs (q6_K.npz,
    q5_K.npz)."""
    from refs import xorshift_noise

    g = np.load(GOLD / f"{NAMES[t]}.npz")
    w = dev(g["w"])
    for n in g["ns"]:
        y = host(N.mul_mat(t, w, 96, 256, dev(xorshift_noise((int(n), 256), 10 + int(n)))))
        close(y, g[f"y{n}"], f"{NAMES[t]} n={n}")
    y = host(N.mul_mat(t, dev(g["rand_w"]), 40, 1024, dev(synth.normal(xseed, (3, 1024)))))
    close(y, g["rand_y"], f"{NAMES[t]} random blocks")


@pytest.mark.parametrize("n", [1, 2, 5, 16, 40])
@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 14336)], ids=["up", "down"])
def test_q5_K_ffn_row_sample(gpu, n, M, K):
    """q5_K FFN matrices of a Q5_K_M 8B model: register GEMV (n <= 2), MFMA
    few-column kernel (n = 5, 16; K = 14336 in K chunks) and 16-column slabs
    (n = 40), checked by the oracle on 64 rows spread over M."""
    w = synth.random_blocks(Q5_K, 700 + n + K, M, K)
    x = synth.normal(701 + n, (n, K))
    y = host(N.mul_mat(Q5_K, dev(w), M, K, dev(x)))
    rows = np.unique(synth.integers(702 + n, 0, M - 1, 64))
    want = oracle().mul_mat(Q5_K, w[rows], len(rows), K, x, nthreads=16)
    close(y[:, rows], want, f"q5_K {M}x{K} n={n}")


@pytest.mark.parametrize("n", [1, 2, 8, 40])
def test_q6_K_lm_head_row_sample(gpu, n):
    """The q6_K output projection of a Q4_K_M 8B model (128256 x 4096): register GEMV
    (n <= 2), MFMA few-column kernel (n = 8) and its 16-column slabs (n = 40), checked
    by the oracle on 96 rows spread over M."""
    M, K = 128256, 4096
    w = synth.random_blocks(Q6_K, 610 + n, M, K)
    x = synth.normal(611 + n, (n, K))
    y = host(N.mul_mat(Q6_K, dev(w), M, K, dev(x)))
    rows = np.unique(synth.integers(612, 0, M - 1, 96))
    want = oracle().mul_mat(Q6_K, w[rows], len(rows), K, x, nthreads=16)
    close(y[:, rows], want, f"q6_K lm_head n={n}")


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("M,K,n", [(65552, 4096, 8), (65545, 1024, 3), (70000, 4096, 16)])
def test_tall_few_column_form(gpu, t, M, K, n):
    """4096 or more 16-row groups with 3..16 columns and K <= 4096 (a multiple of
    256): each wave owns whole row groups over all of K (k_gemv_cols). Against
    the oracle on a row sample that includes the last rows (M not a multiple of
    16 in one case)."""
    w = synth.random_blocks(t, 620 + n, M, K)
    x = synth.normal(621 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    rows = np.unique(np.concatenate([synth.integers(622 + n, 0, M - 1, 96), np.arange(M - 20, M)]))
    want = oracle().mul_mat(t, np.ascontiguousarray(w[rows]), len(rows), K, x, nthreads=16)
    close(y[:, rows], want, f"tall {NAMES[t]} {M}x{K} n={n}")


def test_config1_q8_0_4096_golden(gpu):
    g = np.load(GOLD / "config1.npz")
    w = synth.q8_0_config1(int(g["seeds"][0]), 4096, 4096)
    x = synth.normal(int(g["seeds"][1]), (1, 4096))
    y = host(N.mul_mat(Q8_0, dev(w), 4096, 4096, dev(x)))
    close(y, g["y"], "config1")


SHAPES = [(4096, 4096), (6144, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


@pytest.mark.parametrize("t", [Q4_0, Q4_K], ids=["q4_0", "q4_K"])
@pytest.mark.parametrize("M,K", SHAPES, ids=[f"{m}x{k}" for m, k in SHAPES])
@pytest.mark.parametrize("n", [1, 8])
def test_config2_decode_gemv_shapes(gpu, t, M, K, n):
    """BASELINE config 2 at full size. 4096 x 4096 uses weights quantized from N(0, 0.02)
    by the oracle's ggml quantizer; larger shapes use structurally valid random blocks
    (quantizing 0.5 G weights on the host would dominate the test)."""
    if (M, K) == (4096, 4096):
        w = oracle().quantize(t, synth.normal(600, (M, K), 0.02))
    else:
        w = synth.random_blocks(t, 601 + M + K, M, K)
    x = synth.normal(700 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    want = oracle().mul_mat(t, w, M, K, x, nthreads=16)
    close(y, want, f"{NAMES[t]} {M}x{K} n={n}")


@pytest.mark.parametrize("n", [512, 2048])
@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 14336)], ids=["14336x4096", "4096x14336"])
def test_config3_prefill_gemm_row_sample(gpu, M, K, n):
    """BASELINE config 3 (Q4_K, N = 512 / 2048) at full size on the GPU; the oracle
    checks a sample of 96 rows spread over M (each output row is independent)."""
    w = synth.random_blocks(Q4_K, 800 + K, M, K)
    x = synth.normal(801 + n, (n, K))
    y = host(N.mul_mat(Q4_K, dev(w), M, K, dev(x)))
    rows = np.unique(synth.integers(802, 0, M - 1, 96))
    want = oracle().mul_mat(Q4_K, w[rows], len(rows), K, x, nthreads=16)
    close(y[:, rows], want, f"q4_K {M}x{K} n={n}")


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 6, 7, 8, 9, 16, 33, 100])
def test_every_column_count(gpu, t, n):
    """Odd M (partial row groups) and every GEMV column specialisation."""
    M, K = 197, 1024
    w = synth.random_blocks(t, 900 + n, M, K)
    x = synth.normal(901 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    close(y, oracle().mul_mat(t, w, M, K, x), f"{NAMES[t]} n={n}")


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("n", [3, 20])
def test_broadcast_batches_and_strides(gpu, t, n):
    """src0 [K, M, 2, 1] broadcast over src1 [K, N, 4, 3] (r2 = 2, r3 = 3), src1 rows
    padded (non-contiguous), dst with a padded row stride; GEMV (n=3) and GEMM (n=20)."""
    import ctypes as C

    import torch

    M, K, w_ne2, w_ne3, ne2, ne3 = 64, 512, 2, 1, 4, 3
    rb = N.row_bytes(t, K)
    w = synth.random_blocks(t, 950, M * w_ne2 * w_ne3, K)
    xpad = K + 64
    x = synth.normal(951, (ne3, ne2, n, xpad))
    dpad = M + 16
    dst = torch.full((ne3, ne2, n, dpad), float("nan"), dtype=torch.float32, device="cuda")
    op = N.mul_mat_op(t, M, K, n, ne2=ne2, ne3=ne3, w_ne2=w_ne2, w_ne3=w_ne3,
                      x_nb=[4, xpad * 4, xpad * 4 * n, xpad * 4 * n * ne2],
                      d_nb=[4, dpad * 4, dpad * 4 * n, dpad * 4 * n * ne2])
    nbytes = N.mul_mat_scratch_bytes(op)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    wd, xd = dev(w), dev(x)
    N.check(N.lib().tlh_mul_mat(C.byref(op), C.c_void_p(wd.data_ptr()), C.c_void_p(xd.data_ptr()),
                                C.c_void_p(dst.data_ptr()), C.c_void_p(scratch.data_ptr()), nbytes,
                                C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    got = host(dst)
    o = oracle()
    for i3 in range(ne3):
        for i2 in range(ne2):
            wi = (i2 // (ne2 // w_ne2)) + w_ne2 * (i3 // (ne3 // w_ne3))
            want = o.mul_mat(t, w[wi * M:(wi + 1) * M], M, K, x[i3, i2, :, :K])
            close(got[i3, i2, :, :M], want, f"batch {i3},{i2}")
            assert np.isnan(got[i3, i2, :, M:]).all()  # padding untouched


def test_zero_activations_and_zero_blocks(gpu):
    M, K = 64, 1024
    for t in WTYPES:
        w = synth.random_blocks(t, 960, M, K)
        x = synth.normal(961, (3, K))
        x[0] = 0.0
        x[1, :512] = 0.0
        y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
        close(y, oracle().mul_mat(t, w, M, K, x), NAMES[t])
        assert np.all(y[0] == 0.0)


def test_repeated_launches_are_deterministic(gpu):
    """The same node replayed (exec.rs:186 run loop) gives identical bits."""
    import torch

    M, K, n = 4096, 4096, 8
    w = dev(synth.random_blocks(Q4_K, 970, M, K))
    x = dev(synth.normal(971, (n, K)))
    mm = N.MulMat(Q4_K, M, K, n)
    y0 = torch.empty((n, M), dtype=torch.float32, device="cuda")
    y1 = torch.empty_like(y0)
    mm(w, x, y0)
    for _ in range(5):
        mm(w, x, y1)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))


@pytest.mark.parametrize("t,K", [(Q8_0, 96), (Q4_0, 160), (Q4_K, 16640), (Q8_0, 8224), (Q6_K, 16640), (Q5_K, 16640)],
                         ids=["q8_0-K96", "q4_0-K160", "q4_K-K16640", "q8_0-K8224", "q6_K-K16640", "q5_K-K16640"])
@pytest.mark.parametrize("n", [1, 2, 5, 8])
def test_other_K_shapes(gpu, t, K, n):
    """K outside the register-resident GEMV (K % 64 != 0 or K > 16384), so every N runs on
    the int8-MFMA kernel: K % 256 != 0 takes its direct weight loads, K > 4096 its chunked
    K with the ordered partial-sum merge."""
    M = 77
    w = synth.random_blocks(t, 980 + K, M, K)
    x = synth.normal(981 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    close(y, oracle().mul_mat(t, w, M, K, x), f"{NAMES[t]} K={K} n={n}")


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("K,n", [(8192, 3), (14336, 8), (14336, 16), (16384, 11)])
def test_mfma_long_K_chunks(gpu, t, K, n):
    """The few-column MFMA kernel splits K above 4096 into chunks whose partial sums a
    second kernel adds in order; odd M leaves a partial 16-row group."""
    M = 261
    w = synth.random_blocks(t, 1020 + K + n, M, K)
    x = synth.normal(1021 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    close(y, oracle().mul_mat(t, w, M, K, x, nthreads=16), f"{NAMES[t]} K={K} n={n}")


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("n", [1, 2])
def test_unaligned_activation_rows_take_the_quantize_launch(gpu, t, n):
    """Rows whose stride is not 16-byte aligned cannot use the fused in-register
    quantization; the node falls back to a quantize launch with the same result."""
    import ctypes as C

    import torch

    M, K = 130, 1024
    xpad = K + 1
    w = synth.random_blocks(t, 990, M, K)
    x = synth.normal(991, (n, xpad))
    op = N.mul_mat_op(t, M, K, n, x_nb=[4, xpad * 4, xpad * 4 * n, xpad * 4 * n])
    nbytes = N.mul_mat_scratch_bytes(op)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    y = torch.empty((n, M), dtype=torch.float32, device="cuda")
    wd, xd = dev(w), dev(x)
    N.check(N.lib().tlh_mul_mat(C.byref(op), C.c_void_p(wd.data_ptr()), C.c_void_p(xd.data_ptr()),
                                C.c_void_p(y.data_ptr()), C.c_void_p(scratch.data_ptr()), nbytes,
                                C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    close(host(y), oracle().mul_mat(t, w, M, K, x[:, :K]), NAMES[t])


@pytest.mark.parametrize("K", [4096, 14336])
@pytest.mark.parametrize("n", [1, 2])
def test_q4_0_weights_at_two_byte_offset(gpu, n, K):
    """The register GEMV loads q4_0 units as dwords, so it takes 4-byte aligned
    weights; weights at a 2-byte offset (allowed by the ABI) take the int8-MFMA
    kernel instead -- after a quantize launch, K-split above 4096 -- with the
    same result against the oracle."""
    import ctypes as C

    import torch

    M = 130
    w = synth.random_blocks(Q4_0, 996, M, K)
    x = synth.normal(997, (n, K))
    op = N.mul_mat_op(Q4_0, M, K, n)
    nbytes = N.mul_mat_scratch_bytes(op)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    raw = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    raw[2:2 + w.size] = dev(w.reshape(-1))
    xd = dev(x)
    want = oracle().mul_mat(Q4_0, w, M, K, x)
    for off in (0, 2):  # the aligned copy takes the register GEMV
        wd = raw[off:] if off else dev(w)
        y = torch.full((n, M), float("nan"), dtype=torch.float32, device="cuda")
        N.check(N.lib().tlh_mul_mat(C.byref(op), C.c_void_p(wd.data_ptr()), C.c_void_p(xd.data_ptr()),
                                    C.c_void_p(y.data_ptr()), C.c_void_p(scratch.data_ptr()), nbytes,
                                    C.c_void_p(torch.cuda.current_stream().cuda_stream)))
        close(host(y), want, f"q4_0 weights at offset {off}")


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
def test_split_phases_match_fused_node(gpu, t):
    """tlh_mul_mat_quantize + tlh_mul_mat_compute (the CPU's two phases) equal the
    single-call node, which fuses the quantization for N <= 2."""
    import torch

    M, K = 300, 4096
    w = dev(synth.random_blocks(t, 995, M, K))
    for n in (1, 2, 8):
        x = dev(synth.normal(996 + n, (n, K)))
        mm = N.MulMat(t, M, K, n)
        y0 = torch.empty((n, M), dtype=torch.float32, device="cuda")
        y1 = torch.empty_like(y0)
        mm(w, x, y0)
        mm.quantize(x)
        mm.compute(w, y1)
        torch.cuda.synchronize()
        close(y1.cpu().numpy(), y0.cpu().numpy(), f"{NAMES[t]} n={n}")


def tie_rows(n, K, seed):
    """Activations that exercise the quantizers' rules: N(0, 1) rows whose
    32-element blocks, in turn, hold +-127 as their largest magnitude (so d = 1
    and half-integers land exactly on rounding ties: roundf away from zero for
    q8_0, to even for q8_K), the largest magnitude twice with opposite signs
    (the first one sets q8_K's sign), or nothing but zeros."""
    x = synth.normal(seed, (n, K))
    for r in range(n):
        for b in range(K // 32):
            kind = (b + r) % 4
            blk = x[r, 32 * b:32 * b + 32]
            if kind == 0:
                blk[:] = np.round(blk * 20) + 0.5
                blk[5] = -127.0 if (b // 8) % 2 else 127.0
            elif kind == 1:
                blk[3], blk[20] = -9.0, 9.0
            elif kind == 2:
                blk[:] = 0.0
    return x.astype(np.float32)


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("K", [256, 1024, 4096, 14336])
def test_in_kernel_quantization_is_the_quantize_launch(gpu, t, K):
    """For N <= 2 and K <= 4096 the GEMV quantizes src1 itself (each workgroup
    into LDS). Its products must be bit-identical to the same GEMV reading the
    scratch of the separate quantize launch, which is pinned bit-exact to
    ggml's quantize_row_q8_0 / q8_K (test_gpu_quant.py): so are the in-kernel
    codes. (K = 14336 runs the quantize launch in both forms.)"""
    import torch

    M = 300
    w = dev(synth.random_blocks(t, 1990, M, K))
    for n in (1, 2):
        x = dev(tie_rows(n, K, 1991 + n))
        mm = N.MulMat(t, M, K, n)
        y0 = torch.empty((n, M), dtype=torch.float32, device="cuda")
        y1 = torch.empty_like(y0)
        mm(w, x, y0)
        mm.quantize(x)
        mm.compute(w, y1)
        torch.cuda.synchronize()
        a, b = y0.cpu().numpy(), y1.cpu().numpy()
        assert np.array_equal(a.view(np.int32), b.view(np.int32)), (NAMES[t], K, n, np.abs(a - b).max())


@pytest.mark.parametrize("M,K,n", [(128, 256, 128), (256, 512, 129), (300, 2304, 257), (1000, 4096, 64)])
def test_q4K_mfma_gemm_tiles(gpu, M, K, n):
    """The q4_K MFMA GEMM on exact tile multiples and ragged edges, weights quantized
    from f32 by the ggml quantizer (so scales/mins span their real ranges)."""
    w = oracle().quantize(Q4_K, synth.normal(1010 + M, (M, K), 0.02))
    x = synth.normal(1011 + n, (n, K))
    y = host(N.mul_mat(Q4_K, dev(w), M, K, dev(x)))
    close(y, oracle().mul_mat(Q4_K, w, M, K, x), f"{M}x{K} n={n}")


@pytest.mark.parametrize("t,M,K", [(Q8_0, 77, 4096), (Q4_0, 77, 4096), (Q8_0, 130, 160), (Q4_0, 64, 8224),
                                   (Q5_K, 200, 4096), (Q5_K, 77, 14336), (Q8_0, 300, 14336)],
                         ids=["q8_0", "q4_0", "q8_0-K160", "q4_0-K8224", "q5_K", "q5_K-K14336", "q8_0-K14336"])
@pytest.mark.parametrize("n", [17, 129, 300])
def test_prefill_gemm_tiles(gpu, t, M, K, n):
    """The tiled prefill GEMMs (q8_0 / q4_0: int8 MFMA per 32-element block,
    gemm_q8.hip; q5_K: the f16-MFMA k-quant GEMM) over row and token tails, K
    not a multiple of the 128-element stage, and K chunks up to 14336."""
    w = synth.random_blocks(t, 990 + K + M, M, K)
    x = synth.normal(991 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    rows = np.arange(M) if M <= 130 else np.unique(synth.integers(992, 0, M - 1, 96))
    close(y[:, rows], oracle().mul_mat(t, w[rows], len(rows), K, x, nthreads=16), f"{NAMES[t]} {M}x{K} n={n}")


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q8_0, Q4_0], ids=["q4_K", "q5_K", "q8_0", "q4_0"])
@pytest.mark.parametrize("M,K,n", [(1024, 4096, 40), (512, 14336, 200), (96, 2560, 33)])
def test_prefill_gemm_k_chunks(gpu, t, M, K, n):
    """Few output tiles: the tiled GEMM splits K into chunks whose partial sums are
    added in chunk order by a second launch (shares of whole stages, trailing
    chunks possibly empty)."""
    w = synth.random_blocks(t, 1200 + K + M, M, K)
    x = synth.normal(1201 + n, (n, K))
    y = host(N.mul_mat(t, dev(w), M, K, dev(x)))
    rows = np.unique(synth.integers(1202, 0, M - 1, 64))
    close(y[:, rows], oracle().mul_mat(t, w[rows], len(rows), K, x, nthreads=16), f"{NAMES[t]} {M}x{K} n={n}")

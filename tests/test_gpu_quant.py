"""GPU parity: activation quantizers and weight dequantizers, bit-exact against the
oracle and the golden vectors of the reference's compiled ggml (through the C ABI)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, oracle
from tensorlisp_amd import native as N
from tensorlisp_amd import synth

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("wt", [Q4_0, Q4_K], ids=["q8_0", "q8_K"])
def test_quantize_act_golden(gpu, wt):
    g = np.load(GOLD / "act.npz")
    got = host(N.quantize_act(wt, dev(g["x"])))
    assert np.array_equal(got, g["q8_0" if wt == Q4_0 else "q8_K"])


@pytest.mark.parametrize("wt", [Q4_0, Q4_K], ids=["q8_0", "q8_K"])
@pytest.mark.parametrize("scale", [1.0, 1e-3, 3e4])
def test_quantize_act_random_vs_oracle(gpu, wt, scale):
    x = synth.normal(500 + int(scale), (37, 4096), scale)
    x[5, 256:768] = 0.0
    x[6, :] = 0.0
    got = host(N.quantize_act(wt, dev(x)))
    assert np.array_equal(got, oracle().quantize_act(wt, x))


def test_quantize_act_strided_rows(gpu):
    import torch

    x = synth.normal(510, (9, 1280))
    xt = dev(x)[:, :1024]  # row stride 1280 floats
    assert xt.stride(0) == 1280
    for wt in (Q4_0, Q4_K):
        got = host(N.quantize_act(wt, xt))
        assert np.array_equal(got, oracle().quantize_act(wt, x[:, :1024]))
    torch.cuda.synchronize()


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K], ids=[NAMES[t] for t in (Q4_0, Q8_0, Q4_K)])
def test_dequantize_golden(gpu, t):
    g = np.load(GOLD / "quant.npz")
    q = g[f"{NAMES[t]}_bytes"]
    got = host(N.dequantize(t, dev(q), g["w"].shape[1]))
    assert np.array_equal(got.view(np.uint32), g[f"{NAMES[t]}_deq"].view(np.uint32))


@pytest.mark.parametrize("t", [Q6_K, Q5_K], ids=["q6_K", "q5_K"])
def test_dequantize_kquant_golden(gpu, t):
    """dequantize_row_q6_K / _q5_K of the compiled reference (q6_K.npz, q5_K.npz), bit-exact."""
    g = np.load(GOLD / f"{NAMES[t]}.npz")
    for key, deq, k in (("w", "deq", 256), ("rand_w", "rand_deq", 1024)):
        got = host(N.dequantize(t, dev(g[key]), k))
        assert np.array_equal(got.view(np.uint32), g[deq].view(np.uint32)), key


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q5_K, Q6_K], ids=[NAMES[t] for t in (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K)])
def test_dequantize_random_blocks(gpu, t):
    """Every code and scale pattern (random bytes, subnormal f16 scales) bit-exact."""
    M, K = 257, 2048
    w = synth.random_blocks(t, 520, M, K)
    got = host(N.dequantize(t, dev(w), K))
    want = oracle().dequantize(t, w, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))

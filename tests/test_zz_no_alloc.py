"""tlh_mul_mat_noalloc: tlh_mul_mat with its scratch in the library's static
device array (include/tlhip.h). It runs the same kernels as tlh_mul_mat, so
its outputs must equal tlh_mul_mat's bit for bit. Each case makes two calls in
a row through the C ABI, the second on a smaller input, so the second call
reads a scratch that still holds the first call's (larger) contents; a node
beyond the static size is refused before anything is launched."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tensorlisp_amd import native as N
from tensorlisp_amd import synth

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 64 << 20


def _noalloc(op, w, x, y, stream):
    return N.lib().tlh_mul_mat_noalloc(C.byref(op), N._ptr(w), N._ptr(x), N._ptr(y), N._stream(stream))


def _pair(torch, t, M, K, n, seed):
    w = torch.from_numpy(synth.random_blocks(t, seed, M, K)).cuda()
    x = torch.from_numpy(synth.normal(seed + 1, (n, K))).cuda()
    want = torch.empty((n, M), dtype=torch.float32, device="cuda")
    N.MulMat(t, M, K, n)(w, x, want)
    got = torch.full((n, M), float("nan"), dtype=torch.float32, device="cuda")
    return w, x, want, got


# (type, first call M, K, N), (second call M, K, N): the second is smaller. The
# calls cover the fused register GEMV (N <= 2, no scratch read), the int8-MFMA
# few-column kernel with and without K-chunk partials (N 3..16), and the tiled
# GEMM with and without its K split (N > 16).
CASES = [
    ((N.Q4_K, 4096, 4096, 8), (N.Q4_K, 1000, 2048, 3)),
    ((N.Q4_K, 2048, 14336, 16), (N.Q4_K, 512, 4096, 1)),
    ((N.Q8_0, 1024, 4096, 64), (N.Q8_0, 300, 1024, 20)),
    ((N.Q4_0, 4096, 4096, 40), (N.Q4_0, 128, 512, 2)),
    ((N.Q6_K, 4096, 4096, 24), (N.Q6_K, 256, 2048, 5)),
    ((N.Q5_K, 14336, 4096, 512), (N.Q5_K, 256, 4096, 33)),
]


@pytest.mark.parametrize("first,second", CASES, ids=[f"{N.TYPE_NAMES[a[0]]}-{a[3]}-then-{b[3]}" for a, b in CASES])
def test_noalloc_matches_mul_mat_on_two_calls(gpu, first, second):
    import torch

    stream = torch.cuda.current_stream()
    for i, (t, M, K, n) in enumerate((first, second)):
        op = N.mul_mat_op(t, M, K, n)
        assert N.mul_mat_scratch_bytes(op) <= NOALLOC_BYTES
        w, x, want, got = _pair(torch, t, M, K, n, 4100 + 10 * i + n)
        N.check(_noalloc(op, w, x, got, stream))
        torch.cuda.synchronize()
        a, b = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(a.view(np.int32), b.view(np.int32)), (i, np.nanmax(np.abs(a - b)))


def test_noalloc_refuses_beyond_static_scratch(gpu):
    """A prefill node whose scratch exceeds the static array is TLH_INVALID, and its
    destination is untouched (nothing launched)."""
    import torch

    t, M, K, n = N.Q4_K, 256, 14336, 2048
    op = N.mul_mat_op(t, M, K, n)
    assert N.mul_mat_scratch_bytes(op) > NOALLOC_BYTES
    w = torch.zeros((M, N.row_bytes(t, K)), dtype=torch.uint8, device="cuda")
    x = torch.zeros((n, K), dtype=torch.float32, device="cuda")
    y = torch.full((n, M), 7.0, dtype=torch.float32, device="cuda")
    st = _noalloc(op, w, x, y, torch.cuda.current_stream())
    assert N.STATUS[st] == "INVALID", N.lib().tlh_last_error()
    assert b"static" in N.lib().tlh_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())

"""tlh_memset: a stream-ordered byte fill (the CUDA backend's Backend::zero,
crates/kernels/src/cuda/backend.rs:334-343, with any byte value). Every start
alignment and length around the 16-byte stores fills exactly the asked bytes;
the bytes around them keep their values."""
from __future__ import annotations

import numpy as np
import pytest

from tensorlisp_amd import native as N

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("offset", [0, 1, 3, 8, 15, 16, 17])
@pytest.mark.parametrize("n", [0, 1, 5, 15, 16, 17, 31, 33, 100, 4099, (1 << 20) + 7])
def test_fill_exact_bytes(gpu, offset, n):
    import torch

    size = n + offset + 40
    host = np.random.default_rng(offset * 1000 + n).integers(0, 256, size, dtype=np.uint8)
    t = torch.from_numpy(host.copy()).cuda()
    value = 0xA5 + 0x100 * (n % 3)  # only the low 8 bits count
    N.memset(t, value, n, offset)
    got = t.cpu().numpy()
    want = host.copy()
    want[offset:offset + n] = value & 0xFF
    np.testing.assert_array_equal(got, want)


def test_fill_is_stream_ordered(gpu):
    """A fill on a side stream lands after the work queued before it there and
    before the work queued after it."""
    import torch

    s = torch.cuda.Stream()
    t = torch.zeros(1 << 22, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        t.fill_(7)
        N.memset(t, 0, stream=s)
        t[::3] += 1
    s.synchronize()
    got = t.cpu().numpy()
    assert (got[::3] == 1).all() and got.sum() == got[::3].size

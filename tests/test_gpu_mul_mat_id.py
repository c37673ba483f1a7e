"""GGML_OP_MUL_MAT_ID through the executor (tlh_mul_mat_id): every case of
refs.MMID_CASES against the CPU backend's outputs (mul_mat_id.npz), within the
MUL_MAT bar |got - want| <= 1e-4 + 1e-3 |want|; an expert id out of range
gives NaN in its column only."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import MMID_CASES, mmid_case
from tensorlisp_amd import graph as G

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run(b, y, w, inputs):
    import torch

    prog = G.Program(b, [y], [dev(x) for x in w])
    for i, a in enumerate(inputs):
        prog.write_input(i, dev(a))
    prog.run()
    out = prog.read(y, torch.float32).cpu().numpy()
    torch.cuda.synchronize()
    return out.reshape(y.ne[2], y.ne[1], y.ne[0])


@pytest.mark.parametrize("case", MMID_CASES, ids=[c[0] for c in MMID_CASES])
def test_mul_mat_id_matches_reference_golden(gpu, case):
    print(f"[mul_mat_id] {case}", flush=True)
    b, y, w, inputs = mmid_case(case)
    got = run(b, y, w, inputs)
    want = np.load(GOLD / "mul_mat_id.npz")[case[0]][0]
    err = np.abs(got - want)
    bad = err > 1e-4 + 1e-3 * np.abs(want)
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tol, max err {err.max():.3e}"


def test_mul_mat_id_out_of_range_expert_is_nan(gpu):
    case = MMID_CASES[0]
    b, y, w, (x, ids) = mmid_case(case)
    ids = ids.copy()
    n_as = case[4]
    ids[1, 0] = n_as
    ids[2, 1] = -1
    got = run(b, y, w, [x, ids])
    want = np.load(GOLD / "mul_mat_id.npz")[case[0]][0]
    assert np.isnan(got[1, 0]).all() and np.isnan(got[2, 1]).all()
    keep = np.ones(got.shape[:2], bool)
    keep[1, 0] = keep[2, 1] = False
    assert np.allclose(got[keep], want[keep], rtol=1e-3, atol=1e-4)

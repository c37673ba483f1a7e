"""GPU parity: dense GGML_OP_FLASH_ATTN_EXT through the C ABI (tlh_flash_attn_ext).

Pins, on the same seeded inputs:
  * the reference's own outputs on the shapes of its attention tests
    (tests/golden/flash_attn_ext.npz, crates/tensorlisp/tests/native.rs:156-345),
    with the reference's tolerance for flash attention against its CPU backend:
    max |got - want| <= 8e-3 * max |want| (native.rs:51-57, :183);
  * the oracle (the CPU backend's algorithm, f16 P.V accumulator) on every query,
    same tolerance, or, where the CPU backend's own f16 accumulator drifts further
    from the truth (hundreds of keys), that drift plus the GPU's error;
  * a float64 brute force over exactly the f16 inputs: 2e-3 * max |truth|. The GPU
    keeps scores, softmax and P.V in f32 with probabilities rounded to f16 for the
    MFMA, so it sits closer to the truth than the CPU backend does.
Cases cover every head size the kernels take, GQA ratios 1..64, key counts around
the 16-key tiles and the split partitions, masks that empty whole rows, tiles and
partitions, soft cap, ALiBi, strided views of a KV cache, and the refusals.
"""
from __future__ import annotations

import numpy as np
import pytest

from refs import FA_CASES, fa_case_inputs, fa_mask, flash_attn_f64, oracle
from tensorlisp_amd import native as N
from tensorlisp_amd import synth

pytestmark = pytest.mark.gpu
TOL_CPU = 8e-3
TOL_F64 = 2e-3


def gold(name):
    from pathlib import Path

    return np.load(Path(__file__).resolve().parent / "golden" / f"{name}.npz")


def to_dev(a):
    """numpy (f32, or uint16 f16 bits) -> torch cuda tensor with the same strides."""
    import torch

    if a.dtype == np.uint16:
        t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.float16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t


def run_gpu(q, k, v, m, scale, max_bias=0.0, softcap=0.0):
    import torch

    out = N.flash_attn_ext(to_dev(q), to_dev(k), to_dev(v), None if m is None else to_dev(m), scale, max_bias,
                           softcap)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(got, q, k, v, m, scale, max_bias=0.0, softcap=0.0, what=""):
    truth = flash_attn_f64(q, k, v, m, scale, max_bias, softcap)
    want = oracle().flash_attn_ext(q, k, v, m, scale, max_bias, softcap)
    assert np.all(np.isfinite(got)), what
    s_t, s_w = np.abs(truth).max(), np.abs(want).max()
    e_t, e_w = np.abs(got - truth).max(), np.abs(got - want).max()
    e_ot = np.abs(want - truth).max()  # the CPU algorithm's own f16-accumulator error
    print(f"{what}: |gpu - f64| {e_t:.2e} (scale {s_t:.2e}), |gpu - oracle| {e_w:.2e}, "
          f"|oracle - f64| {e_ot:.2e}", flush=True)
    assert e_t <= TOL_F64 * s_t + 1e-6, what
    # the reference's tolerance, or (long key ranges, where the CPU backend's f16
    # accumulator drifts past it) the oracle's own distance from the truth plus ours
    assert e_w <= max(TOL_CPU * s_w, e_ot + e_t) + 1e-6, what


@pytest.mark.parametrize("case", FA_CASES, ids=[c[0] for c in FA_CASES])
def test_reference_test_shapes_vs_golden_oracle_and_f64(gpu, case):
    g = gold("flash_attn_ext")
    q, k, v, m, scale, max_bias, softcap = fa_case_inputs(case, int(g[f"{case[0]}/seed"][0]))
    got = run_gpu(q, k, v, m, scale, max_bias, softcap)
    want = g[f"{case[0]}/out"]
    rows = got[:, g[f"{case[0]}/rows"]]
    assert np.abs(rows - want).max() <= TOL_CPU * np.abs(want).max() + 1e-6
    check(got, q, k, v, m, scale, max_bias, softcap, case[0])


HEAD_SIZES = [(32, 32), (40, 40), (64, 64), (72, 72), (80, 80), (96, 96), (112, 112), (128, 128), (192, 192),
              (192, 128), (256, 256)]


@pytest.mark.parametrize("nq", [1, 6])
@pytest.mark.parametrize("D,DV", HEAD_SIZES)
def test_head_sizes(gpu, D, DV, nq):
    case = ("hs", 2, 8, 2, nq, 150, D, DV, "holes", 0.0, 0.0)
    q, k, v, m, scale, mb, sc = fa_case_inputs(case, 10 * D + DV + nq)
    check(run_gpu(q, k, v, m, scale), q, k, v, m, scale, what=f"D={D} DV={DV} nq={nq}")
    check(run_gpu(q, k, v, None, scale), q, k, v, None, scale, what=f"D={D} DV={DV} nq={nq} nomask")


@pytest.mark.parametrize("nh,nhkv", [(4, 4), (4, 2), (6, 2), (8, 1), (16, 1), (32, 8), (32, 1), (48, 1), (64, 2)])
@pytest.mark.parametrize("nq", [1, 3, 20])
def test_gqa_groups(gpu, nh, nhkv, nq):
    """Tiles hold up to 16 rows: gc heads of a group x qr queries; groups above 16
    heads split into head chunks (48 = 3 x 16, 64 / 2 = 2 x 16)."""
    case = ("gqa", 1, nh, nhkv, nq, 97, 64, 64, "holes", 0.0, 0.0)
    q, k, v, m, scale, _, _ = fa_case_inputs(case, nh * 100 + nhkv + nq)
    check(run_gpu(q, k, v, m, scale), q, k, v, m, scale, what=f"nh={nh} nhkv={nhkv} nq={nq}")


@pytest.mark.parametrize("L", [0, 1, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 257, 511, 1000, 4097])
@pytest.mark.parametrize("nq,nb", [(1, 1), (3, 2)])
def test_key_counts(gpu, L, nq, nb):
    """Around the 16-key tiles, the 4-wave groups and the partition sizes; L = 0 gives
    zeros (the CPU backend's S = 0 case)."""
    case = ("keys", nb, 8, 2, nq, L, 128, 128, "none", 0.0, 0.0)
    q, k, v, _, scale, _, _ = fa_case_inputs(case, 31 + L)
    got = run_gpu(q, k, v, None, scale)
    if L == 0:
        assert np.all(got == 0)
        return
    check(got, q, k, v, None, scale, what=f"L={L} nq={nq} nb={nb}")


def test_masked_rows_tiles_and_partitions(gpu):
    """A row with every key masked gives 0; whole 16-key tiles, 4-wave groups and
    split partitions that are fully masked contribute nothing; the live keys sit in
    the last partition only for one row."""
    nb, nh, nhkv, nq, L, D = 1, 4, 1, 4, 3000, 64
    q = synth.normal(61, (nb, nh, nq, D))
    k = synth.f16_bits(synth.normal(62, (nb, nhkv, L, D)))
    v = synth.f16_bits(synth.normal(63, (nb, nhkv, L, D)))
    mf = np.zeros((nb, 1, nq, L), np.float32)
    mf[0, 0, 0, :] = -np.inf  # row 0: nothing
    mf[0, 0, 1, :L - 5] = -np.inf  # row 1: the last 5 keys
    mf[0, 0, 2, 16:2800] = -np.inf  # row 2: a hole of whole tiles and partitions
    mf[0, 0, 3, ::2] = -np.inf  # row 3: every other key
    m = mf.astype(np.float16).view(np.uint16)
    got = run_gpu(q, k, v, m, 0.125)
    assert np.all(got[:, 0] == 0)
    check(got, q, k, v, m, 0.125, what="masked rows")
    # decode shape (one query: the split path) with only the last keys live
    m1 = np.ascontiguousarray(m[:, :, 1:2])
    q1 = np.ascontiguousarray(q[:, :, 1:2])
    check(run_gpu(q1, k, v, m1, 0.125), q1, k, v, m1, 0.125, what="decode, last keys only")


def test_nan_keys_behind_the_mask_are_skipped(gpu):
    """The CPU backend skips keys whose mask is -inf before reading them
    (ops.cpp:8603-8606): NaN keys there must not reach the scores."""
    nb, nh, nhkv, nq, L, D = 1, 4, 2, 2, 80, 64
    q = synth.normal(71, (nb, nh, nq, D))
    kf = synth.normal(72, (nb, nhkv, L, D))
    kf[:, :, 40:50] = np.nan
    k = synth.f16_bits(kf)
    v = synth.f16_bits(synth.normal(73, (nb, nhkv, L, D)))
    mf = np.zeros((nb, 1, nq, L), np.float32)
    mf[..., 40:50] = -np.inf
    m = mf.astype(np.float16).view(np.uint16)
    got = run_gpu(q, k, v, m, 0.125)
    assert np.all(np.isfinite(got))
    want = oracle().flash_attn_ext(q, k, v, m, 0.125)
    assert np.abs(got - want).max() <= TOL_CPU * np.abs(want).max()


@pytest.mark.parametrize("softcap,max_bias", [(50.0, 0.0), (2.0, 0.0), (0.0, 8.0), (10.0, 4.0)])
def test_softcap_and_alibi(gpu, softcap, max_bias):
    case = ("cap", 2, 12, 4, 3, 200, 128, 128, "bias", max_bias, softcap)
    q, k, v, m, scale, mb, sc = fa_case_inputs(case, 81)
    check(run_gpu(q, k, v, m, scale, mb, sc), q, k, v, m, scale, mb, sc, what=f"softcap={sc} max_bias={mb}")


def test_strided_views_of_a_kv_cache(gpu):
    """K/V as views into a larger cache [nb][L_max][nhkv][D] (rows of nhkv*D halves,
    heads D apart), q as the split-heads permutation of [nb][nq][nh][D], and a
    per-head mask broadcast over the batch."""
    import torch

    nb, nh, nhkv, nq, L, Lmax, D = 2, 8, 2, 5, 300, 512, 128
    cache_k = synth.f16_bits(synth.normal(91, (nb, Lmax, nhkv, D)))
    cache_v = synth.f16_bits(synth.normal(92, (nb, Lmax, nhkv, D)))
    qbuf = synth.normal(93, (nb, nq, nh, D))
    mf = np.where(synth.normal(94, (1, nh, nq, L)) > 1.0, -np.inf, 0.0).astype(np.float16)
    m = mf.view(np.uint16)
    k = cache_k[:, :L].transpose(0, 2, 1, 3)  # (nb, nhkv, L, D), row stride nhkv*D
    v = cache_v[:, :L].transpose(0, 2, 1, 3)
    q = qbuf.transpose(0, 2, 1, 3)  # (nb, nh, nq, D), ggml nb1 = nh*D*4
    dk = to_dev(cache_k)[:, :L].permute(0, 2, 1, 3)
    dv = to_dev(cache_v)[:, :L].permute(0, 2, 1, 3)
    dq = to_dev(qbuf).permute(0, 2, 1, 3)
    out = N.flash_attn_ext(dq, dk, dv, to_dev(m), 1.0 / np.sqrt(D))
    torch.cuda.synchronize()
    check(out.cpu().numpy(), q, k, v, m, 1.0 / np.sqrt(D), what="strided views")


def test_decode_batch_bench_shape(gpu):
    """The measured workload (32 sequences x 32 heads / 8 kv heads x 128, 4096 keys,
    no mask): every output against the oracle's algorithm on a sample of sequences
    and the float64 truth on them."""
    import torch

    nb, nh, nhkv, L, D = 32, 32, 8, 4096, 128
    q = synth.normal(3, (nb, nh, 1, D))
    k = synth.f16_bits(synth.normal(4, (nb, nhkv, L, D)))
    v = synth.f16_bits(synth.normal(5, (nb, nhkv, L, D)))
    got = run_gpu(q, k, v, None, 1.0 / np.sqrt(D))
    assert np.all(np.isfinite(got))
    for b in (0, 17, 31):
        sl = slice(b, b + 1)
        check(got[sl], q[sl], k[sl], v[sl], None, 1.0 / np.sqrt(D), what=f"bench shape, sequence {b}")
    del torch


def test_refusals(gpu):
    import torch

    q = torch.zeros((1, 4, 1, 64), device="cuda")
    k = torch.zeros((1, 2, 10, 64), device="cuda", dtype=torch.float16)
    with pytest.raises(N.TlhError, match="UNSUPPORTED.*K/V of type f32"):
        N.flash_attn_ext(q, k.float(), k, None, 1.0)
    q48 = torch.zeros((1, 4, 1, 48), device="cuda")
    k48 = torch.zeros((1, 2, 10, 48), device="cuda", dtype=torch.float16)
    with pytest.raises(N.TlhError, match="UNSUPPORTED.*head sizes"):
        N.flash_attn_ext(q48, k48, k48, None, 1.0)
    big = torch.zeros((1, 10, 2, 68), device="cuda", dtype=torch.float16)[..., :64].permute(0, 2, 1, 3)
    with pytest.raises(N.TlhError, match="UNSUPPORTED.*16 bytes"):
        N.flash_attn_ext(q, big, k, None, 1.0)
    with pytest.raises(N.TlhError, match="INVALID.*max_bias needs a mask"):
        N.flash_attn_ext(q, k, k, None, 1.0, max_bias=8.0)
    k3 = torch.zeros((1, 3, 10, 64), device="cuda", dtype=torch.float16)
    with pytest.raises(N.TlhError, match="UNSUPPORTED.*inconsistent"):
        N.flash_attn_ext(q, k3, k3, None, 1.0)


def test_window_and_causal_masks_clip_key_ranges(gpu):
    """Per-head sliding windows and causal masks: each row's live keys are a window
    that starts past 0 and ends before L, different across the rows of a tile and
    across heads (mask per head, mne2 = nh), so the kernels' key loops are clipped
    to per-tile ranges that do not line up with 16-key tiles or partitions."""
    nb, nh, nhkv, nq, L, D = 2, 8, 2, 100, 700, 64
    q = synth.normal(101, (nb, nh, nq, D))
    k = synth.f16_bits(synth.normal(102, (nb, nhkv, L, D)))
    v = synth.f16_bits(synth.normal(103, (nb, nhkv, L, D)))
    pos = np.arange(nq)[:, None] + (L - nq)  # query i sits at position L - nq + i
    j = np.arange(L)[None, :]
    mf = np.full((nb, nh, nq, L), -np.inf, np.float32)
    for h in range(nh):
        w = 13 + 29 * h  # window per head
        mf[:, h] = np.where((j <= pos) & (j > pos - w), 0.0, -np.inf)
    mf[1, :, :, :350] = -np.inf  # batch 1: also a padding prefix
    m = mf.astype(np.float16).view(np.uint16)
    check(run_gpu(q, k, v, m, 0.125), q, k, v, m, 0.125, what="windows")
    # causal decode-style rows: one query per batch at the last position, split path
    q1 = np.ascontiguousarray(q[:, :, -1:])
    m1 = np.ascontiguousarray(m[:, :, -1:])
    check(run_gpu(q1, k, v, m1, 0.125), q1, k, v, m1, 0.125, what="windows, one query")


def _causal(nb, nh, nq, L, per_head=False, window=0, pad=0):
    """f16 bits of a causal mask (query i at position L - nq + i), optionally a
    window of `window` keys and a padding prefix of `pad` keys in batch 1."""
    pos = np.arange(nq)[:, None] + (L - nq)
    j = np.arange(L)[None, :]
    live = j <= pos
    if window:
        live &= j > pos - window
    mf = np.where(live, 0.0, -np.inf).astype(np.float32)
    mf = np.broadcast_to(mf, (nb, nh if per_head else 1, nq, L)).copy()
    if pad:
        mf[min(1, nb - 1), :, :, :pad] = -np.inf
    return mf.astype(np.float16).view(np.uint16)


# (nb, nh, nhkv, nq, L, mask kind, softcap, max_bias): head size 128, at least
# 128 workgroups of 64 rows and (with a mask) L a multiple of 8, so these run
# the prefill form (k_flash_attn_rows); GQA groups 4 (4 heads a workgroup), 8
# (two head groups), 1 and 3 (one head, 64 queries), 2 (two heads, 32
# queries), partial query blocks and key tiles, causal / window / padding
# masks, none, soft cap and ALiBi. The last case (L = 700) takes the 16-row
# kernel: same checks.
ROWS_CASES = [
    (1, 32, 8, 512, 512, "causal", 0.0, 0.0),
    (1, 64, 8, 256, 250, "none", 0.0, 0.0),
    (4, 8, 8, 300, 704, "window", 0.0, 0.0),
    (2, 24, 8, 130, 400, "pad", 30.0, 4.0),
    (8, 16, 8, 40, 1000, "causal", 0.0, 0.0),
    (4, 8, 8, 300, 700, "window", 0.0, 0.0),
]


@pytest.mark.parametrize("case", ROWS_CASES, ids=[f"{c[0]}x{c[1]}/{c[2]}-q{c[3]}-L{c[4]}-{c[5]}" for c in ROWS_CASES])
def test_prefill_rows_form(gpu, case):
    nb, nh, nhkv, nq, L, kind, softcap, max_bias = case
    D = 128
    q = synth.normal(201, (nb, nh, nq, D))
    k = synth.f16_bits(synth.normal(202, (nb, nhkv, L, D)))
    v = synth.f16_bits(synth.normal(203, (nb, nhkv, L, D)))
    m = {"none": None, "causal": _causal(nb, 1, nq, L), "window": _causal(nb, nh, nq, L, True, 97),
         "pad": _causal(nb, 1, nq, L, pad=150)}[kind]
    scale = 1.0 / np.sqrt(D)
    print(f"[fa-rows] {case}", flush=True)
    check(run_gpu(q, k, v, m, scale, max_bias, softcap), q, k, v, m, scale, max_bias, softcap, what=str(case))

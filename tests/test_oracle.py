"""Pins the CPU oracle (oracle/tlq_oracle.c) before anything is checked against it.

Each oracle function is pinned by at least one check that a plausible mistake
(dropped term, wrong sign or index, swapped nibble halves, wrong rounding tie)
fails:
  * the golden vectors of tests/golden/ (outputs of the reference's own compiled
    ggml, written by make_golden.py) -- bit-exact;
  * the compiled reference itself on fresh random inputs, where oracle/_ref is
    built (this container) -- bit-exact;
  * mathematics: numpy's IEEE float16 conversion, float64 brute-force sums of the
    dequantized operands, quantizer invariants, softmax brute force.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

from refs import (BF16, F16, F32, NAMES, Q2_K, Q3_K, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, Q8_1, Q8_K,
                  fp16_probe_values,
                  oracle, ref, row_bytes)
from tensorlisp_amd import synth

GOLD = Path(__file__).resolve().parent / "golden"
WTYPES = (Q4_0, Q8_0, Q4_K)


def gold(name):
    return np.load(GOLD / f"{name}.npz")


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


# ------------------------------------------------------------------- fp16
def test_fp16_to_fp32_all_halves_golden_and_numpy():
    o = oracle()
    halves = np.arange(65536, dtype=np.uint16)
    got = o.f16_to_f32(halves)
    want = gold("fp16")["h2f_bits"].view(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert same_bits(got[~nan], want[~nan])
    # independent: numpy's IEEE binary16 decoder
    assert same_bits(got[~nan], halves.view(np.float16).astype(np.float32)[~nan])


def test_fp32_to_fp16_rounding_boundaries():
    o = oracle()
    f = fp16_probe_values()
    got = o.f32_to_f16(f)
    assert np.array_equal(got, gold("fp16")["f2h"])
    with np.errstate(over="ignore"):
        assert np.array_equal(got, f.astype(np.float16).view(np.uint16))  # IEEE round-to-nearest-even
    nan = np.array([np.nan, -np.nan], np.float32)
    assert np.array_equal(o.f32_to_f16(nan) & 0x7FFF, np.array([0x7E00, 0x7E00], np.uint16))


# ------------------------------------------------------ weight quantization
@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
def test_weight_quantize_and_dequantize_golden(t):
    o, g = oracle(), gold("quant")
    q = o.quantize(t, g["w"])
    assert np.array_equal(q, g[f"{NAMES[t]}_bytes"])
    assert same_bits(o.dequantize(t, q, g["w"].shape[1]), g[f"{NAMES[t]}_deq"])


@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
def test_weight_quantize_error_bounds(t):
    """Round-to-nearest quantization: each dequantized value lies within its block's
    step of the input (q8_0/q4_0: |d|/2 plus the f16 rounding of d; q4_K: the stored
    sub-block scale)."""
    o = oracle()
    w = synth.normal(21, (16, 512), 0.02)
    deq = o.dequantize(t, o.quantize(t, w), 512)
    err = np.abs(deq - w)
    amax = np.abs(w).reshape(16, -1, 32).max(-1, keepdims=True)
    eb = err.reshape(16, -1, 32)
    if t == Q8_0:
        assert np.all(eb <= amax / 127 * (0.5 + 127 * 2.0 ** -11))  # d/2 plus the f16 rounding of d
    elif t == Q4_0:
        # d = max/-8: codes span [-8, 7], so the opposite-sign extreme clamps at 7 (error <= |d|)
        assert np.all(eb <= amax / 8 * 1.001)
        assert np.mean(eb <= amax / 16 * 1.001) > 0.9
    else:
        assert err.max() < 0.25 * np.abs(w).max()
    # dequantized values are exactly code * scale: q8_0 codes recovered as integers
    if t == Q8_0:
        q = o.quantize(t, w).reshape(-1, 34)
        d = q[:, :2].copy().view(np.float16).astype(np.float32)
        codes = q[:, 2:].view(np.int8).astype(np.float32)
        assert same_bits((codes * d).reshape(deq.shape), deq)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
@pytest.mark.parametrize("scale", [0.02, 1.0, 300.0])
def test_weight_quantize_matches_reference_random(t, scale):
    o, r = oracle(), ref()
    w = synth.normal(31 + int(scale), (64, 1024), scale)
    q = o.quantize(t, w)
    assert np.array_equal(q, r.quantize_weights(t, w))
    assert same_bits(o.dequantize(t, q, 1024), r.dequantize(t, q, 1024))


# ------------------------------------------------- activation quantization
def test_act_quantize_golden():
    o, g = oracle(), gold("act")
    assert np.array_equal(o.quantize(Q8_0, g["x"]), g["q8_0"])
    assert np.array_equal(o.quantize(Q8_K, g["x"]), g["q8_K"])


def _q8_0_fields(q, k):
    b = q.reshape(-1, 34)
    return b[:, :2].copy().view(np.float16).astype(np.float32).ravel(), b[:, 2:].view(np.int8)


def _q8_K_fields(q):
    b = q.reshape(-1, 292)
    d = b[:, :4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].view(np.int8)
    bs = b[:, 260:].copy().view(np.int16)
    return d, qs, bs


def test_act_quantize_invariants():
    o = oracle()
    x = np.concatenate([gold("act")["x"], synth.normal(41, (8, 1024), 3.0)])
    d, qs = _q8_0_fields(o.quantize(Q8_0, x), 1024)
    xb = x.reshape(-1, 32)
    assert np.abs(qs.astype(int)).max() <= 127
    amax = np.abs(xb).max(1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    dd = (amax / np.float32(127)).astype(np.float32)
    nz = dd > 0
    assert np.all(np.abs(xb[nz] - qs[nz] * dd[nz, None]) <= dd[nz, None] * 0.5 * (1 + 1e-5))
    assert np.all(qs[~nz] == 0)
    d, qs, bs = _q8_K_fields(o.quantize(Q8_K, x))
    assert np.array_equal(bs, qs.reshape(-1, 16, 16).astype(np.int32).sum(-1).astype(np.int16))
    xk = x.reshape(-1, 256)
    nz = np.abs(xk).max(1) > 0
    assert np.all(d[~nz] == 0) and np.all(qs[~nz] == 0)
    assert np.all(np.abs(xk[nz] - qs[nz] * d[nz, None]) <= np.abs(d[nz, None]) * 0.5 * (1 + 1e-5))
    # the element of largest magnitude maps to -127 * sign-convention: d carries -max/127
    i = np.abs(xk[nz]).argmax(1)
    assert np.all(qs[nz][np.arange(nz.sum()), i] == -127)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
@pytest.mark.parametrize("wt", [Q4_0, Q4_K], ids=["q8_0", "q8_K"])
def test_act_quantize_matches_reference_random(wt):
    o, r = oracle(), ref()
    for seed, s in ((51, 1.0), (52, 1e-3), (53, 1e5)):
        x = synth.normal(seed, (32, 2048), s)
        x[3, 100:400] = 0.0
        assert np.array_equal(o.quantize_act(wt, x), r.quantize_act(wt, x))


# ----------------------------------------------------------- dot products
@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
def test_vec_dot_against_f64_bruteforce(t):
    """vec_dot = sum of the dequantized operands, to f32 accumulation error."""
    o = oracle()
    K = 4096
    w = o.quantize(t, synth.normal(61, (8, K), 0.02))
    x = synth.normal(62, (4, K))
    xq = o.quantize_act(t, x)
    at = Q8_K if t == Q4_K else Q8_0
    wd = o.dequantize(t, w, K).astype(np.float64)
    xd = o.dequantize(at, xq, K).astype(np.float64)
    want = wd @ xd.T
    got = np.array([[o.vec_dot(t, K, w[i], xq[j]) for j in range(4)] for i in range(8)])
    scale = np.abs(wd).sum(1)[:, None] * np.abs(xd).max()
    assert np.all(np.abs(got - want) <= 1e-6 * scale)


def test_q4_K_block_integer_sums():
    """The integer parts of a q4_K x q8_K block: sum_s sc*dot and sum_s m*sum(q8),
    against codes recovered independently from dequantized values."""
    o = oracle()
    w = o.quantize(Q4_K, synth.normal(71, (4, 256), 0.02))
    xq = o.quantize(Q8_K, synth.normal(72, (4, 256)))
    for i in range(4):
        sq, sm = o.block_ints_q4_K(w[i], xq[i])
        blk = w[i]
        d = blk[0:2].copy().view(np.float16).astype(np.float64)[0]
        dmin = blk[2:4].copy().view(np.float16).astype(np.float64)[0]
        y = o.dequantize(Q4_K, blk, 256).astype(np.float64)
        q8 = xq[i][4:260].view(np.int8).astype(np.int64)
        # y = d*sc*q - dmin*m  => sum(y*q8) = d*sq - dmin*sm (up to f32 rounding of y)
        lhs = (y * q8).sum()
        assert abs(lhs - (d * sq - dmin * sm)) <= 1e-5 * (abs(d * sq) + abs(dmin * sm) + 1)


# ---------------------------------------------------------------- mul_mat
@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
def test_mul_mat_golden_reference_cases(t):
    """The reference test's shapes (native.rs:73-107), CPU backend outputs, bit-exact."""
    o, g = oracle(), gold("mul_mat")
    for n in g["ns"]:
        y = o.mul_mat(t, g[f"{NAMES[t]}_w"], 96, 256, g[f"x{n}"])
        assert same_bits(y, g[f"{NAMES[t]}_y{n}"]), n


def test_mul_mat_config1_golden():
    """BASELINE config 1 through the oracle equals the CPU backend's output bit for bit;
    the input hashes pin the synthetic generator."""
    o, g = oracle(), gold("config1")
    w = synth.q8_0_config1(int(g["seeds"][0]), 4096, 4096)
    x = synth.normal(int(g["seeds"][1]), (1, 4096))
    assert hashlib.sha256(w.tobytes()).digest() == g["w_sha256"].tobytes()
    assert hashlib.sha256(x.tobytes()).digest() == g["x_sha256"].tobytes()
    assert same_bits(o.mul_mat(Q8_0, w, 4096, 4096, x), g["y"])
    # ~30% of the f16 scales are subnormal, as the config states
    d = w.reshape(-1, 34)[:, :2].copy().view(np.uint16)
    frac = np.mean((d & 0x7C00) == 0)
    assert 0.2 < frac < 0.4, frac


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
@pytest.mark.parametrize("t", WTYPES, ids=[NAMES[t] for t in WTYPES])
def test_mul_mat_matches_reference_random_blocks(t):
    o, r = oracle(), ref()
    M, K = 200, 1024
    w = synth.random_blocks(t, 81, M, K)
    for n in (1, 8, 17):
        x = synth.normal(82 + n, (n, K))
        y, _ = r.mul_mat(t, w, M, K, x)
        assert same_bits(o.mul_mat(t, w, M, K, x), y)


# ------------------------------------------------------------------ q6_K
# tlq_dequantize_row_q6_K (ggml-quants.c:1939-1968) and tlq_vec_dot_q6_K_q8_K
# (ggml-cpu/quants.c:851-904): pinned by the compiled reference's outputs
# (q6_K.npz, from ggml_quantize_chunk weights and random blocks), bit-exact;
# the live reference; and float64 brute force over the dequantized operands.
def test_q6_K_golden_dequantize_and_mul_mat():
    o, g = oracle(), gold("q6_K")
    assert same_bits(o.dequantize(Q6_K, g["w"], 256), g["deq"])
    assert same_bits(o.dequantize(Q6_K, g["rand_w"], 1024), g["rand_deq"])
    from refs import xorshift_noise

    for n in g["ns"]:
        y = o.mul_mat(Q6_K, g["w"], 96, 256, xorshift_noise((int(n), 256), 10 + int(n)))
        assert same_bits(y, g[f"y{n}"]), n
    assert same_bits(o.mul_mat(Q6_K, g["rand_w"], 40, 1024, synth.normal(62, (3, 1024))), g["rand_y"])


def test_q6_K_codes_against_an_independent_unpacking():
    """dequantize = d * scale * (code - 32) with code rebuilt here from ql / qh by
    a different route (numpy bit fields over the whole block at once)."""
    o = oracle()
    w = synth.random_blocks(Q6_K, 91, 6, 512).reshape(-1, 210)
    ql, qh = w[:, :128].astype(np.int64), w[:, 128:192].astype(np.int64)
    sc = w[:, 192:208].view(np.int8).astype(np.float64)
    d = w[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    codes = np.zeros((w.shape[0], 256), np.int64)
    for h in range(2):
        for q in range(4):
            lo = ql[:, 64 * h + 32 * (q & 1): 64 * h + 32 * (q & 1) + 32]
            nib = (lo >> 4) if q >= 2 else (lo & 15)
            hi = (qh[:, 32 * h: 32 * h + 32] >> (2 * q)) & 3
            codes[:, 128 * h + 32 * q: 128 * h + 32 * q + 32] = (nib | (hi << 4)) - 32
    want = d[:, None] * np.repeat(sc, 16, axis=1) * codes
    got = o.dequantize(Q6_K, w, 256).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-6, atol=0)


def test_q6_K_vec_dot_against_f64_bruteforce():
    o = oracle()
    K = 2048
    w = synth.random_blocks(Q6_K, 93, 8, K)
    x = synth.normal(94, (4, K))
    xq = o.quantize_act(Q6_K, x)
    wd = o.dequantize(Q6_K, w, K).astype(np.float64)
    xd = o.dequantize(Q8_K, xq, K).astype(np.float64)
    want = wd @ xd.T
    got = np.array([[o.vec_dot(Q6_K, K, w[i], xq[j]) for j in range(4)] for i in range(8)])
    scale = np.abs(wd).sum(1)[:, None] * np.abs(xd).max()
    assert np.all(np.abs(got - want) <= 1e-6 * scale)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
def test_q6_K_matches_reference_live():
    o, r = oracle(), ref()
    M, K = 120, 2048
    w = synth.random_blocks(Q6_K, 95, M, K)
    assert same_bits(o.dequantize(Q6_K, w, K), r.dequantize(Q6_K, w, K))
    wq = r.quantize_weights(Q6_K, synth.normal(96, (8, K), 0.02))
    for n in (1, 2, 9):
        x = synth.normal(97 + n, (n, K))
        y, _ = r.mul_mat(Q6_K, w, M, K, x)
        assert same_bits(o.mul_mat(Q6_K, w, M, K, x), y)
        y, _ = r.mul_mat(Q6_K, wq, 8, K, x)
        assert same_bits(o.mul_mat(Q6_K, wq, 8, K, x), y)


# ------------------------------------------------------------------ q5_K
# tlq_dequantize_row_q5_K (ggml-quants.c:1731-1756) and tlq_vec_dot_q5_K_q8_K
# (ggml-cpu/quants.c:771-850): pinned by the compiled reference's outputs
# (q5_K.npz), bit-exact; an independent numpy unpacking of the codes and the
# 6-bit scale/min field; float64 brute force; the live reference.
def test_q5_K_golden_dequantize_and_mul_mat():
    o, g = oracle(), gold("q5_K")
    assert same_bits(o.dequantize(Q5_K, g["w"], 256), g["deq"])
    assert same_bits(o.dequantize(Q5_K, g["rand_w"], 1024), g["rand_deq"])
    from refs import xorshift_noise

    for n in g["ns"]:
        y = o.mul_mat(Q5_K, g["w"], 96, 256, xorshift_noise((int(n), 256), 10 + int(n)))
        assert same_bits(y, g[f"y{n}"]), n
    assert same_bits(o.mul_mat(Q5_K, g["rand_w"], 40, 1024, synth.normal(72, (3, 1024))), g["rand_y"])


def test_q5_K_codes_against_an_independent_unpacking():
    """y = (d * sc) * code - dmin * m in f32, with code = nibble | fifth bit << 4 and
    the 6-bit sc / m rebuilt here over whole arrays (the block layout of
    ggml-common.h:345-352), bit-exact."""
    o = oracle()
    w = synth.random_blocks(Q5_K, 92, 6, 512).reshape(-1, 176)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = w[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = w[:, 4:16].astype(np.int64)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    qh, qs = w[:, 16:48].astype(np.int64), w[:, 48:176].astype(np.int64)
    codes = np.zeros((w.shape[0], 256), np.int64)
    for sb in range(8):
        byte = qs[:, 32 * (sb // 2): 32 * (sb // 2) + 32]
        nib = (byte >> 4) if sb & 1 else (byte & 15)
        codes[:, 32 * sb: 32 * sb + 32] = nib | (((qh >> sb) & 1) << 4)
    d1 = np.repeat(d[:, None] * sc.astype(np.float32), 32, axis=1)
    m1 = np.repeat(dmin[:, None] * mn.astype(np.float32), 32, axis=1)
    want = (d1 * codes.astype(np.float32) - m1).astype(np.float32)
    assert codes.max() == 31 and codes.min() == 0
    assert same_bits(o.dequantize(Q5_K, w, 256), want)


def test_q5_K_vec_dot_against_f64_bruteforce():
    o = oracle()
    K = 2048
    w = synth.random_blocks(Q5_K, 93, 8, K)
    x = synth.normal(94, (4, K))
    xq = o.quantize_act(Q5_K, x)
    wd = o.dequantize(Q5_K, w, K).astype(np.float64)
    xd = o.dequantize(Q8_K, xq, K).astype(np.float64)
    want = wd @ xd.T
    got = np.array([[o.vec_dot(Q5_K, K, w[i], xq[j]) for j in range(4)] for i in range(8)])
    scale = np.abs(wd).sum(1)[:, None] * np.abs(xd).max()
    assert np.all(np.abs(got - want) <= 1e-6 * scale)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
def test_q5_K_matches_reference_live():
    o, r = oracle(), ref()
    M, K = 120, 2048
    w = synth.random_blocks(Q5_K, 95, M, K)
    assert same_bits(o.dequantize(Q5_K, w, K), r.dequantize(Q5_K, w, K))
    wq = r.quantize_weights(Q5_K, synth.normal(96, (8, K), 0.02))
    for n in (1, 2, 9):
        x = synth.normal(97 + n, (n, K))
        y, _ = r.mul_mat(Q5_K, w, M, K, x)
        assert same_bits(o.mul_mat(Q5_K, w, M, K, x), y)
        y, _ = r.mul_mat(Q5_K, wq, 8, K, x)
        assert same_bits(o.mul_mat(Q5_K, wq, 8, K, x), y)


# ---------------------------------------------------------- q2_K / q3_K
# tlq_dequantize_row_q2_K / _q3_K (ggml-quants.c:961-989, :1305-1351) and the
# generic vec_dots (ggml-cpu/quants.c:565-615, :617-694): pinned by the
# compiled reference's outputs (q2_K.npz, q3_K.npz), bit-exact; an
# independent numpy unpacking of the codes, scales and mins over whole
# arrays; float64 brute force; the live reference.
LOWK = ((Q2_K, "q2_K", 82), (Q3_K, "q3_K", 92))


@pytest.mark.parametrize("t,name,xseed", LOWK, ids=[n for _, n, _ in LOWK])
def test_lowk_golden_dequantize_and_mul_mat(t, name, xseed):
    o, g = oracle(), gold(name)
    assert same_bits(o.dequantize(t, g["w"], 256), g["deq"])
    assert same_bits(o.dequantize(t, g["rand_w"], 1024), g["rand_deq"])
    from refs import xorshift_noise

    for n in g["ns"]:
        y = o.mul_mat(t, g["w"], 96, 256, xorshift_noise((int(n), 256), 10 + int(n)))
        assert same_bits(y, g[f"y{n}"]), n
    assert same_bits(o.mul_mat(t, g["rand_w"], 40, 1024, synth.normal(xseed, (3, 1024))), g["rand_y"])


def lowk_numpy_dequant(t, w):
    """Element values of q2_K / q3_K super-blocks [nb, bytes] by whole-array
    numpy, from the block layouts of ggml-common.h:298-323: element 32j + l of
    half h has its 2-bit code in qs[32h + l] at bit 2j; q2_K: (d * (sc & 15))
    * code - dmin * (sc >> 4) with sc the byte of its 16-element sub-block;
    q3_K: (d * (scale - 32)) * (code - 4 * (1 - bit)), bit = hmask[l] >> (4h
    + j), scale the 6-bit field (low 4 bits from bytes 0..7, high 2 bits from
    bytes 8..11)."""
    nb = w.shape[0]
    e = np.arange(256)
    h, j, l, s = e // 128, (e % 128) // 32, e % 32, e // 16
    if t == Q2_K:
        qs = w[:, 16:80].astype(np.int64)
        code = (qs[:, 32 * h + l] >> (2 * j)) & 3
        sc = w[:, s].astype(np.int64)
        d = w[:, 80:82].copy().view(np.float16).astype(np.float32)
        dmin = w[:, 82:84].copy().view(np.float16).astype(np.float32)
        dl = d * (sc & 15).astype(np.float32)
        ml = dmin * (sc >> 4).astype(np.float32)
        return (dl * code.astype(np.float32) - ml).astype(np.float32), code
    hm, qs = w[:, 0:32].astype(np.int64), w[:, 32:96].astype(np.int64)
    code = ((qs[:, 32 * h + l] >> (2 * j)) & 3) - 4 * (1 - ((hm[:, l] >> (4 * h + j)) & 1))
    b = w[:, 96:108].astype(np.int64)
    ss = np.arange(16)
    low = np.where(ss < 8, b[:, np.minimum(ss, 7)] & 15, b[:, np.maximum(ss - 8, 0)] >> 4)
    high = (b[:, 8 + ss % 4] >> (2 * (ss // 4))) & 3
    scale = (low | high << 4) - 32
    d = w[:, 108:110].copy().view(np.float16).astype(np.float32)
    dl = d * scale[:, s].astype(np.float32)
    return (dl * code.astype(np.float32)).astype(np.float32), code


@pytest.mark.parametrize("t,name,xseed", LOWK, ids=[n for _, n, _ in LOWK])
def test_lowk_codes_against_an_independent_unpacking(t, name, xseed):
    o = oracle()
    w = synth.random_blocks(t, 190 + t, 6, 512)
    bb = 84 if t == Q2_K else 110
    want, code = lowk_numpy_dequant(t, w.reshape(-1, bb))
    assert (code.min(), code.max()) == ((0, 3) if t == Q2_K else (-4, 3))
    assert same_bits(o.dequantize(t, w, 512), want.reshape(6, 512))
    # and on ggml-quantized weights (scales and mins the quantizer chose)
    g = gold(name)
    want, _ = lowk_numpy_dequant(t, g["w"].reshape(-1, bb))
    assert same_bits(g["deq"], want.reshape(g["deq"].shape))


@pytest.mark.parametrize("t,name,xseed", LOWK, ids=[n for _, n, _ in LOWK])
def test_lowk_vec_dot_against_f64_bruteforce(t, name, xseed):
    o = oracle()
    K = 2048
    w = synth.random_blocks(t, 193 + t, 8, K)
    x = synth.normal(194, (4, K))
    xq = o.quantize_act(t, x)
    wd = o.dequantize(t, w, K).astype(np.float64)
    xd = o.dequantize(Q8_K, xq, K).astype(np.float64)
    want = wd @ xd.T
    got = np.array([[o.vec_dot(t, K, w[i], xq[j]) for j in range(4)] for i in range(8)])
    scale = np.abs(wd).sum(1)[:, None] * np.abs(xd).max()
    assert np.all(np.abs(got - want) <= 1e-6 * scale)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
@pytest.mark.parametrize("t,name,xseed", LOWK, ids=[n for _, n, _ in LOWK])
def test_lowk_matches_reference_live(t, name, xseed):
    o, r = oracle(), ref()
    M, K = 120, 2048
    w = synth.random_blocks(t, 195 + t, M, K)
    assert same_bits(o.dequantize(t, w, K), r.dequantize(t, w, K))
    wq = r.quantize_weights(t, synth.normal(196, (8, K), 0.02))
    assert same_bits(o.dequantize(t, wq, K), r.dequantize(t, wq, K))
    xq = r.quantize_act(t, synth.normal(197, (2, K)))
    for m in range(8):
        for n in range(2):
            assert np.float32(o.vec_dot(t, K, wq[m], xq[n])) == np.float32(r.vec_dot(t, K, wq[m], xq[n]))
    for n in (1, 2, 9):
        x = synth.normal(198 + n, (n, K))
        y, _ = r.mul_mat(t, w, M, K, x)
        assert same_bits(o.mul_mat(t, w, M, K, x), y)
        y, _ = r.mul_mat(t, wq, 8, K, x)
        assert same_bits(o.mul_mat(t, wq, 8, K, x), y)


def test_lowk_oracle_catches_planted_mistakes():
    """The unpacking check above is sensitive to the mistakes a restatement
    could plausibly make: a swapped nibble, the wrong hmask bit, a dropped
    min term or a transposed scale index each change the values."""
    w = synth.random_blocks(Q3_K, 199, 4, 256).reshape(-1, 110)
    good, _ = lowk_numpy_dequant(Q3_K, w)
    o = oracle()
    assert same_bits(o.dequantize(Q3_K, w, 256), good)
    bad = w.copy()
    bad[:, 0:32] ^= 0x01  # one hmask bit of every element run 0
    assert not same_bits(o.dequantize(Q3_K, bad, 256), good)
    w2 = synth.random_blocks(Q2_K, 199, 4, 256).reshape(-1, 84)
    good2, code = lowk_numpy_dequant(Q2_K, w2)
    d = w2[:, 80:82].copy().view(np.float16).astype(np.float32)
    no_min = (d * (w2[:, np.arange(256) // 16] & 15).astype(np.float32) * code.astype(np.float32)).astype(np.float32)
    assert not same_bits(no_min, good2)
    swapped = w2.copy()
    swapped[:, :16] = ((w2[:, :16] & 15) << 4) | (w2[:, :16] >> 4)  # scale and min nibbles exchanged
    assert not same_bits(o.dequantize(Q2_K, swapped, 256), good2)


# ---------------------------------------------- q4_1 / q5_0 / q5_1 and q8_1
# tlq_dequantize_row_q4_1 / _q5_0 / _q5_1 (ggml-quants.c:479-551),
# tlq_quantize_row_q8_1 (:302-335) and the generic vec_dots
# (ggml-cpu/quants.c:262-296, :365-449): pinned by the compiled reference's
# outputs (legacy_quants.npz), bit-exact; an independent numpy unpacking of the
# codes; q8_1's s against numpy's float16 cast; float64 brute force; the live
# reference.
LEGACY = ((Q4_1, "q4_1", 111), (Q5_0, "q5_0", 121), (Q5_1, "q5_1", 131))
LEGACY_IDS = [n for _, n, _ in LEGACY]


@pytest.mark.parametrize("t,name,seed", LEGACY, ids=LEGACY_IDS)
def test_legacy_quants_golden(t, name, seed):
    from refs import xorshift_noise

    o, g = oracle(), gold("legacy_quants")
    assert same_bits(o.dequantize(t, g[f"{name}_w"], 256), g[f"{name}_deq"])
    for n in g["ns"]:
        y = o.mul_mat(t, g[f"{name}_w"], 96, 256, xorshift_noise((int(n), 256), 10 + int(n)))
        assert same_bits(y, g[f"{name}_y{n}"]), n
    rw = synth.random_blocks(t, seed, 40, 1024)
    assert np.array_equal(rw, g[f"{name}_rand_w"])  # the generator still makes the fixture's blocks
    assert same_bits(o.dequantize(t, rw[:8], 1024), g[f"{name}_rand_deq8"])
    assert same_bits(o.mul_mat(t, rw, 40, 1024, synth.normal(seed + 1, (3, 1024))), g[f"{name}_rand_y"])


def test_q8_1_golden_and_against_numpy():
    """q8_1 = q8_0's f16 d and codes, plus s = f16(code sum * the f32 d): the codes
    and d against the (separately pinned) q8_0 quantizer, s rebuilt with
    numpy's float16 cast from the codes and amax / 127."""
    o, g = oracle(), gold("legacy_quants")
    x = g["act_x"]
    q = o.quantize(Q8_1, x)
    assert np.array_equal(q, g["q8_1"])
    b1, b0 = q.reshape(-1, 36), o.quantize(Q8_0, x).reshape(-1, 34)
    assert np.array_equal(b1[:, 0:2], b0[:, 0:2]) and np.array_equal(b1[:, 4:], b0[:, 2:])
    d32 = (np.abs(x).reshape(-1, 32).max(1) / np.float32(127)).astype(np.float32)
    sums = b1[:, 4:].view(np.int8).astype(np.int32).sum(1).astype(np.float32)
    with np.errstate(over="ignore"):  # the 1e4-scaled row's sums overflow f16 to inf, as ggml's do
        want = (sums * d32).astype(np.float16).view(np.uint16)
    assert np.array_equal(b1[:, 2:4].copy().view(np.uint16)[:, 0], want)


def _legacy_fields(t, w):
    """(d, m, codes) of q4_1 / q5_0 / q5_1 blocks by numpy, from the block
    layouts of ggml-common.h:201-249 (m = 0 for q5_0, codes with q5_0's -16)."""
    bb = {Q4_1: 20, Q5_0: 22, Q5_1: 24}[t]
    b = w.reshape(-1, bb)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    m = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0] if t != Q5_0 else np.zeros_like(d)
    qs = b[:, bb - 16:].astype(np.int64)
    codes = np.concatenate([qs & 15, qs >> 4], axis=1)
    if t != Q4_1:
        qh = b[:, bb - 20: bb - 16].copy().view(np.uint32)[:, 0].astype(np.int64)
        codes |= ((qh[:, None] >> np.arange(32)) & 1) << 4
    if t == Q5_0:
        codes -= 16
    return d, m, codes


@pytest.mark.parametrize("t,name,seed", LEGACY, ids=LEGACY_IDS)
def test_legacy_codes_against_an_independent_unpacking(t, name, seed):
    """y = code * d (+ m) in f32 with the codes rebuilt here over whole arrays,
    bit-exact; every code value occurs."""
    o = oracle()
    w = synth.random_blocks(t, seed + 5, 12, 512)
    d, m, codes = _legacy_fields(t, w)
    want = (codes.astype(np.float32) * d[:, None]).astype(np.float32)
    if t != Q5_0:
        want = (want + m[:, None]).astype(np.float32)
    lo, hi = {Q4_1: (0, 15), Q5_0: (-16, 15), Q5_1: (0, 31)}[t]
    assert codes.min() == lo and codes.max() == hi
    assert same_bits(o.dequantize(t, w, 512).reshape(-1, 32), want)


@pytest.mark.parametrize("t,name,seed", LEGACY, ids=LEGACY_IDS)
def test_legacy_vec_dot_against_f64_bruteforce(t, name, seed):
    """vec_dot = the float64 sum of the dequantized weights times the activation
    values d8 * q8, up to f32 accumulation and, for q4_1 / q5_1, the f16
    rounding of q8_1's s (m * s stands for m * d8 * sum q8): a dropped min term,
    a wrong fifth bit or sign fails."""
    o = oracle()
    K = 2048
    w = synth.random_blocks(t, seed + 6, 8, K)
    x = synth.normal(seed + 7, (4, K))
    xq = o.quantize_act(t, x)
    at = Q8_1 if t != Q5_0 else Q8_0
    ab = {Q8_1: 36, Q8_0: 34}[at]
    yb = xq.reshape(4, -1, ab)
    d8 = yb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    q8 = yb[:, :, ab - 32:].view(np.int8).astype(np.float64)
    xd = (d8[:, :, None] * q8).reshape(4, K)
    wd = o.dequantize(t, w, K).astype(np.float64)
    want = wd @ xd.T
    got = np.array([[o.vec_dot(t, K, w[i], xq[j]) for j in range(4)] for i in range(8)])
    tol = 1e-6 * (np.abs(wd) @ np.abs(xd).T)
    if at == Q8_1:
        _, m, _ = _legacy_fields(t, w)
        s8 = np.abs(yb[:, :, 2:4].copy().view(np.float16).astype(np.float64)[:, :, 0])
        tol += np.abs(m.reshape(8, -1)) @ s8.T * 2.0 ** -10
    assert np.all(np.abs(got - want) <= tol)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
@pytest.mark.parametrize("t,name,seed", LEGACY, ids=LEGACY_IDS)
def test_legacy_matches_reference_live(t, name, seed):
    o, r = oracle(), ref()
    M, K = 72, 1024
    w = synth.random_blocks(t, seed + 8, M, K)
    assert same_bits(o.dequantize(t, w, K), r.dequantize(t, w, K))
    wq = r.quantize_weights(t, synth.normal(seed + 9, (8, K), 0.02))
    for n in (1, 2, 9):
        x = synth.normal(seed + 10 + n, (n, K)) * 3
        assert np.array_equal(o.quantize_act(t, x), r.quantize_act(t, x))
        assert same_bits(o.mul_mat(t, w, M, K, x), r.mul_mat(t, w, M, K, x)[0])
        assert same_bits(o.mul_mat(t, wq, 8, K, x), r.mul_mat(t, wq, 8, K, x)[0])


# ------------------------------------------------ float weights (f32 / f16 / bf16)
FLOATS = ((F32, "f32"), (F16, "f16"), (BF16, "bf16"))


def test_bf16_conversion_against_torch():
    """tlq_fp32_to_bf16 rounds to nearest, ties to even, as torch's bfloat16 cast
    does (an independent implementation), on random bit patterns, exact ties with
    even and odd kept halves, and the rounding into infinity; a NaN stays a NaN
    with the quiet bit set; bf16 -> f32 puts the bits in the upper half."""
    import torch

    o = oracle()
    bits = synth.integers(91, 0, 2**32 - 1, 3000).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000]  # finite
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000, 0x7F7F7FFF, 0x00008000, 0x00018000,
                     0x7F7FFFFF, 0x80000000, 0x00000001], np.uint32)
    f = np.concatenate([bits, ties]).view(np.float32)
    got = o.f32_to_bf16(f)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    assert list(got[-10:-6]) == [0x3F80, 0x3F82, 0xBF80, 0x7F80]  # ties to even, and into +inf
    nan = np.array([0x7F800001, 0xFF800001, 0x7FC00000], np.uint32).view(np.float32)
    assert list(o.f32_to_bf16(nan)) == [0x7FC0, 0xFFC0, 0x7FC0]
    h = np.arange(0, 65536, 7, dtype=np.uint16)
    h = h[((h & 0x7F80) != 0x7F80) | ((h & 0x7F) == 0)]  # NaNs lose their payload on the way through a double
    np.testing.assert_array_equal(o.bf16_to_f32(h).view(np.uint32), h.astype(np.uint32) << 16)


def test_float_mul_mat_golden_reference_cases():
    """The reference test's cases (native.rs:73-107, 96 x 256 noise weights, n in
    1,3,5,8,9,40) with f32 / f16 / bf16 weights, src1 already of the weight type,
    and a ragged K = 100: bit-exact with the CPU backend (mul_mat_float.npz)."""
    from refs import xorshift_noise

    o, g = oracle(), gold("mul_mat_float")
    for t, name in FLOATS:
        w = g[f"{name}_w"]
        for n in g["ns"]:
            assert same_bits(o.mul_mat(t, w, 96, 256, xorshift_noise((int(n), 256), 10 + int(n))), g[f"{name}_y{n}"])
        assert same_bits(o.mul_mat(t, g[f"k100_{name}_w"], 33, 100, g["k100_x"]), g[f"k100_{name}_y"])
    for name, up in (("f16", o.f16_to_f32), ("bf16", o.bf16_to_f32)):
        t = F16 if name == "f16" else BF16
        for n in (1, 9):
            x = up(g[f"{name}_x{n}_same"])  # exact in f32; the oracle's conversion back is the identity
            assert same_bits(o.mul_mat(t, g[f"{name}_w"], 96, 256, x), g[f"{name}_y{n}_same"])


@pytest.mark.parametrize("t,name", FLOATS, ids=[n for _, n in FLOATS])
def test_float_mul_mat_against_f64(t, name):
    """Every output is the f64 sum of f32 products of the weights and src1 rounded
    to the weight type (numpy float16 / torch bfloat16 casts), to the last f32
    rounding: an unrounded src1 (about 1e-3 relative for f16) or a dropped term fails."""
    import torch

    o = oracle()
    M, K, N = 40, 1000, 3
    wf, x = synth.normal(92, (M, K)), synth.normal(93, (N, K)) * 3
    if t == F32:
        wq, wd, xd = wf, wf, x
    elif t == F16:
        wq = wf.astype(np.float16).view(np.uint16)
        wd, xd = wf.astype(np.float16).astype(np.float32), x.astype(np.float16).astype(np.float32)
    else:
        bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()  # noqa: E731
        wq = torch.from_numpy(wf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        wd, xd = bf(wf), bf(x)
    prods = wd[None, :, :] * xd[:, None, :]  # f32 products [N, M, K]
    want = prods.astype(np.float64).sum(-1)
    got = o.mul_mat(t, wq, M, K, x).astype(np.float64)
    bound = np.abs(want) * 2.0**-24 + 1e-14 * np.abs(prods).astype(np.float64).sum(-1)
    assert (np.abs(got - want) <= bound).all()


@pytest.mark.parametrize("t,name", FLOATS, ids=[n for _, n in FLOATS])
def test_float_mul_mat_matches_reference_live(t, name):
    r = ref()
    o = oracle()
    for M, K, N in ((7, 33, 3), (64, 256, 5), (40, 4096, 17)):
        wq = r.quantize_weights(t, synth.normal(94 + K, (M, K)))
        x = synth.normal(95 + N, (N, K))
        assert same_bits(o.mul_mat(t, wq, M, K, x), r.mul_mat(t, wq, M, K, x)[0])


# ------------------------------------------------------------- MUL_MAT_ID
def test_mul_mat_id_golden_is_the_per_expert_mul_mat():
    """The CPU backend's MUL_MAT_ID (mul_mat_id.npz) equals, column by column, the
    oracle's MUL_MAT of the selected expert's matrix with src1 row (e % n_b1, t),
    bit for bit (ggml-cpu.c:1460-1640 quantizes src1 once and runs the same vec_dot)."""
    from refs import MMID_CASES, mmid_case

    o, g = oracle(), gold("mul_mat_id")
    for case in MMID_CASES:
        name, t, K, M, n_as, n_used, n_b1, n_tok, _ = case
        _, _, (wh,), (xh, idh) = mmid_case(case)
        res = g[name][0]
        W = wh.reshape(n_as, M, -1)
        for tt in range(n_tok):
            for e in range(n_used):
                want = o.mul_mat(t, W[idh[tt, e]], M, K, xh[tt, e % n_b1][None])
                assert same_bits(want.reshape(-1), res[tt, e]), (name, tt, e)


# -------------------------------------------------------- paged attention
def _random_paged(seqs, heads, kvh, hs, bs, lens, seed, pool=None):
    """Random paged KV cache with scattered block tables (as BASELINE config 4)."""
    maxb = max(1, max((L + bs - 1) // bs for L in lens))
    need = sum((L + bs - 1) // bs for L in lens)
    nblocks = pool or max(need * 2, 4)
    perm = synth.bits(seed, nblocks).argsort()[:need]
    tables = np.zeros((seqs, maxb), np.int32)
    c = 0
    for s, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        tables[s, :nb] = perm[c:c + nb]
        c += nb
    kc = synth.f16_bits(synth.normal(seed + 1, (nblocks, kvh, hs // 8, bs, 8)))
    vc = synth.f16_bits(synth.normal(seed + 2, (nblocks, kvh, hs, bs)))
    q = synth.f16_bits(synth.normal(seed + 3, (seqs, heads, hs)))
    return q, kc, vc, tables, np.array(lens, np.int32)


def attention_f64(q, kc, vc, tables, lens, kvh, bs, scale):
    """Brute-force softmax(scale q k^T) v in float64 over exactly the f16 K/V."""
    o = oracle()
    seqs, heads, hs = q.shape
    out = np.zeros((seqs, heads, hs))
    qf = q.view(np.float16).astype(np.float64)
    for s in range(seqs):
        L = int(lens[s])
        if L == 0:
            continue
        k, v = o.gather_kv(kc, vc, tables[s], L, kvh, hs, bs)
        k = k.view(np.float16).astype(np.float64)
        v = v.view(np.float16).astype(np.float64)
        for h in range(heads):
            g = h // (heads // kvh)
            lg = scale * (k[g] @ qf[s, h])
            p = np.exp(lg - lg.max())
            out[s, h] = (p / p.sum()) @ v[g]
    return out


@pytest.mark.parametrize("hs,bs,kvh,heads,lens", [
    (128, 16, 2, 8, [70, 33, 5]),
    (64, 8, 1, 4, [1, 17, 64]),
    (256, 32, 4, 4, [100, 1]),
    (80, 16, 1, 2, [40]),
])
def test_paged_attention_oracle_vs_bruteforce(hs, bs, kvh, heads, lens):
    o = oracle()
    q, kc, vc, tables, L = _random_paged(len(lens), heads, kvh, hs, bs, lens, 90)
    scale = 1.0 / np.sqrt(hs)
    got = o.paged_attention(q, kc, vc, kvh, scale, tables, L, bs).view(np.float16).astype(np.float64)
    want = attention_f64(q, kc, vc, tables, L, kvh, bs, scale)
    # f16 probabilities and f16 output: ~1e-3 of the output scale
    assert np.abs(got - want).max() <= 3e-3 * np.abs(want).max()


def test_paged_attention_oracle_vs_ggml_flash_attn_golden():
    """The oracle on a one-sequence paged cache holding the golden dense K/V equals
    ggml's CPU FLASH_ATTN_EXT (f16 Q and f16 V accumulation there) within f16 error."""
    o, g = oracle(), gold("flash_attn")
    for i in range(4):
        q32, k, v, want = g[f"q{i}"], g[f"k{i}"], g[f"v{i}"], g[f"o{i}"]
        Hkv, L, D = k.shape
        H = q32.shape[0]
        bs = 16
        nb = (L + bs - 1) // bs
        kc = np.zeros((nb, Hkv, D // 8, bs, 8), np.uint16)
        vc = np.zeros((nb, Hkv, D, bs), np.uint16)
        key = k.transpose(1, 0, 2).reshape(L, Hkv * D)
        val = v.transpose(1, 0, 2).reshape(L, Hkv * D)
        o.reshape_and_cache(key, val, kc, vc, np.arange(L, dtype=np.int64), Hkv, D, bs)
        q16 = synth.f16_bits(q32)[None]
        got = o.paged_attention(q16, kc, vc, Hkv, 1.0 / np.sqrt(D), np.arange(nb, dtype=np.int32)[None],
                                np.array([L], np.int32), bs)
        got = got.view(np.float16).astype(np.float32)[0]
        assert np.abs(got - want).max() <= 4e-3 * np.abs(want).max(), i


def test_reshape_and_cache_gather_roundtrip():
    """Scatter through slots (negative = skip) then gather: bit-exact."""
    o = oracle()
    kvh, hs, bs, T = 2, 64, 8, 40
    nblocks = 12
    key = synth.f16_bits(synth.normal(95, (T, kvh * hs)))
    val = synth.f16_bits(synth.normal(96, (T, kvh * hs)))
    table = (synth.bits(97, nblocks).argsort()[:5]).astype(np.int32)
    slots = np.array([table[t // bs] * bs + t % bs for t in range(T)], np.int64)
    slots[7] = -1
    kc = np.zeros((nblocks, kvh, hs // 8, bs, 8), np.uint16)
    vc = np.zeros((nblocks, kvh, hs, bs), np.uint16)
    o.reshape_and_cache(key, val, kc, vc, slots, kvh, hs, bs)
    k, v = o.gather_kv(kc, vc, table, T, kvh, hs, bs)
    kk = key.reshape(T, kvh, hs).transpose(1, 0, 2)
    vv = val.reshape(T, kvh, hs).transpose(1, 0, 2)
    keep = np.ones(T, bool)
    keep[7] = False
    assert np.array_equal(k[:, keep], kk[:, keep]) and np.array_equal(v[:, keep], vv[:, keep])
    assert np.all(k[:, 7] == 0) and np.all(v[:, 7] == 0)


# --------------------------------------------------------- FLASH_ATTN_EXT
# tlq_flash_attn_ext restates the CPU backend's vec path (ops.cpp:8468-8700) and
# split-KV decode path (ops.cpp:9115-9145, :8996-9063). Pins: the reference's own
# outputs on its test shapes (golden, bit-exact where the backend takes those two
# paths; its tiled path for >= 64 queries accumulates in f32 instead), the compiled
# reference live, and a float64 brute force (f16 accumulator error only).
from refs import FA_CASES, fa_case_inputs, flash_attn_f64  # noqa: E402


def _fa_tiled(case):
    return case[4] >= 64  # ggml_fa_tile_config::Q (common.h:9): the backend's tiled path


@pytest.mark.parametrize("case", FA_CASES, ids=[c[0] for c in FA_CASES])
def test_flash_attn_oracle_golden(case):
    g = gold("flash_attn_ext")
    name = case[0]
    q, k, v, m, scale, max_bias, softcap = fa_case_inputs(case, int(g[f"{name}/seed"][0]))
    got = oracle().flash_attn_ext(q, k, v, m, scale, max_bias, softcap, nthreads=8)[:, g[f"{name}/rows"]]
    want = g[f"{name}/out"]
    if _fa_tiled(case):
        assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max() + 1e-6
    else:
        assert same_bits(got, want), np.abs(got - want).max()


def test_flash_attn_oracle_dense_golden_of_paged_tests():
    """The one-query dense goldens (flash_attn.npz: L = 70, 33, 515, 5), bit-exact;
    L = 515 takes the split-KV path with 8 chunks."""
    g = gold("flash_attn")
    for i in range(4):
        q32, k, v, want = g[f"q{i}"], g[f"k{i}"], g[f"v{i}"], g[f"o{i}"]
        Hkv, L, D = k.shape
        H = q32.shape[0]
        got = oracle().flash_attn_ext(q32.reshape(1, H, 1, D), k[None], v[None], None, 1.0 / np.sqrt(D),
                                      nthreads=8)
        assert same_bits(got.reshape(H, D), want), i


FA_RANDOM = [
    # nb, nh, nhkv, nq, L, D, DV, mask kind, max_bias, softcap
    (1, 4, 1, 1, 70, 128, 128, "none", 0.0, 0.0),
    (2, 8, 2, 7, 45, 64, 64, "holes", 0.0, 0.0),
    (1, 6, 3, 3, 33, 80, 80, "bias", 8.0, 0.0),  # ALiBi, heads past n_head_log2 = 4 use m1
    (2, 4, 4, 5, 20, 96, 96, "many", 0.0, 50.0),
    (1, 8, 1, 1, 900, 112, 112, "holes", 0.0, 0.0),  # split-KV decode
    (2, 4, 2, 2, 64, 192, 128, "bias", 2.0, 0.0),
]


@pytest.mark.parametrize("nthreads", [8, 3])
@pytest.mark.parametrize("shape", FA_RANDOM)
def test_flash_attn_oracle_vs_reference_live(shape, nthreads):
    r = ref()
    if r is None:
        pytest.skip("oracle/_ref is not built here (needs /root/reference)")
    case = ("live",) + shape
    q, k, v, m, scale, max_bias, softcap = fa_case_inputs(case, 4242 + shape[4])
    got = oracle().flash_attn_ext(q, k, v, m, scale, max_bias, softcap, nthreads=nthreads)
    want, _ = r.flash_attn_ext(q, k, v, m, scale, max_bias, softcap, nthreads=nthreads)
    assert same_bits(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("shape", FA_RANDOM)
def test_flash_attn_oracle_vs_f64(shape):
    """Within the f16 accumulator's error of the exact softmax over the f16 inputs:
    a dropped soft cap, slope, mask term or scale moves results by O(1) of the scale."""
    case = ("f64",) + shape
    q, k, v, m, scale, max_bias, softcap = fa_case_inputs(case, 777 + shape[5])
    got = oracle().flash_attn_ext(q, k, v, m, scale, max_bias, softcap)
    want = flash_attn_f64(q, k, v, m, scale, max_bias, softcap)
    assert np.abs(got - want).max() <= 8e-3 * np.abs(want).max()


def test_flash_attn_f64_pins_against_closed_forms():
    """The brute force itself: a single key gives v exactly; identical keys give the
    mean of the values; a fully masked row gives 0; softcap -> tanh bound."""
    rng = np.random.default_rng(5)
    D = 64
    q = rng.standard_normal((1, 2, 3, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, D)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((1, 1, 1, D)).astype(np.float16).view(np.uint16)
    o = flash_attn_f64(q, k, v, None, 0.3)
    assert np.allclose(o, v.view(np.float16).astype(np.float64)[0, 0, 0])
    k4 = np.repeat(k, 5, axis=2)
    v4 = rng.standard_normal((1, 1, 5, D)).astype(np.float16).view(np.uint16)
    o = flash_attn_f64(q, k4, v4, None, 0.3)
    assert np.allclose(o, v4.view(np.float16).astype(np.float64)[0, 0].mean(0))
    m = np.full((1, 1, 3, 5), np.float16(-np.inf)).view(np.uint16)
    assert np.all(flash_attn_f64(q, k4, v4, m, 0.3) == 0)
    # the oracle agrees on those three closed forms too
    got = oracle().flash_attn_ext(q, k4, v4, m, 0.3)
    assert np.all(got == 0)


def test_flash_attn_oracle_catches_planted_mistakes():
    """Mistakes planted in the inputs the oracle sees (on the CPU): a wrong scale, a
    dropped soft cap or a dropped ALiBi slope each move the result far outside the
    f64 tolerance the oracle meets."""
    case = ("plant", 1, 6, 2, 2, 40, 64, 64, "bias", 8.0, 1.5)  # a cap that saturates tanh
    q, k, v, m, scale, max_bias, softcap = fa_case_inputs(case, 99)
    want = flash_attn_f64(q, k, v, m, scale, max_bias, softcap)
    tol = 8e-3 * np.abs(want).max()
    o = oracle()
    assert np.abs(o.flash_attn_ext(q, k, v, m, scale, max_bias, softcap) - want).max() <= tol
    assert np.abs(o.flash_attn_ext(q, k, v, m, scale * 1.5, max_bias, softcap) - want).max() > 10 * tol
    assert np.abs(o.flash_attn_ext(q, k, v, m, scale, 0.0, softcap) - want).max() > 10 * tol
    assert np.abs(o.flash_attn_ext(q, k, v, m, scale, max_bias, 0.0) - want).max() > 10 * tol


# ------------------------------------------------------------------ core ops
from refs import (CORE_KINDS, F16, F32, I32, core_cases, core_oracle, core_ref)  # noqa: E402

CORE = core_cases()


def _as_f32(o, a):
    return o.f16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float64)


@pytest.mark.parametrize("case", CORE, ids=[c["name"] for c in CORE])
def test_core_oracle_golden(case):
    """The restated core ops against the reference CPU backend's outputs:
    bit-exact, except where that backend's x86 build takes a polynomial exp
    (silu, soft_max), where a few ulp separate them."""
    o = oracle()
    want = gold("core")[case["name"]]
    got = core_oracle(o, case)
    assert got.shape == want.shape and got.dtype == want.dtype
    if case["exact"]:
        np.testing.assert_array_equal(got, want)
    else:
        g, w = _as_f32(o, got), _as_f32(o, want)
        assert np.all(np.abs(g - w) <= 1e-6 * np.abs(w) + 1e-9), np.abs(g - w).max()


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_core_oracle_vs_reference_live(seed):
    """Fresh shapes and parameters through both: norms of odd widths, rope with
    random bases / YaRN parameters, get_rows of every weight type."""
    o, r = oracle(), ref()
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000))
    x = (rng.standard_normal((3, n)) * rng.uniform(0.1, 10) + rng.uniform(-2, 2)).astype(np.float32)
    for rms in (0, 1):
        c = dict(kind=CORE_KINDS["norm"], srcs=[(x, F32)], dst=(x.shape, F32), ip=(rms,), fp=(1e-5,), init=None,
                 perm=None)
        np.testing.assert_array_equal(core_oracle(o, c), core_ref(r, c))
    nd = int(rng.integers(1, 33)) * 2
    a = rng.standard_normal((4, 3, nd + 2 * int(rng.integers(0, 4)))).astype(np.float32)
    pos = rng.integers(0, 40000, 4).astype(np.int32)
    fp = (float(rng.uniform(100, 1e6)), float(rng.uniform(0.1, 1)), float(rng.integers(0, 2)),
          float(rng.uniform(0.5, 2)), float(rng.uniform(16, 64)), float(rng.uniform(0.5, 2)))
    for mode in (0, 2):
        c = dict(kind=CORE_KINDS["rope"], srcs=[(a, F32), (pos, I32)], dst=(a.shape, F32),
                 ip=(nd, mode, int(rng.integers(512, 8192))), fp=fp, init=None, perm=None)
        np.testing.assert_array_equal(core_oracle(o, c), core_ref(r, c))
    for t in (Q4_0, Q8_0, Q4_K, Q6_K):
        k = 256 * int(rng.integers(1, 4))
        w = synth.random_blocks(t, seed + t, 9, k)
        ids = rng.integers(0, 9, 5).astype(np.int32)
        c = dict(kind=CORE_KINDS["get_rows"], srcs=[(w, t, k), (ids, I32)], dst=((5, k), F32), ip=(), fp=(),
                 init=None, perm=None)
        np.testing.assert_array_equal(core_oracle(o, c), core_ref(r, c))


def test_core_oracle_against_the_mathematics():
    """What the mathematics fixes, independent of the reference: rms_norm and norm
    against float64, softmax rows against float64 (and summing to one), rope
    as a rotation by pos * base^(-2p/n) (neox pairs p, p + n/2), argmax as the
    last maximum, get_rows of q8_0 as the dequantized rows, cpy of a permuted
    view as numpy's transpose."""
    o = oracle()
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((4, 1000)) * 3 + 1).astype(np.float32)
    xd = x.astype(np.float64)
    rms = xd / np.sqrt((xd * xd).mean(1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(o.core_norm(True, 1e-5, x), rms, rtol=2e-6, atol=1e-6)
    c = xd - xd.mean(1, keepdims=True)
    np.testing.assert_allclose(o.core_norm(False, 1e-5, x), c / np.sqrt((c * c).mean(1, keepdims=True) + 1e-5),
                               rtol=2e-6, atol=1e-5)
    s = rng.standard_normal((1, 3, 2, 50)).astype(np.float32)
    m = rng.standard_normal((1, 1, 2, 50)).astype(np.float32)
    got = o.core_soft_max(s, 0.5, 0.0, m, F32)
    e = np.exp(s.astype(np.float64) * 0.5 + m - (s.astype(np.float64) * 0.5 + m).max(-1, keepdims=True))
    np.testing.assert_allclose(got, e / e.sum(-1, keepdims=True), rtol=1e-6, atol=1e-8)
    a = rng.standard_normal((3, 2, 16)).astype(np.float32)
    pos = np.array([0, 5, 300], np.int32)
    got = o.core_rope(a, F32, pos, 16, 2, 0, 10000.0, 1.0, 0.0, 1.0, 0.0, 0.0)
    th = pos[:, None].astype(np.float64) * 10000.0 ** (-2.0 * np.arange(8) / 16)
    x0, x1 = a[..., :8].astype(np.float64), a[..., 8:].astype(np.float64)
    cs, sn = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    np.testing.assert_allclose(got[..., :8], x0 * cs - x1 * sn, atol=2e-5)
    np.testing.assert_allclose(got[..., 8:], x0 * sn + x1 * cs, atol=2e-5)
    b = rng.integers(0, 4, (5, 64)).astype(np.float32)
    want = b.shape[1] - 1 - np.argmax(b[:, ::-1], axis=1)
    np.testing.assert_array_equal(o.core_argmax(b), want)
    w = synth.random_blocks(Q8_0, 9, 6, 256)
    ids = np.array([5, 0, 5], np.int32)
    np.testing.assert_array_equal(o.core_get_rows(w, Q8_0, ids, I32, k=256), o.dequantize(Q8_0, w, 256)[ids])
    q = rng.standard_normal((2, 3, 4)).astype(np.float32)
    np.testing.assert_array_equal(o.core_cpy(q.transpose(1, 0, 2), F32, (3, 2, 4), F32), q.transpose(1, 0, 2))


def test_fast_reference_builds_agree_with_the_parity_build():
    """The x86-64-v3 / v4 builds of the reference (oracle/Makefile ref_fast,
    ggml's SIMD paths) that bench.py times as a labelled fast CPU baseline
    compute the same MUL_MAT as the parity build up to f32 rounding (the
    north star's 1e-3 relative / 1e-4 absolute), so their speed is the speed
    of the same work."""
    from refs import ISA_LEVELS, REF_SO, Ref

    builds = [(lv, REF_SO.parent / lv / REF_SO.name) for lv, _ in ISA_LEVELS]
    builds = [(lv, p) for lv, p in builds if p.exists()]
    if ref() is None or not builds:
        pytest.skip("oracle/_ref ISA builds not built here")
    flags = ""
    for ln in Path("/proc/cpuinfo").read_text().splitlines():
        if ln.startswith("flags"):
            flags = ln
            break
    r = ref()
    for lv, p in builds:
        need = dict(ISA_LEVELS)[lv]
        if not all(f in flags.split() for f in need):
            continue
        f = Ref(p)
        for t in (Q4_0, Q8_0, Q4_K, Q6_K, Q2_K):
            w = synth.random_blocks(t, 150 + t, 64, 1024)
            x = synth.normal(151, (3, 1024))
            want, _ = r.mul_mat(t, w, 64, 1024, x)
            got, _ = f.mul_mat(t, w, 64, 1024, x)
            assert np.all(np.abs(got - want) <= 1e-4 + 1e-3 * np.abs(want)), (lv, t)

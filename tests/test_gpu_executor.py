"""GPU parity: whole graphs through the executor (tlh_program_compile / run).

* A llama-style decoder step (tensorlisp_amd.graph.decoder_step: embedding
  GET_ROWS, RMS_NORM x weight, Q/K/V MUL_MATs, RoPE, SET_ROWS into f16 KV
  caches, FLASH_ATTN_EXT over cache views, output projection, SwiGLU FFN,
  residual adds, lm_head, ARGMAX) for a 5-token prompt, three single-token
  steps and a 3-token chunk, against the reference CPU backend running the same
  graph (tests/golden/decoder.npz; live through oracle/_ref where it is built):
  logits and KV caches within 8e-3 of their largest magnitude -- the
  reference's own tolerance for flash attention against its CPU backend
  (crates/tensorlisp/tests/native.rs:51-57, :183), the one op whose results
  differ beyond rounding: the CPU accumulates P.V in f16 (ops.cpp:8468-8650,
  VKQ16), the GPU in f32, about 4e-4 of an attention output per layer, which
  the following layers carry to about 3e-3 at the logits; everything else
  agrees to ~1e-7 -- and the same argmax.
* Graph replay: the captured hipGraph gives bit-identical results to the eager
  launches on every replay, with eager work in between.
* MUL_MATs that share one quantized activation give bit-identical results to
  each computed alone.
"""
from __future__ import annotations

import numpy as np
import pytest

from refs import (DECODER_STEPS, decoder_ref_run, decoder_step_inputs, decoder_tiny_config, decoder_weights, oracle,
                  ref)
from tensorlisp_amd import graph as G
from tensorlisp_amd import native as N

pytestmark = pytest.mark.gpu


def gold():
    from pathlib import Path

    return np.load(Path(__file__).resolve().parent / "golden" / "decoder.npz")


def dev(a):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


class GpuDecoder:
    def __init__(self, c, weights, on_device=False):
        import torch

        self.c = c
        self.w = list(weights) if on_device else [dev(w) for w in weights]
        self.offs, total = c.state_bytes()
        self.state = torch.zeros(total, dtype=torch.uint8, device="cuda")

    def step(self, step, graph=False, stream=None):
        import torch

        toks, p0, n_kv, every = step
        st = G.decoder_step(self.c, len(toks), n_kv, last_only=not every)
        prog = G.Program(st.builder, st.keep, self.w, self.offs)
        for i, a in enumerate(decoder_step_inputs(step)):
            prog.write_input(i, dev(a), stream)
        prog.run(self.state, stream, graph)
        lg = prog.read(st.logits, torch.float32, self.state, stream)
        am = prog.read(st.argmax, torch.int32, self.state, stream)
        torch.cuda.synchronize()
        return prog, st, lg.cpu().numpy().reshape(-1, self.c.n_vocab), am.cpu().numpy().reshape(-1)

    def caches(self):
        c = self.c
        s = self.state.cpu().numpy()
        per = c.n_embd_kv * c.n_ctx * 2
        return [s[o:o + per].view(np.uint16).reshape(c.n_ctx, c.n_embd_kv) for o in self.offs]


def close(got, want, tol, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    print(f"[executor] {what}: max err {err:.3e} (scale {scale:.3e})", flush=True)
    assert err <= tol * scale + 1e-6, (what, err, scale)


def check_steps(results, logits, ams, caches, dec):
    o = oracle()
    for i, (lg, am) in enumerate(results):
        close(lg, logits[i], 8e-3, f"step {i} logits")
        np.testing.assert_array_equal(am, ams[i])
    for i, (g, w) in enumerate(zip(dec.caches(), caches)):
        close(o.f16_to_f32(g), o.f16_to_f32(w), 8e-3, f"cache {i}")


def test_decoder_steps_match_reference_golden(gpu):
    c = decoder_tiny_config()
    dec = GpuDecoder(c, decoder_weights(c))
    res = [dec.step(s)[2:] for s in DECODER_STEPS]
    g = gold()
    n = len(DECODER_STEPS)
    check_steps(res, [g[f"logits{i}"] for i in range(n)], [g[f"argmax{i}"] for i in range(n)],
                [g[f"cache{i}"] for i in range(2 * c.n_layer)], dec)


@pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")
def test_decoder_steps_match_reference_live(gpu):
    """Other weights (seed 300) through both."""
    c = decoder_tiny_config()
    w = decoder_weights(c, seed=300)
    logits, ams, caches = decoder_ref_run(ref(), c, w)
    dec = GpuDecoder(c, w)
    check_steps([dec.step(s)[2:] for s in DECODER_STEPS], logits, ams, caches, dec)


def test_graph_replay_matches_eager(gpu):
    import torch

    c = decoder_tiny_config()
    dec = GpuDecoder(c, decoder_weights(c))
    for s in DECODER_STEPS[:1]:
        dec.step(s)
    step = DECODER_STEPS[1]
    stream = torch.cuda.Stream()
    prog, st, want, want_am = dec.step(step, graph=False, stream=stream)
    for rep in range(4):
        with torch.cuda.stream(stream):
            prog.run(dec.state, stream, graph=True)
            lg = prog.read(st.logits, torch.float32, dec.state, stream)
        stream.synchronize()
        np.testing.assert_array_equal(lg.cpu().numpy().reshape(-1, c.n_vocab), want, err_msg=f"replay {rep}")
        prog.run(dec.state, stream, graph=False)  # eager work between replays
        stream.synchronize()
    assert prog.stats()["launches"] > 0


def test_shared_quantization_matches_separate(gpu):
    """Q/K/V of one 8-column activation: the grouped launches (one quantization)
    against tlh_mul_mat per weight."""
    import torch

    from tensorlisp_amd import synth

    b = G.Builder()
    ws = [(N.Q4_K, 256), (N.Q4_K, 128), (N.Q6_K, 128)]
    W = [b.weight(ty, [512, m]) for ty, m in ws]
    x = b.input(N.F32, [512, 8])
    h = b.rms_norm(x, 1e-5)
    outs = [b.mul_mat(w, h) for w in W]
    for o in outs:
        b.expand(o)
    wd = [dev(synth.random_blocks(ty, 40 + i, m, 512)) for i, (ty, m) in enumerate(ws)]
    prog = G.Program(b, outs, wd)
    xv = dev(synth.normal(41, (8, 512)))
    prog.write_input(0, xv)
    prog.run()
    hv = N.rms_norm(xv, 1e-5)
    for (ty, m), wdev, o in zip(ws, wd, outs):
        want = N.mul_mat(ty, wdev, m, 512, hv)
        got = prog.read(o, torch.float32)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().reshape(want.shape), want.cpu().numpy())
    # norm; the two q4_K products: one quantization + one compute over both
    # matrices' rows; the q6_K one alone
    assert prog.stats()["launches"] == 1 + 2 + 1


@pytest.mark.parametrize("t", [N.Q4_K, N.Q5_K], ids=["q4_K", "q5_K"])
@pytest.mark.parametrize("n", [64, 512])
def test_prefill_qkv_one_gemm(gpu, t, n):
    """Q / K / V of a prefill (3 matrices of 512, 128 and 128 rows reading one
    RMS-normed activation of n >= 64 tokens): one GEMM launch over the 768 rows.
    Its K split follows all 768 rows, so its sums may split K unlike each
    matrix alone: every product is checked against the CPU oracle's
    mul_mat (quants.c dot products) to 1e-4 + 1e-3 |want|, and the
    dispatches are the norm chain (which quantizes) and the one GEMM."""
    import torch

    from tensorlisp_amd import synth

    K = 4096
    Ms = (512, 128, 128)
    b = G.Builder()
    x = b.input(N.F32, [K, n])
    nw = b.weight(N.F32, [K])
    W = [b.weight(t, [K, m]) for m in Ms]
    y = b.mul(b.rms_norm(x, 1e-5), nw)
    outs = [b.mul_mat(w, y) for w in W]
    for o in outs:
        b.expand(o)
    nwh = dev((1.0 + 0.1 * synth.normal(121, (K,))).astype(np.float32))
    wh = [synth.random_blocks(t, 122 + i, m, K) for i, m in enumerate(Ms)]
    prog = G.Program(b, outs + [y], [nwh] + [dev(w) for w in wh])
    xv = dev(synth.normal(123, (n, K)))
    prog.write_input(0, xv)
    print(f"[qkv-gemm] {N.TYPE_NAMES[t]} n={n}", flush=True)
    prog.run()
    yv = prog.read(y, torch.float32).reshape(n, K)
    torch.cuda.synchronize()
    yh = yv.cpu().numpy()
    rows = slice(0, n) if n <= 64 else np.r_[0:8, n - 8:n]  # the oracle on a sample of tokens at n = 512
    for m, w, o in zip(Ms, wh, outs):
        got = prog.read(o, torch.float32).reshape(n, m)
        torch.cuda.synchronize()
        want = oracle().mul_mat(t, w, m, K, np.ascontiguousarray(yh[rows]))
        g = got.cpu().numpy()[rows]
        bad = np.abs(g - want) > 1e-4 + 1e-3 * np.abs(want)  # the GEMM tests' tolerance
        assert not bad.any(), (N.TYPE_NAMES[t], m, n, float(np.abs(g - want).max()))
    assert prog.stats()["launches"] == 2


GQ_TYPES = [N.Q4_K, N.Q6_K, N.Q5_K, N.Q4_0, N.Q8_0, N.Q4_1, N.Q5_0, N.Q5_1]


@pytest.mark.parametrize("t", GQ_TYPES, ids=[N.TYPE_NAMES[t] for t in GQ_TYPES])
@pytest.mark.parametrize("K,n,op,group", [(14336, 16, "swiglu", False), (4096, 8, "geglu", True),
                                          (1024, 40, "swiglu", True), (512, 3, "swiglu", False)])
def test_glu_quantizes_for_its_mul_mats(gpu, t, K, n, op, group):
    """A GLU feeding MUL_MATs of n >= 3 columns (the SwiGLU before the down
    projection): the GLU kernel also writes the quantized activation (q8_K /
    q8_0 / q8_1 codes, scales and sums; at n > 16 the q4_K / q5_K GEMM's f16
    codes too) and no quantize launch runs. The GLU's output and every product
    are bit-identical to the core GLU and tlh_mul_mat (its own quantize launch)
    run one by one; K = 14336 takes the few-column kernel's K chunks."""
    import torch

    from tensorlisp_amd import synth

    Ms = (256, 128) if group else (256,)
    b = G.Builder()
    gt = b.input(N.F32, [K, n])
    up = b.input(N.F32, [K, n])
    W = [b.weight(t, [K, m]) for m in Ms]
    h = b.glu_split(gt, up, op)
    outs = [b.mul_mat(w, h) for w in W]
    for o in outs:
        b.expand(o)
    wd = [dev(synth.random_blocks(t, 102 + i, m, K)) for i, m in enumerate(Ms)]
    prog = G.Program(b, outs + [h], wd)
    gv, uv = dev(synth.normal(103, (n, K)) * 2), dev(synth.normal(104, (n, K)))
    prog.write_input(0, gv)
    prog.write_input(1, uv)
    print(f"[glu-quant] {N.TYPE_NAMES[t]} K={K} n={n} {op} group={group}", flush=True)
    prog.run()
    hv = N.glu(op, gv, uv)
    np.testing.assert_array_equal(prog.read(h, torch.float32).reshape(hv.shape).cpu().numpy(), hv.cpu().numpy())
    for m, wdev, o in zip(Ms, wd, outs):
        want = N.mul_mat(t, wdev, m, K, hv)
        got = prog.read(o, torch.float32)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().reshape(want.shape).view(np.uint32),
                              want.cpu().numpy().view(np.uint32)), f"{N.TYPE_NAMES[t]} M={m}"
    # dispatches: the GLU, then the products' compute launches (a group at
    # n <= 16: one few-column launch over both matrices' rows; above, one GEMM
    # launch over them for q4_K / q5_K)
    apart = group and n > 16 and t not in (N.Q4_K, N.Q5_K)
    assert prog.stats()["launches"] == 1 + (2 if apart else 1)


@pytest.mark.parametrize("t,K,n,order", [(N.Q4_K, 14336, 16, 0), (N.Q4_K, 14336, 8, 1), (N.Q4_0, 8192, 5, 0),
                                         (N.Q4_K, 4096, 512, 0), (N.Q8_0, 4096, 512, 1)])
def test_k_split_partials_summed_by_the_norm_chain(gpu, t, K, n, order):
    """A K-split MUL_MAT whose only reader is the ADD of a norm chain (the
    down or output projection, then the residual ADD and the next RMS_NORM)
    leaves its chunk partials, and the norm chain adds them in chunk order as
    it reads them: the chunk-sum launch goes. The residual sum and the norm's
    output are bit-identical to the same graph with the product kept as an
    output (which keeps the chunk-sum launch), with the product as either
    operand of the ADD; few-column and GEMM forms."""
    import torch

    from tensorlisp_amd import synth

    M = 4096
    outs = {}
    for keep in (False, True):
        b = G.Builder()
        x = b.input(N.F32, [M, n])
        h = b.input(N.F32, [K, n])
        nw = b.weight(N.F32, [M])
        W = b.weight(t, [K, M])
        y = b.mul_mat(W, h)
        s = b.add(y, x) if order else b.add(x, y)
        z = b.mul(b.rms_norm(s, 1e-5), nw)
        b.expand(z)
        wanted = [z, s] + ([y] if keep else [])
        prog = G.Program(b, wanted, [dev((1.0 + 0.1 * synth.normal(121, (M,))).astype(np.float32)),
                                     dev(synth.random_blocks(t, 122, M, K))])
        prog.write_input(0, dev(synth.normal(123, (n, M))))
        prog.write_input(1, dev(synth.normal(124, (n, K))))
        print(f"[partials-norm] {N.TYPE_NAMES[t]} K={K} n={n} order={order} keep={keep}", flush=True)
        trace = prog.trace()  # one eager run, recording each dispatch's kernel launches
        sums = sum(labels.count("partial_reduce") for _, labels in trace)
        outs[keep] = ([prog.read(v, torch.float32).cpu().numpy() for v in (z, s)], sums)
        torch.cuda.synchronize()
    (zf, sf), rf = outs[False]
    (zk, sk), rk = outs[True]
    assert np.array_equal(sf.view(np.uint32), sk.view(np.uint32))
    assert np.array_equal(zf.view(np.uint32), zk.view(np.uint32))
    assert (rf, rk) == (0, 1), (rf, rk)  # the chunk-sum launch goes only where the product is not kept


NQ_TYPES = [N.Q4_K, N.Q5_K, N.Q6_K, N.Q4_0, N.Q8_0, N.Q4_1, N.Q5_0]


@pytest.mark.parametrize("t", NQ_TYPES, ids=[N.TYPE_NAMES[t] for t in NQ_TYPES])
@pytest.mark.parametrize("K,n,add", [(4096, 64, True), (1024, 100, False), (4096, 16, True), (2048, 3, False)])
def test_norm_chain_quantizes_for_its_mul_mats(gpu, t, K, n, add):
    """[ADD ->] RMS_NORM -> MUL feeding MUL_MATs over 3 or more rows: the norm
    kernel also writes the group's quantized activation (q8_K / q8_0 / q8_1
    codes, scales and sums; at n > 16 the q4_K GEMM's f16 codes and bsums too)
    and no quantize launch runs. Below 64 rows (a batched decode step) each
    row's 1024-element groups go to workgroups of their own, each reading the
    whole row for the sums. Either way the norm's outputs and every product are
    bit-identical to the core ops and tlh_mul_mat run one by one. Over more
    than 16 rows the q4_K / q5_K products are one GEMM launch over the three
    matrices' rows (the first two whole 128-row tiles, the last not): its K
    split here is the one each matrix gets alone, so the sums agree bit for
    bit."""
    import torch

    from tensorlisp_amd import synth

    Ms = (256, 128, 100)
    b = G.Builder()
    p = b.input(N.F32, [K, n])
    q = b.input(N.F32, [K, n])
    nw = b.weight(N.F32, [K])
    W = [b.weight(t, [K, m]) for m in Ms]
    s = b.add(p, q) if add else p
    y = b.mul(b.rms_norm(s, 1e-5), nw)
    outs = [b.mul_mat(w, y) for w in W]
    for o in outs:
        b.expand(o)
    nwh = dev((1.0 + 0.1 * synth.normal(111, (K,))).astype(np.float32))
    wd = [dev(synth.random_blocks(t, 112 + i, m, K)) for i, m in enumerate(Ms)]
    prog = G.Program(b, outs + [y] + ([s] if add else []), [nwh] + wd)
    pv, qv = dev(synth.normal(113, (n, K)) * 2 + 0.3), dev(synth.normal(114, (n, K)))
    prog.write_input(0, pv)
    prog.write_input(1, qv)
    print(f"[norm-quant] {N.TYPE_NAMES[t]} K={K} n={n} add={add}", flush=True)
    prog.run()
    sv = N.add(pv, qv) if add else pv
    yv = N.mul(N.norm(sv, 1e-5, rms=True), nwh)
    np.testing.assert_array_equal(prog.read(y, torch.float32).reshape(yv.shape).cpu().numpy(), yv.cpu().numpy())
    for m, wdev, o in zip(Ms, wd, outs):
        want = N.mul_mat(t, wdev, m, K, yv)
        got = prog.read(o, torch.float32)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().reshape(want.shape).view(np.uint32),
                              want.cpu().numpy().view(np.uint32)), f"{N.TYPE_NAMES[t]} M={m}"
    # dispatches: the norm chain, the quantize launch when it stays apart, then
    # the products (n <= 16: one few-column launch over all matrices' rows;
    # more rows: one GEMM launch for q4_K / q5_K, else one per matrix)
    fused = n >= 3
    merged = n <= 16 or t in (N.Q4_K, N.Q5_K)
    assert prog.stats()["launches"] == 1 + (0 if fused else 1) + (1 if merged else len(Ms))


def test_program_refusals(gpu):
    c = decoder_tiny_config()
    dec = GpuDecoder(c, decoder_weights(c))
    st = G.decoder_step(c, 1, 8)
    prog = G.Program(st.builder, st.keep, dec.w, dec.offs)
    with pytest.raises(N.TlhError, match="state"):
        prog.run(None)
    with pytest.raises(N.TlhError, match="null stream"):
        N.check(N.lib().tlh_program_run(prog.ptr, dec.state.data_ptr(), None, 1))


@pytest.mark.parametrize("n,rms,add", [(4096, True, True), (4096, False, True), (8195, True, True), (8195, False, False),
                                       (100, False, True), (256, True, False)])
def test_fused_norm_chains_match_unfused(gpu, n, rms, add):
    """[ADD ->] RMS_NORM / NORM -> MUL(weight) runs as one kernel in a program;
    its outputs (the ADD's, which stays readable, and the MUL's) are bit-identical
    to the three core ops run one by one. Rows past the 4096 held in registers
    and tails of fewer than four elements included."""
    import torch

    from tensorlisp_amd import synth

    b = G.Builder()
    p = b.input(N.F32, [n, 3])
    q = b.input(N.F32, [n, 3])
    w = b.weight(N.F32, [n])
    s = b.add(p, q) if add else p
    t = b.rms_norm(s, 1e-5) if rms else b.norm(s, 1e-5)
    y = b.mul(t, w)
    b.expand(y)
    keep = [y, s] if add else [y]
    wd = dev(synth.normal(61, (n,)))
    prog = G.Program(b, keep, [wd])
    pv, qv = dev(synth.normal(62, (3, n)) * 2 + 0.5), dev(synth.normal(63, (3, n)))
    prog.write_input(0, pv)
    prog.write_input(1, qv)
    prog.run()
    sv = N.add(pv, qv) if add else pv
    tv = N.norm(sv, 1e-5, rms=rms)
    want = N.mul(tv, wd)
    got = prog.read(y, torch.float32).reshape(want.shape)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
    if add:
        np.testing.assert_array_equal(prog.read(s, torch.float32).reshape(sv.shape).cpu().numpy(), sv.cpu().numpy())
    assert prog.stats()["launches"] == 1


FUSE_TYPES = [N.Q4_K, N.Q4_0, N.Q8_0, N.Q6_K, N.Q5_K]


@pytest.mark.parametrize("t", FUSE_TYPES, ids=[N.TYPE_NAMES[t] for t in FUSE_TYPES])
@pytest.mark.parametrize("K,M,add", [(4096, 1536, True), (4096, 300, False), (256, 1000, True), (2048, 17, True)])
def test_norm_gemv_swiglu_is_one_launch(gpu, t, K, M, add):
    """[ADD ->] RMS_NORM -> MUL(weight) feeding a gate / up MUL_MAT pair at one
    column, then SwiGLU, runs as one register-GEMV launch that forms the
    normalized row itself and stores silu(gate) * up. Its outputs (h, and the
    ADD's sum) equal the same ops launched one by one (core ops, MUL_MAT, GLU)."""
    import torch

    from tensorlisp_amd import synth

    b = G.Builder()
    p = b.input(N.F32, [K, 1])
    q = b.input(N.F32, [K, 1])
    nw = b.weight(N.F32, [K])
    wg = b.weight(t, [K, M])
    wu = b.weight(t, [K, M])
    s = b.add(p, q) if add else p
    cur = b.mul(b.rms_norm(s, 1e-5), nw)
    h = b.glu_split(b.mul_mat(wg, cur), b.mul_mat(wu, cur), "swiglu")
    b.expand(h)
    nwh = (1.0 + 0.1 * synth.normal(81, (K,))).astype(np.float32)
    gw, uw = (synth.random_blocks(t, 82 + i, M, K) for i in range(2))
    prog = G.Program(b, [h] + ([s] if add else []), [dev(nwh), dev(gw), dev(uw)])
    pv, qv = dev(synth.normal(84, (1, K)) * 2 + 0.3), dev(synth.normal(85, (1, K)))
    prog.write_input(0, pv)
    prog.write_input(1, qv)
    prog.run()
    sv = N.add(pv, qv) if add else pv
    y = N.mul(N.norm(sv, 1e-5, rms=True), dev(nwh))
    want = N.glu("swiglu", N.mul_mat(t, dev(gw), M, K, y), N.mul_mat(t, dev(uw), M, K, y))
    got = prog.read(h, torch.float32).reshape(want.shape)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
    if add:
        np.testing.assert_array_equal(prog.read(s, torch.float32).reshape(sv.shape).cpu().numpy(), sv.cpu().numpy())
    assert prog.stats()["launches"] == 1


@pytest.mark.parametrize("t", FUSE_TYPES, ids=[N.TYPE_NAMES[t] for t in FUSE_TYPES])
def test_norm_feeding_one_gemv_is_one_launch(gpu, t):
    """The head's shape: RMS_NORM -> MUL(weight) -> one MUL_MAT at one column is
    one launch, equal to the ops launched one by one."""
    import torch

    from tensorlisp_amd import synth

    K, M = 4096, 5000
    b = G.Builder()
    x = b.input(N.F32, [K, 1])
    nw = b.weight(N.F32, [K])
    wo = b.weight(t, [K, M])
    out = b.mul_mat(wo, b.mul(b.rms_norm(x, 1e-5), nw))
    b.expand(out)
    nwh = (1.0 + 0.1 * synth.normal(86, (K,))).astype(np.float32)
    ow = synth.random_blocks(t, 87, M, K)
    prog = G.Program(b, [out], [dev(nwh), dev(ow)])
    xv = dev(synth.normal(88, (1, K)))
    prog.write_input(0, xv)
    prog.run()
    want = N.mul_mat(t, dev(ow), M, K, N.mul(N.norm(xv, 1e-5, rms=True), dev(nwh)))
    got = prog.read(out, torch.float32).reshape(want.shape)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
    assert prog.stats()["launches"] == 1


def qkv_rope_cache_graph(t, paged, norm, keep_members, E=1024, H=8, HKV=2, hd=128, n_ctx=64, bs=16, nblk=8):
    """[RMS_NORM -> MUL ->] Q / K / V at one column, RoPE (mode 0) of Q and K,
    then the K / V cache writes: dense f16 caches by SET_ROWS (Q stays f32), or
    one paged-cache write of f16 casts (Q cast to f16 too), as the decoder step
    builds them. keep_members keeps the three projections, which the store
    epilogue fusion then refuses: the same graph runs piece by piece."""
    b = G.Builder()
    ekv = HKV * hd
    x = b.input(N.F32, [E, 1])
    pos = b.input(N.I32, [1])
    slots = b.input(N.I32, [2]) if paged else b.input(N.I64, [1])
    nw = b.weight(N.F32, [E])
    wq, wk, wv = b.weight(t, [E, E]), b.weight(t, [E, ekv]), b.weight(t, [E, ekv])
    cur = b.mul(b.rms_norm(x, 1e-5), nw) if norm else x
    qm, km, vm = b.mul_mat(wq, cur), b.mul_mat(wk, cur), b.mul_mat(wv, cur)
    rope = lambda a, h: b.rope_ext(b.reshape(a, hd, h, 1), pos, None, hd, 0, 4096, 500000.0, 1.0, 0.0, 1.0, 32.0,  # noqa: E731
                                   1.0)
    q, k = rope(qm, H), rope(km, HKV)
    if paged:
        n = nblk * HKV * hd * bs
        kc, vc = b.state(N.F16, [n]), b.state(N.F16, [n])
        q = b.cast(q, N.F16)
        b.expand(q)
        b.expand(b.paged_cache_write(b.cast(b.reshape(k, ekv, 1), N.F16), b.cast(vm, N.F16), kc, vc, slots, bs, HKV))
        cache_bytes = 2 * n
    else:
        kc, vc = b.state(N.F16, [ekv, n_ctx]), b.state(N.F16, [ekv, n_ctx])
        b.expand(b.set_rows(kc, b.reshape(k, ekv, 1), slots))
        b.expand(b.set_rows(vc, vm, slots))
        b.expand(q)
        cache_bytes = 2 * ekv * n_ctx
    keep = [q] + ([qm, km, vm] if keep_members else [])
    return b, keep, q, cache_bytes, (E, ekv)


@pytest.mark.parametrize("t", [N.Q4_K, N.Q8_0, N.Q6_K], ids=lambda t: N.TYPE_NAMES[t])
@pytest.mark.parametrize("paged,norm,slot", [(False, True, 5), (False, False, 63), (True, True, 3 * 16 + 7),
                                             (True, False, 0), (True, True, -1)],
                         ids=["dense-norm", "dense", "paged-norm", "paged", "paged-skip"])
def test_qkv_rope_cache_epilogue_is_one_launch(gpu, t, paged, norm, slot):
    """The Q / K / V projection of a decode step with its RoPE and cache writes
    (SET_ROWS into dense caches, or the one-token paged write, whose negative
    slot writes nothing) runs as one register-GEMV launch, and its Q and caches
    are bit-identical to the same graph launched piece by piece."""
    import torch

    from tensorlisp_amd import synth

    outs = []
    for keep_members in (False, True):
        b, keep, q, cache_bytes, (E, ekv) = qkv_rope_cache_graph(t, paged, norm, keep_members)
        nwh = (1.0 + 0.1 * synth.normal(91, (E,))).astype(np.float32)
        ws = [dev(nwh)] + [dev(synth.random_blocks(t, 92 + i, M, E)) for i, M in enumerate((E, ekv, ekv))]
        state = torch.zeros(2 * cache_bytes, dtype=torch.uint8, device="cuda")
        prog = G.Program(b, keep, ws, [0, cache_bytes])
        prog.write_input(0, dev(synth.normal(95, (1, E)) * 2 + 0.1))
        prog.write_input(1, dev(np.array([37], np.int32)))
        prog.write_input(2, dev(np.array([slot], np.int64).view(np.int32) if paged else np.array([slot], np.int64)))
        prog.run(state)
        got_q = prog.read(q, torch.int16 if paged else torch.float32, state)
        torch.cuda.synchronize()
        outs.append((got_q.cpu().numpy().copy(), state.cpu().numpy().copy(), prog.stats()["launches"]))
    (fq, fs, fl), (uq, us, ul) = outs
    np.testing.assert_array_equal(fq, uq)
    np.testing.assert_array_equal(fs, us)
    assert fl == 1 and ul > 1, (fl, ul)
    if slot < 0:
        assert not fs.any()
    else:
        assert fs.any()


@pytest.mark.parametrize("n", [8192, 4100])
def test_inplace_add_feeding_norm(gpu, n):
    """An in-place ADD (ggml_add_inplace: the sum overwrites src0) feeding
    RMS_NORM -> MUL(weight) on rows longer than the fused kernel's register
    cache: the fused chain would read the row's tail from the overwritten src0,
    so the ADD keeps its own launch. Results equal the core ops run one by one
    and the reference backend running the same graph."""
    import torch

    from tensorlisp_amd import synth

    b = G.Builder()
    p = b.input(N.F32, [n, 2])
    q = b.input(N.F32, [n, 2])
    w = b.weight(N.F32, [n])
    s = b.add_inplace(p, q)
    y = b.mul(b.rms_norm(s, 1e-5), w)
    b.expand(y)
    wn = synth.normal(71, (n,))
    pn, qn = synth.normal(72, (2, n)) * 2 + 0.5, synth.normal(73, (2, n))
    prog = G.Program(b, [y, s], [dev(wn)])
    prog.write_input(0, dev(pn))
    prog.write_input(1, dev(qn))
    prog.run()
    sv = N.add(dev(pn), dev(qn))
    want = N.mul(N.norm(sv, 1e-5, rms=True), dev(wn))
    got = prog.read(y, torch.float32).reshape(want.shape)
    got_s = prog.read(s, torch.float32).reshape(sv.shape)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
    np.testing.assert_array_equal(got_s.cpu().numpy(), sv.cpu().numpy())
    ry, rs = ref().ir_run(b, [wn], [], [pn.copy(), qn], [(y, np.float32), (s, np.float32)])
    np.testing.assert_array_equal(got_s.cpu().numpy().reshape(rs.shape), rs)
    np.testing.assert_allclose(got.cpu().numpy().reshape(ry.shape), ry, rtol=1e-6, atol=1e-7)


def test_argmax_of_a_vocabulary(gpu):
    """ARGMAX over 128256 logits runs in chunks over many workgroups in a
    program; the last index of equal maxima wins, as on the CPU."""
    import torch

    from tensorlisp_amd import synth

    b = G.Builder()
    lg = b.input(N.F32, [128256, 4])
    am = b.argmax(lg)
    b.expand(am)
    prog = G.Program(b, [am], [])
    x = synth.normal(64, (4, 128256))
    x[1, 5] = x[1, 70000] = x[1, 128255] = 50.0
    x[2, :] = 1.0
    x[3, 2047:2049] = 60.0  # a tie across the chunk boundary
    prog.write_input(0, dev(x))
    prog.run()
    got = prog.read(am, torch.int32).cpu().numpy().reshape(-1)
    np.testing.assert_array_equal(got, oracle().core_argmax(x))
    assert list(got[1:]) == [128255, 128255, 2048]


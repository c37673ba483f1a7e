"""GPU parity of configs[4]'s run shape -- a 512-token prefill, then decode --
on the 8B decoder slice through the executor, against the reference CPU
backend on the same graphs (the reference's pattern: native executor against
the CPU backend, crates/tensorlisp/tests/native.rs:61-70, over the llama layer
of stdlib/nn.ss:23-43 and attn.ss:74-101).

The slice is refs.decoder_8b_slice_config (hidden 4096, 32 / 8 heads of 128,
FFN 14336, vocab 128256, RoPE theta 500000, every matrix q4_K) cut to two
layers. The steps are refs.prefill_8b_steps: a 512-token prompt, a 64-token
chunk at position 512, then two single-token steps; and, over a paged cache,
the same prompt and two decode steps (refs.prefill_8b_paged_steps). At more
than 16 tokens every MUL_MAT takes the prefill lowering: the norm chain
quantizing for the GEMM, one q4_K GEMM launch over the merged Q/K/V rows and
one over the merged gate/up rows, the SwiGLU quantizing for the down
projection's GEMM, per-token RoPE into the cache, and the 64-row
FLASH_ATTN_EXT form; the launch trace (tlh_program_trace) shows each ran.

Tolerances. Every MUL_MAT input is re-quantized to q8_K, so a layer's output
is chaotic in its rounding: on the CPU backend itself, flipping the last
mantissa bit of random elements of a layer's input either moves the output by
~1e-5 or, once one q8_K code flips (a block maximum changes every code of its
block), by a mean of 0.02-0.03 at a scale of 20-30
(test_executor.py::test_8b_layer_rounding_cascade_on_the_cpu). No GPU sum
order can stay under that floor, so the bar is the CPU's own spread: the
reference runs each graph with its attention's P.V accumulated in f32 (the
cached values read through an f32 cast) and again in f16 (the CPU backend's
default, ops.cpp:8617-8632), and the fixture keeps the first run's outputs and
how far the second moves them (largest, mean, and largest per-row mean
|difference|). The GPU accumulates in f32; a layer fed the reference's own
input must give the reference's output
  * with a mean |error| no larger than the mean distance between the CPU's two
    runs (a wrong row, index or term moves many elements by far more),
  * with no row's mean |error| above 1.5 x the CPU's largest per-row mean (a
    single wrong row or token position),
  * with no element further than 1.25 x the CPU's largest distance, or 8e-3 of
    the output's largest magnitude, whichever is larger.
The head fed the reference's last residual row must match within 1e-3 of the
largest |logit| (the north star's MUL_MAT bound). Free-running logits stay
within 1.25 x the CPU's own spread plus 8e-3 of the largest |logit|; the
argmax must agree wherever the reference's top-two margin exceeds twice the
measured error."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import (PREFILL_8B_SAMPLE, decoder_8b_slice_config, decoder_8b_weights, decoder_step_inputs, embed_rows,
                  prefill_8b_paged_steps, prefill_8b_steps, prefill_8b_tokens)
from tensorlisp_amd import graph as G

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden" / "decoder_8b_prefill.npz"
TOL = 8e-3


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def slice8b():
    c = decoder_8b_slice_config()
    w = decoder_8b_weights(c)
    return c, w, [dev(x) for x in w]


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def argmax_agrees(got_am, want_logits, err, what):
    idx = np.argsort(-want_logits, kind="stable")[:8]
    val = want_logits[idx]
    margin = float(val[0] - val[1])
    if margin > 2 * err:
        assert got_am == idx[0], (what, got_am, idx[0], margin, err)
    else:  # a near tie in the reference: the GPU's pick must be one of the tied ones
        tied = idx[val >= val[0] - 2 * err]
        assert got_am in tied, (what, got_am, tied, margin, err)


def layer_close(got, want, spread, stats, what):
    """A layer's output against the reference's, fed the reference's input
    (stats: the CPU's f16-vs-f32 P.V distance: mean, 99.9th percentile and
    largest per-row mean)."""
    scale = float(np.abs(want).max())
    d = np.abs(got - want)
    err, mean, q999, row = float(d.max()), float(d.mean()), float(np.quantile(d, 0.999)), float(d.mean(axis=1).max())
    print(f"[8b prefill] {what}: max err {err:.3e} mean {mean:.3e} q99.9 {q999:.3e} row mean {row:.3e} "
          f"(scale {scale:.3e}; CPU f16 vs f32 P.V max {spread:.3e} mean {stats[0]:.3e} q99.9 {stats[1]:.3e} "
          f"row mean {stats[2]:.3e})", flush=True)
    assert mean <= max(float(stats[0]), 1e-5 * scale), (what, mean, stats)
    assert row <= max(1.5 * float(stats[2]), 1e-5 * scale), (what, row, stats)
    assert err <= max(TOL * scale, 1.25 * spread), (what, err, scale, spread)
    return err


def free_close(got, want, spread, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    print(f"[8b prefill] {what}: max err {err:.3e} (scale {scale:.3e}; CPU f16 vs f32 P.V {spread:.3e})", flush=True)
    assert err <= 1.25 * spread + TOL * scale, (what, err, scale, spread)
    return err


def head_close(got, want, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    print(f"[8b prefill] {what}: max err {err:.3e} (scale {scale:.3e})", flush=True)
    assert err <= 1e-3 * scale, (what, err, scale)
    return err


def count(trace, label):
    return sum(labels.count(label) for _, labels in trace)


def f16(rows):
    return rows.view(np.float16).astype(np.float32)


def dense_state(c, g, torch):
    """The reference's cache rows (after the last step) in a dense state buffer."""
    offs, total = c.state_bytes()
    init = np.zeros(total, np.uint8)
    for j in range(2 * c.n_layer):
        rows = g[f"cache{j}"]
        init[offs[j]:offs[j] + rows.nbytes] = rows.view(np.uint8).reshape(-1)
    return offs, torch.from_numpy(init).cuda()


def cache_rows(c, s, offs, j, p0, n):
    per = c.n_embd_kv * c.n_ctx * 2
    return s[offs[j]:offs[j] + per].view(np.uint16).reshape(c.n_ctx, c.n_embd_kv)[p0:p0 + n]


def test_8b_prefill_layers_teacher_forced(gpu, slice8b, gold):
    """Each layer of each step alone, fed the reference's residual stream over
    the reference's cache rows; then the head fed the reference's last row."""
    import torch

    c, w, wd = slice8b
    g = gold
    for i, step in enumerate(prefill_8b_steps()):
        toks, p0, n_kv, _ = step
        T_ = len(toks)
        pos = np.arange(T_, dtype=np.int32) + p0
        inputs = [embed_rows(c, w, toks), g[f"tap{i}_1"]]
        for layer in range(c.n_layer):
            offs, state = dense_state(c, g, torch)
            ls = G.decoder_layer_step(c, layer, T_, n_kv)
            prog = G.Program(ls.builder, ls.keep, wd, offs)
            for k, a in enumerate([inputs[layer], pos, pos.astype(np.int64), G.causal_mask(pos, n_kv)]):
                prog.write_input(k, dev(a))
            trace = prog.trace(state)  # one eager run, recording its launches
            got = prog.read(ls.out, torch.float32, state).cpu().numpy().reshape(T_, c.n_embd)
            if i == 0:
                # the prefill lowering: one GEMM each for the merged Q/K/V, the
                # output projection, the merged gate/up and the down projection,
                # the 64-row flash attention, no GEMV
                print(f"[8b prefill] step 0 layer {layer} launches: {[l for _, ls_ in trace for l in ls_]}", flush=True)
                assert count(trace, "gemm_q4k") == 4, trace
                assert count(trace, "flash_attn_ext (rows)") == 1, trace
                assert count(trace, "gemv") + count(trace, "gemv_mfma") + count(trace, "gemv_cols") == 0, trace
            if layer == 0:
                want, rows = g[f"tap{i}_1"], slice(None)
            elif i == 0:
                want, rows = g["tap0_2s"], PREFILL_8B_SAMPLE
            else:
                want, rows = g[f"tap{i}_2"], slice(None)
            layer_close(got[rows], want, float(g[f"tfspread{i}_{layer}"]), g[f"tfstats{i}_{layer}"],
                        f"step {i} ({T_} tokens at {p0}) layer {layer}")
            s = state.cpu().numpy()
            for kv in (2 * layer, 2 * layer + 1):  # the rows this step writes
                gr, wr = f16(cache_rows(c, s, offs, kv, p0, T_)), f16(g[f"cache{kv}"][p0:p0 + T_])
                err, scale = float(np.abs(gr - wr).max()), float(np.abs(wr).max())
                print(f"[8b prefill] step {i} layer {layer} cache {kv} rows: max err {err:.3e} (scale {scale:.3e})",
                      flush=True)
                assert err <= TOL * scale, (i, layer, kv, err, scale)
        last = g["tap0_2s"][-1:] if i == 0 else g[f"tap{i}_2"][-1:]
        hs = G.decoder_head_step(c, 1)
        prog = G.Program(hs.builder, hs.keep, wd, [])
        prog.write_input(0, dev(last))
        prog.run()
        lg = prog.read(hs.out, torch.float32).cpu().numpy().reshape(-1)
        am = int(prog.read(hs.argmax, torch.int32).cpu().numpy().reshape(-1)[0])
        err = head_close(lg, g[f"logits{i}"], f"step {i} head (teacher-forced)")
        argmax_agrees(am, g[f"logits{i}"], max(err, 1e-6), f"step {i} head")


def test_8b_prefill_free_running(gpu, slice8b, gold):
    """The whole slice over the four steps (the decode steps as hipGraph
    replays), from an empty cache: logits, argmax and the cache rows."""
    import torch

    c, _, wd = slice8b
    g = gold
    offs, total = c.state_bytes()
    state = torch.zeros(total, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for i, step in enumerate(prefill_8b_steps()):
        toks, p0, n_kv, _ = step
        st = G.decoder_step(c, len(toks), n_kv)
        prog = G.Program(st.builder, st.keep, wd, offs)
        graph = len(toks) == 1
        stream = torch.cuda.Stream() if graph else None
        for k, a in enumerate(decoder_step_inputs(step)):
            prog.write_input(k, dev(a), stream)
        if i == 0:
            trace = prog.trace(state)
            assert count(trace, "gemm_q4k") == 4 * c.n_layer, trace
            assert count(trace, "flash_attn_ext (rows)") == c.n_layer, trace
            print(f"[8b prefill] 512-token step: {len(trace)} dispatches, "
                  f"{sum(len(x) for _, x in trace)} launches", flush=True)
        else:
            prog.run(state, stream, graph)
        lg = prog.read(st.logits, torch.float32, state, stream)
        am = prog.read(st.argmax, torch.int32, state, stream)
        torch.cuda.synchronize()
        lg, am = lg.cpu().numpy().reshape(-1), int(am.cpu().numpy().reshape(-1)[0])
        err = free_close(lg, g[f"logits{i}"], float(g[f"spread{i}"]), f"step {i} ({len(toks)} tokens at {p0})")
        argmax_agrees(am, g[f"logits{i}"], err, f"step {i}")
        assert lg[am] == lg.max()
    s = state.cpu().numpy()
    rows = len(g["cache0"])
    for j in range(2 * c.n_layer):
        gr, wr = f16(cache_rows(c, s, offs, j, 0, rows)), f16(g[f"cache{j}"])
        err, scale = float(np.abs(gr - wr).max()), float(np.abs(wr).max())
        tol = TOL if j < 2 else 0.05  # layer 1's rows carry layer 0's free-running error
        print(f"[8b prefill] cache {j} ({rows} rows): max err {err:.3e} (scale {scale:.3e})", flush=True)
        assert err <= tol * scale, (j, err, scale)


def to_pool(rows, table, c, pc, kpool, vpool, p0=0):
    """Dense f16 cache rows (K, V) [n, kvh * hd] of one sequence, from position
    p0, into vLLM's pool layouts (keys [blocks, kvh, hd / 8, bs, 8], values
    [blocks, kvh, hd, bs])."""
    k, v = rows
    kvh, hd, bs = c.n_head_kv, c.head_dim, pc.block_size
    for r in range(len(k)):
        p = p0 + r
        b, o = table[p // bs], p % bs
        kpool[b, :, :, o, :] = k[r].reshape(kvh, hd // 8, 8)
        vpool[b, :, :, o] = v[r].reshape(kvh, hd)


def from_pool(table, n, c, pc, kpool, vpool):
    """The inverse of to_pool for positions 0..n-1."""
    kvh, hd, bs = c.n_head_kv, c.head_dim, pc.block_size
    k = np.zeros((n, kvh * hd), np.uint16)
    v = np.zeros((n, kvh * hd), np.uint16)
    for p in range(n):
        b, o = table[p // bs], p % bs
        k[p] = kpool[b, :, :, o, :].reshape(-1)
        v[p] = vpool[b, :, :, o].reshape(-1)
    return k, v


def pool_views(c, pc, buf, offs, layer):
    kvh, hd, bs = c.n_head_kv, c.head_dim, pc.block_size
    n = pc.pool_bytes(c)
    kp = buf[offs[2 * layer]:offs[2 * layer] + n].view(np.uint16).reshape(pc.n_blocks, kvh, hd // 8, bs, 8)
    vp = buf[offs[2 * layer + 1]:offs[2 * layer + 1] + n].view(np.uint16).reshape(pc.n_blocks, kvh, hd, bs)
    return kp, vp


def test_8b_prefill_paged(gpu, slice8b, gold):
    """The 512-token prompt through the paged prefill graph (keys and values
    into the pools by paged-cache-write), then two decode steps with the
    paged-attention node: the prompt's pools equal the dense run's cache rows
    bit for bit; logits against the reference; and each paged decode layer fed
    the reference's residual row over pools holding the reference's rows."""
    import torch

    c, w, wd = slice8b
    g = gold
    prompt, _, _ = prefill_8b_tokens()
    T_ = len(prompt)
    pc = G.PagedConfig(block_size=16, n_blocks=48, max_blocks=40)
    table = [int(b) for b in np.random.default_rng(12).permutation(pc.n_blocks)[:34]]
    poffs, ptotal = pc.state_bytes(c)
    pools = torch.zeros(ptotal, dtype=torch.uint8, device="cuda")
    # the dense run of the same prompt, for its cache rows
    offs, total = c.state_bytes()
    dstate = torch.zeros(total, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    step0 = prefill_8b_steps()[0]
    st = G.decoder_step(c, T_, T_)
    prog = G.Program(st.builder, st.keep, wd, offs)
    for k, a in enumerate(decoder_step_inputs(step0)):
        prog.write_input(k, dev(a))
    prog.run(dstate)

    pos = np.arange(T_, dtype=np.int32)
    ps = G.decoder_prefill_paged(c, pc, T_)
    prog = G.Program(ps.builder, ps.keep, wd, poffs)
    for k, a in enumerate([np.array(prompt, np.int32), pos, G.paged_slots(table, pos, pc.block_size),
                           G.causal_mask(pos, T_)]):
        prog.write_input(k, dev(a))
    trace = prog.trace(pools)
    assert count(trace, "gemm_q4k") == 4 * c.n_layer, trace
    assert count(trace, "flash_attn_ext (rows)") == c.n_layer, trace
    # the prompt's keys and values reach the pools from the Q / K / V GEMM's
    # reduce (its store epilogue also writes the rotated Q, the f16 K and V
    # rows the attention reads): no RoPE, cast or cache-write launch of their own
    assert count(trace, "partial_reduce (epilogue)") == c.n_layer, trace
    assert count(trace, "reshape_and_cache") == 0 and not any(op in ("ROPE", "CPY") for op, _ in trace), trace
    lg = prog.read(ps.logits, torch.float32, pools).cpu().numpy().reshape(-1)
    am = int(prog.read(ps.argmax, torch.int32, pools).cpu().numpy().reshape(-1)[0])
    err = free_close(lg, g["logits0"], float(g["spread0"]), "paged prefill (512 tokens)")
    argmax_agrees(am, g["logits0"], err, "paged prefill")
    pb, ds = pools.cpu().numpy(), dstate.cpu().numpy()
    for layer in range(c.n_layer):
        k, v = from_pool(table, T_, c, pc, *pool_views(c, pc, pb, poffs, layer))
        for h, got in ((0, k), (1, v)):
            want = cache_rows(c, ds, offs, 2 * layer + h, 0, T_)
            diff = int(np.count_nonzero(got != want))
            print(f"[8b prefill] paged layer {layer} {'kv'[h]} pool vs dense cache: {diff} f16 values differ", flush=True)
            assert diff == 0, (layer, h, diff)

    # decode steps, free-running from the GPU's own pools
    tab = np.zeros((1, pc.max_blocks), np.int32)
    tab[0, :len(table)] = table
    for k, (toks, p0, _, _) in enumerate(prefill_8b_paged_steps()):
        p = np.array([p0], np.int32)
        dst = G.decoder_decode_paged(c, pc, 1)
        prog = G.Program(dst.builder, dst.keep, wd, poffs)
        stream = torch.cuda.Stream() if k == 1 else None
        for i, a in enumerate([np.array(toks, np.int32), p, G.paged_slots(table, p, pc.block_size), tab, p + 1]):
            prog.write_input(i, dev(a), stream)
        prog.run(pools, stream, graph=k == 1)
        lg = prog.read(dst.logits, torch.float32, pools, stream)
        am = prog.read(dst.argmax, torch.int32, pools, stream)
        torch.cuda.synchronize()
        lg, am = lg.cpu().numpy().reshape(-1), int(am.cpu().numpy().reshape(-1)[0])
        err = free_close(lg, g[f"plogits{k}"], float(g[f"pspread{k}"]), f"paged decode {k} (position {p0})")
        argmax_agrees(am, g[f"plogits{k}"], err, f"paged decode {k}")

    # each paged decode layer, teacher-forced: pools hold the reference's rows
    # 0..511 (and row 512 for the second step), input the reference's row
    for k, (toks, p0, _, _) in enumerate(prefill_8b_paged_steps()):
        p = np.array([p0], np.int32)
        for layer in range(c.n_layer):
            buf = np.zeros(ptotal, np.uint8)
            for ly in range(c.n_layer):
                kp, vp = pool_views(c, pc, buf, poffs, ly)
                to_pool((g[f"cache{2 * ly}"][:512], g[f"cache{2 * ly + 1}"][:512]), table, c, pc, kp, vp)
                if k == 1:
                    to_pool((g[f"pcache{2 * ly}"][:1], g[f"pcache{2 * ly + 1}"][:1]), table, c, pc, kp, vp, 512)
            pst = dev(buf)
            ls = G.decoder_layer_decode_paged(c, pc, layer, 1)
            prog = G.Program(ls.builder, ls.keep, wd, poffs)
            for i, a in enumerate([g[f"ptap{k}_{layer}"], p, G.paged_slots(table, p, pc.block_size), tab, p + 1]):
                prog.write_input(i, dev(a))
            prog.run(pst)
            got = prog.read(ls.out, torch.float32, pst).cpu().numpy().reshape(1, c.n_embd)
            layer_close(got, g[f"ptap{k}_{layer + 1}"], float(g[f"ptfspread{k}_{layer}"]), g[f"ptfstats{k}_{layer}"],
                        f"paged decode {k} layer {layer}")
            kp, vp = pool_views(c, pc, pst.cpu().numpy(), poffs, layer)
            kr, vr = from_pool(table, p0 + 1, c, pc, kp, vp)
            for h, got_row in ((0, kr[p0:]), (1, vr[p0:])):
                want = f16(g[f"pcache{2 * layer + h}"][k:k + 1])
                e, scale = float(np.abs(f16(got_row) - want).max()), float(np.abs(want).max())
                print(f"[8b prefill] paged decode {k} layer {layer} {'kv'[h]} row: max err {e:.3e} "
                      f"(scale {scale:.3e})", flush=True)
                assert e <= TOL * scale, (k, layer, h, e, scale)

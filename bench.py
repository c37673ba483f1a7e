#!/usr/bin/env python3
"""Benchmark of the quantized decode hot path on one MI355X.

Workload: the decode GEMV sweep at 8B-class shapes,
Q4_0 and Q4_K weights, batch 1 and 8:
  M x K in 4096x4096, 6144x4096, 14336x4096, 4096x14336, 128256x4096.
One "step" is one pass over all 20 (type, shape, N) GGML_OP_MUL_MAT nodes,
each through the C ABI (activation quantization + GEMV) on its own stream
order. Weights are resident in HBM before timing and every node rotates over
enough distinct weight copies (>= 640 MB per node) that no launch finds its
weights in the 256 MB Infinity Cache (MALL) or L2.

value  = whole-sweep algorithmic bytes (M*row_bytes + N*K*4 + N*M*4 per node)
         / wall time of the timed steps, GB/s.
roofline = the GEMV kernel of the sweep's heaviest node: its algorithmic bytes
         (weights, the activation it reads, f32 outputs) / its mean duration
         (HIP events on the launch stream around a run of back-to-back
         launches), against 8 TB/s. A node above N = 2 is a quantize launch
         and the GEMV; the GEMV is timed alone.
cpu_baseline = the reference's own ggml CPU backend (oracle/_ref, compiled from
         the reference sources) on the same sweep, timed on this host's cores
         the GPU box allots the job (16), with the host's CPU model and count;
         and its decode token rate on the same 8B model over a few steps.
Also reported: configs[4] end to end through the executor -- Llama-3-8B
shapes, random q4_K weights including the lm_head, paged KV cache, batch 1
(the headline decode tokens/s) and batch 16 -- plus the dense-cache batch-1
path with a q6_K lm_head; an 8B bs=1 token rate counting only the sweep's
matmuls; the q4_K prefill GEMM alone and as the whole node with
its quantize launch; paged-attention decode; dense
FLASH_ATTN_EXT decode (32 sequences x 4096 keys) and a causal 512-token prefill.

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tokens/sec (8B Q4_K, bs=1) + quant GEMV HBM GB/s (% of 8 TB/s)"
HBM_PEAK_GBS = 8000.0
SHAPES = [(4096, 4096), (6144, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]
ROTATE_BYTES = 640 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gpu_blocks(torch, wtype, M, K, gen):
    """Structurally valid random weight blocks generated on the GPU (finite f16 scales)."""
    from tensorlisp_amd import native as N

    be, bb = N.BLOCK[wtype]
    nb = M * (K // be)
    raw = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device="cuda", generator=gen)
    nscale = 2 if wtype == N.Q4_K else 1
    d = (torch.randn((nb, nscale), device="cuda", generator=gen).abs() * (0.02 / 63)).to(torch.float16)
    if wtype == N.Q6_K:  # d is the block's last field
        raw[:, bb - 2:] = d.view(torch.uint8).reshape(nb, 2)
    else:
        raw[:, : 2 * nscale] = d.view(torch.uint8).reshape(nb, 2 * nscale)
    return raw.reshape(M, (K // be) * bb)


def decoder_weights_gpu(torch, gen, c):
    """Random weights of the decoder `c` on the GPU, in weight-index order: RMS
    norm weights 1 + 0.1 N(0,1); q4_K matrices drawn zero-mean (synth's
    q4_K_model_blocks distribution, so that greedy decoding does not collapse
    onto one token); other quantized types as structurally valid random blocks."""
    from tensorlisp_amd import native as N
    from tensorlisp_amd import synth

    W = []
    for _, ty, ne in c.weight_shapes():
        if ty == N.F32:
            W.append(1.0 + 0.1 * torch.randn(ne[0], device="cuda", generator=gen))
        elif ty == N.Q4_K:
            W.append(synth.q4_K_model_blocks_gpu(torch, gen, ne[1], ne[0]))
        else:
            W.append(gpu_blocks(torch, ty, ne[1], ne[0], gen))
    return W


def e2e_decoder(torch, gen, prefill_tokens=512, decode_steps=256, eager_steps=32, cpu_steps=0):
    """configs[4] as BASELINE states it, through the executor (tlh_program_*):
    Llama-3-8B shapes with random q4_K weights (token embedding, every matrix
    and the lm_head), a 512-token prefill, then greedy decode steps over the
    paged KV cache at batch 1 (the headline) and batch 16. Labelled extra: the
    dense f16 cache (FLASH_ATTN_EXT) at batch 1 with a q6_K lm_head, as
    Q4_K_M files have. cpu_steps > 0: ggml's CPU backend runs that many
    decode steps of the same model (dense cache) for a CPU token rate."""
    import dataclasses

    from tensorlisp_amd import native as N

    from tensorlisp_amd import graph as G

    c = G.DecoderConfig(n_ctx=1024, out_type=N.Q4_K)
    W = decoder_weights_gpu(torch, gen, c)
    weight_bytes = sum(w.numel() * w.element_size() for w in W)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()  # the weights (default stream) before `stream` uses them
    copy = lambda dst, src, n: N.check(N.lib().tlh_copy(dst, src, n, N._stream(stream)))  # noqa: E731
    out = {"model": "Llama-3-8B shapes: 32 layers, hidden 4096, 32/8 heads x 128, SwiGLU 14336, vocab 128256, "
                    "RoPE 500000; random q4_K weights (token embedding, matrices, lm_head)"}
    for batch in (1, 16):
        out[f"paged_bs{batch}"] = e2e_decoder_paged(torch, gen, c, W, weight_bytes, stream, copy, prefill_tokens,
                                                    decode_steps, batch=batch, eager_steps=eager_steps)
    if cpu_steps > 0:
        out["cpu_decode"] = cpu_decode(c, W, cpu_steps)
        out["cpu_decode_fast"] = cpu_decode(c, W, cpu_steps, fast=True)
    c6 = dataclasses.replace(c, out_type=N.Q6_K)
    W[-1] = gpu_blocks(torch, N.Q6_K, c.n_vocab, c.n_embd, gen)
    out["dense_bs1_q6k_lm_head"] = e2e_decoder_dense(torch, gen, c6, W, stream, copy, prefill_tokens, decode_steps,
                                                     eager_steps)
    del W
    torch.cuda.empty_cache()
    return out


def cpu_decode(c, W, steps, fast=False):
    """Decode token rate of ggml's CPU backend (oracle/_ref, compiled from the
    reference's sources) on the same model: `steps` single-token greedy steps
    of the dense-cache decode graph at positions 0.. (the CPU backend cannot
    run the paged-attention nodes), each a ggml_graph_compute over the whole
    8B model, on the threads the GPU box allots this job. fast: the fastest
    ISA build of the same sources this host runs (x86-64-v4 / v3, ggml's SIMD
    paths; labelled, not the parity build)."""
    import dataclasses

    import numpy as np

    sys.path.insert(0, str(ROOT / "tests"))
    import refs

    from tensorlisp_amd import graph as G

    r, isa = refs.ref_fast() if fast else (refs.ref(), None)
    if r is None:
        return None
    threads = cpu_threads()
    cc = dataclasses.replace(c, n_ctx=max(64, steps + 1))
    hw = [w.cpu().numpy() for w in W]
    states = [np.zeros((cc.n_ctx, cc.n_embd_kv), np.uint16) for _ in range(2 * cc.n_layer)]
    st = G.decoder_step(cc, 1, cc.n_ctx)
    tok, total = 1, 0.0
    for i in range(steps + 1):  # the first step (page-ins) untimed
        ins = [np.array([tok], np.int32), np.array([i], np.int32), np.array([i], np.int64),
               G.causal_mask([i], cc.n_ctx)]
        t0 = time.perf_counter()
        _, am = r.ir_run(st.builder, hw, states, ins, [(st.logits, np.float32), (st.argmax, np.int32)],
                         nthreads=threads)
        if i > 0:
            total += time.perf_counter() - t0
        tok = int(am.reshape(-1)[0])
    del hw
    res = {"tokens_per_s": round(steps / total, 2), "ms_per_token": round(total / steps * 1e3, 1), "steps": steps,
           "threads": threads, "kind": "reference",
           "build": f"-march=x86-64-{isa} (SIMD paths)" if fast else "no -march (the parity build: scalar paths)",
           "sample": f"{steps} single-token greedy decode steps at positions 1..{steps} (after one untimed step), "
                     "dense f16 cache, the same random q4_K weights; ggml_graph_compute wall time per step"}
    log(f"  cpu decode (ggml CPU backend, {res['build']}, {threads} threads): {res['tokens_per_s']} tok/s "
        f"over {steps} steps")
    return res


def e2e_decoder_dense(torch, gen, c, W, stream, copy, prefill_tokens=512, decode_steps=256, eager_steps=32):
    """Batch 1 with the dense f16 caches written with SET_ROWS and read with
    FLASH_ATTN_EXT: a 512-token prefill, then greedy decode steps whose next
    token is the previous step's argmax, copied on the device into the next
    step's input (no host round trip). Decode attends a cache view padded to
    768 rows (the mask hides the rows not yet written) so one program, captured
    once as a hipGraph, serves every step."""
    import numpy as np

    from tensorlisp_amd import graph as G

    weight_bytes = sum(w.numel() * w.element_size() for w in W)
    offs, total = c.state_bytes()
    state = torch.zeros(total, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()  # the zeroed state (default stream) before `stream` uses it

    # prefill: 512 tokens at positions 0..511, logits of the last one
    T = prefill_tokens
    pre = G.decoder_step(c, T, T)
    P = G.Program(pre.builder, pre.keep, W, offs)
    toks = torch.randint(0, c.n_vocab, (T,), device="cuda", generator=gen, dtype=torch.int32)
    pos = torch.arange(T, device="cuda", dtype=torch.int32)
    mask = torch.from_numpy(G.causal_mask(np.arange(T), T).view(np.int16)).cuda()
    with torch.cuda.stream(stream):
        for i, a in enumerate((toks, pos, pos.to(torch.int64), mask)):
            P.write_input(i, a, stream)
    P.run(state, stream)  # warm
    stream.synchronize()
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        P.run(state, stream, graph=True)
    stream.synchronize()
    prefill_ms = (time.perf_counter() - t0) / reps * 1e3

    # decode: one token a step at positions 512.., over a 768-row cache view
    n_kv = 768
    dec = G.decoder_step(c, 1, n_kv)
    D = G.Program(dec.builder, dec.keep, W, offs)
    steps = decode_steps
    dpos = torch.arange(T, T + steps, device="cuda", dtype=torch.int32)
    dslot = dpos.to(torch.int64)
    dmask = torch.from_numpy(G.causal_mask(np.arange(T, T + steps), n_kv).view(np.int16)).cuda()
    inp = [D.input(i)[0] for i in range(4)]
    am_dec = D.tensor_ptr(dec.argmax, state)
    am_pre = P.tensor_ptr(pre.argmax, state)

    def run_decode(n, graph):
        copy(inp[0], am_pre, 4)  # the prompt's greedy token starts the decode
        for i in range(n):
            copy(inp[1], dpos.data_ptr() + 4 * i, 4)
            copy(inp[2], dslot.data_ptr() + 8 * i, 8)
            copy(inp[3], dmask.data_ptr() + 2 * n_kv * i, 2 * n_kv)
            D.run(state, stream, graph)
            copy(inp[0], am_dec, 4)

    run_decode(4, True)  # capture and warm
    stream.synchronize()
    t0 = time.perf_counter()
    run_decode(steps, True)
    stream.synchronize()
    graph_ms = (time.perf_counter() - t0) / steps * 1e3
    t0 = time.perf_counter()
    run_decode(eager_steps, False)
    stream.synchronize()
    eager_ms = (time.perf_counter() - t0) / eager_steps * 1e3
    kv_bytes = 2 * c.n_layer * n_kv * c.n_embd_kv * 2  # every cache row the padded view attends
    tok_bytes = weight_bytes - W[0].numel() + c.n_embd * 2 + kv_bytes  # embedding: one row
    out = {
        "lm_head": "q6_K", "kv_cache": "dense f16, FLASH_ATTN_EXT over a 768-row view",
        "batch": 1, "prefill_tokens": T, "decode_steps": steps,
        "prefill_ms": round(prefill_ms, 2), "prefill_tokens_per_s": round(T / prefill_ms * 1e3, 1),
        "decode_ms_per_token_hipgraph": round(graph_ms, 4), "decode_tokens_per_s": round(1e3 / graph_ms, 1),
        "decode_ms_per_token_eager": round(eager_ms, 4),
        "decode_bytes_per_token": tok_bytes, "decode_gbs": round(tok_bytes / graph_ms / 1e6, 1),
        "decode_frac_of_hbm_peak": round(tok_bytes / graph_ms / 1e6 / HBM_PEAK_GBS, 4),
        "dispatches_per_decode_step": D.stats()["launches"],
    }
    log(f"  e2e 8B q4_K dense cache, q6_K lm_head: prefill {T} tok {prefill_ms:.1f} ms "
        f"({out['prefill_tokens_per_s']} tok/s); decode {graph_ms:.3f} ms/tok graph, {eager_ms:.3f} eager -> "
        f"{out['decode_tokens_per_s']} tok/s, {out['decode_gbs']} GB/s")
    del P, D, state
    return out


def e2e_decoder_paged(torch, gen, c, W, weight_bytes, stream, copy, prefill_tokens=512, decode_steps=256,
                      batch=16, block_size=16, eager_steps=32):
    """configs[4] at `batch` sequences with the paged KV cache: each sequence's
    512-token prompt runs alone (keys and values into the pools through
    paged-cache-write, attention over the prompt with FLASH_ATTN_EXT), then
    all sequences decode together, one token each per step, through the
    paged-attention node; each step's next tokens are the previous step's
    argmax, copied on the device (no host round trip). Blocks of a sequence
    are a random draw from the pool. The decode program is captured once as a
    hipGraph and replayed every step."""
    import numpy as np

    from tensorlisp_amd import graph as G

    S, T, steps = batch, prefill_tokens, decode_steps
    per_seq = (T + steps + block_size - 1) // block_size
    pc = G.PagedConfig(block_size=block_size, n_blocks=S * per_seq, max_blocks=per_seq)
    offs, total = pc.state_bytes(c)
    state = torch.zeros(total, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()  # the zeroed pools (default stream) before `stream` uses them
    rng = np.random.default_rng(4)
    tables = rng.permutation(pc.n_blocks).astype(np.int32).reshape(S, per_seq)

    pre = G.decoder_prefill_paged(c, pc, T)
    P = G.Program(pre.builder, pre.keep, W, offs)
    pos = np.arange(T, dtype=np.int32)
    mask = torch.from_numpy(G.causal_mask(pos, T).view(np.int16)).cuda()
    toks = torch.randint(0, c.n_vocab, (S, T), device="cuda", generator=gen, dtype=torch.int32)
    first = torch.empty(S, dtype=torch.int32, device="cuda")
    slots = [torch.from_numpy(G.paged_slots(tables[s], pos, block_size)).cuda() for s in range(S)]
    pin = [P.input(i)[0] for i in range(4)]
    am_pre = P.tensor_ptr(pre.argmax, state)
    with torch.cuda.stream(stream):
        P.write_input(1, torch.from_numpy(pos).cuda(), stream)
        P.write_input(3, mask, stream)

    def prefill_all(graph):
        for s in range(S):
            copy(pin[0], toks[s].data_ptr(), 4 * T)
            copy(pin[2], slots[s].data_ptr(), 8 * T)
            P.run(state, stream, graph)
            copy(first.data_ptr() + 4 * s, am_pre, 4)

    prefill_all(True)  # capture and warm
    stream.synchronize()
    t0 = time.perf_counter()
    prefill_all(True)
    stream.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3

    dec = G.decoder_decode_paged(c, pc, S)
    D = G.Program(dec.builder, dec.keep, W, offs)
    dpos = T + np.arange(steps, dtype=np.int32)[:, None] + np.zeros((1, S), np.int32)
    dslots = np.stack([np.concatenate([G.paged_slots(tables[s], [p], block_size) for s, p in enumerate(row)])
                       for row in dpos])
    dpos_d, dlens_d = torch.from_numpy(dpos).cuda(), torch.from_numpy(dpos + 1).cuda()
    dslots_d = torch.from_numpy(np.ascontiguousarray(dslots)).cuda()
    din = [D.input(i)[0] for i in range(5)]
    am_dec = D.tensor_ptr(dec.argmax, state)
    with torch.cuda.stream(stream):
        D.write_input(3, torch.from_numpy(tables).cuda(), stream)

    def run_decode(n, graph):
        copy(din[0], first.data_ptr(), 4 * S)
        for i in range(n):
            copy(din[1], dpos_d.data_ptr() + 4 * S * i, 4 * S)
            copy(din[2], dslots_d.data_ptr() + 8 * S * i, 8 * S)
            copy(din[4], dlens_d.data_ptr() + 4 * S * i, 4 * S)
            D.run(state, stream, graph)
            copy(din[0], am_dec, 4 * S)

    run_decode(4, True)  # capture and warm (rewrites rows T..T+3, rewritten again below)
    stream.synchronize()
    t0 = time.perf_counter()
    run_decode(steps, True)
    stream.synchronize()
    step_ms = (time.perf_counter() - t0) / steps * 1e3
    t0 = time.perf_counter()
    run_decode(min(eager_steps, steps), False)
    stream.synchronize()
    eager_ms = (time.perf_counter() - t0) / min(eager_steps, steps) * 1e3
    # bytes a step reads: the weights once (one embedding row per sequence),
    # every sequence's keys and values
    kv_rows = S * (T + (steps - 1) / 2 + 1)
    step_bytes = weight_bytes - W[0].numel() + S * c.n_embd * 2 + 2 * c.n_layer * kv_rows * c.n_embd_kv * 2
    out = {
        "batch": S, "lm_head": "q4_K",
        "kv_cache": f"paged, block size {block_size}, {pc.n_blocks} blocks per layer drawn at random",
        "prefill_tokens_per_seq": T, "decode_steps": steps,
        "prefill_ms_all_seqs": round(prefill_ms, 1), "prefill_tokens_per_s": round(S * T / prefill_ms * 1e3, 1),
        "decode_ms_per_step_hipgraph": round(step_ms, 4), "decode_ms_per_step_eager": round(eager_ms, 4),
        "decode_tokens_per_s": round(S / step_ms * 1e3, 1),
        "decode_bytes_per_step": int(step_bytes), "decode_gbs": round(step_bytes / step_ms / 1e6, 1),
        "decode_frac_of_hbm_peak": round(step_bytes / step_ms / 1e6 / HBM_PEAK_GBS, 4),
        "dispatches_per_decode_step": D.stats()["launches"],
    }
    log(f"  e2e 8B q4_K paged, batch {S}: prefill {S}x{T} tok {prefill_ms:.1f} ms ({out['prefill_tokens_per_s']} "
        f"tok/s); decode {step_ms:.3f} ms/step graph, {eager_ms:.3f} eager -> {out['decode_tokens_per_s']} tok/s, "
        f"{out['decode_gbs']} GB/s")
    del P, D, state
    torch.cuda.empty_cache()
    return out


def gemv_vs_floor(torch, gen, stream, shapes, pool_bytes=1200 << 20, reps=50):
    """Cold N = 1 q4_K GEMV time (tlh_mul_mat, activation quantized in the
    kernel) beside a plain streaming read of the same weight bytes
    (tlh_read_floor, best of grids 256..4096 with 1 or 4 loads in flight per
    lane), both back to back over `reps` launches that rotate through copies
    in a 1.2 GB pool so no launch finds its bytes in MALL or L2; the launches
    are captured as one hipGraph and timed with events around its replay."""
    from tensorlisp_amd import native as N

    pool = torch.randint(0, 256, (pool_bytes,), dtype=torch.uint8, device="cuda", generator=gen)
    out = []

    def timed(fn):
        # the launches captured once as a graph and replayed: a Python loop of
        # launches would leave the GPU idle between kernels of a few us
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(3):
                fn(i, side)
            side.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for i in range(reps):
                    fn(i, torch.cuda.current_stream())
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(side)
            g.replay()
            e1.record(side)
        e1.synchronize()
        del g
        return e0.elapsed_time(e1) / reps * 1e3  # us

    for M, K in shapes:
        rb = N.row_bytes(N.Q4_K, K)
        nbytes = M * rb
        slot = (nbytes + 4095) // 4096 * 4096
        ncopy = min(64, pool_bytes // slot)
        w = [synth_q4k_into(torch, gen, pool, i * slot, M, K) for i in range(ncopy)]
        x = torch.randn((1, K), device="cuda", generator=gen)
        y = torch.empty((1, M), dtype=torch.float32, device="cuda")
        node = N.MulMat(N.Q4_K, M, K, 1)
        torch.cuda.synchronize()
        gemv_us = timed(lambda i, s: node(w[i % ncopy], x, y, s))
        floor = []
        for grid in (256, 512, 1024, 2048, 4096):
            for loads in (1, 4):
                us = timed(lambda i, s: N.check(N.lib().tlh_read_floor(
                    pool.data_ptr() + (i % ncopy) * slot, nbytes // 16 * 16, grid, loads, N._stream(s))))
                floor.append((us, grid, loads))
        f_us, f_grid, f_loads = min(floor)
        out.append({"M": M, "K": K, "weight_bytes": nbytes, "copies": ncopy, "gemv_us": round(gemv_us, 2),
                    "read_floor_us": round(f_us, 2), "floor_grid": f_grid, "floor_loads_per_lane": f_loads,
                    "gemv_gbs": round(nbytes / gemv_us / 1e3, 1), "floor_gbs": round(nbytes / f_us / 1e3, 1)})
        log(f"  cold q4_K GEMV {M:6d}x{K:<5d}: {gemv_us:6.2f} us vs read floor {f_us:6.2f} us "
            f"(grid {f_grid}, {f_loads} load(s)/lane)")
    del pool
    torch.cuda.empty_cache()
    return out


def synth_q4k_into(torch, gen, pool, offset, M, K):
    """A [M, row_bytes] uint8 view of `pool` at `offset` holding random q4_K
    blocks with small finite f16 scales."""
    from tensorlisp_amd import native as N

    rb = N.row_bytes(N.Q4_K, K)
    w = pool[offset:offset + M * rb].view(M, rb)
    blk = w.view(M * (K // 256), 144)
    d = (torch.rand((blk.shape[0], 2), device="cuda", generator=gen) * 1e-3 + 1e-4).to(torch.float16)
    blk[:, :4] = d.view(torch.uint8).reshape(-1, 4)
    return w


def algorithmic_bytes(wtype, M, K, n):
    from tensorlisp_amd import native as N

    return M * N.row_bytes(wtype, K) + n * K * 4 + n * M * 4


def cpu_threads() -> int:
    """Threads for the CPU legs: the cores the GPU box allots a one-GPU job
    (OMP_NUM_THREADS there, 16), never more than the host has."""
    n = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or 16
    return max(1, min(n, os.cpu_count() or 1))


def cpu_model() -> str:
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(host_weights, cases, seconds: float, fast: bool = False):
    """The reference's ggml CPU backend (oracle/_ref) on the same sweep; falls back to
    our C port of it (oracle/liboracle.so) where the reference was not built.
    fast: the fastest ISA build of the same sources this host runs (None if
    there is none)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np

    import refs

    threads = cpu_threads()
    r, isa = refs.ref_fast() if fast else (refs.ref(), None)
    if fast and r is None:
        return None
    kind = "reference" if r is not None else "port"
    xs = {c: np.random.default_rng(1).standard_normal((c[3], c[2])).astype(np.float32) for c in cases}
    total_bytes, total_s, passes = 0, 0.0, 0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or passes == 0:
        for c in cases:
            t, M, K, n = c
            if r is not None:
                _, s = r.mul_mat(t, host_weights[(t, M, K)], M, K, xs[c], nthreads=threads)
            else:
                t0 = time.perf_counter()
                refs.oracle().mul_mat(t, host_weights[(t, M, K)], M, K, xs[c], nthreads=threads)
                s = time.perf_counter() - t0
            total_s += s
            total_bytes += algorithmic_bytes(t, M, K, n)
        passes += 1
    return {"value": total_bytes / total_s / 1e9, "unit": "GB/s", "cores": threads, "kind": kind,
            "build": f"-march=x86-64-{isa} (ggml's SIMD paths; labelled fast build)" if fast
            else "no -march (the parity build: ggml's scalar _ref/_generic paths, as the reference's cc build)",
            "host": {"cpu_model": cpu_model(), "nproc": os.cpu_count(), "threads_used": threads},
            "sample": f"{passes} pass(es) of the full 20-node sweep (same shapes, N in 1,8), "
                      f"ggml_graph_compute wall time, {threads} threads (the cores the GPU box allots a one-GPU "
                      f"job; the host reports {os.cpu_count()} CPUs, {cpu_model()}), {total_s:.1f} s"}


FLOOR_SHAPES = [(4096, 4096), (6144, 4096), (14336, 4096), (4096, 14336), (28672, 4096), (128256, 4096)]


def copy_scale_kernel(torch):
    """A plain device copy of known size (256 MiB): the scale for rocprof's
    FETCH_SIZE / WRITE_SIZE counters when profiles/ derive HBM traffic per
    launch."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def run_prefill(torch, gen, stream):
    """the q4_K prefill GEMM on 14336x4096 and 4096x14336 at N = 512
    and 2048, the GEMM launch alone and the whole MUL_MAT node with its
    quantize launch, HIP events on the stream, weights rotated."""
    from tensorlisp_amd import native as N

    # prefill GEMM: q4_K 14336x4096 and 4096x14336, N = 512 / 2048, GEMM kernel
    # alone (the activation quantization runs first as its own phase), rotated weights
    prefill = []
    for (M, K) in ((14336, 4096), (4096, 14336)):
        base = gpu_blocks(torch, N.Q4_K, M, K, gen)
        ws = [base] + [base.clone() for _ in range(max(1, math.ceil(ROTATE_BYTES / base.numel())) - 1)]
        for n in (512, 2048):
            node = N.MulMat(N.Q4_K, M, K, n)
            x = torch.randn((n, K), device="cuda", generator=gen)
            y = torch.empty((n, M), dtype=torch.float32, device="cuda")
            node.quantize(x, stream)
            for i in range(2):
                node.compute(ws[i % len(ws)], y, stream)
            reps = 6
            evs = []
            for i in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                node.compute(ws[i % len(ws)], y, stream)
                e1.record(stream)
                evs.append((e0, e1))
            # the whole MUL_MAT node: the Q8_K quantize launch, then the GEMM
            nevs = []
            for i in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                node(ws[i % len(ws)], x, y, stream)
                e1.record(stream)
                nevs.append((e0, e1))
            torch.cuda.synchronize()
            ms = sum(a.elapsed_time(b) for a, b in evs) / reps
            node_ms_p = sum(a.elapsed_time(b) for a, b in nevs) / reps
            tflops = 2.0 * M * n * K / (ms * 1e-3) / 1e12
            node_tflops = 2.0 * M * n * K / (node_ms_p * 1e-3) / 1e12
            prefill.append({"M": M, "K": K, "N": n, "us": round(ms * 1e3, 1), "tflops": round(tflops, 1),
                            "frac_of_int8_mfma_peak": round(tflops / 5000.0, 4),
                            "frac_of_f16_mfma_peak": round(tflops / 2500.0, 4),
                            "node_us_incl_quantize": round(node_ms_p * 1e3, 1),
                            "node_tflops": round(node_tflops, 1)})
            log(f"  prefill q4_K {M}x{K} N={n}: GEMM {ms * 1e3:8.1f} us  {tflops:7.1f} TFLOP/s; node with its "
                f"quantize launch {node_ms_p * 1e3:8.1f} us  {node_tflops:7.1f} TFLOP/s")
        del ws, base
    torch.cuda.empty_cache()

    return prefill


def run_q6_lm_head(torch, gen, stream):
    from tensorlisp_amd import native as N

    # q6_K output projection (the lm_head of Q4_K_M files), 128256 x 4096, N = 1 and 8
    q6 = []
    base = gpu_blocks(torch, N.Q6_K, 128256, 4096, gen)
    ws = [base] + [base.clone() for _ in range(max(1, math.ceil(ROTATE_BYTES / base.numel())) - 1)]
    for n in (1, 8):
        node = N.MulMat(N.Q6_K, 128256, 4096, n)
        x = torch.randn((n, 4096), device="cuda", generator=gen)
        y = torch.empty((n, 128256), dtype=torch.float32, device="cuda")
        for i in range(2):
            node(ws[i % len(ws)], x, y, stream)
        evs = []
        for i in range(10):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            node(ws[i % len(ws)], x, y, stream)
            e1.record(stream)
            evs.append((e0, e1))
        torch.cuda.synchronize()
        ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
        b = algorithmic_bytes(N.Q6_K, 128256, 4096, n)
        q6.append({"M": 128256, "K": 4096, "N": n, "us": round(ms * 1e3, 1), "gbs": round(b / ms / 1e6, 1),
                   "frac_of_hbm_peak": round(b / ms / 1e6 / HBM_PEAK_GBS, 4)})
        log(f"  q6_K  128256x4096  n={n}: {ms * 1e3:8.1f} us  {b / ms / 1e6:7.0f} GB/s")
    del ws, base
    torch.cuda.empty_cache()

    return q6


def run_attention(torch, gen, stream):
    """configs[3] paged-attention decode, and dense FLASH_ATTN_EXT decode and
    causal prefill. The inputs come from a generator of their own (seed 3), so
    `--only attention` (the profiles' command) and the full run draw the same
    context lengths and pages."""
    from tensorlisp_amd import native as N

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)

    # paged-attention decode: 32 sequences, 32 q / 8 kv heads, hs 128, 16-token
    # pages scattered over a 65,536-page pool (2 GiB per cache), lens ~ U[512, 8192]
    seqs, heads, kvh, hs, bs, pool = 32, 32, 8, 128, 16, 65536
    lens = torch.randint(512, 8193, (seqs,), device="cuda", generator=gen, dtype=torch.int32)
    maxb = 8192 // bs
    kc = torch.randn((pool, kvh, hs // 8, bs, 8), device="cuda", generator=gen, dtype=torch.float16)
    vc = torch.randn((pool, kvh, hs, bs), device="cuda", generator=gen, dtype=torch.float16)
    tables = torch.randperm(pool, device="cuda", generator=gen)[: seqs * maxb].to(torch.int32).reshape(seqs, maxb)
    qa = torch.randn((seqs, heads, hs), device="cuda", generator=gen, dtype=torch.float16)
    oa = torch.empty_like(qa)
    pa = N.PagedAttention(seqs, heads, kvh, hs, bs, maxb, 8192, hs ** -0.5)
    lsum = int(lens.sum().item())
    pages = int(((lens + bs - 1) // bs).sum().item())
    attn_bytes = lsum * kvh * hs * 2 * 2 + 2 * seqs * heads * hs * 2 + pages * 4 + seqs * 4
    for _ in range(2):
        pa(oa, qa, kc, vc, tables, lens, stream)
    evs = []
    for _ in range(10):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        pa(oa, qa, kc, vc, tables, lens, stream)
        e1.record(stream)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    attn_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    attn_gbs = attn_bytes / attn_ms / 1e6
    attention = {"seqs": seqs, "heads": heads, "kv_heads": kvh, "head_size": hs, "block_size": bs,
                 "context_tokens": lsum, "bytes": attn_bytes, "us": round(attn_ms * 1e3, 1),
                 "gbs": round(attn_gbs, 1), "frac_of_hbm_peak": round(attn_gbs / HBM_PEAK_GBS, 4)}
    log(f"  paged attention {seqs} seqs, {lsum} tokens: {attn_ms * 1e3:8.1f} us  {attn_gbs:7.0f} GB/s")
    del kc, vc
    torch.cuda.empty_cache()

    # dense FLASH_ATTN_EXT decode: the same 32 sequences x 32 q / 8 kv heads x 128 with a
    # per-sequence f16 cache of 4096 keys (ggml k/v [128, 4096, 8, 32]), one query each;
    # and a causal 512-token prefill of one sequence (q [128, 512, 32, 1], mask [512, 512])
    fa = {}
    for name, nb, nq, L, causal in (("decode", 32, 1, 4096, False), ("prefill_causal", 1, 512, 512, True)):
        fq = torch.randn((nb, heads, nq, hs), device="cuda", generator=gen, dtype=torch.float32)
        fk = torch.randn((nb, kvh, L, hs), device="cuda", generator=gen, dtype=torch.float16)
        fv = torch.randn((nb, kvh, L, hs), device="cuda", generator=gen, dtype=torch.float16)
        fm = None
        if causal:
            fm = torch.full((nq, L), float("-inf"), device="cuda").triu(1 + L - nq).to(torch.float16)[None, None]
            fm = fm.contiguous()
        fo = torch.empty((nb, nq, heads, hs), device="cuda", dtype=torch.float32)
        node = N.FlashAttnExt(fq, fk, fv, fm, fo, hs ** -0.5)
        for _ in range(2):
            node(fq, fk, fv, fm, fo, stream)
        evs = []
        for _ in range(10):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            node(fq, fk, fv, fm, fo, stream)
            e1.record(stream)
            evs.append((e0, e1))
        torch.cuda.synchronize()
        fms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
        fbytes = nb * kvh * L * hs * 2 * 2 + 2 * nb * nq * heads * hs * 4 + (nq * L * 2 if causal else 0)
        # QK and PV over the (query, key) pairs the mask leaves live: query i of
        # a causal mask sits at position L - nq + i and sees L - nq + i + 1 keys
        live = sum(min(L, L - nq + i + 1) for i in range(nq)) if causal else nq * L
        flops = 4.0 * nb * heads * live * hs
        fa[name] = {"batch": nb, "queries": nq, "keys": L, "heads": heads, "kv_heads": kvh, "head_size": hs,
                    "causal_mask": causal, "bytes": fbytes, "us": round(fms * 1e3, 1),
                    "gbs": round(fbytes / fms / 1e6, 1), "frac_of_hbm_peak": round(fbytes / fms / 1e6 / HBM_PEAK_GBS, 4),
                    "tflops": round(flops / (fms * 1e-3) / 1e12, 1)}
        log(f"  flash_attn_ext {name}: {fms * 1e3:8.1f} us  {fbytes / fms / 1e6:7.0f} GB/s  "
            f"{flops / (fms * 1e-3) / 1e12:6.1f} TFLOP/s")
        del fq, fk, fv, fm, fo, node
    torch.cuda.empty_cache()

    return attention, fa


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["sweep", "floor", "prefill", "attention", "e2e"], default=None,
                    help="run one part and print its JSON (for profiler runs); the default runs everything and "
                         "prints the bench line")
    ap.add_argument("--e2e-only", action="store_true",
                    help="run only the end-to-end 8B decoder (configs[4]) and print its JSON")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--cpu-decode-steps", type=int, default=8,
                    help="decode steps of the 8B model on ggml's CPU backend for the CPU token rate (0: skip)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from tensorlisp_amd import native as N

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    props = N.device_props(0)
    log(f"device {props['name']} {props['arch']} CUs={props['compute_units']}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    only = "e2e" if args.e2e_only else args.only
    if only == "e2e":
        print(json.dumps(e2e_decoder(torch, gen, decode_steps=args.decode_steps,
                                     cpu_steps=0 if args.no_cpu else args.cpu_decode_steps)), flush=True)
        return 0
    if only == "floor":
        print(json.dumps(gemv_vs_floor(torch, gen, torch.cuda.current_stream(), FLOOR_SHAPES)), flush=True)
        return 0
    if only == "prefill":
        print(json.dumps(run_prefill(torch, gen, torch.cuda.current_stream())), flush=True)
        return 0
    if only == "attention":
        att, fa = run_attention(torch, gen, torch.cuda.current_stream())
        copy_scale_kernel(torch)
        print(json.dumps({"paged_attention_decode": att, "flash_attn_ext": fa}), flush=True)
        return 0

    cases = [(t, M, K, n) for t in (N.Q4_0, N.Q4_K) for (M, K) in SHAPES for n in (1, 8)]
    weights, nodes, xs, ys, bytes_per = {}, {}, {}, {}, {}
    for t in (N.Q4_0, N.Q4_K):
        for (M, K) in SHAPES:
            base = gpu_blocks(torch, t, M, K, gen)
            copies = max(2, math.ceil(ROTATE_BYTES / base.numel()))
            weights[(t, M, K)] = [base] + [base.clone() for _ in range(copies - 1)]
    for c in cases:
        t, M, K, n = c
        nodes[c] = N.MulMat(t, M, K, n)
        xs[c] = torch.randn((n, K), device="cuda", generator=gen)
        ys[c] = torch.empty((n, M), dtype=torch.float32, device="cuda")
        bytes_per[c] = algorithmic_bytes(t, M, K, n)
    torch.cuda.synchronize()
    log(f"setup: {len(cases)} nodes, {sum(w[0].numel() * len(w) for w in weights.values()) / 2**30:.1f} GiB "
        "of rotated weights resident")

    stream = torch.cuda.current_stream()
    ev = {c: [] for c in cases}

    def step(i: int, record: bool) -> None:
        # one MUL_MAT node per case through tlh_mul_mat (activation quantization fused
        # into the GEMV when N*K is small, else a quantize launch + the GEMV); with
        # `record`, HIP events on the launch stream bracket each node
        for c in cases:
            t, M, K, _ = c
            ws = weights[(t, M, K)]
            if record:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
            nodes[c](ws[i % len(ws)], xs[c], ys[c], stream)
            if record:
                e1.record(stream)
                ev[c].append((e0, e1))

    for i in range(args.warmup):
        step(i, False)
    torch.cuda.synchronize()
    log(f"warmup: {args.warmup} steps")

    # wall-clock timed region: exactly K steps, synchronized on both sides
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i, False)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    log(f"timed: {args.steps} steps in {wall * 1e3:.1f} ms")

    # per-node durations (a separate pass, events around each node; a fused node is one kernel)
    for i in range(args.steps):
        step(args.warmup + args.steps + i, True)
    torch.cuda.synchronize()
    node_ms = {c: sum(a.elapsed_time(b) for a, b in ev[c]) / len(ev[c]) for c in cases}
    for c in cases:
        t, M, K, n = c
        log(f"  {N.TYPE_NAMES[t]:5s} {M:6d}x{K:<5d} n={n}: {node_ms[c] * 1e3:8.1f} us  "
            f"{bytes_per[c] / node_ms[c] / 1e6:7.0f} GB/s")

    sweep_bytes = sum(bytes_per.values())
    value = sweep_bytes * args.steps / wall / 1e9

    # the roofline kernel: the GEMV of the sweep's heaviest node. A node at
    # N <= 2 is one launch (the GEMV quantizes its activation itself); above,
    # the node is a quantize launch and the GEMV, timed here alone (events on
    # the launch stream around back-to-back compute launches, the activation
    # quantized once before)
    dom = max(cases, key=lambda c: node_ms[c])
    dt, dM, dK, dn = dom
    if dn <= 2:
        # one launch a node: back-to-back launches (weights rotated) between
        # one pair of events, as for the GEMV launch below
        node = nodes[dom]
        ws = weights[(dt, dM, dK)]
        reps = max(args.steps, 20)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # one untimed launch ahead of e0 keeps the GPU busy while the host
        # issues the first timed one, so the interval holds no host latency
        node(ws[-1], xs[dom], ys[dom], stream)
        e0.record(stream)
        for i in range(reps):
            node(ws[i % len(ws)], xs[dom], ys[dom], stream)
        e1.record(stream)
        torch.cuda.synchronize()
        dom_ms = e0.elapsed_time(e1) / reps
        dom_bytes = bytes_per[dom]
        dom_kernel = (f"{N.TYPE_NAMES[dt]} GEMV N={dn}, {dM}x{dK}, activation quantized in the kernel "
                      "(tlh::k_gemv_reg), the node's one launch")
    else:
        node = nodes[dom]
        ws = weights[(dt, dM, dK)]
        node.quantize(xs[dom], stream)
        # back-to-back compute launches (weights rotated) between one pair of
        # events: the average launch duration on the stream, without a
        # dispatch latency in every sample (nor the first one's)
        reps = max(args.steps, 20)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        node.compute(ws[-1], ys[dom], stream)  # untimed, as above
        e0.record(stream)
        for i in range(reps):
            node.compute(ws[i % len(ws)], ys[dom], stream)
        e1.record(stream)
        torch.cuda.synchronize()
        dom_ms = e0.elapsed_time(e1) / reps
        # the compute launch reads the weights and the quantized activation, writes f32 rows
        dom_bytes = dM * N.row_bytes(dt, dK) + dn * N.row_bytes(N.VEC_DOT_TYPE[dt], dK) + dn * dM * 4
        # tall matrices with K <= 4096 take the few-column form whose waves own
        # whole 16-row groups (gemv_cols_ok in gemv_mfma.hip)
        kname = ("tlh::k_gemv_cols" if dM // 16 >= 4096 and dK <= 4096 and dK % 256 == 0
                 else "tlh::k_gemv_mfma")
        dom_kernel = (f"{N.TYPE_NAMES[dt]} GEMV N={dn}, {dM}x{dK}: the GEMV launch of the MUL_MAT node "
                      f"({kname}), after its quantize launch; node incl. quantize "
                      f"{node_ms[dom] * 1e3:.1f} us")
    dom_gbs = dom_bytes / dom_ms / 1e6
    log(f"roofline kernel: {dom_kernel}: {dom_ms * 1e3:.1f} us, {dom_gbs:.0f} GB/s")
    # matmul-only decode token rate of an 8B Llama with Q4_K weights at bs = 1
    q = lambda M, K: node_ms[(N.Q4_K, M, K, 1)]  # noqa: E731
    tok_ms = 32 * (q(6144, 4096) + q(4096, 4096) + 2 * q(14336, 4096) + q(4096, 14336)) + q(128256, 4096)

    # the decode GEMV shapes cold, beside a plain streaming read of the same bytes
    if only == "sweep":  # the sweep and its roofline kernel alone (for counter runs), then the copy scale
        copy_scale_kernel(torch)
        print(json.dumps({"value_gbs": round(value, 2), "roofline_kernel": dom_kernel, "us": round(dom_ms * 1e3, 2),
                          "gbs": round(dom_gbs, 1)}), flush=True)
        return 0
    floor = gemv_vs_floor(torch, gen, stream, FLOOR_SHAPES)

    prefill = run_prefill(torch, gen, stream)
    q6 = run_q6_lm_head(torch, gen, stream)
    attention, fa = run_attention(torch, gen, stream)
    e2e = e2e_decoder(torch, gen, decode_steps=args.decode_steps,
                      cpu_steps=0 if args.no_cpu else args.cpu_decode_steps)

    copy_scale_kernel(torch)

    # HBM bytes per launch of the roofline kernel, as measured by the rocprofv3 PMC runs
    # summarised in profiles/ (FETCH_SIZE / WRITE_SIZE scaled by a copy of known size)
    traffic = None
    tfile = ROOT / "profiles" / "traffic.txt"
    if tfile.exists():
        for ln in tfile.read_text().splitlines():
            key, _, val = ln.partition("=")
            if key.strip() == f"gemv_{N.TYPE_NAMES[dt]}_{dM}x{dK}_n{dn}_bytes" and val.strip().isdigit():
                traffic = int(val.strip())

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline: ggml CPU backend on the same sweep (~{args.cpu_seconds:.0f} s)")
        host_w = {k: v[0].cpu().numpy() for k, v in weights.items()}
        cpu = cpu_baseline(host_w, cases, args.cpu_seconds)
        cpu["decode_8b_q4k"] = e2e.get("cpu_decode")
        log(f"cpu baseline: {cpu['value']:.1f} GB/s ({cpu['kind']}, {cpu['cores']} threads)")
        fast = cpu_baseline(host_w, cases, args.cpu_seconds, fast=True)
        if fast is not None:
            fast["decode_8b_q4k"] = e2e.get("cpu_decode_fast")
            log(f"cpu baseline, fast build: {fast['value']:.1f} GB/s ({fast['build']})")
        cpu["fast_build"] = fast

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "configs[1] decode GEMV sweep: {q4_0,q4_K} x {4096x4096, 6144x4096, 14336x4096, "
                        "4096x14336, 128256x4096} x N {1, 8}; GGML_OP_MUL_MAT incl. Q8_0/Q8_K activation "
                        "quantization; weights rotated over >= 640 MB of HBM copies per node",
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "decode_tokens_per_s_8b_q4k_bs1": e2e["paged_bs1"]["decode_tokens_per_s"],
            "e2e_decoder_8b_q4k": e2e,
            "decode_tokens_per_s_8b_q4k_bs1_matmul_only": round(1e3 / tok_ms, 1),
            "gemv_q4k_n1_cold_vs_read_floor": floor,
            "prefill_gemm_q4k": prefill,
            "gemv_q6k_lm_head": q6,
            "paged_attention_decode": attention,
            "flash_attn_ext": fa,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom_kernel,
            "us": round(dom_ms * 1e3, 2),
            "bytes": int(dom_bytes),
            "achieved": round(dom_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

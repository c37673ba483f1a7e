"""Writes the golden fixtures of this directory from the reference's own
compiled ggml CPU code (oracle/_ref/libggml_ref.so, built in place from
/root/reference by oracle/Makefile).

The reference commits no golden vectors (its tests compute expectations at run
time from ggml's CPU backend: crates/tensorlisp/tests/native.rs:61-107), so
these are the reference's outputs on fixed inputs, captured once:

  fp16.npz         ggml_fp16_to_fp32_row over all 65536 halves; ggml_fp32_to_fp16_row
                   over refs.fp16_probe_values() (every rounding boundary between
                   adjacent halves +-1 ulp, and a random sample over all exponents)
  quant.npz        ggml_quantize_chunk (q4_0, q8_0, q4_K; imatrix NULL, the path of
                   DType::from_f32, crates/tensorlisp/src/dtype.rs:98-124) and
                   dequantize_row_* on the same rows
  act.npz          quantize_row_q8_0 / quantize_row_q8_K (the x86 from_float of the
                   CPU mul_mat) on random and edge-case rows
  mul_mat.npz      one GGML_OP_MUL_MAT on the CPU backend for the reference test's
                   cases (native.rs:73-107: 96 x 256 weights from noise(seed 1),
                   x = noise(seed 10 + n), n in 1,3,5,8,9,40) per weight type
  q2_K.npz, q3_K.npz  as q5_K.npz for the two lowest k-quants
  decoder_lowk.npz the tiny decoder with a Q2_K model file's matrix types
                   (refs.decoder_lowk_config: q2_K embedding and matrices, q3_K value
                   and down projections and lm_head) over refs.LOWK_STEPS (decoder.npz's
                   steps plus a 20-token chunk) with P.V accumulated in f32: logits,
                   argmax, final caches, and how far the default f16 accumulation moves
                   the logits (largest and mean |difference|) and the caches
  legacy_quants.npz  q4_1, q5_0 and q5_1 (the reference test's other 32-element
                   types, native.rs:84): ggml_quantize_chunk of its 96 x 256 noise
                   matrix, dequantize_row_*, one GGML_OP_MUL_MAT per n in 1,3,5,8,9,40;
                   structurally random blocks (synth seeds 111, 121, 131) against x
                   (seed + 1, 3 x 1024); quantize_row_q8_1 (src1 of q4_1 / q5_1) on the
                   activation edge rows and random rows
  mul_mat_float.npz  the same cases with f32, f16 and bf16 weights (ggml_quantize_chunk
                   of the noise matrix), plus f16 / bf16 weights against src1 already
                   of the weight type and a ragged K = 100 (the element-wise path), and
                   attn:sdpa's non-flash graph on refs.SDPA_CASES (inputs regenerated
                   from seeds by refs.sdpa_inputs)
  config1.npz      BASELINE config 1 (Q8_0 4096 x 4096, N = 1, seed 0): input hashes
                   and the CPU backend's output vector
  flash_attn.npz   GGML_OP_FLASH_ATTN_EXT (ops.cpp:8468) on dense f16 K/V, the
                   dense-cache counterpart of paged attention
  q6_K.npz         q6_K weights from ggml_quantize_chunk on the reference test's
                   96 x 256 noise matrix (native.rs:73-107, the same inputs as
                   mul_mat.npz), their dequantize_row_q6_K, and one
                   GGML_OP_MUL_MAT per n in 1,3,5,8,9,40; plus structurally
                   random q6_K blocks (synth seed 61) against x (seed 62)
  q5_K.npz         the same for q5_K (random blocks: synth seed 71, x seed 72)
  flash_attn_ext.npz  GGML_OP_FLASH_ATTN_EXT with masks, GQA, batch, soft cap and
                   ALiBi on the shapes of the reference's attention tests
                   (refs.FA_CASES, native.rs:156-345), 8 CPU threads, outputs of the
                   first and last 6 queries; inputs are regenerated from the
                   stored seeds by refs.fa_case_inputs
  core.npz         the ops around them in a decoder step (add/sub/mul/div, every
                   unary op, norm/rms_norm, get_rows of every weight type,
                   set_rows, cpy, rope_ext normal/neox/YaRN, soft_max_ext,
                   argmax) on refs.core_cases(): the reference tests' shapes and
                   inputs (native.rs:109-498) and decoder-sized ones; inputs are
                   regenerated from seeds, the file keeps the outputs

  mul_mat_id.npz   GGML_OP_MUL_MAT_ID on refs.MMID_CASES (every weight type,
                   broadcast src1, K chunks, repeated experts) through the CPU
                   backend; inputs are regenerated from the stored seeds by
                   refs.mmid_case, the file keeps the outputs

  decoder_paged.npz  refs.PAGED_SEQS (three sequences: a prompt, then three
                   decode tokens) each alone through the dense-cache decoder
                   step on the CPU backend (refs.paged_ref_run): the logits
                   and argmax a batched paged decode must reproduce

  decoder.npz      a llama-style decoder step graph (tensorlisp_amd.graph.decoder_step,
                   refs.decoder_tiny_config: 2 layers, 4 heads of 64, 2 KV heads,
                   q4_K / q6_K weights from refs.decoder_weights) run on the CPU
                   backend for refs.DECODER_STEPS (a 5-token prompt, three
                   single-token steps, a 3-token chunk): logits and argmax per
                   step and the f16 KV caches after the last one

  decoder_8b.npz   BASELINE configs[4]'s decoder at its own shapes (hidden 4096, 32 / 8
                   heads of 128, FFN 14336, vocab 128256, every matrix q4_K) cut to two
                   layers (refs.decoder_8b_slice_config, weights refs.decoder_8b_weights):
                   logits, argmax and written cache rows of refs.DECODER_8B_STEPS on the
                   CPU backend with the attention's P.V accumulated in f32 (the cached
                   values read through an f32 cast), and the default run's logits
                   (f16 P.V accumulation) as f16; the residual stream after the
                   embedding and each layer, and each layer fed that stream with f16 P.V
                   accumulation; for refs.paged_8b_seqs, each sequence run alone, the
                   argmax and 8 largest logits of each step (f32 P.V) and how far the
                   two accumulations move that step's logits.
  decoder_8b_prefill.npz  the same slice over configs[4]'s run shape (refs.prefill_8b_steps: a
                   512-token prompt, a 64-token chunk at position 512, two single-token
                   steps), dense cache, P.V in f32: last-token logits per step and how far
                   the f16 P.V run moves them; the residual stream after layer 0 (all
                   rows) and after layer 1 (a row sample for the prompt, all rows for the
                   later steps); the cache rows after the last step; per layer, how far
                   f16 P.V accumulation moves that layer's output from the same input
                   (largest, mean, 99.9th percentile and largest per-row mean |difference|);
                   and the paged form's two decode steps after the same prompt
                   (refs.prefill_8b_paged_steps) with their logits, residual streams and
                   written cache rows.
Run: python tests/golden/make_golden.py [flash_attn_ext | q6_K | q5_K | core | decoder | decoder_paged | mul_mat_id | decoder_8b
     | decoder_8b_prefill | lowk | mul_mat_float | legacy_quants]   (needs oracle/_ref built)
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

from refs import (DECODER_8B_STEPS, decoder_8b_layer_ref, decoder_8b_ref_run, decoder_8b_slice_config,  # noqa: E402
                  decoder_8b_weights, paged_8b_ref)
from refs import PREFILL_8B_SAMPLE, decoder_8b_run_states, prefill_8b_paged_steps, prefill_8b_steps  # noqa: E402
from refs import SDPA_CASES, sdpa_graph, sdpa_inputs  # noqa: E402
from refs import Q4_1, Q5_0, Q5_1  # noqa: E402
from refs import LOWK_STEPS, Q2_K, Q3_K, decoder_lowk_config  # noqa: E402
from refs import (BF16, F16, F32, FA_CASES, MMID_CASES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, Ref, core_cases, core_ref, decoder_ref_run,  # noqa: E402
                  decoder_tiny_config, decoder_weights, fa_case_inputs, fp16_probe_values, mmid_case, paged_ref_run,
                  xorshift_noise)
from tensorlisp_amd import synth  # noqa: E402


def edge_rows_act(k: int) -> np.ndarray:
    """Rows that exercise the activation quantizers' corner cases."""
    rows = []
    rows.append(np.zeros(k, np.float32))  # all-zero blocks: d = 0
    rows.append(np.full(k, 0.37, np.float32))  # constant blocks
    r = synth.normal(101, (k,))
    r[::32] = 3.0
    r[16::32] = -3.0  # |max| ties with opposite signs: the first one wins (q8_K)
    rows.append(r)
    r = synth.normal(102, (k,))
    r[::256] = -5.0
    r[128::256] = 5.0
    rows.append(r)
    # codes landing exactly on .5 after scaling: amax 127 -> id = 1, x = n + 0.5
    r = (np.arange(k) % 64 - 32).astype(np.float32) + np.float32(0.5)
    r[::32] = 127.0
    rows.append(r)
    r = (np.arange(k) % 64 - 32).astype(np.float32) + np.float32(0.5)
    r[::256] = -127.0
    rows.append(r)
    rows.append(synth.normal(103, (k,)) * np.float32(1e-30))  # tiny: subnormal f16 d
    rows.append(synth.normal(104, (k,)) * np.float32(1e4))  # large
    r = synth.normal(105, (k,))
    r[32:64] = 0.0  # one zero block among others
    r[256:512] = 0.0
    rows.append(r)
    return np.stack(rows).astype(np.float32)


def flash_attn_ext_golden(ref) -> None:
    out = {}
    for i, case in enumerate(FA_CASES):
        seed = 500 + 10 * i
        q, k, v, m, scale, max_bias, softcap = fa_case_inputs(case, seed)
        o, _ = ref.flash_attn_ext(q, k, v, m, scale, max_bias, softcap, nthreads=8)
        nq = o.shape[1]
        rows = np.unique(np.r_[np.arange(min(nq, 6)), np.arange(max(nq - 6, 0), nq)])  # first and last queries
        out[f"{case[0]}/seed"] = np.array([seed])
        out[f"{case[0]}/rows"] = rows
        out[f"{case[0]}/out"] = o[:, rows]
    np.savez_compressed(HERE / "flash_attn_ext.npz", **out)


def kquant_golden(ref, t: int, name: str, wseed: int, xseed: int) -> None:
    rows, k = 96, 256
    wn = xorshift_noise((rows, k), 1)
    ns = [1, 3, 5, 8, 9, 40]
    q = ref.quantize_weights(t, wn)
    out = {"w": q, "deq": ref.dequantize(t, q, k), "ns": np.array(ns)}
    for n in ns:
        y, _ = ref.mul_mat(t, q, rows, k, xorshift_noise((n, k), 10 + n))
        out[f"y{n}"] = y
    M, K = 40, 1024
    wr = synth.random_blocks(t, wseed, M, K)
    xr = synth.normal(xseed, (3, K))
    y, _ = ref.mul_mat(t, wr, M, K, xr)
    out.update({"rand_w": wr, "rand_y": y, "rand_deq": ref.dequantize(t, wr, K)})
    np.savez_compressed(HERE / f"{name}.npz", **out)


def q6_K_golden(ref) -> None:
    kquant_golden(ref, Q6_K, "q6_K", 61, 62)


def q5_K_golden(ref) -> None:
    kquant_golden(ref, Q5_K, "q5_K", 71, 72)


def lowk_golden(ref) -> None:
    """q2_K.npz and q3_K.npz (as q5_K.npz), and decoder_lowk.npz: the tiny
    decoder with a Q2_K file's matrix types (refs.decoder_lowk_config) over
    refs.LOWK_STEPS on the CPU backend."""
    kquant_golden(ref, Q2_K, "q2_K", 81, 82)
    kquant_golden(ref, Q3_K, "q3_K", 91, 92)
    c = decoder_lowk_config()
    w = decoder_weights(c)
    logits, ams, caches = decoder_ref_run(ref, c, w, LOWK_STEPS, f32_values=True)
    lg16, _, c16 = decoder_ref_run(ref, c, w, LOWK_STEPS)
    out = {f"logits{i}": lg for i, lg in enumerate(logits)}
    out.update({f"argmax{i}": a for i, a in enumerate(ams)})
    out.update({f"cache{i}": s for i, s in enumerate(caches)})
    for i, (a, b) in enumerate(zip(logits, lg16)):
        d = np.abs(a - b)
        out[f"spread{i}"] = np.array([d.max(), d.mean()], np.float32)
    for j, (a, b) in enumerate(zip(caches, c16)):
        out[f"cspread{j}"] = np.float32(np.abs(ref.f16_to_f32(a) - ref.f16_to_f32(b)).max())
    np.savez_compressed(HERE / "decoder_lowk.npz", **out)


def legacy_quants_golden(ref) -> None:
    rows, k = 96, 256
    wn = xorshift_noise((rows, k), 1)
    ns = [1, 3, 5, 8, 9, 40]
    out = {"ns": np.array(ns)}
    for t, name, seed in ((Q4_1, "q4_1", 111), (Q5_0, "q5_0", 121), (Q5_1, "q5_1", 131)):
        q = ref.quantize_weights(t, wn)
        out[f"{name}_w"] = q
        out[f"{name}_deq"] = ref.dequantize(t, q, k)
        for n in ns:
            out[f"{name}_y{n}"] = ref.mul_mat(t, q, rows, k, xorshift_noise((n, k), 10 + n))[0]
        rw = synth.random_blocks(t, seed, 40, 1024)
        out[f"{name}_rand_w"] = rw
        out[f"{name}_rand_deq8"] = ref.dequantize(t, rw[:8], 1024)  # the first 8 rows
        out[f"{name}_rand_y"] = ref.mul_mat(t, rw, 40, 1024, synth.normal(seed + 1, (3, 1024)))[0]
    x = np.concatenate([edge_rows_act(1024), synth.normal(141, (6, 1024))]).astype(np.float32)
    out["act_x"] = x
    out["q8_1"] = ref.quantize_act(Q4_1, x)
    np.savez_compressed(HERE / "legacy_quants.npz", **out)


def mul_mat_float_golden(ref) -> None:
    rows, k = 96, 256
    wn = xorshift_noise((rows, k), 1)
    ns = [1, 3, 5, 8, 9, 40]
    out = {"ns": np.array(ns)}
    for t, name in ((F32, "f32"), (F16, "f16"), (BF16, "bf16")):
        wq = ref.quantize_weights(t, wn)
        out[f"{name}_w"] = wq
        for n in ns:
            y, _ = ref.mul_mat(t, wq, rows, k, xorshift_noise((n, k), 10 + n))
            out[f"{name}_y{n}"] = y
    # src1 already f16 / bf16 (the graph form ggml_mul_mat takes then), through
    # ref_ir_run: weights [k, rows], x [k, n] of the weight type
    from tensorlisp_amd import graph as G

    for t, name in ((F16, "f16"), (BF16, "bf16")):
        for n in (1, 9):
            b = G.Builder()
            w = b.weight(t, [k, rows])
            x = b.input(t, [k, n])
            y = b.mul_mat(w, x)
            b.expand(y)
            xq = ref.quantize_weights(t, xorshift_noise((n, k), 20 + n)).view(np.uint16)
            out[f"{name}_x{n}_same"] = xq
            out[f"{name}_y{n}_same"] = ref.ir_run(b, [out[f"{name}_w"].view(np.uint16)], [], [xq],
                                                  [(y, np.float32)])[0].reshape(n, rows)
    # K = 100: no multiple of 8 (the element-wise path)
    w100 = synth.normal(81, (33, 100))
    x100 = synth.normal(82, (5, 100))
    out["k100_x"] = x100
    for t, name in ((F32, "f32"), (F16, "f16"), (BF16, "bf16")):
        wq = ref.quantize_weights(t, w100)
        out[f"k100_{name}_w"] = wq
        out[f"k100_{name}_y"] = ref.mul_mat(t, wq, 33, 100, x100)[0]
    # attn:sdpa's non-flash graph (float MUL_MATs of K and V) on refs.SDPA_CASES
    for i, case in enumerate(SDPA_CASES):
        b, merged, _ = sdpa_graph(*case)
        out[f"sdpa{i}"] = ref.ir_run(b, [], [], sdpa_inputs(case, 300 + 10 * i), [(merged, np.float32)])[0]
    np.savez_compressed(HERE / "mul_mat_float.npz", **out)


def mul_mat_id_golden(ref) -> None:
    out = {}
    for case in MMID_CASES:
        b, y, w, inputs = mmid_case(case)
        (res,) = ref.ir_run(b, w, [], inputs, [(y, np.float32)])
        out[case[0]] = res
    np.savez_compressed(HERE / "mul_mat_id.npz", **out)


def decoder_paged_golden(ref) -> None:
    c = decoder_tiny_config()
    pl, pa, dl, da = paged_ref_run(ref, c, decoder_weights(c))
    np.savez_compressed(HERE / "decoder_paged.npz", prompt_logits=pl, prompt_argmax=pa, decode_logits=dl,
                        decode_argmax=da)


def core_golden(ref) -> None:
    np.savez_compressed(HERE / "core.npz", **{c["name"]: core_ref(ref, c) for c in core_cases()})


def decoder_golden(ref) -> None:
    c = decoder_tiny_config()
    logits, ams, caches = decoder_ref_run(ref, c, decoder_weights(c))
    out = {f"logits{i}": lg for i, lg in enumerate(logits)}
    out.update({f"argmax{i}": a for i, a in enumerate(ams)})
    out.update({f"cache{i}": s for i, s in enumerate(caches)})
    np.savez_compressed(HERE / "decoder.npz", **out)


def decoder_8b_golden(ref) -> None:
    """The 8B-shaped two-layer slice (refs.decoder_8b_slice_config) on the CPU
    backend, with f32 and with f16 P.V accumulation: logits and argmax of
    DECODER_8B_STEPS, the cache rows they write, the residual stream per layer
    (and each layer's output from it with the other accumulation), and the 16
    paged_8b_seqs sequences each run alone."""
    c = decoder_8b_slice_config()
    w = decoder_8b_weights(c)
    logits, ams, _, _ = decoder_8b_ref_run(ref, c, w)
    rows = max(p0 + len(t) for t, p0, _, _ in DECODER_8B_STEPS)
    # the default run's logits as f16 (they bound how far the CPU's own f16 P.V
    # accumulation moves the logits, a few percent; f16 keeps 3 decimal digits)
    out = {f"logits{i}": lg.astype(np.float16) for i, lg in enumerate(logits)}
    out.update({f"argmax{i}": a for i, a in enumerate(ams)})
    logits32, ams32, caches32, taps32 = decoder_8b_ref_run(ref, c, w, f32_values=True)
    out.update({f"logits_f32pv{i}": lg for i, lg in enumerate(logits32)})
    out.update({f"argmax_f32pv{i}": a for i, a in enumerate(ams32)})
    caches = [s[:rows] for s in caches32]
    out.update({f"cache{i}": s for i, s in enumerate(caches)})
    # the residual stream after the embedding and each layer (f32 P.V run), and
    # each layer fed that stream with f16 P.V accumulation instead (how far the
    # CPU's own two accumulations put one layer's output apart)
    for i, step in enumerate(DECODER_8B_STEPS):
        for layer in range(c.n_layer + 1):
            out[f"tap{i}_{layer}"] = taps32[i][layer]
        for layer in range(c.n_layer):
            out[f"tf16_{i}_{layer}"] = decoder_8b_layer_ref(ref, c, w, caches, step, layer, taps32[i][layer], False)
    am, ti, tv, spread = paged_8b_ref(ref, c, w)
    out.update(paged_argmax=am, paged_top_index=ti, paged_top_logit=tv, paged_spread=spread)
    np.savez_compressed(HERE / "decoder_8b.npz", **out)


def decoder_8b_prefill_golden(ref) -> None:
    """configs[4]'s run shape on the 8B slice: refs.prefill_8b_steps (a
    512-token prompt, a 64-token chunk, two single-token steps) on the CPU
    backend, dense cache, P.V accumulated in f32 and, again, in f16 (the
    backend's default); and the paged form's two decode steps after the same
    prompt (refs.prefill_8b_paged_steps)."""
    c = decoder_8b_slice_config()
    w = decoder_8b_weights(c)
    steps, psteps = prefill_8b_steps(), prefill_8b_paged_steps()
    zero = lambda: [np.zeros((c.n_ctx, c.n_embd_kv), np.uint16) for _ in range(2 * c.n_layer)]  # noqa: E731
    runs = {}
    for f32v in (True, False):
        st = zero()
        lg, taps = decoder_8b_run_states(ref, c, w, steps[:1], st, f32v)
        stp = [s.copy() for s in st]
        plg, ptaps = decoder_8b_run_states(ref, c, w, psteps, stp, f32v)
        lg2, taps2 = decoder_8b_run_states(ref, c, w, steps[1:], st, f32v)
        runs[f32v] = (lg + lg2, taps + taps2, st, plg, ptaps, stp)
        print(f"prefill_8b: f32 P.V {f32v} done", flush=True)
    lg, taps, st, plg, ptaps, stp = runs[True]
    lg16, plg16 = runs[False][0], runs[False][3]
    rows = max(p0 + len(t) for t, p0, _, _ in steps)
    out = {"tap0_0s": taps[0][0][:4], "tap0_1": taps[0][1], "tap0_2s": taps[0][2][PREFILL_8B_SAMPLE]}
    for i in range(len(steps)):
        out[f"logits{i}"] = lg[i].reshape(-1)
        d = np.abs(lg[i] - lg16[i])
        out[f"spread{i}"] = np.float32(d.max())
        out[f"spreadstats{i}"] = np.array([d.mean(), np.quantile(d, 0.999)], np.float32)
        if i:
            out[f"tap{i}_1"], out[f"tap{i}_2"] = taps[i][1], taps[i][2]
    for j in range(2 * c.n_layer):
        out[f"cache{j}"] = st[j][:rows]
        out[f"pcache{j}"] = stp[j][512:514]  # the rows the paged decode steps write
    caches = [s[:rows] for s in st]
    pcaches = [s[:514] for s in stp]
    for i, step in enumerate(steps):
        for layer in range(c.n_layer):
            tf = decoder_8b_layer_ref(ref, c, w, caches, step, layer, taps[i][layer], False)
            d = np.abs(tf - taps[i][layer + 1])
            out[f"tfspread{i}_{layer}"] = np.float32(d.max())
            out[f"tfstats{i}_{layer}"] = np.array([d.mean(), np.quantile(d, 0.999), d.mean(axis=1).max()], np.float32)
    for k, step in enumerate(psteps):
        out[f"plogits{k}"] = plg[k].reshape(-1)
        d = np.abs(plg[k] - plg16[k])
        out[f"pspread{k}"] = np.float32(d.max())
        out[f"pspreadstats{k}"] = np.array([d.mean(), np.quantile(d, 0.999)], np.float32)
        for layer in range(c.n_layer + 1):
            out[f"ptap{k}_{layer}"] = ptaps[k][layer]
        for layer in range(c.n_layer):
            tf = decoder_8b_layer_ref(ref, c, w, pcaches, step, layer, ptaps[k][layer], False)
            d = np.abs(tf - ptaps[k][layer + 1])
            out[f"ptfspread{k}_{layer}"] = np.float32(d.max())
            out[f"ptfstats{k}_{layer}"] = np.array([d.mean(), np.quantile(d, 0.999), d.mean(axis=1).max()],
                                                   np.float32)
    np.savez_compressed(HERE / "decoder_8b_prefill.npz", **out)


def main() -> None:
    ref = Ref()
    if sys.argv[1:] == ["lowk"]:  # only the q2_K / q3_K fixtures
        lowk_golden(ref)
        return
    if sys.argv[1:] == ["decoder_8b_prefill"]:  # only the 8B-shaped prefill fixture
        decoder_8b_prefill_golden(ref)
        return
    if sys.argv[1:] == ["decoder_8b"]:  # only the 8B-shaped decoder fixture
        decoder_8b_golden(ref)
        return
    if sys.argv[1:] == ["legacy_quants"]:  # only the q4_1 / q5_0 / q5_1 fixture
        legacy_quants_golden(ref)
        return
    if sys.argv[1:] == ["mul_mat_float"]:  # only the float-weight MUL_MAT fixture
        mul_mat_float_golden(ref)
        return
    if sys.argv[1:] == ["mul_mat_id"]:  # only the MUL_MAT_ID fixture
        mul_mat_id_golden(ref)
        return
    if sys.argv[1:] == ["decoder_paged"]:  # only the paged-decoder fixture
        decoder_paged_golden(ref)
        return
    if sys.argv[1:] == ["decoder"]:  # only the decoder-step fixture
        decoder_golden(ref)
        return
    if sys.argv[1:] == ["core"]:  # only the core-op fixture
        core_golden(ref)
        return
    if sys.argv[1:] == ["flash_attn_ext"]:  # only the FLASH_ATTN_EXT fixture
        flash_attn_ext_golden(ref)
        return
    if sys.argv[1:] == ["q6_K"]:  # only the q6_K fixture
        q6_K_golden(ref)
        return
    if sys.argv[1:] == ["q5_K"]:  # only the q5_K fixture
        q5_K_golden(ref)
        return
    # ---------------------------------------------------------------- fp16
    halves = np.arange(65536, dtype=np.uint16)
    h2f = ref.f16_to_f32(halves)
    f = fp16_probe_values()
    np.savez_compressed(HERE / "fp16.npz", h2f_bits=h2f.view(np.uint32), f2h=ref.f32_to_f16(f))

    # ------------------------------------------------------ weight quantization
    K = 512
    w = synth.normal(11, (12, K), 0.02)
    w[0] = 0.0
    w[1] = 0.01
    w[2, :256] = synth.normal(12, (256,), 1.0)
    w[3] = np.abs(w[3])  # non-negative rows: min > 0 is clamped to 0 in q4_K
    out = {"w": w}
    for t, name in ((Q4_0, "q4_0"), (Q8_0, "q8_0"), (Q4_K, "q4_K")):
        q = ref.quantize_weights(t, w)
        out[f"{name}_bytes"] = q
        out[f"{name}_deq"] = ref.dequantize(t, q, K)
    np.savez_compressed(HERE / "quant.npz", **out)

    # ----------------------------------------------- activation quantization
    K = 1024
    x = np.concatenate([edge_rows_act(K), synth.normal(13, (6, K))]).astype(np.float32)
    np.savez_compressed(HERE / "act.npz", x=x, q8_0=ref.quantize_act(Q4_0, x), q8_K=ref.quantize_act(Q4_K, x))

    # ------------------------------------------ mul_mat, the reference test's cases
    rows, k = 96, 256
    wn = xorshift_noise((rows, k), 1)
    ns = [1, 3, 5, 8, 9, 40]
    out = {"w_f32": wn, "ns": np.array(ns)}
    for n in ns:
        out[f"x{n}"] = xorshift_noise((n, k), 10 + n)
    for t, name in ((Q4_0, "q4_0"), (Q8_0, "q8_0"), (Q4_K, "q4_K")):
        q = ref.quantize_weights(t, wn)
        out[f"{name}_w"] = q
        for n in ns:
            y, _ = ref.mul_mat(t, q, rows, k, out[f"x{n}"])
            out[f"{name}_y{n}"] = y
    np.savez_compressed(HERE / "mul_mat.npz", **out)

    # ------------------------------------------------------------ config 1
    M = K1 = 4096
    wq = synth.q8_0_config1(0, M, K1)
    x1 = synth.normal(1000, (1, K1))
    y1, _ = ref.mul_mat(Q8_0, wq, M, K1, x1, nthreads=8)
    np.savez_compressed(HERE / "config1.npz", w_sha256=np.frombuffer(hashlib.sha256(wq.tobytes()).digest(), np.uint8),
                        x_sha256=np.frombuffer(hashlib.sha256(x1.tobytes()).digest(), np.uint8), y=y1,
                        seeds=np.array([0, 1000]))

    # ----------------------------------------------------------- flash attn
    out = {}
    for i, (H, Hkv, D, L) in enumerate(((4, 1, 128, 70), (8, 2, 64, 33), (8, 2, 128, 515), (4, 4, 256, 5))):
        q = synth.normal(200 + i, (H, D))
        kk = synth.f16_bits(synth.normal(300 + i, (Hkv, L, D)))
        vv = synth.f16_bits(synth.normal(400 + i, (Hkv, L, D)))
        o, _ = ref.flash_attn(q, kk, vv, 1.0 / np.sqrt(D))
        out.update({f"q{i}": q, f"k{i}": kk, f"v{i}": vv, f"o{i}": o})
    np.savez_compressed(HERE / "flash_attn.npz", **out)
    flash_attn_ext_golden(ref)
    q6_K_golden(ref)
    q5_K_golden(ref)
    lowk_golden(ref)
    core_golden(ref)
    decoder_golden(ref)
    decoder_paged_golden(ref)
    decoder_8b_golden(ref)
    decoder_8b_prefill_golden(ref)
    mul_mat_id_golden(ref)
    mul_mat_float_golden(ref)
    legacy_quants_golden(ref)
    for p in sorted(HERE.glob("*.npz")):
        print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()

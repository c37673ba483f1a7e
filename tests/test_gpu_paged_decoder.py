"""A batched decoder over a paged KV cache through the executor: the prompt of
each sequence runs alone (its keys and values written into the pools with the
`paged-cache-write` node, crates/tensorlisp/src/scheme/core.ss:260-272), then
all sequences decode together, one token each per step, with the
`paged-attention` node (core.ss:247-258) reading the pools through block
tables. The reference cannot run these CUSTOM nodes (ggml has no function for
them), so each sequence's logits are checked against the same model with the
dense cache, sequence by sequence, on the reference CPU backend
(decoder_paged.npz, refs.paged_ref_run); tolerance 8e-3 of the largest logit,
the reference's own for FLASH_ATTN_EXT (its f16 P.V accumulation)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from refs import PAGED_SEQS, PAGED_TABLES, decoder_tiny_config, decoder_weights
from tensorlisp_amd import graph as G

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def close(got, want, tol, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    print(f"[paged] {what}: max err {err:.3e} (scale {scale:.3e})", flush=True)
    assert err <= tol * scale + 1e-6, (what, err, scale)


class PagedDecoder:
    def __init__(self, c, pc, weights):
        import torch

        self.c, self.pc = c, pc
        self.w = [dev(w) for w in weights]
        self.offs, total = pc.state_bytes(c)
        self.state = torch.zeros(total, dtype=torch.uint8, device="cuda")

    def run(self, st, inputs, graph=False):
        import torch

        prog = G.Program(st.builder, st.keep, self.w, self.offs)
        stream = torch.cuda.Stream() if graph else None  # a hipGraph is captured on a stream of its own
        for i, a in enumerate(inputs):
            prog.write_input(i, dev(a), stream)
        prog.run(self.state, stream, graph)
        lg = prog.read(st.logits, torch.float32, self.state, stream)
        am = prog.read(st.argmax, torch.int32, self.state, stream)
        torch.cuda.synchronize()
        return prog, lg.cpu().numpy().reshape(-1, self.c.n_vocab), am.cpu().numpy().reshape(-1)

    def prefill(self, tokens, table):
        T = len(tokens)
        pos = np.arange(T, dtype=np.int32)
        st = G.decoder_prefill_paged(self.c, self.pc, T)
        return self.run(st, [np.array(tokens, np.int32), pos, G.paged_slots(table, pos, self.pc.block_size),
                             G.causal_mask(pos, T)])[1:]

    def decode_inputs(self, tokens, positions, tables):
        pc = self.pc
        pos = np.array(positions, np.int32)
        slots = np.concatenate([G.paged_slots(t, [p], pc.block_size) for t, p in zip(tables, pos)])
        tab = np.zeros((len(tables), pc.max_blocks), np.int32)
        for s, t in enumerate(tables):
            tab[s, :len(t)] = t
        return [np.array(tokens, np.int32), pos, slots, tab, pos + 1]


def test_batched_paged_decode_matches_reference_per_sequence(gpu):
    c = decoder_tiny_config()
    pc = G.PagedConfig(block_size=16, n_blocks=16, max_blocks=4)
    g = np.load(GOLD / "decoder_paged.npz")
    dec = PagedDecoder(c, pc, decoder_weights(c))
    for s, (prompt, _) in enumerate(PAGED_SEQS):
        lg, am = dec.prefill(prompt, PAGED_TABLES[s])
        close(lg[0], g["prompt_logits"][s], 8e-3, f"prompt of sequence {s}")
        assert am[0] == g["prompt_argmax"][s]
    S = len(PAGED_SEQS)
    st = G.decoder_decode_paged(c, pc, S)
    for j in range(len(PAGED_SEQS[0][1])):
        toks = [dec_toks[j] for _, dec_toks in PAGED_SEQS]
        pos = [len(prompt) + j for prompt, _ in PAGED_SEQS]
        prog, lg, am = dec.run(st, dec.decode_inputs(toks, pos, PAGED_TABLES), graph=j == 2)
        close(lg, g["decode_logits"][j], 8e-3, f"decode step {j}")
        np.testing.assert_array_equal(am, g["decode_argmax"][j])


def test_paged_decode_pools_hold_the_dense_caches(gpu):
    """After the prompts, each pool block holds exactly the f16 rows the
    dense-cache step writes for the same tokens (read back through the vLLM
    layouts: keys [blocks, kv_heads, hs/8, block_size, 8], values [blocks,
    kv_heads, hs, block_size])."""
    import torch

    c = decoder_tiny_config()
    pc = G.PagedConfig(block_size=16, n_blocks=16, max_blocks=4)
    w = decoder_weights(c)
    dec = PagedDecoder(c, pc, w)
    prompt, table = PAGED_SEQS[1][0], PAGED_TABLES[1]
    dec.prefill(prompt, table)
    # the same prompt through the dense-cache program
    dense = torch.zeros(c.state_bytes()[1], dtype=torch.uint8, device="cuda")
    T = len(prompt)
    st = G.decoder_step(c, T, T)
    prog = G.Program(st.builder, st.keep, dec.w, c.state_bytes()[0])
    pos = np.arange(T, dtype=np.int32)
    for i, a in enumerate([np.array(prompt, np.int32), pos, pos.astype(np.int64), G.causal_mask(pos, T)]):
        prog.write_input(i, dev(a))
    prog.run(dense)
    torch.cuda.synchronize()
    pools = dec.state.cpu().numpy()
    per = pc.pool_bytes(c)
    hd, kvh, bs = c.head_dim, c.n_head_kv, pc.block_size
    dn = dense.cpu().numpy()
    dper = c.n_embd_kv * c.n_ctx * 2
    for layer in range(c.n_layer):
        kp = pools[dec.offs[2 * layer]:dec.offs[2 * layer] + per].view(np.uint16).reshape(pc.n_blocks, kvh, hd // 8,
                                                                                            bs, 8)
        vp = pools[dec.offs[2 * layer + 1]:dec.offs[2 * layer + 1] + per].view(np.uint16).reshape(pc.n_blocks, kvh,
                                                                                                     hd, bs)
        kd = dn[2 * layer * dper:(2 * layer + 1) * dper].view(np.uint16).reshape(c.n_ctx, kvh, hd)
        vd = dn[(2 * layer + 1) * dper:(2 * layer + 2) * dper].view(np.uint16).reshape(c.n_ctx, kvh, hd)
        for p in range(T):
            b, o = table[p // bs], p % bs
            np.testing.assert_array_equal(kp[b, :, :, o, :].reshape(kvh, hd), kd[p], err_msg=f"K l{layer} p{p}")
            np.testing.assert_array_equal(vp[b, :, :, o], vd[p], err_msg=f"V l{layer} p{p}")

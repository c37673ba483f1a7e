"""GPU parity: paged-attention decode and reshape_and_cache through the C ABI.

Pins: the oracle (vLLM v1 arithmetic: f32 logits, f16 probabilities, f32 P.V),
a float64 brute-force softmax over exactly the f16 K/V, and a bit-exact cache
write. Tolerance for the f16 output: max |got - want| <= 3e-3 * max |want|, the
reference's own f16 tolerance for this kernel
(crates/kernels/tests/paged_attn_cuda.rs:39-56); the GPU keeps probabilities in
f32 with an online softmax, so its error to the f64 truth is below the oracle's.
Cases follow the reference tests: head sizes 64..256, kv heads 1/2 and GQA,
block sizes 8/16/32, lens {70, 33, 5}, long contexts {700, 1300}, {515, 5}
(paged_attn_cuda.rs:235-266, native.rs:354-412), plus BASELINE config 4.
"""
from __future__ import annotations

import numpy as np
import pytest

from refs import oracle
from tensorlisp_amd import native as N
from tensorlisp_amd import synth
from test_oracle import _random_paged, attention_f64

pytestmark = pytest.mark.gpu
TOL = 3e-3


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_gpu(q, kc, vc, tables, lens, kvh, bs, scale, max_ctx=None):
    import torch

    qd = dev(q).view(torch.float16)
    out = N.paged_attention(qd, dev(kc).view(torch.float16), dev(vc).view(torch.float16), dev(tables), dev(lens),
                            bs, int(max_ctx if max_ctx is not None else max(1, lens.max())), scale, kvh)
    return host(out.view(torch.int16)).view(np.uint16)


CASES = [
    # hs, bs, kvh, heads, lens
    (128, 16, 2, 8, [70, 33, 5]),
    (64, 8, 1, 4, [70, 33, 5]),
    (256, 32, 2, 4, [70, 33, 5]),
    (80, 32, 1, 4, [1, 31, 32, 33]),
    (96, 16, 1, 1, [17]),
    (112, 8, 2, 2, [9, 64]),
    (192, 16, 1, 2, [48]),
    (128, 16, 1, 4, [700, 1300]),
    (128, 16, 1, 4, [515, 5]),
    (128, 16, 8, 32, [512, 1, 1024, 513]),
    (128, 8, 2, 6, [77, 300]),  # group of 3 query heads per kv head
    # 64..256 workgroups of (sequence, kv head) and contexts up to 1024 tokens:
    # the one-partition form (8 waves over the whole context, no merge)
    (128, 16, 8, 32, [1, 1024, 513, 37, 700, 16, 17, 300]),
    (64, 8, 8, 24, [5, 77, 1000, 8, 9, 256, 511, 33]),  # groups of 3, 8-token pages
    (96, 32, 16, 32, [100, 1, 900, 64, 65, 31, 32, 512]),  # groups of 2, 128 workgroups
    (128, 16, 8, 32, [1, 512, 300, 37, 16, 17, 255, 500]),  # contexts of at most 512 tokens
    # 4 sequences x 8 kv heads x ceil(8192 / 512) = 512 workgroups: these take the
    # 512-token partitions (fewer workgroups would take 256-token ones), at block
    # sizes 8 and 32 and head sizes 64 and 256
    (64, 8, 8, 32, [8192, 100, 3000, 511]),
    (256, 32, 8, 32, [8192, 1, 4097, 512]),
]


@pytest.mark.parametrize("hs,bs,kvh,heads,lens", CASES)
def test_paged_attention_vs_oracle_and_bruteforce(gpu, hs, bs, kvh, heads, lens):
    q, kc, vc, tables, L = _random_paged(len(lens), heads, kvh, hs, bs, lens, 1000 + hs + bs)
    scale = 1.0 / np.sqrt(hs)
    got = run_gpu(q, kc, vc, tables, L, kvh, bs, scale).view(np.float16).astype(np.float64)
    want = oracle().paged_attention(q, kc, vc, kvh, scale, tables, L, bs).view(np.float16).astype(np.float64)
    truth = attention_f64(q, kc, vc, tables, L, kvh, bs, scale)
    assert np.abs(got - want).max() <= TOL * np.abs(want).max()
    assert np.abs(got - truth).max() <= TOL * np.abs(truth).max()


def test_paged_attention_masks_nan_past_context(gpu):
    """Slots past the context in the last page hold NaN: they must not reach the output
    (the reference zeroes them, pagedattention.cuh:405-416)."""
    hs, bs, kvh, heads, lens = 128, 16, 1, 4, [37, 5]
    q, kc, vc, tables, L = _random_paged(2, heads, kvh, hs, bs, lens, 1100)
    nan = np.float16(np.nan).view(np.uint16)
    for s, Ls in enumerate(lens):
        last = tables[s, (Ls - 1) // bs]
        kc[last, :, :, Ls % bs:, :] = nan
        vc[last, :, :, Ls % bs:] = nan
    scale = 1.0 / np.sqrt(hs)
    got = run_gpu(q, kc, vc, tables, L, kvh, bs, scale).view(np.float16).astype(np.float64)
    assert np.isfinite(got).all()
    truth = attention_f64(q, kc, vc, tables, L, kvh, bs, scale)
    assert np.abs(got - truth).max() <= TOL * np.abs(truth).max()


def test_paged_attention_empty_context(gpu):
    hs, bs = 64, 16
    q, kc, vc, tables, L = _random_paged(2, 2, 1, hs, bs, [0, 20], 1200)
    got = run_gpu(q, kc, vc, tables, L, 1, bs, 0.125, max_ctx=20).view(np.float16)
    assert np.all(got[0] == 0)
    truth = attention_f64(q, kc, vc, tables, L, 1, bs, 0.125)
    assert np.abs(got[1].astype(np.float64) - truth[1]).max() <= TOL * np.abs(truth[1]).max()


@pytest.mark.slow
def test_config4_full(gpu):
    """32 sequences, 32 q / 8 kv heads, hs 128, 16-token pages drawn
    without replacement from a 65,536-page pool, lens ~ U[512, 8192]. Only the pages in
    use are filled (the rest of the 2 GiB pools is never read)."""
    import torch

    seqs, heads, kvh, hs, bs, pool = 32, 32, 8, 128, 16, 65536
    lens = synth.integers(1300, 512, 8192, seqs).astype(np.int32)
    pages = [(int(L) + bs - 1) // bs for L in lens]
    maxb = 8192 // bs  # max_blocks_per_seq * block_size covers max_context_len
    order = synth.bits(1301, pool).argsort()[: sum(pages)].astype(np.int32)
    tables = np.zeros((seqs, maxb), np.int32)
    c = 0
    for s, p in enumerate(pages):
        tables[s, :p] = order[c:c + p]
        c += p
    used = order
    kvals = synth.f16_bits(synth.normal(1302, (len(used), kvh, hs // 8, bs, 8)))
    vvals = synth.f16_bits(synth.normal(1303, (len(used), kvh, hs, bs)))
    q = synth.f16_bits(synth.normal(1304, (seqs, heads, hs)))
    kc = torch.zeros((pool, kvh, hs // 8, bs, 8), dtype=torch.int16, device="cuda")
    vc = torch.zeros((pool, kvh, hs, bs), dtype=torch.int16, device="cuda")
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    kc[idx] = torch.from_numpy(kvals.view(np.int16)).cuda()
    vc[idx] = torch.from_numpy(vvals.view(np.int16)).cuda()
    scale = 1.0 / np.sqrt(hs)
    out = N.paged_attention(dev(q).view(torch.float16), kc.view(torch.float16), vc.view(torch.float16), dev(tables),
                            dev(lens), bs, 8192, scale, kvh)
    got = host(out.view(torch.int16)).view(np.float16).astype(np.float64)
    # oracle on a compact pool holding just the used pages, with remapped tables
    remap = np.zeros(pool, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    ctables = remap[tables]
    want = oracle().paged_attention(q, kvals, vvals, kvh, scale, ctables, lens, bs).view(np.float16)
    want = want.astype(np.float64)
    assert np.abs(got - want).max() <= TOL * np.abs(want).max()


@pytest.mark.parametrize("kvh,hs,bs", [(2, 64, 8), (8, 128, 16), (1, 256, 32)])
def test_reshape_and_cache_bit_exact(gpu, kvh, hs, bs):
    import torch

    T, nblocks = 45, 16
    key = synth.f16_bits(synth.normal(1400 + hs, (T, kvh * hs)))
    val = synth.f16_bits(synth.normal(1401 + hs, (T, kvh * hs)))
    slots = synth.bits(1402, nblocks * bs).argsort()[:T].astype(np.int64)
    slots[3] = -1
    slots[T - 1] = -7
    kc = np.full((nblocks, kvh, hs // 8, bs, 8), 0x1234, np.uint16)
    vc = np.full((nblocks, kvh, hs, bs), 0x4321, np.uint16)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    N.reshape_and_cache(dev(key.view(np.int16)), dev(val.view(np.int16)), kd, vd, dev(slots), kvh, bs)
    oracle().reshape_and_cache(key, val, kc, vc, slots, kvh, hs, bs)
    assert np.array_equal(host(kd).view(np.uint16), kc)
    assert np.array_equal(host(vd).view(np.uint16), vc)
    torch.cuda.synchronize()


def test_reshape_and_cache_drops_slots_past_the_pools(gpu):
    """Slots at or past num_blocks * block_size write nothing (the pools' length
    comes from the cache tensors). The pools here are the first blocks of larger
    buffers, and every dropped slot lies inside the spare blocks behind them, so
    the spare blocks must come back untouched."""
    import torch

    kvh, hs, bs, nblocks, spare = 2, 64, 16, 8, 4
    T = 6
    key = synth.f16_bits(synth.normal(1410, (T, kvh * hs)))
    val = synth.f16_bits(synth.normal(1411, (T, kvh * hs)))
    slots = np.array([0, nblocks * bs, 5, nblocks * bs + 17, (nblocks + spare) * bs - 1, nblocks * bs - 1], np.int64)
    kc = np.full((nblocks + spare, kvh, hs // 8, bs, 8), 0x1234, np.uint16)
    vc = np.full((nblocks + spare, kvh, hs, bs), 0x4321, np.uint16)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    N.reshape_and_cache(dev(key.view(np.int16)), dev(val.view(np.int16)), kd[:nblocks], vd[:nblocks], dev(slots),
                        kvh, bs)
    kept = np.where(slots < nblocks * bs, slots, -1)
    oracle().reshape_and_cache(key, val, kc, vc, kept, kvh, hs, bs)
    assert np.array_equal(host(kd).view(np.uint16), kc)
    assert np.array_equal(host(vd).view(np.uint16), vc)
    assert np.all(kc[nblocks:] == 0x1234) and np.all(vc[nblocks:] == 0x4321)
    torch.cuda.synchronize()


def test_cache_write_then_attention_matches_dense(gpu):
    """The reference's paged-vs-dense pattern (native.rs:354-412): write K/V through the
    cache-write node with a reversed block table, attend, compare with dense brute force."""
    import torch

    kvh, heads, hs, bs = 2, 8, 128, 16
    lens = [70, 33, 5]
    maxb = max((L + bs - 1) // bs for L in lens)
    nblocks = len(lens) * maxb
    tables = np.array([[(s + 1) * maxb - 1 - j for j in range(maxb)] for s in range(len(lens))], np.int32)
    kc = torch.zeros((nblocks, kvh, hs // 8, bs, 8), dtype=torch.int16, device="cuda")
    vc = torch.zeros((nblocks, kvh, hs, bs), dtype=torch.int16, device="cuda")
    dense_k, dense_v = [], []
    for s, L in enumerate(lens):
        k = synth.f16_bits(synth.normal(1500 + s, (L, kvh * hs)))
        v = synth.f16_bits(synth.normal(1600 + s, (L, kvh * hs)))
        slots = np.array([tables[s, t // bs] * bs + t % bs for t in range(L)], np.int64)
        N.reshape_and_cache(dev(k.view(np.int16)), dev(v.view(np.int16)), kc, vc, dev(slots), kvh, bs)
        dense_k.append(k.view(np.float16).astype(np.float64).reshape(L, kvh, hs))
        dense_v.append(v.view(np.float16).astype(np.float64).reshape(L, kvh, hs))
    q = synth.f16_bits(synth.normal(1700, (len(lens), heads, hs)))
    scale = hs ** -0.5
    out = N.paged_attention(dev(q).view(torch.float16), kc.view(torch.float16), vc.view(torch.float16), dev(tables),
                            dev(np.array(lens, np.int32)), bs, max(lens), scale, kvh)
    got = host(out.view(torch.int16)).view(np.float16).astype(np.float64)
    qf = q.view(np.float16).astype(np.float64)
    for s, L in enumerate(lens):
        for h in range(heads):
            g = h // (heads // kvh)
            lg = scale * dense_k[s][:, g, :] @ qf[s, h]
            p = np.exp(lg - lg.max())
            want = (p / p.sum()) @ dense_v[s][:, g, :]
            assert np.abs(got[s, h] - want).max() <= TOL * np.abs(want).max()


@pytest.mark.parametrize("hs,bs,kvh,heads,lens", [
    (128, 16, 8, 32, [768]),                   # a batch-1 decode step (3 partitions)
    (128, 16, 8, 32, [512, 1, 1024, 513]),
    (64, 8, 8, 32, [8192, 100, 3000, 511]),   # 512-token partitions
    (128, 16, 2, 6, [0, 300, 2049]),          # an empty context, a group of 3
    (128, 16, 8, 32, [0, 300, 1024, 5, 64, 65, 17, 900]),  # one partition (64 workgroups)
])
def test_one_launch_merge_matches_two_launches(gpu, hs, bs, kvh, heads, lens):
    """A paged-attention node in a program runs as one launch whose last
    partition of each (sequence, head group) merges the others (on counters it
    leaves zeroed). Its output is bit-identical to the two-launch form of the
    C ABI on every run, eager and replayed as a graph."""
    import torch

    from tensorlisp_amd import graph as G

    q, kc, vc, tables, L = _random_paged(len(lens), heads, kvh, hs, bs, lens, 1400 + hs + len(lens))
    scale = 1.0 / np.sqrt(hs)
    max_ctx = int(max(1, max(lens)))
    want = run_gpu(q, kc, vc, tables, L, kvh, bs, scale, max_ctx)
    b = G.Builder()
    qi = b.input(N.F16, [hs, heads, len(lens)])
    ti = b.input(N.I32, [tables.shape[1], len(lens)])
    li = b.input(N.I32, [len(lens)])
    kw, vw = b.weight(N.F16, [kc.size]), b.weight(N.F16, [vc.size])
    out = b.paged_attention(qi, kw, vw, ti, li, bs, max_ctx, scale, kvh)
    b.expand(out)
    prog = G.Program(b, [out], [dev(kc.view(np.int16)), dev(vc.view(np.int16))])
    assert prog.stats()["launches"] == 1
    ins = [dev(a) for a in (q.view(np.int16), tables, L)]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    for i, a in enumerate(ins):
        prog.write_input(i, a, stream)
    for rep in range(5):
        with torch.cuda.stream(stream):
            prog.run(None, stream, graph=rep >= 2)
            got = prog.read(out, torch.int16, None, stream)
        stream.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16).reshape(want.shape), want,
                                      err_msg=f"run {rep}")

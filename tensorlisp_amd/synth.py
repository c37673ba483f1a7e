"""Deterministic synthetic inputs for parity tests and the benchmark.

A counter-based generator (splitmix64 of seed and element index) so any slice
of any input can be regenerated independently of numpy's RNG stream policy:
uniform in [0, 1) from the top 24 bits, N(0, 1) by Box-Muller. BASELINE's
configs fix distributions but no RNG; this one is ours, and fixtures record
the seeds they were made with.
"""
from __future__ import annotations

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    x = x + np.uint64(0x9E3779B97F4A7C15)
    z = x
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def bits(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n pseudo-random uint64 for stream `seed`, elements offset..offset+n-1."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset, offset + n, dtype=np.uint64)
        base = _splitmix64(np.array([seed], dtype=np.uint64))[0]
        return _splitmix64(idx ^ base)


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """float64 in [0, 1) with 24 random bits (exact in float32)."""
    return (bits(seed, n, offset) >> np.uint64(40)).astype(np.float64) / float(1 << 24)


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """float32 N(0, std^2) of `shape` by Box-Muller on pairs of uniforms."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m)
    z[0::2] = r * np.cos(2 * np.pi * u2)
    z[1::2] = r * np.sin(2 * np.pi * u2)
    return (z[:n] * std).astype(np.float32).reshape(shape)


def integers(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    """int64 uniform in [lo, hi] (inclusive)."""
    span = np.uint64(hi - lo + 1)
    return (bits(seed, n) % span).astype(np.int64) + lo


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


# ------------------------------------------------------------ weight blocks
def q8_0_config1(seed: int, M: int, K: int) -> np.ndarray:
    """BASELINE config 1's Q8_0 weight built directly: codes uniform in [-127, 127],
    f16 scale |N(0, 0.02)| / 127 (about 30% of them f16-subnormal). uint8 [M, K/32*34]."""
    nb = M * (K // 32)
    qs = integers(seed, -127, 127, nb * 32).astype(np.int8).view(np.uint8).reshape(nb, 32)
    d = f16_bits(np.abs(normal(seed + 1, (nb,), 0.02)) / np.float32(127))
    blocks = np.empty((nb, 34), np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = qs
    return blocks.reshape(M, (K // 32) * 34)


def random_blocks(wtype: int, seed: int, M: int, K: int, std: float = 0.02) -> np.ndarray:
    """Structurally valid random blocks of a weight type, sized like weights
    quantized from N(0, std) (finite f16 scales, random codes). Used where
    quantizing full-size f32 weights on the host would dominate run time."""
    from .native import Q2_K, Q3_K, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K

    if wtype == Q8_0:
        return q8_0_config1(seed, M, K)
    if wtype == Q4_0:
        nb = M * (K // 32)
        d = f16_bits(normal(seed + 1, (nb,), std) / np.float32(8))
        qs = (bits(seed, nb * 2) & np.uint64(0xFFFFFFFFFFFFFFFF)).view(np.uint8).reshape(nb, 16)
        blocks = np.empty((nb, 18), np.uint8)
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:] = qs
        return blocks.reshape(M, (K // 32) * 18)
    if wtype == Q4_K:
        nb = M * (K // 256)
        d = f16_bits(np.abs(normal(seed + 1, (nb,), std)) / np.float32(63 * 4))
        dmin = f16_bits(np.abs(normal(seed + 2, (nb,), std)) / np.float32(63 * 2))
        raw = bits(seed, nb * 18).view(np.uint8).reshape(nb, 144)
        blocks = raw.copy()
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
        return blocks.reshape(M, (K // 256) * 144)
    if wtype == Q5_K:
        # q4_K's header statistics, random qh / qs bytes (codes 0..31)
        nb = M * (K // 256)
        d = f16_bits(np.abs(normal(seed + 1, (nb,), std)) / np.float32(63 * 8))
        dmin = f16_bits(np.abs(normal(seed + 2, (nb,), std)) / np.float32(63 * 2))
        blocks = bits(seed, nb * 22).view(np.uint8).reshape(nb, 176).copy()
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
        return blocks.reshape(M, (K // 256) * 176)
    if wtype == Q6_K:
        # random ql/qh bytes, int8 scales over the whole range the quantizer
        # emits (|scale| <= 127 plus -128), f16 d ~ |N(0, std)| / (32 * 127)
        nb = M * (K // 256)
        d = f16_bits(np.abs(normal(seed + 1, (nb,), std)) / np.float32(32 * 127))
        raw = bits(seed, nb * 27).view(np.uint8).reshape(nb, 216)[:, :210]
        blocks = raw.copy()
        blocks[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
        return blocks.reshape(M, (K // 256) * 210)
    if wtype == Q2_K:
        # random 4-bit scale / min pairs and 2-bit codes; d, dmin > 0 sized so
        # d * 15 * 3 and dmin * 15 span about the weights' range
        nb = M * (K // 256)
        d = f16_bits(np.abs(normal(seed + 1, (nb,), std)) / np.float32(15 * 1.5))
        dmin = f16_bits(np.abs(normal(seed + 2, (nb,), std)) / np.float32(15))
        blocks = bits(seed, (nb * 84 + 7) // 8).view(np.uint8)[:nb * 84].reshape(nb, 84).copy()
        blocks[:, 80:82] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 82:84] = dmin.view(np.uint8).reshape(nb, 2)
        return blocks.reshape(M, (K // 256) * 84)
    if wtype == Q3_K:
        # random high bits, 2-bit codes and packed 6-bit scales (-32..31); a
        # signed d, as the quantizer's 1 / iscale may be
        nb = M * (K // 256)
        d = f16_bits(normal(seed + 1, (nb,), std) / np.float32(32 * 2))
        blocks = bits(seed, (nb * 110 + 7) // 8).view(np.uint8)[:nb * 110].reshape(nb, 110).copy()
        blocks[:, 108:110] = d.view(np.uint8).reshape(nb, 2)
        return blocks.reshape(M, (K // 256) * 110)
    if wtype in (Q4_1, Q5_0, Q5_1):
        # random code bytes (nibbles and fifth bits); q5_0 a signed d as q4_0,
        # q4_1 / q5_1 d > 0 with a min m < 0 about half the block's range
        bb, levels = {Q4_1: (20, 15), Q5_0: (22, 16), Q5_1: (24, 31)}[wtype]
        nb = M * (K // 32)
        blocks = bits(seed, (nb * bb + 7) // 8).view(np.uint8)[:nb * bb].reshape(nb, bb).copy()
        if wtype == Q5_0:
            d = f16_bits(normal(seed + 1, (nb,), std) / np.float32(levels))
        else:
            d = f16_bits(np.abs(normal(seed + 1, (nb,), std)) * np.float32(3 / levels))
            m = f16_bits(-np.abs(normal(seed + 2, (nb,), std)) * np.float32(1.5))
            blocks[:, 2:4] = m.view(np.uint8).reshape(nb, 2)
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        return blocks.reshape(M, (K // 32) * bb)
    raise ValueError(wtype)


def q4_K_model_blocks(seed: int, M: int, K: int, std: float = 0.02) -> np.ndarray:
    """Random q4_K blocks that behave like quantized zero-mean weights of
    standard deviation about `std`: per 32-element sub-block a scale sc in
    1..63 and a min m = round(15 sc / 16) against dmin = 8 d, so each
    sub-block's values d sc q - 8 d m (q uniform in 0..15) are centred on zero
    to within 4 d. (Independent random d, dmin, sc and m, as random_blocks
    draws them, give every row a large common offset, and with it a model whose
    logits hardly depend on its input.) uint8 [M, K/256*144]."""
    nb = M * (K // 256)
    u = uniform(seed + 1, nb).astype(np.float32)
    d32 = (np.float32(std) / np.float32(32 * 4.6)) * (np.float32(0.5) + u)
    d = f16_bits(d32)
    dmin = f16_bits(d.view(np.float16).astype(np.float32) * np.float32(8))
    sc = (integers(seed + 2, 1, 63, nb * 8)).astype(np.int64).reshape(nb, 8)
    mn = np.rint(sc * 15 / 16).astype(np.int64)
    f = np.zeros((nb, 12), np.uint8)
    # the 6-bit fields as get_scale_min_k4 reads them (ggml-quants.c:880-887)
    f[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    f[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    f[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    blocks = np.empty((nb, 144), np.uint8)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    blocks[:, 4:16] = f
    blocks[:, 16:] = bits(seed, nb * 16).view(np.uint8).reshape(nb, 128)
    return blocks.reshape(M, (K // 256) * 144)


def q4_K_model_blocks_gpu(torch, gen, M: int, K: int, std: float = 0.02):
    """q4_K_model_blocks' distribution drawn on the GPU with a torch generator
    (for full-size models, where host generation would dominate): a uint8
    device tensor [M, K/256*144]. Not bit-identical to the host version."""
    nb = M * (K // 256)
    dev = gen.device
    d32 = (std / (32 * 4.6)) * (0.5 + torch.rand(nb, device=dev, generator=gen))
    d = d32.to(torch.float16)
    dmin = (d.to(torch.float32) * 8).to(torch.float16)
    sc = torch.randint(1, 64, (nb, 8), device=dev, generator=gen, dtype=torch.int32)
    mn = torch.round(sc.to(torch.float32) * 15 / 16).to(torch.int32)
    f = torch.empty((nb, 12), dtype=torch.int32, device=dev)
    f[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    f[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    f[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    blocks = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device=dev, generator=gen)
    blocks[:, 0:2] = d.view(torch.uint8).reshape(nb, 2)
    blocks[:, 2:4] = dmin.view(torch.uint8).reshape(nb, 2)
    blocks[:, 4:16] = f.to(torch.uint8)
    return blocks.reshape(M, (K // 256) * 144)

// Shared device-side definitions of the gfx950 executor: block formats,
// conversions, the quantized-activation scratch layout and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tlhip.h"

namespace tlh {

// ----------------------------------------------------------- block formats
// vendor/ggml/src/ggml-common.h:194-198 (q4_0), :201-211 (q4_1), :229-248
// (q5_0, q5_1), :251-269 (q8_0, q8_1), :325-337 (q4_K), :345-352 (q5_K),
// :362-368 (q6_K), :370-375 (q8_K), :298-323 (q2_K, q3_K). Byte sizes per
// block and elements per block.
constexpr int QK = 32;    // q4_0 / q4_1 / q5_0 / q5_1 / q8_0 / q8_1 block
constexpr int QKK = 256;  // k-quant super-block
constexpr int Q4_0_BYTES = 18;
constexpr int Q8_0_BYTES = 34;
constexpr int Q4_1_BYTES = 20;  // f16 d, f16 m, qs[16] (nibbles: elements j and j + 16)
constexpr int Q5_0_BYTES = 22;  // f16 d, qh[4] (fifth bits, bit j of element j), qs[16]
constexpr int Q5_1_BYTES = 24;  // f16 d, f16 m, qh[4], qs[16]
constexpr int Q8_1_BYTES = 36;  // f16 d, f16 s (= code sum * d), qs[32]
constexpr int Q4_K_BYTES = 144;
constexpr int Q5_K_BYTES = 176;  // f16 d, dmin; scales[12] as q4_K; qh[32] (fifth bits); qs[128] (low nibbles)
constexpr int Q6_K_BYTES = 210;  // ql[128] (low 4 bits), qh[64] (high 2 bits), int8 scales[16], f16 d
constexpr int Q8_K_BYTES = 292;
constexpr int Q2_K_BYTES = 84;   // scales[16] (4-bit scale | 4-bit min << 4), qs[64] (2-bit codes), f16 d, dmin
constexpr int Q3_K_BYTES = 110;  // hmask[32] (third code bits), qs[64] (2-bit low parts), scales[12] (6-bit), f16 d

__host__ __device__ constexpr bool kquant_type(int t) {
    return t == TLH_TYPE_Q2_K || t == TLH_TYPE_Q3_K || t == TLH_TYPE_Q4_K || t == TLH_TYPE_Q5_K || t == TLH_TYPE_Q6_K;
}

__host__ __device__ constexpr int block_elems(int t) {
    return (kquant_type(t) || t == TLH_TYPE_Q8_K) ? QKK
           : (t == TLH_TYPE_Q4_0 || t == TLH_TYPE_Q8_0 || t == TLH_TYPE_Q4_1 || t == TLH_TYPE_Q5_0 ||
              t == TLH_TYPE_Q5_1 || t == TLH_TYPE_Q8_1)
               ? QK
               : 1;
}
__host__ __device__ constexpr int block_bytes(int t) {
    return t == TLH_TYPE_Q4_0   ? Q4_0_BYTES
           : t == TLH_TYPE_Q8_0 ? Q8_0_BYTES
           : t == TLH_TYPE_Q4_K ? Q4_K_BYTES
           : t == TLH_TYPE_Q5_K ? Q5_K_BYTES
           : t == TLH_TYPE_Q6_K ? Q6_K_BYTES
           : t == TLH_TYPE_Q8_K ? Q8_K_BYTES
           : t == TLH_TYPE_Q4_1 ? Q4_1_BYTES
           : t == TLH_TYPE_Q5_0 ? Q5_0_BYTES
           : t == TLH_TYPE_Q5_1 ? Q5_1_BYTES
           : t == TLH_TYPE_Q8_1 ? Q8_1_BYTES
           : t == TLH_TYPE_Q2_K ? Q2_K_BYTES
           : t == TLH_TYPE_Q3_K ? Q3_K_BYTES
           : t == TLH_TYPE_F16  ? 2
                                : 4;
}
// vec_dot_type on x86 (vendor/ggml/src/ggml-cpu/ggml-cpu.c:239-319).
__host__ __device__ constexpr int vec_dot_type(int wtype) {
    return kquant_type(wtype)                                                            ? TLH_TYPE_Q8_K
           : (wtype == TLH_TYPE_Q4_1 || wtype == TLH_TYPE_Q5_1)                          ? TLH_TYPE_Q8_1
                                                                                          : TLH_TYPE_Q8_0;
}
// 32-element block types that carry a min (q4_1, q5_1: x = q * d + m) or a
// fifth code bit (q5_0, q5_1)
__host__ __device__ constexpr bool has_min(int wtype) { return wtype == TLH_TYPE_Q4_1 || wtype == TLH_TYPE_Q5_1; }
__host__ __device__ constexpr bool has_qh(int wtype) { return wtype == TLH_TYPE_Q5_0 || wtype == TLH_TYPE_Q5_1; }
// Byte offsets in a 32-element block: the min, the fifth bits, the nibbles
__host__ __device__ constexpr int blk_qh_off(int wtype) { return wtype == TLH_TYPE_Q5_1 ? 4 : 2; }
__host__ __device__ constexpr int blk_qs_off(int wtype) {
    return wtype == TLH_TYPE_Q4_1 ? 4 : wtype == TLH_TYPE_Q5_0 ? 6 : wtype == TLH_TYPE_Q5_1 ? 8 : 2;
}

// ---------------------------------------------------------- conversions
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// v_cvt_f16_f32: round to nearest even, f16 denormals kept (kernel default mode).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
// bf16: the upper half of an f32; f32 -> bf16 rounds to nearest even and keeps
// a NaN a (quiet) NaN
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// q4_K packed 6-bit scale/min of sub-block j from the 12-byte field
// (ggml-quants.c:880-887), given the field as three little-endian words.
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
    // bytes 0..3 = s0, 4..7 = s1, 8..11 = s2
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63;
        mn = (s1 >> (8 * j)) & 63;
    } else {
        const int jj = j - 4;
        const uint32_t b8 = (s2 >> (8 * jj)) & 0xff;
        sc = (b8 & 0x0f) | (((s0 >> (8 * jj)) >> 6 & 3) << 4);
        mn = (b8 >> 4) | (((s1 >> (8 * jj)) >> 6 & 3) << 4);
    }
}

// Four bits (of a q5 block's qh word) to bit 4 of four bytes: bit i lands at
// bit 8i by the multiply (the shifted copies never overlap), then moves up 4.
__device__ __forceinline__ uint32_t spread4(uint32_t b4) { return ((b4 * 0x00204081u) & 0x01010101u) << 4; }

// ------------------------------------------------------ element dequantizers
// Element `col` of a row of ggml blocks of type WT, rounded as the reference's
// dequantize_row_* rounds it (integer codes convert exactly): q4_0
// (q-8)*d (ggml-quants.c:459-476), q8_0 q*d (:553-565), q4_K (d*sc)*q -
// (dmin*m) (:1529-1550), q5_K the same with a fifth code bit (:1731-1756),
// q6_K (d*sc)*q (:1939-1968), q4_1 q*d + m (:479-498), q5_0 (q-16)*d
// (:500-524), q5_1 q*d + m (:526-551), q2_K (d*sc)*q - (dmin*m) (:961-989),
// q3_K (d*(sc-32))*q (:1305-1351).
template <int WT> __device__ __forceinline__ float dequant_elem(const uint8_t *r, int64_t col) {
#pragma clang fp contract(off)
    if constexpr (WT == TLH_TYPE_Q2_K || WT == TLH_TYPE_Q3_K) {
        // element e = 32j + l of half h: 2-bit code in qs[32h + l] at bit 2j
        // (q3_K: its third bit in hmask[l] at bit 4h + j, clear = minus 4)
        constexpr bool Q3 = WT == TLH_TYPE_Q3_K;
        const uint8_t *b = r + (col / QKK) * (Q3 ? Q3_K_BYTES : Q2_K_BYTES);
        const int i = (int)(col % QKK);
        const int h = i >> 7, j = (i >> 5) & 3, l = i & 31, s = i >> 4;
        const int lo = (b[(Q3 ? 32 : 16) + 32 * h + l] >> (2 * j)) & 3;
        if constexpr (Q3) {
            const int code = lo - (((b[l] >> (4 * h + j)) & 1) ? 0 : 4);
            const uint8_t *sc = b + 96;  // 6-bit scales: low 4 bits, then high 2 bits at byte 8 + s % 4
            const int scale = ((s < 8 ? (sc[s] & 15) : (sc[s - 8] >> 4)) | (((sc[8 + (s & 3)] >> (2 * (s >> 2))) & 3) << 4)) - 32;
            const float d = h2f((uint16_t)(b[108] | (b[109] << 8)));
            return (d * (float)scale) * (float)code;
        } else {
            const float d = h2f((uint16_t)(b[80] | (b[81] << 8))), dmin = h2f((uint16_t)(b[82] | (b[83] << 8)));
            const float dl = d * (float)(b[s] & 15), ml = dmin * (float)(b[s] >> 4);
            return dl * (float)lo - ml;
        }
    } else if constexpr (WT == TLH_TYPE_Q4_1 || WT == TLH_TYPE_Q5_0 || WT == TLH_TYPE_Q5_1) {
        const uint8_t *b = r + (col / QK) * block_bytes(WT);
        const int j = (int)(col % QK);
        const uint8_t byte = b[blk_qs_off(WT) + (j & 15)];
        int code = j < 16 ? (byte & 0x0f) : (byte >> 4);
        if constexpr (has_qh(WT)) {
            uint32_t qh;
            __builtin_memcpy(&qh, b + blk_qh_off(WT), 4);
            code |= (int)((qh >> j) & 1u) << 4;
        }
        const float d = h2f(*(const uint16_t *)b);
        if constexpr (WT == TLH_TYPE_Q5_0) return (float)(code - 16) * d;
        else return (float)code * d + h2f(*(const uint16_t *)(b + 2));
    } else if constexpr (WT == TLH_TYPE_Q4_0) {
        const uint8_t *b = r + (col / QK) * Q4_0_BYTES;
        const int j = (int)(col % QK);
        const float d = h2f(*(const uint16_t *)b);
        const int code = j < 16 ? (b[2 + j] & 0x0f) : (b[2 + j - 16] >> 4);
        return (float)(code - 8) * d;
    } else if constexpr (WT == TLH_TYPE_Q8_0) {
        const uint8_t *b = r + (col / QK) * Q8_0_BYTES;
        const float d = h2f(*(const uint16_t *)b);
        return (float)(int8_t)b[2 + col % QK] * d;
    } else if constexpr (WT == TLH_TYPE_Q6_K) {
        // element e of a 128-element half: low 4 bits in ql[l + 32 * (q & 1)]
        // (high nibble for q >= 2), high 2 bits in qh[l] at 2q; e = 32q + l
        const uint8_t *b = r + (col / QKK) * Q6_K_BYTES;
        const int i = (int)(col % QKK);
        const int h = i >> 7, e = i & 127, q = e >> 5, l = e & 31;
        const uint8_t lo = b[64 * h + l + 32 * (q & 1)];
        const uint8_t hi2 = b[128 + 32 * h + l];
        const int code = (int)(((q >= 2 ? lo >> 4 : lo & 0x0f) | (((hi2 >> (2 * q)) & 3) << 4))) - 32;
        const float d = h2f(*(const uint16_t *)(b + 208));
        const int sc = (int)(int8_t)b[192 + 8 * h + (e >> 4)];
        return (d * (float)sc) * (float)code;
    } else {
        static_assert(WT == TLH_TYPE_Q4_K || WT == TLH_TYPE_Q5_K, "dequant_elem: type");
        constexpr bool Q5 = WT == TLH_TYPE_Q5_K;
        const uint8_t *b = r + (col / QKK) * (Q5 ? Q5_K_BYTES : Q4_K_BYTES);
        const int i = (int)(col % QKK);
        const int c = i / 64, pos = i % 64, hi = pos >= 32, l = pos & 31;
        int sc, mn;
        uint32_t s[3];
        __builtin_memcpy(s, b + 4, 12);
        q4k_scale_min(2 * c + hi, s[0], s[1], s[2], sc, mn);
        const float d = h2f(*(const uint16_t *)b), dmin = h2f(*(const uint16_t *)(b + 2));
        const uint8_t byte = b[(Q5 ? 48 : 16) + 32 * c + l];
        int code = hi ? byte >> 4 : byte & 0x0f;
        if constexpr (Q5) code |= ((b[16 + l] >> (2 * c + hi)) & 1) << 4;
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)mn;
        return d1 * (float)code - m1;
    }
}

// ------------------------------------------------ quantized activation scratch
// The CPU backend quantizes src1 into `wdata` in ggml's block layout
// (ggml-cpu.c:1318-1359). Here the same values (bit-exact d and codes) go to
// a split layout the kernels can stream with aligned 128-bit loads: for R
// activation rows of K values,
//   qs  : int8  [R][K]            codes, 64-byte aligned rows
//   d   : f32   [R][K/blk]        block scales (q8_0 / q8_1: the f16-rounded d as f32)
//   sum : int32 [R][K/32] (q8_0)  per-block code sums
//         f32   [R][K/32] (q8_1)  per-block s (f16-rounded code sum * d, as f32)
//         int16 [R][K/16] (q8_K)  bsums
//   q16 : f16   [R][K]            (GEMM launches only) the codes as f16,
//         exact, so the MFMA operand needs no conversion
//   b16 : f16   [R][K/16]         (GEMM launches, q8_K only) the bsums as f16 (exact)
struct ActView {
    const int8_t *qs;
    const float *d;
    const int32_t *sum32;  // q8_0: code sums; q8_1: the bits of s as f32
    const int16_t *bsums;  // q8_K only
    const _Float16 *q16;   // GEMM launches only
    const _Float16 *b16;   // GEMM launches, q8_K only
    int64_t K;
};

struct ActLayout {
    int64_t qs_off, d_off, sum_off, q16_off, b16_off, total;
};

// Weight types with a tiled prefill GEMM (more than 16 activation columns);
// the others run it as 16-column slabs of the few-column kernel.
__host__ __device__ constexpr bool has_gemm(int wtype) {
    return wtype == TLH_TYPE_Q4_K || wtype == TLH_TYPE_Q5_K || wtype == TLH_TYPE_Q8_0 || wtype == TLH_TYPE_Q4_0;
}
// q4_K / q5_K GEMM launches also get the activation codes as f16.
__host__ __device__ constexpr bool act_has_f16(int wtype, int64_t n_cols) {
    return (wtype == TLH_TYPE_Q4_K || wtype == TLH_TYPE_Q5_K) && n_cols > 16;
}

__host__ __device__ inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

__host__ __device__ inline ActLayout act_layout(int act_type, int64_t K, int64_t rows, bool f16 = false) {
    ActLayout L;
    L.qs_off = 0;
    L.d_off = align_up(rows * K, 256);
    const int64_t nblk = K / block_elems(act_type);
    L.sum_off = align_up(L.d_off + rows * nblk * 4, 256);
    const int64_t sum_bytes = act_type == TLH_TYPE_Q8_K ? rows * (K / 16) * 2 : rows * (K / 32) * 4;
    L.q16_off = align_up(L.sum_off + sum_bytes, 256);
    L.b16_off = align_up(L.q16_off + rows * K * 2, 256);
    L.total = f16 ? align_up(L.b16_off + (act_type == TLH_TYPE_Q8_K ? rows * (K / 16) * 2 : 0), 256)
                  : align_up(L.q16_off, 256);
    return L;
}

__host__ __device__ inline ActView act_view(const void *base, int act_type, int64_t K, int64_t rows) {
    const ActLayout L = act_layout(act_type, K, rows);
    const char *b = (const char *)base;
    ActView v;
    v.qs = (const int8_t *)(b + L.qs_off);
    v.d = (const float *)(b + L.d_off);
    v.sum32 = (const int32_t *)(b + L.sum_off);
    v.bsums = (const int16_t *)(b + L.sum_off);
    v.q16 = (const _Float16 *)(b + L.q16_off);
    v.b16 = (const _Float16 *)(b + L.b16_off);
    v.K = K;
    return v;
}

// ------------------------------------- activation quantizers on registers
// Shared by the quantize launch and by kernels that quantize the rows they
// produce (the norm chain, SwiGLU), so both write the same bytes.

// q8_K (quantize_row_q8_K_ref, ggml-quants.c:2768-2804) of NB 256-element
// blocks held by one wave, elements 4l..4l+3 of block b in v[b] of lane l:
// the signed value of largest magnitude (the first one on ties), iscale =
// -127/max, codes rint(iscale*x) clamped to 127, d = 1/iscale; an all-zero
// block gets d = 0 and zero codes. packed[b]: the lane's four codes; psum[b]:
// the sum of the codes of lanes 4k..4k+3 (bsum k of the block). The NB
// blocks' reductions are interleaved (independent shuffle chains in flight
// together); each block's arithmetic is the same for any NB.
template <int NB>
__device__ __forceinline__ void q8K_waves(const float (&v)[NB][4], int lane, uint32_t (&packed)[NB], int (&psum)[NB],
                                          float (&d)[NB]) {
#pragma clang fp contract(off)
    float ba[NB], bv[NB];
    int bi[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        ba[b] = 0.0f, bv[b] = 0.0f, bi[b] = 1 << 30;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = fabsf(v[b][i]);
            if (a > ba[b]) { ba[b] = a; bv[b] = v[b][i]; bi[b] = 4 * lane + i; }
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float oa[NB], ov[NB];
        int oi[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            oa[b] = __shfl_xor(ba[b], m, 64);
            ov[b] = __shfl_xor(bv[b], m, 64);
            oi[b] = __shfl_xor(bi[b], m, 64);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (oa[b] > ba[b] || (oa[b] == ba[b] && oi[b] < bi[b])) { ba[b] = oa[b]; bv[b] = ov[b]; bi[b] = oi[b]; }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        packed[b] = 0;
        psum[b] = 0;
        d[b] = 0.0f;
        if (ba[b] != 0.0f) {  // wave-uniform
            const float iscale = -127.0f / bv[b];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int q = (int)rintf(iscale * v[b][i]);
                q = q > 127 ? 127 : q;
                packed[b] |= (uint32_t)(uint8_t)(int8_t)q << (8 * i);
                psum[b] += q;
            }
            d[b] = 1.0f / iscale;
        }
    }
#pragma unroll
    for (int m = 1; m <= 2; m <<= 1)
#pragma unroll
        for (int b = 0; b < NB; ++b) psum[b] += __shfl_xor(psum[b], m, 64);
}

// One q8_K block (q8K_waves' results) into the split layout at activation
// row `orow`, super-block `blk`.
__device__ __forceinline__ void q8K_store_split(char *out, const ActLayout &L, int64_t K, int64_t orow, int64_t blk,
                                                int lane, uint32_t packed, int psum, float d, bool f16) {
    const int64_t e0 = orow * K + blk * QKK + 4 * lane;
    *(uint32_t *)(out + L.qs_off + e0) = packed;
    if (f16) {
        uint32_t h[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c0 = (int)(int8_t)(packed >> (16 * i)), c1 = (int)(int8_t)(packed >> (16 * i + 8));
            h[i] = (uint32_t)f2h((float)c0) | ((uint32_t)f2h((float)c1) << 16);
        }
        *(uint2 *)(out + L.q16_off + e0 * 2) = make_uint2(h[0], h[1]);
    }
    if ((lane & 3) == 0) {
        ((int16_t *)(out + L.sum_off))[orow * (K / 16) + blk * 16 + (lane >> 2)] = (int16_t)psum;
        if (f16) ((uint16_t *)(out + L.b16_off))[orow * (K / 16) + blk * 16 + (lane >> 2)] = f2h((float)psum);
    }
    if (lane == 0) ((float *)(out + L.d_off))[orow * (K / QKK) + blk] = d;
}

// q8_0 (quantize_row_q8_0_ref, ggml-quants.c:276-297) / q8_1 (:302-335) of
// 32-element blocks held by 8 consecutive lanes (8-lane aligned), four
// consecutive elements per lane: v[b] starts at element col[b] of activation
// row `orow` (live[b] false: not stored; whole 8-lane groups agree): amax,
// d = amax/127, f16(d), codes roundf(x * (1/d)) with the unrounded d; q8_1
// also s = f16(code sum * unrounded d). Written to the split layout (d as f32
// of its f16; the sum slot: q8_0 the code sum, q8_1 s as f32). The NB sets'
// reductions are interleaved.
template <int NB, bool Q81>
__device__ __forceinline__ void q80_quads_store_split(const float (&v)[NB][4], const bool (&live)[NB], int lane,
                                                      char *out, const ActLayout &L, int64_t K, int64_t orow,
                                                      const int64_t (&col)[NB], bool f16) {
#pragma clang fp contract(off)
    float amax[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
        amax[b] = fmaxf(fmaxf(fabsf(v[b][0]), fabsf(v[b][1])), fmaxf(fabsf(v[b][2]), fabsf(v[b][3])));
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1)
#pragma unroll
        for (int b = 0; b < NB; ++b) amax[b] = fmaxf(amax[b], __shfl_xor(amax[b], m, 64));
    float d[NB];
    uint32_t packed[NB];
    int s[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        d[b] = amax[b] / 127.0f;
        const float id = d[b] != 0.0f ? 1.0f / d[b] : 0.0f;
        packed[b] = 0;
        s[b] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = (int)roundf(v[b][i] * id);
            packed[b] |= (uint32_t)(uint8_t)(int8_t)q << (8 * i);
            s[b] += q;
        }
    }
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1)
#pragma unroll
        for (int b = 0; b < NB; ++b) s[b] += __shfl_xor(s[b], m, 64);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (!live[b]) continue;
        const int64_t e0 = orow * K + col[b];
        *(uint32_t *)(out + L.qs_off + e0) = packed[b];
        if (f16) {
            uint32_t h[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int c0 = (int)(int8_t)(packed[b] >> (16 * i)), c1 = (int)(int8_t)(packed[b] >> (16 * i + 8));
                h[i] = (uint32_t)f2h((float)c0) | ((uint32_t)f2h((float)c1) << 16);
            }
            *(uint2 *)(out + L.q16_off + e0 * 2) = make_uint2(h[0], h[1]);
        }
        if ((lane & 7) == 0) {
            const int64_t bk = orow * (K / 32) + col[b] / 32;
            ((float *)(out + L.d_off))[bk] = h2f(f2h(d[b]));
            ((int32_t *)(out + L.sum_off))[bk] = Q81 ? __float_as_int(h2f(f2h((float)s[b] * d[b]))) : s[b];
        }
    }
}

// ------------------------------------------------------- wave64 reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations
// and meets the other waves, but leaves its global loads in flight.
// __syncthreads() also drains the outstanding global loads (its workgroup
// fence waits for vmcnt 0), which would stall every load issued ahead of a
// barrier as a prefetch. Global memory written before this barrier is not
// made visible to the other waves.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Every 64-byte line of the first L * 64 bytes of the kernel arguments, read
// by scalar loads in one round (one wait). The compiler spreads its own
// argument loads over the set-up in several rounds, each waiting for the
// last -- about 700 cycles each when the lines are not in the scalar cache,
// as after a weight stream has gone through L2 -- and these then hit. The
// loads and their wait are one statement, so no loaded register is reused
// while its load is in flight. L must not exceed the explicit arguments.
template <int L> __device__ __forceinline__ void kernarg_prefetch() {
    static_assert(L >= 1 && L <= 16, "1 to 16 lines");
    const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    int d[16];
    if constexpr (L == 1) {
        asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]) : "s"(kp) : "memory");
    } else if constexpr (L == 2) {
        asm volatile("s_load_dword %0, %2, 0x0\n\ts_load_dword %1, %2, 0x40\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]) : "s"(kp) : "memory");
    } else if constexpr (L == 3) {
        asm volatile("s_load_dword %0, %3, 0x0\n\ts_load_dword %1, %3, 0x40\n\ts_load_dword %2, %3, 0x80\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]) : "s"(kp) : "memory");
    } else if constexpr (L == 4) {
        asm volatile("s_load_dword %0, %4, 0x0\n\ts_load_dword %1, %4, 0x40\n\ts_load_dword %2, %4, 0x80\n\ts_load_dword %3, %4, 0xc0\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]) : "s"(kp) : "memory");
    } else if constexpr (L == 5) {
        asm volatile("s_load_dword %0, %5, 0x0\n\ts_load_dword %1, %5, 0x40\n\ts_load_dword %2, %5, 0x80\n\ts_load_dword %3, %5, 0xc0\n\ts_load_dword %4, %5, 0x100\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]) : "s"(kp) : "memory");
    } else if constexpr (L == 6) {
        asm volatile("s_load_dword %0, %6, 0x0\n\ts_load_dword %1, %6, 0x40\n\ts_load_dword %2, %6, 0x80\n\ts_load_dword %3, %6, 0xc0\n\ts_load_dword %4, %6, 0x100\n\ts_load_dword %5, %6, 0x140\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]) : "s"(kp) : "memory");
    } else if constexpr (L == 7) {
        asm volatile("s_load_dword %0, %7, 0x0\n\ts_load_dword %1, %7, 0x40\n\ts_load_dword %2, %7, 0x80\n\ts_load_dword %3, %7, 0xc0\n\ts_load_dword %4, %7, 0x100\n\ts_load_dword %5, %7, 0x140\n\ts_load_dword %6, %7, 0x180\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]) : "s"(kp) : "memory");
    } else if constexpr (L == 8) {
        asm volatile("s_load_dword %0, %8, 0x0\n\ts_load_dword %1, %8, 0x40\n\ts_load_dword %2, %8, 0x80\n\ts_load_dword %3, %8, 0xc0\n\ts_load_dword %4, %8, 0x100\n\ts_load_dword %5, %8, 0x140\n\ts_load_dword %6, %8, 0x180\n\ts_load_dword %7, %8, 0x1c0\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]) : "s"(kp) : "memory");
    } else if constexpr (L == 9) {
        asm volatile("s_load_dword %0, %9, 0x0\n\ts_load_dword %1, %9, 0x40\n\ts_load_dword %2, %9, 0x80\n\ts_load_dword %3, %9, 0xc0\n\ts_load_dword %4, %9, 0x100\n\ts_load_dword %5, %9, 0x140\n\ts_load_dword %6, %9, 0x180\n\ts_load_dword %7, %9, 0x1c0\n\ts_load_dword %8, %9, 0x200\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]) : "s"(kp) : "memory");
    } else if constexpr (L == 10) {
        asm volatile("s_load_dword %0, %10, 0x0\n\ts_load_dword %1, %10, 0x40\n\ts_load_dword %2, %10, 0x80\n\ts_load_dword %3, %10, 0xc0\n\ts_load_dword %4, %10, 0x100\n\ts_load_dword %5, %10, 0x140\n\ts_load_dword %6, %10, 0x180\n\ts_load_dword %7, %10, 0x1c0\n\ts_load_dword %8, %10, 0x200\n\ts_load_dword %9, %10, 0x240\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]) : "s"(kp) : "memory");
    } else if constexpr (L == 11) {
        asm volatile("s_load_dword %0, %11, 0x0\n\ts_load_dword %1, %11, 0x40\n\ts_load_dword %2, %11, 0x80\n\ts_load_dword %3, %11, 0xc0\n\ts_load_dword %4, %11, 0x100\n\ts_load_dword %5, %11, 0x140\n\ts_load_dword %6, %11, 0x180\n\ts_load_dword %7, %11, 0x1c0\n\ts_load_dword %8, %11, 0x200\n\ts_load_dword %9, %11, 0x240\n\ts_load_dword %10, %11, 0x280\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]), "=s"(d[10]) : "s"(kp) : "memory");
    } else if constexpr (L == 12) {
        asm volatile("s_load_dword %0, %12, 0x0\n\ts_load_dword %1, %12, 0x40\n\ts_load_dword %2, %12, 0x80\n\ts_load_dword %3, %12, 0xc0\n\ts_load_dword %4, %12, 0x100\n\ts_load_dword %5, %12, 0x140\n\ts_load_dword %6, %12, 0x180\n\ts_load_dword %7, %12, 0x1c0\n\ts_load_dword %8, %12, 0x200\n\ts_load_dword %9, %12, 0x240\n\ts_load_dword %10, %12, 0x280\n\ts_load_dword %11, %12, 0x2c0\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]), "=s"(d[10]), "=s"(d[11]) : "s"(kp) : "memory");
    } else if constexpr (L == 13) {
        asm volatile("s_load_dword %0, %13, 0x0\n\ts_load_dword %1, %13, 0x40\n\ts_load_dword %2, %13, 0x80\n\ts_load_dword %3, %13, 0xc0\n\ts_load_dword %4, %13, 0x100\n\ts_load_dword %5, %13, 0x140\n\ts_load_dword %6, %13, 0x180\n\ts_load_dword %7, %13, 0x1c0\n\ts_load_dword %8, %13, 0x200\n\ts_load_dword %9, %13, 0x240\n\ts_load_dword %10, %13, 0x280\n\ts_load_dword %11, %13, 0x2c0\n\ts_load_dword %12, %13, 0x300\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]), "=s"(d[10]), "=s"(d[11]), "=s"(d[12]) : "s"(kp) : "memory");
    } else if constexpr (L == 14) {
        asm volatile("s_load_dword %0, %14, 0x0\n\ts_load_dword %1, %14, 0x40\n\ts_load_dword %2, %14, 0x80\n\ts_load_dword %3, %14, 0xc0\n\ts_load_dword %4, %14, 0x100\n\ts_load_dword %5, %14, 0x140\n\ts_load_dword %6, %14, 0x180\n\ts_load_dword %7, %14, 0x1c0\n\ts_load_dword %8, %14, 0x200\n\ts_load_dword %9, %14, 0x240\n\ts_load_dword %10, %14, 0x280\n\ts_load_dword %11, %14, 0x2c0\n\ts_load_dword %12, %14, 0x300\n\ts_load_dword %13, %14, 0x340\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]), "=s"(d[10]), "=s"(d[11]), "=s"(d[12]), "=s"(d[13]) : "s"(kp) : "memory");
    } else if constexpr (L == 15) {
        asm volatile("s_load_dword %0, %15, 0x0\n\ts_load_dword %1, %15, 0x40\n\ts_load_dword %2, %15, 0x80\n\ts_load_dword %3, %15, 0xc0\n\ts_load_dword %4, %15, 0x100\n\ts_load_dword %5, %15, 0x140\n\ts_load_dword %6, %15, 0x180\n\ts_load_dword %7, %15, 0x1c0\n\ts_load_dword %8, %15, 0x200\n\ts_load_dword %9, %15, 0x240\n\ts_load_dword %10, %15, 0x280\n\ts_load_dword %11, %15, 0x2c0\n\ts_load_dword %12, %15, 0x300\n\ts_load_dword %13, %15, 0x340\n\ts_load_dword %14, %15, 0x380\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]), "=s"(d[10]), "=s"(d[11]), "=s"(d[12]), "=s"(d[13]), "=s"(d[14]) : "s"(kp) : "memory");
    } else if constexpr (L == 16) {
        asm volatile("s_load_dword %0, %16, 0x0\n\ts_load_dword %1, %16, 0x40\n\ts_load_dword %2, %16, 0x80\n\ts_load_dword %3, %16, 0xc0\n\ts_load_dword %4, %16, 0x100\n\ts_load_dword %5, %16, 0x140\n\ts_load_dword %6, %16, 0x180\n\ts_load_dword %7, %16, 0x1c0\n\ts_load_dword %8, %16, 0x200\n\ts_load_dword %9, %16, 0x240\n\ts_load_dword %10, %16, 0x280\n\ts_load_dword %11, %16, 0x2c0\n\ts_load_dword %12, %16, 0x300\n\ts_load_dword %13, %16, 0x340\n\ts_load_dword %14, %16, 0x380\n\ts_load_dword %15, %16, 0x3c0\n\ts_waitcnt lgkmcnt(0)" : "=s"(d[0]), "=s"(d[1]), "=s"(d[2]), "=s"(d[3]), "=s"(d[4]), "=s"(d[5]), "=s"(d[6]), "=s"(d[7]), "=s"(d[8]), "=s"(d[9]), "=s"(d[10]), "=s"(d[11]), "=s"(d[12]), "=s"(d[13]), "=s"(d[14]), "=s"(d[15]) : "s"(kp) : "memory");
    }
    (void)d;
}
// Lines of an argument block of `bytes` bytes (the last one starts inside it).
constexpr int kernarg_lines(size_t bytes) { return (int)((bytes + 63) / 64); }

// Sum over the 256 threads of a workgroup, in an order fixed by the lane and
// wave layout (so every kernel that uses it adds the same values alike).
template <typename T> __device__ __forceinline__ T wave_sum_t(T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}
template <typename T> __device__ __forceinline__ T block_sum_t(T v, T *sh) {
    v = wave_sum_t(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const T r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}
// The same sum with LDS-only barriers: global loads issued before it stay in flight.
template <typename T> __device__ __forceinline__ T block_sum_lds(T v, T *sh) {
    v = wave_sum_t(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    lds_barrier();
    const T r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    lds_barrier();
    return r;
}

// ggml's silu in f32 as the CPU's x86-64 build evaluates it (vec.h
// ggml_silu_f32: x / (1 + expf(-x))), then SwiGLU's product with the gate's
// partner (vec.h ggml_vec_swiglu_f32).
__device__ __forceinline__ float swiglu_val(float x, float g) {
#pragma clang fp contract(off)
    return (x / (1.0f + expf(-x))) * g;
}

// ROPE's angle parameters as the lowering derives them from op_params
// (lower.rs:422-466 with ggml_rope_yarn_corr_dims, ggml.c:4369-4381).
struct RopeParams {
    int n_dims = 0, mode = 0;
    float freq_scale = 1.0f, ext_factor = 0.0f, attn_factor = 1.0f, theta_scale = 1.0f, corr0 = 0.0f, corr1 = 0.0f;
};

// cos and sin of pair p's angle at position pos, times the YaRN magnitude
// scale (ggml's rope_yarn, ops.cpp:5820-5835). theta_p = pos * theta_scale^p
// by repeated f32 products, in the order ggml_rope_cache_init
// (ops.cpp:5846-5860) forms it, so the angles match the CPU's bit for bit
// (a powf would differ in the last bits, which at positions in the
// thousands moves the angle visibly). ff: the pair's frequency factor.
// The angle of pair p from tp = pos * theta_scale^p, and the magnitude scale.
__device__ __forceinline__ float rope_theta(float tp, int64_t p, float ff, const RopeParams &r, float &mscale) {
#pragma clang fp contract(off)
    const float theta_extrap = ff == 1.0f ? tp : tp / ff;  // x / 1 is exact: the same value, no division
    float theta = r.freq_scale * theta_extrap;
    mscale = r.attn_factor;
    if (r.ext_factor != 0.0f) {
        const float y = ((float)p - r.corr0) / fmaxf(0.001f, r.corr1 - r.corr0);
        const float ramp_mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * r.ext_factor;
        theta = r.freq_scale * theta_extrap * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / r.freq_scale);
    }
    return theta;
}
__device__ __forceinline__ void rope_cs_sn(float pos, int64_t p, float ff, const RopeParams &r, float &cs, float &sn) {
#pragma clang fp contract(off)
    float tp = pos;
    for (int64_t k = 0; k < p; ++k) tp *= r.theta_scale;
    float mscale;
    const float theta = rope_theta(tp, p, ff, r, mscale);
    cs = cosf(theta) * mscale;
    sn = sinf(theta) * mscale;
}

// the rotated pair (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos)
__device__ __forceinline__ float rope_first(float x0, float x1, float cs, float sn) {
#pragma clang fp contract(off)
    return x0 * cs - x1 * sn;
}
__device__ __forceinline__ float rope_second(float x0, float x1, float cs, float sn) {
#pragma clang fp contract(off)
    return x0 * sn + x1 * cs;
}

// int8x4 dot product with accumulate (v_dot4c_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

}  // namespace tlh

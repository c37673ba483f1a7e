// Test infrastructure only: the CPU oracle (see tlq_oracle.h). Compiled with
// -ffp-contract=off so every a*b+c below rounds twice, as the reference's
// x86-64 build (no FMA) does.
#include "tlq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

// ---------------------------------------------------------------- geometry
// ggml-common.h:194-198 (q4_0: f16 d + 16 nibble bytes), :251-255 (q8_0: f16 d
// + 32 int8), :325-337 (q4_K: f16 d, f16 dmin, 12 packed 6-bit scale/min
// bytes, 128 nibble bytes), :345-352 (q5_K: q4_K's header, 32 bytes of fifth
// bits, 128 nibble bytes), :362-368 (q6_K: 128 low-nibble bytes, 64 bytes of
// 2-bit high parts, 16 int8 scales, f16 d), :370-375 (q8_K: f32 d, 256 int8,
// 16 int16 sums); :298-323 (q2_K: 16 bytes of 4-bit scale | 4-bit min << 4, 64
// bytes of 2-bit codes, f16 d, f16 dmin; q3_K: 32 bytes of high code bits, 64
// bytes of 2-bit low code parts, 12 bytes of packed 6-bit scales, f16 d).
enum { QK32 = 32, QKK = 256, Q4_0_B = 18, Q8_0_B = 34, Q4_K_B = 144, Q5_K_B = 176, Q6_K_B = 210, Q8_K_B = 292,
       Q4_1_B = 20, Q5_0_B = 22, Q5_1_B = 24, Q8_1_B = 36, Q2_K_B = 84, Q3_K_B = 110 };

int64_t tlq_block_elems(int type) {
    switch (type) {
    case TLQ_F32: case TLQ_F16: case TLQ_BF16: return 1;
    case TLQ_Q4_0: case TLQ_Q8_0: case TLQ_Q4_1: case TLQ_Q5_0: case TLQ_Q5_1: case TLQ_Q8_1: return QK32;
    case TLQ_Q2_K: case TLQ_Q3_K: case TLQ_Q4_K: case TLQ_Q5_K: case TLQ_Q6_K: case TLQ_Q8_K: return QKK;
    default: return 0;
    }
}

int64_t tlq_block_bytes(int type) {
    switch (type) {
    case TLQ_F32: return 4;
    case TLQ_F16: case TLQ_BF16: return 2;
    case TLQ_Q4_0: return Q4_0_B;
    case TLQ_Q8_0: return Q8_0_B;
    case TLQ_Q4_1: return Q4_1_B;
    case TLQ_Q5_0: return Q5_0_B;
    case TLQ_Q5_1: return Q5_1_B;
    case TLQ_Q8_1: return Q8_1_B;
    case TLQ_Q4_K: return Q4_K_B;
    case TLQ_Q5_K: return Q5_K_B;
    case TLQ_Q6_K: return Q6_K_B;
    case TLQ_Q8_K: return Q8_K_B;
    case TLQ_Q2_K: return Q2_K_B;
    case TLQ_Q3_K: return Q3_K_B;
    default: return 0;
    }
}

int64_t tlq_row_bytes(int type, int64_t k) {
    int64_t be = tlq_block_elems(type);
    return be ? (k / be) * tlq_block_bytes(type) : 0;
}

int tlq_vec_dot_type(int wtype) {
    switch (wtype) {
    case TLQ_Q4_0: case TLQ_Q8_0: case TLQ_Q5_0: return TLQ_Q8_0;
    case TLQ_Q4_1: case TLQ_Q5_1: return TLQ_Q8_1;
    case TLQ_Q2_K: case TLQ_Q3_K: case TLQ_Q4_K: case TLQ_Q5_K: case TLQ_Q6_K: return TLQ_Q8_K;
    case TLQ_F32: case TLQ_F16: case TLQ_BF16: return wtype;
    default: return -1;
    }
}

// Little-endian field access on packed block bytes.
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline float rdf32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }
static inline void wrf32(uint8_t *p, float f) { memcpy(p, &f, 4); }
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

// ------------------------------------------------------------------- fp16
// IEEE binary16 conversions (semantics of ggml-impl.h:384-430), written from
// the IEEE 754 encodings: half = s | e5 | m10, bias 15; float bias 127.
float tlq_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return bitsf(sign | 0x7f800000u | (m << 13) | (m ? 0x00400000u : 0));
    if (e != 0) return bitsf(sign | ((e + (127 - 15)) << 23) | (m << 13));
    // zero or subnormal: m * 2^-24, exact in binary32
    return bitsf(sign | fbits((float)m * 0x1p-24f));
}

uint16_t tlq_fp32_to_fp16(float f) {
    const uint32_t x = fbits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;   // NaN -> canonical quiet NaN
    if (ax >= 0x477ff000u) return sign | 0x7c00u;  // |f| >= 65520 rounds to infinity
    if (ax >= 0x38800000u) {                       // normal half: |f| >= 2^-14
        const uint32_t r = ax - ((uint32_t)(127 - 15) << 23);
        const uint32_t rounded = r + 0x0fffu + ((r >> 13) & 1u);  // round to nearest even on 13 dropped bits
        return sign | (uint16_t)(rounded >> 13);
    }
    // subnormal half (or zero): count of 2^-24 units, rounded to nearest even
    const int e = (int)(ax >> 23);
    if (e < 102) return sign;  // |f| < 2^-25 (or a binary32 subnormal): rounds to 0
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const int shift = 126 - e;  // value/2^-24 = mant * 2^(e-126), shift in [14, 24]
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

void tlq_fp16_to_fp32_row(const uint16_t *h, float *f, int64_t n) {
    for (int64_t i = 0; i < n; ++i) f[i] = tlq_fp16_to_fp32(h[i]);
}

void tlq_fp32_to_fp16_row(const float *f, uint16_t *h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = tlq_fp32_to_fp16(f[i]);
}

// ggml-impl.h:590-624
float tlq_bf16_to_fp32(uint16_t h) { return bitsf((uint32_t)h << 16); }

uint16_t tlq_fp32_to_bf16(float f) {
    const uint32_t u = fbits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Round to nearest, ties to even, for |v| < 2^22: what ggml's nearest_int
// (ggml-quants.c:621-626) computes with its 1.5*2^23 addend.
static inline int round_even(float v) { return (int)rintf(v); }

// ------------------------------------------------------ weight quantizers
// ggml-quants.c:113-147. Scale from the signed value of largest magnitude
// (first one wins ties), d = max/-8, codes trunc(x/d + 8.5) clamped to 15.
void tlq_quantize_row_q4_0(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / QK32; ++b, x += QK32, y += Q4_0_B) {
        float amax = 0.0f, smax = 0.0f;
        for (int j = 0; j < QK32; ++j) {
            if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); smax = x[j]; }
        }
        const float d = smax / -8;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(y, tlq_fp32_to_fp16(d));
        for (int j = 0; j < QK32 / 2; ++j) {
            int lo = (int8_t)(x[j] * id + 8.5f);
            int hi = (int8_t)(x[j + QK32 / 2] * id + 8.5f);
            if (lo > 15) lo = 15;
            if (hi > 15) hi = 15;
            y[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// make_qkx2_quants (ggml-quants.c:799-878): asymmetric 4-bit fit of n values
// with weights: a grid fit from [min, max], then nstep+1 least-squares refits
// with perturbed inverse scales, keeping the lowest weighted squared error.
// Returns the scale; *neg_min receives -min.
static float fit_scale_min(int n, int nmax, const float *x, const float *w, uint8_t *L, float *neg_min,
                           uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float lo = x[0], hi = x[0];
    float sw = w[0];
    float sx = sw * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sw += w[i];
        sx += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        memset(L, 0, (size_t)n);
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = nmax / (hi - lo);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        int l = round_even(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * L[i] + lo - x[i];
        best += w[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; ++i) {
            int l = round_even(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            sl += w[i] * l;
            sl2 += w[i] * l * l;
            sxl += w[i] * l * x[i];
        }
        const float D = sw * sl2 - sl * sl;
        if (D > 0) {
            float s = (sw * sxl - sx * sl) / D;
            float m = (sl2 * sx - sl * sxl) / D;
            if (m > 0) {
                m = 0;
                s = sxl / sl2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                float diff = s * Laux[i] + m - x[i];
                err += w[i] * (diff * diff);
            }
            if (err < best) {
                memcpy(L, Laux, (size_t)n);
                best = err;
                scale = s;
                lo = m;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

// The 12-byte q4_K scale field (ggml-quants.c:880-887): sub-blocks 0..3 keep
// their 6-bit scale/min in the low 6 bits of bytes 0..3 / 4..7; sub-blocks
// 4..7 keep their low 4 bits in bytes 8..11 (scale low nibble, min high
// nibble) and their top 2 bits in bits 6..7 of bytes 0..3 / 4..7.
static inline void q4k_scale_min(int j, const uint8_t *s, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static inline void q4k_put_scale_min(int j, uint8_t *s, int sc, int mn) {
    if (j < 4) {
        s[j] = (uint8_t)sc;
        s[j + 4] = (uint8_t)mn;
    } else {
        s[j + 4] = (uint8_t)((sc & 0x0f) | ((mn & 0x0f) << 4));
        s[j - 4] |= (uint8_t)((sc >> 4) << 6);
        s[j] |= (uint8_t)((mn >> 4) << 6);
    }
}

// ggml-quants.c:1457-1527: per 32-element sub-block an importance-weighted
// fit (weights sqrt(mean x^2) + |x|), 6-bit quantized scales and mins against
// the super-block maxima, then codes re-derived from the stored scales.
void tlq_quantize_row_q4_K(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    uint8_t L[QKK], Laux[32];
    float w[32], mins[8], scales[8];
    for (int64_t b = 0; b < k / QKK; ++b, x += QKK, y += Q4_K_B) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            const float *xs = x + 32 * j;
            float s2 = 0;
            for (int l = 0; l < 32; ++l) s2 += xs[l] * xs[l];
            const float av = sqrtf(s2 / 32);
            for (int l = 0; l < 32; ++l) w[l] = av + fabsf(xs[l]);
            scales[j] = fit_scale_min(32, 15, xs, w, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        uint8_t *sfield = y + 4;
        for (int j = 0; j < 8; ++j) {
            int ls = (uint8_t)round_even(inv_scale * scales[j]);
            int lm = (uint8_t)round_even(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            q4k_put_scale_min(j, sfield, ls, lm);
        }
        const uint16_t dh = tlq_fp32_to_fp16(max_scale / 63.f);
        const uint16_t mh = tlq_fp32_to_fp16(max_min / 63.f);
        wr16(y, dh);
        wr16(y + 2, mh);
        for (int j = 0; j < 8; ++j) {
            int sc, mn;
            q4k_scale_min(j, sfield, &sc, &mn);
            const float d = tlq_fp16_to_fp32(dh) * sc;
            if (d == 0.0f) continue;
            const float dm = tlq_fp16_to_fp32(mh) * mn;
            for (int i = 0; i < 32; ++i) {
                int l = round_even((x[32 * j + i] + dm) / d);
                L[32 * j + i] = (uint8_t)(l < 0 ? 0 : (l > 15 ? 15 : l));
            }
        }
        uint8_t *q = y + 16;
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l) q[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

// -------------------------------------------------- activation quantizers
// ggml-quants.c:276-297: symmetric int8 with d = amax/127 stored as f16, the
// multiplier computed from the unrounded f32 d, codes roundf (ties away).
void tlq_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / QK32; ++b, x += QK32, y += Q8_0_B) {
        float amax = 0.0f;
        for (int j = 0; j < QK32; ++j) {
            const float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(y, tlq_fp32_to_fp16(d));
        for (int j = 0; j < QK32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    }
}

// ggml-quants.c:302-335 (quantize_row_q8_1_ref; the x86 entry without AVX,
// arch/x86/quants.c:400-501): q8_0's d and codes, plus s = f16(sum of the
// codes * the unrounded d).
void tlq_quantize_row_q8_1(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / QK32; ++b, x += QK32, y += Q8_1_B) {
        float amax = 0.0f;
        for (int j = 0; j < QK32; ++j) {
            const float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(y, tlq_fp32_to_fp16(d));
        int sum = 0;
        for (int j = 0; j < QK32; ++j) {
            const int q = (int)roundf(x[j] * id);
            y[4 + j] = (uint8_t)(int8_t)q;
            sum += q;
        }
        wr16(y + 2, tlq_fp32_to_fp16((float)sum * d));
    }
}

// ggml-quants.c:2768-2804: iscale = -127/(signed value of largest magnitude,
// first wins), codes round-half-even clamped to 127, 16-element code sums,
// d = 1/iscale in f32. An all-zero block stores d = 0 and zero codes; the
// reference leaves its bsums untouched there, we store zeros.
void tlq_quantize_row_q8_K(const float *x, void *vy, int64_t k) {
    uint8_t *y = (uint8_t *)vy;
    for (int64_t b = 0; b < k / QKK; ++b, x += QKK, y += Q8_K_B) {
        float amax = 0, smax = 0;
        for (int j = 0; j < QKK; ++j) {
            const float a = fabsf(x[j]);
            if (a > amax) { amax = a; smax = x[j]; }
        }
        int8_t *qs = (int8_t *)(y + 4);
        if (amax == 0) {
            wrf32(y, 0.0f);
            memset(y + 4, 0, Q8_K_B - 4);
            continue;
        }
        const float iscale = -127.f / smax;
        for (int j = 0; j < QKK; ++j) {
            int v = round_even(iscale * x[j]);
            qs[j] = (int8_t)(v > 127 ? 127 : v);
        }
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += qs[16 * g + i];
            int16_t s16 = (int16_t)s;
            memcpy(y + 4 + QKK + 2 * g, &s16, 2);
        }
        wrf32(y, 1 / iscale);
    }
}

int tlq_quantize_act(int wtype, const float *x, void *y, int64_t k) {
    switch (tlq_vec_dot_type(wtype)) {
    case TLQ_Q8_0: tlq_quantize_row_q8_0(x, y, k); return 0;
    case TLQ_Q8_K: tlq_quantize_row_q8_K(x, y, k); return 0;
    case TLQ_Q8_1: tlq_quantize_row_q8_1(x, y, k); return 0;
    case TLQ_F32: memcpy(y, x, (size_t)k * 4); return 0;
    case TLQ_F16: tlq_fp32_to_fp16_row(x, (uint16_t *)y, k); return 0;
    case TLQ_BF16:
        for (int64_t i = 0; i < k; ++i) ((uint16_t *)y)[i] = tlq_fp32_to_bf16(x[i]);
        return 0;
    default: return -1;
    }
}

// ----------------------------------------------------------- dequantizers
// ggml-quants.c:459-476
void tlq_dequantize_row_q4_0(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q4_0_B, y += QK32) {
        const float d = tlq_fp16_to_fp32(rd16(x));
        for (int j = 0; j < 16; ++j) {
            y[j] = ((x[2 + j] & 0x0f) - 8) * d;
            y[j + 16] = ((x[2 + j] >> 4) - 8) * d;
        }
    }
}

// ggml-quants.c:553-565
void tlq_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q8_0_B, y += QK32) {
        const float d = tlq_fp16_to_fp32(rd16(x));
        for (int j = 0; j < QK32; ++j) y[j] = (int8_t)x[2 + j] * d;
    }
}

// ggml-quants.c:1529-1550: per 64 elements, two sub-blocks sharing 32 code
// bytes (low nibbles first); y = (d*sc)*q - (dmin*m), rounded after each step.
void tlq_dequantize_row_q4_K(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q4_K_B) {
        const float d = tlq_fp16_to_fp32(rd16(x));
        const float dmin = tlq_fp16_to_fp32(rd16(x + 2));
        const uint8_t *q = x + 16;
        for (int c = 0; c < 4; ++c, q += 32) {
            int sc, mn;
            q4k_scale_min(2 * c, x + 4, &sc, &mn);
            const float d1 = d * sc, m1 = dmin * mn;
            q4k_scale_min(2 * c + 1, x + 4, &sc, &mn);
            const float d2 = d * sc, m2 = dmin * mn;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0x0f) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
        }
    }
}

// ggml-quants.c:1731-1756: q4_K's arithmetic on 5-bit codes. Element l of
// sub-block s (32 elements, s = 0..7) has its low 4 bits in nibble s & 1 of
// qs[32 (s / 2) + l] (qs at byte 48) and its fifth bit at bit s of qh[l].
static int q5k_code(const uint8_t *blk, int s, int l) {
    const uint8_t q = blk[48 + 32 * (s / 2) + l];
    return ((s & 1) ? (q >> 4) : (q & 0x0f)) | (((blk[16 + l] >> s) & 1) << 4);
}

void tlq_dequantize_row_q5_K(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q5_K_B) {
        const float d = tlq_fp16_to_fp32(rd16(x));
        const float dmin = tlq_fp16_to_fp32(rd16(x + 2));
        for (int s = 0; s < 8; ++s) {
            int sc, mn;
            q4k_scale_min(s, x + 4, &sc, &mn);
            const float d1 = d * sc, m1 = dmin * mn;
            for (int l = 0; l < 32; ++l) *y++ = d1 * q5k_code(x, s, l) - m1;
        }
    }
}

// ggml-quants.c:1939-1968: per 128-element half, element 32q + l has its low
// 4 bits in ql[l + 32 (q & 1)] (high nibble for q >= 2) and its high 2 bits
// in qh[l] at bit 2q; y = (d * scale) * (code - 32), scale per 16 elements.
static int q6k_code(const uint8_t *blk, int i) {
    const int h = i / 128, e = i % 128, q = e / 32, l = e % 32;
    const uint8_t lo = blk[64 * h + l + 32 * (q & 1)];
    const uint8_t hi = blk[128 + 32 * h + l];
    return (int)(((q >= 2 ? lo >> 4 : lo & 0x0f) | (((hi >> (2 * q)) & 3) << 4))) - 32;
}

void tlq_dequantize_row_q6_K(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q6_K_B) {
        const float d = tlq_fp16_to_fp32(rd16(x + 208));
        const int8_t *sc = (const int8_t *)(x + 192);
        for (int i = 0; i < QKK; ++i) *y++ = d * sc[i / 16] * q6k_code(x, i);
    }
}

// q2_K element i of a super-block (ggml-quants.c:961-989): per 128-element
// half h, element 32j + l keeps its 2-bit code in byte qs[32h + l] at bit 2j;
// sub-block i / 16 has scale = low nibble, min = high nibble of scales[i / 16].
static int q2k_code(const uint8_t *blk, int i) {
    const int h = i / 128, e = i % 128, j = e / 32, l = e % 32;
    return (blk[16 + 32 * h + l] >> (2 * j)) & 3;
}

// y = (d * scale) * code - (dmin * min): two roundings, as the reference.
void tlq_dequantize_row_q2_K(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q2_K_B) {
        const float d = tlq_fp16_to_fp32(rd16(x + 80)), dmin = tlq_fp16_to_fp32(rd16(x + 82));
        for (int i = 0; i < QKK; ++i) {
            const uint8_t sc = x[i / 16];
            const float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
            *y++ = dl * (float)q2k_code(x, i) - ml;
        }
    }
}

// q3_K element i (ggml-quants.c:1305-1351): the low 2 bits as q2_K's (qs at
// byte 32), the third bit in hmask[l] at bit 4h + j; a clear bit subtracts 4,
// so codes are -4..3.
static int q3k_code(const uint8_t *blk, int i) {
    const int h = i / 128, e = i % 128, j = e / 32, l = e % 32;
    const int lo = (blk[32 + 32 * h + l] >> (2 * j)) & 3;
    return lo - (((blk[l] >> (4 * h + j)) & 1) ? 0 : 4);
}

// The 6-bit scale of q3_K sub-block s minus 32, from the 12 packed bytes at
// byte 96: low 4 bits in byte s (s < 8) or the high nibble of byte s - 8,
// high 2 bits in byte 8 + s % 4 at bit 2 (s / 4) (the kmask unpacking of
// ggml-quants.c:1324-1328).
static int q3k_scale(const uint8_t *blk, int s) {
    const uint8_t *sc = blk + 96;
    const int lo = s < 8 ? (sc[s] & 15) : (sc[s - 8] >> 4);
    const int hi = (sc[8 + s % 4] >> (2 * (s / 4))) & 3;
    return (lo | hi << 4) - 32;
}

void tlq_dequantize_row_q3_K(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q3_K_B) {
        const float d = tlq_fp16_to_fp32(rd16(x + 108));
        for (int i = 0; i < QKK; ++i) {
            const float dl = d * (float)q3k_scale(x, i / 16);
            *y++ = dl * (float)q3k_code(x, i);
        }
    }
}

void tlq_dequantize_row_q8_K(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q8_K_B, y += QKK) {
        const float d = rdf32(x);
        for (int j = 0; j < QKK; ++j) y[j] = d * (int8_t)x[4 + j];
    }
}

// ggml-quants.c:479-498: q*d + m per element (two roundings), nibbles as q4_0.
void tlq_dequantize_row_q4_1(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q4_1_B, y += QK32) {
        const float d = tlq_fp16_to_fp32(rd16(x)), m = tlq_fp16_to_fp32(rd16(x + 2));
        for (int j = 0; j < 16; ++j) {
            y[j] = (float)(x[4 + j] & 0x0f) * d + m;
            y[j + 16] = (float)(x[4 + j] >> 4) * d + m;
        }
    }
}

// The fifth bit of element j of a q5 block: bit j of the little-endian qh word.
static inline int q5_code(const uint8_t *qh, const uint8_t *qs, int j) {
    const uint32_t h = (uint32_t)qh[0] | (uint32_t)qh[1] << 8 | (uint32_t)qh[2] << 16 | (uint32_t)qh[3] << 24;
    const int nib = j < 16 ? (qs[j] & 0x0f) : (qs[j - 16] >> 4);
    return nib | (int)((h >> j) & 1u) << 4;
}

// ggml-quants.c:500-524: (q - 16) * d.
void tlq_dequantize_row_q5_0(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q5_0_B, y += QK32) {
        const float d = tlq_fp16_to_fp32(rd16(x));
        for (int j = 0; j < QK32; ++j) y[j] = (float)(q5_code(x + 2, x + 6, j) - 16) * d;
    }
}

// ggml-quants.c:526-551: q * d + m.
void tlq_dequantize_row_q5_1(const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q5_1_B, y += QK32) {
        const float d = tlq_fp16_to_fp32(rd16(x)), m = tlq_fp16_to_fp32(rd16(x + 2));
        for (int j = 0; j < QK32; ++j) y[j] = (float)q5_code(x + 4, x + 8, j) * d + m;
    }
}

int tlq_dequantize_row(int type, const void *x, float *y, int64_t k) {
    switch (type) {
    case TLQ_Q4_1: tlq_dequantize_row_q4_1(x, y, k); return 0;
    case TLQ_Q5_0: tlq_dequantize_row_q5_0(x, y, k); return 0;
    case TLQ_Q5_1: tlq_dequantize_row_q5_1(x, y, k); return 0;
    case TLQ_Q4_0: tlq_dequantize_row_q4_0(x, y, k); return 0;
    case TLQ_Q8_0: tlq_dequantize_row_q8_0(x, y, k); return 0;
    case TLQ_Q4_K: tlq_dequantize_row_q4_K(x, y, k); return 0;
    case TLQ_Q5_K: tlq_dequantize_row_q5_K(x, y, k); return 0;
    case TLQ_Q6_K: tlq_dequantize_row_q6_K(x, y, k); return 0;
    case TLQ_Q8_K: tlq_dequantize_row_q8_K(x, y, k); return 0;
    case TLQ_Q2_K: tlq_dequantize_row_q2_K(x, y, k); return 0;
    case TLQ_Q3_K: tlq_dequantize_row_q3_K(x, y, k); return 0;
    default: return -1;
    }
}

// ----------------------------------------------------------- dot products
// ggml-cpu/quants.c:225-258 (and the identical scalar tail of the x86 entry,
// arch/x86/quants.c:839-853): f32 accumulation of (sumi * dx) * dy per block.
float tlq_vec_dot_q4_0_q8_0(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float acc = 0;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q4_0_B, y += Q8_0_B) {
        int s = 0;
        for (int j = 0; j < 16; ++j) {
            s += ((x[2 + j] & 0x0f) - 8) * (int8_t)y[2 + j];
            s += ((x[2 + j] >> 4) - 8) * (int8_t)y[2 + 16 + j];
        }
        acc += s * tlq_fp16_to_fp32(rd16(x)) * tlq_fp16_to_fp32(rd16(y));
    }
    return acc;
}

// ggml-cpu/quants.c:262-296 (x86 entry without AVX: arch/x86/quants.c:859-915):
// per block sumf += (dx * dy) * sumi + mx * sy.
float tlq_vec_dot_q4_1_q8_1(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float acc = 0;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q4_1_B, y += Q8_1_B) {
        int s = 0;
        for (int j = 0; j < 16; ++j) {
            s += (x[4 + j] & 0x0f) * (int8_t)y[4 + j];
            s += (x[4 + j] >> 4) * (int8_t)y[4 + 16 + j];
        }
        acc += (tlq_fp16_to_fp32(rd16(x)) * tlq_fp16_to_fp32(rd16(y))) * (float)s +
               tlq_fp16_to_fp32(rd16(x + 2)) * tlq_fp16_to_fp32(rd16(y + 2));
    }
    return acc;
}

// ggml-cpu/quants.c:365-406 (arch/x86/quants.c:1142-1219): codes q - 16,
// sumf += (dx * dy) * sumi.
float tlq_vec_dot_q5_0_q8_0(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float acc = 0;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q5_0_B, y += Q8_0_B) {
        int s = 0;
        for (int j = 0; j < QK32; ++j) s += (q5_code(x + 2, x + 6, j) - 16) * (int8_t)y[2 + j];
        acc += (tlq_fp16_to_fp32(rd16(x)) * tlq_fp16_to_fp32(rd16(y))) * (float)s;
    }
    return acc;
}

// ggml-cpu/quants.c:408-449 (arch/x86/quants.c:1222-1305): as q4_1 with 5-bit codes.
float tlq_vec_dot_q5_1_q8_1(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float acc = 0;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q5_1_B, y += Q8_1_B) {
        int s = 0;
        for (int j = 0; j < QK32; ++j) s += q5_code(x + 4, x + 8, j) * (int8_t)y[4 + j];
        acc += (tlq_fp16_to_fp32(rd16(x)) * tlq_fp16_to_fp32(rd16(y))) * (float)s +
               tlq_fp16_to_fp32(rd16(x + 2)) * tlq_fp16_to_fp32(rd16(y + 2));
    }
    return acc;
}

// ggml-cpu/quants.c:451-476: f32 accumulation of sumi * (dx * dy).
float tlq_vec_dot_q8_0_q8_0(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float acc = 0;
    for (int64_t b = 0; b < k / QK32; ++b, x += Q8_0_B, y += Q8_0_B) {
        int s = 0;
        for (int j = 0; j < QK32; ++j) s += (int8_t)x[2 + j] * (int8_t)y[2 + j];
        acc += s * (tlq_fp16_to_fp32(rd16(x)) * tlq_fp16_to_fp32(rd16(y)));
    }
    return acc;
}

void tlq_block_ints_q4_K(const void *vx, const void *vy, int32_t *sum_q, int32_t *sum_m) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    const int8_t *q8 = (const int8_t *)(y + 4);
    int32_t sq = 0, sm = 0;
    for (int s = 0; s < 8; ++s) {
        int sc, mn;
        q4k_scale_min(s, x + 4, &sc, &mn);
        const uint8_t *q = x + 16 + 32 * (s / 2);
        int dot = 0, sum8 = 0;
        for (int l = 0; l < 32; ++l) {
            const int c = (s & 1) ? (q[l] >> 4) : (q[l] & 0x0f);
            dot += c * q8[32 * s + l];
            sum8 += q8[32 * s + l];
        }
        sq += sc * dot;
        sm += mn * sum8;
    }
    *sum_q = sq;
    *sum_m = sm;
}

// ggml-cpu/quants.c:696-773. Integer part per super-block: eight int32 lane
// accumulators (element e feeds lane e % 8) of scale_s * q4 * q8, and the min
// correction sum_g bsums[g] * m_{g/2}. Float part: sums[lane] += (dx*dy) *
// lane, acc -= (dminx*dy) * minsum per block, then acc += sums[0..7] in order.
float tlq_vec_dot_q4_K_q8_K(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float lanes_f[8] = {0};
    float acc = 0;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q4_K_B, y += Q8_K_B) {
        const int8_t *q8 = (const int8_t *)(y + 4);
        int32_t lanes[8] = {0};
        int32_t msum = 0;
        for (int g = 0; g < 16; ++g) {
            int16_t bs;
            memcpy(&bs, y + 4 + QKK + 2 * g, 2);
            int sc, mn;
            q4k_scale_min(g / 2, x + 4, &sc, &mn);
            msum += bs * mn;
        }
        for (int s = 0; s < 8; ++s) {
            int sc, mn;
            q4k_scale_min(s, x + 4, &sc, &mn);
            const uint8_t *q = x + 16 + 32 * (s / 2);
            for (int l = 0; l < 32; ++l) {
                const int c = (s & 1) ? (q[l] >> 4) : (q[l] & 0x0f);
                lanes[l % 8] += sc * (c * q8[32 * s + l]);
            }
        }
        const float dy = rdf32(y);
        const float d = tlq_fp16_to_fp32(rd16(x)) * dy;
        for (int l = 0; l < 8; ++l) lanes_f[l] += d * lanes[l];
        const float dmin = tlq_fp16_to_fp32(rd16(x + 2)) * dy;
        acc -= dmin * msum;
    }
    for (int l = 0; l < 8; ++l) acc += lanes_f[l];
    return acc;
}

// ggml-cpu/quants.c:771-850: the q4_K arithmetic of tlq_vec_dot_q4_K_q8_K on
// 5-bit codes. Per super-block eight int32 lane accumulators (element e feeds
// lane e % 8) of scale_s * (int16)(code * q8), the min correction
// sum_g bsums[g] * m_{g/2}; sums[lane] += (dx*dy) * lane, sumf -= (dminx*dy) *
// minsum, and sums[0..7] added to sumf at the end.
float tlq_vec_dot_q5_K_q8_K(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float sums[8] = {0};
    float sumf = 0;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q5_K_B, y += Q8_K_B) {
        const int8_t *q8 = (const int8_t *)(y + 4);
        int32_t aux32[8] = {0};
        int32_t sumi = 0;
        for (int g = 0; g < 16; ++g) {
            int16_t bs;
            memcpy(&bs, y + 4 + QKK + 2 * g, 2);
            int sc, mn;
            q4k_scale_min(g / 2, x + 4, &sc, &mn);
            sumi += bs * mn;
        }
        for (int s = 0; s < 8; ++s) {
            int sc, mn;
            q4k_scale_min(s, x + 4, &sc, &mn);
            for (int l = 0; l < 32; ++l) aux32[l % 8] += sc * (int16_t)(q5k_code(x, s, l) * q8[32 * s + l]);
        }
        const float dy = rdf32(y);
        const float d = tlq_fp16_to_fp32(rd16(x)) * dy;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = tlq_fp16_to_fp32(rd16(x + 2)) * dy;
        sumf -= dmin * sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

// ggml-cpu/quants.c:851-904. Per super-block: codes in element order, eight
// int32 lane accumulators (element e of each 16-element sub-block feeds lane
// e % 8) of scale_j * (code * q8); float part sums[lane] += (dx * dy) * lane,
// then sumf = sums[0] + ... + sums[7].
float tlq_vec_dot_q6_K_q8_K(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float sums[8] = {0};
    for (int64_t b = 0; b < k / QKK; ++b, x += Q6_K_B, y += Q8_K_B) {
        const int8_t *q8 = (const int8_t *)(y + 4);
        const int8_t *sc = (const int8_t *)(x + 192);
        int32_t aux32[8] = {0};
        for (int j = 0; j < 16; ++j)
            for (int l = 0; l < 16; ++l) {
                const int e = 16 * j + l;
                aux32[l % 8] += sc[j] * (int16_t)(q6k_code(x, e) * q8[e]);
            }
        const float d = tlq_fp16_to_fp32(rd16(x + 208)) * rdf32(y);
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

// ggml-cpu/quants.c:565-615. Per super-block: the min term as an int
// (summs = sum_s bsums_s * min_s), the code sum isum = sum_s scale_s *
// sum_{e in s} q8_e * code_e, then sumf += dall * isum - dmin * summs with
// dall = d8 * d, dmin = d8 * dmin in f32, super-block by super-block.
float tlq_vec_dot_q2_K_q8_K(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float sumf = 0;
    for (int64_t b = 0; b < k / QKK; ++b, x += Q2_K_B, y += Q8_K_B) {
        const int8_t *q8 = (const int8_t *)(y + 4);
        int summs = 0, isum = 0;
        for (int s = 0; s < 16; ++s) {
            const int16_t bsum = (int16_t)rd16(y + 260 + 2 * s);
            summs += bsum * (x[s] >> 4);
            int part = 0;
            for (int l = 0; l < 16; ++l) part += q8[16 * s + l] * q2k_code(x, 16 * s + l);
            isum += (x[s] & 15) * part;
        }
        const float d8 = rdf32(y);
        const float dall = d8 * tlq_fp16_to_fp32(rd16(x + 80));
        const float dmin = d8 * tlq_fp16_to_fp32(rd16(x + 82));
        sumf += dall * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

// ggml-cpu/quants.c:617-694. Per super-block: eight int32 lane accumulators
// (element e of each 16-element sub-block feeds lane e % 8) of (scale_s - 32)
// * (q8 * code) with the int16 product, then sums[lane] += (d * d8) * lane,
// and sumf = sums[0] + ... + sums[7] at the end.
float tlq_vec_dot_q3_K_q8_K(int64_t k, const void *vx, const void *vy) {
    const uint8_t *x = (const uint8_t *)vx, *y = (const uint8_t *)vy;
    float sums[8] = {0};
    for (int64_t b = 0; b < k / QKK; ++b, x += Q3_K_B, y += Q8_K_B) {
        const int8_t *q8 = (const int8_t *)(y + 4);
        int32_t aux32[8] = {0};
        for (int s = 0; s < 16; ++s) {
            const int sc = q3k_scale(x, s);
            for (int l = 0; l < 16; ++l) {
                const int e = 16 * s + l;
                aux32[l % 8] += sc * (int16_t)(q8[e] * q3k_code(x, e));
            }
        }
        const float d = tlq_fp16_to_fp32(rd16(x + 108)) * rdf32(y);
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

// ------------------------------------------------------ float dot products
// vec.cpp:11-143 / :139-262 / :264-352 without GGML_SIMD: f32 products, double sum.
float tlq_vec_dot_f32(int64_t k, const void *vx, const void *vy) {
    const float *x = (const float *)vx, *y = (const float *)vy;
    double s = 0.0;
    for (int64_t i = 0; i < k; ++i) s += (double)(x[i] * y[i]);
    return (float)s;
}

float tlq_vec_dot_f16(int64_t k, const void *vx, const void *vy) {
    const uint16_t *x = (const uint16_t *)vx, *y = (const uint16_t *)vy;
    double s = 0.0;
    for (int64_t i = 0; i < k; ++i) s += (double)(tlq_fp16_to_fp32(x[i]) * tlq_fp16_to_fp32(y[i]));
    return (float)s;
}

float tlq_vec_dot_bf16(int64_t k, const void *vx, const void *vy) {
    const uint16_t *x = (const uint16_t *)vx, *y = (const uint16_t *)vy;
    double s = 0.0;
    for (int64_t i = 0; i < k; ++i) s += (double)(tlq_bf16_to_fp32(x[i]) * tlq_bf16_to_fp32(y[i]));
    return (float)s;
}

// -------------------------------------------------------------- mul_mat
typedef float (*dot_fn)(int64_t, const void *, const void *);

struct mm_job {
    dot_fn dot;
    const uint8_t *w;
    const uint8_t *xq;
    int64_t M, K, N, wrow, xrow;
    float *y;
    int64_t m0, m1;
};

static void *mm_worker(void *p) {
    struct mm_job *j = (struct mm_job *)p;
    for (int64_t n = 0; n < j->N; ++n)
        for (int64_t m = j->m0; m < j->m1; ++m)
            j->y[n * j->M + m] = j->dot(j->K, j->w + m * j->wrow, j->xq + n * j->xrow);
    return NULL;
}

int tlq_mul_mat(int wtype, const void *w, int64_t M, int64_t K, const float *x, int64_t N, float *y,
                int nthreads) {
    dot_fn dot;
    switch (wtype) {
    case TLQ_Q4_0: dot = tlq_vec_dot_q4_0_q8_0; break;
    case TLQ_Q8_0: dot = tlq_vec_dot_q8_0_q8_0; break;
    case TLQ_Q4_K: dot = tlq_vec_dot_q4_K_q8_K; break;
    case TLQ_Q5_K: dot = tlq_vec_dot_q5_K_q8_K; break;
    case TLQ_Q6_K: dot = tlq_vec_dot_q6_K_q8_K; break;
    case TLQ_Q2_K: dot = tlq_vec_dot_q2_K_q8_K; break;
    case TLQ_Q3_K: dot = tlq_vec_dot_q3_K_q8_K; break;
    case TLQ_Q4_1: dot = tlq_vec_dot_q4_1_q8_1; break;
    case TLQ_Q5_0: dot = tlq_vec_dot_q5_0_q8_0; break;
    case TLQ_Q5_1: dot = tlq_vec_dot_q5_1_q8_1; break;
    case TLQ_F32: dot = tlq_vec_dot_f32; break;
    case TLQ_F16: dot = tlq_vec_dot_f16; break;
    case TLQ_BF16: dot = tlq_vec_dot_bf16; break;
    default: return -1;
    }
    const int at = tlq_vec_dot_type(wtype);
    if (K % tlq_block_elems(wtype) != 0) return -2;
    const int64_t xrow = tlq_row_bytes(at, K);
    uint8_t *xq = (uint8_t *)malloc((size_t)(xrow * (N > 0 ? N : 1)));
    if (!xq) return -3;
    for (int64_t n = 0; n < N; ++n) tlq_quantize_act(wtype, x + n * K, xq + n * xrow, K);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (nthreads > M) nthreads = (int)(M > 0 ? M : 1);
    struct mm_job jobs[256];
    pthread_t th[256];
    int joinable[256] = {0};
    const int64_t per = (M + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; ++t) {
        const int64_t m0 = t * per, m1 = (t + 1) * per < M ? (t + 1) * per : M;
        jobs[t] = (struct mm_job){dot, (const uint8_t *)w, xq, M, K, N, tlq_row_bytes(wtype, K), xrow, y, m0, m1};
    }
    for (int t = 1; t < nthreads; ++t) {
        if (jobs[t].m0 >= jobs[t].m1) continue;
        joinable[t] = pthread_create(&th[t], NULL, mm_worker, &jobs[t]) == 0;
        if (!joinable[t]) mm_worker(&jobs[t]);
    }
    mm_worker(&jobs[0]);
    for (int t = 1; t < nthreads; ++t)
        if (joinable[t]) pthread_join(th[t], NULL);
    free(xq);
    return 0;
}

// ------------------------------------------------------- FLASH_ATTN_EXT
// ops.cpp:8468-8700: one query row over keys [ic0, ic1) (no sinks). Leaves the
// running max M, sum S and the f16 accumulator VKQ16 (DV values).
struct fa_shape {
    const void *q, *k, *v, *mask;
    const int64_t *q_nb, *k_nb, *v_nb, *m_ne, *m_nb;
    int64_t DK, DV, rk2, rk3, rv2, rv3;
    float scale, max_bias, softcap, m0, m1;
    uint32_t n_head_log2;
};

static void fa_row_chunk(const struct fa_shape *f, int64_t iq1, int64_t iq2, int64_t iq3, int64_t ic0, int64_t ic1,
                         uint16_t *Q16, uint16_t *VKQ16, float *Mout, float *Sout) {
    const uint32_t h = (uint32_t)iq2;
    const uint32_t nhl2 = f->n_head_log2;
    const float slope = (f->max_bias > 0.0f) ? h < nhl2 ? powf(f->m0, h + 1) : powf(f->m1, 2 * (h - nhl2) + 1)
                                             : 1.0f;
    float S = 0.0f, M = -INFINITY;
    memset(VKQ16, 0, sizeof(uint16_t) * (size_t)f->DV);
    const uint16_t *mp = f->mask ? (const uint16_t *)((const char *)f->mask + iq1 * f->m_nb[1] +
                                                      (iq2 % f->m_ne[2]) * f->m_nb[2] + (iq3 % f->m_ne[3]) * f->m_nb[3])
                                 : NULL;
    const int64_t ik3 = iq3 / f->rk3, ik2 = iq2 / f->rk2, iv3 = iq3 / f->rv3, iv2 = iq2 / f->rv2;
    const float *pq =
        (const float *)((const char *)f->q + iq1 * f->q_nb[1] + iq2 * f->q_nb[2] + iq3 * f->q_nb[3]);
    tlq_fp32_to_fp16_row(pq, Q16, f->DK);  // q_to_vec_dot: f16 for f16 keys
    for (int64_t ic = ic0; ic < ic1; ++ic) {
        const float mv = mp ? slope * tlq_fp16_to_fp32(mp[ic]) : 0.0f;
        if (mv == -INFINITY) continue;
        // ggml_vec_dot_f16, scalar: double sum of f32 products
        const uint16_t *kr =
            (const uint16_t *)((const char *)f->k + ic * f->k_nb[1] + ik2 * f->k_nb[2] + ik3 * f->k_nb[3]);
        double sumf = 0.0;
        for (int64_t d = 0; d < f->DK; ++d) sumf += (double)(tlq_fp16_to_fp32(kr[d]) * tlq_fp16_to_fp32(Q16[d]));
        float s = (float)sumf;
        s = s * f->scale;
        if (f->softcap != 0.0f) s = f->softcap * tanhf(s);
        s += mv;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        const uint16_t *vr =
            (const uint16_t *)((const char *)f->v + ic * f->v_nb[1] + iv2 * f->v_nb[2] + iv3 * f->v_nb[3]);
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            for (int64_t d = 0; d < f->DV; ++d)  // ggml_vec_scale_f16
                VKQ16[d] = tlq_fp32_to_fp16(tlq_fp16_to_fp32(VKQ16[d]) * ms);
        } else {
            vs = expf(s - M);
        }
        for (int64_t d = 0; d < f->DV; ++d)  // ggml_vec_mad_f16
            VKQ16[d] = tlq_fp32_to_fp16(tlq_fp16_to_fp32(VKQ16[d]) + tlq_fp16_to_fp32(vr[d]) * vs);
        S = S * ms + vs;
    }
    *Mout = M;
    *Sout = S;
}

int tlq_flash_attn_ext(const void *q, const int64_t q_ne[4], const int64_t q_nb[4], const void *k,
                       const int64_t k_ne[4], const int64_t k_nb[4], const void *v, const int64_t v_ne[4],
                       const int64_t v_nb[4], const void *mask, const int64_t m_ne[4], const int64_t m_nb[4],
                       void *dst, const int64_t d_nb[4], float scale, float max_bias, float softcap, int nthreads) {
    const int64_t DK = k_ne[0], DV = v_ne[0], N = q_ne[1], nh = q_ne[2], nb = q_ne[3], L = k_ne[1];
    if (q_ne[0] != DK || v_ne[1] != L || nh % k_ne[2] || nb % k_ne[3] || nh % v_ne[2] || nb % v_ne[3]) return -1;
    struct fa_shape f = {q, k, v, mask, q_nb, k_nb, v_nb, m_ne, m_nb, DK, DV, nh / k_ne[2], nb / k_ne[3],
                         nh / v_ne[2], nb / v_ne[3], scale, max_bias, softcap, 0, 0, 0};
    // ops.cpp:8523-8533
    if (softcap != 0) f.scale /= softcap;
    f.n_head_log2 = 1u << (uint32_t)floor(log2((double)(uint32_t)nh));
    f.m0 = powf(2.0f, -(max_bias) / f.n_head_log2);
    f.m1 = powf(2.0f, -(max_bias / 2.0f) / f.n_head_log2);
    const int nth = nthreads > 0 ? nthreads : 1;
    uint16_t *Q16 = malloc(sizeof(uint16_t) * (size_t)(DK > 0 ? DK : 1));
    uint16_t *VKQ16 = malloc(sizeof(uint16_t) * (size_t)(DV > 0 ? DV : 1));
    float *acc = malloc(sizeof(float) * (size_t)(DV > 0 ? DV : 1));
    if (!Q16 || !VKQ16 || !acc) {
        free(Q16);
        free(VKQ16);
        free(acc);
        return -2;
    }
    if (N == 1 && nb == 1 && L >= 512) {
        // split-KV decode (ops.cpp:9115-9145): thread t covers keys
        // [t*chunk, (t+1)*chunk) and leaves (M, S, VKQ) partials, merged in
        // chunk order by ggml_flash_attn_ext_reduce_partials (ops.cpp:8996-9063)
        const int64_t chunk = (L + nth - 1) / nth;
        for (int64_t h = 0; h < nh; ++h) {
            float Mf = -INFINITY, Sf = 0.0f;
            for (int64_t d = 0; d < DV; ++d) acc[d] = 0.0f;
            for (int t = 0; t < nth; ++t) {
                const int64_t ic0 = t * chunk;
                if (ic0 >= L) continue;
                const int64_t ic1 = ic0 + chunk < L ? ic0 + chunk : L;
                float Mc, Sc;
                fa_row_chunk(&f, 0, h, 0, ic0, ic1, Q16, VKQ16, &Mc, &Sc);
                if (Sc == 0.0f) continue;
                const float Mn = fmaxf(Mf, Mc);
                const float so = expf(Mf - Mn), sn = expf(Mc - Mn);
                for (int64_t d = 0; d < DV; ++d) acc[d] = acc[d] * so + tlq_fp16_to_fp32(VKQ16[d]) * sn;
                Sf = Sf * so + Sc * sn;
                Mf = Mn;
            }
            if (Sf != 0.0f) {
                const float S_inv = 1.0f / Sf;
                for (int64_t d = 0; d < DV; ++d) acc[d] *= S_inv;
            }
            memcpy((char *)dst + h * d_nb[1], acc, sizeof(float) * (size_t)DV);
        }
    } else {
        for (int64_t iq3 = 0; iq3 < nb; ++iq3)
            for (int64_t iq2 = 0; iq2 < nh; ++iq2)
                for (int64_t iq1 = 0; iq1 < N; ++iq1) {
                    float M, S;
                    fa_row_chunk(&f, iq1, iq2, iq3, 0, L, Q16, VKQ16, &M, &S);
                    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
                    float *out = (float *)((char *)dst + iq2 * d_nb[1] + iq1 * d_nb[2] + iq3 * d_nb[3]);
                    for (int64_t d = 0; d < DV; ++d) out[d] = tlq_fp16_to_fp32(VKQ16[d]) * S_inv;
                }
    }
    free(Q16);
    free(VKQ16);
    free(acc);
    return 0;
}

// ------------------------------------------------------------ core ops
// The ggml CPU backend's ops around MUL_MAT in a decoder step, on ggml tensors
// given as (data, ne[4], nb[4], type). f32/f16/bf16 data, i32/i64 indices.
static float t_ld(const tlq_t *t, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    const char *p = (const char *)t->data + i0 * t->nb[0] + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
    if (t->ty == TLQ_F16) return tlq_fp16_to_fp32(rd16((const uint8_t *)p));
    if (t->ty == TLQ_BF16) return tlq_bf16_to_fp32(rd16((const uint8_t *)p));
    float f;
    memcpy(&f, p, 4);
    return f;
}
static void t_st(const tlq_t *t, int64_t i0, int64_t i1, int64_t i2, int64_t i3, float v) {
    char *p = (char *)t->data + i0 * t->nb[0] + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
    if (t->ty == TLQ_F16 || t->ty == TLQ_BF16) {
        const uint16_t h = t->ty == TLQ_F16 ? tlq_fp32_to_fp16(v) : tlq_fp32_to_bf16(v);
        memcpy(p, &h, 2);
    } else {
        memcpy(p, &v, 4);
    }
}
static int64_t t_idx(const tlq_t *t, int64_t i0, int64_t i1, int64_t i2) {
    const char *p = (const char *)t->data + i0 * t->nb[0] + i1 * t->nb[1] + i2 * t->nb[2];
    if (t->ty == 27) {
        int64_t v;
        memcpy(&v, p, 8);
        return v;
    }
    int32_t v;
    memcpy(&v, p, 4);
    return v;
}

#define FOR4(t) \
    for (int64_t i3 = 0; i3 < (t)->ne[3]; ++i3) \
        for (int64_t i2 = 0; i2 < (t)->ne[2]; ++i2) \
            for (int64_t i1 = 0; i1 < (t)->ne[1]; ++i1)

// binary-ops.cpp: dst = a (op) b, b repeated; code 0 add, 1 sub, 2 mul, 3 div.
void tlq_core_bin(int code, const tlq_t *a, const tlq_t *b, const tlq_t *d) {
    FOR4(d) for (int64_t i0 = 0; i0 < d->ne[0]; ++i0) {
        const float x = t_ld(a, i0, i1, i2, i3);
        const float y = t_ld(b, i0 % b->ne[0], i1 % b->ne[1], i2 % b->ne[2], i3 % b->ne[3]);
        t_st(d, i0, i1, i2, i3, code == 0 ? x + y : code == 1 ? x - y : code == 2 ? x * y : x / y);
    }
}

// unary-ops.cpp:3-97 op_* and vec.h's ggml_vec_*_f32 (gelu and gelu_quick
// through the f16 tables of ggml-cpu.c:3840-3849, GGML_GELU_FP16), plus the
// lowering's 100 scale (x*s, or x*s + b when b != 0; ops.cpp:4568-4620),
// 101 fill, 102 clamp MAX(MIN(x, max), min), 103 leaky relu, 104 sqr,
// 105 sqrt, 106 sin, 107 cos, 108 log.
static float gelu_f(float x) {
    return 0.5f * x * (1.0f + tanhf(0.79788456080286535587989211986876f * x * (1.0f + 0.044715f * x * x)));
}
static float via_f16(float x) { return tlq_fp16_to_fp32(tlq_fp32_to_fp16(x)); }
static float unary1(int code, float x, float p1, float p2) {
    switch (code) {
    case 0: return fabsf(x);
    case 1: return (x > 0.f) ? 1.f : ((x < 0.f) ? -1.f : 0.f);
    case 2: return -x;
    case 3: return (x > 0.f) ? 1.f : 0.f;
    case 4: return tanhf(x);
    case 5: return (x > 0.f) ? x : expm1f(x);
    case 6: return (x > 0.f) ? x : 0.f;
    case 7: return 1.f / (1.f + expf(-x));
    case 8: return x <= -10.0f ? 0.0f : x >= 10.0f ? x : via_f16(gelu_f(via_f16(x)));
    case 9: {
        const float h = via_f16(x);
        return via_f16(h * (1.0f / (1.0f + expf(-1.702f * h))));
    }
    case 10: return x / (1.0f + expf(-x));
    case 11: return x * fminf(1.0f, fmaxf(0.0f, (x + 3.0f) / 6.0f));
    case 12: return fminf(1.0f, fmaxf(0.0f, (x + 3.0f) / 6.0f));
    case 13: return expf(x);
    case 14: return expf(x) - 1.0f;
    case 15: return (x > 20.0f) ? x : logf(1.0f + expf(x));
    case 16: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
    case 18: return floorf(x);
    case 19: return ceilf(x);
    case 20: return roundf(x);
    case 21: return truncf(x);
    case 100: return p2 == 0.0f ? x * p1 : x * p1 + p2;
    case 101: return p1;
    case 102: {
        const float t = x < p2 ? x : p2;
        return t > p1 ? t : p1;
    }
    case 103: return ((x > 0.f) ? x : 0.f) + p1 * ((x < 0.f) ? x : 0.f);
    case 104: return x * x;
    case 105: return sqrtf(x);
    case 106: return sinf(x);
    case 107: return cosf(x);
    case 108: return logf(x);
    default: return NAN;
    }
}
// On f16 data the CPU reads the gelu table for every input (vec.h ggml_vec_gelu_f16),
// without the f32 path's +-10 cut-offs.
void tlq_core_unary(int code, float p1, float p2, const tlq_t *a, const tlq_t *d) {
    FOR4(d) for (int64_t i0 = 0; i0 < d->ne[0]; ++i0) {
        const float x = t_ld(a, i0, i1, i2, i3);
        t_st(d, i0, i1, i2, i3, code == 8 && a->ty == TLQ_F16 ? via_f16(gelu_f(x)) : unary1(code, x, p1, p2));
    }
}

// ops.cpp:3795-3840 rms_norm_f32: sum of x*x in double, mean = (float)(sum/n).
// ops.cpp:3698-3740 norm_f32 (contiguous rows): mean = (float)sum / n with the
// sum in double (ggml_vec_sum_f32); the variance as ggml_vec_cvar_f32's SSE2
// build forms it (vec.cpp): ((d0^2 + d1^2) + (d2^2 + d3^2)) per group of four
// in f32, accumulated in double, the tail element by element, / n in double.
void tlq_core_norm(int rms, float eps, const tlq_t *a, const tlq_t *d) {
    const int64_t n = a->ne[0];
    FOR4(a) {
        float mean = 0.0f;
        double s2 = 0.0;
        if (rms) {
            for (int64_t i = 0; i < n; ++i) {
                const float v = t_ld(a, i, i1, i2, i3);
                s2 += (double)(v * v);
            }
        } else {
            double s = 0.0;
            for (int64_t i = 0; i < n; ++i) s += (double)t_ld(a, i, i1, i2, i3);
            mean = (float)s / (float)n;
            int64_t i = 0;
            for (; i + 3 < n; i += 4) {
                float q[4];
                for (int j = 0; j < 4; ++j) {
                    const float v = t_ld(a, i + j, i1, i2, i3) - mean;
                    q[j] = v * v;
                }
                s2 += (double)((q[0] + q[1]) + (q[2] + q[3]));
            }
            for (; i < n; ++i) {
                const float v = t_ld(a, i, i1, i2, i3) - mean;
                s2 += (double)(v * v);
            }
        }
        const float var = (float)(s2 / n);
        const float scale = 1.0f / sqrtf(var + eps);
        for (int64_t i = 0; i < n; ++i) t_st(d, i, i1, i2, i3, (t_ld(a, i, i1, i2, i3) - mean) * scale);
    }
}

// ops.cpp get_rows: dst row (i1, i2, i3) = src row idx[i1, i2, i3] of plane (i2, i3).
void tlq_core_get_rows(const tlq_t *a, const tlq_t *idx, const tlq_t *d) {
    float *tmp = malloc(sizeof(float) * (size_t)(a->ne[0] > 0 ? a->ne[0] : 1));
    FOR4(d) {
        const int64_t r = t_idx(idx, i1, i2, i3);
        const char *row = (const char *)a->data + r * a->nb[1] + i2 * a->nb[2] + i3 * a->nb[3];
        if (a->ty == TLQ_F32 || a->ty == TLQ_F16 || a->ty == TLQ_BF16) {
            for (int64_t i = 0; i < d->ne[0]; ++i) {
                tlq_t one = *a;
                one.data = (void *)row;
                t_st(d, i, i1, i2, i3, t_ld(&one, i, 0, 0, 0));
            }
        } else {
            tlq_dequantize_row(a->ty, row, tmp, a->ne[0]);
            for (int64_t i = 0; i < d->ne[0]; ++i) t_st(d, i, i1, i2, i3, tmp[i]);
        }
    }
    free(tmp);
}

// ops.cpp set_rows: src row (i1, i2, i3) to dst row idx[i1, i2 % n1, i3 % n2] of plane (i2, i3).
void tlq_core_set_rows(const tlq_t *a, const tlq_t *idx, const tlq_t *d) {
    FOR4(a) {
        const int64_t r = t_idx(idx, i1, i2 % idx->ne[1], i3 % idx->ne[2]);
        for (int64_t i = 0; i < a->ne[0]; ++i) t_st(d, i, r, i2, i3, t_ld(a, i, i1, i2, i3));
    }
}

// ops.cpp dup: element k of a in row-major order to element k of d.
void tlq_core_cpy(const tlq_t *a, const tlq_t *d) {
    float *tmp = malloc(sizeof(float) * (size_t)(a->ne[0] > 0 ? a->ne[0] : 1));
    int64_t k = 0;
    FOR4(a) {
        const char *row = (const char *)a->data + i1 * a->nb[1] + i2 * a->nb[2] + i3 * a->nb[3];
        if (a->ty == TLQ_F32 || a->ty == TLQ_F16 || a->ty == TLQ_BF16) {
            tlq_t one = *a;
            one.data = (void *)row;
            for (int64_t i = 0; i < a->ne[0]; ++i) tmp[i] = t_ld(&one, i, 0, 0, 0);
        } else {
            tlq_dequantize_row(a->ty, row, tmp, a->ne[0]);
        }
        for (int64_t i = 0; i < a->ne[0]; ++i, ++k) {
            int64_t j = k;
            const int64_t j0 = j % d->ne[0];
            j /= d->ne[0];
            const int64_t j1 = j % d->ne[1];
            j /= d->ne[1];
            t_st(d, j0, j1, j % d->ne[2], j / d->ne[2], tmp[i]);
        }
    }
    free(tmp);
}

// ops.cpp:5822-5860 (rope_yarn_ramp, rope_yarn, ggml_rope_cache_init) and
// :5934-6100 (rope_flt, rotate_pairs): mode 0 normal, 2 neox.
void tlq_core_rope(int mode, int n_dims, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                   float attn_factor, float beta_fast, float beta_slow, const tlq_t *a, const int32_t *pos,
                   const float *ff, const tlq_t *d) {
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    // ggml_rope_yarn_corr_dims (ggml.c)
    const float pi = 3.14159265358979323846f;
    const float start = floorf(n_dims * logf(n_ctx_orig / (beta_fast * 2 * pi)) / (2 * logf(freq_base)));
    const float end = ceilf(n_dims * logf(n_ctx_orig / (beta_slow * 2 * pi)) / (2 * logf(freq_base)));
    const float c0 = fmaxf(0, start), c1 = fminf(n_dims - 1, end);
    const int64_t ne0 = a->ne[0];
    float *cache = malloc(sizeof(float) * (size_t)(ne0 + 2));
    FOR4(a) {
        float theta = (float)pos[i2];
        for (int64_t i0 = 0; i0 < ne0; i0 += 2) {
            const float f = ff ? ff[i0 / 2] : 1.0f;
            const float theta_extrap = theta / f;
            float theta_interp = freq_scale * theta_extrap, th = theta_interp, mscale = attn_factor;
            if (ext_factor != 0.0f) {
                const float y = (i0 / 2 - c0) / fmaxf(0.001f, c1 - c0);
                const float ramp = (1 - fminf(1, fmaxf(0, y))) * ext_factor;
                th = theta_interp * (1 - ramp) + theta_extrap * ramp;
                mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
            }
            cache[i0] = cosf(th) * mscale;
            cache[i0 + 1] = sinf(th) * mscale;
            theta *= theta_scale;
        }
        for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
            const int64_t ia = mode == 0 ? i0 : i0 / 2, ib = mode == 0 ? i0 + 1 : i0 / 2 + n_dims / 2;
            const float x0 = t_ld(a, ia, i1, i2, i3), x1 = t_ld(a, ib, i1, i2, i3);
            t_st(d, ia, i1, i2, i3, x0 * cache[i0] - x1 * cache[i0 + 1]);
            t_st(d, ib, i1, i2, i3, x0 * cache[i0 + 1] + x1 * cache[i0]);
        }
        for (int64_t i0 = n_dims; i0 < ne0; ++i0) t_st(d, i0, i1, i2, i3, t_ld(a, i0, i1, i2, i3));
    }
    free(cache);
}

// ops.cpp soft_max_f32 (:5460-5560): w = x*scale + slope*mask; y = expf(w - max)
// * (float)(1.0 / sum), sum in double; mask row i1, broadcast over i2/i3.
void tlq_core_soft_max(float scale, float max_bias, const tlq_t *a, const tlq_t *mask, const tlq_t *d) {
    const uint32_t n_head = (uint32_t)a->ne[2];
    const uint32_t nhl2 = 1u << (uint32_t)floor(log2((double)n_head));
    const float m0 = powf(2.0f, -(max_bias) / nhl2), m1 = powf(2.0f, -(max_bias / 2.0f) / nhl2);
    const int64_t n = a->ne[0];
    float *w = malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    FOR4(a) {
        const uint32_t h = (uint32_t)i2;
        const float slope = max_bias > 0.0f ? (h < nhl2 ? powf(m0, h + 1) : powf(m1, 2 * (h - nhl2) + 1)) : 1.0f;
        float mx = -INFINITY;
        for (int64_t i = 0; i < n; ++i) {
            w[i] = t_ld(a, i, i1, i2, i3) * scale;
            if (mask) w[i] += slope * t_ld(mask, i, i1, i2 % mask->ne[2], i3 % mask->ne[3]);
            mx = w[i] > mx ? w[i] : mx;
        }
        double sum = 0.0;
        for (int64_t i = 0; i < n; ++i) {
            w[i] = expf(w[i] - mx);
            sum += (double)w[i];
        }
        const float inv = (float)(1.0 / sum);
        for (int64_t i = 0; i < n; ++i) t_st(d, i, i1, i2, i3, w[i] * inv);
    }
    free(w);
}

// ops.cpp ggml_compute_forward_glu (reglu/geglu/swiglu/geglu_erf/geglu_quick f32)
// with vec.h's ggml_vec_*glu_f32: y = act(x) * g; x, g = a, b (split) or the
// halves of a's rows (x first unless swapped).
void tlq_core_glu(int code, int swapped, const tlq_t *a, const tlq_t *b, const tlq_t *d) {
    const int64_t nc = d->ne[0];
    FOR4(d) for (int64_t i = 0; i < nc; ++i) {
        float x, g;
        if (b) {
            x = t_ld(a, i, i1, i2, i3);
            g = t_ld(b, i, i1, i2, i3);
        } else {
            x = t_ld(a, i + (swapped ? nc : 0), i1, i2, i3);
            g = t_ld(a, i + (swapped ? 0 : nc), i1, i2, i3);
        }
        float y;
        switch (code) {
        case 0: y = x > 0.f ? x * g : 0.f; break;
        case 1: y = x <= -10.0f ? 0.0f : x >= 10.0f ? x * g : via_f16(gelu_f(via_f16(x))) * g; break;
        case 2: y = (x / (1.0f + expf(-x))) * g; break;
        case 4: y = 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)) * g; break;
        case 5: y = unary1(9, x, 0, 0) * g; break;
        default: y = NAN;
        }
        t_st(d, i, i1, i2, i3, y);
    }
}

// vec.h ggml_vec_argmax_f32: the last index of the maximum.
void tlq_core_argmax(const tlq_t *a, int32_t *out) {
    for (int64_t r = 0; r < a->ne[1]; ++r) {
        float mx = -INFINITY;
        int idx = 0;
        for (int64_t i = 0; i < a->ne[0]; ++i) {
            const float v = t_ld(a, i, r, 0, 0);
            mx = mx > v ? mx : v;
            if (mx == v) idx = (int)i;
        }
        out[r] = idx;
    }
}

// ------------------------------------------------------- paged attention
// Key cache element (block, kv head, dim i, slot s) sits at
// [block][kvh][i/8][s][i%8]; value cache at [block][kvh][i][s]
// (crates/kernels/src/cuda/paged_attn.rs:9-11, x = 16 bytes / sizeof(f16) = 8).
static inline int64_t kidx(int64_t blk, int h, int i, int s, int kvh, int hs, int bs) {
    return (((blk * kvh + h) * (hs / 8) + i / 8) * bs + s) * 8 + (i % 8);
}
static inline int64_t vidx(int64_t blk, int h, int i, int s, int kvh, int hs, int bs) {
    return ((blk * kvh + h) * (int64_t)hs + i) * bs + s;
}

int tlq_paged_attention(uint16_t *out, const uint16_t *q, const uint16_t *kc, const uint16_t *vc, int kvh,
                        float scale, const int32_t *tables, const int32_t *lens, int max_blocks, int seqs,
                        int heads, int hs, int bs) {
    if (kvh <= 0 || heads % kvh != 0 || hs % 8 != 0) return -1;
    int maxlen = 0;
    for (int s = 0; s < seqs; ++s) maxlen = lens[s] > maxlen ? lens[s] : maxlen;
    float *logits = (float *)malloc(sizeof(float) * (size_t)(maxlen > 0 ? maxlen : 1));
    float *qf = (float *)malloc(sizeof(float) * (size_t)hs);
    float *acc = (float *)malloc(sizeof(float) * (size_t)hs);
    if (!logits || !qf || !acc) return -2;
    const int group = heads / kvh;
    for (int s = 0; s < seqs; ++s) {
        const int L = lens[s];
        const int32_t *bt = tables + (int64_t)s * max_blocks;
        for (int h = 0; h < heads; ++h) {
            const int g = h / group;
            for (int i = 0; i < hs; ++i) qf[i] = tlq_fp16_to_fp32(q[((int64_t)s * heads + h) * hs + i]);
            float mx = -INFINITY;
            for (int t = 0; t < L; ++t) {
                const int64_t blk = bt[t / bs];
                float dot = 0;
                for (int i = 0; i < hs; ++i) dot += qf[i] * tlq_fp16_to_fp32(kc[kidx(blk, g, i, t % bs, kvh, hs, bs)]);
                logits[t] = scale * dot;
                if (logits[t] > mx) mx = logits[t];
            }
            float sum = 0;
            for (int t = 0; t < L; ++t) {
                logits[t] = expf(logits[t] - mx);
                sum += logits[t];
            }
            const float inv = 1.f / (sum + 1e-6f);
            for (int i = 0; i < hs; ++i) acc[i] = 0;
            for (int t = 0; t < L; ++t) {
                const float p = tlq_fp16_to_fp32(tlq_fp32_to_fp16(logits[t] * inv));
                const int64_t blk = bt[t / bs];
                for (int i = 0; i < hs; ++i) acc[i] += p * tlq_fp16_to_fp32(vc[vidx(blk, g, i, t % bs, kvh, hs, bs)]);
            }
            for (int i = 0; i < hs; ++i) out[((int64_t)s * heads + h) * hs + i] = tlq_fp32_to_fp16(acc[i]);
        }
    }
    free(logits);
    free(qf);
    free(acc);
    return 0;
}

void tlq_reshape_and_cache(const uint16_t *key, const uint16_t *value, uint16_t *kc, uint16_t *vc,
                           const int64_t *slots, int tokens, int kvh, int hs, int bs) {
    for (int t = 0; t < tokens; ++t) {
        const int64_t slot = slots[t];
        if (slot < 0) continue;
        const int64_t blk = slot / bs;
        const int off = (int)(slot % bs);
        for (int h = 0; h < kvh; ++h)
            for (int i = 0; i < hs; ++i) {
                kc[kidx(blk, h, i, off, kvh, hs, bs)] = key[((int64_t)t * kvh + h) * hs + i];
                vc[vidx(blk, h, i, off, kvh, hs, bs)] = value[((int64_t)t * kvh + h) * hs + i];
            }
    }
}

void tlq_gather_kv(const uint16_t *kc, const uint16_t *vc, const int32_t *bt, int L, int kvh, int hs, int bs,
                   uint16_t *k_out, uint16_t *v_out) {
    for (int h = 0; h < kvh; ++h)
        for (int t = 0; t < L; ++t) {
            const int64_t blk = bt[t / bs];
            for (int i = 0; i < hs; ++i) {
                k_out[((int64_t)h * L + t) * hs + i] = kc[kidx(blk, h, i, t % bs, kvh, hs, bs)];
                v_out[((int64_t)h * L + t) * hs + i] = vc[vidx(blk, h, i, t % bs, kvh, hs, bs)];
            }
        }
}

// Decode GEMV with register-resident activations, gfx950 (N <= 2, K <= 16384,
// K a multiple of 64).
//
// Each lane owns one 64-element unit of K for the whole kernel: its slice of
// the quantized activations lives in VGPRs, and the lane streams the matching
// weight bytes of row after row (q4_K: the 32 code bytes of one chunk plus the
// 16-byte super-block header; q4_0: two 18-byte blocks; q8_0: two 34-byte
// blocks). A wave covers up to 64 units, so a row of K = 4096 is one wave-wide
// contiguous load; for larger K, KSPLIT (2 or 4) waves of a workgroup take
// contiguous K ranges of the same rows and merge their partials through LDS.
//
// FUSED: every wave quantizes its own activation slice in registers
// from the f32 input (the rules of quantize_row_q8_0_ref, ggml-quants.c:276-297,
// and quantize_row_q8_K_ref, :2768-2804; a q8_K super-block is 4 lanes, which
// agree on its signed maximum with two butterflies), so a decode MUL_MAT is
// one launch and no workgroup waits on a barrier before its first weight
// load. Otherwise the codes come from the split scratch a quantize launch
// wrote.
//
// Block products follow the CPU's vec_dot (ggml-cpu/quants.c:225-258,
// :451-476, :696-773): exact int32 sums on v_dot4, scaled in f32.
#include "kernels.hpp"

namespace tlh {

__device__ __forceinline__ void q4k_sm_r(int s, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
    const int sh = 8 * (s & 3);
    const uint32_t b0 = (s0 >> sh) & 0xff, b1 = (s1 >> sh) & 0xff, b2 = (s2 >> sh) & 0xff;
    const int lo_sc = b0 & 63, lo_mn = b1 & 63;
    const int hi_sc = (b2 & 0x0f) | ((b0 >> 6) << 4);
    const int hi_mn = (b2 >> 4) | ((b1 >> 6) << 4);
    sc = s < 4 ? lo_sc : hi_sc;
    mn = s < 4 ? lo_mn : hi_mn;
}

__device__ __forceinline__ uint4 ldu16(const void *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// One lane's 64 activation codes with their scales and code sums.
// q8_0: d0/d1 are the two blocks' (f16-rounded) scales, s0/s1 their sums;
// q8_K: d0 is the super-block scale, s0/s1 the sums of the two 32-element
// halves and b[0..3] of the four 16-element quarters.
struct AUnit {
    int q[16];
    float d0, d1;
    int s0, s1;
    int b[4];
};

// The elements of unit u: two runs of 32 at e0 and e0 + off1. Contiguous 64
// for every type but q6_K, whose 128-element halves keep element e's low 4
// bits in ql[e % 64] (high nibble from e = 64) and its high 2 bits in
// qh[e % 32]: there a unit is the 32-element runs at 32c and 64 + 32c of half
// h, which share ql bytes 32c..32c+31 and all of qh[0..31], so a lane loads
// 64 weight bytes for 64 elements (u = 4 * super-block + 2h + c).
template <int WT> __device__ __forceinline__ int64_t unit_e0(int64_t u) {
    if constexpr (WT == TLH_TYPE_Q6_K) return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * (u & 1);
    return 64 * u;
}
template <int WT> constexpr int unit_off1() { return WT == TLH_TYPE_Q6_K ? 64 : 32; }

template <int AT, int WT>
__device__ __forceinline__ void quantize_unit(const float *xr, int64_t u, bool valid, AUnit &o) {
#pragma clang fp contract(off)
    const int64_t e0 = unit_e0<WT>(u);
    constexpr int OFF1 = unit_off1<WT>();
    float v[64];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid) f = *(const float4 *)(xr + e0 + (i < 8 ? 4 * i : OFF1 + 4 * (i - 8)));
        v[4 * i] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
    if constexpr (AT == TLH_TYPE_Q8_0) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[32 * b + i]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int sum = 0;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                uint32_t packed = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int c = (int)roundf(v[32 * b + 4 * w + i] * id);
                    packed |= (uint32_t)(uint8_t)(int8_t)c << (8 * i);
                    sum += c;
                }
                o.q[8 * b + w] = (int)packed;
            }
            if (b == 0) {
                o.d0 = h2f(f2h(d));
                o.s0 = sum;
            } else {
                o.d1 = h2f(f2h(d));
                o.s1 = sum;
            }
        }
    } else {
        // signed value of largest magnitude in the 256-element super-block,
        // first index on ties: in-lane over 64 (in element order), then across
        // the 4 lanes
        float ba = 0.0f, bv = 0.0f;
        int bi = 1 << 30;
        const int base = (int)(e0 & 255);
#pragma unroll
        for (int i = 0; i < 64; ++i) {
            const float a = fabsf(v[i]);
            if (a > ba) {
                ba = a;
                bv = v[i];
                bi = base + (i < 32 ? i : OFF1 + i - 32);
            }
        }
#pragma unroll
        for (int m = 1; m <= 2; m <<= 1) {
            const float oa = __shfl_xor(ba, m, 64);
            const float ov = __shfl_xor(bv, m, 64);
            const int oi = __shfl_xor(bi, m, 64);
            if (oa > ba || (oa == ba && oi < bi)) {
                ba = oa;
                bv = ov;
                bi = oi;
            }
        }
        float d = 0.0f, iscale = 0.0f;
        if (ba != 0.0f) {
            iscale = -127.0f / bv;
            d = 1.0f / iscale;
        }
        int s[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            uint32_t packed = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int c = 0;
                if (ba != 0.0f) {
                    c = (int)rintf(iscale * v[4 * w + i]);
                    c = c > 127 ? 127 : c;
                }
                packed |= (uint32_t)(uint8_t)(int8_t)c << (8 * i);
                s[w / 4] += c;
            }
            o.q[w] = (int)packed;
        }
        o.d0 = d;
        o.d1 = 0.0f;
        o.s0 = s[0] + s[1];
        o.s1 = s[2] + s[3];
#pragma unroll
        for (int k = 0; k < 4; ++k) o.b[k] = s[k];
    }
}

// Lanes past K read unit 0 (in bounds) and keep zeros: branch-free, so the
// unit stays in registers.
template <int AT, int WT>
__device__ __forceinline__ void load_unit(const ActView g, int64_t arow, int64_t K, int64_t u, bool valid, AUnit &o) {
    const int64_t uc = valid ? u : 0;
    const int64_t e0 = unit_e0<WT>(uc);
    const int8_t *qs = g.qs + arow * K + e0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int4 t = *(const int4 *)(qs + (i < 2 ? 16 * i : unit_off1<WT>() + 16 * (i - 2)));
        o.q[4 * i] = valid ? t.x : 0;
        o.q[4 * i + 1] = valid ? t.y : 0;
        o.q[4 * i + 2] = valid ? t.z : 0;
        o.q[4 * i + 3] = valid ? t.w : 0;
    }
    if constexpr (AT == TLH_TYPE_Q8_0) {
        const float d0 = g.d[arow * (K / 32) + 2 * uc], d1 = g.d[arow * (K / 32) + 2 * uc + 1];
        const int s0 = g.sum32[arow * (K / 32) + 2 * uc], s1 = g.sum32[arow * (K / 32) + 2 * uc + 1];
        o.d0 = valid ? d0 : 0.0f;
        o.d1 = valid ? d1 : 0.0f;
        o.s0 = valid ? s0 : 0;
        o.s1 = valid ? s1 : 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) o.b[k] = 0;
    } else {
        const float d0 = g.d[arow * (K / QKK) + uc / 4];
        o.d0 = valid ? d0 : 0.0f;
        o.d1 = 0.0f;
        const int16_t *b = g.bsums + arow * (K / 16) + e0 / 16;
        const int off = unit_off1<WT>() / 16;  // quarters 2 and 3 start this many bsums further
        o.b[0] = valid ? b[0] : 0;
        o.b[1] = valid ? b[1] : 0;
        o.b[2] = valid ? b[off] : 0;
        o.b[3] = valid ? b[off + 1] : 0;
        o.s0 = o.b[0] + o.b[1];
        o.s1 = o.b[2] + o.b[3];
    }
}

template <int LV>
__device__ __forceinline__ float treduce(float (&v)[1 << LV], int lane, int &vidx) {
    constexpr int V = 1 << LV;
    float w[V];
#pragma unroll
    for (int i = 0; i < V; ++i) w[i] = v[i];
    vidx = 0;
#pragma unroll
    for (int step = 0; step < LV; ++step) {
        const int half = V >> (step + 1);
        const int mask = 32 >> step;
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float keep = upper ? w[half + i] : w[i];
            const float give = upper ? w[i] : w[half + i];
            w[i] = keep + __shfl_xor(give, mask, 64);
        }
        vidx += upper ? half : 0;
    }
    float r = w[0];
#pragma unroll
    for (int m = 32 >> LV; m >= 1; m >>= 1) r += __shfl_xor(r, m, 64);
    return r;
}

template <int X> struct L2 { static constexpr int v = 1 + L2<X / 2>::v; };
template <> struct L2<1> { static constexpr int v = 0; };

// One lane's weight bytes for its unit u of R rows, and their products with
// the lane's activation slice.
template <int WT, int R> struct WRegs;

template <int R> struct WRegs<TLH_TYPE_Q4_K, R> {
    uint4 hd[R], q0[R], q1[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
        const int64_t sb = u >> 2;
        const int j = (int)(u & 3);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + sb * Q4_K_BYTES;
            hd[r] = ldu16(blk);
            q0[r] = ldu16(blk + 16 + 32 * j);
            q1[r] = ldu16(blk + 32 + 32 * j);
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t u, float (&acc)[R][NC]) const {
        const int j = (int)(u & 3);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
            int lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = (int)(w[i] & 0x0f0f0f0fu);
                hi[i] = (int)((w[i] >> 4) & 0x0f0f0f0fu);
            }
            int sclo, mnlo, schi, mnhi;
            q4k_sm_r(2 * j, hd[r].y, hd[r].z, hd[r].w, sclo, mnlo);
            q4k_sm_r(2 * j + 1, hd[r].y, hd[r].z, hd[r].w, schi, mnhi);
            const float d = h2f((uint16_t)(hd[r].x & 0xffff));
            const float dmin = h2f((uint16_t)(hd[r].x >> 16));
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int dl = 0, dh = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    dl = dot4(lo[i], act[n].q[i], dl);
                    dh = dot4(hi[i], act[n].q[8 + i], dh);
                }
                const int S = sclo * dl + schi * dh;
                const int Mn = mnlo * act[n].s0 + mnhi * act[n].s1;
                acc[r][n] += (d * act[n].d0) * (float)S - (dmin * act[n].d0) * (float)Mn;
            }
        }
    }
};

// q5_K (vec_dot_q5_K_q8_K_generic, ggml-cpu/quants.c:771-850): q4_K's
// header and nibbles (at byte 48 + 32j) plus the 32 qh bytes, whose bits 2j
// and 2j + 1 are the fifth bits of the unit's two runs; codes 0..31.
template <int R> struct WRegs<TLH_TYPE_Q5_K, R> {
    uint4 hd[R], q0[R], q1[R], h0[R], h1[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
        const int64_t sb = u >> 2;
        const int j = (int)(u & 3);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + sb * Q5_K_BYTES;
            hd[r] = ldu16(blk);
            h0[r] = ldu16(blk + 16);
            h1[r] = ldu16(blk + 32);
            q0[r] = ldu16(blk + 48 + 32 * j);
            q1[r] = ldu16(blk + 64 + 32 * j);
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t u, float (&acc)[R][NC]) const {
        const int j = (int)(u & 3);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
            const uint32_t h[8] = {h0[r].x, h0[r].y, h0[r].z, h0[r].w, h1[r].x, h1[r].y, h1[r].z, h1[r].w};
            int lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                lo[i] = (int)((w[i] & 0x0f0f0f0fu) | (((h[i] >> (2 * j)) & 0x01010101u) << 4));
                hi[i] = (int)(((w[i] >> 4) & 0x0f0f0f0fu) | (((h[i] >> (2 * j + 1)) & 0x01010101u) << 4));
            }
            int sclo, mnlo, schi, mnhi;
            q4k_sm_r(2 * j, hd[r].y, hd[r].z, hd[r].w, sclo, mnlo);
            q4k_sm_r(2 * j + 1, hd[r].y, hd[r].z, hd[r].w, schi, mnhi);
            const float d = h2f((uint16_t)(hd[r].x & 0xffff));
            const float dmin = h2f((uint16_t)(hd[r].x >> 16));
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int dl = 0, dh = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    dl = dot4(lo[i], act[n].q[i], dl);
                    dh = dot4(hi[i], act[n].q[8 + i], dh);
                }
                const int S = sclo * dl + schi * dh;
                const int Mn = mnlo * act[n].s0 + mnhi * act[n].s1;
                acc[r][n] += (d * act[n].d0) * (float)S - (dmin * act[n].d0) * (float)Mn;
            }
        }
    }
};

// q6_K (vec_dot_q6_K_q8_K_generic, ggml-cpu/quants.c:851-904): the lane's 32
// ql bytes (low nibbles: its first run, high nibbles: its second), the half's
// 32 qh bytes (2-bit fields 2c and 4 + 2c), the 8 scales of the half and d.
// codes = ql | qh << 4 in 0..63; per 16-element sub-block k
// sum (code - 32) * q8 = dot(code, q8) - 32 * bsum_k, then sum scale_k * that
// in int32 and one f32 scaling by d * d8 as the CPU does per super-block.
template <int R> struct WRegs<TLH_TYPE_Q6_K, R> {
    uint4 l0[R], l1[R], h0[R], h1[R];
    uint2 sc[R];
    uint32_t dq[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
        const int64_t sb = u >> 2;
        const int h = (int)((u >> 1) & 1), c = (int)(u & 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + sb * Q6_K_BYTES;
            l0[r] = ldu16(blk + 64 * h + 32 * c);
            l1[r] = ldu16(blk + 64 * h + 32 * c + 16);
            h0[r] = ldu16(blk + 128 + 32 * h);
            h1[r] = ldu16(blk + 128 + 32 * h + 16);
            uint2 s;
            __builtin_memcpy(&s, blk + 192 + 8 * h, 8);
            sc[r] = s;
            uint16_t d;
            __builtin_memcpy(&d, blk + 208, 2);
            dq[r] = d;
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t u, float (&acc)[R][NC]) const {
        const int c = (int)(u & 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t ql[8] = {l0[r].x, l0[r].y, l0[r].z, l0[r].w, l1[r].x, l1[r].y, l1[r].z, l1[r].w};
            const uint32_t qh[8] = {h0[r].x, h0[r].y, h0[r].z, h0[r].w, h1[r].x, h1[r].y, h1[r].z, h1[r].w};
            int code[16];
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                code[w] = (int)((ql[w] & 0x0f0f0f0fu) | (((qh[w] >> (2 * c)) & 0x03030303u) << 4));
                code[8 + w] = (int)(((ql[w] >> 4) & 0x0f0f0f0fu) | (((qh[w] >> (4 + 2 * c)) & 0x03030303u) << 4));
            }
            // this unit's sub-blocks: 2c, 2c + 1 (first run) and 4 + 2c, 5 + 2c (second) of the half
            const uint32_t sw = c ? (sc[r].x >> 16) | (sc[r].y & 0xffff0000u) : (sc[r].x & 0xffffu) | (sc[r].y << 16);
            const float d = h2f((uint16_t)dq[r]);
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int tot = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    int s = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) s = dot4(code[4 * k + i], act[n].q[4 * k + i], s);
                    const int scale = (int)(int8_t)((sw >> (8 * k)) & 0xff);
                    tot += scale * (s - 32 * act[n].b[k]);
                }
                acc[r][n] += (d * act[n].d0) * (float)tot;
            }
        }
    }
};

template <int R> struct WRegs<TLH_TYPE_Q4_0, R> {
    uint4 w0[R], w1[R];
    float dw0[R], dw1[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + u * (2 * Q4_0_BYTES);
            dw0[r] = h2f(*(const uint16_t *)blk);
            w0[r] = ldu16(blk + 2);
            dw1[r] = h2f(*(const uint16_t *)(blk + Q4_0_BYTES));
            w1[r] = ldu16(blk + Q4_0_BYTES + 2);
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t, float (&acc)[R][NC]) const {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t wa[4] = {w0[r].x, w0[r].y, w0[r].z, w0[r].w};
            const uint32_t wb[4] = {w1[r].x, w1[r].y, w1[r].z, w1[r].w};
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int s0 = 0, s1 = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s0 = dot4((int)(wa[i] & 0x0f0f0f0fu), act[n].q[i], s0);
                    s0 = dot4((int)((wa[i] >> 4) & 0x0f0f0f0fu), act[n].q[4 + i], s0);
                    s1 = dot4((int)(wb[i] & 0x0f0f0f0fu), act[n].q[8 + i], s1);
                    s1 = dot4((int)((wb[i] >> 4) & 0x0f0f0f0fu), act[n].q[12 + i], s1);
                }
                s0 -= 8 * act[n].s0;  // codes are nibble - 8
                s1 -= 8 * act[n].s1;
                acc[r][n] += ((float)s0 * dw0[r]) * act[n].d0;
                acc[r][n] += ((float)s1 * dw1[r]) * act[n].d1;
            }
        }
    }
};

template <int R> struct WRegs<TLH_TYPE_Q8_0, R> {
    uint4 w0[R], w1[R], w2[R], w3[R];
    float dw0[R], dw1[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + u * (2 * Q8_0_BYTES);
            dw0[r] = h2f(*(const uint16_t *)blk);
            w0[r] = ldu16(blk + 2);
            w1[r] = ldu16(blk + 18);
            dw1[r] = h2f(*(const uint16_t *)(blk + Q8_0_BYTES));
            w2[r] = ldu16(blk + Q8_0_BYTES + 2);
            w3[r] = ldu16(blk + Q8_0_BYTES + 18);
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t, float (&acc)[R][NC]) const {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t wv[16] = {w0[r].x, w0[r].y, w0[r].z, w0[r].w, w1[r].x, w1[r].y, w1[r].z, w1[r].w,
                                     w2[r].x, w2[r].y, w2[r].z, w2[r].w, w3[r].x, w3[r].y, w3[r].z, w3[r].w};
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int s0 = 0, s1 = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    s0 = dot4((int)wv[i], act[n].q[i], s0);
                    s1 = dot4((int)wv[8 + i], act[n].q[8 + i], s1);
                }
                acc[r][n] += (float)s0 * (dw0[r] * act[n].d0);
                acc[r][n] += (float)s1 * (dw1[r] * act[n].d1);
            }
        }
    }
};

// PIPE: double-buffer the weight registers so the next row block's loads are
// in flight while this one is multiplied (for grids that loop over many row
// blocks; it costs the registers of a second weight set).
template <int WT, int NC, int R, bool FUSED, bool PIPE>
__global__ void __launch_bounds__(256) k_gemv_reg(const MatmulArgs a, const float *__restrict__ x,
                                                  int64_t x_row_bytes, int ksplit, int upw) {
    constexpr int AT = vec_dot_type(WT);
    constexpr int V = R * NC;
    constexpr int LV = L2<V>::v + ((V & (V - 1)) ? 1 : 0);
    constexpr int VP = 1 << LV;
    __shared__ float part[4][VP];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int groups = 4 / ksplit;
    const int grp = wave / ksplit, kw = wave % ksplit;
    const int64_t K = a.K;
    const int64_t units = K / 64;
    const int64_t u = (int64_t)kw * upw + lane;
    const bool uvalid = lane < upw && u < units;
    const int64_t batch = blockIdx.z;
    const int64_t i12 = batch % a.ne12, i13 = batch / a.ne12;
    const uint8_t *W = a.w + (i12 / a.r2) * a.w_nb2 + (i13 / a.r3) * a.w_nb3;
    const int64_t arow0 = a.n0 + a.N_total * batch;
    const int64_t rows_per_block = (int64_t)groups * R;

    // segment of launch row m (a.nseg > 0): which matrix it belongs to
    auto seg_of = [&](int64_t m) { return (int)(m >= a.seg_m0[1]) + (int)(a.nseg > 2 && m >= a.seg_m0[2]); };
    auto row_ptrs = [&](int64_t rb, const uint8_t *(&wrow)[R]) {
        const int64_t m0 = rb * rows_per_block + (int64_t)grp * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;  // clamp: loads in bounds, store skipped
            if (a.nseg > 0) {
                const int sg = seg_of(m);
                wrow[r] = a.seg_w[sg] + (m - a.seg_m0[sg]) * a.seg_w_nb1[sg];
            } else {
                wrow[r] = W + m * a.w_nb1;
            }
        }
    };


    // the first row block's weights are requested before the activation
    // slice is read and quantized, so the two memory latencies overlap
    WRegs<WT, R> cur;
    int64_t rb = blockIdx.x;
    bool have = rb * rows_per_block < a.M;
    if (have && uvalid) {
        const uint8_t *wrow[R];
        row_ptrs(rb, wrow);
        cur.load(wrow, u);
    }

    AUnit act[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) {
        const int64_t arow = arow0 + (n < a.N ? n : a.N - 1);
        if constexpr (FUSED) {
            quantize_unit<AT, WT>((const float *)((const char *)x + arow * x_row_bytes), u, uvalid, act[n]);
        } else {
            const ActView g = act_view(a.act, AT, K, a.N_total * a.ne12 * a.ne13);
            load_unit<AT, WT>(g, arow, K, u, uvalid, act[n]);
        }
    }

    char *dbase = a.nseg > 0 ? nullptr : (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
    auto store = [&](int64_t m, int n, float v) {
        if (a.nseg > 0) {
            const int sg = seg_of(m);
            a.seg_dst[sg][m - a.seg_m0[sg]] = v;
        } else {
            *(float *)(dbase + (a.n0 + n) * a.d_nb1 + m * 4) = v;
        }
    };
    while (have) {
        const int64_t rb_next = rb + gridDim.x;
        const bool have_next = rb_next * rows_per_block < a.M;
        WRegs<WT, R> nxt;
        if constexpr (PIPE) {
            if (have_next && uvalid) {
                const uint8_t *wrow[R];
                row_ptrs(rb_next, wrow);
                nxt.load(wrow, u);
            }
        }
        float acc[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int n = 0; n < NC; ++n) acc[r][n] = 0.0f;
        if (uvalid) cur.template compute<NC>(act, u, acc);

        const int64_t m0 = rb * rows_per_block + (int64_t)grp * R;
        float vals[VP];
#pragma unroll
        for (int i = 0; i < VP; ++i) vals[i] = i < V ? acc[i / NC][i % NC] : 0.0f;
        int vi;
        const float tot = treduce<LV>(vals, lane, vi);
        const bool holder = (lane & ((64 / VP) - 1)) == 0;
        if (ksplit == 1) {
            if (holder && vi < V) {
                const int r = vi / NC, n = vi % NC;
                if (m0 + r < a.M && n < a.N) store(m0 + r, n, tot);
            }
        } else {
            if (holder) part[wave][vi] = tot;
            lds_barrier();
            if (kw == 0 && holder && vi < V) {
                float t = 0.0f;
                for (int s2 = 0; s2 < ksplit; ++s2) t += part[grp * ksplit + s2][vi];
                const int r = vi / NC, n = vi % NC;
                if (m0 + r < a.M && n < a.N) store(m0 + r, n, t);
            }
            lds_barrier();
        }
        if constexpr (PIPE) {
            cur = nxt;
        } else if (have_next && uvalid) {
            const uint8_t *wrow[R];
            row_ptrs(rb_next, wrow);
            cur.load(wrow, u);
        }
        rb = rb_next;
        have = have_next;
    }
}

// Workgroups of `kern` that the device holds at once (cached per kernel).
template <typename Kern> static int64_t resident_blocks(Kern kern, int &cache) {
    if (cache < 0) {
        int dev = 0, cus = 0, nb = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, 256, 0) != hipSuccess || nb < 1) nb = 1;
        cache = cus * nb;
    }
    return cache;
}

template <int WT, int NC, int R, bool FUSED, bool PIPE>
static tlh_status launch_reg_pipe(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                                  int64_t row_blocks, hipStream_t stream) {
    auto kern = k_gemv_reg<WT, NC, R, FUSED, PIPE>;
    static int slots = -1;
    const int64_t batches = a.ne12 * a.ne13;
    int64_t resident = resident_blocks(kern, slots) / (batches > 0 ? batches : 1);
    if (resident < 1) resident = 1;
    const unsigned gx = (unsigned)(row_blocks < resident ? row_blocks : resident);
    hipLaunchKernelGGL(kern, dim3(gx, 1, (unsigned)batches), dim3(256), 0, stream, a, x, x_row_bytes, ksplit, upw);
    return check_launch("gemv");
}

// A persistent grid walks the row blocks; once each workgroup has several to
// walk, the double-buffered kernel keeps the weight stream busy.
template <int WT, int NC, int R, bool FUSED>
static tlh_status launch_reg_cfg(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                                 hipStream_t stream) {
    static int slots = -1;
    const int groups = 4 / ksplit;
    const int64_t row_blocks = (a.M + (int64_t)groups * R - 1) / ((int64_t)groups * R);
    const int64_t batches = a.ne12 * a.ne13 > 0 ? a.ne12 * a.ne13 : 1;
    const int64_t resident = resident_blocks(k_gemv_reg<WT, NC, R, FUSED, false>, slots);
    if (row_blocks * batches > 2 * resident)
        return launch_reg_pipe<WT, NC, R, FUSED, true>(a, x, x_row_bytes, ksplit, upw, row_blocks, stream);
    return launch_reg_pipe<WT, NC, R, FUSED, false>(a, x, x_row_bytes, ksplit, upw, row_blocks, stream);
}

template <int WT, int NC, bool FUSED>
static tlh_status launch_reg_nc(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                                hipStream_t stream) {
    // q6_K holds 19 weight registers per row: two columns take 2 rows per wave
    constexpr int R = ((WT == TLH_TYPE_Q6_K || WT == TLH_TYPE_Q5_K) && NC == 2) ? 2 : NC <= 2 ? 4 : (NC <= 4 ? 2 : 1);
    return launch_reg_cfg<WT, NC, R, FUSED>(a, x, x_row_bytes, ksplit, upw, stream);
}

// N = 1 or 2 only: more columns of register-resident activations (20 VGPRs
// per column) leave too few registers and spill.
template <int WT, bool FUSED>
static tlh_status launch_reg_wt(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                                hipStream_t stream) {
    if (a.N == 1) return launch_reg_nc<WT, 1, FUSED>(a, x, x_row_bytes, ksplit, upw, stream);
    return launch_reg_nc<WT, 2, FUSED>(a, x, x_row_bytes, ksplit, upw, stream);
}

// Geometry of the register-resident GEMV for K: waves per row group and
// units per wave (a multiple of 4 so q8_K super-blocks never straddle waves).
bool gemv_reg_geometry(int64_t K, int &ksplit, int &upw) {
    if (K % 64 != 0) return false;
    const int64_t units = K / 64;
    if (units > 256) return false;
    ksplit = units <= 64 ? 1 : (units <= 128 ? 2 : 4);
    upw = (int)(4 * ((units + 4 * ksplit - 1) / (4 * ksplit)));
    return upw <= 64;
}

tlh_status launch_gemv_reg(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream) {
    int ksplit = 1, upw = 64;
    if (!gemv_reg_geometry(a.K, ksplit, upw)) return set_error(TLH_INVALID, "gemv_reg: K=%lld", (long long)a.K);
    const bool fused = x != nullptr;
    switch (a.wtype) {
    case TLH_TYPE_Q4_0:
        return fused ? launch_reg_wt<TLH_TYPE_Q4_0, true>(a, x, x_row_bytes, ksplit, upw, stream)
                     : launch_reg_wt<TLH_TYPE_Q4_0, false>(a, x, x_row_bytes, ksplit, upw, stream);
    case TLH_TYPE_Q8_0:
        return fused ? launch_reg_wt<TLH_TYPE_Q8_0, true>(a, x, x_row_bytes, ksplit, upw, stream)
                     : launch_reg_wt<TLH_TYPE_Q8_0, false>(a, x, x_row_bytes, ksplit, upw, stream);
    case TLH_TYPE_Q4_K:
        return fused ? launch_reg_wt<TLH_TYPE_Q4_K, true>(a, x, x_row_bytes, ksplit, upw, stream)
                     : launch_reg_wt<TLH_TYPE_Q4_K, false>(a, x, x_row_bytes, ksplit, upw, stream);
    case TLH_TYPE_Q5_K:
        return fused ? launch_reg_wt<TLH_TYPE_Q5_K, true>(a, x, x_row_bytes, ksplit, upw, stream)
                     : launch_reg_wt<TLH_TYPE_Q5_K, false>(a, x, x_row_bytes, ksplit, upw, stream);
    case TLH_TYPE_Q6_K:
        return fused ? launch_reg_wt<TLH_TYPE_Q6_K, true>(a, x, x_row_bytes, ksplit, upw, stream)
                     : launch_reg_wt<TLH_TYPE_Q6_K, false>(a, x, x_row_bytes, ksplit, upw, stream);
    default: return set_error(TLH_UNSUPPORTED, "gemv: weight type %d", a.wtype);
    }
}

}  // namespace tlh

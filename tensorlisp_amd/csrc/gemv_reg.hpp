// Register-resident decode GEMV kernels (templates), shared by gemv_reg.hip
// (q4_0, q8_0, q4_K, q5_K, q6_K with every prologue / epilogue) and
// gemv_reg_q.hip (q4_1, q5_0, q5_1, plain stores), which compile in parallel.
//
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
// In-kernel activations (IN_X, IN_NORM; K <= 4096): each workgroup loads its
// activation column(s), requests its first weights, then quantizes the column
// once into LDS with the rules of quantize_row_q8_0_ref (ggml-quants.c:276-297)
// and quantize_row_q8_K_ref (:2768-2804), so a decode MUL_MAT is one launch.
// IN_NORM forms the column from the executor's [ADD ->] RMS_NORM -> MUL chain
// first. IN_SCRATCH reads the split scratch a quantize launch wrote. The
// outputs leave as f32 rows (OUT_STORE), as SwiGLU of gate / up row pairs
// (OUT_GLU) or through the store epilogue (OUT_EPI: RoPE, f16, cache rows,
// paged pools).
//
// Block products follow the CPU's vec_dot (ggml-cpu/quants.c:225-258,
// :451-476, :696-773): exact int32 sums on v_dot4, scaled in f32.
#pragma once

#include <algorithm>

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
// q8_1: the same with s0/s1 the bits of the blocks' f32 s (f16(sum * d));
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

// ------------------------------------------------ in-kernel activation rows
// A workgroup quantizes each activation column once into LDS, in the layout
// of the split scratch (codes int8 [K], block scales f32, per-block code sums:
// int32 per 32 for q8_0, int16 bsums per 16 for q8_K), and every wave then
// reads its lanes' units from there. Thread t quantizes 16-element groups
// t, t + 256, ...: a q8_K super-block is a team of 16 consecutive threads, a
// q8_0 block a pair. The values and rules are quantize_row_q8_K_ref's
// (ggml-quants.c:2768-2804: the first element of largest magnitude keeps its
// sign, iscale = -127 / max, codes min(127, round-half-even(iscale * x)),
// d = 1 / iscale, zero blocks all zero) and quantize_row_q8_0_ref's
// (:276-297: d = amax / 127, codes roundf(x / d) with the unrounded d, the
// f16-rounded d stored).
struct ActLds {
    int64_t q_off, d_off, s_off, bytes;  // per activation column
};
__host__ __device__ inline ActLds act_lds(int act_type, int64_t K) {
    ActLds L;
    L.q_off = 0;
    L.d_off = align_up(K, 16);
    const int64_t nd = K / (act_type == TLH_TYPE_Q8_K ? QKK : QK);
    L.s_off = align_up(L.d_off + 4 * nd, 16);
    L.bytes = align_up(L.s_off + (act_type == TLH_TYPE_Q8_K ? 2 * (K / 16) : 4 * (K / 32)), 16);
    return L;
}

// A thread's share of one activation column: the 16-element group t (K <=
// 4096: one group per thread), loaded into registers before the weight
// loads are issued, so that quantizing them does not wait for the weights
// (vector loads complete in order). IN_X: the values of x; IN_NORM: x = p + q
// and the norm weight w (K <= 4096).
// Cross-lane moves within a row of 16 lanes by DPP (no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1] exchange lanes 1 and 2 apart; row_half_mirror
// pairs each quad of a half row with the other quad, row_mirror each half row
// with the other. Applied in that order, every step pairs groups of lanes
// that already agree, so the four steps reduce a team of 16 lanes (the first
// step alone a pair).
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL> __device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

// One step of the team search for the first element of largest magnitude:
// take the partner group's (magnitude, value) when larger, or equal and the
// partner group comes first (lower lanes hold earlier elements).
template <int CTRL>
__device__ __forceinline__ void first_max_step(float &ba, float &bv, bool partner_first) {
    const float oa = dpp_mov<CTRL>(ba), ov = dpp_mov<CTRL>(bv);
    if (oa > ba || (oa == ba && partner_first)) ba = oa, bv = ov;
}

// IN_X: x with K <= 4096; IN_NORM: the prologue's p, q, w with K <= 4096.
// (A longer K reads the scratch of a quantize launch: quantizing a whole
// column in every workgroup costs more there than that launch.)
enum { IN_SCRATCH = 0, IN_X = 1, IN_NORM = 2 };
// OUT: how rows leave the kernel (OUT_STORE: f32 rows of dst or the
// segments; OUT_GLU: the GemvPro SwiGLU epilogue; OUT_EPI: the GemvPro
// store epilogue)
enum { OUT_STORE = 0, OUT_GLU = 1, OUT_EPI = 2 };

template <int IN> struct ActRegs {
    static constexpr int G = 1;
    static constexpr int NQ = IN == IN_NORM ? 16 : 1;
    float v[G][16];
    float q[NQ], w[NQ];  // IN_NORM: the ADD's second operand (or x again) and the norm weight
    // Every load is unconditional (an ADD-less chain loads x twice), so that
    // using these values waits for these loads only.
    __device__ __forceinline__ void load(const float *__restrict__ xr, const float *__restrict__ qr,
                                         const float *__restrict__ wr, int64_t K) {
        const int t = threadIdx.x;
        const int64_t groups = K / 16;
        const float *qq = qr ? qr : xr;
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int64_t g = t + 256 * gi;
            const int64_t gc = g < groups ? g : 0;  // in bounds; unused
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 f = *(const float4 *)(xr + 16 * gc + 4 * k);
                v[gi][4 * k] = f.x, v[gi][4 * k + 1] = f.y, v[gi][4 * k + 2] = f.z, v[gi][4 * k + 3] = f.w;
                if constexpr (IN == IN_NORM) {
                    const float4 h = *(const float4 *)(qq + 16 * gc + 4 * k);
                    const float4 ww = *(const float4 *)(wr + 16 * gc + 4 * k);
                    q[4 * k] = h.x, q[4 * k + 1] = h.y, q[4 * k + 2] = h.z, q[4 * k + 3] = h.w;
                    w[4 * k] = ww.x, w[4 * k + 1] = ww.y, w[4 * k + 2] = ww.z, w[4 * k + 3] = ww.w;
                }
            }
        }
    }
    // IN_NORM: x = p + q (with the ADD), then y = (x * scale) * w with scale =
    // 1 / sqrtf((float)(sum of x*x in double / K) + eps), as ggml's ADD,
    // RMS_NORM and MUL form them (the double sum in another order than the
    // CPU's: equal after its rounding to f32 but for sums within 1e-16 of a
    // rounding boundary); x goes to sr.
    __device__ __forceinline__ void norm(bool add, float *__restrict__ sr, int64_t K, float eps, double *shd) {
#pragma clang fp contract(off)
        const int t = threadIdx.x;
        const bool live = t < K / 16;
        if (add) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[0][i] = v[0][i] + q[i];
        }
        double s1 = 0.0;
        if (live) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s1 += (double)(v[0][i] * v[0][i]);
            if (sr) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    *(float4 *)(sr + 16 * t + 4 * k) = make_float4(v[0][4 * k], v[0][4 * k + 1], v[0][4 * k + 2],
                                                                   v[0][4 * k + 3]);
            }
        }
        const float mean = (float)(block_sum_lds(s1, shd) / (double)K);
        const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[0][i] = (v[0][i] * scale) * w[i];
    }
};

template <int AT, int IN>
__device__ void coop_quantize(const ActRegs<IN> &ar, int64_t K, char *lds) {
#pragma clang fp contract(off)
    const ActLds L = act_lds(AT, K);
    int8_t *sq = (int8_t *)(lds + L.q_off);
    float *sd = (float *)(lds + L.d_off);
    const int t = threadIdx.x, lane = t & 63;
    const int64_t groups = K / 16;
#pragma unroll
    for (int gi = 0; gi < ActRegs<IN>::G; ++gi) {
        const int64_t g = t + 256 * gi;
        if (256 * gi + (t & ~(AT == TLH_TYPE_Q8_K ? 15 : 1)) >= groups) continue;  // whole teams drop out
        const float *v = ar.v[gi];
        int c[16];
        if constexpr (AT == TLH_TYPE_Q8_K) {
            // the first element of largest magnitude: within the thread, then
            // across the team (on equal magnitudes the lower lane's is earlier)
            float ba = 0.0f, bv = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float a = fabsf(v[i]);
                if (a > ba) ba = a, bv = v[i];
            }
            first_max_step<DPP_XOR1>(ba, bv, lane & 1);
            first_max_step<DPP_XOR2>(ba, bv, lane & 2);
            first_max_step<DPP_HALF_MIRROR>(ba, bv, lane & 4);
            first_max_step<DPP_MIRROR>(ba, bv, lane & 8);
            float iscale = 0.0f, d = 0.0f;
            if (ba != 0.0f) {
                iscale = -127.0f / bv;
                d = 1.0f / iscale;
            }
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                int q = 0;
                if (ba != 0.0f) {
                    q = (int)rintf(iscale * v[i]);
                    q = q > 127 ? 127 : q;
                }
                c[i] = q;
                sum += q;
            }
            ((int16_t *)(lds + L.s_off))[g] = (int16_t)sum;
            if ((lane & 15) == 0) sd[g / 16] = d;
        } else {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
            amax = fmaxf(amax, dpp_mov<DPP_XOR1>(amax));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                c[i] = (int)roundf(v[i] * id);
                sum += c[i];
            }
            sum += dpp_mov<DPP_XOR1>(sum);
            if ((lane & 1) == 0) {
                sd[g / 2] = h2f(f2h(d));
                // q8_1 (quantize_row_q8_1_ref, ggml-quants.c:302-335) also keeps
                // s = f16(sum * d), with the unrounded d
                ((int32_t *)(lds + L.s_off))[g / 2] =
                    AT == TLH_TYPE_Q8_1 ? __float_as_int(h2f(f2h((float)sum * d))) : sum;
            }
        }
        uint32_t w4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w4[k] = (uint32_t)(uint8_t)c[4 * k] | ((uint32_t)(uint8_t)c[4 * k + 1] << 8) |
                    ((uint32_t)(uint8_t)c[4 * k + 2] << 16) | ((uint32_t)(uint8_t)c[4 * k + 3] << 24);
        *(uint4 *)(sq + 16 * g) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
}

// A lane's unit u from an LDS activation column (zeros when !valid).
template <int AT, int WT>
__device__ __forceinline__ void lds_unit(const char *lds, int64_t K, int64_t u, bool valid, AUnit &o) {
    const ActLds L = act_lds(AT, K);
    const int64_t uc = valid ? u : 0;
    const int e0 = (int)unit_e0<WT>(uc);
    constexpr int OFF1 = unit_off1<WT>();
    const int8_t *sq = (const int8_t *)(lds + L.q_off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int4 t = *(const int4 *)(sq + e0 + (i < 2 ? 16 * i : OFF1 + 16 * (i - 2)));
        o.q[4 * i] = valid ? t.x : 0;
        o.q[4 * i + 1] = valid ? t.y : 0;
        o.q[4 * i + 2] = valid ? t.z : 0;
        o.q[4 * i + 3] = valid ? t.w : 0;
    }
    const float *sd = (const float *)(lds + L.d_off);
    if constexpr (AT == TLH_TYPE_Q8_0 || AT == TLH_TYPE_Q8_1) {
        const int32_t *ss = (const int32_t *)(lds + L.s_off);
        const float d0 = sd[e0 / 32], d1 = sd[e0 / 32 + 1];
        const int s0 = ss[e0 / 32], s1 = ss[e0 / 32 + 1];
        o.d0 = valid ? d0 : 0.0f;
        o.d1 = valid ? d1 : 0.0f;
        o.s0 = valid ? s0 : 0;
        o.s1 = valid ? s1 : 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) o.b[k] = 0;
    } else {
        const int16_t *bs = (const int16_t *)(lds + L.s_off);
        const float d0 = sd[e0 / QKK];
        const int b0 = bs[e0 / 16], b1 = bs[e0 / 16 + 1], b2 = bs[(e0 + OFF1) / 16], b3 = bs[(e0 + OFF1) / 16 + 1];
        o.d0 = valid ? d0 : 0.0f;
        o.d1 = 0.0f;
        o.b[0] = valid ? b0 : 0;
        o.b[1] = valid ? b1 : 0;
        o.b[2] = valid ? b2 : 0;
        o.b[3] = valid ? b3 : 0;
        o.s0 = o.b[0] + o.b[1];
        o.s1 = o.b[2] + o.b[3];
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
    if constexpr (AT == TLH_TYPE_Q8_0 || AT == TLH_TYPE_Q8_1) {
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

// Sum of v over the 64 lanes of a wave, the same in every lane: each row of
// 16 lanes adds by DPP row shifts (an inclusive scan: lane 15 of the row ends
// with the row's sum), then the four row sums are read out of lanes 15, 31,
// 47 and 63 and added in a fixed order. No LDS round trips.
template <int CTRL> __device__ __forceinline__ float dpp_row_shr(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_total(float v) {
    v += dpp_row_shr<0x111>(v);  // row_shr:1
    v += dpp_row_shr<0x112>(v);  // row_shr:2
    v += dpp_row_shr<0x114>(v);  // row_shr:4
    v += dpp_row_shr<0x118>(v);  // row_shr:8
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 47));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 63));
    return (r0 + r1) + (r2 + r3);
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

// q2_K and q3_K: a lane's unit u = 4 * super-block + 2h + c is the 64
// contiguous elements 128h + 64c.. of the super-block, the code runs j = 2c
// and 2c + 1 of half h. Element 32j + l of the half keeps its 2-bit code in
// the half's qs byte l at bit 2j, so the lane loads the half's 32 qs bytes
// and takes bits 4c and 4c + 2 of each. Its four 16-element sub-blocks are
// 8h + 4c .. 8h + 4c + 3.
//
// q2_K (vec_dot_q2_K_q8_K_generic, ggml-cpu/quants.c:565-615): sub-block s
// has scale (low nibble) and min (high nibble) in byte s of the block; per
// super-block the CPU forms isum = sum_s scale_s * sum(q8 * code) and summs =
// sum_s min_s * bsum_s exactly, then (d8 * d) * isum - (d8 * dmin) * summs.
template <int R> struct WRegs<TLH_TYPE_Q2_K, R> {
    uint4 q0[R], q1[R];
    uint32_t sc[R], dm[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
        const int64_t sb = u >> 2;
        const int h = (int)((u >> 1) & 1), c = (int)(u & 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + sb * Q2_K_BYTES;
            q0[r] = ldu16(blk + 16 + 32 * h);
            q1[r] = ldu16(blk + 32 + 32 * h);
            __builtin_memcpy(&sc[r], blk + 8 * h + 4 * c, 4);
            __builtin_memcpy(&dm[r], blk + 80, 4);
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t u, float (&acc)[R][NC]) const {
        const int c = (int)(u & 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
            int code[16];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                code[i] = (int)((w[i] >> (4 * c)) & 0x03030303u);
                code[8 + i] = (int)((w[i] >> (4 * c + 2)) & 0x03030303u);
            }
            const float d = h2f((uint16_t)(dm[r] & 0xffff)), dmin = h2f((uint16_t)(dm[r] >> 16));
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int isum = 0, summs = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    int s = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) s = dot4(code[4 * k + i], act[n].q[4 * k + i], s);
                    const int b = (int)((sc[r] >> (8 * k)) & 0xff);
                    isum += (b & 15) * s;
                    summs += (b >> 4) * act[n].b[k];
                }
                acc[r][n] += (d * act[n].d0) * (float)isum - (dmin * act[n].d0) * (float)summs;
            }
        }
    }
};

// q3_K (vec_dot_q3_K_q8_K_generic, ggml-cpu/quants.c:617-694): the low 2 bits
// as q2_K's (qs at block byte 32), the third bit of element 32j + l of half h
// in hmask byte l at bit 4h + j; code = low | bit << 2 in 0..7 stands for
// code - 4, applied as -4 * bsum per sub-block. Sub-block s has the 6-bit
// scale (low 4 bits: byte s for s < 8, else the high nibble of byte s - 8;
// high 2 bits: byte 8 + s % 4 at bit 2 (s / 4)) minus 32. Per super-block the
// int32 sum of scale * (dot - 4 * bsum), scaled by d * d8.
template <int R> struct WRegs<TLH_TYPE_Q3_K, R> {
    uint4 m0[R], m1[R], q0[R], q1[R];
    uint4 sd[R];  // block bytes 94..109: the 12 scale bytes at 2..13, d at 14..15
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
        const int64_t sb = u >> 2;
        const int h = (int)((u >> 1) & 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + sb * Q3_K_BYTES;
            m0[r] = ldu16(blk);
            m1[r] = ldu16(blk + 16);
            q0[r] = ldu16(blk + 32 + 32 * h);
            q1[r] = ldu16(blk + 48 + 32 * h);
            sd[r] = ldu16(blk + 94);
        }
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t u, float (&acc)[R][NC]) const {
        const int h = (int)((u >> 1) & 1), c = (int)(u & 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
            const uint32_t m[8] = {m0[r].x, m0[r].y, m0[r].z, m0[r].w, m1[r].x, m1[r].y, m1[r].z, m1[r].w};
            const int ba = 4 * h + 2 * c;  // hmask bit of the unit's first run
            int code[16];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                code[i] = (int)(((w[i] >> (4 * c)) & 0x03030303u) | (((m[i] >> ba) & 0x01010101u) << 2));
                code[8 + i] = (int)(((w[i] >> (4 * c + 2)) & 0x03030303u) | (((m[i] >> (ba + 1)) & 0x01010101u) << 2));
            }
            // the unit's four scale bytes: low 4 bits from scale bytes 4c..4c+3
            // (high nibbles for h = 1), high 2 bits from bytes 8..11 at bit
            // 2 (2h + c) = ba
            const uint32_t s0 = (sd[r].x >> 16) | (sd[r].y << 16);  // scale bytes 0..3
            const uint32_t s1 = (sd[r].y >> 16) | (sd[r].z << 16);  // 4..7
            const uint32_t s2 = (sd[r].z >> 16) | (sd[r].w << 16);  // 8..11
            const uint32_t sc4 = (((c ? s1 : s0) >> (4 * h)) & 0x0f0f0f0fu) | (((s2 >> ba) & 0x03030303u) << 4);
            const float d = h2f((uint16_t)(sd[r].w >> 16));
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int tot = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    int s = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) s = dot4(code[4 * k + i], act[n].q[4 * k + i], s);
                    const int scale = (int)((sc4 >> (8 * k)) & 0xff) - 32;
                    tot += scale * (s - 4 * act[n].b[k]);
                }
                acc[r][n] += (d * act[n].d0) * (float)tot;
            }
        }
    }
};

// q4_1 / q5_0 / q5_1 (vec_dot_q4_1_q8_1_generic, _q5_0_q8_0_generic,
// _q5_1_q8_1_generic, ggml-cpu/quants.c:262-296, :365-449): the lane's two
// blocks of 32 as q4_0's, nibble bytes 4i..4i+3 hold elements 4i.. (low) and
// 16 + 4i.. (high), their fifth bits are qh bits 4i.. and 16 + 4i... Per
// block sumi = sum code * q8 exactly (q5_0: codes q - 16 as sum q*q8 - 16 *
// sum q8), then q5_0 adds (d * d8) * sumi and q4_1 / q5_1 (d * d8) * sumi +
// m * s8 in f32, as the CPU's per-block step does.
template <int WT, int R> struct WRegsLegacy {
    static constexpr int BB = block_bytes(WT);
    uint4 w0[R], w1[R];
    uint32_t h0[R], h1[R];    // fifth bits (q5_0 / q5_1)
    uint32_t dm0[R], dm1[R];  // f16 d (and m) of each block
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = wrow[r] + u * (2 * BB);
            uint32_t a, b;
            __builtin_memcpy(&a, blk, 4);
            __builtin_memcpy(&b, blk + BB, 4);
            dm0[r] = a, dm1[r] = b;
            if constexpr (has_qh(WT)) {
                __builtin_memcpy(&h0[r], blk + blk_qh_off(WT), 4);
                __builtin_memcpy(&h1[r], blk + BB + blk_qh_off(WT), 4);
            }
            w0[r] = ldu16(blk + blk_qs_off(WT));
            w1[r] = ldu16(blk + BB + blk_qs_off(WT));
        }
    }
    // one block: its nibble words, fifth bits, and the 8 activation words q
    __device__ __forceinline__ static int block_sum(const uint4 &w, uint32_t h, const int *q) {
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo = wv[i] & 0x0f0f0f0fu, hi = (wv[i] >> 4) & 0x0f0f0f0fu;
            if constexpr (has_qh(WT)) {
                lo |= spread4((h >> (4 * i)) & 0xfu);
                hi |= spread4((h >> (16 + 4 * i)) & 0xfu);
            }
            s = dot4((int)lo, q[i], s);
            s = dot4((int)hi, q[4 + i], s);
        }
        return s;
    }
    template <int NC>
    __device__ __forceinline__ void compute(const AUnit (&act)[NC], int64_t, float (&acc)[R][NC]) const {
#pragma clang fp contract(off)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d0 = h2f((uint16_t)(dm0[r] & 0xffff)), d1 = h2f((uint16_t)(dm1[r] & 0xffff));
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                int s0 = block_sum(w0[r], h0[r], act[n].q);
                int s1 = block_sum(w1[r], h1[r], act[n].q + 8);
                if constexpr (WT == TLH_TYPE_Q5_0) {
                    s0 -= 16 * act[n].s0;  // codes are q - 16
                    s1 -= 16 * act[n].s1;
                    acc[r][n] += (d0 * act[n].d0) * (float)s0;
                    acc[r][n] += (d1 * act[n].d1) * (float)s1;
                } else {
                    const float m0 = h2f((uint16_t)(dm0[r] >> 16)), m1 = h2f((uint16_t)(dm1[r] >> 16));
                    acc[r][n] += (d0 * act[n].d0) * (float)s0 + m0 * __int_as_float(act[n].s0);
                    acc[r][n] += (d1 * act[n].d1) * (float)s1 + m1 * __int_as_float(act[n].s1);
                }
            }
        }
    }
};
template <int R> struct WRegs<TLH_TYPE_Q4_1, R> : WRegsLegacy<TLH_TYPE_Q4_1, R> {};
template <int R> struct WRegs<TLH_TYPE_Q5_0, R> : WRegsLegacy<TLH_TYPE_Q5_0, R> {};
template <int R> struct WRegs<TLH_TYPE_Q5_1, R> : WRegsLegacy<TLH_TYPE_Q5_1, R> {};

// A unit is two 18-byte blocks, 36 bytes at a 4-byte aligned address (the
// launcher checks the weight pointers and strides, gemv_reg_weights_ok):
// three dword-aligned loads, and the first block's codes (bytes 2..17)
// shifted into place, instead of 16-byte loads at 2-byte aligned addresses
// and separate scale loads.
template <int R> struct WRegs<TLH_TYPE_Q4_0, R> {
    uint4 w0[R], w1[R];
    float dw0[R], dw1[R];
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[R], int64_t u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t *blk = (const uint32_t *)(wrow[r] + u * (2 * Q4_0_BYTES));
            const uint4 p0 = *(const uint4 *)blk, p1 = *(const uint4 *)(blk + 4);
            const uint32_t p2 = blk[8];
            dw0[r] = h2f((uint16_t)(p0.x & 0xffff));
            w0[r] = make_uint4(__builtin_amdgcn_alignbyte(p0.y, p0.x, 2), __builtin_amdgcn_alignbyte(p0.z, p0.y, 2),
                               __builtin_amdgcn_alignbyte(p0.w, p0.z, 2), __builtin_amdgcn_alignbyte(p1.x, p0.w, 2));
            dw1[r] = h2f((uint16_t)(p1.x >> 16));
            w1[r] = make_uint4(p1.y, p1.z, p1.w, p2);
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
// IN: where the activation comes from (IN_SCRATCH: the split scratch a
// quantize launch filled; IN_X: src1 rows, quantized by the workgroup into
// LDS; IN_NORM: the GemvPro prologue's rows, likewise). GLU: the GemvPro
// SwiGLU epilogue (rows of a wave pair gate and up rows: R / 2 of each).
template <int WT, int NC, int R, int IN, bool PIPE, int OUT>
__global__ void __launch_bounds__(256) k_gemv_reg(const MatmulArgs a, const float *__restrict__ x,
                                                  int64_t x_row_bytes, int ksplit, int upw, const GemvPro pro) {
    constexpr int AT = vec_dot_type(WT);
    constexpr int V = R * NC;
    constexpr bool GLU = OUT == OUT_GLU;
    static_assert(!GLU || R % 2 == 0, "GLU pairs R / 2 gate rows with R / 2 up rows");
    static_assert(OUT != OUT_EPI || (NC == 1 && R % 2 == 0), "the store epilogue pairs rows of one column");
    __shared__ float part[4][V];
    __shared__ double shd[4];
    extern __shared__ __align__(16) char s_act[];  // IN != IN_SCRATCH: NC activation columns
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // The set-up is branch-free 32-bit arithmetic (the host keeps every count
    // below 2^31): a branch splits the kernel-argument loads into rounds the
    // kernel waits for one after another before its first weight load.
    const int groups = ksplit == 1 ? 4 : ksplit == 2 ? 2 : 1;  // 4 / ksplit
    const int grp = wave / ksplit, kw = wave % ksplit;
    const int64_t K = a.K;
    const int64_t units = K / 64;
    const int64_t u = (int64_t)kw * upw + lane;
    const bool uvalid = lane < upw && u < units;
    const uint32_t batch = blockIdx.z;
    const MmSlice sl = mm_slice(a, batch);
    const uint32_t i12 = (uint32_t)sl.i12, i13 = (uint32_t)sl.i13;
    const uint8_t *W = sl.w;
    const int64_t arow0 = a.n0 + a.N_total * batch;
    // output rows a workgroup covers per step (GLU: rows of h, R / 2 per wave)
    constexpr int RO = GLU ? R / 2 : R;
    const int64_t rows_per_block = (int64_t)groups * RO;

    // segment of launch row m (a.nseg > 0): which matrix it belongs to. The
    // segment fields are picked by selects, never indexed by a run-time value
    // (that would read the kernel arguments with vector loads and a wait).
    auto seg_of = [&](int64_t m) { return (int)(m >= a.seg_m0[1]) + (int)(a.nseg > 2 && m >= a.seg_m0[2]); };
    auto sel = [](int sg, auto x0, auto x1, auto x2) { return sg == 0 ? x0 : sg == 1 ? x1 : x2; };
    auto row_ptrs = [&](int64_t rb, const uint8_t *(&wrow)[R]) {
        const int64_t m0 = rb * rows_per_block + (int64_t)grp * RO;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (GLU) {  // gate rows m0 .. m0 + RO - 1, then the same rows of up
                const int rr = r % RO;
                const int64_t m = m0 + rr < a.M ? m0 + rr : a.M - 1;
                wrow[r] = r < RO ? a.seg_w[0] + m * a.seg_w_nb1[0] : a.seg_w[1] + m * a.seg_w_nb1[1];
            } else {
                const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;  // clamp: loads in bounds, store skipped
                if (a.nseg > 0) {
                    const int sg = seg_of(m);
                    wrow[r] = sel(sg, a.seg_w[0], a.seg_w[1], a.seg_w[2]) +
                              (m - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2])) *
                                  sel(sg, a.seg_w_nb1[0], a.seg_w_nb1[1], a.seg_w_nb1[2]);
                } else {
                    wrow[r] = W + m * a.w_nb1;
                }
            }
        }
    };

    // OUT_EPI: the token's position, cache rows / slots and frequency
    // factors are read before anything else (the epilogue would otherwise
    // wait on cold loads after the products), and the pairs' cos / sin go to
    // LDS while the weights are in flight (written before the quantization's
    // barrier, read after it).
    constexpr int EPI_PAIRS = OUT == OUT_EPI ? 256 : 1;
    __shared__ float s_cs[EPI_PAIRS], s_sn[EPI_PAIRS];
    // raw words, converted only where they are used (a conversion here would
    // wait for the loads): row / slot k is hi:lo (i64) or lo & hi (i32, one
    // word read twice), then the position and four frequency factors
    int32_t e_lo[3] = {0, 0, 0}, e_hi[3] = {0, 0, 0}, e_rpos = 0, e_rff[4] = {0, 0, 0, 0};
    const bool e_rope = OUT == OUT_EPI && (pro.epi.rope[0] | pro.epi.rope[1] | pro.epi.rope[2]);
    if constexpr (OUT == OUT_EPI) {
        // vector loads: a scalar load's wait would cover every scalar load in
        // flight and stall the kernel here (the offset `z` is a zero the
        // compiler cannot see through, so the addresses are per lane); every
        // load is unconditional, from the weights where a pointer is absent,
        // so no branch makes the compiler wait for it either
        const GemvEpi &e = pro.epi;
        const char *any = (const char *)a.seg_w[0];
        int z;
        asm volatile("v_mov_b32 %0, 0" : "=v"(z));
        auto ld32 = [z](const char *p) { return *(const int32_t *)(p + z); };
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const char *ip = e.idx[k] ? e.idx[k] : any;
            e_lo[k] = ld32(ip);
            e_hi[k] = ld32(ip + 4 * e.idx_i64[k]);
        }
        e_rpos = ld32(e.pos ? (const char *)e.pos : any);
        const float *ffp = e.ff ? e.ff : (const float *)any;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = (threadIdx.x & 63) + 64 * i;
            e_rff[i] = ld32((const char *)(ffp + (e.ff && p < e.ne0 / 2 ? p : 0)));
        }
    }
    // In-kernel activations are loaded first, then the first row block's
    // weights are requested, so quantizing waits only for the activations
    // while the weights are in flight.
    ActRegs<IN == IN_SCRATCH ? IN_X : IN> ar[IN == IN_SCRATCH ? 1 : NC];
    if constexpr (IN != IN_SCRATCH) {
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const int64_t arow = arow0 + (n < a.N ? n : a.N - 1);
            if constexpr (IN == IN_NORM)
                ar[n].load((const float *)((const char *)pro.p + arow * pro.p_nb1),
                           pro.q ? (const float *)((const char *)pro.q + arow * pro.q_nb1) : nullptr, pro.w, K);
            else
                ar[n].load((const float *)((const char *)x + arow * x_row_bytes), nullptr, nullptr, K);
        }
    }
    // Weight loads are never predicated: lanes past K load unit 0 (in bounds;
    // their activations are zero) and rows past M are clamped. A load behind a
    // branch would make the compiler wait for every outstanding load where the
    // branch rejoins, instead of only for the ones the next step needs.
    WRegs<WT, R> cur, nxt;
    const int64_t nblocks = ((uint32_t)a.M + (uint32_t)rows_per_block - 1) / (uint32_t)rows_per_block;
    int64_t rb = blockIdx.x;  // the launch never has more workgroups than row blocks
    const int64_t ul = uvalid ? u : 0;
    {
        const uint8_t *wrow[R];
        row_ptrs(rb, wrow);
        cur.load(wrow, ul);
    }
    // double-buffered: every workgroup walks at least two row blocks (the
    // launcher's rule), so the second block is requested before the
    // activation work too
    int64_t rn = rb + gridDim.x;
    if constexpr (PIPE) {
        const uint8_t *wrow[R];
        row_ptrs(rn < nblocks ? rn : rb, wrow);
        nxt.load(wrow, ul);
    }

    AUnit act[NC];
    if constexpr (IN == IN_SCRATCH) {
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const int64_t arow = arow0 + (n < a.N ? n : a.N - 1);
            const ActView g = act_view(a.act, AT, K, a.N_total * a.ne12 * a.ne13);
            load_unit<AT, WT>(g, arow, K, u, uvalid, act[n]);
        }
    } else {
        const ActLds L = act_lds(AT, K);
        const bool writer = blockIdx.x == 0 && blockIdx.z == 0;
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            if constexpr (IN == IN_NORM) {
                const int64_t arow = arow0 + (n < a.N ? n : a.N - 1);
                float *sr = (writer && pro.s && n < a.N) ? (float *)((char *)pro.s + arow * pro.s_nb1) : nullptr;
                ar[n].norm(pro.q != nullptr, sr, K, pro.eps, shd);
            }
            coop_quantize<AT>(ar[n], K, s_act + n * L.bytes);
        }
        lds_barrier();
#pragma unroll
        for (int n = 0; n < NC; ++n) lds_unit<AT, WT>(s_act + n * L.bytes, K, u, uvalid, act[n]);
    }
    if constexpr (OUT == OUT_EPI) {
        // the pairs' cos (wave 1) and sin (wave 0) into LDS while the weights
        // land: lane l takes pairs l, l + 64, ...; the angles' chain of
        // products runs in every lane and each lane keeps the terms of its
        // pairs, so no lane loops on its own
        const int np = min(pro.epi.ne0, (int64_t)pro.epi.rp.n_dims) / 2;
        if (e_rope && wave < 2) {
            const int l = lane;
            const float e_pos = (float)e_rpos;
            float cap[4] = {e_pos, e_pos, e_pos, e_pos};
            float tp = e_pos;
            if (np <= 64) {  // straight-line: 63 products, each kept by its lane
                const float ts = pro.epi.rp.theta_scale;
#pragma unroll
                for (int k = 1; k < 64; ++k) {
                    tp *= ts;
                    cap[0] = k == l ? tp : cap[0];
                }
            } else {
                for (int k = 1; k < np; ++k) {
                    tp *= pro.epi.rp.theta_scale;
#pragma unroll
                    for (int i = 0; i < 4; ++i) cap[i] = k == l + 64 * i ? tp : cap[i];
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = l + 64 * i;
                if (p < np) {
                    float mscale;
                    const float ff = pro.epi.ff ? __builtin_bit_cast(float, e_rff[i]) : 1.0f;
                    const float theta = rope_theta(cap[i], p, ff, pro.epi.rp, mscale);
                    if (wave == 0) s_sn[p] = sinf(theta) * mscale;
                    else s_cs[p] = cosf(theta) * mscale;
                }
            }
        }
        lds_barrier();
    }

    char *dbase = a.nseg > 0 ? nullptr : (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
    auto store = [&](int64_t m, int n, float v) {
        if (a.nseg > 0) {
            const int sg = seg_of(m);
            sel(sg, a.seg_dst[0], a.seg_dst[1], a.seg_dst[2])[m - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2])] = v;
        } else {
            *(float *)(dbase + (a.n0 + n) * a.d_nb1 + m * 4) = v;
        }
    };
    // OUT_EPI: row m (segment sg, row j of it) with value v and its pair's
    // value o. The launcher keeps segment starts multiples of R, so a wave's
    // rows share a segment and the selects below are on wave-uniform values.
    auto epi_store = [&](int64_t m, float v, float o) {
        const GemvEpi &e = pro.epi;
        const int sg = seg_of(m);
        const int64_t j = m - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2]);
        const int lay = sel(sg, e.layout[0], e.layout[1], e.layout[2]);
        if (lay == EPI_F32) {
            sel(sg, a.seg_dst[0], a.seg_dst[1], a.seg_dst[2])[j] = v;
            return;
        }
        float y = v;
        const uint32_t ju = (uint32_t)j;  // rows, heads and slots are below 2^31 (the launcher's check)
        if (sel(sg, e.rope[0], e.rope[1], e.rope[2])) {
            const uint32_t el = ju % (uint32_t)e.ne0, p = el / 2;
            if (2 * p < e.rp.n_dims) {
                const float cs = s_cs[p], sn = s_sn[p];
                y = (el & 1) == 0 ? rope_first(v, o, cs, sn) : rope_second(o, v, cs, sn);
            }
        }
        char *base = sel(sg, e.dst[0], e.dst[1], e.dst[2]);
        const bool h16 = sel(sg, e.f16[0], e.f16[1], e.f16[2]) != 0;
        int64_t at;  // element offset
        if (lay == EPI_CONTIG) {
            at = j;
        } else {
            const int32_t lo = sel(sg, e_lo[0], e_lo[1], e_lo[2]), hi = sel(sg, e_hi[0], e_hi[1], e_hi[2]);
            const int64_t r = sel(sg, e.idx_i64[0], e.idx_i64[1], e.idx_i64[2])
                                  ? (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo)
                                  : (int64_t)(lo & hi);
            if (r < 0 || r >= sel(sg, e.rows[0], e.rows[1], e.rows[2])) return;
            if (lay == EPI_CACHE_ROW) {
                base += r * sel(sg, e.row_nb[0], e.row_nb[1], e.row_nb[2]);
                at = j;
            } else {  // the paged pools' layouts: keys [blocks, kvh, hs/8, bs, 8], values [blocks, kvh, hs, bs]
                const uint32_t ru = (uint32_t)r, bs = (uint32_t)e.bs, hs = (uint32_t)e.hs;
                const int64_t blk = ru / bs, off = ru % bs, h = ju / hs, el = ju % hs;
                at = lay == EPI_PAGED_KEY ? (((blk * e.kvh + h) * (e.hs / 8) + el / 8) * e.bs + off) * 8 + el % 8
                                          : ((blk * e.kvh + h) * e.hs + el) * e.bs + off;
            }
        }
        if (h16) ((uint16_t *)base)[at] = f2h(y);
        else ((float *)base)[at] = y;
    };
    // products of row block rbk, their wave sums, the K slices merged, stored
    auto finish = [&](const WRegs<WT, R> &w, int64_t rbk) {
        float acc[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int n = 0; n < NC; ++n) acc[r][n] = 0.0f;
        if (uvalid) w.template compute<NC>(act, u, acc);

        const int64_t m0 = rbk * rows_per_block + (int64_t)grp * RO;
        // every lane ends with all V totals (value i = row i / NC, column i % NC)
        float tot[V];
#pragma unroll
        for (int i = 0; i < V; ++i) tot[i] = wave_total(acc[i / NC][i % NC]);
        bool emit = ksplit == 1;
        if (ksplit > 1) {  // the K slices of a row group meet in LDS; the first wave adds them in order
            if (lane < V) {
                float mine = tot[0];
#pragma unroll
                for (int i = 1; i < V; ++i) mine = lane == i ? tot[i] : mine;
                part[wave][lane] = mine;
            }
            lds_barrier();
            emit = kw == 0;
            if (emit) {
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    float t = 0.0f;
                    for (int s2 = 0; s2 < ksplit; ++s2) t += part[grp * ksplit + s2][i];
                    tot[i] = t;
                }
            }
            lds_barrier();
        }
        // lane i < V (or < V / 2 with the epilogue) stores value i
        float mine = tot[0], up = GLU ? tot[V / 2] : 0.0f;
#pragma unroll
        for (int i = 1; i < V; ++i) mine = lane == i ? tot[i] : mine;
        if constexpr (GLU) {
#pragma unroll
            for (int i = 1; i < V / 2; ++i) up = lane == i ? tot[V / 2 + i] : up;
            if (emit && lane < V / 2) {
                const int r = lane / NC, n = lane % NC;
                if (m0 + r < a.M && n < a.N)
                    *(float *)((char *)pro.glu + (a.n0 + n) * pro.glu_nb1 + (m0 + r) * 4) = swiglu_val(mine, up);
            }
        } else if constexpr (OUT == OUT_EPI) {
            // lane i stores row m0 + i; its rotation partner is row m0 + (i ^ 1)
            float other = tot[0];
#pragma unroll
            for (int i = 1; i < V; ++i) other = (lane ^ 1) == i ? tot[i] : other;
            if (emit && lane < V && m0 + lane < a.M) epi_store(m0 + lane, mine, other);
        } else {
            if (emit && lane < V) {
                const int r = lane / NC, n = lane % NC;
                if (m0 + r < a.M && n < a.N) store(m0 + r, n, mine);
            }
        }
    };
    if constexpr (PIPE) {
        // two weight buffers in turn, one block's loads in flight while the
        // other is multiplied. No register copies and no loads behind a branch
        // in the steady state: the compiler then waits only for the older
        // buffer's loads.
        const int64_t g = gridDim.x, b0 = blockIdx.x;
        const int64_t mine = (uint32_t)(nblocks - b0 + g - 1) / (uint32_t)g;  // blocks of this workgroup, >= 2
        auto blk = [&](int64_t i) { return b0 + i * g; };
        int64_t i = 0;
        for (; i + 3 < mine; i += 2) {
            const uint8_t *wrow[R];
            finish(cur, blk(i));
            row_ptrs(blk(i + 2), wrow);
            cur.load(wrow, ul);
            finish(nxt, blk(i + 1));
            row_ptrs(blk(i + 3), wrow);
            nxt.load(wrow, ul);
        }
        if (mine - i == 3) {
            const uint8_t *wrow[R];
            finish(cur, blk(i));
            row_ptrs(blk(i + 2), wrow);
            cur.load(wrow, ul);
            finish(nxt, blk(i + 1));
            finish(cur, blk(i + 2));
        } else {
            finish(cur, blk(i));
            finish(nxt, blk(i + 1));
        }
    } else {
        for (;;) {
            finish(cur, rb);
            rb += gridDim.x;
            if (rb >= nblocks) break;
            const uint8_t *wrow[R];
            row_ptrs(rb, wrow);
            cur.load(wrow, ul);
        }
    }
}

// Workgroups of `kern` that the current device holds at once (the per-CU
// count cached per kernel, the CU count per device).
template <typename Kern> static int64_t resident_blocks(Kern kern, std::atomic<int> &cache) {
    return (int64_t)device_cus() * blocks_per_cu(kern, 256, 0, cache);
}

template <int WT, int NC, int R, int IN, bool PIPE, int OUT>
static tlh_status launch_reg_pipe(const MatmulArgs &a, const float *x, int64_t x_row_bytes, const GemvPro &pro,
                                  int ksplit, int upw, unsigned gx, hipStream_t stream) {
    auto kern = k_gemv_reg<WT, NC, R, IN, PIPE, OUT>;
    const int64_t batches = a.ne12 * a.ne13;
    const size_t lds = IN == IN_SCRATCH ? 0 : (size_t)(NC * act_lds(vec_dot_type(WT), a.K).bytes);
    hipLaunchKernelGGL(kern, dim3(gx, 1, (unsigned)batches), dim3(256), lds, stream, a, x, x_row_bytes, ksplit, upw,
                       pro);
    return check_launch("gemv");
}

// A persistent grid walks the row blocks. A workgroup that quantizes its
// activation itself reads 4 K bytes of it per column (and quantizes them)
// however few rows it then streams, so the grid is capped to give each
// workgroup at least twice that in weight bytes. Once each workgroup has
// several row blocks to walk, the double-buffered kernel keeps the weight
// stream busy.
template <int WT, int NC, int R, int IN, int OUT>
static tlh_status launch_reg_cfg(const MatmulArgs &a, const float *x, int64_t x_row_bytes, const GemvPro &pro,
                                 int ksplit, int upw, hipStream_t stream) {
    constexpr bool GLU = OUT == OUT_GLU;
    static std::atomic<int> slots{0};
    const int groups = 4 / ksplit;
    const int64_t rows_per_block = (int64_t)groups * (GLU ? R / 2 : R);
    const int64_t row_blocks = (a.M + rows_per_block - 1) / rows_per_block;
    const int64_t batches = a.ne12 * a.ne13 > 0 ? a.ne12 * a.ne13 : 1;
    int64_t gx = resident_blocks(k_gemv_reg<WT, NC, R, IN, false, OUT>, slots) / batches;
    if (IN != IN_SCRATCH) {
        const int64_t wbytes = rows_per_block * (GLU ? 2 : 1) * (a.K / block_elems(WT)) * block_bytes(WT);
        const int64_t per_wg = (2 * 4 * a.K * NC + wbytes - 1) / wbytes;  // row blocks per workgroup, at least
        gx = std::min(gx, (row_blocks + per_wg - 1) / per_wg);
    }
    gx = std::max<int64_t>(1, std::min(gx, row_blocks));
    if (row_blocks >= 2 * gx)
        return launch_reg_pipe<WT, NC, R, IN, true, OUT>(a, x, x_row_bytes, pro, ksplit, upw, (unsigned)gx, stream);
    return launch_reg_pipe<WT, NC, R, IN, false, OUT>(a, x, x_row_bytes, pro, ksplit, upw, (unsigned)gx, stream);
}

template <int WT, int NC, int IN, int OUT>
static tlh_status launch_reg_nc(const MatmulArgs &a, const float *x, int64_t x_row_bytes, const GemvPro &pro,
                                int ksplit, int upw, hipStream_t stream) {
    // q6_K / q5_K / q3_K hold about 20 weight registers per row: two columns take 2 rows per wave
    constexpr int R = ((WT == TLH_TYPE_Q6_K || WT == TLH_TYPE_Q5_K || WT == TLH_TYPE_Q3_K) && NC == 2) ? 2
                      : NC <= 2                                                                       ? 4
                      : (NC <= 4 ? 2 : 1);
    return launch_reg_cfg<WT, NC, R, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
}

// N = 1 or 2 only: more columns of register-resident activations (20 VGPRs
// per column) leave too few registers and spill.
template <int WT, int IN, int OUT>
static tlh_status launch_reg_wt(const MatmulArgs &a, const float *x, int64_t x_row_bytes, const GemvPro &pro,
                                int ksplit, int upw, hipStream_t stream) {
    if (OUT == OUT_EPI || a.N == 1) return launch_reg_nc<WT, 1, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
    if constexpr (OUT != OUT_EPI) return launch_reg_nc<WT, 2, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
}


}  // namespace tlh

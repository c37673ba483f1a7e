// Decode GEMV for GGML_OP_MUL_MAT with N <= 8 activation columns, gfx950.
//
// Replaces mm_vec (crates/kernels/src/cuda/native/mm.cu:16-42), which
// dequantized every weight to f32. Here the activations are already quantized
// to the weight type's vec_dot type (Q8_0 / Q8_K, bit-exact with the CPU
// backend), and each 32-weight unit is reduced as the CPU's vec_dot does:
// exact int32 block sums on v_dot4 (int8x4), scaled in f32
// (ggml-cpu/quants.c:225-258, :451-476, :696-773).
//
// Mapping: one wave64 owns R weight rows; lane l walks the row's 32-weight
// units u = l, l+64, ... (K/32 units), so each wave-wide load of a row is 1 KB
// of contiguous weight bytes (q4_K: 8 lanes per 144-byte super-block read its
// 128 code bytes with 16-byte loads plus the 16-byte header). The R rows
// share every activation load, which comes from L1/L2 (the activations of a
// launch are at most 8 * K bytes of codes). Partials are reduced across the
// wave with butterflies at the end.
#include "kernels.hpp"

namespace tlh {

// The 6-bit scale/min pair of q4_K sub-block s (0..7) without divergent
// branches (lanes of a wave hold different sub-blocks).
__device__ __forceinline__ void q4k_sm(int s, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
    const int sh = 8 * (s & 3);
    const uint32_t b0 = (s0 >> sh) & 0xff, b1 = (s1 >> sh) & 0xff, b2 = (s2 >> sh) & 0xff;
    const int lo_sc = b0 & 63, lo_mn = b1 & 63;
    const int hi_sc = (b2 & 0x0f) | ((b0 >> 6) << 4);
    const int hi_mn = (b2 >> 4) | ((b1 >> 6) << 4);
    sc = s < 4 ? lo_sc : hi_sc;
    mn = s < 4 ? lo_mn : hi_mn;
}

__device__ __forceinline__ uint4 ld16(const void *p) { return *(const uint4 *)p; }
// 16 bytes from a 2-byte aligned address (q4_0 / q8_0 blocks are 18 / 34
// bytes): one unaligned global_load_dwordx4 on gfx950.
__device__ __forceinline__ uint4 ld16u(const void *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

template <int WT, int NC, int R>
__global__ void __launch_bounds__(256) k_gemv(const MatmulArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t m0 = ((int64_t)blockIdx.x * 4 + wave) * R;
    if (m0 >= a.M) return;
    const int64_t batch = blockIdx.z;
    const int64_t i12 = batch % a.ne12, i13 = batch / a.ne12;
    const uint8_t *W = a.w + (i12 / a.r2) * a.w_nb2 + (i13 / a.r3) * a.w_nb3;
    constexpr int AT = vec_dot_type(WT);
    const int64_t K = a.K;
    const ActView act = act_view(a.act, AT, K, a.N_total * a.ne12 * a.ne13);
    const int64_t arow0 = a.n0 + a.N_total * batch;

    const uint8_t *wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;  // clamp: loads stay in bounds, store is skipped
        wrow[r] = W + m * a.w_nb1;
    }
    int64_t arow[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) arow[n] = arow0 + (n < a.N ? n : a.N - 1);

    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < NC; ++n) acc[r][n] = 0.0f;

    const int64_t units = K / 32;
    for (int64_t u = lane; u < units; u += 64) {
        if constexpr (WT == TLH_TYPE_Q4_K) {
            const int64_t sb = u >> 3;
            const int q = (int)(u & 7), j = q >> 1, h = q & 1;
            uint4 wq[R], hd[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t *blk = wrow[r] + sb * Q4_K_BYTES;
                hd[r] = ld16u(blk);
                wq[r] = ld16u(blk + 16 + 16 * q);
            }
            uint4 alo[NC], ahi[NC];
            float yd[NC];
            int bslo[NC], bshi[NC];
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int8_t *aq = act.qs + arow[n] * K + sb * QKK + 64 * j + 16 * h;
                alo[n] = ld16(aq);
                ahi[n] = ld16(aq + 32);
                yd[n] = act.d[arow[n] * (K / QKK) + sb];
                const int16_t *bs = act.bsums + arow[n] * (K / 16) + sb * 16 + 4 * j + h;
                bslo[n] = bs[0];
                bshi[n] = bs[2];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float d = h2f((uint16_t)(hd[r].x & 0xffff));
                const float dmin = h2f((uint16_t)(hd[r].x >> 16));
                int sclo, mnlo, schi, mnhi;
                q4k_sm(2 * j, hd[r].y, hd[r].z, hd[r].w, sclo, mnlo);
                q4k_sm(2 * j + 1, hd[r].y, hd[r].z, hd[r].w, schi, mnhi);
                const uint32_t w0 = wq[r].x, w1 = wq[r].y, w2 = wq[r].z, w3 = wq[r].w;
                const int l0 = w0 & 0x0f0f0f0f, l1 = w1 & 0x0f0f0f0f, l2 = w2 & 0x0f0f0f0f, l3 = w3 & 0x0f0f0f0f;
                const int h0 = (w0 >> 4) & 0x0f0f0f0f, h1 = (w1 >> 4) & 0x0f0f0f0f, h2 = (w2 >> 4) & 0x0f0f0f0f,
                          h3 = (w3 >> 4) & 0x0f0f0f0f;
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    int dl = dot4(l0, (int)alo[n].x, 0);
                    dl = dot4(l1, (int)alo[n].y, dl);
                    dl = dot4(l2, (int)alo[n].z, dl);
                    dl = dot4(l3, (int)alo[n].w, dl);
                    int dh = dot4(h0, (int)ahi[n].x, 0);
                    dh = dot4(h1, (int)ahi[n].y, dh);
                    dh = dot4(h2, (int)ahi[n].z, dh);
                    dh = dot4(h3, (int)ahi[n].w, dh);
                    const int S = sclo * dl + schi * dh;
                    const int Mn = mnlo * bslo[n] + mnhi * bshi[n];
                    acc[r][n] += (d * yd[n]) * (float)S - (dmin * yd[n]) * (float)Mn;
                }
            }
        } else if constexpr (WT == TLH_TYPE_Q4_0) {
            uint4 wq[R];
            float dw[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t *blk = wrow[r] + u * Q4_0_BYTES;
                dw[r] = h2f(*(const uint16_t *)blk);
                wq[r] = ld16u(blk + 2);
            }
            uint4 alo[NC], ahi[NC];
            float da[NC];
            int sa[NC];
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int8_t *aq = act.qs + arow[n] * K + u * 32;
                alo[n] = ld16(aq);
                ahi[n] = ld16(aq + 16);
                da[n] = act.d[arow[n] * (K / 32) + u];
                sa[n] = act.sum32[arow[n] * (K / 32) + u];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t w0 = wq[r].x, w1 = wq[r].y, w2 = wq[r].z, w3 = wq[r].w;
                const int l0 = w0 & 0x0f0f0f0f, l1 = w1 & 0x0f0f0f0f, l2 = w2 & 0x0f0f0f0f, l3 = w3 & 0x0f0f0f0f;
                const int h0 = (w0 >> 4) & 0x0f0f0f0f, h1 = (w1 >> 4) & 0x0f0f0f0f, h2 = (w2 >> 4) & 0x0f0f0f0f,
                          h3 = (w3 >> 4) & 0x0f0f0f0f;
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    int s = dot4(l0, (int)alo[n].x, 0);
                    s = dot4(l1, (int)alo[n].y, s);
                    s = dot4(l2, (int)alo[n].z, s);
                    s = dot4(l3, (int)alo[n].w, s);
                    s = dot4(h0, (int)ahi[n].x, s);
                    s = dot4(h1, (int)ahi[n].y, s);
                    s = dot4(h2, (int)ahi[n].z, s);
                    s = dot4(h3, (int)ahi[n].w, s);
                    s -= 8 * sa[n];  // codes are nibble - 8
                    acc[r][n] += ((float)s * dw[r]) * da[n];
                }
            }
        } else {  // Q8_0
            uint4 wa[R], wb[R];
            float dw[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint8_t *blk = wrow[r] + u * Q8_0_BYTES;
                dw[r] = h2f(*(const uint16_t *)blk);
                wa[r] = ld16u(blk + 2);
                wb[r] = ld16u(blk + 18);
            }
            uint4 xa[NC], xb[NC];
            float da[NC];
#pragma unroll
            for (int n = 0; n < NC; ++n) {
                const int8_t *aq = act.qs + arow[n] * K + u * 32;
                xa[n] = ld16(aq);
                xb[n] = ld16(aq + 16);
                da[n] = act.d[arow[n] * (K / 32) + u];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    int s = dot4((int)wa[r].x, (int)xa[n].x, 0);
                    s = dot4((int)wa[r].y, (int)xa[n].y, s);
                    s = dot4((int)wa[r].z, (int)xa[n].z, s);
                    s = dot4((int)wa[r].w, (int)xa[n].w, s);
                    s = dot4((int)wb[r].x, (int)xb[n].x, s);
                    s = dot4((int)wb[r].y, (int)xb[n].y, s);
                    s = dot4((int)wb[r].z, (int)xb[n].z, s);
                    s = dot4((int)wb[r].w, (int)xb[n].w, s);
                    acc[r][n] += (float)s * (dw[r] * da[n]);
                }
            }
        }
    }

    char *dbase = (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const float v = wave_sum(acc[r][n]);
            if (lane == 0 && m0 + r < a.M && n < a.N)
                *(float *)(dbase + (a.n0 + n) * a.d_nb1 + (m0 + r) * 4) = v;
        }
}

template <int WT, int NC>
static void launch_wt_nc(const MatmulArgs &a, hipStream_t stream) {
    constexpr int R = 2;
    const unsigned gx = (unsigned)((a.M + 4 * R - 1) / (4 * R));
    hipLaunchKernelGGL((k_gemv<WT, NC, R>), dim3(gx, 1, (unsigned)(a.ne12 * a.ne13)), dim3(256), 0, stream, a);
}

template <int WT>
static void launch_wt(const MatmulArgs &a, hipStream_t stream) {
    switch (a.N) {
    case 1: launch_wt_nc<WT, 1>(a, stream); break;
    case 2: launch_wt_nc<WT, 2>(a, stream); break;
    case 3: launch_wt_nc<WT, 3>(a, stream); break;
    case 4: launch_wt_nc<WT, 4>(a, stream); break;
    case 5: launch_wt_nc<WT, 5>(a, stream); break;
    case 6: launch_wt_nc<WT, 6>(a, stream); break;
    case 7: launch_wt_nc<WT, 7>(a, stream); break;
    default: launch_wt_nc<WT, 8>(a, stream); break;
    }
}

tlh_status launch_gemv(const MatmulArgs &a, hipStream_t stream) {
    if (a.N < 1 || a.N > 8) return set_error(TLH_INVALID, "gemv: N=%lld outside 1..8", (long long)a.N);
    switch (a.wtype) {
    case TLH_TYPE_Q4_0: launch_wt<TLH_TYPE_Q4_0>(a, stream); break;
    case TLH_TYPE_Q8_0: launch_wt<TLH_TYPE_Q8_0>(a, stream); break;
    case TLH_TYPE_Q4_K: launch_wt<TLH_TYPE_Q4_K>(a, stream); break;
    default: return set_error(TLH_UNSUPPORTED, "gemv: weight type %d", a.wtype);
    }
    return check_launch("gemv");
}

}  // namespace tlh

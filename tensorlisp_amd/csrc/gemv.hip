// Decode GEMV for GGML_OP_MUL_MAT with N <= 8 activation columns, gfx950:
// the LDS-staged variant, used for K the register-resident kernel
// (gemv_reg.hip) does not cover (K > 16384 or K not a multiple of 64), and
// the GEMV dispatch.
//
// Replaces mm_vec (crates/kernels/src/cuda/native/mm.cu:16-42), which
// dequantized every weight to f32. Here the activations are quantized to the
// weight type's vec_dot type (Q8_0 / Q8_K, bit-exact with the CPU backend)
// and every block is reduced as the CPU's vec_dot does: exact int32 block
// sums on v_dot4 (int8x4), scaled in f32 (ggml-cpu/quants.c:225-258,
// :451-476, :696-773).
//
// Structure (HBM-bound: the weight stream is the only large operand):
//  * each workgroup first puts the N activation rows into LDS, either by
//    quantizing the f32 input itself (FUSED: small N*K, saves a launch) or by
//    copying codes a separate quantize kernel wrote (large N*K);
//  * every wave then owns R weight rows at a time; lane l walks the row's
//    work units (q4_K: 64-element chunks, 32 code bytes + the 16-byte
//    super-block header; q4_0 / q8_0: one 32-element block) u = l, l+64, ...,
//    so a wave-wide load of a row is one contiguous run of weight bytes, and
//    the R rows share each activation read from LDS;
//  * the R x N partial sums are reduced across the wave by a transposing
//    butterfly (half the values change hands per step);
//  * the grid is persistent (at most one resident wave of workgroups) so the
//    activation staging is paid once per workgroup, not once per row group.
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

// 16 bytes from a 2-byte aligned address (q4_0 / q8_0 blocks are 18 / 34
// bytes): one unaligned global_load_dwordx4 on gfx950.
__device__ __forceinline__ uint4 ld16u(const void *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// LDS image of N activation rows: codes int8 [N][K], block scales f32
// [N][K/blk], code sums int32 per 32 elements [N][K/32].
struct LdsAct {
    int8_t *qs;
    float *d;
    int32_t *s32;
};

__host__ __device__ inline int64_t lds_act_bytes(int act_type, int64_t K, int64_t N) {
    const int64_t blk = act_type == TLH_TYPE_Q8_K ? QKK : QK;
    return align_up(N * K, 16) + align_up(N * (K / blk) * 4, 16) + N * (K / 32) * 4;
}

__device__ inline LdsAct lds_act(char *base, int act_type, int64_t K, int64_t N) {
    const int64_t blk = act_type == TLH_TYPE_Q8_K ? QKK : QK;
    LdsAct a;
    a.qs = (int8_t *)base;
    a.d = (float *)(base + align_up(N * K, 16));
    a.s32 = (int32_t *)(base + align_up(N * K, 16) + align_up(N * (K / blk) * 4, 16));
    return a;
}

// Quantize N rows of f32 into the LDS image (the rules of k_quantize_q8_0 /
// k_quantize_q8_K: quantize_row_q8_0_ref ggml-quants.c:276-297 and
// quantize_row_q8_K_ref :2768-2804), all threads of the workgroup.
template <int AT, int NTHREADS>
__device__ void stage_quantize(const float *x, int64_t x_row_bytes, int64_t K, int N, LdsAct s) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int WAVES = NTHREADS / 64;
    if constexpr (AT == TLH_TYPE_Q8_0) {
        // one lane per element, 32 lanes per block
        const int64_t total = (int64_t)N * K;
        for (int64_t e = threadIdx.x; e < total; e += NTHREADS) {
            const int64_t n = e / K, k = e - n * K;
            const float v = *(const float *)((const char *)x + n * x_row_bytes + k * 4);
            float amax = fabsf(v);
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int q = (int)roundf(v * id);
            s.qs[e] = (int8_t)q;
            int sum = q;
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 32);
            if ((threadIdx.x & 31) == 0) {
                s.d[e / QK] = h2f(f2h(d));
                s.s32[e / QK] = sum;
            }
        }
    } else {
        // one wave per 256-element block, four consecutive elements per lane
        const int64_t nblk = K / QKK;
        for (int64_t b = wave; b < (int64_t)N * nblk; b += WAVES) {
            const int64_t n = b / nblk, kb = b - n * nblk;
            const float *src = (const float *)((const char *)x + n * x_row_bytes) + kb * QKK + 4 * lane;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = src[i];
            float ba = 0.0f, bv = 0.0f;
            int bi = 1 << 30;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = fabsf(v[i]);
                if (a > ba) { ba = a; bv = v[i]; bi = 4 * lane + i; }
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                const float oa = __shfl_xor(ba, m, 64);
                const float ov = __shfl_xor(bv, m, 64);
                const int oi = __shfl_xor(bi, m, 64);
                if (oa > ba || (oa == ba && oi < bi)) { ba = oa; bv = ov; bi = oi; }
            }
            uint32_t packed = 0;
            int psum = 0;
            float d = 0.0f;
            if (ba != 0.0f) {
                const float iscale = -127.0f / bv;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    int q = (int)rintf(iscale * v[i]);
                    q = q > 127 ? 127 : q;
                    packed |= (uint32_t)(uint8_t)(int8_t)q << (8 * i);
                    psum += q;
                }
                d = 1.0f / iscale;
            }
            // sums per 32 elements = 8 lanes
            psum += __shfl_xor(psum, 1, 64);
            psum += __shfl_xor(psum, 2, 64);
            psum += __shfl_xor(psum, 4, 64);
            *(uint32_t *)(s.qs + n * K + kb * QKK + 4 * lane) = packed;
            if ((lane & 7) == 0) s.s32[n * (K / 32) + kb * 8 + (lane >> 3)] = psum;
            if (lane == 0) s.d[n * nblk + kb] = d;
        }
    }
}

// Copy N pre-quantized rows (split scratch layout) into the LDS image.
template <int AT, int NTHREADS>
__device__ void stage_copy(const ActView g, int64_t arow0, int64_t K, int N, LdsAct s) {
    const int64_t nq16 = (int64_t)N * K / 16;
    for (int64_t i = threadIdx.x; i < nq16; i += NTHREADS) {
        const int64_t n = i / (K / 16), j = i - n * (K / 16);
        *(uint4 *)(s.qs + n * K + 16 * j) = *(const uint4 *)(g.qs + (arow0 + n) * K + 16 * j);
    }
    constexpr int64_t blk = AT == TLH_TYPE_Q8_K ? QKK : QK;
    for (int64_t i = threadIdx.x; i < (int64_t)N * (K / blk); i += NTHREADS) {
        const int64_t n = i / (K / blk), j = i - n * (K / blk);
        s.d[i] = g.d[(arow0 + n) * (K / blk) + j];
    }
    for (int64_t i = threadIdx.x; i < (int64_t)N * (K / 32); i += NTHREADS) {
        const int64_t n = i / (K / 32), j = i - n * (K / 32);
        if constexpr (AT == TLH_TYPE_Q8_K)
            s.s32[i] = (int32_t)g.bsums[(arow0 + n) * (K / 16) + 2 * j] + (int32_t)g.bsums[(arow0 + n) * (K / 16) + 2 * j + 1];
        else
            s.s32[i] = g.sum32[(arow0 + n) * (K / 32) + j];
    }
}

// Sum V = 2^LV values across the 64 lanes of a wave. Each butterfly step
// hands half of the remaining values to the partner lane, so after LV steps
// lane l holds the partial of value index v(l) (bits of l from bit 5 down);
// the remaining 6 - LV steps reduce that single value. Returns the total of
// value v(lane), valid in every lane.
template <int LV>
__device__ __forceinline__ float transpose_reduce(float (&v)[1 << LV], int lane, int &vidx) {
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

template <int X> struct Log2 { static constexpr int v = 1 + Log2<X / 2>::v; };
template <> struct Log2<1> { static constexpr int v = 0; };

template <int WT, int NC, int R, int NTHREADS, bool FUSED>
__global__ void __launch_bounds__(NTHREADS) k_gemv(const MatmulArgs a, const float *__restrict__ x,
                                                   int64_t x_row_bytes) {
    extern __shared__ __attribute__((aligned(16))) char lds_raw[];
    constexpr int AT = vec_dot_type(WT);
    constexpr int WAVES = NTHREADS / 64;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t K = a.K;
    const int N = (int)a.N;
    const int64_t batch = blockIdx.z;
    const int64_t i12 = batch % a.ne12, i13 = batch / a.ne12;
    const uint8_t *W = a.w + (i12 / a.r2) * a.w_nb2 + (i13 / a.r3) * a.w_nb3;
    const int64_t arow0 = a.n0 + a.N_total * batch;

    const LdsAct s = lds_act(lds_raw, AT, K, NC);
    if constexpr (FUSED) {
        stage_quantize<AT, NTHREADS>((const float *)((const char *)x + arow0 * x_row_bytes), x_row_bytes, K, N, s);
    } else {
        const ActView g = act_view(a.act, AT, K, a.N_total * a.ne12 * a.ne13);
        stage_copy<AT, NTHREADS>(g, arow0, K, N, s);
    }
    __syncthreads();

    char *dbase = (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
    constexpr int V = R * NC;
    constexpr int VP = 1 << (Log2<V>::v + ((V & (V - 1)) ? 1 : 0));  // next power of two
    const int64_t stride_rows = (int64_t)gridDim.x * WAVES * R;
    for (int64_t m0 = ((int64_t)blockIdx.x * WAVES + wave) * R; m0 < a.M; m0 += stride_rows) {
        const uint8_t *wrow[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;  // clamp: loads stay in bounds, store is skipped
            wrow[r] = W + m * a.w_nb1;
        }
        float acc[R][NC];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int n = 0; n < NC; ++n) acc[r][n] = 0.0f;

        if constexpr (WT == TLH_TYPE_Q4_K) {
            const int64_t chunks = K / 64;
            for (int64_t c = lane; c < chunks; c += 64) {
                const int64_t sb = c >> 2;
                const int j = (int)(c & 3);
                uint4 hd[R], q0[R], q1[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint8_t *blk = wrow[r] + sb * Q4_K_BYTES;
                    hd[r] = ld16u(blk);
                    q0[r] = ld16u(blk + 16 + 32 * j);
                    q1[r] = ld16u(blk + 32 + 32 * j);
                }
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    const int8_t *aq = s.qs + n * K + 64 * c;
                    const int4 x0 = *(const int4 *)(aq), x1 = *(const int4 *)(aq + 16);
                    const int4 x2 = *(const int4 *)(aq + 32), x3 = *(const int4 *)(aq + 48);
                    const float yd = s.d[n * (K / QKK) + sb];
                    const int xs_lo = s.s32[n * (K / 32) + 2 * c], xs_hi = s.s32[n * (K / 32) + 2 * c + 1];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t w[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
                        const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                        const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
                        int dl = 0, dh = 0;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            dl = dot4((int)(w[i] & 0x0f0f0f0fu), xl[i], dl);
                            dh = dot4((int)((w[i] >> 4) & 0x0f0f0f0fu), xh[i], dh);
                        }
                        int sclo, mnlo, schi, mnhi;
                        q4k_sm(2 * j, hd[r].y, hd[r].z, hd[r].w, sclo, mnlo);
                        q4k_sm(2 * j + 1, hd[r].y, hd[r].z, hd[r].w, schi, mnhi);
                        const int S = sclo * dl + schi * dh;
                        const int Mn = mnlo * xs_lo + mnhi * xs_hi;
                        const float d = h2f((uint16_t)(hd[r].x & 0xffff));
                        const float dmin = h2f((uint16_t)(hd[r].x >> 16));
                        acc[r][n] += (d * yd) * (float)S - (dmin * yd) * (float)Mn;
                    }
                }
            }
        } else if constexpr (WT == TLH_TYPE_Q4_0) {
            const int64_t units = K / 32;
            for (int64_t u = lane; u < units; u += 64) {
                uint4 wq[R];
                float dw[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint8_t *blk = wrow[r] + u * Q4_0_BYTES;
                    dw[r] = h2f(*(const uint16_t *)blk);
                    wq[r] = ld16u(blk + 2);
                }
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    const int8_t *aq = s.qs + n * K + 32 * u;
                    const int4 xa = *(const int4 *)(aq), xb = *(const int4 *)(aq + 16);
                    const float da = s.d[n * (K / 32) + u];
                    const int sa = s.s32[n * (K / 32) + u];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t w[4] = {wq[r].x, wq[r].y, wq[r].z, wq[r].w};
                        const int xl[4] = {xa.x, xa.y, xa.z, xa.w};
                        const int xh[4] = {xb.x, xb.y, xb.z, xb.w};
                        int sum = 0;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            sum = dot4((int)(w[i] & 0x0f0f0f0fu), xl[i], sum);
                            sum = dot4((int)((w[i] >> 4) & 0x0f0f0f0fu), xh[i], sum);
                        }
                        sum -= 8 * sa;  // codes are nibble - 8
                        acc[r][n] += ((float)sum * dw[r]) * da;
                    }
                }
            }
        } else {  // Q8_0
            const int64_t units = K / 32;
            for (int64_t u = lane; u < units; u += 64) {
                uint4 wa[R], wb[R];
                float dw[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint8_t *blk = wrow[r] + u * Q8_0_BYTES;
                    dw[r] = h2f(*(const uint16_t *)blk);
                    wa[r] = ld16u(blk + 2);
                    wb[r] = ld16u(blk + 18);
                }
#pragma unroll
                for (int n = 0; n < NC; ++n) {
                    const int8_t *aq = s.qs + n * K + 32 * u;
                    const int4 xa = *(const int4 *)(aq), xb = *(const int4 *)(aq + 16);
                    const float da = s.d[n * (K / 32) + u];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        int sum = dot4((int)wa[r].x, xa.x, 0);
                        sum = dot4((int)wa[r].y, xa.y, sum);
                        sum = dot4((int)wa[r].z, xa.z, sum);
                        sum = dot4((int)wa[r].w, xa.w, sum);
                        sum = dot4((int)wb[r].x, xb.x, sum);
                        sum = dot4((int)wb[r].y, xb.y, sum);
                        sum = dot4((int)wb[r].z, xb.z, sum);
                        sum = dot4((int)wb[r].w, xb.w, sum);
                        acc[r][n] += (float)sum * (dw[r] * da);
                    }
                }
            }
        }

        float vals[VP];
#pragma unroll
        for (int i = 0; i < VP; ++i) vals[i] = i < V ? acc[i / NC][i % NC] : 0.0f;
        int vi;
        const float tot = transpose_reduce<Log2<VP>::v>(vals, lane, vi);
        // lanes whose bits below the value bits are zero hold distinct values
        if ((lane & ((64 / VP) - 1)) == 0 && vi < V) {
            const int r = vi / NC, n = vi % NC;
            if (m0 + r < a.M && n < N) *(float *)(dbase + (a.n0 + n) * a.d_nb1 + (m0 + r) * 4) = tot;
        }
    }
}

// ------------------------------------------------------------------ launch
template <int WT, int NC, int R, int NT, bool FUSED>
static tlh_status launch_cfg(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream) {
    constexpr int AT = vec_dot_type(WT);
    const size_t lds = (size_t)lds_act_bytes(AT, a.K, NC);
    auto kern = k_gemv<WT, NC, R, NT, FUSED>;
    static int max_blocks_per_cu = -1;
    static int cus = 0;
    static size_t cached_lds = 0;
    if (max_blocks_per_cu < 0 || cached_lds != lds) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (lds > 64 * 1024)
            (void)hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, NT, lds) != hipSuccess || nb < 1) nb = 1;
        max_blocks_per_cu = nb;
        cached_lds = lds;
    }
    const int64_t row_groups = (a.M + R - 1) / R;
    const int64_t wgs_needed = (row_groups + NT / 64 - 1) / (NT / 64);
    const int64_t batches = a.ne12 * a.ne13;
    int64_t resident = (int64_t)cus * max_blocks_per_cu / (batches > 0 ? batches : 1);
    if (resident < 1) resident = 1;
    const unsigned gx = (unsigned)(wgs_needed < resident ? wgs_needed : resident);
    hipLaunchKernelGGL(kern, dim3(gx, 1, (unsigned)batches), dim3(NT), lds, stream, a, x, x_row_bytes);
    return check_launch("gemv");
}

// Largest LDS image the GEMV stages (act codes + scales + sums): 8 columns of
// K = 16384 fit in gfx950's 160 KB.
static bool fits_lds(int wtype, int64_t K, int nc) {
    return lds_act_bytes(vec_dot_type(wtype), K, nc) <= 150 * 1024;
}

template <int WT, int NC>
static tlh_status launch_nc(const MatmulArgs &a, hipStream_t stream) {
    constexpr int R = NC <= 2 ? 4 : 2;
    return launch_cfg<WT, NC, R, 512, false>(a, nullptr, 0, stream);
}

template <int WT>
static tlh_status launch_wt(const MatmulArgs &a, hipStream_t stream) {
    switch (a.N) {
    case 1: return launch_nc<WT, 1>(a, stream);
    case 2: return launch_nc<WT, 2>(a, stream);
    case 3: return launch_nc<WT, 3>(a, stream);
    case 4: return launch_nc<WT, 4>(a, stream);
    case 5: return launch_nc<WT, 5>(a, stream);
    case 6: return launch_nc<WT, 6>(a, stream);
    case 7: return launch_nc<WT, 7>(a, stream);
    default: return launch_nc<WT, 8>(a, stream);
    }
}

bool gemv_fuses_quantize(const MatmulArgs &a, const float *x, int64_t x_row_bytes) {
    int ksplit, upw;
    return x != nullptr && a.N <= 2 && gemv_reg_geometry(a.K, ksplit, upw) && ((uintptr_t)x & 15) == 0 &&
           (x_row_bytes & 15) == 0;
}

bool gemv_uses_reg(const MatmulArgs &a) {
    int ksplit, upw;
    return a.N <= 2 && gemv_reg_geometry(a.K, ksplit, upw);
}

// N <= 2 with K the register kernel covers: the register-resident GEMV
// (fused quantization when x is given); otherwise the int8-MFMA kernel.
tlh_status launch_gemv(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream) {
    if (a.N < 1 || a.N > 16) return set_error(TLH_INVALID, "gemv: N=%lld outside 1..16", (long long)a.N);
    if (gemv_uses_reg(a)) return launch_gemv_reg(a, x, x_row_bytes, stream);
    if (x != nullptr) return set_error(TLH_INVALID, "gemv: fused quantization needs N <= 2, K <= 16384, K %% 64 == 0");
    return launch_gemv_mfma(a, stream);
}

}  // namespace tlh

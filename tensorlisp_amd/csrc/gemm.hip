// Prefill GEMM for GGML_OP_MUL_MAT with N > 8 activation columns, gfx950.
//
// Replaces mm_tile (crates/kernels/src/cuda/native/mm.cu:50-103). For q4_K
// weights it computes what the CPU backend computes per super-block
// (ggml_vec_dot_q4_K_q8_K_generic, ggml-cpu/quants.c:696-773):
//   y += (d * dy) * S - (dmin * dy) * Mn,
//   S  = sum over the 256 elements of (sc_s * q4) * q8   (integer),
//   Mn = sum over the 8 sub-blocks of m_s * (sum of q8 in s) (integer),
// on CDNA4 matrix cores:
//  * S runs on v_mfma_f32_32x32x16_f16 with integer-valued operands: the
//    weight operand is w' = sc_s * q4 (<= 945) and the activation operand is the
//    q8 code (|q| <= 127), both exact in f16; products (< 2^17) and the sums
//    of a super-block are exact in the f32 accumulator for any realistic data
//    (a partial above 2^24 would round by one unit in 2^24).
//  * Mn is one more K=16 MFMA per super-block: A'[m][k] = m_{k/2}(m) and
//    B'[k][n] = bsums[k](n) (|bsum| <= 2032, exact in f16).
//  * The f32 finalize folds S and Mn into the output accumulators per
//    super-block, as the CPU does (its f32 accumulation order differs).
// Tiling: 128 (weight rows) x 128 (tokens) per workgroup of 4 waves, each
// wave 64 x 64 as 2 x 2 MFMA tiles of 32 x 32; K advances in stages of one
// 64-element q4_K chunk. LDS holds two stage buffers: while the waves
// multiply stage s, stage s + 1 fills the other one. Its activation codes
// (exact f16 from the quantize pass) go straight from global memory to LDS
// (global_load_lds_dwordx4: no registers, no LDS writes); its weight codes
// come to registers and are converted once per workgroup (nibble -> (1024 +
// n) * sc - 1024 * sc with one packed FMA) and written after the products.
// One barrier per stage.
//
// q5_K runs the same kernel with the fifth code bit OR-ed in before the f16
// conversion (sc * q <= 63 * 31 stays exact). q8_0 / q4_0 have their own
// int8-MFMA GEMM (gemm_q8.hip). q6_K weights with N > 16 run through the
// int8-MFMA few-column kernel (gemv_mfma.hip) in slabs of 16 columns (correct
// for any N; each slab re-reads the weights).
#include "kernels.hpp"

namespace tlh {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 64;

// LDS: two stage buffers of f16 tiles (row = 64 halves = 8 chunks of 16 bytes,
// chunk c of row r stored at chunk position c ^ (r & 7) so the b128 operand
// reads of 8 consecutive rows hit distinct banks), and two buffers of the
// per-super-block metadata (by super-block parity).
struct __attribute__((aligned(16))) GemmSmem {
    _Float16 A[2][GBM][GBK];
    _Float16 B[2][GBN][GBK];
    uint8_t Amin[2][GBM][8];    // the 8 sub-block mins per weight row
    _Float16 Bsum[2][GBN][16];  // bsums per token
    float dA[2][GBM], dminA[2][GBM], dB[2][GBN];
};

__device__ __forceinline__ int swz(int row, int chunk) { return ((chunk ^ (row & 7)) << 3); }  // halves

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4 nibbles (one per byte of v) -> two half2 of sc * n, exact:
// (1024 + n) * sc - 1024 * sc in one packed FMA (the product is exact inside the FMA).
__device__ __forceinline__ void nib4_to_h(uint32_t v, half2_t sc2, half2_t nsc2, uint32_t &o01, uint32_t &o23) {
    const half2_t a = __builtin_bit_cast(half2_t, perm(0x64646464u, v, 0x04010400u));  // 1024 + n0, 1024 + n1
    const half2_t b = __builtin_bit_cast(half2_t, perm(0x64646464u, v, 0x04030402u));  // 1024 + n2, 1024 + n3
    o01 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(a, sc2, nsc2));
    o23 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, sc2, nsc2));
}

__device__ __forceinline__ void q4k_sm_g(int s, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
    const int sh = 8 * (s & 3);
    const uint32_t b0 = (s0 >> sh) & 0xff, b1 = (s1 >> sh) & 0xff, b2 = (s2 >> sh) & 0xff;
    sc = s < 4 ? (int)(b0 & 63) : (int)((b2 & 0x0f) | ((b0 >> 6) << 4));
    mn = s < 4 ? (int)(b1 & 63) : (int)((b2 >> 4) | ((b1 >> 6) << 4));
}

__device__ __forceinline__ uint4 ldg16(const void *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// What one thread fetches to registers for a stage: its weight row's 16 code
// bytes (half h of the chunk); at a super-block's first stage also its header.
struct StageRegs {
    uint4 wq, hdr, qh;  // hdr: at a super-block's first stage only; qh: q5_K's fifth bits
};
typedef __attribute__((address_space(3))) void lds_void;

template <int WT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) k_gemm_q4k(const MatmulArgs a) {
    constexpr bool Q5 = WT == TLH_TYPE_Q5_K;
    constexpr int SB = Q5 ? Q5_K_BYTES : Q4_K_BYTES;
    constexpr int QS = Q5 ? 48 : 16;  // offset of the nibble bytes
    __shared__ GemmSmem sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // wave tile position (2 x 2)
    const int64_t K = a.K;
    const int64_t nsb = K / QKK;
    const uint32_t batches = (uint32_t)(a.ne12 * a.ne13);
    // K chunk kc of gridDim.z / batches (one batch slice: no division)
    const uint32_t kc = batches == 1 ? blockIdx.z : blockIdx.z / batches, batch = blockIdx.z - kc * batches;
    const MmSlice sl = mm_slice(a, batch);
    const int64_t i12 = sl.i12, i13 = sl.i13;
    const uint8_t *W = sl.w;
    const ActView act = act_view(a.act, TLH_TYPE_Q8_K, K, a.N_total * a.ne12 * a.ne13);
    const int64_t m_base = (int64_t)blockIdx.y * GBM;
    const int64_t n_base = (int64_t)blockIdx.x * GBN;

    // staging roles: weight row / token tid >> 1, half h = tid & 1 of the 64-element chunk
    const int srow = tid >> 1, sh = tid & 1;
    // segments (a.nseg > 0, one batch slice): rows seg_m0[s] .. seg_m0[s+1] of
    // the launch are the rows of weight matrix seg_w[s] (row stride w_nb1),
    // written to seg_dst[s]; every segment but the last is a whole number of
    // tiles, so a tile lies in one (sg) and its rows start at m0 in it
    int sg = 0;
    int64_t m0 = 0;
    if (a.nseg > 0) {
        sg = (int)(m_base >= a.seg_m0[1]) + (int)(a.nseg > 2 && m_base >= a.seg_m0[2]);
        m0 = a.seg_m0[sg];
        W = a.seg_w[sg];
    }
    const int64_t grow = m_base + srow < a.M ? m_base + srow : a.M - 1;  // clamped: loads in bounds
    const uint8_t *wrow = W + (grow - m0) * a.w_nb1;
    // B tile rows (tokens) this lane fills by direct-to-LDS loads: instruction
    // i of wave w fills rows 8 (4 w + i) .. + 7, lane l row + l / 8 at chunk
    // position l % 8, i.e. the chunk (l % 8) ^ (row & 7) of the token's stage
    const _Float16 *brow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * (4 * wave + i) + (lane >> 3);
        const int64_t col = n_base + r < a.N ? n_base + r : a.N - 1;
        brow[i] = act.q16 + (a.n0 + col + a.N_total * batch) * K + 8 * ((lane & 7) ^ (r & 7));
    }
    // the tokens' metadata of a super-block, also straight to LDS: bsums (f16
    // from the quantize pass), wave w tokens 32 w .. + 31, lane l token
    // 32 w + l / 2, bsums 8 (l & 1) .. + 7; scales, waves 0 and 1, 64 tokens each
    const _Float16 *bsrow;
    const float *dxrow;
    {
        const int r = 32 * wave + (lane >> 1);
        const int64_t col = n_base + r < a.N ? n_base + r : a.N - 1;
        bsrow = act.b16 + (a.n0 + col + a.N_total * batch) * (K / 16) + 8 * (lane & 1);
        const int rd = 64 * (wave & 1) + lane;
        const int64_t cold = n_base + rd < a.N ? n_base + rd : a.N - 1;
        dxrow = act.d + (a.n0 + cold + a.N_total * batch) * nsb;
    }
    auto load_b = [&](int64_t stage) {
        const int buf = (int)(stage & 1);
        const int64_t sb = stage >> 2;
        const int64_t off = sb * QKK + 64 * (stage & 3);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(brow[i] + off), (lds_void *)&sm.B[buf][8 * (4 * wave + i)][0], 16,
                                             0, 0);
        if ((stage & 3) == 0) {
            const int mb = (int)(sb & 1);
            __builtin_amdgcn_global_load_lds((const void *)(bsrow + sb * 16), (lds_void *)&sm.Bsum[mb][32 * wave][0], 16, 0,
                                             0);
            if (wave < 2)
                __builtin_amdgcn_global_load_lds((const void *)(dxrow + sb), (lds_void *)&sm.dB[mb][64 * wave], 4, 0, 0);
        }
    };

    auto fetch = [&](int64_t stage, StageRegs &r) {
        const int64_t sb = stage >> 2;
        const int j = (int)(stage & 3);
        const uint8_t *blk = wrow + sb * SB;
        if (j == 0) r.hdr = ldg16(blk);
        r.wq = ldg16(blk + QS + 32 * j + 16 * sh);
        if constexpr (Q5) r.qh = ldg16(blk + 16 + 16 * sh);
    };
    uint32_t scw[2] = {0, 0};  // the current super-block's 8 sub-block scales (bytes), from its header

    auto commit = [&](int64_t stage, const StageRegs &r) {
        const int buf = (int)(stage & 1), mb = (int)((stage >> 2) & 1);
        const int j = (int)(stage & 3);
        if (j == 0) {
            uint32_t mv[2] = {0, 0};
            scw[0] = scw[1] = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                int sc, mn;
                q4k_sm_g(s, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
                scw[s >> 2] |= (uint32_t)sc << (8 * (s & 3));
                mv[s >> 2] |= (uint32_t)mn << (8 * (s & 3));
            }
            if (sh == 0) {
                sm.dA[mb][srow] = h2f((uint16_t)(r.hdr.x & 0xffff));
                sm.dminA[mb][srow] = h2f((uint16_t)(r.hdr.x >> 16));
                *(uint2 *)&sm.Amin[mb][srow][0] = make_uint2(mv[0], mv[1]);
            }
        }
        const int sclo = (int)((scw[j >> 1] >> (16 * (j & 1))) & 0xff);
        const int schi = (int)((scw[j >> 1] >> (16 * (j & 1) + 8)) & 0xff);
        const _Float16 fl = (_Float16)sclo, fh = (_Float16)schi;
        const half2_t sl2 = {fl, fl}, sh2 = {fh, fh};
        const half2_t nsl2 = {(_Float16)(-1024 * sclo), (_Float16)(-1024 * sclo)};
        const half2_t nsh2 = {(_Float16)(-1024 * schi), (_Float16)(-1024 * schi)};
        const uint32_t w[4] = {r.wq.x, r.wq.y, r.wq.z, r.wq.w};
        const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t cl = w[i] & 0x0f0f0f0fu, ch = (w[i] >> 4) & 0x0f0f0f0fu;
            if constexpr (Q5) {  // codes 0..31: (1024 + n) stays exact in f16
                cl |= ((qh[i] >> (2 * j)) & 0x01010101u) << 4;
                ch |= ((qh[i] >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            nib4_to_h(cl, sl2, nsl2, lo[2 * i], lo[2 * i + 1]);
            nib4_to_h(ch, sh2, nsh2, hi[2 * i], hi[2 * i + 1]);
        }
        // low nibbles: k = 16h + i (chunks 2h, 2h+1); high nibbles: k = 32 + 16h + i (chunks 4+2h, 5+2h)
        _Float16 *ar = sm.A[buf][srow];
        *(uint4 *)(ar + swz(srow, 2 * sh)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4 *)(ar + swz(srow, 2 * sh + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        *(uint4 *)(ar + swz(srow, 4 + 2 * sh)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4 *)(ar + swz(srow, 5 + 2 * sh)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    };

    float16_t S[2][2], acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) {
            S[i][jn] = (float16_t){};
            acc[i][jn] = (float16_t){};
        }

    const int lr = lane & 31, lg = lane >> 5;  // MFMA operand row/col and k-group
    // this workgroup's super-blocks: chunk kc of equal shares (stage indices are global)
    const int64_t nkc = gridDim.z / batches, share = (nsb + nkc - 1) / nkc;
    const int64_t sb0 = kc * share, sb1 = sb0 + share < nsb ? sb0 + share : nsb;
    const int64_t g0 = 4 * sb0, stages = 4 * sb1;
    StageRegs pre;
    if (g0 < stages) {
        load_b(g0);
        fetch(g0, pre);
        commit(g0, pre);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the direct-to-LDS loads landed
    lds_barrier();
    for (int64_t st = g0; st < stages; ++st) {
        const int buf = (int)(st & 1);
        // stage st + 1: B straight to the free LDS buffer, A to registers
        if (st + 1 < stages) {
            load_b(st + 1);
            fetch(st + 1, pre);
        }
#pragma unroll
        for (int t = 0; t < GBK / 16; ++t) {
            half8_t av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra = 64 * wm + 32 * i + lr, rb = 64 * wn + 32 * i + lr;
                av[i] = *(const half8_t *)&sm.A[buf][ra][swz(ra, 2 * t + lg)];
                bv[i] = *(const half8_t *)&sm.B[buf][rb][swz(rb, 2 * t + lg)];
            }
            if (t == 0 && (st & 3) == 0) {  // a super-block's first products start from zero
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int jn = 0; jn < 2; ++jn)
                        S[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[jn], (float16_t){}, 0, 0, 0);
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int jn = 0; jn < 2; ++jn)
                        S[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[jn], S[i][jn], 0, 0, 0);
            }
        }
        if ((st & 3) == 3) {
            // super-block finalize: acc += dy * (d * S - dmin * Mn)
            const int mb = (int)((st >> 2) & 1);
            // Mn operands: A'[m][k] = m_{k/2}, k = 8g..8g+7 -> mins 4g..4g+3, each twice
            half8_t am[2], bm[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t mw = *(const uint32_t *)&sm.Amin[mb][64 * wm + 32 * i + lr][4 * lg];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const _Float16 h = (_Float16)(float)((mw >> (8 * e)) & 0xff);
                    am[i][2 * e] = h;
                    am[i][2 * e + 1] = h;
                }
                bm[i] = *(const half8_t *)&sm.Bsum[mb][64 * wn + 32 * i + lr][8 * lg];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int jn = 0; jn < 2; ++jn) {
                    const float16_t Mn =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(am[i], bm[jn], (float16_t){}, 0, 0, 0);
                    const float dy = sm.dB[mb][64 * wn + 32 * jn + lr];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int m0 = 64 * wm + 32 * i + 8 * q + 4 * lg;
                        const float4 d4 = *(const float4 *)&sm.dA[mb][m0];
                        const float4 dm4 = *(const float4 *)&sm.dminA[mb][m0];
                        const float dv[4] = {d4.x, d4.y, d4.z, d4.w}, dmv[4] = {dm4.x, dm4.y, dm4.z, dm4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * q + e;
                            acc[i][jn][r] += dy * (dv[e] * S[i][jn][r] - dmv[e] * Mn[r]);
                        }
                    }
                }
            }
        }
        // stage st + 1's A to the other buffer (free since the last barrier)
        if (st + 1 < stages) commit(st + 1, pre);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): stage st + 1's B landed
        lds_barrier();
    }

    // store: lane holds token n = lane % 32 of each 32 x 32 tile and rows 8q + 4g + (0..3);
    // with K chunks, to this chunk's partials [chunk][batch][N][M]
    char *dbase = (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
    float *pbase = nkc > 1 ? a.part + (kc * batches + batch) * a.N * a.M : nullptr;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) {
            const int64_t n = n_base + 64 * wn + 32 * jn + lr;
            if (n >= a.N) continue;
            // partials hold every row of the launch; a segment's own output
            // holds its rows from m0
            const int64_t moff = pbase ? 0 : m0;
            float *drow = pbase      ? pbase + n * a.M
                          : a.nseg ? (float *)((char *)a.seg_dst[sg] + (a.n0 + n) * a.seg_d_nb1[sg])
                                   : (float *)(dbase + (a.n0 + n) * a.d_nb1);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t m = m_base + 64 * wm + 32 * i + 8 * q + 4 * lg;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (m + e < a.M) drow[m + e - moff] = acc[i][jn][4 * q + e];
            }
        }
}

int gemm_ksplit(int wtype, int64_t M, int64_t N, int64_t K, int64_t batches) {
    if (!has_gemm(wtype) || N <= 16) return 1;
    constexpr int64_t CUS = 256;  // MI355X
    const int64_t tiles = (N + 127) / 128 * ((M + 127) / 128) * batches;
    if (tiles >= CUS) return 1;  // two workgroups fit a CU: up to 512 tiles run in one wave
    // stages of 256 elements (k-quants: a super-block; q8_0 / q4_0: 2 stages of 4 blocks)
    const int64_t units = (K + 255) / 256, min_units = 4;
    int64_t ks = (2 * CUS + tiles - 1) / tiles;
    if (ks > units / min_units) ks = units / min_units;
    if (ks > 16) ks = 16;
    return ks > 1 ? (int)ks : 1;
}

int64_t gemm_partial_bytes(int wtype, int64_t M, int64_t N, int64_t K, int64_t batches) {
    const int ks = gemm_ksplit(wtype, M, N, K, batches);
    return ks > 1 ? (int64_t)ks * batches * N * M * 4 : 0;
}

tlh_status launch_gemm(const MatmulArgs &a, hipStream_t stream) {
    const int64_t batches = a.ne12 * a.ne13;
    const int ks = gemm_ksplit(a.wtype, a.M, a.N, a.K, batches);
    if (ks > 1 && !a.part) return set_error(TLH_INVALID, "gemm: a K split of %d needs a partials buffer", ks);
    if (a.wtype == TLH_TYPE_Q8_0 || a.wtype == TLH_TYPE_Q4_0) {
        const tlh_status st = launch_gemm_q8(a, ks, stream);
        return st != TLH_OK || ks == 1 ? st : launch_partial_reduce(a, ks, stream);
    }
    if (a.wtype == TLH_TYPE_Q4_K || a.wtype == TLH_TYPE_Q5_K) {
        const dim3 grid((unsigned)((a.N + GBN - 1) / GBN), (unsigned)((a.M + GBM - 1) / GBM), (unsigned)(batches * ks));
        if (a.wtype == TLH_TYPE_Q4_K) hipLaunchKernelGGL(k_gemm_q4k<TLH_TYPE_Q4_K>, grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(k_gemm_q4k<TLH_TYPE_Q5_K>, grid, dim3(256), 0, stream, a);
        const tlh_status st = check_launch("gemm_q4k");
        return st != TLH_OK || ks == 1 ? st : launch_partial_reduce(a, ks, stream);
    }
    for (int64_t c = 0; c < a.N; c += 16) {
        MatmulArgs s = a;
        s.n0 = a.n0 + c;
        s.N = a.N - c < 16 ? a.N - c : 16;
        const tlh_status st = launch_gemv_mfma(s, stream);
        if (st != TLH_OK) return st;
    }
    return TLH_OK;
}

}  // namespace tlh

// Prefill GEMM for GGML_OP_MUL_MAT with q8_0 / q4_0 weights and more than 16
// activation columns, gfx950.
//
// The CPU backend multiplies a q8_0 / q4_0 row with a q8_0 activation row
// block by block (ggml_vec_dot_q8_0_q8_0_generic, ggml-cpu/quants.c:451-476:
// sum += sumi * (dx * dy); ggml_vec_dot_q4_0_q8_0_generic, :225-258:
// sum += (sumi * dx) * dy), where sumi is the exact integer dot product of one
// 32-element block. Here each block of a 32 x 32 output tile is one
// v_mfma_i32_32x32x32_i8 (K = 32 = one block, exact int32), and the f32 scaling
// follows per block in the CPU's rounding order (only the order of the f32
// sum over blocks differs). The per-block scaling is VALU work of the same
// order as the MFMA issue; the kernel is bound by both together, well under
// the int8 peak, but it reads each weight once per 128-token tile instead of
// once per 16 tokens.
//
// Tiling: 128 weight rows x 128 tokens per workgroup of 4 waves, each wave
// 64 x 64 as 2 x 2 MFMA tiles; K advances in stages of four blocks (128
// elements). Weight codes are staged to LDS as int8 (q4_0 nibbles expanded to
// q - 8), activation codes as they are; LDS holds two stage buffers, written
// one stage ahead and fetched two stages ahead, with one barrier per stage.
#include "kernels.hpp"

namespace tlh {

typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef int v16i32 __attribute__((ext_vector_type(16)));

constexpr int QBM = 128, QBN = 128, QBK = 128, QSB = QBK / 32;  // rows, tokens, K per stage, blocks per stage

// Rows of 128 code bytes = 8 chunks of 16; chunk c of row r sits at chunk
// position c ^ (r & 7), so the 16-byte operand reads of 8 consecutive rows hit
// distinct banks. Scales are block-major so 4 consecutive rows read as a float4.
struct __attribute__((aligned(16))) Q8GemmSmem {
    int8_t A[2][QBM][QBK];
    int8_t B[2][QBN][QBK];
    float dA[2][QSB][QBM];
    float dB[2][QSB][QBN];
};

__device__ __forceinline__ int swz16(int row, int chunk) { return (chunk ^ (row & 7)) << 4; }

__device__ __forceinline__ uint4 ld16(const void *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

// q4_0 nibble bytes -> int8 (n - 8): byte i of `v` -> elements i (low) and i + 16 (high)
// (no borrow crosses a byte: each byte is at least 0x80 before the subtraction)
__device__ __forceinline__ uint32_t nib_lo_m8(uint32_t v) {
    return (((v & 0x0f0f0f0fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}
__device__ __forceinline__ uint32_t nib_hi_m8(uint32_t v) {
    return ((((v >> 4) & 0x0f0f0f0fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// One thread's share of a stage: weight row / token tid / 2, blocks 2h, 2h + 1
// (h = tid & 1) of the stage's four.
struct Q8StageRegs {
    uint4 w[4];   // 64 weight code bytes (q8_0) or the two blocks' nibble bytes in w[0], w[1] (q4_0)
    uint32_t wd;  // the two blocks' f16 scales
    uint4 x[4];   // 64 activation code bytes
    float xd[2];  // the two blocks' activation scales
};

template <int WT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) k_gemm_q8(const MatmulArgs a) {
    __shared__ Q8GemmSmem sm;
    constexpr int BB = block_bytes(WT);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t K = a.K;
    const int64_t nblk = K / QK;
    const uint32_t batches = (uint32_t)(a.ne12 * a.ne13);
    // K chunk kc of gridDim.z / batches (one batch slice: no division)
    const uint32_t kc = batches == 1 ? blockIdx.z : blockIdx.z / batches, batch = blockIdx.z - kc * batches;
    const MmSlice sl = mm_slice(a, batch);
    const int64_t i12 = sl.i12, i13 = sl.i13;
    const uint8_t *W = sl.w;
    const ActView act = act_view(a.act, TLH_TYPE_Q8_0, K, mm_act_rows(a));
    const int64_t m_base = (int64_t)blockIdx.y * QBM;
    const int64_t n_base = (int64_t)blockIdx.x * QBN;

    const int srow = tid >> 1, sh = tid & 1;
    const int64_t grow = m_base + srow < a.M ? m_base + srow : a.M - 1;  // clamped: loads in bounds
    const int64_t gcol = n_base + srow < a.N ? n_base + srow : a.N - 1;
    const uint8_t *wrow = W + grow * a.w_nb1;
    const int64_t arow = a.n0 + gcol + a.N_total * batch;
    const int8_t *xrow = act.qs + arow * K;
    const float *xdrow = act.d + arow * nblk;

    // blocks past K (the last stage of a K that is not a multiple of 128)
    // load block 0 and get zero scales
    auto fetch = [&](int64_t stage, Q8StageRegs &r) {
        const int64_t b0 = stage * QSB + 2 * sh;
        uint16_t d16[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const bool ok = b0 + i < nblk;
            const int64_t b = ok ? b0 + i : 0;
            const uint8_t *bp = wrow + b * BB;
            __builtin_memcpy(&d16[i], bp, 2);
            if constexpr (WT == TLH_TYPE_Q8_0) {
                r.w[2 * i] = ld16(bp + 2);
                r.w[2 * i + 1] = ld16(bp + 18);
            } else {
                r.w[i] = ld16(bp + 2);
            }
            r.x[2 * i] = *(const uint4 *)(xrow + 32 * b);
            r.x[2 * i + 1] = *(const uint4 *)(xrow + 32 * b + 16);
            r.xd[i] = ok ? xdrow[b] : 0.0f;
            if (!ok) d16[i] = 0;
        }
        r.wd = (uint32_t)d16[0] | ((uint32_t)d16[1] << 16);
    };

    auto commit = [&](int64_t stage, const Q8StageRegs &r) {
        const int buf = (int)(stage & 1);
        int8_t *ar = sm.A[buf][srow];
        int8_t *br = sm.B[buf][srow];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint4 c0, c1;
            if constexpr (WT == TLH_TYPE_Q8_0) {
                c0 = r.w[2 * i];
                c1 = r.w[2 * i + 1];
            } else {
                const uint4 v = r.w[i];
                c0 = make_uint4(nib_lo_m8(v.x), nib_lo_m8(v.y), nib_lo_m8(v.z), nib_lo_m8(v.w));
                c1 = make_uint4(nib_hi_m8(v.x), nib_hi_m8(v.y), nib_hi_m8(v.z), nib_hi_m8(v.w));
            }
            const int c = 4 * sh + 2 * i;  // the block's first 16-byte chunk in the row
            *(uint4 *)(ar + swz16(srow, c)) = c0;
            *(uint4 *)(ar + swz16(srow, c + 1)) = c1;
            *(uint4 *)(br + swz16(srow, c)) = r.x[2 * i];
            *(uint4 *)(br + swz16(srow, c + 1)) = r.x[2 * i + 1];
            sm.dA[buf][2 * sh + i][srow] = h2f((uint16_t)(r.wd >> (16 * i)));
            sm.dB[buf][2 * sh + i][srow] = r.xd[i];
        }
    };

    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][jn][r] = 0.0f;

    const int lr = lane & 31, lg = lane >> 5;  // operand row / column; k half of the block
    // this workgroup's stages: chunk kc of equal shares (stage indices are global)
    const int64_t nst = (nblk + QSB - 1) / QSB, nkc = gridDim.z / batches, share = (nst + nkc - 1) / nkc;
    const int64_t g0 = kc * share, stages = g0 + share < nst ? g0 + share : nst;
    Q8StageRegs pre;
    if (g0 < stages) {
        fetch(g0, pre);
        commit(g0, pre);
        if (g0 + 1 < stages) fetch(g0 + 1, pre);
    }
    lds_barrier();
    const v16i32 zero = {};
    for (int64_t st = g0; st < stages; ++st) {
        const int buf = (int)(st & 1);
        // one block at a time: its four products are finished before the next
        // block's MFMAs issue (all of them in flight at once would hold 256
        // result registers)
#pragma unroll 1
        for (int j = 0; j < QSB; ++j) {
            v4i32 av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra = 64 * wm + 32 * i + lr, rb = 64 * wn + 32 * i + lr;
                av[i] = *(const v4i32 *)&sm.A[buf][ra][swz16(ra, 2 * j + lg)];
                bv[i] = *(const v4i32 *)&sm.B[buf][rb][swz16(rb, 2 * j + lg)];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int jn = 0; jn < 2; ++jn) {
                    const v16i32 S = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[jn], zero, 0, 0, 0);
                    const float dy = sm.dB[buf][j][64 * wn + 32 * jn + lr];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 d4 = *(const float4 *)&sm.dA[buf][j][64 * wm + 32 * i + 8 * q + 4 * lg];
                        const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
                            const float s = (float)S[4 * q + e];
                            if constexpr (WT == TLH_TYPE_Q8_0)
                                acc[i][jn][4 * q + e] += s * (dv[e] * dy);
                            else
                                acc[i][jn][4 * q + e] += (s * dv[e]) * dy;
                        }
                    }
                }
        }
        if (st + 1 < stages) {
            commit(st + 1, pre);
            if (st + 2 < stages) fetch(st + 2, pre);
        }
        lds_barrier();
    }

    // lane holds token n = lane % 32 of each 32 x 32 tile and rows 8q + 4 lg + (0..3)
    // (with K chunks, to this chunk's partials [chunk][batch][N][M])
    char *dbase = (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
    float *pbase = nkc > 1 ? a.part + (kc * batches + batch) * a.N * a.M : nullptr;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jn = 0; jn < 2; ++jn) {
            const int64_t n = n_base + 64 * wn + 32 * jn + lr;
            if (n >= a.N) continue;
            float *drow = pbase ? pbase + n * a.M : (float *)(dbase + (a.n0 + n) * a.d_nb1);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t m = m_base + 64 * wm + 32 * i + 8 * q + 4 * lg;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (m + e < a.M) drow[m + e] = acc[i][jn][4 * q + e];
            }
        }
}

tlh_status launch_gemm_q8(const MatmulArgs &a, int ksplit, hipStream_t stream) {
    const dim3 grid((unsigned)((a.N + QBN - 1) / QBN), (unsigned)((a.M + QBM - 1) / QBM),
                    (unsigned)(a.ne12 * a.ne13 * ksplit));
    if (a.wtype == TLH_TYPE_Q8_0) hipLaunchKernelGGL(k_gemm_q8<TLH_TYPE_Q8_0>, grid, dim3(256), 0, stream, a);
    else if (a.wtype == TLH_TYPE_Q4_0) hipLaunchKernelGGL(k_gemm_q8<TLH_TYPE_Q4_0>, grid, dim3(256), 0, stream, a);
    else return set_error(TLH_UNSUPPORTED, "gemm_q8: weight type %d", a.wtype);
    return check_launch("gemm_q8");
}

}  // namespace tlh

// Dense-cache GGML_OP_FLASH_ATTN_EXT over f16 K/V, gfx950.
//
// Computes what ggml's CPU backend computes for FLASH_ATTN_EXT
// (vendor/ggml/src/ggml-cpu/ops.cpp:8468-8700) and what the reference's CUDA
// executor dispatches as fa_main / fa_split + fa_reduce
// (crates/kernels/src/cuda/native/fa.cu:21-232, lowered at
// crates/kernels/src/cuda/lower.rs:575-657):
//   q    f32 [D, nq, nh, nb]           (nb0 = 4)
//   k    f16 [D, L, nhkv, nbk]         (nb0 = 2), head h reads kv head h / (nh / nhkv)
//   v    f16 [DV, L, nhkv, nbk]        (nb0 = 2)
//   mask f16 [>= L, >= nq, mne2, mne3] optional, broadcast over heads and batch
//   dst  f32 [DV, nh, nq, nb]          (nb0 = 4)
// per (query, head): s_j = scale * q.k_j, soft-capped (softcap * tanh), plus
// slope(h) * mask_j (ALiBi slopes from m0, m1, n_head_log2); keys whose mask
// is -inf are skipped; out = sum_j softmax(s)_j v_j (0 when every key is
// masked). q is rounded to f16 first, as the CPU backend does for f16 keys.
//
// Design (MI355X-first, not the CUDA block-per-query structure):
//  * a workgroup (4 waves) owns a tile of up to 16 query rows that share one
//    kv head: gc query heads of the GQA group x qr queries (gc * qr <= 16),
//    so each K/V row is read once for the whole group; a long key range is
//    split into partitions across workgroups (flash-decoding) and merged by a
//    second kernel;
//  * each wave streams 16-key tiles and runs v_mfma_f32_16x16x16_f16 (lane l,
//    g = l / 16, c = l % 16; A lane holds A[c][4g..4g+3], B lane
//    B[4g..4g+3][c], D lane D[4g + r][c]):
//      S^T = K_tile (16 keys x D) . Q^T (D x 16 rows): the A operand (key c,
//            four dims) comes from 16-byte loads of the key row, 64
//            contiguous bytes per key for each group of 4 lanes;
//      P   = softmax numerators (f16): lane (key 4g + r, row c) of S^T is the
//            A operand (row c, keys 4g..4g+3) of
//      O  += P (16 rows x 16 keys) . V_tile (16 keys x DV): lane (c, g) loads
//            the 16-byte pieces of keys 4g..4g+3 at dims 8c..8c+7 (a
//            contiguous 256-byte row per 16 lanes), and its B operand for
//            output tile m is element m of each of the four pieces (two byte
//            permutes), so output tile m holds dims 8c + m;
//  * online softmax in f32 (running max and sum per row), f32 accumulation;
//    waves merge through LDS.
#include "kernels.hpp"

namespace tlh {

constexpr int FA_WAVES = 4;
constexpr int FA_TARGET_WGS = 1024;  // workgroups a split launch aims for
constexpr int FA_MIN_PART = 64;      // fewest keys per partition when split

typedef _Float16 fa_half4 __attribute__((ext_vector_type(4)));
typedef float fa_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ fa_f32x4 fa_mfma(fa_half4 a, fa_half4 b, fa_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ fa_half4 as_h4(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(fa_half4, make_uint2(lo, hi));
}

typedef _Float16 fa_half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ fa_f32x4 fa_mfma32(fa_half8 a, fa_half8 b, fa_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ fa_half8 as_h8(uint4 v) { return __builtin_bit_cast(fa_half8, v); }

// max over lanes c, c + 16, c + 32, c + 48 (the four lane groups of a
// 16 x 16 MFMA output column), with gfx950's lane-swap moves instead of LDS
// permutes: permlane32_swap(v, v) gives (v[l % 32], v[32 + l % 32]) in lane l,
// permlane16_swap(v, v) the lanes l and l ^ 16 of each 32-lane half.
__device__ __forceinline__ float max_across_groups(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int w) { return w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w; }

// Key-row geometry: full 32-dim chunks (one 16-byte load, two MFMA steps
// with dims 32i + 8g + 4s..+3), then a 16-dim step (8-byte load, dims
// 32F + 4g..+3), then an 8-dim step (lanes g < 2 only).
template <int D>
struct KGeom {
    static constexpr int F = D / 32;
    static constexpr bool R16 = (D % 32) >= 16;
    static constexpr bool R8 = (D % 16) == 8;
    static constexpr int STEPS = 2 * F + R16 + R8;
    static constexpr int B16 = 32 * F, B8 = B16 + 16 * R16;
};

// Value-row geometry: 128-dim chunks (16-byte pieces, 8 output tiles with
// dims 128f + 8c + m), then 64 (8-byte, dims 4c + m), 32 (4-byte, 2c + m),
// 16 (2-byte, c) and 8 dims (2-byte, c < 8).
template <int DV>
struct VGeom {
    static constexpr int F = DV / 128;
    static constexpr int REM = DV % 128;
    static constexpr bool R64 = REM >= 64, R32 = (REM % 64) >= 32, R16 = (REM % 32) >= 16, R8 = (REM % 16) == 8;
    static constexpr int B64 = 128 * F, B32 = B64 + 64 * R64, B16 = B32 + 32 * R32, B8 = B16 + 16 * R16;
    static constexpr int T64 = 8 * F, T32 = T64 + 4 * R64, T16 = T32 + 2 * R32, T8 = T16 + R16;
    static constexpr int NO = T8 + R8;  // output tiles
    // output dim of tile n in column c
    __device__ static constexpr int dim(int n, int c) {
        return n < T64   ? 128 * (n / 8) + 8 * c + n % 8
               : n < T32 ? B64 + 4 * c + (n - T64)
               : n < T16 ? B32 + 2 * c + (n - T32)
               : n < T8  ? B16 + c
                         : B8 + c;
    }
    __device__ static constexpr bool live(int n, int c) { return n < T8 || c < 8; }
};

struct FaArgs {
    const char *q, *k, *v, *mask;
    char *dst;
    float *part;   // partials [nb][nh][nq][P][DV + 2] when P > 1
    int mask_vec;  // mask rows 16-byte aligned: scanned in 16-byte runs
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int64_t d_nb1, d_nb2, d_nb3;
    int m_ne2, m_ne3;
    int nq, nh, nb, L, nhkv, rk3;  // rk3 = nb / nbk
    int G, gc, qr, HC, QC;         // heads per kv head; tile = gc heads x qr queries
    int P, part_len;
    float scale, max_bias, m0, m1, softcap;
    int nhl2;
};

template <int D, int DV, bool MASK>
struct FaRegs {
    using KG = KGeom<D>;
    using VG = VGeom<DV>;
    uint4 kf[KG::F > 0 ? KG::F : 1];
    uint2 k16, k8;
    uint4 vf[VG::F > 0 ? VG::F : 1][4];
    uint2 v64[4];
    uint32_t v32[4], v16[4], v8[4];
    uint32_t mk[4];
};

template <int D, int DV, bool MASK, bool PIPE>
__global__ void __launch_bounds__(256) k_flash_attn(const FaArgs a) {
    using KG = KGeom<D>;
    using VG = VGeom<DV>;
    using Regs = FaRegs<D, DV, MASK>;
    __shared__ float s_m[FA_WAVES][16], s_l[FA_WAVES][16];
    __shared__ float s_acc[FA_WAVES][16][DV];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;

    // workgroup -> (query chunk, head chunk, partition); kv head; batch
    const int qc = blockIdx.x % a.QC;
    const int hc = (blockIdx.x / a.QC) % a.HC;
    const int p = blockIdx.x / (a.QC * a.HC);
    const int hk = blockIdx.y, ib = blockIdx.z;
    int j0 = p * a.part_len;
    int j1 = min(a.L, j0 + a.part_len);
    const int nrows = min(a.qr, a.nq - qc * a.qr) * a.gc;  // live rows: a prefix of the tile

    // row c of the tile: query qc*qr + c/gc, head hk*G + hc*gc + c%gc
    const bool rlive = c < nrows;
    const int rr = rlive ? c : 0;
    const int iq = qc * a.qr + rr / a.gc;
    const int h = hk * a.G + hc * a.gc + rr % a.gc;
    if constexpr (MASK) {
        // keys that are -inf in every mask row of the tile are skipped: the
        // live range [lo, hi) of the tile's rows inside [j0, j1), lane (g, c)
        // scanning row c in runs of 8 keys j0 + 8 (g + 4 k), then the union
        // over the 16 rows and 4 groups
        int lo = INT32_MAX, hi = 0;
        if (rlive) {
            const uint16_t *mr = (const uint16_t *)(a.mask + iq * a.m_nb1 + (int64_t)(h % a.m_ne2) * a.m_nb2 +
                                                    (int64_t)(ib % a.m_ne3) * a.m_nb3);
            int jt = j0;  // keys past the 16-byte runs, one by one
            if (a.mask_vec) {
                const int jv = j0 + (j1 - j0) / 8 * 8;
#pragma unroll 8
                for (int jb = j0 + 8 * g; jb < jv; jb += 32) {
                    const uint4 w = *(const uint4 *)(mr + jb);
                    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (((ws[e / 2] >> (16 * (e & 1))) & 0xffffu) != 0xfc00u) {  // not f16 -inf
                            lo = min(lo, jb + e);
                            hi = max(hi, jb + e + 1);
                        }
                }
                jt = jv;
            }
#pragma unroll 8
            for (int j = jt + g; j < j1; j += 4)
                if (mr[j] != 0xfc00u) {
                    lo = min(lo, j);
                    hi = max(hi, j + 1);
                }
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            lo = min(lo, __shfl_xor(lo, o, 64));
            hi = max(hi, __shfl_xor(hi, o, 64));
        }
        j0 = max(j0, lo);
        j1 = min(j1, hi);
    }

    // Q^T operand (row c, dims of step st for group g), rounded to f16
    fa_half4 qb[KG::STEPS];
    {
        const float *qrow = (const float *)(a.q + iq * a.q_nb1 + h * a.q_nb2 + ib * a.q_nb3);
#pragma unroll
        for (int st = 0; st < KG::STEPS; ++st) {
            const int d0 = st < 2 * KG::F ? 32 * (st / 2) + 8 * g + 4 * (st % 2)
                           : (KG::R16 && st == 2 * KG::F) ? KG::B16 + 4 * g
                                                          : KG::B8 + 4 * (g & 1);
            const bool ok = rlive && !(KG::R8 && st == KG::STEPS - 1 && g >= 2);
            fa_half4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (_Float16)qrow[d0 + e];
            qb[st] = ok ? v : (fa_half4){};
        }
    }
    float slope = 1.0f;
    const uint16_t *mrow = nullptr;
    if constexpr (MASK) {
        if (a.max_bias > 0.0f)
            slope = h < a.nhl2 ? powf(a.m0, (float)(h + 1)) : powf(a.m1, (float)(2 * (h - a.nhl2) + 1));
        mrow = (const uint16_t *)(a.mask + iq * a.m_nb1 + (h % a.m_ne2) * a.m_nb2 + (ib % a.m_ne3) * a.m_nb3);
    }
    const float scale = a.scale, softcap = a.softcap;

    const char *kb = a.k + hk * a.k_nb2 + (ib / a.rk3) * a.k_nb3;
    const char *vb = a.v + hk * a.v_nb2 + (ib / a.rk3) * a.v_nb3;
    const int64_t k_nb1 = a.k_nb1, v_nb1 = a.v_nb1;

    float m_run = -INFINITY, l_run = 0.0f;  // row c: running max; this lane's partial sum
    fa_f32x4 o[VG::NO];
#pragma unroll
    for (int n = 0; n < VG::NO; ++n) o[n] = (fa_f32x4){};

    const int ntiles = j1 > j0 ? (j1 - j0 + 15) / 16 : 0;
    const int my_tiles = ntiles > wave ? (ntiles - wave + FA_WAVES - 1) / FA_WAVES : 0;

    // Loads of tile k of this wave (keys t..t+15, t = j0 + 16 (wave + 4k)).
    // Rows past the partition read its last row instead (their scores are
    // masked), so every load is unconditional and in bounds.
    auto load_tile = [&](int k, Regs &R) {
        const int t = j0 + 16 * (wave + FA_WAVES * k);
        const char *kr = kb + (int64_t)min(t + c, j1 - 1) * k_nb1;
#pragma unroll
        for (int i = 0; i < KG::F; ++i) R.kf[i] = *(const uint4 *)(kr + 64 * i + 16 * g);
        if constexpr (KG::R16) R.k16 = *(const uint2 *)(kr + 2 * KG::B16 + 8 * g);
        if constexpr (KG::R8) R.k8 = *(const uint2 *)(kr + 2 * KG::B8 + 8 * (g & 1));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = min(t + 4 * g + j, j1 - 1);
            const char *vr = vb + (int64_t)key * v_nb1;
#pragma unroll
            for (int f = 0; f < VG::F; ++f) R.vf[f][j] = *(const uint4 *)(vr + 256 * f + 16 * c);
            if constexpr (VG::R64) R.v64[j] = *(const uint2 *)(vr + 2 * VG::B64 + 8 * c);
            if constexpr (VG::R32) R.v32[j] = *(const uint32_t *)(vr + 2 * VG::B32 + 4 * c);
            if constexpr (VG::R16) R.v16[j] = *(const uint16_t *)(vr + 2 * VG::B16 + 2 * c);
            if constexpr (VG::R8) R.v8[j] = *(const uint16_t *)(vr + 2 * VG::B8 + 2 * (c & 7));
            if constexpr (MASK) R.mk[j] = mrow[key];
        }
    };
    auto compute_tile = [&](int k, const Regs &R) {
        const int t = j0 + 16 * (wave + FA_WAVES * k);
        fa_f32x4 S = (fa_f32x4){};
#pragma unroll
        for (int i = 0; i < KG::F; ++i) {
            S = fa_mfma(as_h4(R.kf[i].x, R.kf[i].y), qb[2 * i], S);
            S = fa_mfma(as_h4(R.kf[i].z, R.kf[i].w), qb[2 * i + 1], S);
        }
        if constexpr (KG::R16) S = fa_mfma(as_h4(R.k16.x, R.k16.y), qb[2 * KG::F], S);
        if constexpr (KG::R8) {
            const uint2 kk = g < 2 ? R.k8 : make_uint2(0, 0);
            S = fa_mfma(as_h4(kk.x, kk.y), qb[KG::STEPS - 1], S);
        }
        // lane (row c, keys t + 4g + r)
        float x[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float s = S[r] * scale;
            if (softcap != 0.0f) s = softcap * tanhf(s);
            if constexpr (MASK) {
                const float mv = slope * h2f((uint16_t)R.mk[r]);
                s = mv == -INFINITY ? -INFINITY : s + mv;
            }
            x[r] = t + 4 * g + r < j1 ? s : -INFINITY;
            mx = fmaxf(mx, x[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        // exp(-inf - (-inf)) is NaN: a row with every key so far masked keeps 0
        const bool none = m_new == -INFINITY;
        const float alpha = none ? 1.0f : __expf(m_run - m_new);
        m_run = m_new;
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = none ? 0.0f : __expf(x[r] - m_new);
        l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
        const fa_half4 pa = {(_Float16)pr[0], (_Float16)pr[1], (_Float16)pr[2], (_Float16)pr[3]};
        // output rows are tile rows 4g + r: their alphas live in lanes 4g + r
        float ao[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ao[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int n = 0; n < VG::NO; ++n) {
            uint32_t lo, hi;
            if (n < VG::T64) {
                const int f = n / 8, w = (n % 8) / 2;
                const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
                lo = __builtin_amdgcn_perm(word(R.vf[f][1], w), word(R.vf[f][0], w), sel);
                hi = __builtin_amdgcn_perm(word(R.vf[f][3], w), word(R.vf[f][2], w), sel);
            } else if (n < VG::T32) {
                const int m = n - VG::T64, w = m / 2;
                const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t a0 = w ? R.v64[0].y : R.v64[0].x, a1 = w ? R.v64[1].y : R.v64[1].x;
                const uint32_t a2 = w ? R.v64[2].y : R.v64[2].x, a3 = w ? R.v64[3].y : R.v64[3].x;
                lo = __builtin_amdgcn_perm(a1, a0, sel);
                hi = __builtin_amdgcn_perm(a3, a2, sel);
            } else if (n < VG::T16) {
                const uint32_t sel = ((n - VG::T32) & 1) ? 0x07060302u : 0x05040100u;
                lo = __builtin_amdgcn_perm(R.v32[1], R.v32[0], sel);
                hi = __builtin_amdgcn_perm(R.v32[3], R.v32[2], sel);
            } else if (n < VG::T8) {
                lo = (R.v16[0] & 0xffffu) | (R.v16[1] << 16);
                hi = (R.v16[2] & 0xffffu) | (R.v16[3] << 16);
            } else {
                lo = (R.v8[0] & 0xffffu) | (R.v8[1] << 16);
                hi = (R.v8[2] & 0xffffu) | (R.v8[3] << 16);
            }
            fa_f32x4 on = o[n];
#pragma unroll
            for (int r = 0; r < 4; ++r) on[r] *= ao[r];
            o[n] = fa_mfma(pa, as_h4(lo, hi), on);
        }
    };

    Regs ra;
    if (my_tiles > 0) load_tile(0, ra);
    if constexpr (PIPE) {
        // two register sets in turn: the next tile's loads are in flight while
        // this one is multiplied (past the last tile it rereads its own, a
        // cache hit, so the compiler can count the loads)
        Regs rb;
        for (int k = 0; k < my_tiles; k += 2) {
            load_tile(k + 1 < my_tiles ? k + 1 : k, rb);
            compute_tile(k, ra);
            if (k + 1 >= my_tiles) break;
            load_tile(k + 2 < my_tiles ? k + 2 : k + 1, ra);
            compute_tile(k + 1, rb);
        }
    } else {
        for (int k = 0; k < my_tiles; ++k) {
            compute_tile(k, ra);
            if (k + 1 < my_tiles) load_tile(k + 1, ra);
        }
    }

    // row sums over the 4 key groups, then merge the waves through LDS
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (g == 0) {
        s_m[wave][c] = m_run;
        s_l[wave][c] = l_run;
    }
#pragma unroll
    for (int n = 0; n < VG::NO; ++n)
        if (VG::live(n, c))
#pragma unroll
            for (int r = 0; r < 4; ++r) s_acc[wave][4 * g + r][VG::dim(n, c)] = o[n][r];
    __syncthreads();
    for (int e = threadIdx.x; e < nrows * DV; e += blockDim.x) {
        const int row = e / DV, d = e % DV;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < FA_WAVES; ++w) M = fmaxf(M, s_m[w][row]);
        float lsum = 0.0f, acc = 0.0f;
#pragma unroll
        for (int w = 0; w < FA_WAVES; ++w) {
            const float f = s_m[w][row] == -INFINITY ? 0.0f : __expf(s_m[w][row] - M);
            lsum += f * s_l[w][row];
            acc += f * s_acc[w][row][d];
        }
        const int riq = qc * a.qr + row / a.gc;
        const int rh = hk * a.G + hc * a.gc + row % a.gc;
        if (a.P == 1) {
            const float inv = lsum == 0.0f ? 0.0f : 1.0f / lsum;
            float *out = (float *)(a.dst + rh * a.d_nb1 + riq * a.d_nb2 + ib * a.d_nb3);
            out[d] = acc * inv;
        } else {
            float *slot = a.part + ((((int64_t)ib * a.nh + rh) * a.nq + riq) * a.P + p) * (DV + 2);
            slot[2 + d] = acc;
            if (d == 0) {
                slot[0] = M;
                slot[1] = lsum;
            }
        }
    }
}

// Prefill form for head size 128 (D = DV), many queries: a workgroup of 8
// waves owns 64 rows in 4 groups of 16 -- group r the 16 queries qb + 16 (r /
// gw) .. + 15 of head hk * G + hc * gw + r % gw (gw = min(G, 4) heads of the KV
// head's group) -- and walks the keys in 64-key tiles that every wave reads
// from LDS: each K / V row is fetched from L2 once per 64 rows instead of once
// per 16. Waves r and r + 4 share row group r, each taking 32 of a tile's 64
// keys (two waves a SIMD hide each other's latencies), and merge at the end. The tiles
// come straight from global memory (global_load_lds_dwordx4, double-buffered:
// tile t + 1 loads while tile t is multiplied). K rows are stored with their
// 16-byte chunks XOR-swizzled by the key (chunk q of key c at position
// q ^ (c % 16)), so the A-operand reads of 16 keys hit distinct banks; V rows
// as they are (the B-operand pieces of one key are contiguous). Per wave and
// 32-key step the products run on gfx950's v_mfma_f32_16x16x32_f16 (S^T = K .
// Q^T, online softmax on S^T's lane layout in the log2 domain, O += P . V on 8
// output tiles); a step whose mask values are all zero skips the mask
// arithmetic; no key partitions.
constexpr int FR_TK = 64;    // keys per tile
constexpr int FR_ROW = 256;  // bytes of a K / V row (128 f16)
constexpr int FR_KV = FR_TK * FR_ROW;           // bytes of a tile's K (or V) rows
constexpr int FR_BUF = 2 * FR_KV + 64 * FR_TK * 2;  // a tile buffer: K, V, the f16 mask tile
typedef __attribute__((address_space(3))) void fa_lds_void;

// 16 bytes a lane from global memory straight to LDS (lane l's bytes land at
// lds + 16 l)
__device__ __forceinline__ void dma16(const void *g, fa_lds_void *lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

struct FaRowsArgs {
    FaArgs f;
    int gw;   // heads per workgroup (waves share the query block when gw < 4)
    int QB;   // query blocks of 64 / gw queries
};

template <bool MASK>
__global__ void __launch_bounds__(512) k_flash_attn_rows(const FaRowsArgs ra) {
    const FaArgs &a = ra.f;
    // two tile buffers (K rows, V rows, then the 64 x 64 mask tile, row
    // 16 rg + c), each a separate array named statically where it is read or
    // filled: the compiler then sees that the reads of one buffer do not overlap
    // the direct-to-LDS loads into the other, and inserts no wait for those
    // loads before every read
    __shared__ __attribute__((aligned(16))) uint8_t T0[FR_BUF], T1[FR_BUF];
    __shared__ float Mo[4][16][128], Mm[4][16], Ml[4][16];  // the key halves' merge
    // the wave index in a scalar register: the per-wave step conditions below
    // are then scalar branches, not exec masks
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = wave & 3, kh = wave >> 2;  // row group, key half
    const int g = lane >> 4, c = lane & 15;
    const int gw = ra.gw, qpw = 64 / gw;  // queries per workgroup
    // heavy (late) query blocks first: causal rows at the end see the most keys
    const int qblk = ra.QB - 1 - (int)(blockIdx.x % ra.QB);
    const int hc = (int)(blockIdx.x / ra.QB);
    const int hk = blockIdx.y, ib = blockIdx.z;
    const int q0 = qblk * qpw + 16 * (rg / gw);
    const int h = hk * a.G + hc * gw + rg % gw;
    const int iq = q0 + c;  // this lane's row (query) in S^T's layout
    const bool rlive = iq < a.nq;
    const int iqc = rlive ? iq : a.nq - 1;
    const int L = a.L;

    // Q^T operand of the wave's rows (row c: query iq of head h), rounded to f16
    // (B operand of S^T = K . Q^T on v_mfma_f32_16x16x32_f16: lane (c, g) holds
    // row c's dims 32 s + 8 g .. + 7 for step s)
    // (loaded after the first tile's loads are issued, so the two latencies
    // overlap; all eight loads go out before any is used. A row past nq reads
    // row nq - 1 instead: its results are never stored)
    fa_half8 qb[4];
    auto load_q = [&](float4 (&qv)[4][2]) {
        const float *qrow = (const float *)(a.q + iqc * a.q_nb1 + h * a.q_nb2 + ib * a.q_nb3);
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            qv[st][0] = *(const float4 *)(qrow + 32 * st + 8 * g);
            qv[st][1] = *(const float4 *)(qrow + 32 * st + 8 * g + 4);
        }
    };
    auto convert_q = [&](const float4 (&qv)[4][2]) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const float4 lo = qv[st][0], hi = qv[st][1];
            qb[st] = (fa_half8){(_Float16)lo.x, (_Float16)lo.y, (_Float16)lo.z, (_Float16)lo.w,
                                (_Float16)hi.x, (_Float16)hi.y, (_Float16)hi.z, (_Float16)hi.w};
        }
    };
    float slope = 1.0f;
    const char *mdma = nullptr;  // the mask row this lane's DMA fills: row 8 wave + lane / 8, keys 8 (lane % 8) ..
    if constexpr (MASK) {
        if (a.max_bias > 0.0f)
            slope = h < a.nhl2 ? powf(a.m0, (float)(h + 1)) : powf(a.m1, (float)(2 * (h - a.nhl2) + 1));
        const int R = 8 * wave + (lane >> 3), rgR = R >> 4, cR = R & 15;
        const int qR = min(qblk * qpw + 16 * (rgR / gw) + cR, a.nq - 1);
        const int hR = hk * a.G + hc * gw + rgR % gw;
        mdma = a.mask + qR * a.m_nb1 + (int64_t)(hR % a.m_ne2) * a.m_nb2 + (int64_t)(ib % a.m_ne3) * a.m_nb3;
    }
    const float scale = a.scale, softcap = a.softcap;
    const char *kb = a.k + hk * a.k_nb2 + (ib / a.rk3) * a.k_nb3;
    const char *vb = a.v + hk * a.v_nb2 + (ib / a.rk3) * a.v_nb3;

    // tile loads: instruction i of wave w fills keys 4 (2 w + i) .. + 3 of the
    // tile, lane l key + l / 16 at chunk position l % 16 (K: the chunk
    // (l % 16) ^ (key % 16) of the row; V: chunk l % 16). Keys past L read
    // row L - 1 (their scores are masked).
    const int ntiles = (L + FR_TK - 1) / FR_TK;
    auto load_tile = [&](int t, uint8_t (&Td)[FR_BUF]) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int kk = 4 * (2 * wave + i) + (lane >> 4);
            const int key = min(FR_TK * t + kk, L - 1);
            const int pos = lane & 15;
            dma16(kb + (int64_t)key * a.k_nb1 + 16 * (pos ^ (kk & 15)), (fa_lds_void *)(Td + 4 * (2 * wave + i) * FR_ROW));
            dma16(vb + (int64_t)key * a.v_nb1 + 16 * pos, (fa_lds_void *)(Td + FR_KV + 4 * (2 * wave + i) * FR_ROW));
        }
    };
    // the mask tile (64 rows x 64 keys) straight to LDS with K and V: wave w
    // fills rows 8w .. 8w + 7, lane l 16 bytes (keys 8 (l % 8) ..) of row
    // 8w + l / 8. L is a multiple of 8, so no 8-key chunk straddles the end;
    // chunks past it reread the last one (those keys are masked by index).
    auto load_mask = [&](int t, uint8_t (&Td)[FR_BUF]) {
        if constexpr (MASK) {
            const int key = min(FR_TK * t + 8 * (lane & 7), L - 8);
            dma16(mdma + 2 * key, (fa_lds_void *)(Td + 2 * FR_KV + 8 * wave * FR_TK * 2));
        }
    };

    // Online softmax with lazy rescaling, in the log2 domain (x = s * log2 e):
    // m_ref, the value the exponentials are taken against, moves to the
    // running max only when that has grown by more than 8 (then O and l are
    // rescaled); otherwise p = 2^(x - m_ref) <= 2^8, well inside f16 for the P
    // operand, and the final O / l is unchanged.
    constexpr float LOG2E = 1.4426950408889634f;
    const float cs = scale * LOG2E;
    float m_ref = -INFINITY, l_run = 0.0f;
    fa_f32x4 o[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) o[n] = (fa_f32x4){};

    // tile t from buffer Tc, while tile t + 1 goes to Tn; this
    // wave takes the tile's keys 32 kh .. + 31 as one step of two 16-key
    // halves. S^T of a half is four v_mfma_f32_16x16x32_f16 (lane (c, g): key
    // c's dims 32 s + 8 g .. + 7, one 16-byte LDS read); its lane layout (key
    // 16 hf + 4 g + r, row c) is, over both halves, exactly the A operand of
    // O += P . V with the step's 32 keys in the order (4 g .. 4 g + 3, 16 + 4 g
    // .. + 3) for lane group g -- and the V operand takes its keys in the same
    // order: lane (c, g) reads those 8 keys' 16-byte pieces at dims 8 c .. + 7,
    // and output tile m (dims 8 c + m) gets element m of each (four byte
    // permutes).
    auto tile = [&](int t, const uint8_t (&Tc)[FR_BUF], uint8_t (&Tn)[FR_BUF]) {
        if (t + 1 < ntiles) {  // the other buffer: free since the last barrier
            load_tile(t + 1, Tn);
            load_mask(t + 1, Tn);
        }
        const int kt = FR_TK * t + 32 * kh;  // first key of this wave's step
        uint4 kf[2][4];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const uint8_t *kr = Tc + (32 * kh + 16 * hf + c) * FR_ROW;
#pragma unroll
            for (int s = 0; s < 4; ++s) kf[hf][s] = *(const uint4 *)(kr + 16 * ((4 * s + g) ^ c));
        }
        // V pieces: keys 16 hf + 4g + j of the step, dims 8c .. 8c + 7 (read with
        // the keys, so their latency overlaps the S^T products)
        uint4 vf[2][4];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int j = 0; j < 4; ++j) vf[hf][j] = *(const uint4 *)(Tc + FR_KV + (32 * kh + 16 * hf + 4 * g + j) * FR_ROW + 16 * c);
        // this lane's mask values: row c of the group, keys 4g .. 4g + 3 of each half.
        // A step whose keys are all inside L and whose mask values are all +-0 for
        // every row of the wave (and no soft cap) takes the plain path: s + slope * 0
        // is s.
        uint2 mw[2] = {};
        bool plain = kt + 32 <= L && softcap == 0.0f;
        if constexpr (MASK) {
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
                mw[hf] = *(const uint2 *)(Tc + 2 * FR_KV + ((16 * rg + c) * FR_TK + 32 * kh + 16 * hf + 4 * g) * 2);
            plain = plain && __builtin_amdgcn_ballot_w64(((mw[0].x | mw[0].y | mw[1].x | mw[1].y) & 0x7fff7fffu) != 0) == 0;
        }
        auto mk = [&](int hf, int r) -> uint32_t {
            const uint32_t w = r < 2 ? mw[hf].x : mw[hf].y;
            return r & 1 ? w >> 16 : w & 0xffffu;
        };
        // nothing live for any of the wave's rows in its 32 keys: skip (uniform)
        bool live = kt < L;
        if (!plain) {
            bool any = false;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    bool k_live = kt + 16 * hf + 4 * g + r < L;
                    if constexpr (MASK) k_live = k_live & (mk(hf, r) != 0xfc00u);
                    any = any | k_live;
                }
            live = live && __builtin_amdgcn_ballot_w64(any && rlive) != 0;
        }
        if (live) {
            fa_f32x4 S[2];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                fa_f32x4 S0 = fa_mfma32(as_h8(kf[hf][0]), qb[0], (fa_f32x4){});
                fa_f32x4 S1 = fa_mfma32(as_h8(kf[hf][1]), qb[1], (fa_f32x4){});
                S0 = fa_mfma32(as_h8(kf[hf][2]), qb[2], S0);
                S1 = fa_mfma32(as_h8(kf[hf][3]), qb[3], S1);
                S[hf] = S0 + S1;
            }
            float x[2][4];
            if (plain) {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[hf][r] = S[hf][r] * cs;
            } else {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sv = S[hf][r] * scale;
                        if (softcap != 0.0f) sv = softcap * tanhf(sv);
                        if constexpr (MASK) {
                            const float mv = slope * h2f((uint16_t)mk(hf, r));
                            sv = mv == -INFINITY ? -INFINITY : sv + mv;
                        }
                        x[hf][r] = kt + 16 * hf + 4 * g + r < L ? sv * LOG2E : -INFINITY;
                    }
            }
            float mx = fmaxf(fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3])),
                             fmaxf(fmaxf(x[1][0], x[1][1]), fmaxf(x[1][2], x[1][3])));
            mx = max_across_groups(mx);
            // row c's new reference when its max grew by more than 8 (or was -inf)
            const bool grow = mx > m_ref + 8.0f || (m_ref == -INFINITY && mx != -INFINITY);
            if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // some row rescales: O and l of every row
                const float m_new = grow ? mx : m_ref;
                const float alpha = m_ref == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_ref - m_new);
                m_ref = m_new;
                l_run *= alpha;
                float ao[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) ao[r] = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
                for (int n = 0; n < 8; ++n)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[n][r] *= ao[r];
            }
            const bool none = m_ref == -INFINITY;
            float pr[2][4];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int r = 0; r < 4; ++r) pr[hf][r] = none ? 0.0f : __builtin_amdgcn_exp2f(x[hf][r] - m_ref);
            l_run += ((pr[0][0] + pr[0][1]) + (pr[0][2] + pr[0][3])) + ((pr[1][0] + pr[1][1]) + (pr[1][2] + pr[1][3]));
            const fa_half8 pa = {(_Float16)pr[0][0], (_Float16)pr[0][1], (_Float16)pr[0][2], (_Float16)pr[0][3],
                                 (_Float16)pr[1][0], (_Float16)pr[1][1], (_Float16)pr[1][2], (_Float16)pr[1][3]};
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const int w = n / 2;
                const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
                uint4 b;
                b.x = __builtin_amdgcn_perm(word(vf[0][1], w), word(vf[0][0], w), sel);
                b.y = __builtin_amdgcn_perm(word(vf[0][3], w), word(vf[0][2], w), sel);
                b.z = __builtin_amdgcn_perm(word(vf[1][1], w), word(vf[1][0], w), sel);
                b.w = __builtin_amdgcn_perm(word(vf[1][3], w), word(vf[1][2], w), sel);
                o[n] = fa_mfma32(pa, as_h8(b), o[n]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): tile t + 1 landed
        lds_barrier();
    };

    // even tiles in buffer 0, odd ones in buffer 1; q's loads go out with tile 0's
    if (ntiles > 0) {
        load_tile(0, T0);
        load_mask(0, T0);
    }
    float4 qv[4][2];
    load_q(qv);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): tile 0 and q landed
    convert_q(qv);
    lds_barrier();
    for (int t = 0; t < ntiles; t += 2) {
        tile(t, T0, T1);
        if (t + 1 < ntiles) tile(t + 1, T1, T0);
    }

    // merge the key halves: the second wave of each row group hands its
    // reference, sum and accumulators (rows 4g + r, dims 8c .. 8c + 7) to the
    // first, which rescales both to the larger reference, normalizes and stores
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (kh == 1) {
        if (g == 0) Mm[rg][c] = m_ref, Ml[rg][c] = l_run;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            *(float4 *)&Mo[rg][4 * g + r][8 * c] = make_float4(o[0][r], o[1][r], o[2][r], o[3][r]);
            *(float4 *)&Mo[rg][4 * g + r][8 * c + 4] = make_float4(o[4][r], o[5][r], o[6][r], o[7][r]);
        }
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        const float m0 = __shfl(m_ref, row, 64), l0 = __shfl(l_run, row, 64);
        const float m1 = Mm[rg][row], l1 = Ml[rg][row];
        const float M = fmaxf(m0, m1);
        const float f0 = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
        const float f1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
        const float lsum = f0 * l0 + f1 * l1;
        const int orow = q0 + row;
        if (orow >= a.nq) continue;
        const float inv = lsum == 0.0f ? 0.0f : 1.0f / lsum;
        const float4 p0 = *(const float4 *)&Mo[rg][row][8 * c], p1 = *(const float4 *)&Mo[rg][row][8 * c + 4];
        float *out = (float *)(a.dst + h * a.d_nb1 + orow * a.d_nb2 + ib * a.d_nb3) + 8 * c;
        *(float4 *)out = make_float4((f0 * o[0][r] + f1 * p0.x) * inv, (f0 * o[1][r] + f1 * p0.y) * inv,
                                     (f0 * o[2][r] + f1 * p0.z) * inv, (f0 * o[3][r] + f1 * p0.w) * inv);
        *(float4 *)(out + 4) = make_float4((f0 * o[4][r] + f1 * p1.x) * inv, (f0 * o[5][r] + f1 * p1.y) * inv,
                                           (f0 * o[6][r] + f1 * p1.z) * inv, (f0 * o[7][r] + f1 * p1.w) * inv);
    }
}

// Merge the partitions of one (batch, head, query) row: every partition was
// written (an empty one as max -inf, sum 0). Each thread reads the maxima,
// sums and its dims of up to 16 partitions in one round of loads and folds
// them into a running (max, sum, acc) rescaled online.
template <int DV>
__global__ void __launch_bounds__(256) k_flash_attn_reduce(const FaArgs a) {
    constexpr int CHUNK = 16;
    const int iq = blockIdx.x, h = blockIdx.y, ib = blockIdx.z;
    const int P = a.P;
    const float *base = a.part + (((int64_t)ib * a.nh + h) * a.nq + iq) * P * (DV + 2);
    float *out = (float *)(a.dst + h * a.d_nb1 + iq * a.d_nb2 + ib * a.d_nb3);
    for (int d = threadIdx.x; d < DV; d += blockDim.x) {
        float M = -INFINITY, lsum = 0.0f, acc = 0.0f;
        for (int p0 = 0; p0 < P; p0 += CHUNK) {
            float m[CHUNK], l[CHUNK], v[CHUNK];
#pragma unroll
            for (int i = 0; i < CHUNK; ++i) {
                const int64_t o = (int64_t)(p0 + i < P ? p0 + i : p0) * (DV + 2);
                m[i] = base[o];
                l[i] = base[o + 1];
                v[i] = base[o + 2 + d];
            }
            float cm = -INFINITY;
#pragma unroll
            for (int i = 0; i < CHUNK; ++i) cm = fmaxf(cm, m[i]);  // repeats of p0 change nothing
            const float Mn = fmaxf(M, cm);
            if (Mn == -INFINITY) continue;
            const float so = __expf(M - Mn);  // 0 while M is -inf (then lsum and acc are 0)
            lsum *= so;
            acc *= so;
#pragma unroll
            for (int i = 0; i < CHUNK; ++i) {
                const float w = p0 + i < P ? __expf(m[i] - Mn) : 0.0f;  // exp(-inf) = 0: empty partitions
                lsum += w * l[i];
                acc += w * v[i];
            }
            M = Mn;
        }
        out[d] = acc * (lsum == 0.0f ? 0.0f : 1.0f / lsum);
    }
}

// ------------------------------------------------------------------ host
bool flash_attn_head_sizes_ok(int64_t D, int64_t DV) {
    if (D == 192 && DV == 128) return true;
    if (D != DV) return false;
    switch (D) {
    case 32: case 40: case 64: case 72: case 80: case 96: case 112: case 128: case 192: case 256: return true;
    default: return false;
    }
}

// Row tiles and key partitions of a launch (a pure function of the shape,
// so the scratch size can be planned ahead).
struct FaPlan {
    int G, gc, qr, HC, QC, P, part_len;
};

static FaPlan fa_plan(int64_t nq, int64_t nh, int64_t nhkv, int64_t nb, int64_t L) {
    FaPlan pl;
    pl.G = (int)(nh / nhkv);
    pl.gc = pl.G < 16 ? pl.G : 16;  // a divisor of G, at most 16
    while (pl.G % pl.gc) --pl.gc;
    pl.qr = nq > 1 ? 16 / pl.gc : 1;
    if (pl.qr > nq) pl.qr = (int)nq;
    pl.HC = pl.G / pl.gc;
    pl.QC = (int)((nq + pl.qr - 1) / pl.qr);
    const int64_t tiles = (int64_t)pl.QC * pl.HC * nhkv * nb;
    int64_t P = (FA_TARGET_WGS + tiles - 1) / tiles;
    const int64_t maxP = L / FA_MIN_PART;
    if (P > maxP) P = maxP;
    if (P < 1) P = 1;
    int64_t part = (L + P - 1) / P;
    part = (part + 63) / 64 * 64;
    if (part < 64) part = 64;
    pl.part_len = (int)part;
    pl.P = L > 0 ? (int)((L + part - 1) / part) : 1;
    return pl;
}

static int64_t fa_partial_bytes(int64_t DV, int64_t nq, int64_t nh, int64_t nhkv, int64_t nb, int64_t L) {
    const FaPlan pl = fa_plan(nq, nh, nhkv, nb, L);
    const int64_t b = pl.P > 1 ? nb * nh * nq * pl.P * (DV + 2) * (int64_t)sizeof(float) : 0;
    return (b + 255) / 256 * 256;
}

int64_t flash_attn_scratch_bytes(int64_t DV, int64_t nq, int64_t nh, int64_t nhkv, int64_t nb, int64_t L,
                                 int64_t mask_rows) {
    (void)mask_rows;  // the kernels scan the mask themselves
    return fa_partial_bytes(DV, nq, nh, nhkv, nb, L);
}

template <int D, int DV>
static void launch_fa(const FaArgs &a, bool mask, hipStream_t stream) {
    constexpr bool PIPE = D <= 128 && DV <= 128;  // two register sets fit
    const dim3 grid(a.QC * a.HC * a.P, a.nhkv, a.nb);
    if (mask)
        hipLaunchKernelGGL((k_flash_attn<D, DV, true, PIPE>), grid, dim3(64 * FA_WAVES), 0, stream, a);
    else
        hipLaunchKernelGGL((k_flash_attn<D, DV, false, PIPE>), grid, dim3(64 * FA_WAVES), 0, stream, a);
    if (a.P > 1)
        hipLaunchKernelGGL((k_flash_attn_reduce<DV>), dim3(a.nq, a.nh, a.nb), dim3(DV < 256 ? DV : 256), 0, stream,
                           a);
}

tlh_status launch_flash_attn(const FlashAttnDesc &d, hipStream_t stream) {
    FaArgs a;
    a.q = (const char *)d.q;
    a.k = (const char *)d.k;
    a.v = (const char *)d.v;
    a.mask = (const char *)d.mask;
    a.dst = (char *)d.dst;
    a.part = (float *)d.scratch;
    a.mask_vec = !((uintptr_t)d.mask & 15) && d.m_nb[1] % 16 == 0 && d.m_nb[2] % 16 == 0 && d.m_nb[3] % 16 == 0;
    a.q_nb1 = d.q_nb[1], a.q_nb2 = d.q_nb[2], a.q_nb3 = d.q_nb[3];
    a.k_nb1 = d.k_nb[1], a.k_nb2 = d.k_nb[2], a.k_nb3 = d.k_nb[3];
    a.v_nb1 = d.v_nb[1], a.v_nb2 = d.v_nb[2], a.v_nb3 = d.v_nb[3];
    a.m_nb1 = d.m_nb[1], a.m_nb2 = d.m_nb[2], a.m_nb3 = d.m_nb[3];
    a.d_nb1 = d.d_nb[1], a.d_nb2 = d.d_nb[2], a.d_nb3 = d.d_nb[3];
    a.m_ne2 = (int)d.m_ne2, a.m_ne3 = (int)d.m_ne3;
    a.nq = (int)d.nq, a.nh = (int)d.nh, a.nb = (int)d.nb, a.L = (int)d.L, a.nhkv = (int)d.nhkv;
    a.rk3 = (int)(d.nb / d.nbk);
    const FaPlan pl = fa_plan(d.nq, d.nh, d.nhkv, d.nb, d.L);
    a.G = pl.G, a.gc = pl.gc, a.qr = pl.qr, a.HC = pl.HC, a.QC = pl.QC, a.P = pl.P, a.part_len = pl.part_len;
    a.scale = d.scale, a.max_bias = d.max_bias, a.m0 = d.m0, a.m1 = d.m1, a.softcap = d.softcap;
    a.nhl2 = d.n_head_log2;
    const bool mask = d.mask != nullptr && d.L > 0;
    // prefill: the 64-row form when it fills the GPU without key partitions and
    // the K / V / dst rows allow 16-byte accesses
    if (d.D == 128 && d.DV == 128 && d.nq >= 32 && d.L > 0) {
        const int gw = pl.G % 4 == 0 ? 4 : pl.G % 2 == 0 ? 2 : 1;
        const int64_t QB = (d.nq + 64 / gw - 1) / (64 / gw), HC = pl.G / gw;
        auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
        bool ok = QB * HC * d.nhkv * d.nb >= 128 && al16(d.q) && al16(d.k) && al16(d.v) && al16(d.dst) &&
                  (!mask || (a.mask_vec && d.L % 8 == 0));
        for (int i = 1; i < 4; ++i)
            ok = ok && d.q_nb[i] % 16 == 0 && d.k_nb[i] % 16 == 0 && d.v_nb[i] % 16 == 0 && d.d_nb[i] % 16 == 0;
        if (ok && QB * HC < 65536) {
            FaRowsArgs ra;
            ra.f = a;
            ra.gw = gw;
            ra.QB = (int)QB;
            const dim3 grid((unsigned)(QB * HC), (unsigned)d.nhkv, (unsigned)d.nb);
            if (mask) hipLaunchKernelGGL(k_flash_attn_rows<true>, grid, dim3(512), 0, stream, ra);
            else hipLaunchKernelGGL(k_flash_attn_rows<false>, grid, dim3(512), 0, stream, ra);
            return check_launch("flash_attn_ext (rows)");
        }
    }
    switch (d.D * 1000 + d.DV) {
    case 32032: launch_fa<32, 32>(a, mask, stream); break;
    case 40040: launch_fa<40, 40>(a, mask, stream); break;
    case 64064: launch_fa<64, 64>(a, mask, stream); break;
    case 72072: launch_fa<72, 72>(a, mask, stream); break;
    case 80080: launch_fa<80, 80>(a, mask, stream); break;
    case 96096: launch_fa<96, 96>(a, mask, stream); break;
    case 112112: launch_fa<112, 112>(a, mask, stream); break;
    case 128128: launch_fa<128, 128>(a, mask, stream); break;
    case 192192: launch_fa<192, 192>(a, mask, stream); break;
    case 192128: launch_fa<192, 128>(a, mask, stream); break;
    case 256256: launch_fa<256, 256>(a, mask, stream); break;
    default:
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: head sizes D=%lld DV=%lld", (long long)d.D,
                         (long long)d.DV);
    }
    return check_launch("flash_attn_ext");
}

}  // namespace tlh

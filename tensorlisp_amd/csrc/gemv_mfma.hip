// Few-column GEMM for GGML_OP_MUL_MAT with 3..16 activation columns, gfx950:
// integer matrix cores (v_mfma_i32_16x16x32_i8) instead of v_dot4.
//
// With more than two columns the dot4 GEMV needs every activation column in
// every lane, so it streams them from LDS, about ten LDS bytes per weight
// byte, and LDS bandwidth, not HBM, sets its speed. An MFMA shares its
// operands across the wave: the 16 x 32 activation operand of one step is
// 8 bytes per lane. Here each wave keeps the activation operands of its own
// slice of K in registers for the whole launch and streams weight row groups
// past them, so activations cost no memory traffic after the first read.
//
// The MFMA is oriented so that each lane's outputs share one weight row:
//   D[i][j] = sum_k A[i][k] * B[k][j],  A = activation codes (i = column,
//   16 columns, the ones past N zero), B = weight codes (j = weight row of a
//   16-row group), k = 32 elements of one block / sub-block.
// Operand lane layout (16x16x32 int8): lane l holds A[l % 16][8g .. 8g+7] and
// B[8g .. 8g+7][l % 16] with g = l / 16; D lane l holds D[4g + r][l % 16],
// r = 0..3. So the weight row's scales, read by the lane that holds its
// codes, are also the scales of that lane's outputs.
//
// Per block the integer sums are exactly those of the CPU's vec_dot
// (ggml-cpu/quants.c): q4_0 / q8_0 blocks of 32 elements are one MFMA each
// (sumi), scaled in f32 as the CPU does (:255, :475); a q4_K super-block is
// eight sub-block MFMAs, each S_s folded into an int32 as sum sc_s * S_s, and
// the min term Mn = sum_s m_s * (sum of q8 in s) is eight more MFMAs whose
// weight operand is m_s broadcast over the sub-block (:696-773).
//
// Work split: a unit is 256 elements (one q4_K super-block or eight q4_0 /
// q8_0 blocks). A launch covers units [u_begin, u_end); wave w of a
// workgroup owns KS of them; the workgroup walks 16-row groups (persistent
// grid), loading the next group's weights while it multiplies this one. The
// waves' 16 x 16 partials meet in LDS and are summed in wave order
// (deterministic). A K longer than one workgroup covers (16 waves x KS
// units) is split into chunks (grid y); each chunk writes its partial sums to
// the scratch and a second kernel adds the chunks in order.
//
// Weight loads (STAGED, K a multiple of 256): the operand layout wants 8
// bytes from each of several places in 16 different rows per instruction, and
// a load instruction costs the address unit about as many cycles as cache
// lines it touches, which made such loads, not HBM, the limit. So a wave
// reads its 16-row x KS-unit slice as consecutive 16-byte pieces per lane
// (each row's slice is contiguous), writes them to a wave-private LDS buffer
// and reads the operand layout back from there. Other K: direct loads.
#include <type_traits>

#include "kernels.hpp"

namespace tlh {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int SK_COLS = 16;
constexpr int SK_MAXW = 16;
constexpr int SK_OUTBUF = 16;  // row groups of outputs held in LDS between stores

__device__ __forceinline__ v4i mfma_i8(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

template <typename T> __device__ __forceinline__ T ldu(const void *p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

// Four nibbles n (one per byte) -> the int8 bytes n - 8 (q4_0 codes):
// (n | 0x80) - 8 stays in 0x78..0x87 without borrows, ^ 0x80 recentres it.
__device__ __forceinline__ uint32_t nib_minus8(uint32_t x) {
    return ((x | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// 4 / 8 bytes at byte offset `off` (2-byte aligned) of a 4-byte aligned LDS
// buffer, by aligned dword reads. (Offsets, not integer-cast pointers, keep
// the accesses in the LDS address space.)
__device__ __forceinline__ uint32_t lds_u32(const uint32_t *base, uint32_t off) {
    const uint32_t *q = base + (off >> 2);
    return __builtin_amdgcn_alignbyte(q[1], q[0], off & 3);
}
__device__ __forceinline__ uint2 lds_u64(const uint32_t *base, uint32_t off) {
    const uint32_t *q = base + (off >> 2);
    const uint32_t sh = off & 3;
    const uint32_t a0 = q[0], a1 = q[1], a2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(a1, a0, sh), __builtin_amdgcn_alignbyte(a2, a1, sh));
}

// Bytes of one row per unit (the stride between units).
template <int WT> constexpr int unit_bytes() { return kquant_type(WT) ? block_bytes(WT) : 8 * block_bytes(WT); }
// 32-element block types whose codes are nibbles (q5: plus a fifth bit):
// a lane's weight bytes 4g..4g+3 hold elements 4g.. (low) and 16 + 4g.. (high)
template <int WT> constexpr bool nibble_type() { return WT == TLH_TYPE_Q4_0 || legacy_type(WT); }
// Bytes of a unit staged through LDS (a multiple of 16): all of it, but for
// q6_K its first 208 (ql, qh, scales; d, the last 2 bytes, is loaded apart),
// q2_K its first 80 (scales, qs; d and dmin loaded apart) and q3_K its first
// 96 (hmask, qs; the 12 scale bytes and d loaded apart).
template <int WT> constexpr int staged_bytes() {
    return WT == TLH_TYPE_Q6_K ? 208 : WT == TLH_TYPE_Q2_K ? 80 : WT == TLH_TYPE_Q3_K ? 96 : unit_bytes<WT>();
}
// Types with bytes loaded beside the staged ones (one unit per wave).
template <int WT> constexpr bool staged_extra() {
    return WT == TLH_TYPE_Q6_K || WT == TLH_TYPE_Q2_K || WT == TLH_TYPE_Q3_K;
}
// Types whose unit is one k-quant super-block (one activation scale slot).
template <int WT> constexpr bool kquant() { return kquant_type(WT); }

// One lane's weight data of one unit in operand form: q4_K the super-block
// header and bytes 8g..8g+7 of each 32-byte chunk; q8_0 / q4_0 per block the
// scale and codes 8g..8g+7 / nibble bytes 4g..4g+3.
template <int WT> struct UnitW;

template <> struct UnitW<TLH_TYPE_Q4_K> {
    uint4 hdr;
    uint2 q[4];
    // blk: the unit's 144 bytes; global (unaligned) or LDS (16-byte aligned)
    __device__ __forceinline__ void load(const uint8_t *blk, int g) {
        hdr = ldu<uint4>(blk);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = ldu<uint2>(blk + 16 + 32 * c + 8 * g);
    }
    __device__ __forceinline__ void load_lds(const uint8_t *blk, int g) {
        hdr = *(const uint4 *)blk;
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *(const uint2 *)(blk + 16 + 32 * c + 8 * g);
    }
};

// q5_K: q4_K's header and lane bytes (nibbles at 48 + 32c + 8g) plus qh bytes
// 16 + 8g, whose bit j is the fifth bit of those elements in sub-block j.
template <> struct UnitW<TLH_TYPE_Q5_K> {
    uint4 hdr;
    uint2 q[4];
    uint2 qh;
    __device__ __forceinline__ void load(const uint8_t *blk, int g) {
        hdr = ldu<uint4>(blk);
        qh = ldu<uint2>(blk + 16 + 8 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = ldu<uint2>(blk + 48 + 32 * c + 8 * g);
    }
    __device__ __forceinline__ void load_lds(const uint8_t *blk, int g) {
        hdr = *(const uint4 *)blk;
        qh = *(const uint2 *)(blk + 16 + 8 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *(const uint2 *)(blk + 48 + 32 * c + 8 * g);
    }
};

// q6_K from the staged LDS copy: lane g's operand bytes of 32-element step m
// (elements 32m + 8g..+7; half h = m / 4, m' = m % 4, e = 32m' + 8g) are the
// 8 ql bytes at 64h + 32 (m' & 1) + 8g (low nibbles for m' < 2, else high)
// and the 8 qh bytes at 128 + 32h + 8g (2-bit fields 2m'); all 16 scales.
template <> struct UnitW<TLH_TYPE_Q6_K> {
    uint2 ql[4];  // [2h + (m' & 1)]
    uint2 qh[2];  // [h]
    uint4 sc;
    __device__ __forceinline__ void load_lds(const uint8_t *blk, int g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ql[i] = *(const uint2 *)(blk + 32 * i + 8 * g);
#pragma unroll
        for (int h = 0; h < 2; ++h) qh[h] = *(const uint2 *)(blk + 128 + 32 * h + 8 * g);
        sc = *(const uint4 *)(blk + 192);
    }
};

// q2_K / q3_K from the staged LDS copy: lane g's operand bytes of step m
// (elements 32m + 8g..+7; half h = m / 4, run j = m % 4, l = 8g..8g+7) are
// the half's qs bytes l (2-bit fields 2j) at 16 + 32h + 8g (q2_K, after the
// 16 scale bytes) or 32 + 32h + 8g (q3_K, after the 32 hmask bytes); q3_K
// adds hmask bytes 8g..8g+7 (bit 4h + j); q2_K keeps all 16 scale bytes.
template <> struct UnitW<TLH_TYPE_Q2_K> {
    uint2 q[2];  // [h]
    uint4 sc;
    __device__ __forceinline__ void load_lds(const uint8_t *blk, int g) {
#pragma unroll
        for (int h = 0; h < 2; ++h) q[h] = *(const uint2 *)(blk + 16 + 32 * h + 8 * g);
        sc = *(const uint4 *)blk;
    }
};
template <> struct UnitW<TLH_TYPE_Q3_K> {
    uint2 q[2];  // [h]
    uint2 hm;
    __device__ __forceinline__ void load_lds(const uint8_t *blk, int g) {
#pragma unroll
        for (int h = 0; h < 2; ++h) q[h] = *(const uint2 *)(blk + 32 + 32 * h + 8 * g);
        hm = *(const uint2 *)(blk + 8 * g);
    }
};

// blk0: the unit's first block; the `nb` valid blocks of the unit are read
// (blocks past them reread the last valid one: a row's last unit may end
// early, and its bytes past the row are not the row's)
template <> struct UnitW<TLH_TYPE_Q8_0> {
    uint2 q[8];
    uint16_t d[8];
    __device__ __forceinline__ void load(const uint8_t *blk0, int g, int nb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint8_t *b = blk0 + (j < nb ? j : nb - 1) * Q8_0_BYTES;
            d[j] = ldu<uint16_t>(b);
            q[j] = ldu<uint2>(b + 2 + 8 * g);
        }
    }
};

// q4_1 / q5_0 / q5_1: per block the f16 d (and m) word, the fifth bits and
// nibble bytes 4g..4g+3
template <int WT> struct UnitWLegacy {
    uint32_t q[8], dm[8], qh[8];
    __device__ __forceinline__ void load(const uint8_t *blk0, int g, int nb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint8_t *b = blk0 + (j < nb ? j : nb - 1) * block_bytes(WT);
            dm[j] = ldu<uint32_t>(b);
            qh[j] = has_qh(WT) ? ldu<uint32_t>(b + blk_qh_off(WT)) : 0u;
            q[j] = ldu<uint32_t>(b + blk_qs_off(WT) + 4 * g);
        }
    }
};
template <> struct UnitW<TLH_TYPE_Q4_1> : UnitWLegacy<TLH_TYPE_Q4_1> {};
template <> struct UnitW<TLH_TYPE_Q5_0> : UnitWLegacy<TLH_TYPE_Q5_0> {};
template <> struct UnitW<TLH_TYPE_Q5_1> : UnitWLegacy<TLH_TYPE_Q5_1> {};

// The weight operand of one q4_1 / q5_0 / q5_1 block for lane group g from its
// nibble bytes 4g..4g+3 (v) and qh: codes as int8 (q5_0: q - 16, no borrows
// with the byte-wise bias trick)
template <int WT> __device__ __forceinline__ long legacy_B(uint32_t v, uint32_t qh, int g) {
    uint32_t lo = v & 0x0f0f0f0fu, hi = (v >> 4) & 0x0f0f0f0fu;
    if constexpr (has_qh(WT)) {
        lo |= spread4((qh >> (4 * g)) & 0xfu);
        hi |= spread4((qh >> (16 + 4 * g)) & 0xfu);
    }
    if constexpr (WT == TLH_TYPE_Q5_0) {
        lo = ((lo | 0x80808080u) - 0x10101010u) ^ 0x80808080u;
        hi = ((hi | 0x80808080u) - 0x10101010u) ^ 0x80808080u;
    }
    return pack2(lo, hi);
}

// One q4_1 / q5_0 / q5_1 block: y[r] += (d * d8) * sumi (+ m * s8), the CPU's
// per-block step (ggml-cpu/quants.c:262-296, :365-449); dm: the block's f16 d
// (and m) word; sdb / ssb: the block's activation d8 / s8 [16 columns].
template <int WT>
__device__ __forceinline__ void block_mma_legacy(long A, long B, uint32_t dm, const float *sdb, const float *ssb,
                                                 int g, float (&y)[4]) {
#pragma clang fp contract(off)
    const v4i zero = {0, 0, 0, 0};
    const v4i Sb = mfma_i8(A, B, zero);
    const float dw = h2f((uint16_t)(dm & 0xffff));
    const float4 d8 = *(const float4 *)(sdb + 4 * g);
    const float d8r[4] = {d8.x, d8.y, d8.z, d8.w};
    if constexpr (has_min(WT)) {
        const float mw = h2f((uint16_t)(dm >> 16));
        const float4 s8 = *(const float4 *)(ssb + 4 * g);
        const float s8r[4] = {s8.x, s8.y, s8.z, s8.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] += (dw * d8r[r]) * (float)Sb[r] + mw * s8r[r];
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] += (dw * d8r[r]) * (float)Sb[r];
    }
}

template <> struct UnitW<TLH_TYPE_Q4_0> {
    uint32_t q[8];
    uint16_t d[8];
    __device__ __forceinline__ void load(const uint8_t *blk0, int g, int nb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint8_t *b = blk0 + (j < nb ? j : nb - 1) * Q4_0_BYTES;
            d[j] = ldu<uint16_t>(b);
            q[j] = ldu<uint32_t>(b + 2 + 4 * g);
        }
    }
};

// One q4_0 / q8_0 block: y[r] += its integer dot product (one MFMA) scaled
// as the CPU scales it; sdb: the block's activation scales [16 columns].
template <int WT>
__device__ __forceinline__ void block_mma(long A, long B, uint16_t dwh, const float *sdb, int g, float (&y)[4]) {
    const v4i zero = {0, 0, 0, 0};
    const v4i Sb = mfma_i8(A, B, zero);
    const float dw = h2f(dwh);
    const float4 d8 = *(const float4 *)(sdb + 4 * g);
    const float d8r[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if constexpr (WT == TLH_TYPE_Q4_0)
            y[r] += ((float)Sb[r] * dw) * d8r[r];  // quants.c:255
        else
            y[r] += (float)Sb[r] * (dw * d8r[r]);  // quants.c:475
    }
}

// q6_K super-block (vec_dot_q6_K_q8_K_generic, ggml-cpu/quants.c:851-904):
// 16 sub-blocks of 16 with int8 scales. A 32-element MFMA step holds two
// sub-blocks (lanes g < 2 the first, g >= 2 the second), so each step runs
// twice with the other sub-block's lanes of the weight operand zeroed; codes
// are (ql | qh << 4) - 32 as signed bytes. S = sum scale_s * S_s in int32,
// scaled by d * d8 in f32 (the CPU splits the int32 sums in 8 lanes before its
// f32 products; the difference is f32 rounding). dq: the unit's f16 d.
__device__ __forceinline__ void unit_mma_q6k(const UnitW<TLH_TYPE_Q6_K> &w, uint32_t dq, const long (&A)[8],
                                             const float *sdu, int g, float (&y)[4]) {
    const v4i zero = {0, 0, 0, 0};
    v4i S = {0, 0, 0, 0};
    const uint32_t scw[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int h = m >> 2, mp = m & 3;
        const uint2 l = w.ql[2 * h + (mp & 1)], hq = w.qh[h];
        const int nsh = mp >= 2 ? 4 : 0, hsh = 2 * mp;
        uint32_t b[2];
        const uint32_t lv[2] = {l.x, l.y}, hv[2] = {hq.x, hq.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t u = ((lv[i] >> nsh) & 0x0f0f0f0fu) | (((hv[i] >> hsh) & 0x03030303u) << 4);
            b[i] = ((u | 0x80808080u) - 0x20202020u) ^ 0x80808080u;  // u - 32 per byte, no borrows
        }
        const long B = pack2(b[0], b[1]);
        const v4i S0 = mfma_i8(A[m], g < 2 ? B : 0, zero);   // sub-block 2m
        const v4i S1 = mfma_i8(A[m], g >= 2 ? B : 0, zero);  // sub-block 2m + 1
        const uint32_t sw = scw[m >> 1];
        const int s0 = (int)(int8_t)((sw >> (16 * (m & 1))) & 0xff);
        const int s1 = (int)(int8_t)((sw >> (16 * (m & 1) + 8)) & 0xff);
#pragma unroll
        for (int r = 0; r < 4; ++r) S[r] += __mul24(s0, S0[r]) + __mul24(s1, S1[r]);  // |S_s| < 2^16
    }
    const float d = h2f((uint16_t)dq);
    const float4 d8 = *(const float4 *)(sdu + 4 * g);
    const float dy[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] += (d * dy[r]) * (float)S[r];
}

// q2_K super-block (vec_dot_q2_K_q8_K_generic, ggml-cpu/quants.c:565-615):
// 16 sub-blocks of 16, scale (low nibble) and min (high nibble) per
// sub-block. Each 32-element step runs twice with the other sub-block's lanes
// of the weight operand zeroed (as q6_K); S = sum scale_s * S_s in int32, and
// the min term Mn = sum_s min_s * (sum of q8 in s) is one more MFMA per step
// whose weight operand is min_{2m} on lanes g < 2 and min_{2m+1} on g >= 2.
// dm: the unit's f16 d (low half) and dmin (high half).
__device__ __forceinline__ void unit_mma_q2k(const UnitW<TLH_TYPE_Q2_K> &w, uint32_t dm, const long (&A)[8],
                                             const float *sdu, int g, float (&y)[4]) {
    const v4i zero = {0, 0, 0, 0};
    v4i S = {0, 0, 0, 0}, Mn = {0, 0, 0, 0};
    const uint32_t scw[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const uint2 qv = w.q[m >> 2];
        const int sh = 2 * (m & 3);
        const long B = pack2((qv.x >> sh) & 0x03030303u, (qv.y >> sh) & 0x03030303u);
        const v4i S0 = mfma_i8(A[m], g < 2 ? B : 0, zero);   // sub-block 2m
        const v4i S1 = mfma_i8(A[m], g >= 2 ? B : 0, zero);  // sub-block 2m + 1
        const uint32_t b2 = (scw[m >> 1] >> (16 * (m & 1))) & 0xffffu;  // scale bytes 2m, 2m + 1
        const int s0 = (int)(b2 & 15), s1 = (int)((b2 >> 8) & 15);
        const uint32_t mn = g < 2 ? (b2 >> 4) & 15 : (b2 >> 12) & 15;
        const uint32_t m4 = mn * 0x01010101u;
        Mn = mfma_i8(A[m], pack2(m4, m4), Mn);
#pragma unroll
        for (int r = 0; r < 4; ++r) S[r] += __mul24(s0, S0[r]) + __mul24(s1, S1[r]);  // |S_s| < 2^13
    }
    const float d = h2f((uint16_t)(dm & 0xffff)), dmin = h2f((uint16_t)(dm >> 16));
    const float4 d8 = *(const float4 *)(sdu + 4 * g);
    const float dy[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] += (d * dy[r]) * (float)S[r] - (dmin * dy[r]) * (float)Mn[r];
}

// q3_K super-block (vec_dot_q3_K_q8_K_generic, ggml-cpu/quants.c:617-694):
// codes (low 2 bits | third bit << 2) - 4 as signed bytes, steps as q2_K's;
// the 16 6-bit scales (minus 32) unpacked into four words of bytes: low 4
// bits from scale bytes 0..7 (low nibbles: sub-blocks 0..7, high: 8..15),
// high 2 bits of sub-block 4q + k from byte 8 + k at bit 2q. S = sum scale_s
// * S_s in int32, scaled by d * d8. ex: block bytes 94..109 (scale bytes at
// 2..13, d at 14..15).
__device__ __forceinline__ void unit_mma_q3k(const UnitW<TLH_TYPE_Q3_K> &w, uint4 ex, const long (&A)[8],
                                             const float *sdu, int g, float (&y)[4]) {
    const v4i zero = {0, 0, 0, 0};
    v4i S = {0, 0, 0, 0};
    const uint32_t b0 = (ex.x >> 16) | (ex.y << 16), b1 = (ex.y >> 16) | (ex.z << 16);
    const uint32_t b2 = (ex.z >> 16) | (ex.w << 16);
    const uint32_t lo[4] = {b0 & 0x0f0f0f0fu, b1 & 0x0f0f0f0fu, (b0 >> 4) & 0x0f0f0f0fu, (b1 >> 4) & 0x0f0f0f0fu};
    uint32_t scw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) scw[q] = lo[q] | (((b2 >> (2 * q)) & 0x03030303u) << 4);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int h = m >> 2, j = m & 3;
        const uint2 qv = w.q[h];
        const uint32_t hv[2] = {w.hm.x, w.hm.y}, lv[2] = {qv.x, qv.y};
        uint32_t b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t u = ((lv[i] >> (2 * j)) & 0x03030303u) | (((hv[i] >> (4 * h + j)) & 0x01010101u) << 2);
            b[i] = ((u | 0x80808080u) - 0x04040404u) ^ 0x80808080u;  // u - 4 per byte, no borrows
        }
        const long B = pack2(b[0], b[1]);
        const v4i S0 = mfma_i8(A[m], g < 2 ? B : 0, zero);   // sub-block 2m
        const v4i S1 = mfma_i8(A[m], g >= 2 ? B : 0, zero);  // sub-block 2m + 1
        const uint32_t sw = (scw[m >> 1] >> (16 * (m & 1))) & 0xffffu;
        const int s0 = (int)(sw & 0xff) - 32, s1 = (int)(sw >> 8) - 32;
#pragma unroll
        for (int r = 0; r < 4; ++r) S[r] += __mul24(s0, S0[r]) + __mul24(s1, S1[r]);  // |S_s| < 2^13
    }
    const float d = h2f((uint16_t)(ex.w >> 16));
    const float4 d8 = *(const float4 *)(sdu + 4 * g);
    const float dy[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] += (d * dy[r]) * (float)S[r];
}

// y[r] += the unit's contribution to output (column 4g + r, the lane's weight
// row). A: the unit's activation operands; sdu: its activation scales in LDS
// (q4_K one slot, q4_0 / q8_0 one per block) as [slot][16 columns];
// nvalid: blocks of the unit inside K (q4_0 / q8_0).
template <int WT>
__device__ __forceinline__ void unit_mma(const UnitW<WT> &w, const long (&A)[8], const float *sdu, const float *ssu,
                                         int g, int nvalid, float (&y)[4]) {
    const v4i zero = {0, 0, 0, 0};
    if constexpr (WT == TLH_TYPE_Q4_K || WT == TLH_TYPE_Q5_K) {
        const uint4 h = w.hdr;
        // the 6-bit scales / mins of the 8 sub-blocks as bytes, sub-blocks
        // 0..3 and 4..7 (get_scale_min_k4, ggml-quants.c:880-887)
        const uint32_t sc[2] = {h.y & 0x3f3f3f3fu, (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {h.z & 0x3f3f3f3fu, ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u)};
        v4i S = {0, 0, 0, 0}, Mn = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint2 qv = w.q[j >> 1];
            const int sh = (j & 1) ? 4 : 0;
            uint32_t b0 = (qv.x >> sh) & 0x0f0f0f0fu, b1 = (qv.y >> sh) & 0x0f0f0f0fu;
            if constexpr (WT == TLH_TYPE_Q5_K) {
                b0 |= ((w.qh.x >> j) & 0x01010101u) << 4;
                b1 |= ((w.qh.y >> j) & 0x01010101u) << 4;
            }
            const long B = pack2(b0, b1);
            const v4i Sj = mfma_i8(A[j], B, zero);
            const int s = (int)__builtin_amdgcn_ubfe(sc[j >> 2], 8 * (j & 3), 8);
            // m_j in all four bytes (byte j & 3 of the word, selected four times)
            const uint32_t m4 = __builtin_amdgcn_perm(0u, mn[j >> 2], 0x01010101u * (uint32_t)(j & 3));
            Mn = mfma_i8(A[j], pack2(m4, m4), Mn);
#pragma unroll
            for (int r = 0; r < 4; ++r) S[r] += __mul24(s, Sj[r]);  // |Sj| < 2^16, s < 64
        }
        const float d = h2f((uint16_t)(h.x & 0xffff)), dmin = h2f((uint16_t)(h.x >> 16));
        const float4 d8 = *(const float4 *)(sdu + 4 * g);
        const float dy[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] += (d * dy[r]) * (float)S[r] - (dmin * dy[r]) * (float)Mn[r];
    } else if constexpr (legacy_type(WT)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j >= nvalid) continue;  // wave-uniform
            block_mma_legacy<WT>(A[j], legacy_B<WT>(w.q[j], w.qh[j], g), w.dm[j], sdu + j * SK_COLS,
                                 ssu + j * SK_COLS, g, y);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j >= nvalid) continue;  // wave-uniform
            long B;
            if constexpr (WT == TLH_TYPE_Q4_0) {
                const uint32_t v = w.q[j];
                B = pack2(nib_minus8(v & 0x0f0f0f0fu), nib_minus8((v >> 4) & 0x0f0f0f0fu));
            } else {
                B = pack2(w.q[j].x, w.q[j].y);
            }
            block_mma<WT>(A[j], B, w.d[j], sdu + j * SK_COLS, g, y);
        }
    }
}

// Staging of one row group's slice: lane l loads pieces 64i + l (16 bytes
// each) of the 16 rows x KS units, row-major; NL loads per lane.
template <int WT> struct StageExtra { using T = uint32_t; };
template <> struct StageExtra<TLH_TYPE_Q3_K> { using T = uint4; };
template <int WT, int KS> struct Stage {
    static constexpr int RB = KS * staged_bytes<WT>();  // slice bytes per row (a multiple of 16)
    static constexpr int PR = RB / 16;                   // pieces per row
    static constexpr int NL = (16 * PR + 63) / 64;
    static constexpr int BUF = NL * 64 * 16 + 16;        // LDS bytes per wave (with read slack)
    uint4 v[NL];
    // the lane's row's bytes loaded beside the staged ones (KS = 1): q6_K its
    // d, q2_K d and dmin, q3_K the 12 scale bytes and d (block bytes 94..109)
    using ExtraT = typename StageExtra<WT>::T;
    ExtraT dq;
};

// Direct loads of KS units (prefetch set of the unstaged kernel, 32-element
// block types). Units past `last` reread unit `last` (their products are
// skipped); a unit reads only its blocks below `nblk`.
template <int WT, int KS> struct DirectW {
    UnitW<WT> u[KS];
    __device__ __forceinline__ void load(const uint8_t *row, int64_t u0, int64_t last, int64_t nblk, int g) {
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            const int64_t uu = u0 + t < last ? u0 + t : last;
            const int64_t nb = nblk - 8 * uu;
            u[t].load(row + uu * unit_bytes<WT>(), g, (int)(nb < 8 ? nb : 8));
        }
    }
};

// No store epilogue (the kernel argument of the plain launches).
struct NoEpi {
    int unused;
};
// Rotated pairs per head in the epilogue's (cos, sin) table (0: none read).
__host__ __device__ inline int epi_table_pairs(const NoEpi &) { return 0; }
__host__ __device__ inline int epi_table_pairs(const GemvEpi &e) {
    return e.rt_mode == 2 && (e.rope[0] | e.rope[1] | e.rope[2]) ? (int)(e.rp.n_dims < e.ne0 ? e.rp.n_dims : e.ne0) / 2 : 0;
}

// EP = GemvEpi: the outputs of segment s go out through ep.layout[s] at the
// flush instead of seg_dst[s] (one K chunk, segments): the ROPE (mode 0, the
// pair's other row is the neighbouring output of the same column), f16 cast,
// cache-row or paged K / V write that follow a batched Q / K / V projection,
// column n being token n (its position ep.pos[n], its row or slot ep.idx[s][n]).
// Paired blocks (N <= 8). With at most 8 columns, half of a 16 x 16 output is
// zero columns, yet every output takes the per-block f32 scaling. Instead
// v_mfma_i32_16x16x64_i8 takes two 32-element blocks (q4_0 / q8_0) or
// sub-blocks (q4_K / q5_K) 2p and 2p + 1 at once: lane group g carries 16
// bytes of one block (groups 0, 1: block 2p, elements 16g..; groups 2, 3:
// block 2p + 1, elements 16 (g - 2)..); the activation operand is block
// diagonal -- lane (g, i) holds column i & 7's codes where i < 8 matches
// g < 2, zeros elsewhere -- so output row i < 8 is column i's sum over block
// 2p and row i >= 8 column i - 8's over block 2p + 1. A lane (g, j) then holds
// weight row j's sums of columns 4 (g & 1) .. + 3 for one block, every output
// useful: half the MFMAs and half the scaling per block of the unpaired form.
// Both parities' partial sums of an output meet once per row group (lanes l
// and l + 32). Within a parity the blocks are added in K order, so the f32
// order of the block sums differs from the CPU's sequential loop (even and
// odd blocks summed apart, then added).
template <int WT> constexpr bool pair_type() {
    return WT == TLH_TYPE_Q4_0 || WT == TLH_TYPE_Q8_0 || WT == TLH_TYPE_Q4_K || WT == TLH_TYPE_Q5_K;
}
__device__ __forceinline__ v4i mfma_i8_k64(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// One unit (256 elements) of a paired row group from the wave's staged LDS
// copy at byte ub (the lane's weight row); A: the unit's four block-pair
// activation operands; sdu: the unit's activation scales [slot][16 columns].
// (Tried for q4_0: the nibbles as they are and 8 * the blocks' activation
// code sums subtracted from the integer sums, which saves the bias trick's
// three VALU operations per word but adds an LDS read per block: slower.)
template <int WT>
__device__ __forceinline__ void unit_mma_pair(const uint8_t *wbuf, uint32_t ub, const v4i (&A)[4], const float *sdu,
                                              int g, float (&y)[4]) {
    const int par = g >> 1, half = g & 1;  // block parity, 16-element half of the block
    const v4i zero = {0, 0, 0, 0};
    const uint32_t *w32 = (const uint32_t *)wbuf;
    if constexpr (WT == TLH_TYPE_Q4_K || WT == TLH_TYPE_Q5_K) {
        constexpr bool Q5 = WT == TLH_TYPE_Q5_K;
        const uint4 h = *(const uint4 *)(wbuf + ub);
        // the 6-bit scales / mins of sub-blocks 0..3 and 4..7 as bytes (get_scale_min_k4)
        const uint32_t sc[2] = {h.y & 0x3f3f3f3fu, (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {h.z & 0x3f3f3f3fu, ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u)};
        uint4 qh = {0, 0, 0, 0};
        if constexpr (Q5) qh = *(const uint4 *)(wbuf + ub + 16 + 16 * half);
        v4i S = zero, Mn = zero;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int s = 2 * p + par;  // this lane's sub-block
            const uint4 q = *(const uint4 *)(wbuf + ub + (Q5 ? 48 : 16) + 32 * p + 16 * half);
            const uint32_t qv[4] = {q.x, q.y, q.z, q.w}, hv[4] = {qh.x, qh.y, qh.z, qh.w};
            v4i B;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t c = (qv[i] >> (4 * par)) & 0x0f0f0f0fu;
                if constexpr (Q5) c |= ((hv[i] >> s) & 0x01010101u) << 4;
                B[i] = (int)c;
            }
            const v4i Sp = mfma_i8_k64(A[p], B, zero);
            const int scv = (int)__builtin_amdgcn_ubfe(sc[s >> 2], 8 * (s & 3), 8);
            const uint32_t m4 = __builtin_amdgcn_perm(0u, mn[s >> 2], 0x01010101u * (uint32_t)(s & 3));
            const v4i Bm = {(int)m4, (int)m4, (int)m4, (int)m4};
            Mn = mfma_i8_k64(A[p], Bm, Mn);
#pragma unroll
            for (int r = 0; r < 4; ++r) S[r] += __mul24(scv, Sp[r]);  // |Sp| < 2^16, sc < 64
        }
        const float d = h2f((uint16_t)(h.x & 0xffff)), dmin = h2f((uint16_t)(h.x >> 16));
        const float4 d8 = *(const float4 *)(sdu + 4 * half);
        const float dy[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] += (d * dy[r]) * (float)S[r] - (dmin * dy[r]) * (float)Mn[r];
    } else {
        constexpr int BB = block_bytes(WT);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t blk = ub + (2 * p + par) * BB;  // the lane's block (2-byte aligned)
            v4i B;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (WT == TLH_TYPE_Q4_0) {  // low nibbles: elements 0..15, high: 16..31
                    const uint32_t v = lds_u32(w32, blk + 2 + 4 * i);
                    B[i] = (int)nib_minus8((v >> (4 * half)) & 0x0f0f0f0fu);
                } else {
                    B[i] = (int)lds_u32(w32, blk + 2 + 16 * half + 4 * i);
                }
            }
            const v4i Sb = mfma_i8_k64(A[p], B, zero);
            const float dw = h2f((uint16_t)lds_u32(w32, blk));
            const float4 d8 = *(const float4 *)(sdu + (2 * p + par) * SK_COLS + 4 * half);
            const float d8r[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (WT == TLH_TYPE_Q4_0)
                    y[r] += ((float)Sb[r] * dw) * d8r[r];  // quants.c:255
                else
                    y[r] += (float)Sb[r] * (dw * d8r[r]);  // quants.c:475
            }
        }
    }
}

// PAIR (N <= 8, whole units, q4_0 / q8_0 / q4_K / q5_K): block pairs per
// v_mfma_i32_16x16x64_i8 as in k_gemv_cols below (unit_mma_pair); the A
// registers then hold the unit's four block-pair operands.
template <int WT, int KS, bool STAGED, typename EP = NoEpi, bool PAIR = false>
__global__ void __launch_bounds__(1024) k_gemv_mfma(const MatmulArgs a, int64_t share, const EP ep) {
    kernarg_prefetch<kernarg_lines(sizeof(MatmulArgs) + 8 + sizeof(EP))>();
    constexpr bool EPI = !std::is_same<EP, NoEpi>::value;
    extern __shared__ __attribute__((aligned(16))) char sk_lds[];
    constexpr int AT = vec_dot_type(WT);
    constexpr bool KQ = kquant<WT>();
    constexpr int UB = unit_bytes<WT>();
    static_assert(!staged_extra<WT>() || KS == 1, "q6_K / q2_K / q3_K staging keeps one unit's extra bytes per lane");
    using St = Stage<WT, KS>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int g = lane >> 4, wr = lane & 15;  // k group; weight row in the group / activation column
    const int64_t K = a.K;
    const int64_t nblk = K / block_elems(AT);  // activation blocks per row (q8_K: super-blocks)
    // K chunk blockIdx.y: units [u_begin, u_end)
    const int64_t units_all = (K + 255) / 256;
    const int64_t u_begin = (int64_t)blockIdx.y * share;
    const int64_t u_end = u_begin + share < units_all ? u_begin + share : units_all;
    const int64_t u0 = u_begin + (int64_t)wave * KS;
    // scale slots of the launch: q4_K one per unit, q4_0 / q8_0 one per block
    const int64_t s_begin = KQ ? u_begin : 8 * u_begin;
    const int64_t s_end = KQ ? u_end : (8 * u_end < nblk ? 8 * u_end : nblk);
    const int64_t batch = blockIdx.z;
    const MmSlice sl = mm_slice(a, blockIdx.z);
    const int64_t i12 = sl.i12, i13 = sl.i13;
    const uint8_t *W = sl.w;
    int64_t arow0 = a.n0 + a.N_total * batch;
    bool bad_id = false;  // MUL_MAT_ID: an expert id out of range (outputs NaN, loads stay in bounds)
    if (a.ids) {
        const int32_t ex = *(const int32_t *)(a.ids + i12 * a.ids_nb0 + i13 * a.ids_nb1);
        bad_id = ex < 0 || ex >= a.id_nas;
        W = a.w + (bad_id ? 0 : (int64_t)ex) * a.w_nb2;
        arow0 = i12 % a.id_b1 + a.id_b1 * i13;
    }
    const ActView act = act_view(a.act, AT, K, mm_act_rows(a));
    const int N = (int)a.N;

    // LDS: partials [2][nw][64] float4, the activation scales of the
    // launch's scale slots [s_end - s_begin][16 columns], the outputs of up
    // to SK_OUTBUF row groups [SK_OUTBUF][256], then (STAGED) one weight
    // buffer per wave.
    // q8_1 activations (q4_1 / q5_1) add their s values, as many slots again
    constexpr bool S8 = AT == TLH_TYPE_Q8_1;
    float4 *red = (float4 *)sk_lds;
    float *sd = (float *)(sk_lds + 2 * nw * 64 * sizeof(float4));
    float *ss = sd + (s_end - s_begin) * SK_COLS;
    float *obuf = ss + (S8 ? (s_end - s_begin) * SK_COLS : 0);
    uint8_t *wbuf = (uint8_t *)(obuf + SK_OUTBUF * 256) + (size_t)wave * St::BUF;
    // EPI reading the (cos, sin) table: its columns' entries, after the weight buffers
    const int tpairs = epi_table_pairs(ep);
    float2 *s_rt = (float2 *)((uint8_t *)(obuf + SK_OUTBUF * 256) + (size_t)nw * (STAGED ? St::BUF : 0));

    const int64_t groups = (a.M + 15) / 16;
    int64_t rg = blockIdx.x;
    const int64_t row_bytes = K / block_elems(WT) * block_bytes(WT);

    // STAGED: piece i of this lane is row pr[i] = p / PR of the group at byte
    // u0 * UB + 16 * (p % PR) of the row (p = 64i + lane; offsets past the row
    // end, of units past K, are clamped to the row start). pofs[i]: that
    // piece's byte offset from the group's first row; rows past M read row M-1.
    int pr[St::NL];
    int64_t pofs[St::NL];
#pragma unroll
    for (int i = 0; i < St::NL; ++i) {
        const int p = 64 * i + lane;
        const int pc = p < 16 * St::PR ? p : 0;
        pr[i] = pc / St::PR;
        const int64_t off = u0 * UB + 16 * (pc - pr[i] * St::PR);  // (KS = 1 for the staged q6_K bytes)
        pofs[i] = pr[i] * a.w_nb1 + (off + 16 <= row_bytes ? off : 0);
    }
    // segments (a.nseg > 0): row m of the launch is row m - seg_m0[s] of
    // matrix s; a 16-row group never straddles two
    auto seg_of = [&](int64_t m) { return (int)(m >= a.seg_m0[1]) + (int)(a.nseg > 2 && m >= a.seg_m0[2]); };
    auto row_base = [&](int64_t m) {
        if (a.nseg > 0) {
            const int sg = seg_of(m);
            return a.seg_w[sg] + (m - a.seg_m0[sg]) * a.w_nb1;
        }
        return W + m * a.w_nb1;
    };
    const uint8_t *wlast = row_base(a.M - 1);
    auto wrow_of = [&](int64_t grp) {
        const int64_t m = grp * 16 + wr < a.M ? grp * 16 + wr : a.M - 1;  // clamp: loads in bounds
        return row_base(m);
    };
    auto stage_load = [&](St &s, int64_t grp) {
        const uint8_t *gb = row_base(grp * 16);  // wave-uniform
        const int rows_left = (int)(a.M - grp * 16);
#pragma unroll
        for (int i = 0; i < St::NL; ++i) {
            const uint8_t *q = pr[i] < rows_left ? gb + pofs[i] : wlast + (pofs[i] - pr[i] * a.w_nb1);
            s.v[i] = ldu<uint4>(q);
        }
        if constexpr (staged_extra<WT>()) {
            const int64_t ud = u0 < u_end ? u0 : u_begin;  // a unit of the row (products past u_end are skipped)
            const uint8_t *ub = wrow_of(grp) + ud * UB;
            if constexpr (WT == TLH_TYPE_Q6_K) s.dq = ldu<uint16_t>(ub + 208);
            else if constexpr (WT == TLH_TYPE_Q2_K) s.dq = ldu<uint32_t>(ub + 80);
            else s.dq = ldu<uint4>(ub + 94);
        }
    };

    // the first row group's weights go out before the activations are read
    St st;
    DirectW<WT, KS> da, db;
    const int64_t rg0 = rg < groups ? rg : groups - 1;
    if constexpr (STAGED) stage_load(st, rg0);
    else da.load(wrow_of(rg0), u0, (s_end - 1) / (KQ ? 1 : 8), s_end, g);
    // EPI: the flush's column (token) values, read now so that no load waits at
    // the end of the kernel: its position and, per segment, its row or slot
    // (raw words: i64 as two, i32 read twice)
    float e_pos = 0.0f;
    int32_t e_lo[3] = {0, 0, 0}, e_hi[3] = {0, 0, 0};
    // and the rotation table's entries (at most RT_PER per thread), written to LDS before the first barrier
    constexpr int RT_PER = 4;
    float2 rt_v[EPI ? RT_PER : 1];
    if constexpr (EPI) {
        if (tpairs) {  // uniform; the loads are unconditional (clamped), so no wait where a branch rejoins
            const int last = N * tpairs - 1;
#pragma unroll
            for (int k = 0; k < RT_PER; ++k) {
                const int i = threadIdx.x + k * (int)blockDim.x;
                rt_v[k] = ((const float2 *)ep.rt)[(int64_t)a.n0 * tpairs + (i < last ? i : last)];
            }
        }
        const int ec = threadIdx.x >> 4;  // the flush's column of this thread
        const int64_t en = a.n0 + (ec < N ? ec : 0);
        if (ep.pos) e_pos = (float)ep.pos[en];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (ep.idx[k]) {
                const int32_t *ip = (const int32_t *)ep.idx[k];
                e_lo[k] = ip[ep.idx_i64[k] ? 2 * en : en];
                e_hi[k] = ip[ep.idx_i64[k] ? 2 * en + 1 : en];
            }
    }

    // activation operands of this wave's units (zero past N and past the
    // range). Every load goes out first, from clamped addresses; the masks
    // come after the last one (a use of a loaded value waits for every load
    // issued before it, so a mask between loads would split them in rounds).
    static_assert(!PAIR || (pair_type<WT>() && KS == 1 && STAGED), "paired blocks: one staged unit a wave");
    long A[KS][8];
    const bool col_ok = wr < N;
    auto a_ok = [&](int t, int j) {
        const int64_t e = 256 * (u0 + t) + 32 * j;  // first element of the block / sub-block
        return col_ok && e < 256 * u_end && e < K;
    };
    if constexpr (PAIR) {
        // lane (g, i): column i & 7's codes 16 g .. of the unit's 64-element
        // pair p (block 2p for rows i < 8 = groups 0, 1; 2p + 1 for rows i >=
        // 8 = groups 2, 3), zero elsewhere
        const int c = wr & 7;
        const bool pa_ok = ((wr < 8) == (g < 2)) && c < N && u0 < u_end;
        const int8_t *aq = act.qs + (arow0 + (c < N ? c : 0)) * K + 256 * (u0 < u_end ? u0 : u_begin) + 16 * g;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint4 q = ldu<uint4>(aq + 64 * p);
            A[0][2 * p] = (long)(((uint64_t)q.y << 32) | q.x);
            A[0][2 * p + 1] = (long)(((uint64_t)q.w << 32) | q.z);
        }
        for (int64_t i = threadIdx.x; i < (s_end - s_begin) * SK_COLS; i += blockDim.x) {
            const int64_t b = s_begin + (i >> 4);
            const int c2 = (int)(i & 15);
            const float dv = act.d[(arow0 + (c2 < N ? c2 : 0)) * nblk + b];
            sd[i] = c2 < N ? dv : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) A[0][j] = pa_ok ? A[0][j] : 0;
    } else {
        const int8_t *aq = act.qs + (arow0 + (col_ok ? wr : 0)) * K;
#pragma unroll
        for (int t = 0; t < KS; ++t)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t ec = a_ok(t, j) ? 256 * (u0 + t) + 32 * j : 0;
                if constexpr (nibble_type<WT>()) {
                    // the lane's weight bytes 4g..4g+3 hold elements 4g.. (low) and 16+4g.. (high)
                    A[t][j] = pack2(ldu<uint32_t>(aq + ec + 4 * g), ldu<uint32_t>(aq + ec + 16 + 4 * g));
                } else {
                    A[t][j] = ldu<long>(aq + ec + 8 * g);
                }
            }
        for (int64_t i = threadIdx.x; i < (s_end - s_begin) * SK_COLS; i += blockDim.x) {
            const int64_t b = s_begin + (i >> 4);
            const int c = (int)(i & 15);
            const int64_t at = (arow0 + (c < N ? c : 0)) * nblk + b;
            const float dv = act.d[at];
            sd[i] = c < N ? dv : 0.0f;
            if constexpr (S8) {
                const float sv = __int_as_float(act.sum32[at]);
                ss[i] = c < N ? sv : 0.0f;
            }
        }
#pragma unroll
        for (int t = 0; t < KS; ++t)
#pragma unroll
            for (int j = 0; j < 8; ++j) A[t][j] = a_ok(t, j) ? A[t][j] : 0;
    }
    if constexpr (EPI) {
        // the table's entries of this launch's columns, to LDS
#pragma unroll
        for (int k = 0; k < RT_PER; ++k) {
            const int i = threadIdx.x + k * (int)blockDim.x;
            if (i < N * tpairs) s_rt[i] = rt_v[k];
        }
    }
    lds_barrier();

    char *dbase = (char *)a.dst + i12 * a.d_nb2 + i13 * a.d_nb3;
    // output element o = threadIdx.x (< 256) of a row group: column o / 16,
    // row o % 16; to dst, or with several K chunks to this chunk's partials
    // [chunk][batch][N][M]
    const int ocol = threadIdx.x >> 4, orow = threadIdx.x & 15;
    float *pbase = a.part ? a.part + (((int64_t)blockIdx.y * gridDim.z + batch) * a.N + ocol) * a.M : nullptr;
    auto out_ptr = [&](int64_t grp) {
        if (a.nseg > 0) {
            const int64_t m = grp * 16 + orow;
            const int sg = seg_of(grp * 16);
            return (float *)((char *)a.seg_dst[sg] + (a.n0 + ocol) * a.seg_d_nb1[sg] + (m - a.seg_m0[sg]) * 4);
        }
        return pbase ? pbase + grp * 16 + orow : (float *)(dbase + (a.n0 + ocol) * a.d_nb1 + (grp * 16 + orow) * 4);
    };

    // Outputs wait in LDS (each thread rereads only what it wrote) and go to
    // memory every SK_OUTBUF row groups: a store in flight would make the next
    // wait for prefetched weights a wait for everything (loads and stores
    // share one completion counter that is not in order across the two).
    int nbuf = 0;
    int64_t buf_rg = rg;
    // EPI: output (row m, column n) with value v, its rotation partner's value o
    auto epi_store = [&](int64_t m, int n, float v, float o) {
        if constexpr (EPI) {
            auto sel = [](int s, auto x0, auto x1, auto x2) { return s == 0 ? x0 : s == 1 ? x1 : x2; };
            const int sg = seg_of(m);
            const int64_t j = m - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2]);
            const int lay = sel(sg, ep.layout[0], ep.layout[1], ep.layout[2]);
            if (lay == EPI_F32) {
                *(float *)((char *)sel(sg, a.seg_dst[0], a.seg_dst[1], a.seg_dst[2]) +
                           n * sel(sg, a.seg_d_nb1[0], a.seg_d_nb1[1], a.seg_d_nb1[2]) + j * 4) = v;
                return;
            }
            float y = v;
            if (sel(sg, ep.rope[0], ep.rope[1], ep.rope[2])) {
                const uint32_t el = (uint32_t)j % (uint32_t)ep.ne0, pr = el / 2;  // rows below 2^31 (launcher)
                if (2 * pr < (uint32_t)ep.rp.n_dims) {
                    float cs, sn;
                    if (tpairs) {
                        const float2 t = s_rt[(n - a.n0) * tpairs + pr];
                        cs = t.x, sn = t.y;
                    } else {
                        rope_cs_sn(e_pos, pr, ep.ff ? ep.ff[pr] : 1.0f, ep.rp, cs, sn);
                        if (ep.rt_mode == 1 && (el & 1) == 0) {  // one writer per pair, the table's row width
                            const int tw = (int)(ep.rp.n_dims < ep.ne0 ? ep.rp.n_dims : ep.ne0) / 2;
                            ((float2 *)ep.rt)[(int64_t)n * tw + pr] = make_float2(cs, sn);
                        }
                    }
                    y = (el & 1) == 0 ? rope_first(v, o, cs, sn) : rope_second(o, v, cs, sn);
                }
            }
            char *base = sel(sg, ep.dst[0], ep.dst[1], ep.dst[2]);
            const bool h16 = sel(sg, ep.f16[0], ep.f16[1], ep.f16[2]) != 0;
            int64_t at;  // element offset
            if (lay == EPI_CONTIG) {
                at = (int64_t)n * (sel(sg, a.seg_m0[1], a.seg_m0[2], a.seg_m0[3]) - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2])) + j;
            } else {
                const int32_t lo = sel(sg, e_lo[0], e_lo[1], e_lo[2]), hi = sel(sg, e_hi[0], e_hi[1], e_hi[2]);
                const int64_t r = sel(sg, ep.idx_i64[0], ep.idx_i64[1], ep.idx_i64[2])
                                      ? (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo)
                                      : (int64_t)lo;
                if (r < 0 || r >= sel(sg, ep.rows[0], ep.rows[1], ep.rows[2])) return;
                if (lay == EPI_CACHE_ROW) {
                    base += r * sel(sg, ep.row_nb[0], ep.row_nb[1], ep.row_nb[2]);
                    at = j;
                } else {  // the paged pools' layouts: keys [blocks, kvh, hs/8, bs, 8], values [blocks, kvh, hs, bs]
                    const uint32_t ru = (uint32_t)r, bs = (uint32_t)ep.bs, hs = (uint32_t)ep.hs, ju = (uint32_t)j;
                    const int64_t blk = ru / bs, off = ru % bs, h = ju / hs, el = ju % hs;
                    at = lay == EPI_PAGED_KEY ? (((blk * ep.kvh + h) * (ep.hs / 8) + el / 8) * ep.bs + off) * 8 + el % 8
                                              : ((blk * ep.kvh + h) * ep.hs + el) * ep.bs + off;
                }
            }
            if (h16) ((uint16_t *)base)[at] = f2h(y);
            else ((float *)base)[at] = y;
        }
    };
    auto flush = [&]() {
        if (threadIdx.x < 16 * SK_COLS)
            for (int k = 0; k < nbuf; ++k) {
                const int64_t grp = buf_rg + (int64_t)k * gridDim.x;
                if (ocol < N && grp * 16 + orow < a.M) {
                    if constexpr (EPI) {  // the pair partner: the neighbouring row, same column
                        epi_store(grp * 16 + orow, (int)(a.n0 + ocol), obuf[k * 256 + threadIdx.x],
                                  obuf[k * 256 + (threadIdx.x ^ 1)]);
                    } else {
                        *out_ptr(grp) = bad_id ? __builtin_nanf("") : obuf[k * 256 + threadIdx.x];
                    }
                }
            }
        nbuf = 0;
        // the stores complete here, so no later wait for loads is widened by them
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    };

    // reduce the waves' partials through LDS buffer `parity`, buffer the result
    auto finish = [&](const float (&y)[4], int64_t grp, int parity) {
        float4 *slot = red + parity * nw * 64;
        slot[wave * 64 + lane] = make_float4(y[0], y[1], y[2], y[3]);
        lds_barrier();
        if (nbuf == 0) buf_rg = grp;
        if (threadIdx.x < 16 * SK_COLS) {
            const int l = orow + 16 * (ocol >> 2), r = ocol & 3;
            const float *sl = (const float *)slot + 4 * l + r;
            float s = 0.0f;
            for (int wv = 0; wv < nw; ++wv) s += sl[256 * wv];
            obuf[nbuf * 256 + threadIdx.x] = s;
        }
        if (++nbuf == SK_OUTBUF) flush();
    };

    auto unit_slots = [&](int t) { return sd + (KQ ? (u0 + t - s_begin) : 8 * (u0 + t) - s_begin) * SK_COLS; };
    const int64_t s_gap = ss - sd;  // an s slot sits this far after its d slot
    auto unit_nvalid = [&](int t) {
        const int64_t v = s_end - 8 * (u0 + t);
        return KQ ? 8 : (int)(v < 0 ? 0 : v > 8 ? 8 : v);
    };
    // multiply one row group from the wave's LDS buffer
    auto process_staged = [&](int64_t grp, int parity, typename St::ExtraT dq) {
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (PAIR) {
            if (u0 < u_end) {  // wave-uniform
                v4i A2[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint64_t lo = (uint64_t)A[0][2 * p], hi = (uint64_t)A[0][2 * p + 1];
                    A2[p] = (v4i){(int)(uint32_t)lo, (int)(uint32_t)(lo >> 32), (int)(uint32_t)hi, (int)(uint32_t)(hi >> 32)};
                }
                unit_mma_pair<WT>(wbuf, (uint32_t)(wr * St::RB), A2, unit_slots(0), g, y);
            }
            // lanes g < 2 (columns 4 g + r) add the odd blocks' sums of lane l + 32
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] += __shfl_xor(y[r], 32);
            finish(y, grp, parity);
            return;
        }
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            if (u0 + t >= u_end) continue;  // wave-uniform
            const uint32_t ub = (uint32_t)(wr * St::RB + t * staged_bytes<WT>());  // the row's unit in wbuf
            if constexpr (WT == TLH_TYPE_Q6_K) {
                UnitW<WT> w;
                w.load_lds(wbuf + ub, g);
                unit_mma_q6k(w, dq, A[t], unit_slots(t), g, y);
            } else if constexpr (WT == TLH_TYPE_Q2_K) {
                UnitW<WT> w;
                w.load_lds(wbuf + ub, g);
                unit_mma_q2k(w, dq, A[t], unit_slots(t), g, y);
            } else if constexpr (WT == TLH_TYPE_Q3_K) {
                UnitW<WT> w;
                w.load_lds(wbuf + ub, g);
                unit_mma_q3k(w, dq, A[t], unit_slots(t), g, y);
            } else if constexpr (KQ) {
                UnitW<WT> w;
                w.load_lds(wbuf + ub, g);
                unit_mma<WT>(w, A[t], unit_slots(t), nullptr, g, 8, y);
            } else {
                // block by block: the operands of one block live at a time
                const int nv = unit_nvalid(t);
                const float *sdu = unit_slots(t);
                const uint32_t *w32 = (const uint32_t *)wbuf;
                const uint16_t *w16 = (const uint16_t *)wbuf;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (j >= nv) continue;  // wave-uniform
                    const uint32_t blk = ub + j * block_bytes(WT);
                    if constexpr (legacy_type(WT)) {
                        const uint32_t v = lds_u32(w32, blk + blk_qs_off(WT) + 4 * g);
                        const uint32_t qh = has_qh(WT) ? lds_u32(w32, blk + blk_qh_off(WT)) : 0u;
                        block_mma_legacy<WT>(A[t][j], legacy_B<WT>(v, qh, g), lds_u32(w32, blk), sdu + j * SK_COLS,
                                             sdu + s_gap + j * SK_COLS, g, y);
                        __builtin_amdgcn_sched_barrier(0);
                        continue;
                    }
                    long B;
                    if constexpr (WT == TLH_TYPE_Q4_0) {
                        const uint32_t v = lds_u32(w32, blk + 2 + 4 * g);
                        B = pack2(nib_minus8(v & 0x0f0f0f0fu), nib_minus8((v >> 4) & 0x0f0f0f0fu));
                    } else {
                        const uint2 v = lds_u64(w32, blk + 2 + 8 * g);
                        B = pack2(v.x, v.y);
                    }
                    block_mma<WT>(A[t][j], B, w16[blk >> 1], sdu + j * SK_COLS, g, y);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // one unit's operands live at a time
            __builtin_amdgcn_sched_barrier(0);
        }
        finish(y, grp, parity);
    };
    // ... or direct registers
    auto process_direct = [&](const DirectW<WT, KS> &d, int64_t grp, int parity) {
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            if (u0 + t >= u_end) continue;  // wave-uniform
            if constexpr (!staged_extra<WT>())
                unit_mma<WT>(d.u[t], A[t], unit_slots(t), unit_slots(t) + s_gap, g, unit_nvalid(t), y);
        }
        finish(y, grp, parity);
    };

    // The loads of the next row group are in flight while this one is
    // multiplied. Staged: the registers hold only loads in flight (this
    // group's bytes are in LDS by then), one set. Direct: two register sets
    // in turn, so no register copy makes the wave wait for the loads early.
    // The prefetch is unconditional (past the last group it rereads the
    // current one, a cache hit) so that the compiler can count the loads in
    // flight and wait only for the ones it needs.
    if constexpr (STAGED) {
        for (int it = 0; rg < groups; ++it) {
            const int64_t r1 = rg + gridDim.x;
#pragma unroll
            for (int i = 0; i < St::NL; ++i) *(uint4 *)(wbuf + 1024 * i + 16 * lane) = st.v[i];
            const auto dq = st.dq;  // this group's (read with its weight bytes above)
            stage_load(st, r1 < groups ? r1 : rg);
            process_staged(rg, it & 1, dq);
            rg = r1;
        }
    } else {
        const int64_t dlast = (s_end - 1) / (KQ ? 1 : 8);
        for (;;) {
            if (rg >= groups) break;
            const int64_t r1 = rg + gridDim.x;
            db.load(wrow_of(r1 < groups ? r1 : rg), u0, dlast, s_end, g);
            process_direct(da, rg, 0);
            if (r1 >= groups) break;
            const int64_t r2 = r1 + gridDim.x;
            da.load(wrow_of(r2 < groups ? r2 : r1), u0, dlast, s_end, g);
            process_direct(db, r1, 1);
            rg = r2;
        }
    }
    flush();
}

// Tall matrices (the vocabulary projection): every wave owns whole 16-row
// groups over all of K (K <= 4096, a multiple of 256), so no wave waits for
// another in the main loop -- no barrier, no cross-wave sum of partials per
// group, as the K-split form above needs. The activation operands of all K
// (8 bytes a lane a block) and their scales are written to LDS once per
// workgroup; each wave streams its group's weights one 256-element unit at a
// time through its own LDS staging buffer (the next unit's loads in flight
// while this one is multiplied) and keeps its 16 x 16 outputs in registers
// until the group ends. Per block the arithmetic is the K-split form's
// (block_mma / unit_mma), so the products agree bit for bit only up to the
// f32 order of the block sums within a row, which is the same here: blocks
// in K order.
constexpr int GC_WAVES = 16;

template <int WT, bool PAIR>
__global__ void __launch_bounds__(1024) k_gemv_cols(const MatmulArgs a) {
    kernarg_prefetch<(kernarg_lines(sizeof(MatmulArgs)))>();
    extern __shared__ __attribute__((aligned(16))) char gc_lds[];
    constexpr int AT = vec_dot_type(WT);
    constexpr bool KQ = kquant<WT>();
    constexpr int UB = unit_bytes<WT>();
    using St = Stage<WT, 1>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, wr = lane & 15;
    const int64_t K = a.K;
    const int units = (int)(K / 256);
    const int nblk = (int)(K / block_elems(AT));
    const int slots = KQ ? units : 8 * units;
    const ActView act = act_view(a.act, AT, K, mm_act_rows(a));
    const int N = (int)a.N;
    static_assert(!PAIR || pair_type<WT>(), "paired blocks: q4_0, q8_0, q4_K, q5_K");
    long *sA = (long *)gc_lds;                      // [8 * units][64]: block j's A operand of lane l
    v4i *sA2 = (v4i *)gc_lds;                       // PAIR: [4 * units][64]: block pair p's A operand of lane l
    float *sd = (float *)(sA + (size_t)8 * units * 64);  // [slots][16 columns]
    uint8_t *wbuf = (uint8_t *)(sd + (size_t)slots * SK_COLS) + (size_t)wave * St::BUF;

    // A operands (zero past N) and scales of the whole K, once per workgroup
    if constexpr (PAIR) {
        for (int idx = threadIdx.x; idx < 4 * units * 64; idx += blockDim.x) {
            const int p = idx >> 6, l = idx & 63, i = l & 15, gg = l >> 4;
            const int c = i & 7;
            v4i v = {0, 0, 0, 0};
            if ((i < 8) == (gg < 2) && c < N) {  // block 2p for rows 0..7, 2p + 1 for rows 8..15
                const uint4 q = ldu<uint4>(act.qs + (a.n0 + c) * K + 64 * p + 16 * gg);
                v = (v4i){(int)q.x, (int)q.y, (int)q.z, (int)q.w};
            }
            sA2[idx] = v;
        }
    } else {
        for (int idx = threadIdx.x; idx < 8 * units * 64; idx += blockDim.x) {
            const int j = idx >> 6, l = idx & 63, c = l & 15, gg = l >> 4;
            long v = 0;
            if (c < N) {
                const int8_t *aq = act.qs + (a.n0 + c) * K + 32 * j;
                if constexpr (nibble_type<WT>()) v = pack2(ldu<uint32_t>(aq + 4 * gg), ldu<uint32_t>(aq + 16 + 4 * gg));
                else v = ldu<long>(aq + 8 * gg);
            }
            sA[idx] = v;
        }
    }
    for (int idx = threadIdx.x; idx < slots * SK_COLS; idx += blockDim.x) {
        const int b = idx >> 4, c = idx & 15;
        sd[idx] = c < N ? act.d[(a.n0 + c) * nblk + b] : 0.0f;
    }
    __syncthreads();

    // staging pieces of a unit, as in the K-split form (KS = 1)
    int pr[St::NL];
    int poff[St::NL];
#pragma unroll
    for (int i = 0; i < St::NL; ++i) {
        const int p = 64 * i + lane;
        const int pc = p < 16 * St::PR ? p : 0;
        pr[i] = pc / St::PR;
        poff[i] = 16 * (pc - pr[i] * St::PR);
    }
    const int64_t groups = (a.M + 15) / 16;
    auto stage_load = [&](St &s, int64_t grp, int u) {
#pragma unroll
        for (int i = 0; i < St::NL; ++i) {
            const int64_t row = grp * 16 + pr[i] < a.M ? grp * 16 + pr[i] : a.M - 1;  // clamp: loads in bounds
            s.v[i] = ldu<uint4>(a.w + row * a.w_nb1 + (int64_t)u * UB + poff[i]);
        }
        if constexpr (WT == TLH_TYPE_Q6_K) {
            const int64_t row = grp * 16 + wr < a.M ? grp * 16 + wr : a.M - 1;
            s.dq = ldu<uint16_t>(a.w + row * a.w_nb1 + (int64_t)u * UB + 208);
        }
    };

    for (int64_t grp = (int64_t)blockIdx.x * GC_WAVES + wave; grp < groups; grp += (int64_t)gridDim.x * GC_WAVES) {
        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        St st;
        stage_load(st, grp, 0);
        for (int u = 0; u < units; ++u) {
            // this unit's bytes to the wave's own buffer (a wave's LDS accesses
            // are in order: no barrier), the next unit's loads out
#pragma unroll
            for (int i = 0; i < St::NL; ++i) *(uint4 *)(wbuf + 1024 * i + 16 * lane) = st.v[i];
            const uint32_t dq = st.dq;
            if (u + 1 < units) stage_load(st, grp, u + 1);
            const uint32_t ub = (uint32_t)(wr * St::RB);
            const float *sdu = sd + (KQ ? u : 8 * u) * SK_COLS;
            if constexpr (PAIR) {
                v4i A2[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) A2[p] = sA2[(4 * u + p) * 64 + lane];
                unit_mma_pair<WT>(wbuf, ub, A2, sdu, g, y);
                continue;
            }
            long A[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) A[j] = sA[(8 * u + j) * 64 + lane];
            if constexpr (WT == TLH_TYPE_Q6_K) {
                UnitW<WT> w;
                w.load_lds(wbuf + ub, g);
                unit_mma_q6k(w, dq, A, sdu, g, y);
            } else if constexpr (KQ) {
                UnitW<WT> w;
                w.load_lds(wbuf + ub, g);
                unit_mma<WT>(w, A, sdu, nullptr, g, 8, y);
            } else {
                const uint32_t *w32 = (const uint32_t *)wbuf;
                const uint16_t *w16 = (const uint16_t *)wbuf;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t blk = ub + j * block_bytes(WT);
                    long B;
                    if constexpr (WT == TLH_TYPE_Q4_0) {
                        const uint32_t v = lds_u32(w32, blk + 2 + 4 * g);
                        B = pack2(nib_minus8(v & 0x0f0f0f0fu), nib_minus8((v >> 4) & 0x0f0f0f0fu));
                    } else {
                        const uint2 v = lds_u64(w32, blk + 2 + 8 * g);
                        B = pack2(v.x, v.y);
                    }
                    block_mma<WT>(A[j], B, w16[blk >> 1], sdu + j * SK_COLS, g, y);
                }
            }
        }
        // lane (g, wr): columns 4g + r of row grp * 16 + wr (PAIR: 4 (g & 1) + r,
        // lanes g < 2 adding the odd blocks' sums of lane l + 32)
        if constexpr (PAIR) {
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] += __shfl_xor(y[r], 32);
        }
        const int64_t row = grp * 16 + wr;
        if (row < a.M && (!PAIR || g < 2)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int col = 4 * g + r;
                if (col < N) *(float *)((char *)a.dst + (a.n0 + col) * a.d_nb1 + row * 4) = y[r];
            }
        }
    }
}

static bool gemv_cols_ok(const MatmulArgs &a) {
    constexpr int64_t CUS = 256;  // MI355X
    const bool wt = a.wtype == TLH_TYPE_Q4_0 || a.wtype == TLH_TYPE_Q8_0 || a.wtype == TLH_TYPE_Q4_K ||
                    a.wtype == TLH_TYPE_Q5_K || a.wtype == TLH_TYPE_Q6_K;
    return wt && a.K % 256 == 0 && a.K <= 4096 && a.nseg == 0 && !a.ids && a.ne12 * a.ne13 == 1 &&
           (a.M + 15) / 16 >= CUS * GC_WAVES;
}

template <int WT> static tlh_status launch_cols(const MatmulArgs &a, hipStream_t stream) {
    using St = Stage<WT, 1>;
    const int64_t units = a.K / 256;
    const int64_t slots = kquant<WT>() ? units : 8 * units;
    const size_t lds = (size_t)8 * units * 64 * 8 + (size_t)slots * SK_COLS * 4 + (size_t)GC_WAVES * St::BUF;
    const int64_t cus = device_cus();
    const int64_t groups = (a.M + 15) / 16;
    const int64_t wgs = (groups + GC_WAVES - 1) / GC_WAVES;
    const dim3 grid((unsigned)(wgs < cus ? wgs : cus));
    if constexpr (pair_type<WT>()) {
        if (a.N <= 8) {
            hipLaunchKernelGGL((k_gemv_cols<WT, true>), grid, dim3(64 * GC_WAVES), lds, stream, a);
            return check_launch("gemv_cols (pairs)");
        }
    }
    hipLaunchKernelGGL((k_gemv_cols<WT, false>), grid, dim3(64 * GC_WAVES), lds, stream, a);
    return check_launch("gemv_cols");
}

// Units per wave: one (16 activation-operand registers); a workgroup covers
// up to 16 units (K = 4096); longer K takes several chunks.
template <int WT> constexpr int sk_ks() { return 1; }
bool gemv_mfma_supported(int64_t N) { return N >= 1 && N <= SK_COLS; }


// dst (strided, columns n0..) = sum over the K chunks of the partials, in
// chunk order. Grid: (rows / 256, columns, batch slices); columns past the
// grid's y extent loop.
__global__ void __launch_bounds__(256) k_gemv_mfma_reduce(const MatmulArgs a, int chunks) {
    kernarg_prefetch<(kernarg_lines(sizeof(MatmulArgs)))>();
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= a.M) return;
    const int64_t batches = a.ne12 * a.ne13, batch = blockIdx.z;
    const int64_t per_batch = a.N * a.M, cstride = batches * per_batch;
    const MmSlice sl = mm_slice(a, blockIdx.z);
    int sg = 0;
    if (a.nseg > 0) sg = (int)(m >= a.seg_m0[1]) + (int)(a.nseg > 2 && m >= a.seg_m0[2]);
    for (int64_t n = blockIdx.y; n < a.N; n += gridDim.y) {
        const float *p = a.part + batch * per_batch + n * a.M + m;
        float s = 0.0f;
        for (int c = 0; c < chunks; ++c) s += p[c * cstride];
        if (a.nseg > 0)  // one batch slice; row m of the launch is row m - seg_m0[sg] of segment sg
            *(float *)((char *)a.seg_dst[sg] + (a.n0 + n) * a.seg_d_nb1[sg] + (m - a.seg_m0[sg]) * 4) = s;
        else
            *(float *)((char *)a.dst + sl.i12 * a.d_nb2 + sl.i13 * a.d_nb3 + (a.n0 + n) * a.d_nb1 + m * 4) = s;
    }
}

tlh_status launch_partial_reduce(const MatmulArgs &a, int chunks, hipStream_t stream) {
    const int64_t batches = a.ne12 * a.ne13;
    if (a.M <= 0 || a.N <= 0 || batches <= 0) return TLH_OK;
    const dim3 grid((unsigned)((a.M + 255) / 256), (unsigned)(a.N < 65535 ? a.N : 65535), (unsigned)batches);
    hipLaunchKernelGGL(k_gemv_mfma_reduce, grid, dim3(256), 0, stream, a, chunks);
    return check_launch("partial_reduce");
}

// The reduce with the few-column kernel's store epilogue (GemvEpi), for a
// K-split GEMM over Q / K / V segments at many tokens (a prefill): element
// (m, n) = the sum of the chunks' partials in chunk order (as
// k_gemv_mfma_reduce), then rotated with its pair partner m ^ 1 (the
// neighbouring lane: rotated segments start at even rows), cast and stored
// into the segment's layout for token n -- and, with ep.dual[s], also into
// the segment's paged pool (dst2: the key or value layout). A workgroup takes
// 256 rows x RE_TOK tokens: the tokens' rotation (cos, sin) per pair and
// every token's sum of partials first (the CPU's chain of products, once per
// token and pair), then token by token the row-contiguous stores; the paged stores last, from LDS,
// with the lanes walking a value's tokens (or a key's 8-element groups)
// fastest, so consecutive slots of a block are written together. One batch
// slice; grid (rows / 256, columns / RE_TOK).
constexpr int RE_PAIRS = 256;  // ne0 <= 512
constexpr int RE_TOK = 16;
constexpr int RE_CH = 4;  // chunks whose partials are requested before the rotation work
__global__ void __launch_bounds__(256) k_reduce_epi(const MatmulArgs a, int chunks, const GemvEpi ep) {
    kernarg_prefetch<(kernarg_lines(sizeof(MatmulArgs) + sizeof(int) + sizeof(GemvEpi)))>();
    __shared__ float2 s_t[RE_TOK * RE_PAIRS];  // (cos, sin) of token t, pair pr at t * np + pr
    __shared__ __attribute__((aligned(16))) uint16_t s_h[RE_TOK][256];  // f16 results for the paged stores
    // per thread (so every thread writes its entry: a write behind a branch
    // lets the compiler sink the load that feeds it behind the partials')
    __shared__ int64_t s_slot[256];  // [3][RE_TOK]: segment s's slot of token t at s * RE_TOK + t
    __shared__ float s_ff[256], s_pos[256];
    const int tid = threadIdx.x;
    const int64_t m = (int64_t)blockIdx.x * 256 + tid;
    const bool mvalid = m < a.M;
    const int64_t mc = mvalid ? m : a.M - 1;
    const int64_t cstride = a.N * a.M;
    const int64_t nb = (int64_t)blockIdx.y * RE_TOK;
    const int nt = (int)(a.N - nb < RE_TOK ? a.N - nb : RE_TOK);
    auto sel = [](int s, auto x0, auto x1, auto x2) { return s == 0 ? x0 : s == 1 ? x1 : x2; };
    auto seg_of = [&](int64_t r) { return (int)(r >= a.seg_m0[1]) + (int)(a.nseg > 2 && r >= a.seg_m0[2]); };
    const int sg = seg_of(mc);
    const int64_t j = mc - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2]);
    const int lay = sel(sg, ep.layout[0], ep.layout[1], ep.layout[2]);
    const bool rot = sel(sg, ep.rope[0], ep.rope[1], ep.rope[2]) != 0;
    const bool h16 = sel(sg, ep.f16[0], ep.f16[1], ep.f16[2]) != 0;
    const int64_t seg_rows = sel(sg, a.seg_m0[1], a.seg_m0[2], a.seg_m0[3]) - sel(sg, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2]);
    const bool any_rot = ep.rope[0] | ep.rope[1] | ep.rope[2];
    const bool any_dual = ep.dual[0] | ep.dual[1] | ep.dual[2];
    const int np = any_rot ? (int)((ep.rp.n_dims < ep.ne0 ? ep.rp.n_dims : ep.ne0) / 2) : 0;
    // Loads go out in the order their values are needed (vector loads complete
    // in order): the tokens' positions, the pairs' frequency factors and the
    // slot indices, then the partials of up to RE_CH chunks, so the rotation
    // work below runs while the partials land (the stores further down may
    // alias the partials for all the compiler knows, so every load comes
    // before them). Every load is unconditional, from a clamped address.
    // (an absent pointer reads the partials instead; the value is dropped)
    const int64_t tok0 = a.n0 + nb;
    const int32_t pos_raw = (ep.pos ? ep.pos : (const int32_t *)a.part)[tok0 + (tid < nt ? tid : 0)];
    const uint32_t ff_raw = (ep.ff ? (const uint32_t *)ep.ff : (const uint32_t *)a.part)[tid < np ? tid : 0];
    const int s3 = tid < 3 * RE_TOK ? tid / RE_TOK : 0, t3 = tid % RE_TOK;
    const bool i64 = sel(s3, ep.idx_i64[0], ep.idx_i64[1], ep.idx_i64[2]) != 0;
    const char *ip3 = sel(s3, ep.idx[0], ep.idx[1], ep.idx[2]);
    const char *ipl = (ip3 ? ip3 : (const char *)a.part) + (tok0 + (t3 < nt ? t3 : 0)) * (i64 ? 8 : 4);
    const uint32_t idx_lo = *(const uint32_t *)ipl, idx_hi = *(const uint32_t *)(ipl + (i64 ? 4 : 0));
    float pv[RE_CH][RE_TOK];
    const int ch0 = chunks < RE_CH ? chunks : RE_CH;
#pragma unroll
    for (int c = 0; c < RE_CH; ++c) {
        const float *pc = a.part + (c < ch0 ? c : 0) * cstride + mc;
#pragma unroll
        for (int t = 0; t < RE_TOK; ++t) pv[c][t] = pc[(nb + (t < nt ? t : 0)) * a.M];
    }
    // the row / slot indices, positions and factors to LDS (the waits cover
    // those first loads only), then the tokens' rotations
    {
        int64_t r = i64 ? (int64_t)(((uint64_t)idx_hi << 32) | idx_lo) : (int64_t)(int32_t)idx_lo;
        const bool bad = (tid >= 3 * RE_TOK) | (t3 >= nt) | (ip3 == nullptr) | (r >= sel(s3, ep.rows[0], ep.rows[1], ep.rows[2]));
        s_slot[tid] = bad ? -1 : r;
    }
    s_pos[tid] = (float)pos_raw;
    s_ff[tid] = ep.ff ? __uint_as_float(ff_raw) : 1.0f;
    lds_barrier();  // LDS only: the partials stay in flight
    for (int i = tid; i < nt * np; i += 256) {
        const int t = i / np, pr = i - t * np;
        float cs, sn;
        rope_cs_sn(s_pos[t], pr, s_ff[pr], ep.rp, cs, sn);
        s_t[i] = make_float2(cs, sn);
    }
    // every token's sum, adding the chunks in order (chunks past RE_CH, if
    // any, load here)
    float vs[RE_TOK];
#pragma unroll
    for (int t = 0; t < RE_TOK; ++t) vs[t] = 0.0f;
#pragma unroll
    for (int c = 0; c < RE_CH; ++c)
#pragma unroll
        for (int t = 0; t < RE_TOK; ++t)
            if (c < ch0) vs[t] += pv[c][t];
    for (int c = RE_CH; c < chunks; ++c) {
        const float *pc = a.part + c * cstride + mc;
#pragma unroll
        for (int t = 0; t < RE_TOK; ++t) vs[t] += pc[(nb + (t < nt ? t : 0)) * a.M];
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < RE_TOK; ++t) {
        if (t >= nt) break;
        const int64_t n = nb + t, tok = a.n0 + n;
        const float v = vs[t];
        const float o = __shfl_xor(v, 1, 64);
        float y = v;
        if (rot) {
            const uint32_t el = (uint32_t)j % (uint32_t)ep.ne0, pr = el / 2;  // rows below 2^31 (launcher)
            if ((int)pr < np) {
                const float2 c2 = s_t[t * np + pr];
                y = (el & 1) == 0 ? rope_first(v, o, c2.x, c2.y) : rope_second(o, v, c2.x, c2.y);
            }
        }
        const uint16_t yh = f2h(y);
        if (any_dual) s_h[t][tid] = yh;
        if (!mvalid) continue;
        if (lay == EPI_F32) {
            *(float *)((char *)sel(sg, a.seg_dst[0], a.seg_dst[1], a.seg_dst[2]) +
                       tok * sel(sg, a.seg_d_nb1[0], a.seg_d_nb1[1], a.seg_d_nb1[2]) + j * 4) = v;
            continue;
        }
        char *base = sel(sg, ep.dst[0], ep.dst[1], ep.dst[2]);
        int64_t at;  // element offset
        if (lay == EPI_CONTIG) {
            at = tok * seg_rows + j;
        } else {
            const int64_t r = s_slot[sg * RE_TOK + t];
            if (r < 0) continue;
            if (lay == EPI_CACHE_ROW) {
                base += r * sel(sg, ep.row_nb[0], ep.row_nb[1], ep.row_nb[2]);
                at = j;
            } else {
                const uint32_t ru = (uint32_t)r, bs = (uint32_t)ep.bs, hs = (uint32_t)ep.hs, ju = (uint32_t)j;
                const int64_t blk = ru / bs, off = ru % bs, h = ju / hs, e = ju % hs;
                at = lay == EPI_PAGED_KEY ? (((blk * ep.kvh + h) * (ep.hs / 8) + e / 8) * ep.bs + off) * 8 + e % 8
                                          : ((blk * ep.kvh + h) * ep.hs + e) * ep.bs + off;
            }
        }
        if (h16) ((uint16_t *)base)[at] = yh;
        else ((float *)base)[at] = y;
    }
    if (!any_dual) return;
    __syncthreads();
    // the paged stores. A key pool keeps 8 elements of a token together: one
    // 16-byte store per (8-row group, token), consecutive threads on
    // consecutive tokens (segments start at multiples of 8 rows and head
    // sizes are multiples of 8, so a group is 8 elements e % 8 = 0..7 of one
    // head). A value pool keeps a block's tokens together: one element per
    // thread, consecutive threads on consecutive tokens.
    for (int idx = tid; idx < 32 * nt; idx += 256) {
        const int g8 = idx / nt, t = idx - g8 * nt, rr = 8 * g8;
        const int64_t mr = (int64_t)blockIdx.x * 256 + rr;
        if (mr >= a.M) continue;
        const int s2 = seg_of(mr);
        const int64_t r = s_slot[s2 * RE_TOK + t];
        if (sel(s2, ep.dual[0], ep.dual[1], ep.dual[2]) != EPI_PAGED_KEY || r < 0) continue;
        const uint32_t ru = (uint32_t)r, bs = (uint32_t)ep.bs, hs = (uint32_t)ep.hs;
        const uint32_t ju = (uint32_t)(mr - sel(s2, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2]));
        const int64_t blk = ru / bs, off = ru % bs, h = ju / hs, e = ju % hs;
        const int64_t at = (((blk * ep.kvh + h) * (ep.hs / 8) + e / 8) * ep.bs + off) * 8;
        *(uint4 *)((uint16_t *)sel(s2, ep.dst2[0], ep.dst2[1], ep.dst2[2]) + at) = *(const uint4 *)&s_h[t][rr];
    }
    for (int idx = tid; idx < 256 * nt; idx += 256) {
        const int rr = idx / nt, t = idx - rr * nt;
        const int64_t mr = (int64_t)blockIdx.x * 256 + rr;
        if (mr >= a.M) continue;
        const int s2 = seg_of(mr);
        const int64_t r = s_slot[s2 * RE_TOK + t];
        if (sel(s2, ep.dual[0], ep.dual[1], ep.dual[2]) != EPI_PAGED_VALUE || r < 0) continue;
        const uint32_t ru = (uint32_t)r, bs = (uint32_t)ep.bs, hs = (uint32_t)ep.hs;
        const uint32_t ju = (uint32_t)(mr - sel(s2, a.seg_m0[0], a.seg_m0[1], a.seg_m0[2]));
        const int64_t blk = ru / bs, off = ru % bs, h = ju / hs, e = ju % hs;
        ((uint16_t *)sel(s2, ep.dst2[0], ep.dst2[1], ep.dst2[2]))[((blk * ep.kvh + h) * ep.hs + e) * ep.bs + off] =
            s_h[t][rr];
    }
}

// What the store epilogue needs of the launch's segments and of ep (shared by
// the few-column kernel's and the reduce's epilogues).
static tlh_status epi_check(const MatmulArgs &a, const GemvEpi &ep, const char *who) {
    if (a.nseg < 1 || a.M >= ((int64_t)1 << 31) || a.ids || a.ne12 * a.ne13 != 1)
        return set_error(TLH_UNSUPPORTED, "%s: the store epilogue takes segments of one batch slice", who);
    bool rope = false;
    for (int sg = 0; sg < a.nseg; ++sg) {
        const int64_t rows = a.seg_m0[sg + 1] - a.seg_m0[sg];
        if (ep.layout[sg] != EPI_F32 && !ep.dst[sg]) return set_error(TLH_INVALID, "%s: epilogue without a destination", who);
        if ((ep.layout[sg] == EPI_CACHE_ROW || ep.layout[sg] >= EPI_PAGED_KEY) && !ep.idx[sg])
            return set_error(TLH_INVALID, "%s: epilogue row or slot index missing", who);
        if (ep.rows[sg] >= ((int64_t)1 << 31))
            return set_error(TLH_UNSUPPORTED, "%s: epilogue cache rows or pool slots past 2^31", who);
        if (ep.layout[sg] >= EPI_PAGED_KEY && (!ep.f16[sg] || !ep.idx_i64[sg] || ep.kvh < 1 || ep.hs < 8 || ep.hs % 8 ||
                                               ep.bs < 1 || rows != (int64_t)ep.kvh * ep.hs))
            return set_error(TLH_UNSUPPORTED, "%s: paged epilogue geometry", who);
        if (ep.rope[sg]) {
            rope = true;
            if (ep.ne0 < 2 || ep.ne0 % 2 || ep.ne0 > 512 || rows % ep.ne0 || a.seg_m0[sg] % 2)
                return set_error(TLH_UNSUPPORTED, "%s: rotated segments are whole heads of even size", who);
        }
        if (ep.dual[sg] && (ep.layout[sg] != EPI_CONTIG || !ep.f16[sg] || !ep.dst2[sg] || !ep.idx[sg] ||
                            !ep.idx_i64[sg] || (ep.dual[sg] != EPI_PAGED_KEY && ep.dual[sg] != EPI_PAGED_VALUE) ||
                            ep.kvh < 1 || ep.hs < 8 || ep.hs % 8 || ep.bs < 1 || rows != (int64_t)ep.kvh * ep.hs ||
                            (ep.dual[sg] == EPI_PAGED_KEY && (a.seg_m0[sg] % 8 || ((uintptr_t)ep.dst2[sg] & 15)))))
            return set_error(TLH_UNSUPPORTED, "%s: a second, paged store goes with contiguous f16 rows", who);
    }
    if (rope && (!ep.pos || ep.rp.mode != 0 || ep.rp.n_dims % 2 || ep.rp.n_dims < 0))
        return set_error(TLH_UNSUPPORTED, "%s: the epilogue rotates in ROPE mode 0 only", who);
    return TLH_OK;
}

tlh_status reduce_epi_check(const MatmulArgs &a, const GemvEpi &ep) { return epi_check(a, ep, "reduce"); }

tlh_status launch_partial_reduce_epi(const MatmulArgs &a, int chunks, const GemvEpi &ep, hipStream_t stream) {
    const tlh_status st = epi_check(a, ep, "reduce");
    if (st != TLH_OK) return st;
    if (a.M <= 0 || a.N <= 0) return TLH_OK;
    if ((a.N + RE_TOK - 1) / RE_TOK >= 65536)
        return set_error(TLH_UNSUPPORTED, "reduce: %lld columns through the store epilogue", (long long)a.N);
    const dim3 grid((unsigned)((a.M + 255) / 256), (unsigned)((a.N + RE_TOK - 1) / RE_TOK), 1u);
    hipLaunchKernelGGL(k_reduce_epi, grid, dim3(256), 0, stream, a, chunks, ep);
    return check_launch("partial_reduce (epilogue)");
}

static int64_t sk_share(int64_t K, int64_t &chunks) {
    const int64_t units = (K + 255) / 256;
    const int64_t per = (int64_t)SK_MAXW * sk_ks<TLH_TYPE_Q4_K>();
    chunks = (units + per - 1) / per;
    return (units + chunks - 1) / chunks;  // equal shares, so no chunk is left with a sliver
}

int64_t gemv_mfma_chunks(int64_t K) {
    int64_t chunks = 1;
    (void)sk_share(K, chunks);
    return chunks;
}

int64_t gemv_mfma_partial_bytes(int64_t K, int64_t M, int64_t N, int64_t batches) {
    int64_t chunks = 1;
    (void)sk_share(K, chunks);
    return chunks > 1 ? chunks * batches * (N < SK_COLS ? N : SK_COLS) * M * 4 : 0;
}

template <int WT, bool STAGED, typename EP = NoEpi, bool PAIR = false>
static tlh_status launch_sk_form(const MatmulArgs &a, hipStream_t stream, const EP &ep) {
    constexpr int KS = sk_ks<WT>();
    auto kern = k_gemv_mfma<WT, KS, STAGED, EP, PAIR>;
    int64_t chunks = 1;
    const int64_t share = sk_share(a.K, chunks);
    if (chunks > 1 && !a.part) return set_error(TLH_INVALID, "gemv_mfma: K=%lld needs a partials buffer", (long long)a.K);
    // at least 4 waves: the first 256 threads each own one of a row group's outputs
    const int nw = (int)((share + KS - 1) / KS) > 4 ? (int)((share + KS - 1) / KS) : 4;
    const size_t slots = (size_t)(kquant<WT>() ? share : 8 * share) * SK_COLS * 4;
    const size_t lds = (size_t)2 * nw * 64 * 16 + slots * (vec_dot_type(WT) == TLH_TYPE_Q8_1 ? 2 : 1) +
                       (size_t)SK_OUTBUF * 256 * 4 + (STAGED ? (size_t)nw * Stage<WT, KS>::BUF : 0) +
                       (size_t)SK_COLS * epi_table_pairs(ep) * sizeof(float2);
    // per-CU occupancy by wave count (the LDS size follows from it)
    static std::atomic<int> bpc[SK_MAXW + 1];
    const int nb = blocks_per_cu(kern, 64 * nw, lds, bpc[nw <= SK_MAXW ? nw : SK_MAXW]);
    const int64_t groups = (a.M + 15) / 16;
    const int64_t batches = a.ne12 * a.ne13;
    int64_t resident = (int64_t)device_cus() * nb / (batches * chunks > 0 ? batches * chunks : 1);
    if (resident < 1) resident = 1;
    const unsigned gx = (unsigned)(groups < resident ? groups : resident);
    MatmulArgs k = a;
    if (chunks == 1) k.part = nullptr;
    if (!std::is_same<EP, NoEpi>::value && chunks != 1)
        return set_error(TLH_UNSUPPORTED, "gemv_mfma: the store epilogue takes one K chunk");
    hipLaunchKernelGGL(kern, dim3(gx, (unsigned)chunks, (unsigned)batches), dim3(64 * nw), lds, stream, k, share, ep);
    tlh_status st = check_launch(PAIR ? "gemv_mfma (pairs)" : "gemv_mfma");
    if (st != TLH_OK || chunks == 1 || a.keep_part) return st;
    return launch_partial_reduce(a, (int)chunks, stream);
}

// Up to 8 columns of whole units: the paired-block form.
template <int WT, bool STAGED, typename EP = NoEpi>
static tlh_status launch_sk(const MatmulArgs &a, hipStream_t stream, const EP &ep = EP{}) {
    if constexpr (pair_type<WT>() && STAGED && sk_ks<WT>() == 1) {
        if (a.N <= 8 && a.K % 256 == 0) return launch_sk_form<WT, STAGED, EP, true>(a, stream, ep);
    }
    return launch_sk_form<WT, STAGED, EP, false>(a, stream, ep);
}

template <int WT> static tlh_status launch_sk_wt(const MatmulArgs &a, bool staged, hipStream_t stream) {
    if constexpr (kquant<WT>()) {
        return launch_sk<WT, true>(a, stream);  // K is a multiple of 256
    } else {
        return staged ? launch_sk<WT, true>(a, stream) : launch_sk<WT, false>(a, stream);
    }
}

// The few-column kernel with the store epilogue (segments, q4_K / q5_K / q6_K,
// K a multiple of 256 in one chunk, rows and segment rows below 2^31).
tlh_status launch_gemv_mfma_epi(const MatmulArgs &a, const GemvEpi &ep, hipStream_t stream) {
    if (!gemv_mfma_supported(a.N) || a.K % 256 != 0 || (ep.dual[0] | ep.dual[1] | ep.dual[2]))
        return set_error(TLH_UNSUPPORTED, "gemv_mfma: the store epilogue takes N <= 16, K %% 256 == 0, one store a row");
    const tlh_status st = epi_check(a, ep, "gemv_mfma");
    if (st != TLH_OK) return st;
    if (ep.rt_mode && (!ep.rt || ((uintptr_t)ep.rt & 7)))
        return set_error(TLH_INVALID, "gemv_mfma: the rotation table needs an 8-byte aligned buffer");
    if (ep.rt_mode == 2 && a.N * epi_table_pairs(ep) > 4 * 256)  // RT_PER entries a thread, at least 4 waves
        return set_error(TLH_UNSUPPORTED, "gemv_mfma: rotation table larger than the prologue reads");
    switch (a.wtype) {
    case TLH_TYPE_Q4_K: return launch_sk<TLH_TYPE_Q4_K, true, GemvEpi>(a, stream, ep);
    case TLH_TYPE_Q5_K: return launch_sk<TLH_TYPE_Q5_K, true, GemvEpi>(a, stream, ep);
    case TLH_TYPE_Q6_K: return launch_sk<TLH_TYPE_Q6_K, true, GemvEpi>(a, stream, ep);
    default: return set_error(TLH_UNSUPPORTED, "gemv_mfma: no store epilogue for weight type %d", a.wtype);
    }
}

tlh_status launch_gemv_mfma(const MatmulArgs &a, hipStream_t stream) {
    if (!gemv_mfma_supported(a.N)) return set_error(TLH_INVALID, "gemv_mfma: N=%lld", (long long)a.N);
    if (gemv_cols_ok(a)) {
        switch (a.wtype) {
        case TLH_TYPE_Q4_0: return launch_cols<TLH_TYPE_Q4_0>(a, stream);
        case TLH_TYPE_Q8_0: return launch_cols<TLH_TYPE_Q8_0>(a, stream);
        case TLH_TYPE_Q4_K: return launch_cols<TLH_TYPE_Q4_K>(a, stream);
        case TLH_TYPE_Q5_K: return launch_cols<TLH_TYPE_Q5_K>(a, stream);
        case TLH_TYPE_Q6_K: return launch_cols<TLH_TYPE_Q6_K>(a, stream);
        default: break;
        }
    }
    // whole units per row: every staged piece lies inside its row
    const bool staged = a.K % 256 == 0;
    switch (a.wtype) {
    case TLH_TYPE_Q4_0: return launch_sk_wt<TLH_TYPE_Q4_0>(a, staged, stream);
    case TLH_TYPE_Q8_0: return launch_sk_wt<TLH_TYPE_Q8_0>(a, staged, stream);
    case TLH_TYPE_Q4_1: return launch_sk_wt<TLH_TYPE_Q4_1>(a, staged, stream);
    case TLH_TYPE_Q5_0: return launch_sk_wt<TLH_TYPE_Q5_0>(a, staged, stream);
    case TLH_TYPE_Q5_1: return launch_sk_wt<TLH_TYPE_Q5_1>(a, staged, stream);
    case TLH_TYPE_Q4_K: return launch_sk_wt<TLH_TYPE_Q4_K>(a, staged, stream);
    case TLH_TYPE_Q5_K: return launch_sk_wt<TLH_TYPE_Q5_K>(a, staged, stream);
    case TLH_TYPE_Q6_K: return launch_sk_wt<TLH_TYPE_Q6_K>(a, staged, stream);
    case TLH_TYPE_Q2_K: return launch_sk_wt<TLH_TYPE_Q2_K>(a, staged, stream);
    case TLH_TYPE_Q3_K: return launch_sk_wt<TLH_TYPE_Q3_K>(a, staged, stream);
    default: return set_error(TLH_UNSUPPORTED, "gemv_mfma: weight type %d", a.wtype);
    }
}

}  // namespace tlh

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
// Tiling: 128 weight rows x 256 tokens per workgroup of 8 waves (above 128
// tokens; else 128 tokens, 4 waves), each wave 64 x 64 as 2 x 2 MFMA tiles of
// 32 x 32; K advances in stages of one 64-element q4_K chunk. LDS holds two
// stage buffers: while the waves multiply stage s, stage s + 1 fills the
// other one. Its activation codes (exact f16 from the quantize pass) go
// straight from global memory to LDS (buffer_load_dwordx4 ... lds: no
// registers, no LDS writes); its weight codes come to registers two stages
// ahead and are converted once per workgroup (nibble -> (1024 + n) * sc -
// 1024 * sc with one packed FMA) in the same block as the products, so the
// scheduler interleaves the two. One barrier per stage. With 256 tokens each
// weight code is converted once for twice the tokens of a 128-token tile;
// one such workgroup fills a CU's LDS, two of the 128-token ones fit.
//
// q5_K runs the same kernel with the fifth code bit OR-ed in before the f16
// conversion (sc * q <= 63 * 31 stays exact). q8_0 / q4_0 have their own
// int8-MFMA GEMM (gemm_q8.hip). q6_K weights with N > 16 run through the
// int8-MFMA few-column kernel (gemv_mfma.hip) in slabs of 16 columns (correct
// for any N; each slab re-reads the weights).
#include <type_traits>

#include "kernels.hpp"

namespace tlh {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBK = 64;
template <int V> using IC = std::integral_constant<int, V>;

// LDS: two stage buffers of f16 tiles (row = 64 halves = 8 chunks of 16 bytes,
// chunk c of row r stored at chunk position c ^ (r & 7) so the b128 operand
// reads of 8 consecutive rows hit distinct banks), and two buffers of the
// per-super-block metadata (by super-block parity). Each is its own __shared__
// array: the compiler then knows the weight tile's LDS stores do not alias the
// direct-to-LDS loads still in flight into the activation tile, and does not
// wait for those loads before the stores.
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

// What one thread fetches to registers for a stage: its weight row's header
// (every stage, so each stage issues the same loads; only a super-block's
// first stage reads it) and its CB code bytes of the stage; q5_K's fifth bits.
template <int CB>
struct StageRegs {
    uint4 hdr;
    uint32_t wq[CB / 4], qh[CB / 4];
};
typedef __attribute__((address_space(3))) void lds_void;

template <int CB>
__device__ __forceinline__ void ldg_codes(uint32_t (&d)[CB / 4], const uint8_t *p) {
    if constexpr (CB == 16) {
        const uint4 v = ldg16(p);
        d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
    } else {
        uint2 v;
        __builtin_memcpy(&v, p, 8);
        d[0] = v.x, d[1] = v.y;
    }
}

// NW waves per workgroup, each a 64 x 64 output tile (wave w: rows 64 (w & 1),
// tokens 64 (w >> 1)); the workgroup tile is 128 rows x 32 NW tokens. NW = 8
// (256 tokens) converts each weight code once for twice the tokens of NW = 4.
template <int WT, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) k_gemm_q4k(const MatmulArgs a) {
    constexpr bool Q5 = WT == TLH_TYPE_Q5_K;
    constexpr int SB = Q5 ? Q5_K_BYTES : Q4_K_BYTES;
    constexpr int QS = Q5 ? 48 : 16;  // offset of the nibble bytes
    constexpr int BN = 32 * NW;       // tokens per workgroup tile
    constexpr int TPR = NW / 2;       // threads per weight row in the staging
    constexpr int CB = 32 / TPR;      // code bytes of a stage per thread (16 or 8)
    // LDS: two stage buffers each of the f16 weight tile (row = 64 halves = 8
    // chunks of 16 bytes, chunk c of row r at chunk position c ^ (r & 7), so
    // the b128 operand reads of 8 consecutive rows hit distinct banks) and of
    // the f16 activation tile; the weight rows' d / dmin / mins by super-block
    // parity; the tokens' bsums and scales of the current super-block. The
    // activation tiles are each their own __shared__ array (a stage's buffer is
    // static in the loop), so the compiler knows that LDS reads and writes of
    // one do not alias the direct-to-LDS loads still in flight into the other,
    // and does not wait for those loads before them.
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][GBM][GBK];
    __shared__ __attribute__((aligned(16))) _Float16 sB0[BN][GBK];
    __shared__ __attribute__((aligned(16))) _Float16 sB1[BN][GBK];
    __shared__ __attribute__((aligned(16))) uint8_t sAmin[2][GBM][8];
    __shared__ __attribute__((aligned(16))) float sdA[2][GBM];
    __shared__ __attribute__((aligned(16))) float sdminA[2][GBM];
    __shared__ __attribute__((aligned(16))) _Float16 sBsum[BN][16];
    __shared__ __attribute__((aligned(16))) float sdB[BN];
    auto btile = [&](auto bc) -> _Float16(&)[BN][GBK] {
        if constexpr (decltype(bc)::value == 0) return sB0;
        else return sB1;
    };
    const int tid = threadIdx.x;
    // wave index in a scalar register (the direct-to-LDS destinations are wave-uniform)
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;  // wave tile position
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
    const int64_t n_base = (int64_t)blockIdx.x * BN;

    // staging roles: weight row tid / TPR, code bytes CB q .. + CB - 1 of the
    // stage's 32 (their low nibbles are elements CB q .. of the stage's first
    // sub-block, their high nibbles the same of its second)
    const int srow = tid / TPR, q = tid % TPR;
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
    // position l % 8, i.e. the chunk (l % 8) ^ (row & 7) of the token's stage.
    // They are buffer loads: a buffer resource over the activation codes, a
    // fixed 32-bit byte offset per lane and the stage's offset in a scalar
    // register (the launcher checks the activation fits 4 GiB), so no address
    // register is rewritten while a load that reads it may still be in flight.
    const int64_t rows_total = a.N_total * a.ne12 * a.ne13;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void *)act.q16, (short)0, (int)(rows_total * K * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rbs = __builtin_amdgcn_make_buffer_rsrc((void *)act.b16, (short)0, (int)(rows_total * (K / 16) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rdx = __builtin_amdgcn_make_buffer_rsrc((void *)act.d, (short)0, (int)(rows_total * nsb * 4), 0x00020000);
    uint32_t boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * (4 * wave + i) + (lane >> 3);
        const int64_t col = n_base + r < a.N ? n_base + r : a.N - 1;
        boff[i] = (uint32_t)(2 * ((a.n0 + col + a.N_total * batch) * K + 8 * ((lane & 7) ^ (r & 7))));
    }
    // the tokens' metadata of a super-block, also straight to LDS: bsums (f16
    // from the quantize pass), wave w tokens 32 w .. + 31, lane l token
    // 32 w + l / 2, bsums 8 (l & 1) .. + 7; scales, waves w < NW / 2, 64 tokens each
    uint32_t bsoff, dxoff;
    {
        const int r = 32 * wave + (lane >> 1);
        const int64_t col = n_base + r < a.N ? n_base + r : a.N - 1;
        bsoff = (uint32_t)(2 * ((a.n0 + col + a.N_total * batch) * (K / 16) + 8 * (lane & 1)));
        const int rd = 64 * (wave % (NW / 2)) + lane;
        const int64_t cold = n_base + rd < a.N ? n_base + rd : a.N - 1;
        dxoff = (uint32_t)(4 * (a.n0 + cold + a.N_total * batch) * nsb);
    }
    // stage `stage`'s activation codes into tile b
    auto load_b = [&](auto bc, int64_t stage) {
        _Float16(&Bt)[BN][GBK] = btile(bc);
        const uint32_t soff = (uint32_t)(2 * ((stage >> 2) * QKK + 64 * (stage & 3)));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void *)&Bt[8 * (4 * wave + i)][0], 16, boff[i], soff, 0, 0);
    };
    // super-block sb's bsums and token scales (single-buffered: issued at the
    // super-block's first stage, after the previous finalize passed a barrier)
    auto load_meta = [&](int64_t sb) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rbs, (lds_void *)&sBsum[32 * wave][0], 16, bsoff, (uint32_t)(32 * sb), 0, 0);
        if (wave < NW / 2)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rdx, (lds_void *)&sdB[64 * wave], 4, dxoff, (uint32_t)(4 * sb), 0, 0);
    };
    auto fetch = [&](int64_t stage, StageRegs<CB> &r) {
        const uint8_t *blk = wrow + (stage >> 2) * SB;
        r.hdr = ldg16(blk);
        ldg_codes<CB>(r.wq, blk + QS + 32 * (stage & 3) + CB * q);
        if constexpr (Q5) ldg_codes<CB>(r.qh, blk + 16 + CB * q);
    };
    // the current super-block's 8 sub-block scales (bytes), from its header
    uint32_t scw[2] = {0, 0};
    // a super-block's header: its scales to scw; d, dmin and the mins to LDS
    auto header = [&](int64_t stage, const uint4 &hdr) {
        uint32_t mv[2] = {0, 0};
        scw[0] = scw[1] = 0;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            int sc, mn;
            q4k_sm_g(s, hdr.y, hdr.z, hdr.w, sc, mn);
            scw[s >> 2] |= (uint32_t)sc << (8 * (s & 3));
            mv[s >> 2] |= (uint32_t)mn << (8 * (s & 3));
        }
        if (q == 0) {
            const int mb = (int)((stage >> 2) & 1);
            sdA[mb][srow] = h2f((uint16_t)(hdr.x & 0xffff));
            sdminA[mb][srow] = h2f((uint16_t)(hdr.x >> 16));
            *(uint2 *)&sAmin[mb][srow][0] = make_uint2(mv[0], mv[1]);
        }
    };
    // stage `stage`'s weight codes (sc * q in f16) into tile b
    auto commit = [&](auto bc, int64_t stage, const StageRegs<CB> &r) {
        _Float16(&At)[GBM][GBK] = sA[decltype(bc)::value];
        const int j = (int)(stage & 3);
        const int sclo = (int)((scw[j >> 1] >> (16 * (j & 1))) & 0xff);
        const int schi = (int)((scw[j >> 1] >> (16 * (j & 1) + 8)) & 0xff);
        const _Float16 fl = (_Float16)sclo, fh = (_Float16)schi;
        const half2_t sl2 = {fl, fl}, sh2 = {fh, fh};
        const half2_t nsl2 = {(_Float16)(-1024 * sclo), (_Float16)(-1024 * sclo)};
        const half2_t nsh2 = {(_Float16)(-1024 * schi), (_Float16)(-1024 * schi)};
        uint32_t lo[CB / 2], hi[CB / 2];
#pragma unroll
        for (int i = 0; i < CB / 4; ++i) {
            uint32_t cl = r.wq[i] & 0x0f0f0f0fu, ch = (r.wq[i] >> 4) & 0x0f0f0f0fu;
            if constexpr (Q5) {  // codes 0..31: (1024 + n) stays exact in f16
                cl |= ((r.qh[i] >> (2 * j)) & 0x01010101u) << 4;
                ch |= ((r.qh[i] >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            nib4_to_h(cl, sl2, nsl2, lo[2 * i], lo[2 * i + 1]);
            nib4_to_h(ch, sh2, nsh2, hi[2 * i], hi[2 * i + 1]);
        }
        // low nibbles: k = CB q + i (chunks CB q / 8 ..); high nibbles: k = 32 + CB q + i
        _Float16 *ar = At[srow];
#pragma unroll
        for (int c = 0; c < CB / 8; ++c) {
            *(uint4 *)(ar + swz(srow, CB * q / 8 + c)) = make_uint4(lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]);
            *(uint4 *)(ar + swz(srow, 4 + CB * q / 8 + c)) = make_uint4(hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]);
        }
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
    // Pipeline over two stage buffers: during stage st, the weight codes of
    // stage st + 1 (fetched to registers during stage st - 1) are converted
    // into its tile, stage st + 1's activation codes are issued straight to
    // LDS and stage st + 2's weight codes to the register set stage st used;
    // so every load has a whole stage to land, and the only waits are at the
    // stage's two ends. Every share is a whole number of super-blocks
    // (g0 % 4 == 0) and the loop runs two stages an iteration, so a stage's
    // buffer and register set, (st - g0) & 1, are static.
    constexpr int NF = Q5 ? 2 : 1;  // code loads of a fetch (its header load comes first)
    StageRegs<CB> pre[2];
    if (g0 < stages) {
        load_b(IC<0>{}, g0);
        load_meta(sb0);
        fetch(g0, pre[0]);
        fetch(g0 + 1, pre[1]);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): everything above landed
        header(g0, pre[0].hdr);
        commit(IC<0>{}, g0, pre[0]);
    }
    lds_barrier();
    auto stage = [&](auto bc, int64_t st) {
        constexpr int b = decltype(bc)::value, b1 = b ^ 1;  // (st - g0) & 1
        // stage st + 1's weight codes (fetched during stage st - 1) landed
        __builtin_amdgcn_s_waitcnt(0x0f70);
        // past the share's end: the last stage again into the free buffers
        // and the set, so every stage issues the same loads
        const int64_t last = stages - 1;
        const int64_t s1 = st + 1 < stages ? st + 1 : last;
        if (((st + 1) & 3) == 0 && st + 1 < stages) header(st + 1, pre[b1].hdr);
        if ((st & 3) == 0 && st != g0) load_meta(st >> 2);
        // one block the scheduler can interleave: the next stage's weight
        // conversion and loads between this stage's products (S starts each
        // super-block at zero: the finalize clears it)
        commit(IC<b1>{}, s1, pre[b1]);
        load_b(IC<b1>{}, s1);
        // the weight loads stay behind the activation loads (the waits count
        // them as the last ones issued); everything but vector memory
        // instructions may still move across
        __builtin_amdgcn_sched_barrier(0x078f);
        fetch(st + 2 < stages ? st + 2 : last, pre[b]);
#pragma unroll
        for (int t = 0; t < GBK / 16; ++t) {
            half8_t av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra = 64 * wm + 32 * i + lr, rb = 64 * wn + 32 * i + lr;
                av[i] = *(const half8_t *)&sA[b][ra][swz(ra, 2 * t + lg)];
                bv[i] = *(const half8_t *)&btile(bc)[rb][swz(rb, 2 * t + lg)];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int jn = 0; jn < 2; ++jn)
                    S[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[jn], S[i][jn], 0, 0, 0);
        }
        if ((st & 3) == 3) {
            // super-block finalize: acc += dy * (d * S - dmin * Mn)
            const int mb = (int)((st >> 2) & 1);
            // Mn operands: A'[m][k] = m_{k/2}, k = 8g..8g+7 -> mins 4g..4g+3, each twice
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                half8_t am;
                const uint32_t mw = *(const uint32_t *)&sAmin[mb][64 * wm + 32 * i + lr][4 * lg];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const _Float16 h = (_Float16)(float)((mw >> (8 * e)) & 0xff);
                    am[2 * e] = h;
                    am[2 * e + 1] = h;
                }
#pragma unroll
                for (int jn = 0; jn < 2; ++jn) {
                    const half8_t bm = *(const half8_t *)&sBsum[64 * wn + 32 * jn + lr][8 * lg];
                    const float16_t Mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, (float16_t){}, 0, 0, 0);
                    const float dy = sdB[64 * wn + 32 * jn + lr];
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int mr = 64 * wm + 32 * i + 8 * qq + 4 * lg;
                        const float4 d4 = *(const float4 *)&sdA[mb][mr];
                        const float4 dm4 = *(const float4 *)&sdminA[mb][mr];
                        const float dv[4] = {d4.x, d4.y, d4.z, d4.w}, dmv[4] = {dm4.x, dm4.y, dm4.z, dm4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * qq + e;
                            acc[i][jn][r] += dy * (dv[e] * S[i][jn][r] - dmv[e] * Mn[r]);
                        }
                    }
                    S[i][jn] = (float16_t){};
                }
            }
        }
        // stage st + 1's activation codes landed: issued after them, stage
        // st + 2's code loads may still fly (its header load, issued before
        // them, is waited for: odd stages drop it as unused)
        __builtin_amdgcn_s_waitcnt(0x0f70 | NF);
        lds_barrier();
    };
    for (int64_t st = g0; st < stages; st += 2) {
        stage(IC<0>{}, st);
        stage(IC<1>{}, st + 1);
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
            for (int qq = 0; qq < 4; ++qq) {
                const int64_t m = m_base + 64 * wm + 32 * i + 8 * qq + 4 * lg;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (m + e < a.M) drow[m + e - moff] = acc[i][jn][4 * qq + e];
            }
        }
}

// Token tile of the q4_K / q5_K GEMM: 256 (8 waves) above 128 tokens, else 128.
static int gemm_nw(int64_t N) { return N > 128 ? 8 : 4; }

int gemm_ksplit(int wtype, int64_t M, int64_t N, int64_t K, int64_t batches) {
    if (!has_gemm(wtype) || N <= 16) return 1;
    constexpr int64_t CUS = 256;  // MI355X
    // workgroups that fit the CUs at once: two 128 x 128 tiles a CU (q8_0 /
    // q4_0, and q4_K / q5_K up to 128 tokens), one 128 x 256 tile (q4_K / q5_K above)
    const bool wide = (wtype == TLH_TYPE_Q4_K || wtype == TLH_TYPE_Q5_K) && gemm_nw(N) == 8;
    const int64_t bn = wide ? 256 : 128, slots = wide ? CUS : 2 * CUS;
    const int64_t tiles = (N + bn - 1) / bn * ((M + 127) / 128) * batches;
    if (tiles >= CUS) return 1;
    // stages of 256 elements (k-quants: a super-block; q8_0 / q4_0: 2 stages of 4 blocks)
    const int64_t units = (K + 255) / 256, min_units = 4;
    // (one 128 x 256 tile a CU: split only as far as one round holds, the
    // reduce launch costs more than the CUs a round leaves idle)
    int64_t ks = wide ? slots / tiles : (slots + tiles - 1) / tiles;
    if (ks > units / min_units) ks = units / min_units;
    if (ks > 16) ks = 16;
    return ks > 1 ? (int)ks : 1;
}

int64_t gemm_partial_bytes(int wtype, int64_t M, int64_t N, int64_t K, int64_t batches) {
    const int ks = gemm_ksplit(wtype, M, N, K, batches);
    return ks > 1 ? (int64_t)ks * batches * N * M * 4 : 0;
}

static tlh_status launch_gemm_q4k(const MatmulArgs &a, int ks, hipStream_t stream) {
    const int64_t batches = a.ne12 * a.ne13;
    // the kernel addresses the f16 activation codes by 32-bit byte offsets
    if ((double)a.N_total * (double)batches * (double)a.K * 2.0 >= 4294967296.0)
        return set_error(TLH_UNSUPPORTED, "gemm: activation codes of %lld x %lld x %lld exceed 4 GiB",
                         (long long)a.N_total, (long long)batches, (long long)a.K);
    const int nw = gemm_nw(a.N);
    const dim3 grid((unsigned)((a.N + 32 * nw - 1) / (32 * nw)), (unsigned)((a.M + GBM - 1) / GBM), (unsigned)(batches * ks));
    const bool q4 = a.wtype == TLH_TYPE_Q4_K;
    if (nw == 8 && q4) hipLaunchKernelGGL((k_gemm_q4k<TLH_TYPE_Q4_K, 8>), grid, dim3(512), 0, stream, a);
    else if (nw == 8) hipLaunchKernelGGL((k_gemm_q4k<TLH_TYPE_Q5_K, 8>), grid, dim3(512), 0, stream, a);
    else if (q4) hipLaunchKernelGGL((k_gemm_q4k<TLH_TYPE_Q4_K, 4>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((k_gemm_q4k<TLH_TYPE_Q5_K, 4>), grid, dim3(256), 0, stream, a);
    return check_launch("gemm_q4k");
}

tlh_status launch_gemm_epi(const MatmulArgs &a, const GemvEpi &ep, hipStream_t stream) {
    const int ks = gemm_ksplit(a.wtype, a.M, a.N, a.K, a.ne12 * a.ne13);
    if ((a.wtype != TLH_TYPE_Q4_K && a.wtype != TLH_TYPE_Q5_K) || ks < 2 || !a.part)
        return set_error(TLH_UNSUPPORTED, "gemm: the store epilogue rides on the reduce of a K-split q4_K / q5_K GEMM");
    tlh_status st = reduce_epi_check(a, ep);
    if (st == TLH_OK) st = launch_gemm_q4k(a, ks, stream);
    return st != TLH_OK ? st : launch_partial_reduce_epi(a, ks, ep, stream);
}

tlh_status launch_gemm(const MatmulArgs &a, hipStream_t stream) {
    const int64_t batches = a.ne12 * a.ne13;
    const int ks = gemm_ksplit(a.wtype, a.M, a.N, a.K, batches);
    if (ks > 1 && !a.part) return set_error(TLH_INVALID, "gemm: a K split of %d needs a partials buffer", ks);
    if (a.wtype == TLH_TYPE_Q8_0 || a.wtype == TLH_TYPE_Q4_0) {
        const tlh_status st = launch_gemm_q8(a, ks, stream);
        return st != TLH_OK || ks == 1 || a.keep_part ? st : launch_partial_reduce(a, ks, stream);
    }
    if (a.wtype == TLH_TYPE_Q4_K || a.wtype == TLH_TYPE_Q5_K) {
        const tlh_status st = launch_gemm_q4k(a, ks, stream);
        return st != TLH_OK || ks == 1 || a.keep_part ? st : launch_partial_reduce(a, ks, stream);
    }
    if (a.keep_part) return set_error(TLH_UNSUPPORTED, "gemm: no kept partials for weight type %d", a.wtype);
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

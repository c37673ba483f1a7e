// Activation quantizers (f32 -> Q8_0 / Q8_1 / Q8_K, bit-exact with the CPU
// backend's from_float) and weight dequantizers (every weight type -> f32,
// bit-exact with ggml's dequantize_row_*), for gfx950.
//
// Bit-exactness rules kept here: no a*b+c contraction where the reference
// rounds twice (#pragma clang fp contract(off)), IEEE-correct f32 division
// (hipcc's default), f16 conversion by v_cvt_f16_f32 (round to nearest even,
// denormals kept), roundf = ties away from zero, rintf = ties to even.
#include "kernels.hpp"


namespace tlh {

// ------------------------------------------------------------------ Q8_0
// quantize_row_q8_0_ref (vendor/ggml/src/ggml-quants.c:276-297), reached on
// x86 without AVX through quantize_row_q8_0 (arch/x86/quants.c:395-398).
// One lane per element, 32 lanes per block (two blocks per wave64):
// amax over the block, d = amax/127, f16(d) stored, codes roundf(x * (1/d))
// with the multiplier taken from the unrounded f32 d.
// `rows` rows of x (stride x_row_bytes) become activation rows row_off.. of
// an output holding total_rows rows.
// Q81: quantize_row_q8_1_ref (ggml-quants.c:302-335; the x86 entry without
// AVX, arch/x86/quants.c:400-501): the same d and codes, plus s = f16(code
// sum * the unrounded d) (block_q8_1: d, s, codes; split layout: s as f32 in
// the sum slot).
template <bool GGML_LAYOUT, bool Q81>
__global__ void __launch_bounds__(256) k_quantize_q8_0(const float *__restrict__ x, int64_t K, int64_t rows,
                                                       int64_t x_row_bytes, void *__restrict__ out, int64_t row_off,
                                                       int64_t total_rows, bool f16) {
#pragma clang fp contract(off)
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = K * rows;
    if (gid >= total) return;  // K % 32 == 0, so whole 32-lane groups exit together
    const int64_t row = gid / K;
    const int64_t col = gid - row * K;
    const float v = *(const float *)((const char *)x + row * x_row_bytes + col * 4);
    float amax = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)roundf(v * id);
    const uint16_t dh = f2h(d);
    const int lane32 = threadIdx.x & 31;
    const int64_t blk = col / QK;
    const int64_t orow = row + row_off;
    int s = q;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) s += __shfl_xor(s, m, 32);
    const uint16_t sh = f2h((float)s * d);  // q8_1 only
    if (GGML_LAYOUT) {
        constexpr int BB = Q81 ? Q8_1_BYTES : Q8_0_BYTES, CO = Q81 ? 4 : 2;
        uint8_t *b = (uint8_t *)out + orow * (K / QK) * BB + blk * BB;
        b[CO + lane32] = (uint8_t)(int8_t)q;
        if (lane32 == 0) {
            *(uint16_t *)b = dh;
            if (Q81) *(uint16_t *)(b + 2) = sh;
        }
    } else {
        const ActLayout L = act_layout(Q81 ? TLH_TYPE_Q8_1 : TLH_TYPE_Q8_0, K, total_rows, f16);
        int8_t *qs = (int8_t *)out + L.qs_off;
        qs[orow * K + col] = (int8_t)q;
        if (f16) ((_Float16 *)((char *)out + L.q16_off))[orow * K + col] = (_Float16)q;
        if (lane32 == 0) {
            ((float *)((char *)out + L.d_off))[orow * (K / QK) + blk] = h2f(dh);
            ((int32_t *)((char *)out + L.sum_off))[orow * (K / QK) + blk] = Q81 ? __float_as_int(h2f(sh)) : s;
        }
    }
}

// ------------------------------------------------------------------ Q8_K
// quantize_row_q8_K_ref (ggml-quants.c:2768-2804), the x86 entry
// (arch/x86/quants.c:505-507). One wave per 256-element block, four
// consecutive elements per lane, quantized by q8K_waves (the arithmetic the
// fused norm / SwiGLU kernels share).
template <bool GGML_LAYOUT>
__global__ void __launch_bounds__(256) k_quantize_q8_K(const float *__restrict__ x, int64_t K, int64_t rows,
                                                       int64_t x_row_bytes, void *__restrict__ out, int64_t row_off,
                                                       int64_t total_rows, bool f16) {
#pragma clang fp contract(off)
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t nblk = K / QKK;
    if (wave >= nblk * rows) return;
    const int64_t row = rows == 1 ? 0 : wave / nblk;  // one row (a decode step): no 64-bit division
    const int64_t blk = wave - row * nblk;
    const float *src = (const float *)((const char *)x + row * x_row_bytes) + blk * QKK + 4 * lane;
    float v[1][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[0][i] = src[i];
    uint32_t packed[1];
    int psum[1];
    float d[1];
    q8K_waves<1>(v, lane, packed, psum, d);
    const int64_t orow = row + row_off;
    if (GGML_LAYOUT) {
        uint8_t *b = (uint8_t *)out + orow * nblk * Q8_K_BYTES + blk * Q8_K_BYTES;
        *(uint32_t *)(b + 4 + 4 * lane) = packed[0];
        if ((lane & 3) == 0) *(int16_t *)(b + 4 + QKK + 2 * (lane >> 2)) = (int16_t)psum[0];
        if (lane == 0) *(float *)b = d[0];
    } else {
        q8K_store_split((char *)out, act_layout(TLH_TYPE_Q8_K, K, total_rows, f16), K, orow, blk, lane, packed[0],
                        psum[0], d[0], f16);
    }
}

// ------------------------------------------------------------- dequantize
// One thread per output element; integer codes convert exactly, so the only
// roundings are the reference's own: q4_0 ((q-8)*d, ggml-quants.c:459-476),
// q8_0 (q*d, :553-565), q4_K ((d*sc)*q - (dmin*m), :1529-1550), q6_K ((d*sc)*q,
// :1939-1968).
template <int WT>
__global__ void __launch_bounds__(256) k_dequantize(const uint8_t *__restrict__ w, int64_t K, int64_t rows,
                                                    int64_t w_row_bytes, float *__restrict__ y) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= K * rows) return;
    const int64_t row = gid / K;
    const int64_t col = gid - row * K;
    y[gid] = dequant_elem<WT>(w + row * w_row_bytes, col);
}

// --------------------------------------------------------------- launchers
static inline unsigned grid_for(int64_t threads, int per_block) {
    return (unsigned)((threads + per_block - 1) / per_block);
}

tlh_status launch_quantize_act(int wtype, const float *x, int64_t K, int64_t rows, int64_t x_row_bytes, void *out,
                               bool ggml_layout, int64_t row_off, int64_t total_rows, bool f16, hipStream_t stream) {
    if (rows == 0 || K == 0) return TLH_OK;
    if (vec_dot_type(wtype) == TLH_TYPE_Q8_0 || vec_dot_type(wtype) == TLH_TYPE_Q8_1) {
        const unsigned g = grid_for(K * rows, 256);
        const bool q81 = vec_dot_type(wtype) == TLH_TYPE_Q8_1;
        auto kern = ggml_layout ? (q81 ? k_quantize_q8_0<true, true> : k_quantize_q8_0<true, false>)
                                : (q81 ? k_quantize_q8_0<false, true> : k_quantize_q8_0<false, false>);
        hipLaunchKernelGGL(kern, dim3(g), dim3(256), 0, stream, x, K, rows, x_row_bytes, out, row_off, total_rows, f16);
    } else {
        const unsigned g = grid_for((K / QKK) * rows * 64, 256);
        if (ggml_layout)
            hipLaunchKernelGGL(k_quantize_q8_K<true>, dim3(g), dim3(256), 0, stream, x, K, rows, x_row_bytes, out,
                               row_off, total_rows, f16);
        else
            hipLaunchKernelGGL(k_quantize_q8_K<false>, dim3(g), dim3(256), 0, stream, x, K, rows, x_row_bytes, out,
                               row_off, total_rows, f16);
    }
    return check_launch("quantize_act");
}

tlh_status launch_dequantize(int type, const void *w, int64_t K, int64_t rows, int64_t w_row_bytes, float *y,
                             hipStream_t stream) {
    if (rows == 0 || K == 0) return TLH_OK;
    const unsigned g = grid_for(K * rows, 256);
    const uint8_t *wb = (const uint8_t *)w;
    switch (type) {
    case TLH_TYPE_Q4_0:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q4_0>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q8_0:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q8_0>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q4_1:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q4_1>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q5_0:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q5_0>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q5_1:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q5_1>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q4_K:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q4_K>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q5_K:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q5_K>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q6_K:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q6_K>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q2_K:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q2_K>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    case TLH_TYPE_Q3_K:
        hipLaunchKernelGGL(k_dequantize<TLH_TYPE_Q3_K>, dim3(g), dim3(256), 0, stream, wb, K, rows, w_row_bytes, y);
        break;
    default:
        return set_error(TLH_UNSUPPORTED, "dequantize: unsupported type %d", type);
    }
    return check_launch("dequantize");
}

}  // namespace tlh

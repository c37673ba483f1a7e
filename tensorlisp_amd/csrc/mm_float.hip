// GGML_OP_MUL_MAT with f32, f16 or bf16 weights, gfx950.
//
// What ggml's CPU backend computes for these types
// (ggml_compute_forward_mul_mat, ggml-cpu.c:1254-1457, with vec_dot_type the
// weight type itself, ggml-cpu.c:239-319): src1 is converted once to that type
// (f32 -> f16 round-to-nearest-even; f32 -> bf16 round-to-nearest-even with
// NaN kept quiet; a src1 already of that type as is), then every output is
// the dot product of a weight row with a converted src1 row, accumulated in
// f32 (ggml_vec_dot_f16 / _bf16 / _f32; the CPU's own order of the sums
// differs). Every weight and activation value is exact in f32, so the
// products are too; only the accumulation order separates the two.
//
// One workgroup of 4 waves covers 16 weight rows x 8 src1 columns of one
// batch slice: a wave owns 4 rows, each lane a run of K, so a wave reads its
// rows as wide contiguous loads while the 8 columns' runs stay in registers;
// the 32 partial sums per lane meet in DPP wave sums. Aligned rows
// (16-byte rows and strides, K a multiple of 8) move 8 elements per lane per
// step; any other layout runs element by element. Used for attention-shaped
// products (the reference's attn:sdpa path, K and V views of a cache) and
// float weight matrices; none of it is on the quantized decode path.
#include "kernels.hpp"

namespace tlh {

__device__ __forceinline__ float ld_flt(const char *p, int ty) {
    return ty == TLH_TYPE_F32 ? *(const float *)p
           : ty == TLH_TYPE_F16 ? h2f(*(const uint16_t *)p)
                                : bf16_to_f32(*(const uint16_t *)p);
}
// an activation value as the CPU holds it for the dot product: converted to
// the weight type (f16 / bf16) when it arrives as f32
__device__ __forceinline__ float as_dot(float v, int wt, int xt) {
    if (xt != TLH_TYPE_F32 || wt == TLH_TYPE_F32) return v;
    return wt == TLH_TYPE_F16 ? h2f(f2h(v)) : bf16_to_f32(f32_to_bf16(v));
}

// src1 rows -> contiguous rows of the weight type in scratch (the CPU's wdata)
__global__ void __launch_bounds__(256) k_mm_float_convert(const FloatMM f, char *__restrict__ out, int64_t out_row) {
    const int64_t row = blockIdx.y + (int64_t)gridDim.y * blockIdx.z;  // n + N * (i12 + ne12 * i13)
    if (row >= f.N * f.ne12 * f.ne13) return;
    const int64_t n = row % f.N, i12 = (row / f.N) % f.ne12, i13 = row / (f.N * f.ne12);
    const char *xr = f.x + n * f.x_nb1 + i12 * f.x_nb2 + i13 * f.x_nb3;
    char *orow = out + row * out_row;
    const int es = f.wtype == TLH_TYPE_F32 ? 4 : 2;
    const int xs = f.xtype == TLH_TYPE_F32 ? 4 : 2;
    for (int64_t k = blockIdx.x * 256 + threadIdx.x; k < f.K; k += (int64_t)gridDim.x * 256) {
        const float v = as_dot(ld_flt(xr + k * xs, f.xtype), f.wtype, f.xtype);
        if (es == 4) ((float *)orow)[k] = v;
        else if (f.wtype == TLH_TYPE_F16) ((uint16_t *)orow)[k] = f2h(v);  // exact: v is already an f16 value
        else ((uint16_t *)orow)[k] = f32_to_bf16(v);                        // exact likewise
    }
}

// row_shr by 1, 2, 4, 8 (lanes shifted in from outside a row of 16 read 0),
// then the four rows' last lanes: the sum over the 64 lanes, in every lane
template <int CTRL> __device__ __forceinline__ float dpp_shr0(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_f(float v) {
    v += dpp_shr0<0x111>(v);
    v += dpp_shr0<0x112>(v);
    v += dpp_shr0<0x114>(v);
    v += dpp_shr0<0x118>(v);
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 47));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 63));
    return (r0 + r1) + (r2 + r3);
}

constexpr int MMF_ROWS = 4, MMF_COLS = 8;  // per wave; a workgroup is 4 waves (16 rows)

// 8 consecutive elements of type TY at p (16 or 32 bytes, aligned) as f32
template <int TY> __device__ __forceinline__ void ld8(const char *p, float (&v)[8]) {
    if constexpr (TY == TLH_TYPE_F32) {
        const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 16);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
        const uint4 a = *(const uint4 *)p;
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (TY == TLH_TYPE_F16) {
                v[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
                v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
            } else {
                v[2 * i] = __uint_as_float(w[i] << 16);
                v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    }
}

template <int WT, int XT, bool VEC>
__global__ void __launch_bounds__(256) k_mm_float(const FloatMM f) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t batch = blockIdx.z;
    int64_t i12 = 0, i13 = 0;  // batch slice 0 skips the divisions
    const char *W = f.w;
    if (batch != 0) {
        i12 = batch % f.ne12, i13 = batch / f.ne12;
        W += (i12 / f.r2) * f.w_nb2 + (i13 / f.r3) * f.w_nb3;
    }
    const char *X = f.x + i12 * f.x_nb2 + i13 * f.x_nb3;
    const int64_t m0 = (int64_t)blockIdx.x * (4 * MMF_ROWS) + wave * MMF_ROWS;
    const int64_t n0 = (int64_t)blockIdx.y * MMF_COLS;
    constexpr int ES = WT == TLH_TYPE_F32 ? 4 : 2, XS = XT == TLH_TYPE_F32 ? 4 : 2;
    const char *wr[MMF_ROWS];
    const char *xr[MMF_COLS];
#pragma unroll
    for (int r = 0; r < MMF_ROWS; ++r) wr[r] = W + (m0 + r < f.M ? m0 + r : f.M - 1) * f.w_nb1;  // clamped
#pragma unroll
    for (int c = 0; c < MMF_COLS; ++c) xr[c] = X + (n0 + c < f.N ? n0 + c : f.N - 1) * f.x_nb1;
    float acc[MMF_ROWS][MMF_COLS];
#pragma unroll
    for (int r = 0; r < MMF_ROWS; ++r)
#pragma unroll
        for (int c = 0; c < MMF_COLS; ++c) acc[r][c] = 0.0f;
    if constexpr (VEC) {
        for (int64_t k = 8 * (int64_t)lane; k < f.K; k += 512) {
            float xv[MMF_COLS][8];
#pragma unroll
            for (int c = 0; c < MMF_COLS; ++c) {
                ld8<XT>(xr[c] + k * XS, xv[c]);
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[c][e] = as_dot(xv[c][e], WT, XT);
            }
#pragma unroll
            for (int r = 0; r < MMF_ROWS; ++r) {
                float wv[8];
                ld8<WT>(wr[r] + k * ES, wv);
#pragma unroll
                for (int c = 0; c < MMF_COLS; ++c)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[r][c] = __builtin_fmaf(wv[e], xv[c][e], acc[r][c]);
            }
        }
    } else {
        for (int64_t k = lane; k < f.K; k += 64) {
            float xv[MMF_COLS];
#pragma unroll
            for (int c = 0; c < MMF_COLS; ++c) xv[c] = as_dot(ld_flt(xr[c] + k * XS, XT), WT, XT);
#pragma unroll
            for (int r = 0; r < MMF_ROWS; ++r) {
                const float wv = ld_flt(wr[r] + k * ES, WT);
#pragma unroll
                for (int c = 0; c < MMF_COLS; ++c) acc[r][c] = __builtin_fmaf(wv, xv[c], acc[r][c]);
            }
        }
    }
    char *D = (char *)f.d + i12 * f.d_nb2 + i13 * f.d_nb3;
#pragma unroll
    for (int r = 0; r < MMF_ROWS; ++r)
#pragma unroll
        for (int c = 0; c < MMF_COLS; ++c) {
            const float t = wave_sum_f(acc[r][c]);
            if (lane == r * MMF_COLS + c && m0 + r < f.M && n0 + c < f.N)
                *(float *)(D + (n0 + c) * f.d_nb1 + (m0 + r) * 4) = t;
        }
}

static bool aligned16(const void *p, int64_t a, int64_t b, int64_t c) {
    return (((uintptr_t)p | (uintptr_t)a | (uintptr_t)b | (uintptr_t)c) & 15) == 0;
}

template <int WT, int XT>
static void launch_mmf(const FloatMM &f, dim3 grid, bool vec, hipStream_t s) {
    if (vec) hipLaunchKernelGGL((k_mm_float<WT, XT, true>), grid, dim3(256), 0, s, f);
    else hipLaunchKernelGGL((k_mm_float<WT, XT, false>), grid, dim3(256), 0, s, f);
}

tlh_status launch_mm_float(const FloatMM &f, hipStream_t stream) {
    if (f.M == 0 || f.N == 0 || f.ne12 * f.ne13 == 0) return TLH_OK;
    const int64_t gx = (f.M + 15) / 16, gy = (f.N + MMF_COLS - 1) / MMF_COLS, gz = f.ne12 * f.ne13;
    if (gx > INT32_MAX || gy > 65535 || gz > 65535) return set_error(TLH_UNSUPPORTED, "mul_mat (float): grid too large");
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)gz);
    const bool vec = f.K % 8 == 0 && aligned16(f.w, f.w_nb1, f.w_nb2, f.w_nb3) && aligned16(f.x, f.x_nb1, f.x_nb2, f.x_nb3);
    switch (f.wtype * 64 + f.xtype) {
    case TLH_TYPE_F32 * 64 + TLH_TYPE_F32: launch_mmf<TLH_TYPE_F32, TLH_TYPE_F32>(f, grid, vec, stream); break;
    case TLH_TYPE_F16 * 64 + TLH_TYPE_F32: launch_mmf<TLH_TYPE_F16, TLH_TYPE_F32>(f, grid, vec, stream); break;
    case TLH_TYPE_F16 * 64 + TLH_TYPE_F16: launch_mmf<TLH_TYPE_F16, TLH_TYPE_F16>(f, grid, vec, stream); break;
    case TLH_TYPE_BF16 * 64 + TLH_TYPE_F32: launch_mmf<TLH_TYPE_BF16, TLH_TYPE_F32>(f, grid, vec, stream); break;
    case TLH_TYPE_BF16 * 64 + TLH_TYPE_BF16: launch_mmf<TLH_TYPE_BF16, TLH_TYPE_BF16>(f, grid, vec, stream); break;
    default: return set_error(TLH_UNSUPPORTED, "mul_mat: weights %d with activations %d", f.wtype, f.xtype);
    }
    return check_launch("mul_mat_float");
}

tlh_status launch_mm_float_convert(const FloatMM &f, void *out, int64_t out_row, hipStream_t stream) {
    const int64_t rows = f.N * f.ne12 * f.ne13;
    if (rows == 0 || f.K == 0) return TLH_OK;
    const int64_t gx = (f.K + 255) / 256 < 64 ? (f.K + 255) / 256 : 64;
    const int64_t gy = rows < 65535 ? rows : 65535;
    hipLaunchKernelGGL(k_mm_float_convert, dim3((unsigned)gx, (unsigned)gy, (unsigned)((rows + gy - 1) / gy)),
                       dim3(256), 0, stream, f, (char *)out, out_row);
    return check_launch("mul_mat_float_convert");
}

}  // namespace tlh

// The rest of a decoder step on gfx950: the ggml ops around MUL_MAT and
// attention that a tensorlisp program runs per token.
//
// Each kernel computes what ggml's CPU backend computes for the op
// (vendor/ggml/src/ggml-cpu/binary-ops.cpp, unary-ops.cpp, ops.cpp) on ggml
// tensors addressed through their ne/nb (views work unchanged), with the
// parameters the reference's lowering packs for its core kernels
// (crates/kernels/src/cuda/lower.rs:219-500; kernels in
// crates/kernels/src/cuda/native/core.cu). Element types: f32 and f16 data,
// i32/i64 indices; GET_ROWS and CPY also read q4_0, q8_0, q4_K, q5_K and q6_K rows.
//
// Layout on the GPU: rows of ne0 elements. Kernels that map one element per
// thread walk a row per workgroup y-index (row -> i1, i2, i3 decomposed once)
// with consecutive threads on consecutive elements, so contiguous rows are
// read and written in full cache lines; reductions (norms, softmax, argmax)
// give each row one workgroup and reduce in registers, then across waves.
#include <algorithm>

#include "kernels.hpp"

// The CPU backend rounds every product and sum (its x86-64 build has no FMA);
// contracting a*b+c into one fma here would change results in the last bit.
#pragma clang fp contract(off)

namespace tlh {

constexpr int CORE_I32 = 26, CORE_I64 = 27;

__device__ __forceinline__ float ld_f(const char *p, int ty) {
    return ty == TLH_TYPE_F16    ? h2f(*(const uint16_t *)p)
           : ty == TLH_TYPE_BF16 ? bf16_to_f32(*(const uint16_t *)p)
                                 : *(const float *)p;
}
__device__ __forceinline__ void st_f(char *p, int ty, float v) {
    if (ty == TLH_TYPE_F16)
        *(uint16_t *)p = f2h(v);
    else if (ty == TLH_TYPE_BF16)
        *(uint16_t *)p = f32_to_bf16(v);  // ggml_compute_fp32_to_bf16's rounding
    else
        *(float *)p = v;
}
__device__ __forceinline__ int64_t ld_idx(const char *p, int ty) {
    return ty == CORE_I64 ? *(const int64_t *)p : (int64_t)*(const int32_t *)p;
}

struct CoreArgs {
    tlh_op op;
    const char *s0, *s1, *s2;
    char *dst;
    const char *s3;  // ROPE writing rows of a cache: the row index of each token
};

// rows of a tensor: row r -> (i1, i2, i3)
__device__ __forceinline__ void row_coords(int64_t r, const tlh_tensor &t, int64_t &i1, int64_t &i2, int64_t &i3) {
    i1 = r % t.ne[1];
    i2 = (r / t.ne[1]) % t.ne[2];
    i3 = r / (t.ne[1] * t.ne[2]);
}
__device__ __forceinline__ int64_t offs(const tlh_tensor &t, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    return i0 * t.nb[0] + i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}

// grid: (chunks of CORE_CHUNK elements along ne0, rows); 256 threads, 4 elements each
constexpr int CORE_CHUNK = 1024;

// ------------------------------------------------------------------- binary
// binary-ops.cpp: dst = src0 (op) src1 with src1 repeated to src0's shape
// (ggml_can_repeat), in f32.
__device__ __forceinline__ void body_bin(const CoreArgs &a, int64_t bx, int64_t row) {
    const tlh_tensor &x = a.op.t[0], &y = a.op.t[1], &d = a.op.t[4];
    const int code = (int)a.op.x[0];
    if (row >= d.ne[1] * d.ne[2] * d.ne[3]) return;
    int64_t i1, i2, i3;
    row_coords(row, d, i1, i2, i3);
    const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
    const char *yr = a.s1 + offs(y, 0, i1 % y.ne[1], i2 % y.ne[2], i3 % y.ne[3]);
    char *dr = a.dst + offs(d, 0, i1, i2, i3);
    const int64_t e0 = bx * CORE_CHUNK + threadIdx.x;
#pragma unroll
    for (int u = 0; u < CORE_CHUNK / 256; ++u) {
        const int64_t i0 = e0 + 256 * u;
        if (i0 >= d.ne[0]) break;
        const float p = ld_f(xr + i0 * x.nb[0], x.ty);
        const float q = ld_f(yr + (i0 % y.ne[0]) * y.nb[0], y.ty);
        const float r = code == 0 ? p + q : code == 1 ? p - q : code == 2 ? p * q : p / q;
        st_f(dr + i0 * d.nb[0], d.ty, r);
    }
}
__global__ void __launch_bounds__(256) k_core_bin(const CoreArgs a) {
    body_bin(a, blockIdx.x, blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
}

// -------------------------------------------------------------------- unary
// unary-ops.cpp / vec.h per element, in f32. Codes: ggml_unary_op 0..21 and
// the reference's 100 scale (x * s + b), 101 fill, 102 clamp, 103 leaky relu,
// 104 sqr, 105 sqrt, 106 sin, 107 cos, 108 log.
// ggml_gelu_f32 / ggml_gelu_quick_f32 (vec.h:966-1019) as the CPU applies
// them to f32 data: through 64K-entry f16 tables (GGML_GELU_FP16), i.e. x
// rounded to f16, the function of that, rounded to f16 again.
__device__ __forceinline__ float gelu_f16(float h) {
    const float c = 0.044715f, s2pi = 0.79788456080286535587989211986876f;
    return h2f(f2h(0.5f * h * (1.0f + tanhf(s2pi * h * (1.0f + c * h * h)))));
}
__device__ __forceinline__ float gelu_tab(float v) {
    if (v <= -10.0f) return 0.0f;
    if (v >= 10.0f) return v;
    return gelu_f16(h2f(f2h(v)));
}
__device__ __forceinline__ float gelu_quick_tab(float v) {
    const float h = h2f(f2h(v));
    return h2f(f2h(h * (1.0f / (1.0f + expf(-1.702f * h)))));
}

__device__ __forceinline__ float unary_val(int code, float v, float p1, float p2) {
    switch (code) {  // unary-ops.cpp:3-97 op_* and vec.h for the ops.cpp ones
    case 0: return fabsf(v);
    case 1: return (v > 0.f) ? 1.f : ((v < 0.f) ? -1.f : 0.f);
    case 2: return -v;
    case 3: return (v > 0.f) ? 1.f : 0.f;
    case 4: return tanhf(v);
    case 5: return (v > 0.f) ? v : expm1f(v);
    case 6: return (v > 0.f) ? v : 0.f;
    case 7: return 1.f / (1.f + expf(-v));
    case 8: return gelu_tab(v);
    case 9: return gelu_quick_tab(v);
    case 10: return v / (1.0f + expf(-v));  // silu
    case 11: return v * fminf(1.0f, fmaxf(0.0f, (v + 3.0f) / 6.0f));
    case 12: return fminf(1.0f, fmaxf(0.0f, (v + 3.0f) / 6.0f));
    case 13: return expf(v);
    case 14: return expf(v) - 1.0f;
    case 15: return (v > 20.0f) ? v : logf(1.0f + expf(v));  // softplus
    case 16: return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
    case 18: return floorf(v);
    case 19: return ceilf(v);
    case 20: return roundf(v);
    case 21: return truncf(v);
    case 100: return p2 == 0.0f ? v * p1 : v * p1 + p2;  // ggml_vec_scale_f32 / ggml_vec_mad1_f32
    case 101: return p1;
    case 102: {  // MAX(MIN(x, max), min)
        const float t = v < p2 ? v : p2;
        return t > p1 ? t : p1;
    }
    case 103: return ((v > 0.f) ? v : 0.f) + p1 * ((v < 0.f) ? v : 0.f);
    case 104: return v * v;
    case 105: return sqrtf(v);
    case 106: return sinf(v);
    case 107: return cosf(v);
    case 108: return logf(v);
    default: return v;
    }
}

__device__ __forceinline__ void body_unary(const CoreArgs &a, int64_t bx, int64_t row) {
    const tlh_tensor &x = a.op.t[0], &d = a.op.t[4];
    const int code = (int)a.op.x[0];
    const float p1 = __int_as_float((int)a.op.x[1]), p2 = __int_as_float((int)a.op.x[2]);
    if (row >= d.ne[1] * d.ne[2] * d.ne[3]) return;
    int64_t i1, i2, i3;
    row_coords(row, d, i1, i2, i3);
    const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
    char *dr = a.dst + offs(d, 0, i1, i2, i3);
    const int64_t e0 = bx * CORE_CHUNK + threadIdx.x;
#pragma unroll
    for (int u = 0; u < CORE_CHUNK / 256; ++u) {
        const int64_t i0 = e0 + 256 * u;
        if (i0 >= d.ne[0]) break;
        const float v = ld_f(xr + i0 * x.nb[0], x.ty);
        // f16 data reads the CPU's gelu table for every value (no +-10 cut-offs)
        st_f(dr + i0 * d.nb[0], d.ty, code == 8 && x.ty == TLH_TYPE_F16 ? gelu_f16(v) : unary_val(code, v, p1, p2));
    }
}
__global__ void __launch_bounds__(256) k_core_unary(const CoreArgs a) {
    body_unary(a, blockIdx.x, blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
}

// ----------------------------------------------------------------- get_rows
// ops.cpp get_rows: dst [ne0, n_idx, i11, i12] row (i, j, k) = src0 row
// idx[i, j, k] of src0 plane (j, k); quantized rows are dequantized.
template <int ST>
__global__ void __launch_bounds__(256) k_core_get_rows(const CoreArgs a) {
    const tlh_tensor &x = a.op.t[0], &ix = a.op.t[1], &d = a.op.t[4];
    const int64_t row = blockIdx.y + (int64_t)gridDim.y * blockIdx.z;
    if (row >= d.ne[1] * d.ne[2] * d.ne[3]) return;
    int64_t i1, i2, i3;
    row_coords(row, d, i1, i2, i3);
    int64_t r = ld_idx(a.s1 + i1 * ix.nb[0] + i2 * ix.nb[1] + i3 * ix.nb[2], ix.ty);
    r = r < 0 ? 0 : r >= x.ne[1] ? x.ne[1] - 1 : r;  // an index outside src0 reads its nearest row
    const char *xr = a.s0 + r * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
    char *dr = a.dst + offs(d, 0, i1, i2, i3);
    const int64_t e0 = (int64_t)blockIdx.x * CORE_CHUNK + threadIdx.x;
#pragma unroll
    for (int u = 0; u < CORE_CHUNK / 256; ++u) {
        const int64_t i0 = e0 + 256 * u;
        if (i0 >= d.ne[0]) break;
        float v;
        if constexpr (ST == TLH_TYPE_F32 || ST == TLH_TYPE_F16 || ST == TLH_TYPE_BF16)
            v = ld_f(xr + i0 * x.nb[0], ST);
        else
            v = dequant_elem<ST>((const uint8_t *)xr, i0);
        st_f(dr + i0 * d.nb[0], d.ty, v);
    }
}

// ----------------------------------------------------------------- set_rows
// ops.cpp set_rows: src0 row (i, j, k) goes to dst row idx[i, j % n1, k % n2]
// of dst plane (j, k), converted to dst's type.
__device__ __forceinline__ void body_set_rows(const CoreArgs &a, int64_t bx, int64_t row) {
    const tlh_tensor &x = a.op.t[0], &ix = a.op.t[1], &d = a.op.t[4];
    if (row >= x.ne[1] * x.ne[2] * x.ne[3]) return;
    int64_t i1, i2, i3;
    row_coords(row, x, i1, i2, i3);
    const int64_t r = ld_idx(a.s1 + i1 * ix.nb[0] + (i2 % ix.ne[1]) * ix.nb[1] + (i3 % ix.ne[2]) * ix.nb[2], ix.ty);
    if (r < 0 || r >= d.ne[1]) return;  // an index outside dst writes nothing
    const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
    char *dr = a.dst + r * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3];
    const int64_t e0 = bx * CORE_CHUNK + threadIdx.x;
#pragma unroll
    for (int u = 0; u < CORE_CHUNK / 256; ++u) {
        const int64_t i0 = e0 + 256 * u;
        if (i0 >= x.ne[0]) break;
        st_f(dr + i0 * d.nb[0], d.ty, ld_f(xr + i0 * x.nb[0], x.ty));
    }
}
__global__ void __launch_bounds__(256) k_core_set_rows(const CoreArgs a) {
    body_set_rows(a, blockIdx.x, blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
}

// ---------------------------------------------------------------------- cpy
// ops.cpp dup / cpy: element i of src0 in row-major order to element i of dst
// (shapes may differ, element counts are equal), converted; quantized sources
// dequantized (src0 rows of whole blocks).
template <int ST>
__global__ void __launch_bounds__(256) k_core_cpy(const CoreArgs a) {
    const tlh_tensor &x = a.op.t[0], &d = a.op.t[4];
    int64_t i1, i2, i3;
    const int64_t row = blockIdx.y + (int64_t)gridDim.y * blockIdx.z;
    if (row >= x.ne[1] * x.ne[2] * x.ne[3]) return;
    row_coords(row, x, i1, i2, i3);
    const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
    const int64_t e0 = (int64_t)blockIdx.x * CORE_CHUNK + threadIdx.x;
#pragma unroll
    for (int u = 0; u < CORE_CHUNK / 256; ++u) {
        const int64_t i0 = e0 + 256 * u;
        if (i0 >= x.ne[0]) break;
        float v;
        if constexpr (ST == TLH_TYPE_F32 || ST == TLH_TYPE_F16 || ST == TLH_TYPE_BF16)
            v = ld_f(xr + i0 * x.nb[0], ST);
        else
            v = dequant_elem<ST>((const uint8_t *)xr, i0);
        // linear index in src0's logical order -> dst coordinates
        int64_t li = row * x.ne[0] + i0;
        const int64_t j0 = li % d.ne[0];
        li /= d.ne[0];
        const int64_t j1 = li % d.ne[1];
        li /= d.ne[1];
        const int64_t j2 = li % d.ne[2], j3 = li / d.ne[2];
        st_f(a.dst + offs(d, j0, j1, j2, j3), d.ty, v);
    }
}

// ---------------------------------------------------------------------- glu
// ops.cpp ggml_compute_forward_{reglu,geglu,swiglu,geglu_erf,geglu_quick}_f32
// with vec.h's ggml_vec_*glu_f32: y = act(x) * g over nc = ne0 of dst; x and g
// are src0 and src1 (split form) or the two halves of a src0 row (x first
// unless swapped). Codes are ggml_glu_op: 0 reglu, 1 geglu, 2 swiglu,
// 4 geglu_erf, 5 geglu_quick.
__device__ __forceinline__ float glu_val(int code, float x, float g) {
    switch (code) {
    case 0: return (x > 0.f) ? x * g : 0.f;
    case 1: return x <= -10.0f ? 0.0f : x >= 10.0f ? x * g : gelu_f16(h2f(f2h(x))) * g;
    case 2: return swiglu_val(x, g);
    case 4: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)) * g;
    default: return gelu_quick_tab(x) * g;
    }
}

__device__ __forceinline__ void body_glu(const CoreArgs &a, int64_t bx, int64_t row) {
    const tlh_tensor &x = a.op.t[0], &y = a.op.t[1], &d = a.op.t[4];
    const int code = (int)a.op.x[0];
    const bool swapped = a.op.x[1] != 0;
    if (row >= d.ne[1] * d.ne[2] * d.ne[3]) return;
    int64_t i1, i2, i3;
    row_coords(row, d, i1, i2, i3);
    const int64_t nc = d.ne[0];
    const float *xr = (const float *)(a.s0 + offs(x, 0, i1, i2, i3));
    const float *gr;
    if (a.s1) {
        gr = (const float *)(a.s1 + offs(y, 0, i1, i2, i3));
    } else {
        gr = xr + (swapped ? 0 : nc);
        xr += swapped ? nc : 0;
    }
    float *dr = (float *)(a.dst + offs(d, 0, i1, i2, i3));
    const int64_t e0 = bx * CORE_CHUNK + threadIdx.x;
#pragma unroll
    for (int u = 0; u < CORE_CHUNK / 256; ++u) {
        const int64_t i0 = e0 + 256 * u;
        if (i0 >= nc) break;
        dr[i0] = glu_val(code, xr[i0], gr[i0]);
    }
}
__global__ void __launch_bounds__(256) k_core_glu(const CoreArgs a) {
    body_glu(a, blockIdx.x, blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
}

// GLU whose output rows feed a MUL_MAT: the values body_glu computes, stored
// the same way, and quantized into the MUL_MAT's activation scratch in the
// same pass (q8K_waves / q80_quads_store_split: the quantize launch's bytes).
// One wave per 256 elements of a row, four consecutive elements per lane
// (a q8_K super-block, or eight 8-lane q8_0 / q8_1 blocks); row r of dst is
// activation row r. VEC: every row 16-byte aligned (float4 loads / stores).
struct GluQuantArgs {
    CoreArgs c;
    ActQuantOut qo;
    int64_t chunks;  // 256-element chunks per row
};

template <bool VEC>
__global__ void __launch_bounds__(256) k_glu_quantize(const GluQuantArgs a) {
    kernarg_prefetch<(kernarg_lines(sizeof(GluQuantArgs)))>();
    const tlh_tensor &x = a.c.op.t[0], &y = a.c.op.t[1], &d = a.c.op.t[4];
    const int code = (int)a.c.op.x[0];
    const bool swapped = a.c.op.x[1] != 0;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t rows = d.ne[1] * d.ne[2] * d.ne[3];
    if (wave >= rows * a.chunks) return;  // whole waves
    const int64_t row = wave / a.chunks, ch = wave - row * a.chunks;
    int64_t i1, i2, i3;
    row_coords(row, d, i1, i2, i3);
    const int64_t nc = d.ne[0];
    const float *xr = (const float *)(a.c.s0 + offs(x, 0, i1, i2, i3));
    const float *gr;
    if (a.c.s1) {
        gr = (const float *)(a.c.s1 + offs(y, 0, i1, i2, i3));
    } else {
        gr = xr + (swapped ? 0 : nc);
        xr += swapped ? nc : 0;
    }
    float *dr = (float *)(a.c.dst + offs(d, 0, i1, i2, i3));
    const int64_t c0 = 256 * ch + 4 * lane;
    const bool live = c0 < nc;  // whole 8-lane groups: nc is a multiple of 32
    float h[1][4];
    if (live) {
        float xv[4], gv[4];
        if (VEC) {
            const float4 a4 = *(const float4 *)(xr + c0), g4 = *(const float4 *)(gr + c0);
            xv[0] = a4.x, xv[1] = a4.y, xv[2] = a4.z, xv[3] = a4.w;
            gv[0] = g4.x, gv[1] = g4.y, gv[2] = g4.z, gv[3] = g4.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = xr[c0 + e], gv[e] = gr[c0 + e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) h[0][e] = glu_val(code, xv[e], gv[e]);
        if (VEC) {
            *(float4 *)(dr + c0) = make_float4(h[0][0], h[0][1], h[0][2], h[0][3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) dr[c0 + e] = h[0][e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) h[0][e] = 0.0f;
    }
    const ActLayout L = act_layout(a.qo.type, nc, a.qo.rows, a.qo.f16);
    if (a.qo.type == TLH_TYPE_Q8_K) {  // nc % 256 == 0: every lane live
        uint32_t pk[1];
        int ps[1];
        float dd[1];
        q8K_waves<1>(h, lane, pk, ps, dd);
        q8K_store_split((char *)a.qo.out, L, nc, row, ch, lane, pk[0], ps[0], dd[0], a.qo.f16);
    } else {
        const bool lv[1] = {live};
        const int64_t col[1] = {c0};
        if (a.qo.type == TLH_TYPE_Q8_1)
            q80_quads_store_split<1, true>(h, lv, lane, (char *)a.qo.out, L, nc, row, col, a.qo.f16);
        else
            q80_quads_store_split<1, false>(h, lv, lane, (char *)a.qo.out, L, nc, row, col, a.qo.f16);
    }
}

bool glu_quantize_ok(const tlh_op &op, int act_type) {
    const tlh_tensor &x = op.t[0], &d = op.t[4];
    const int be = act_type == TLH_TYPE_Q8_K ? QKK : act_type == TLH_TYPE_Q8_0 || act_type == TLH_TYPE_Q8_1 ? QK : 0;
    return be > 0 && x.ty == TLH_TYPE_F32 && d.ty == TLH_TYPE_F32 && x.nb[0] == 4 && d.nb[0] == 4 &&
           d.ne[0] > 0 && d.ne[0] % be == 0;
}

tlh_status launch_glu_quantize(const tlh_op &op, const void *src0, const void *src1, void *dst, const ActQuantOut &qo,
                               hipStream_t stream) {
    if (!glu_quantize_ok(op, qo.type) || (src1 && (op.t[1].ty != TLH_TYPE_F32 || op.t[1].nb[0] != 4)))
        return set_error(TLH_INVALID, "glu_quantize: operands or row length do not fit activation type %d", qo.type);
    const tlh_tensor &d = op.t[4];
    const int64_t rows = d.ne[1] * d.ne[2] * d.ne[3];
    if (!qo.out || ((uintptr_t)qo.out & 255) || qo.rows != rows)
        return set_error(TLH_INVALID, "glu_quantize: activation scratch");
    if (rows == 0) return TLH_OK;
    GluQuantArgs a;
    a.c.op = op;
    a.c.s0 = (const char *)src0;
    a.c.s1 = (const char *)src1;
    a.c.s2 = nullptr;
    a.c.s3 = nullptr;
    a.c.dst = (char *)dst;
    a.qo = qo;
    a.chunks = (d.ne[0] + 255) / 256;
    // float4 access: the three bases and every row stride 16-byte aligned
    const tlh_tensor *ts[3] = {&op.t[0], &op.t[1], &op.t[4]};
    const void *ps[3] = {src0, src1, dst};
    bool vec = true;
    for (int k = 0; k < 3 && vec; ++k) {
        if (!ps[k]) continue;
        vec = ((uintptr_t)ps[k] & 15) == 0;
        for (int i = 1; i < 4; ++i) vec = vec && ts[k]->nb[i] % 16 == 0;
    }
    if (!src1) vec = vec && (d.ne[0] * 4) % 16 == 0;  // the second half's offset
    const int64_t waves = rows * a.chunks;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (vec) hipLaunchKernelGGL(k_glu_quantize<true>, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(k_glu_quantize<false>, grid, dim3(256), 0, stream, a);
    return check_launch("glu_quantize");
}

// ------------------------------------------------------------ block reduces
// (wave_sum_t and block_sum_t: common.hpp)
__device__ __forceinline__ float block_max_f(float v, float *sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}

// --------------------------------------------------------------------- norm
// ops.cpp rms_norm_f32 (:3795-3840): sum of x*x (f32 products) in double,
// mean = (float)(sum / n), scale = 1/sqrtf(mean + eps), y = x * scale.
// ops.cpp norm_f32 (:3698-3740): mean = (float)sum / n with the sum in double;
// the centred variance as ggml_vec_cvar_f32's x86-64 (SSE2) build forms it
// (vec.cpp): per group of four, ((d0^2 + d1^2) + (d2^2 + d3^2)) in f32 added
// in double, the n % 4 tail element by element, divided by n in double.
// Contiguous f32 rows; one workgroup per row, so only the order of the double
// additions differs from the CPU's.
__global__ void __launch_bounds__(256) k_core_norm(const CoreArgs a) {
    __shared__ double shd[4];
    const tlh_tensor &x = a.op.t[0], &d = a.op.t[4];
    const bool rms = a.op.x[0] != 0;
    const float eps = __int_as_float((int)a.op.x[1]);
    int64_t i1, i2, i3;
    row_coords(blockIdx.x + (int64_t)gridDim.x * blockIdx.y, x, i1, i2, i3);
    const float *xr = (const float *)(a.s0 + offs(x, 0, i1, i2, i3));
    float *dr = (float *)(a.dst + offs(d, 0, i1, i2, i3));
    const int64_t n = x.ne[0];
    float mean = 0.0f;
    double s2 = 0.0;
    if (rms) {
        for (int64_t i = threadIdx.x; i < n; i += 256) s2 += (double)(xr[i] * xr[i]);
    } else {
        double s = 0.0;
        for (int64_t i = threadIdx.x; i < n; i += 256) s += (double)xr[i];
        mean = (float)block_sum_t(s, shd) / (float)n;
        const int64_t n4 = n / 4;
        for (int64_t g = threadIdx.x; g < n4; g += 256) {
            const float *v = xr + 4 * g;  // rows need not be 16-byte aligned
            const float d0 = v[0] - mean, d1 = v[1] - mean, d2 = v[2] - mean, d3 = v[3] - mean;
            s2 += (double)((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3));
        }
        for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += 256) {
            const float v = xr[i] - mean;
            s2 += (double)(v * v);
        }
    }
    const float var = (float)(block_sum_t(s2, shd) / (double)n);
    const float scale = 1.0f / sqrtf(var + eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) dr[i] = (xr[i] - mean) * scale;
}

// ----------------------------------------------------------------- soft_max
// ops.cpp soft_max_f32: v = x * scale + slope * mask, y = exp(v - max) / sum
// (sum in double), slope from ALiBi (m0, m1, n_head_log2) per head i2.
// One workgroup per row.
__global__ void __launch_bounds__(256) k_core_soft_max(const CoreArgs a) {
    __shared__ float shf[4];
    __shared__ double shd[4];
    const tlh_tensor &x = a.op.t[0], &m = a.op.t[1], &d = a.op.t[4];
    const float scale = __int_as_float((int)a.op.x[0]), max_bias = __int_as_float((int)a.op.x[1]);
    const float m0 = __int_as_float((int)a.op.x[2]), m1 = __int_as_float((int)a.op.x[3]);
    const int nhl2 = (int)a.op.x[4];
    int64_t i1, i2, i3;
    row_coords(blockIdx.x + (int64_t)gridDim.x * blockIdx.y, x, i1, i2, i3);
    const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
    const char *mr = a.s1 ? a.s1 + i1 * m.nb[1] + (i2 % m.ne[2]) * m.nb[2] + (i3 % m.ne[3]) * m.nb[3] : nullptr;
    char *dr = a.dst + offs(d, 0, i1, i2, i3);
    float slope = 1.0f;
    if (max_bias > 0.0f) {
        const int h = (int)i2;
        slope = h < nhl2 ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - nhl2) + 1));
    }
    const int64_t n = x.ne[0];
    auto val = [&](int64_t i) {
        float v = ld_f(xr + i * x.nb[0], x.ty) * scale;
        if (mr) v += slope * ld_f(mr + i * m.nb[0], m.ty);
        return v;
    };
    float mx = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, val(i));
    mx = block_max_f(mx, shf);
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) s += (double)expf(val(i) - mx);
    s = block_sum_t(s, shd);
    const float inv = (float)(1.0 / s);
    for (int64_t i = threadIdx.x; i < n; i += 256)
        st_f(dr + i * d.nb[0], d.ty, mx == -INFINITY ? 0.0f : expf(val(i) - mx) * inv);
}

// ------------------------------------------------------------------- argmax
// ops.cpp argmax_f32 / vec.h ggml_vec_argmax_f32: the last index of the
// maximum (max = MAX(max, x); if max == x then idx = i). One workgroup per row.
__global__ void __launch_bounds__(256) k_core_argmax(const CoreArgs a) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const tlh_tensor &x = a.op.t[0], &d = a.op.t[4];
    const int64_t row = blockIdx.x + (int64_t)gridDim.x * blockIdx.y;
    const char *xr = a.s0 + row * x.nb[1];
    float best = -INFINITY;
    int bi = 0;
    for (int64_t i = threadIdx.x; i < x.ne[0]; i += 256) {
        const float v = ld_f(xr + i * x.nb[0], x.ty);
        if (v >= best) {
            best = v;
            bi = (int)i;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > best || (ov == best && oi > bi)) {
            best = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        best = sv[0];
        bi = si[0];
        for (int w = 1; w < 4; ++w)
            if (sv[w] > best || (sv[w] == best && si[w] > bi)) {
                best = sv[w];
                bi = si[w];
            }
        *(int32_t *)(a.dst + row * d.nb[0]) = bi;
    }
}

// Long rows (a vocabulary of logits): the row in chunks over many
// workgroups, each leaving (max, last index of it) in scratch, then one
// workgroup per row folds the chunks in order. Same result as k_core_argmax.
struct ArgmaxPart {
    float v;
    int i;
};
constexpr int ARGMAX_CHUNK = 2048;

__device__ __forceinline__ void argmax_fold(float &best, int &bi, float ov, int oi) {
    if (ov > best || (ov == best && oi > bi)) {
        best = ov;
        bi = oi;
    }
}

__device__ __forceinline__ void argmax_block(float &best, int &bi, float *sv, int *si) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) argmax_fold(best, bi, __shfl_xor(best, o, 64), __shfl_xor(bi, o, 64));
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    best = sv[0];
    bi = si[0];
    for (int w = 1; w < 4; ++w) argmax_fold(best, bi, sv[w], si[w]);
}

__global__ void __launch_bounds__(256) k_argmax_chunks(const CoreArgs a, ArgmaxPart *part, int nchunks) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const tlh_tensor &x = a.op.t[0];
    const int64_t row = blockIdx.y;
    const char *xr = a.s0 + row * x.nb[1];
    const int64_t lo = (int64_t)blockIdx.x * ARGMAX_CHUNK;
    const int64_t hi = lo + ARGMAX_CHUNK < x.ne[0] ? lo + ARGMAX_CHUNK : x.ne[0];
    float best = -INFINITY;
    int bi = (int)lo;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
        const float v = ld_f(xr + i * x.nb[0], x.ty);
        if (v >= best) {
            best = v;
            bi = (int)i;
        }
    }
    argmax_block(best, bi, sv, si);
    if (threadIdx.x == 0) part[row * nchunks + blockIdx.x] = {best, bi};
}

__global__ void __launch_bounds__(256) k_argmax_fold(const CoreArgs a, const ArgmaxPart *part, int nchunks) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int64_t row = blockIdx.x;
    float best = -INFINITY;
    int bi = 0;
    for (int c = threadIdx.x; c < nchunks; c += 256) argmax_fold(best, bi, part[row * nchunks + c].v, part[row * nchunks + c].i);
    argmax_block(best, bi, sv, si);
    if (threadIdx.x == 0) *(int32_t *)(a.dst + row * a.op.t[4].nb[0]) = bi;
}

size_t argmax_split_scratch_bytes(const tlh_op &op) {
    const int64_t nchunks = (op.t[0].ne[0] + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    return (size_t)(op.t[0].ne[1] * nchunks * sizeof(ArgmaxPart));
}

tlh_status launch_argmax_split(const tlh_op &op, const void *x, void *dst, void *scratch, hipStream_t stream) {
    CoreArgs a;
    a.op = op;
    a.s0 = (const char *)x;
    a.s1 = a.s2 = nullptr;
    a.dst = (char *)dst;
    const int64_t rows = op.t[0].ne[1];
    const int nchunks = (int)((op.t[0].ne[0] + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK);
    if (rows == 0 || nchunks == 0) return TLH_OK;
    hipLaunchKernelGGL(k_argmax_chunks, dim3((unsigned)nchunks, (unsigned)rows), dim3(256), 0, stream, a,
                       (ArgmaxPart *)scratch, nchunks);
    hipLaunchKernelGGL(k_argmax_fold, dim3((unsigned)rows), dim3(256), 0, stream, a, (const ArgmaxPart *)scratch,
                       nchunks);
    return check_launch("argmax");
}

// --------------------------------------------------------------------- rope
// ops.cpp rope_flt (:5953-6100; normal mode 0: pairs (2p, 2p+1); neox mode
// 2: (p, p + n_dims/2)) with ggml's YaRN angle (rope_yarn, :5829-5844):
// theta = pos * theta_scale^p / freq_factor, mixed with its interpolation by
// the ramp over [corr0, corr1] when ext_factor != 0; dims past n_dims pass
// through. One thread per pair.
// One token (i2, i3) per block (bx: a chunk of 256 pairs when a row has more),
// every head i1 of it: thread t takes pair t % P of heads t / P, t / P + 256 / P,
// ... (P = pairs per row, at most 256), so the angle's cos / sin -- the
// position times theta_scale^p by repeated products, then cosf / sinf -- is
// formed once per pair and token, not once per head.
__device__ __forceinline__ void body_rope(const CoreArgs &a, int64_t bx, int64_t tok) {
    const tlh_tensor &x = a.op.t[0], &ps = a.op.t[1], &d = a.op.t[4];
    const int n_dims = (int)a.op.x[0], mode = (int)a.op.x[1];
    const float freq_scale = __int_as_float((int)a.op.x[2]), ext_factor = __int_as_float((int)a.op.x[3]);
    const float attn_factor = __int_as_float((int)a.op.x[4]), theta_scale = __int_as_float((int)a.op.x[5]);
    const float corr0 = __int_as_float((int)a.op.x[6]), corr1 = __int_as_float((int)a.op.x[7]);
    const bool has_ff = a.op.x[8] != 0;
    if (tok >= x.ne[2] * x.ne[3]) return;
    const int64_t i2 = tok % x.ne[2], i3 = tok / x.ne[2];
    const int64_t P = x.ne[0] / 2;
    const int64_t per = P < 256 ? P : 256;  // pairs per pass
    const int64_t hstep = 256 / per;          // heads per pass
    const int64_t p = bx * 256 + threadIdx.x % per;
    const int64_t h0 = threadIdx.x / per;
    if (p >= P || h0 >= hstep) return;
    // x9 = 1: the rotated row of token i2 lands in row idx[i2] of a cache whose
    // rows hold every head of a token (the SET_ROWS of the reshaped result)
    const int64_t crow = a.op.x[9] ? ld_idx(a.s3 + i2 * a.op.t[3].nb[0], a.op.t[3].ty) : 0;
    auto dst_row = [&](int64_t i1) {
        return a.op.x[9] ? a.dst + crow * d.nb[1] + i1 * x.ne[0] * d.nb[0] : a.dst + offs(d, 0, i1, i2, i3);
    };
    if (2 * p >= n_dims) {  // past the rotated dims: copy both elements of the pair
        for (int64_t i1 = h0; i1 < x.ne[1]; i1 += hstep) {
            const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
            char *dr = dst_row(i1);
            st_f(dr + 2 * p * d.nb[0], d.ty, ld_f(xr + 2 * p * x.nb[0], x.ty));
            st_f(dr + (2 * p + 1) * d.nb[0], d.ty, ld_f(xr + (2 * p + 1) * x.nb[0], x.ty));
        }
        return;
    }
    const float ff = has_ff ? *(const float *)(a.s2 + p * 4) : 1.0f;
    RopeParams rp;
    rp.n_dims = n_dims, rp.mode = mode, rp.freq_scale = freq_scale, rp.ext_factor = ext_factor;
    rp.attn_factor = attn_factor, rp.theta_scale = theta_scale, rp.corr0 = corr0, rp.corr1 = corr1;
    float cs, sn;
    rope_cs_sn((float)*(const int32_t *)(a.s1 + i2 * ps.nb[0]), p, ff, rp, cs, sn);
    const int64_t ia = mode == 0 ? 2 * p : p;
    const int64_t ib = mode == 0 ? 2 * p + 1 : p + n_dims / 2;
    // heads in groups of eight: the group's loads all go out before its stores
    for (int64_t g0 = h0; g0 < x.ne[1]; g0 += 8 * hstep) {
        float x0[8], x1[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t i1 = g0 + k * hstep;
            if (i1 < x.ne[1]) {
                const char *xr = a.s0 + offs(x, 0, i1, i2, i3);
                x0[k] = ld_f(xr + ia * x.nb[0], x.ty);
                x1[k] = ld_f(xr + ib * x.nb[0], x.ty);
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t i1 = g0 + k * hstep;
            if (i1 < x.ne[1]) {
                char *dr = dst_row(i1);
                st_f(dr + ia * d.nb[0], d.ty, rope_first(x0[k], x1[k], cs, sn));
                st_f(dr + ib * d.nb[0], d.ty, rope_second(x0[k], x1[k], cs, sn));
            }
        }
    }
}
__global__ void __launch_bounds__(256) k_core_rope(const CoreArgs a) {
    body_rope(a, blockIdx.x, blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
}

// ------------------------------------------------------------------ launchers
static dim3 row_grid(int64_t chunks, int64_t rows) {
    // rows over (y, z) so that more than 65535 rows fit
    const int64_t gy = rows < 65535 ? rows : 65535;
    return dim3((unsigned)chunks, (unsigned)gy, (unsigned)((rows + gy - 1) / gy));
}
static dim3 red_grid(int64_t rows) {
    const int64_t gx = rows < 2147483647 ? rows : 2147483647;
    return dim3((unsigned)gx, 1, 1);
}
static int64_t nrows(const tlh_tensor &t) { return t.ne[1] * t.ne[2] * t.ne[3]; }

tlh_status launch_core(int kind, const tlh_op &op, const void *s0, const void *s1, const void *s2, void *dst,
                       hipStream_t stream) {
    CoreArgs a;
    a.op = op;
    a.s0 = (const char *)s0;
    a.s1 = (const char *)s1;
    a.s2 = (const char *)s2;
    a.dst = (char *)dst;
    a.s3 = nullptr;
    const tlh_tensor &x = op.t[0], &d = op.t[4];
    switch (kind) {
    case TLH_CORE_BIN: {
        const int64_t rows = nrows(d);
        if (rows == 0 || d.ne[0] == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_bin, row_grid((d.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows), dim3(256), 0,
                           stream, a);
        break;
    }
    case TLH_CORE_UNARY: {
        const int64_t rows = nrows(d);
        if (rows == 0 || d.ne[0] == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_unary, row_grid((d.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows), dim3(256), 0,
                           stream, a);
        break;
    }
    case TLH_CORE_GET_ROWS: {
        const int64_t rows = nrows(d);
        if (rows == 0 || d.ne[0] == 0) return TLH_OK;
        const dim3 g = row_grid((d.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows);
        switch (x.ty) {
        case TLH_TYPE_F32: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_F32>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_F16: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_F16>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_BF16: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_BF16>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q4_0: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q4_0>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q4_1: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q4_1>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q5_0: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q5_0>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q5_1: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q5_1>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q8_0: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q8_0>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q4_K: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q4_K>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q5_K: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q5_K>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q2_K: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q2_K>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q3_K: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q3_K>, g, dim3(256), 0, stream, a); break;
        default: hipLaunchKernelGGL(k_core_get_rows<TLH_TYPE_Q6_K>, g, dim3(256), 0, stream, a); break;
        }
        break;
    }
    case TLH_CORE_SET_ROWS: {
        const int64_t rows = nrows(x);
        if (rows == 0 || x.ne[0] == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_set_rows, row_grid((x.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows), dim3(256), 0,
                           stream, a);
        break;
    }
    case TLH_CORE_CPY: {
        const int64_t rows = nrows(x);
        if (rows == 0 || x.ne[0] == 0) return TLH_OK;
        const dim3 g = row_grid((x.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows);
        switch (x.ty) {
        case TLH_TYPE_F32: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_F32>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_F16: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_F16>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_BF16: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_BF16>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q4_0: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q4_0>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q4_1: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q4_1>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q5_0: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q5_0>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q5_1: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q5_1>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q8_0: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q8_0>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q4_K: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q4_K>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q5_K: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q5_K>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q2_K: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q2_K>, g, dim3(256), 0, stream, a); break;
        case TLH_TYPE_Q3_K: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q3_K>, g, dim3(256), 0, stream, a); break;
        default: hipLaunchKernelGGL(k_core_cpy<TLH_TYPE_Q6_K>, g, dim3(256), 0, stream, a); break;
        }
        break;
    }
    case TLH_CORE_NORM: {
        const int64_t rows = nrows(x);
        if (rows == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_norm, red_grid(rows), dim3(256), 0, stream, a);
        break;
    }
    case TLH_CORE_SOFT_MAX: {
        const int64_t rows = nrows(x);
        if (rows == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_soft_max, red_grid(rows), dim3(256), 0, stream, a);
        break;
    }
    case TLH_CORE_ARGMAX: {
        const int64_t rows = x.ne[1];
        if (rows == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_argmax, red_grid(rows), dim3(256), 0, stream, a);
        break;
    }
    case TLH_CORE_GLU: {
        const int64_t rows = nrows(d);
        if (rows == 0 || d.ne[0] == 0) return TLH_OK;
        hipLaunchKernelGGL(k_core_glu, row_grid((d.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows), dim3(256), 0,
                           stream, a);
        break;
    }
    case TLH_CORE_ROPE: {
        const int64_t toks = x.ne[2] * x.ne[3];
        if (nrows(x) == 0 || x.ne[0] < 2) return TLH_OK;
        hipLaunchKernelGGL(k_core_rope, row_grid((x.ne[0] / 2 + 255) / 256, toks), dim3(256), 0, stream, a);
        break;
    }
    default: return set_error(TLH_INVALID, "core: unknown kind %d", kind);
    }
    return check_launch("core");
}

// --------------------------------------------------------- several ops at once
// Up to four independent element-wise ops (BIN, UNARY, SET_ROWS, GLU, ROPE)
// in one launch, for the executor: the flattened grid is cut into each op's
// own (chunk, row) blocks, and every block runs the op's body as its own
// kernel would. Saves the fixed cost of the launches it replaces.
constexpr int MULTI_MAX = 4;
struct MultiArgs {
    int n;
    int kind[MULTI_MAX];
    int64_t start[MULTI_MAX + 1];  // first flattened block of each op
    int64_t gx[MULTI_MAX];         // blocks along a row
    CoreArgs sub[MULTI_MAX];
};

__global__ void __launch_bounds__(256) k_core_multi(const MultiArgs m) {
    kernarg_prefetch<(kernarg_lines(sizeof(MultiArgs)) > 16 ? 16 : kernarg_lines(sizeof(MultiArgs)))>();
    const int64_t b = blockIdx.x + (int64_t)gridDim.x * blockIdx.y;
    int k = 0;
    while (k + 1 < m.n && b >= m.start[k + 1]) ++k;
    const int64_t local = b - m.start[k];
    const int64_t bx = local % m.gx[k], row = local / m.gx[k];
    switch (m.kind[k]) {
    case TLH_CORE_BIN: body_bin(m.sub[k], bx, row); break;
    case TLH_CORE_UNARY: body_unary(m.sub[k], bx, row); break;
    case TLH_CORE_SET_ROWS: body_set_rows(m.sub[k], bx, row); break;
    case TLH_CORE_GLU: body_glu(m.sub[k], bx, row); break;
    default: body_rope(m.sub[k], bx, row); break;
    }
}

// blocks along a row and rows of an element-wise op's grid
static bool ew_grid(int kind, const tlh_op &op, int64_t &gx, int64_t &rows) {
    const tlh_tensor &x = op.t[0], &d = op.t[4];
    switch (kind) {
    case TLH_CORE_BIN: case TLH_CORE_UNARY: case TLH_CORE_GLU:
        gx = (d.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows = nrows(d);
        return true;
    case TLH_CORE_SET_ROWS: gx = (x.ne[0] + CORE_CHUNK - 1) / CORE_CHUNK, rows = nrows(x); return true;
    case TLH_CORE_ROPE: gx = (x.ne[0] / 2 + 255) / 256, rows = x.ne[2] * x.ne[3]; return true;  // blocks: tokens
    default: return false;
    }
}

bool core_multi_kind(int kind) {
    return kind == TLH_CORE_BIN || kind == TLH_CORE_UNARY || kind == TLH_CORE_SET_ROWS || kind == TLH_CORE_GLU ||
           kind == TLH_CORE_ROPE;
}

tlh_status launch_core_multi(int n, const int *kinds, const tlh_op *ops, const void *const (*srcs)[4],
                             void *const *dsts, hipStream_t stream) {
    if (n < 1 || n > MULTI_MAX) return set_error(TLH_INVALID, "core_multi: %d ops", n);
    MultiArgs m;
    m.n = n;
    int64_t total = 0;
    for (int k = 0; k < n; ++k) {
        int64_t gx = 0, rows = 0;
        if (!ew_grid(kinds[k], ops[k], gx, rows)) return set_error(TLH_INVALID, "core_multi: kind %d", kinds[k]);
        m.kind[k] = kinds[k];
        m.start[k] = total;
        m.gx[k] = gx > 0 ? gx : 1;
        total += gx * rows;
        CoreArgs &a = m.sub[k];
        a.op = ops[k];
        a.s0 = (const char *)srcs[k][0];
        a.s1 = (const char *)srcs[k][1];
        a.s2 = (const char *)srcs[k][2];
        a.s3 = (const char *)srcs[k][3];
        a.dst = (char *)dsts[k];
    }
    m.start[n] = total;
    if (total == 0) return TLH_OK;
    const int64_t gxx = total < 65535 ? total : 65535;
    hipLaunchKernelGGL(k_core_multi, dim3((unsigned)gxx, (unsigned)((total + gxx - 1) / gxx)), dim3(256), 0, stream, m);
    return check_launch("core_multi");
}

// ---------------------------------------------------------- norm chains
// [ADD ->] RMS_NORM / NORM -> MUL(weight) in one pass per row, for the
// executor: s = p + q (written: it is read again as the residual), the norm
// of s (or of x without the ADD), times a weight row that repeats over rows.
// Every value is the one the separate BIN, NORM and BIN kernels produce:
// s_i = p_i + q_i, t_i = (s_i - mean) * scale, y_i = t_i * w_i, with the
// same sums (double; the variance in groups of four as k_core_norm forms it).
// f32 rows with unit element stride. op: t0 p (or x), t1 q, t2 w, t3 s,
// t4 y; x0 = 1 for RMS_NORM, x1 eps, x2 = 1 with the ADD.
struct NormChainArgs {
    tlh_op op;
    const float *p, *q, *w;
    float *s, *y;
    ActQuantOut qo;  // qo.type != 0: y also goes to a MUL_MAT's activation scratch
    NormPartials qp;  // qp.chunks > 1: q's rows are sums of a MUL_MAT's K-split partials
};

constexpr int NC_CACHE = 4;  // groups of four a thread keeps in registers: rows up to 4096 in one read
constexpr int64_t NC_SPLIT_ROWS = 64;
constexpr int NC_QCH = 4;  // K-split partial chunks a thread loads at once  // fewer rows than this (quantized) split each row over its 1024-element groups

// The weight row has the norm's length (the executor fuses only then), so
// element i of a row multiplies w[i].
// Split (gridDim.z > 1, rows of n <= 4096 quantized for a MUL_MAT): workgroup
// z of a row still reads the whole row for its sums, but writes s, y and the
// quantized blocks of group z only (elements 1024 z .. + 1023), so a few rows
// spread over 4x the workgroups and the quantization does not lengthen one
// workgroup's path by a whole row's.
template <bool VEC>  // VEC: every row 16-byte aligned with n % 4 == 0, groups move as float4
__global__ void __launch_bounds__(256) k_norm_chain(const NormChainArgs a) {
    kernarg_prefetch<(kernarg_lines(sizeof(NormChainArgs)))>();
    __shared__ double shd[4];
    const tlh_tensor &tp = a.op.t[0], &tq = a.op.t[1], &tw = a.op.t[2], &ts = a.op.t[3], &ty = a.op.t[4];
    const bool rms = a.op.x[0] != 0, add = a.op.x[2] != 0;
    const float eps = __int_as_float((int)a.op.x[1]);
    int64_t i1, i2, i3;
    row_coords(blockIdx.x + (int64_t)gridDim.x * blockIdx.y, tp, i1, i2, i3);
    const float *pr = (const float *)((const char *)a.p + offs(tp, 0, i1, i2, i3));
    const bool qsum = add && a.qp.chunks > 1;  // q from the partials: row r at part + r * ne0
    const int64_t prow = blockIdx.x + (int64_t)gridDim.x * blockIdx.y;
    const float *qr = qsum ? a.qp.part + prow * tp.ne[0]
                      : add ? (const float *)((const char *)a.q + offs(tq, 0, i1, i2, i3)) : nullptr;
    // element i of q: the partials' sum in chunk order from 0, as the chunk-sum
    // kernel forms it (k_gemv_mfma_reduce), or q itself
    auto qval = [&](int i) {
        if (!qsum) return qr[i];
        float v = 0.0f;
        for (int c = 0; c < a.qp.chunks; ++c) v += qr[c * a.qp.cstride + i];
        return v;
    };
    auto qval4 = [&](int i) {
        if (!qsum) return *(const float4 *)(qr + i);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int c = 0; c < a.qp.chunks; ++c) {
            const float4 g = *(const float4 *)(qr + c * a.qp.cstride + i);
            v.x += g.x, v.y += g.y, v.z += g.z, v.w += g.w;
        }
        return v;
    };
    float *sr = add ? (float *)((char *)a.s + offs(ts, 0, i1, i2, i3)) : nullptr;
    const float *wr = (const float *)((const char *)a.w + offs(tw, 0, i1 % tw.ne[1], i2 % tw.ne[2], i3 % tw.ne[3]));
    float *yr = (float *)((char *)a.y + offs(ty, 0, i1, i2, i3));
    const int n = (int)tp.ne[0];
    const int t = threadIdx.x;
    auto value = [&](int i) { return add ? pr[i] + qval(i) : pr[i]; };
    // thread t owns groups of four: elements 4 (t + 256 j) .. + 3; the weight
    // row is fetched with the values, so its latency overlaps the reduction
    float c[NC_CACHE][4], wv[NC_CACHE][4];
    if (VEC && qsum && a.qp.chunks <= NC_QCH) {
        // every load first, from clamped addresses (n % 4 == 0), then the sums:
        // q in chunk order from 0, then p + q
        float4 pv[NC_CACHE], w4[NC_CACHE], qv[NC_CACHE][NC_QCH];
#pragma unroll
        for (int j = 0; j < NC_CACHE; ++j) {
            const int i = min(4 * (t + 256 * j), n - 4);
            pv[j] = *(const float4 *)(pr + i);
            w4[j] = *(const float4 *)(wr + i);
#pragma unroll
            for (int k = 0; k < NC_QCH; ++k)
                qv[j][k] = *(const float4 *)(qr + (int64_t)min(k, a.qp.chunks - 1) * a.qp.cstride + i);
        }
#pragma unroll
        for (int j = 0; j < NC_CACHE; ++j) {
            const bool in = 4 * (t + 256 * j) < n;
            float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int k = 0; k < NC_QCH; ++k)
                if (k < a.qp.chunks) g.x += qv[j][k].x, g.y += qv[j][k].y, g.z += qv[j][k].z, g.w += qv[j][k].w;
            c[j][0] = in ? pv[j].x + g.x : 0.0f, c[j][1] = in ? pv[j].y + g.y : 0.0f;
            c[j][2] = in ? pv[j].z + g.z : 0.0f, c[j][3] = in ? pv[j].w + g.w : 0.0f;
            wv[j][0] = in ? w4[j].x : 0.0f, wv[j][1] = in ? w4[j].y : 0.0f;
            wv[j][2] = in ? w4[j].z : 0.0f, wv[j][3] = in ? w4[j].w : 0.0f;
        }
    } else if constexpr (VEC) {
#pragma unroll
        for (int j = 0; j < NC_CACHE; ++j) {
            const int i = 4 * (t + 256 * j);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f), ww = v;
            if (i < n) {
                v = *(const float4 *)(pr + i);
                if (add) {
                    const float4 g = qval4(i);
                    v = make_float4(v.x + g.x, v.y + g.y, v.z + g.z, v.w + g.w);
                }
                ww = *(const float4 *)(wr + i);
            }
            c[j][0] = v.x, c[j][1] = v.y, c[j][2] = v.z, c[j][3] = v.w;
            wv[j][0] = ww.x, wv[j][1] = ww.y, wv[j][2] = ww.z, wv[j][3] = ww.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NC_CACHE; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 4 * (t + 256 * j) + e;
                c[j][e] = i < n ? value(i) : 0.0f;
                wv[j][e] = i < n ? wr[i] : 0.0f;
            }
    }
    const bool split = gridDim.z > 1;
    const int js = (int)blockIdx.z;  // split: the group this workgroup writes
    auto mine = [&](int j) { return !split || j == js; };
    double s1 = 0.0;
#pragma unroll
    for (int j = 0; j < NC_CACHE; ++j) {
        const int i0 = 4 * (t + 256 * j);
        if (VEC && add && i0 < n && mine(j)) *(float4 *)(sr + i0) = make_float4(c[j][0], c[j][1], c[j][2], c[j][3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + e;
            if (i < n) {
                if (!VEC && add && mine(j)) sr[i] = c[j][e];
                s1 += rms ? (double)(c[j][e] * c[j][e]) : (double)c[j][e];
            }
        }
    }
    for (int i = 4 * 256 * NC_CACHE + 4 * t; i < n; i += 4 * 256)  // rows past the registers
        for (int e = 0; e < 4 && i + e < n; ++e) {
            const float v = value(i + e);
            if (add) sr[i + e] = v;
            s1 += rms ? (double)(v * v) : (double)v;
        }
    float mean = 0.0f, var;
    if (rms) {
        var = (float)(block_sum_t(s1, shd) / (double)n);
    } else {
        mean = (float)block_sum_t(s1, shd) / (float)n;
        double s2 = 0.0;
        auto group = [&](int i, float v0, float v1, float v2, float v3) {
            const float d0 = v0 - mean, d1 = v1 - mean, d2 = v2 - mean, d3 = v3 - mean;
            if (i + 3 < n) {
                s2 += (double)((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3));
            } else {  // the row's tail, element by element
                if (i < n) s2 += (double)(d0 * d0);
                if (i + 1 < n) s2 += (double)(d1 * d1);
                if (i + 2 < n) s2 += (double)(d2 * d2);
            }
        };
#pragma unroll
        for (int j = 0; j < NC_CACHE; ++j) {
            const int i = 4 * (t + 256 * j);
            if (i < n) group(i, c[j][0], c[j][1], c[j][2], c[j][3]);
        }
        for (int i = 4 * 256 * NC_CACHE + 4 * t; i < n; i += 4 * 256)
            group(i, value(i), i + 1 < n ? value(i + 1) : 0.0f, i + 2 < n ? value(i + 2) : 0.0f,
                  i + 3 < n ? value(i + 3) : 0.0f);
        var = (float)(block_sum_t(s2, shd) / (double)n);
    }
    const float scale = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int j = 0; j < NC_CACHE; ++j) {
        const int i0 = 4 * (t + 256 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) c[j][e] = ((c[j][e] - mean) * scale) * wv[j][e];  // y (kept for quantizing)
        if (!mine(j)) continue;
        if (VEC) {
            if (i0 < n) *(float4 *)(yr + i0) = make_float4(c[j][0], c[j][1], c[j][2], c[j][3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (i0 + e < n) yr[i0 + e] = c[j][e];
        }
    }
    if (a.qo.type) {
        // c[j] of wave t / 64 holds elements 1024 j + 256 (t / 64) .. + 255 of
        // the row (n <= 4096: all of it): a q8_K super-block in the quantize
        // launch's lane layout, or four 8-lane q8_0 / q8_1 blocks
        const int64_t row = blockIdx.x + (int64_t)gridDim.x * blockIdx.y;  // = the activation row
        const ActLayout QL = act_layout(a.qo.type, n, a.qo.rows, a.qo.f16);
        const int lane = t & 63, w = t >> 6;
        if (a.qo.type == TLH_TYPE_Q8_K && split) {
#pragma unroll
            for (int j = 0; j < NC_CACHE; ++j) {
                if (j != js) continue;  // uniform
                float cj[1][4] = {{c[j][0], c[j][1], c[j][2], c[j][3]}};
                uint32_t pk[1];
                int ps[1];
                float d[1];
                q8K_waves<1>(cj, lane, pk, ps, d);
                if (1024 * j + 256 * w < n)  // wave-uniform (n % 256 == 0)
                    q8K_store_split((char *)a.qo.out, QL, n, row, 4 * j + w, lane, pk[0], ps[0], d[0], a.qo.f16);
            }
        } else if (a.qo.type == TLH_TYPE_Q8_K) {
            uint32_t pk[NC_CACHE];
            int ps[NC_CACHE];
            float d[NC_CACHE];
            q8K_waves<NC_CACHE>(c, lane, pk, ps, d);
#pragma unroll
            for (int j = 0; j < NC_CACHE; ++j)
                if (1024 * j + 256 * w < n)  // wave-uniform (n % 256 == 0)
                    q8K_store_split((char *)a.qo.out, QL, n, row, 4 * j + w, lane, pk[j], ps[j], d[j], a.qo.f16);
        } else {
            bool live[NC_CACHE];
            int64_t col[NC_CACHE];
#pragma unroll
            for (int j = 0; j < NC_CACHE; ++j) {
                col[j] = 4 * (t + 256 * j);
                live[j] = col[j] < n && mine(j);  // whole 8-lane groups (n % 32 == 0)
            }
            if (a.qo.type == TLH_TYPE_Q8_1)
                q80_quads_store_split<NC_CACHE, true>(c, live, lane, (char *)a.qo.out, QL, n, row, col, a.qo.f16);
            else
                q80_quads_store_split<NC_CACHE, false>(c, live, lane, (char *)a.qo.out, QL, n, row, col, a.qo.f16);
        }
    }
    for (int i = 4 * 256 * NC_CACHE + 4 * t; i < n; i += 4 * 256)
        for (int e = 0; e < 4 && i + e < n; ++e) yr[i + e] = ((value(i + e) - mean) * scale) * wr[i + e];
}

bool norm_chain_quantize_ok(const tlh_op &op, int act_type) {
    const int64_t n = op.t[0].ne[0];
    const int be = act_type == TLH_TYPE_Q8_K ? QKK : act_type == TLH_TYPE_Q8_0 || act_type == TLH_TYPE_Q8_1 ? QK : 0;
    return be > 0 && n > 0 && n % be == 0 && n <= NORM_CHAIN_QUANT_MAX;
}

tlh_status launch_norm_chain(const tlh_op &op, const void *p, const void *q, const void *w, void *s, void *y,
                             hipStream_t stream, const ActQuantOut *qo, const NormPartials *qp) {
    NormChainArgs a;
    a.op = op;
    a.p = (const float *)p;
    a.q = (const float *)q;
    a.w = (const float *)w;
    a.s = (float *)s;
    a.y = (float *)y;
    const int64_t rows = nrows(op.t[0]);
    if (rows == 0) return TLH_OK;
    if (qp && qp->chunks > 1) {
        // the partials hold rows of ne0 contiguous elements; q's own tensor is not read
        if (!op.x[2] || !qp->part || ((uintptr_t)qp->part & 15) || qp->cstride < rows * op.t[0].ne[0] ||
            qp->cstride % 4)
            return set_error(TLH_INVALID, "norm_chain: partial sums for q");
        a.qp = *qp;
    }
    if (qo && qo->type) {
        if (!norm_chain_quantize_ok(op, qo->type) || !qo->out || ((uintptr_t)qo->out & 255) || qo->rows != rows)
            return set_error(TLH_INVALID, "norm_chain: cannot quantize rows of %lld into type %d",
                             (long long)op.t[0].ne[0], qo->type);
        a.qo = *qo;
    }
    const tlh_tensor *ts[5] = {&op.t[0], &op.t[1], &op.t[2], &op.t[3], &op.t[4]};
    const void *ps[5] = {p, q, w, s, y};
    bool vec = op.t[0].ne[0] % 4 == 0;
    for (int k = 0; k < 5 && vec; ++k) {
        if (!ps[k]) continue;
        vec = ((uintptr_t)ps[k] & 15) == 0;
        for (int i = 1; i < 4; ++i) vec = vec && ts[k]->nb[i] % 16 == 0;
    }
    // few rows quantized for a MUL_MAT (a batched decode step): one workgroup
    // per 1024-element group of a row
    dim3 grid = red_grid(rows);
    if (a.qo.type && rows < NC_SPLIT_ROWS && op.t[0].ne[0] <= 4 * 256 * NC_CACHE) grid.z = (unsigned)((op.t[0].ne[0] + 1023) / 1024);
    if (vec)
        hipLaunchKernelGGL(k_norm_chain<true>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(k_norm_chain<false>, grid, dim3(256), 0, stream, a);
    return check_launch("norm_chain");
}

// ------------------------------------------------------------------- fill
// bytes of dst set to one value by a kernel (a caller may capture it in a
// hipGraph, where memset nodes are avoided): 16-byte stores from the first
// aligned address, single bytes before and after it
__global__ void __launch_bounds__(256) k_fill_bytes(uint8_t *__restrict__ dst, uint64_t n, uint32_t v8) {
    const uint64_t head = (16 - ((uintptr_t)dst & 15)) & 15;
    const uint64_t h = head < n ? head : n;
    const uint64_t body = (n - h) / 16;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t w = v8 * 0x01010101u;
    uint4 *b = (uint4 *)(dst + h);
    for (uint64_t i = t; i < body; i += stride) b[i] = make_uint4(w, w, w, w);
    const uint64_t tail0 = h + 16 * body;
    if (t < h) dst[t] = (uint8_t)v8;
    if (t < n - tail0) dst[tail0 + t] = (uint8_t)v8;
}

tlh_status launch_fill(void *dst, int value, size_t bytes, hipStream_t stream) {
    const uint64_t chunks = bytes / 16 + 1;
    const uint64_t blocks = std::min<uint64_t>((chunks + 255) / 256, 4096);
    hipLaunchKernelGGL(k_fill_bytes, dim3((unsigned)blocks), dim3(256), 0, stream, (uint8_t *)dst, (uint64_t)bytes,
                       (uint32_t)(value & 0xff));
    return check_launch("fill");
}

// -------------------------------------------------------------- read floor
// A plain streaming read of `bytes` bytes (16-byte loads, U per lane in
// flight, grid-stride), XOR-folded into a value that is stored only if it
// matches an impossible pattern: the bandwidth / latency floor a kernel
// that must read the same bytes cannot beat.
__device__ unsigned g_read_sink;
template <int U>
__global__ void __launch_bounds__(256) k_read_floor(const uint4 *__restrict__ p, uint64_t n16) {
    uint64_t i = (uint64_t)blockIdx.x * 256 * U + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * 256 * U;
    unsigned acc = 0;
    for (; i < n16; i += stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + (uint64_t)u * 256;
            v[u] = j < n16 ? p[j] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u && threadIdx.x == 0x3ff) g_read_sink = acc;
}

tlh_status launch_read_floor(const void *src, size_t bytes, int grid, int loads, hipStream_t stream) {
    const uint64_t n16 = bytes / 16;
    if (loads == 4)
        hipLaunchKernelGGL(k_read_floor<4>, dim3((unsigned)grid), dim3(256), 0, stream, (const uint4 *)src, n16);
    else
        hipLaunchKernelGGL(k_read_floor<1>, dim3((unsigned)grid), dim3(256), 0, stream, (const uint4 *)src, n16);
    return check_launch("read_floor");
}

}  // namespace tlh

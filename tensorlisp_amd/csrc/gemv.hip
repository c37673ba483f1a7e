// Decode GEMV dispatch for GGML_OP_MUL_MAT with N <= 16 activation columns.
//
// Replaces mm_vec (crates/kernels/src/cuda/native/mm.cu:16-42), which
// dequantized every weight to f32. Here the activations are quantized to the
// weight type's vec_dot type (Q8_0 / Q8_K, bit-exact with the CPU backend)
// and every block is reduced as the CPU's vec_dot does: exact int32 block
// sums, scaled in f32 (ggml-cpu/quants.c:225-258, :451-476, :696-773).
//  * N <= 2 with K a multiple of 64 up to 16384: the register-resident GEMV
//    (gemv_reg.hip), which can also quantize src1 itself (one launch); q4_0
//    weights there need 4-byte aligned pointers and strides;
//  * otherwise (N 3..16, or other K): the int8-MFMA few-column kernel
//    (gemv_mfma.hip) from the scratch a quantize launch filled.
#include "kernels.hpp"

namespace tlh {

// One launch that quantizes src1 itself: N <= 2 and K <= 4096 (longer rows
// run a quantize launch first: every workgroup quantizing the whole column
// costs more than that launch).
bool gemv_fuses_quantize(const MatmulArgs &a, const float *x, int64_t x_row_bytes) {
    int ksplit, upw;
    return x != nullptr && a.N <= 2 && a.K <= 4096 && gemv_reg_geometry(a.K, ksplit, upw) && ((uintptr_t)x & 15) == 0 &&
           (x_row_bytes & 15) == 0 && gemv_reg_weights_ok(a);
}

static bool gemv_uses_reg(const MatmulArgs &a) {
    int ksplit, upw;
    return a.N <= 2 && gemv_reg_geometry(a.K, ksplit, upw) && gemv_reg_weights_ok(a);
}

// N <= 2 with K the register kernel covers: the register-resident GEMV
// (fused quantization when x is given); otherwise the int8-MFMA kernel.
tlh_status launch_gemv(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream) {
    if (a.N < 1 || a.N > 16) return set_error(TLH_INVALID, "gemv: N=%lld outside 1..16", (long long)a.N);
    if (gemv_uses_reg(a)) return launch_gemv_reg(a, x, x_row_bytes, stream);
    if (x != nullptr) return set_error(TLH_INVALID, "gemv: fused quantization needs N <= 2, K <= 4096, K %% 64 == 0");
    return launch_gemv_mfma(a, stream);
}

}  // namespace tlh

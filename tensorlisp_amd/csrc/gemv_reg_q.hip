// Decode GEMV launchers for q4_1, q5_0, q5_1, q2_K and q3_K weights: the
// register-resident kernels of gemv_reg.hpp with plain f32 stores, reading
// src1 from the split scratch or quantizing it in the kernel (q8_1 / q8_0 /
// q8_K). Compiled apart from the other types so the two halves build in
// parallel; these types take no prologue / epilogue fusions.
#include "gemv_reg.hpp"

namespace tlh {

template <int IN>
static tlh_status launch_q(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                           hipStream_t stream) {
    const GemvPro none;
    switch (a.wtype) {
    case TLH_TYPE_Q4_1: return launch_reg_wt<TLH_TYPE_Q4_1, IN, OUT_STORE>(a, x, x_row_bytes, none, ksplit, upw, stream);
    case TLH_TYPE_Q5_0: return launch_reg_wt<TLH_TYPE_Q5_0, IN, OUT_STORE>(a, x, x_row_bytes, none, ksplit, upw, stream);
    case TLH_TYPE_Q5_1: return launch_reg_wt<TLH_TYPE_Q5_1, IN, OUT_STORE>(a, x, x_row_bytes, none, ksplit, upw, stream);
    case TLH_TYPE_Q2_K: return launch_reg_wt<TLH_TYPE_Q2_K, IN, OUT_STORE>(a, x, x_row_bytes, none, ksplit, upw, stream);
    case TLH_TYPE_Q3_K: return launch_reg_wt<TLH_TYPE_Q3_K, IN, OUT_STORE>(a, x, x_row_bytes, none, ksplit, upw, stream);
    default: return set_error(TLH_UNSUPPORTED, "gemv: weight type %d", a.wtype);
    }
}

tlh_status launch_gemv_reg_legacy(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                                  hipStream_t stream) {
    if (!x) return launch_q<IN_SCRATCH>(a, nullptr, 0, ksplit, upw, stream);
    if (a.K > 4096) return set_error(TLH_INVALID, "gemv_reg: in-kernel quantization takes K <= 4096");
    return launch_q<IN_X>(a, x, x_row_bytes, ksplit, upw, stream);
}

}  // namespace tlh

// Decode GEMV launchers for q4_0, q8_0, q4_K, q5_K and q6_K weights (the
// kernels are in gemv_reg.hpp); q4_1 / q5_0 / q5_1 / q2_K / q3_K go to
// gemv_reg_q.hip.
#include "gemv_reg.hpp"

namespace tlh {

// Geometry of the register-resident GEMV for K: waves per row group and
// units per wave (a multiple of 4 so q8_K super-blocks never straddle waves).
bool gemv_reg_geometry(int64_t K, int &ksplit, int &upw) {
    if (K % 64 != 0) return false;
    const int64_t units = K / 64;
    if (units > 256) return false;
    ksplit = units <= 64 ? 1 : (units <= 128 ? 2 : 4);
    upw = (int)(4 * ((units + 4 * ksplit - 1) / (4 * ksplit)));
    return upw <= 64;
}

template <int IN, int OUT>
static tlh_status launch_reg_type(const MatmulArgs &a, const float *x, int64_t x_row_bytes, const GemvPro &pro,
                                  int ksplit, int upw, hipStream_t stream) {
    switch (a.wtype) {
    case TLH_TYPE_Q4_0: return launch_reg_wt<TLH_TYPE_Q4_0, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
    case TLH_TYPE_Q8_0: return launch_reg_wt<TLH_TYPE_Q8_0, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
    case TLH_TYPE_Q4_K: return launch_reg_wt<TLH_TYPE_Q4_K, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
    case TLH_TYPE_Q5_K: return launch_reg_wt<TLH_TYPE_Q5_K, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
    case TLH_TYPE_Q6_K: return launch_reg_wt<TLH_TYPE_Q6_K, IN, OUT>(a, x, x_row_bytes, pro, ksplit, upw, stream);
    default: return set_error(TLH_UNSUPPORTED, "gemv: weight type %d", a.wtype);
    }
}

// q4_0 units are loaded as dwords (WRegs<TLH_TYPE_Q4_0>): every weight
// pointer and stride a multiple of 4 (the row bytes are, for K % 64 == 0).
bool gemv_reg_weights_ok(const MatmulArgs &a) {
    if (a.wtype != TLH_TYPE_Q4_0) return true;
    uintptr_t bits = (uintptr_t)a.w | (uintptr_t)a.w_nb1 | (uintptr_t)a.w_nb2 | (uintptr_t)a.w_nb3;
    for (int sg = 0; sg < a.nseg; ++sg) bits |= (uintptr_t)a.seg_w[sg] | (uintptr_t)a.seg_w_nb1[sg];
    return (bits & 3) == 0;
}

// The kernel's set-up arithmetic is 32-bit.
static bool reg_counts_ok(const MatmulArgs &a) {
    const int64_t lim = (int64_t)1 << 31;
    return a.M < lim && a.ne12 >= 1 && a.ne13 >= 1 && a.r2 >= 1 && a.r3 >= 1 && a.ne12 * a.ne13 < lim &&
           a.ne12 < lim;
}

tlh_status launch_gemv_reg(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream) {
    if (!reg_counts_ok(a)) return set_error(TLH_UNSUPPORTED, "gemv_reg: counts past 2^31");
    int ksplit = 1, upw = 64;
    if (!gemv_reg_geometry(a.K, ksplit, upw)) return set_error(TLH_INVALID, "gemv_reg: K=%lld", (long long)a.K);
    if (reg_plain_type(a.wtype)) return launch_gemv_reg_legacy(a, x, x_row_bytes, ksplit, upw, stream);
    if (!gemv_reg_weights_ok(a)) return set_error(TLH_UNSUPPORTED, "gemv_reg: q4_0 weights need 4-byte alignment");
    const GemvPro none;
    if (!x) return launch_reg_type<IN_SCRATCH, OUT_STORE>(a, nullptr, 0, none, ksplit, upw, stream);
    if (a.K > 4096) return set_error(TLH_INVALID, "gemv_reg: in-kernel quantization takes K <= 4096");
    return launch_reg_type<IN_X, OUT_STORE>(a, x, x_row_bytes, none, ksplit, upw, stream);
}

tlh_status launch_gemv_reg_pro(const MatmulArgs &a, const GemvPro &pro, const float *x, int64_t x_row_bytes,
                               hipStream_t stream) {
    int ksplit = 1, upw = 64;
    if (!reg_counts_ok(a)) return set_error(TLH_UNSUPPORTED, "gemv_reg: counts past 2^31");
    if (!gemv_reg_geometry(a.K, ksplit, upw)) return set_error(TLH_INVALID, "gemv_reg: K=%lld", (long long)a.K);
    if (a.ne12 * a.ne13 != 1) return set_error(TLH_INVALID, "gemv_reg: a prologue / epilogue takes one batch slice");
    if (reg_plain_type(a.wtype)) return set_error(TLH_UNSUPPORTED, "gemv_reg: no fused forms for weight type %d", a.wtype);
    if (!gemv_reg_weights_ok(a)) return set_error(TLH_UNSUPPORTED, "gemv_reg: q4_0 weights need 4-byte alignment");
    const bool glu = pro.glu != nullptr;
    if (glu && (a.nseg != 2 || a.seg_m0[1] != a.seg_m0[2] - a.seg_m0[1]))
        return set_error(TLH_INVALID, "gemv_reg: the SwiGLU epilogue needs two segments of equal rows");
    const bool epi = pro.epi.on != 0;
    if (epi) {
        const GemvEpi &e = pro.epi;
        if (glu || a.N != 1 || a.nseg < 1 || a.K > 4096)
            return set_error(TLH_UNSUPPORTED, "gemv_reg: the store epilogue takes one column of segments, K <= 4096, "
                                              "no SwiGLU");
        bool rope = false;
        for (int sg = 0; sg < a.nseg; ++sg) {
            const int64_t rows = a.seg_m0[sg + 1] - a.seg_m0[sg];
            if (a.seg_m0[sg] % 4 != 0)
                return set_error(TLH_UNSUPPORTED, "gemv_reg: epilogue segments start at multiples of 4");
            if (e.layout[sg] != EPI_F32 && !e.dst[sg]) return set_error(TLH_INVALID, "gemv_reg: epilogue without a destination");
            if ((e.layout[sg] == EPI_CACHE_ROW || e.layout[sg] >= EPI_PAGED_KEY) && !e.idx[sg])
                return set_error(TLH_INVALID, "gemv_reg: epilogue row or slot index missing");
            if (e.rows[sg] >= ((int64_t)1 << 31))
                return set_error(TLH_UNSUPPORTED, "gemv_reg: epilogue cache rows or pool slots past 2^31");
            if (e.layout[sg] >= EPI_PAGED_KEY &&
                (!e.f16[sg] || !e.idx_i64[sg] || e.kvh < 1 || e.hs < 8 || e.hs % 8 || e.bs < 1 ||
                 rows != (int64_t)e.kvh * e.hs))
                return set_error(TLH_UNSUPPORTED, "gemv_reg: paged epilogue geometry");
            if (e.rope[sg]) {
                rope = true;
                if (e.ne0 < 2 || e.ne0 % 2 || e.ne0 > 512 || rows % e.ne0)
                    return set_error(TLH_UNSUPPORTED, "gemv_reg: rotated segments are whole heads of even size");
            }
        }
        if (rope && (!e.pos || e.rp.mode != 0 || e.rp.n_dims % 2 || e.rp.n_dims > e.ne0))
            return set_error(TLH_UNSUPPORTED, "gemv_reg: the epilogue rotates in ROPE mode 0 only");
    }
    MatmulArgs b = a;
    if (glu) b.M = a.seg_m0[1];  // rows of h
    if (pro.p) {
        if (x) return set_error(TLH_INVALID, "gemv_reg: a prologue forms the activation itself");
        if (a.K > 4096) return set_error(TLH_INVALID, "gemv_reg: the norm prologue takes K <= 4096");
        return glu ? launch_reg_type<IN_NORM, OUT_GLU>(b, nullptr, 0, pro, ksplit, upw, stream)
               : epi ? launch_reg_type<IN_NORM, OUT_EPI>(b, nullptr, 0, pro, ksplit, upw, stream)
                     : launch_reg_type<IN_NORM, OUT_STORE>(b, nullptr, 0, pro, ksplit, upw, stream);
    }
    if (!x) return set_error(TLH_INVALID, "gemv_reg: no activation");
    if (a.K > 4096) return set_error(TLH_UNSUPPORTED, "gemv_reg: in-kernel quantization takes K <= 4096");
    return glu ? launch_reg_type<IN_X, OUT_GLU>(b, x, x_row_bytes, pro, ksplit, upw, stream)
           : epi ? launch_reg_type<IN_X, OUT_EPI>(b, x, x_row_bytes, pro, ksplit, upw, stream)
                 : launch_reg_type<IN_X, OUT_STORE>(b, x, x_row_bytes, pro, ksplit, upw, stream);
}

}  // namespace tlh

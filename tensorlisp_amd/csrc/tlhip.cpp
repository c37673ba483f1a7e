// C ABI of the gfx950 executor (include/tlhip.h): validation, dispatch policy
// and error reporting around the kernels. Host code only.
//
// The MUL_MAT policy mirrors Ctx::mul_mat (crates/kernels/src/cuda/lower.rs:543-571)
// in what it accepts and how it reports refusals, and the ggml CPU backend
// (vendor/ggml/src/ggml-cpu/ggml-cpu.c:1254-1457) in what it computes:
// quantize src1 to the vec_dot type, then N <= 2 -> register GEMV,
// N <= 16 -> int8-MFMA few-column kernel, else the GEMM.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "kernels.hpp"

namespace tlh {

static thread_local std::string g_last_error;

tlh_status set_error(tlh_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return s;
}

// Launch labels of this thread, recorded while a trace is on (tlh_program_trace).
static thread_local std::string *g_trace = nullptr;

void launch_trace(std::string *sink) { g_trace = sink; }

constexpr int kMaxDevices = 64;

int device_cus() {
    static std::atomic<int> cus[kMaxDevices];  // 0: not looked up yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;  // MI355X
    }
    int c = cus[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 1) {
            (void)hipGetLastError();
            c = 1;
        }
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

tlh_status check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(TLH_EXECUTION, "%s: launch failed: %s", what, hipGetErrorString(e));
    if (g_trace) {
        if (!g_trace->empty()) g_trace->push_back(',');
        g_trace->append(what);
    }
    return TLH_OK;
}

static tlh_status hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return TLH_OK;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
        return set_error(TLH_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
    if (e == hipErrorOutOfMemory) return set_error(TLH_ALLOC, "%s: %s", what, hipGetErrorString(e));
    return set_error(TLH_EXECUTION, "%s: %s", what, hipGetErrorString(e));
}

// Resolves the no-allocation scratch of tlh_mul_mat_noalloc on the current device (below).
tlh_status noalloc_setup_current_device();

static bool weight_type_ok(int t) {
    return t == TLH_TYPE_Q4_0 || t == TLH_TYPE_Q8_0 || kquant_type(t) || legacy_type(t);
}

static const char *type_name(int t) {
    switch (t) {
    case TLH_TYPE_F32: return "f32";
    case TLH_TYPE_F16: return "f16";
    case TLH_TYPE_Q4_0: return "q4_0";
    case TLH_TYPE_Q4_1: return "q4_1";
    case TLH_TYPE_Q5_0: return "q5_0";
    case TLH_TYPE_Q5_1: return "q5_1";
    case TLH_TYPE_Q8_0: return "q8_0";
    case TLH_TYPE_Q8_1: return "q8_1";
    case TLH_TYPE_BF16: return "bf16";
    case TLH_TYPE_Q2_K: return "q2_K";
    case TLH_TYPE_Q3_K: return "q3_K";
    case TLH_TYPE_Q4_K: return "q4_K";
    case TLH_TYPE_Q5_K: return "q5_K";
    case TLH_TYPE_Q6_K: return "q6_K";
    case TLH_TYPE_Q8_K: return "q8_K";
    default: return "?";
    }
}

// Validates a MUL_MAT descriptor; fills the derived sizes.
struct MulMatShape {
    int64_t K, M, N, ne12, ne13, r2, r3, act_rows;
    int wtype, act_type;
    bool flt = false;  // f32 / f16 / bf16 weights (mm_float.hip)
};

static bool float_type(int t) { return t == TLH_TYPE_F32 || t == TLH_TYPE_F16 || t == TLH_TYPE_BF16; }
static int float_size(int t) { return t == TLH_TYPE_F32 ? 4 : 2; }

static tlh_status check_mul_mat(const tlh_op *op, MulMatShape &s) {
    if (!op) return set_error(TLH_INVALID, "mul_mat: null op");
    const tlh_tensor &a = op->t[0], &b = op->t[1], &d = op->t[4];
    s.flt = float_type(a.ty);
    if (!weight_type_ok(a.ty) && !s.flt)
        return set_error(TLH_UNSUPPORTED,
                         "mul_mat: weights of ggml type %d (%s); have q4_0, q4_1, q5_0, q5_1, q8_0, q2_K, q3_K, q4_K, "
                         "q5_K, q6_K, f32, f16, bf16", a.ty,
                         type_name(a.ty));
    // src1 is f32, or (ggml's vec_dot_type rule) already the f16 / bf16 of f16 / bf16 weights
    if (b.ty != TLH_TYPE_F32 && !(s.flt && a.ty != TLH_TYPE_F32 && b.ty == a.ty))
        return set_error(TLH_UNSUPPORTED, "mul_mat: activations of type %d with weights of type %d", b.ty, a.ty);
    if (d.ty != TLH_TYPE_F32) return set_error(TLH_UNSUPPORTED, "mul_mat: the destination must be f32");
    for (int i = 0; i < 4; ++i)
        if (a.ne[i] < 0 || b.ne[i] < 0 || d.ne[i] < 0) return set_error(TLH_INVALID, "mul_mat: negative extent");
    if (a.ne[0] != b.ne[0] || d.ne[0] != a.ne[1] || d.ne[1] != b.ne[1] || d.ne[2] != b.ne[2] || d.ne[3] != b.ne[3] ||
        a.ne[2] == 0 || a.ne[3] == 0)
        return set_error(TLH_UNSUPPORTED, "mul_mat: inconsistent shapes");
    if (b.ne[2] % a.ne[2] != 0 || b.ne[3] % a.ne[3] != 0)
        return set_error(TLH_UNSUPPORTED, "mul_mat: src1 batch dims are not multiples of src0's");
    s.K = a.ne[0];
    s.M = a.ne[1];
    s.N = b.ne[1];
    s.ne12 = b.ne[2];
    s.ne13 = b.ne[3];
    s.r2 = s.ne12 / a.ne[2];
    s.r3 = s.ne13 / a.ne[3];
    if ((op->x[0] != 0 && op->x[0] != s.r2) || (op->x[1] != 0 && op->x[1] != s.r3))
        return set_error(TLH_INVALID, "mul_mat: broadcast factors x[0]=%lld x[1]=%lld disagree with the shapes",
                         (long long)op->x[0], (long long)op->x[1]);
    if (s.flt) {  // element rows: any strides that keep elements aligned
        const int64_t ea = float_size(a.ty), eb = float_size(b.ty);
        if (a.nb[0] != ea || b.nb[0] != eb)
            return set_error(TLH_UNSUPPORTED, "mul_mat: rows must be contiguous (nb0 = element size)");
        for (int i = 1; i < 4; ++i)
            if (a.nb[i] % ea || b.nb[i] % eb) return set_error(TLH_INVALID, "mul_mat: strides not element-aligned");
        if (d.nb[0] != 4 || (d.nb[1] & 3) || (d.nb[2] & 3) || (d.nb[3] & 3))
            return set_error(TLH_UNSUPPORTED, "mul_mat: dst must be f32 with unit element stride");
        s.wtype = a.ty;
        s.act_type = a.ty;
        s.act_rows = s.N * s.ne12 * s.ne13;
        return TLH_OK;
    }
    const int be = block_elems(a.ty);
    if (s.K % be != 0)
        return set_error(TLH_UNSUPPORTED, "mul_mat: K=%lld is not a multiple of the %s block (%d)", (long long)s.K,
                         type_name(a.ty), be);
    if (a.nb[0] != block_bytes(a.ty))
        return set_error(TLH_UNSUPPORTED, "mul_mat: src0 must not be permuted (nb0=%lld)", (long long)a.nb[0]);
    const int64_t rb = s.K / be * block_bytes(a.ty);
    if (a.nb[1] < rb || (a.nb[1] & 1) || (a.nb[2] & 1) || (a.nb[3] & 1))
        return set_error(TLH_UNSUPPORTED, "mul_mat: src0 row stride %lld (row is %lld bytes, 2-byte aligned)",
                         (long long)a.nb[1], (long long)rb);
    if (b.nb[0] != 4 || (b.nb[1] & 3) || (b.nb[2] & 3) || (b.nb[3] & 3))
        return set_error(TLH_UNSUPPORTED, "mul_mat: src1 must have contiguous f32 rows");
    if (d.nb[0] != 4 || d.nb[1] < 4 * s.M || (d.nb[1] & 3) || d.nb[2] < d.nb[1] || d.nb[3] < d.nb[2])
        return set_error(TLH_UNSUPPORTED, "mul_mat: dst must be f32 with ordered strides");
    s.wtype = a.ty;
    s.act_type = vec_dot_type(a.ty);
    s.act_rows = s.N * s.ne12 * s.ne13;
    return TLH_OK;
}

}  // namespace tlh

using namespace tlh;

// Validates a FLASH_ATTN_EXT descriptor the way Ctx::flash_attn_ext
// (crates/kernels/src/cuda/lower.rs:575-657) and ggml_flash_attn_ext
// (vendor/ggml/src/ggml.c:5402-5444) do, narrowed to what the kernels run:
// f32 q and dst, f16 K/V with 16-byte aligned rows, f16 mask.
static float op_float(int64_t x) {
    const int32_t i = (int32_t)x;
    float f;
    memcpy(&f, &i, sizeof f);
    return f;
}

static tlh_status check_flash_attn(const tlh_op *op, bool has_mask, FlashAttnDesc &d) {
    if (!op) return set_error(TLH_INVALID, "flash_attn_ext: null op");
    const tlh_tensor &q = op->t[0], &k = op->t[1], &v = op->t[2], &m = op->t[3], &o = op->t[4];
    if (q.ty != TLH_TYPE_F32 || o.ty != TLH_TYPE_F32)
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: needs f32 queries and destination");
    if (k.ty != TLH_TYPE_F16 || v.ty != TLH_TYPE_F16)
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: K/V of type %s/%s; have f16", type_name(k.ty),
                         type_name(v.ty));
    if (has_mask && m.ty != TLH_TYPE_F16) return set_error(TLH_UNSUPPORTED, "flash_attn_ext: mask must be f16");
    for (int i = 0; i < 4; ++i)
        if (q.ne[i] < 0 || k.ne[i] < 0 || v.ne[i] < 0 || o.ne[i] < 0 || (has_mask && m.ne[i] < 0))
            return set_error(TLH_INVALID, "flash_attn_ext: negative extent");
    d.D = q.ne[0], d.nq = q.ne[1], d.nh = q.ne[2], d.nb = q.ne[3];
    d.L = k.ne[1], d.nhkv = k.ne[2], d.nbk = k.ne[3], d.DV = v.ne[0];
    if (k.ne[0] != d.D || v.ne[1] != d.L || v.ne[2] != d.nhkv || v.ne[3] != d.nbk || d.nhkv == 0 || d.nbk == 0 ||
        d.nh % d.nhkv != 0 || d.nb % d.nbk != 0)
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: inconsistent head shapes");
    if (o.ne[0] != d.DV || o.ne[1] != d.nh || o.ne[2] != d.nq || o.ne[3] != d.nb)
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: destination must be [DV, heads, queries, batch]");
    if (!flash_attn_head_sizes_ok(d.D, d.DV))
        return set_error(TLH_UNSUPPORTED,
                         "flash_attn_ext: head sizes D=%lld DV=%lld (have D = DV in {32, 40, 64, 72, 80, 96, 112, 128, "
                         "192, 256} and D=192 DV=128)",
                         (long long)d.D, (long long)d.DV);
    if (q.nb[0] != 4 || o.nb[0] != 4 || k.nb[0] != 2 || v.nb[0] != 2 || (has_mask && m.nb[0] != 2))
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: rows must be contiguous (nb[0] = element size)");
    for (int i = 1; i < 4; ++i) {
        if ((k.nb[i] | v.nb[i]) & 15)
            return set_error(TLH_UNSUPPORTED, "flash_attn_ext: K/V strides must be multiples of 16 bytes");
        if ((q.nb[i] | o.nb[i]) & 3 || (has_mask && (m.nb[i] & 1)))
            return set_error(TLH_INVALID, "flash_attn_ext: misaligned q/dst/mask strides");
    }
    if (has_mask) {
        if (m.ne[0] < d.L || m.ne[1] < d.nq || m.ne[2] == 0 || m.ne[3] == 0 || d.nh % m.ne[2] != 0 ||
            d.nb % m.ne[3] != 0)
            return set_error(TLH_UNSUPPORTED, "flash_attn_ext: mask must be [>= keys, >= queries, heads/n, batch/n]");
    }
    for (int i = 0; i < 4; ++i) {
        d.q_nb[i] = q.nb[i], d.k_nb[i] = k.nb[i], d.v_nb[i] = v.nb[i], d.d_nb[i] = o.nb[i];
        d.m_nb[i] = has_mask ? m.nb[i] : 0;
    }
    d.m_ne2 = has_mask ? m.ne[2] : 1;
    d.m_ne3 = has_mask ? m.ne[3] : 1;
    d.scale = op_float(op->x[0]);
    d.max_bias = op_float(op->x[1]);
    d.m0 = op_float(op->x[2]);
    d.m1 = op_float(op->x[3]);
    d.n_head_log2 = (int)op->x[4];
    d.softcap = op_float(op->x[5]);
    if (d.nq > INT32_MAX || d.L > INT32_MAX || d.nh > 65535 || d.nhkv > 65535 || d.nb > 65535)
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: extents beyond the launch grid");
    return TLH_OK;
}

// Validates a core-op node (tlh_core_kind) the way Ctx::lower and its helpers
// (crates/kernels/src/cuda/lower.rs:175-500) refuse nodes, narrowed to what
// core.hip runs: f32/f16 data, i32/i64 indices, quantized rows for GET_ROWS
// and CPY.
static bool data_ty(int t) { return t == TLH_TYPE_F32 || t == TLH_TYPE_F16 || t == TLH_TYPE_BF16; }
static bool idx_ty(int t) { return t == 26 || t == 27; }
static bool same_shape(const tlh_tensor &a, const tlh_tensor &b) {
    for (int i = 0; i < 4; ++i)
        if (a.ne[i] != b.ne[i]) return false;
    return true;
}
static int64_t nel(const tlh_tensor &t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }
static bool rows_of_blocks(const tlh_tensor &t) {  // quantized tensor read by whole blocks
    return weight_type_ok(t.ty) && t.ne[0] % block_elems(t.ty) == 0 && t.nb[0] == block_bytes(t.ty);
}
static bool elem_strides_ok(const tlh_tensor &t) {
    const int64_t es = (t.ty == TLH_TYPE_F16 || t.ty == TLH_TYPE_BF16) ? 2 : t.ty == 27 ? 8 : 4;
    for (int i = 0; i < 4; ++i)
        if (t.nb[i] % es) return false;
    return true;
}

static tlh_status check_core(int kind, const tlh_op *op, bool has1, bool has2) {
    if (!op) return set_error(TLH_INVALID, "core: null op");
    const tlh_tensor &a = op->t[0], &b = op->t[1], &c = op->t[2], &d = op->t[4];
    for (int i = 0; i < 4; ++i)
        if (a.ne[i] < 0 || b.ne[i] < 0 || d.ne[i] < 0) return set_error(TLH_INVALID, "core: negative extent");
    auto unsup = [](const char *why) { return set_error(TLH_UNSUPPORTED, "core: %s", why); };
    const bool a_data = data_ty(a.ty) && elem_strides_ok(a);
    const bool d_data = data_ty(d.ty) && elem_strides_ok(d);
    switch (kind) {
    case TLH_CORE_BIN:
        if (!a_data || !data_ty(b.ty) || !elem_strides_ok(b) || !d_data) return unsup("BIN: f32/f16 operands");
        if (!same_shape(a, d)) return unsup("BIN: destination shape differs from src0");
        for (int i = 0; i < 4 && nel(a) > 0; ++i)  // ggml_can_repeat: an empty src1 repeats to an empty src0
            if (b.ne[i] == 0 || a.ne[i] % b.ne[i] != 0) return unsup("BIN: src1 does not repeat to src0");
        if (op->x[0] < 0 || op->x[0] > 3) return set_error(TLH_INVALID, "core: BIN code %lld", (long long)op->x[0]);
        return TLH_OK;
    case TLH_CORE_UNARY: {
        if (!a_data || !d_data) return unsup("UNARY: f32/f16 operands");
        if (!same_shape(a, d)) return unsup("UNARY: destination shape differs from src0");
        const int64_t code = op->x[0];
        if (!((code >= 0 && code <= 16) || (code >= 18 && code <= 21) || (code >= 100 && code <= 108)))
            return set_error(TLH_UNSUPPORTED, "core: unary op %lld", (long long)code);
        return TLH_OK;
    }
    case TLH_CORE_NORM:
        if (a.ty != TLH_TYPE_F32 || d.ty != TLH_TYPE_F32 || a.nb[0] != 4 || d.nb[0] != 4 || !elem_strides_ok(a) ||
            !elem_strides_ok(d))
            return unsup("NORM: f32 rows with unit element stride");
        if (!same_shape(a, d)) return unsup("NORM: destination shape differs from src0");
        return TLH_OK;
    case TLH_CORE_GET_ROWS:
        if (!(a_data || rows_of_blocks(a)) || !idx_ty(b.ty) || !elem_strides_ok(b) || !d_data)
            return unsup("GET_ROWS: f32/f16/bf16 or quantized (q4_0 ... q8_0, q2_K ... q6_K) rows, i32/i64 indices, "
                         "f32/f16 destination");
        if (d.ne[0] != a.ne[0] || d.ne[1] != b.ne[0] || d.ne[2] != b.ne[1] || d.ne[3] != b.ne[2] ||
            a.ne[2] != b.ne[1] || a.ne[3] != b.ne[2] || (a.ne[1] == 0 && nel(d) > 0))
            return unsup("GET_ROWS: shapes");
        return TLH_OK;
    case TLH_CORE_SET_ROWS:
        if (!a_data || !idx_ty(b.ty) || !elem_strides_ok(b) || !d_data)
            return unsup("SET_ROWS: f32/f16 rows, i32/i64 indices, f32/f16 destination");
        if (d.ne[0] != a.ne[0] || d.ne[2] != a.ne[2] || d.ne[3] != a.ne[3] || b.ne[0] != a.ne[1] || b.ne[1] == 0 ||
            b.ne[2] == 0 || a.ne[2] % b.ne[1] != 0 || a.ne[3] % b.ne[2] != 0)
            return unsup("SET_ROWS: shapes");
        return TLH_OK;
    case TLH_CORE_CPY:
        if (!(a_data || rows_of_blocks(a)) || !d_data) return unsup("CPY: f32/f16 (or quantized) to f32/f16");
        if (nel(a) != nel(d)) return unsup("CPY: element counts differ");
        return TLH_OK;
    case TLH_CORE_ROPE: {
        if (!a_data || !d_data || !same_shape(a, d)) return unsup("ROPE: f32/f16 operands of one shape");
        const int64_t n_dims = op->x[0], mode = op->x[1];
        if (mode != 0 && mode != 2) return unsup("ROPE: only normal and neox modes");
        if (b.ty != 26 || b.ne[0] != a.ne[2] || b.nb[0] != 4) return unsup("ROPE: one i32 position per token");
        if (n_dims <= 0 || n_dims > a.ne[0] || n_dims % 2) return set_error(TLH_INVALID, "core: ROPE n_dims");
        if (op->x[8] && (!has2 || c.ty != TLH_TYPE_F32 || c.nb[0] != 4 || c.ne[0] < n_dims / 2))
            return unsup("ROPE: frequency factors must be f32 [n_dims/2]");
        return TLH_OK;
    }
    case TLH_CORE_SOFT_MAX:
        if (a.ty != TLH_TYPE_F32 || !a_data || !d_data || !same_shape(a, d))
            return unsup("SOFT_MAX: f32 source, f32/f16 destination of its shape");
        if (has1 && (!data_ty(b.ty) || !elem_strides_ok(b) || b.ne[0] < a.ne[0] || b.ne[1] < a.ne[1] ||
                     b.ne[2] == 0 || b.ne[3] == 0 || a.ne[2] % b.ne[2] || a.ne[3] % b.ne[3]))
            return unsup("SOFT_MAX: mask must be f32/f16 [>= n, >= rows, broadcast]");
        return TLH_OK;
    case TLH_CORE_ARGMAX:
        if (a.ty != TLH_TYPE_F32 || !a_data || d.ty != 26 || d.nb[0] != 4) return unsup("ARGMAX: f32 rows to i32");
        if (a.ne[2] != 1 || a.ne[3] != 1 || d.ne[0] != a.ne[1] || a.ne[0] > INT32_MAX)
            return unsup("ARGMAX: 2-D source, one i32 per row");
        return TLH_OK;
    case TLH_CORE_GLU: {
        const bool rows_ok = a.ty == TLH_TYPE_F32 && d.ty == TLH_TYPE_F32 && a.nb[0] == 4 && d.nb[0] == 4 &&
                             elem_strides_ok(a) && elem_strides_ok(d) &&
                             (!has1 || (b.ty == TLH_TYPE_F32 && b.nb[0] == 4 && elem_strides_ok(b)));
        if (!rows_ok) return unsup("GLU: f32 rows with unit element stride");
        const int64_t code = op->x[0];
        if (code < 0 || code > 5 || code == 3) return set_error(TLH_UNSUPPORTED, "core: glu op %lld", (long long)code);
        if (has1 ? !(same_shape(a, b) && same_shape(a, d))
                 : (a.ne[0] % 2 != 0 || d.ne[0] != a.ne[0] / 2 || d.ne[1] != a.ne[1] || d.ne[2] != a.ne[2] ||
                    d.ne[3] != a.ne[3]))
            return unsup("GLU: shapes");
        return TLH_OK;
    }
    default: return set_error(TLH_INVALID, "core: unknown kind %d", kind);
    }
}

extern "C" {

const char *tlh_last_error(void) { return g_last_error.c_str(); }

const char *tlh_status_name(tlh_status s) {
    switch (s) {
    case TLH_OK: return "OK";
    case TLH_NO_DEVICE: return "NO_DEVICE";
    case TLH_UNSUPPORTED: return "UNSUPPORTED";
    case TLH_INVALID: return "INVALID";
    case TLH_ALLOC: return "ALLOC";
    case TLH_EXECUTION: return "EXECUTION";
    default: return "?";
    }
}

const char *tlh_version(void) { return "tlhip 0.1 gfx950"; }

tlh_status tlh_device_count(int *count) {
    if (!count) return set_error(TLH_INVALID, "device_count: null pointer");
    *count = 0;
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || (e == hipSuccess && n == 0)) {
        (void)hipGetLastError();
        return TLH_OK;
    }
    if (e != hipSuccess) return hip_check(e, "hipGetDeviceCount");
    *count = n;
    return TLH_OK;
}

tlh_status tlh_device_open(int ordinal, tlh_device_props *props) {
    int n = 0;
    tlh_status st = tlh_device_count(&n);
    if (st != TLH_OK) return st;
    if (n == 0) return set_error(TLH_NO_DEVICE, "no HIP device");
    if (ordinal < 0 || ordinal >= n) return set_error(TLH_NO_DEVICE, "device %d of %d", ordinal, n);
    st = hip_check(hipSetDevice(ordinal), "hipSetDevice");
    if (st != TLH_OK) return st;
    // best effort: resolving tlh_mul_mat_noalloc's array here keeps the look-up
    // out of a later capture; if it fails, that entry point reports it itself
    if (noalloc_setup_current_device() != TLH_OK) (void)hipGetLastError();
    if (!props) return TLH_OK;
    hipDeviceProp_t p;
    st = hip_check(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
    if (st != TLH_OK) return st;
    memset(props, 0, sizeof *props);
    snprintf(props->name, sizeof props->name, "%s", p.name);
    snprintf(props->arch, sizeof props->arch, "%s", p.gcnArchName);
    props->compute_units = p.multiProcessorCount;
    props->wave_size = p.warpSize;
    props->lds_bytes = (int)p.sharedMemPerBlock;
    props->clock_khz = p.clockRate;
    props->hbm_bytes = (int64_t)p.totalGlobalMem;
    return TLH_OK;
}

tlh_status tlh_alloc(size_t bytes, void **ptr) {
    if (!ptr) return set_error(TLH_INVALID, "alloc: null pointer");
    *ptr = nullptr;
    if (bytes == 0) return TLH_OK;
    const hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_error(TLH_ALLOC, "alloc of %zu bytes failed: %s", bytes, hipGetErrorString(e));
    }
    return TLH_OK;
}

tlh_status tlh_free(void *ptr) { return ptr ? hip_check(hipFree(ptr), "hipFree") : TLH_OK; }

tlh_status tlh_h2d(void *dst, const void *src, size_t bytes) {
    return bytes ? hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "h2d") : TLH_OK;
}

tlh_status tlh_d2h(void *dst, const void *src, size_t bytes) {
    return bytes ? hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "d2h") : TLH_OK;
}

tlh_status tlh_stream_sync(void *stream) {
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

// Scratch: the quantized activations, then (when the int8-MFMA few-column
// kernel runs with K split in chunks) its partial sums.
// float weights: src1 converted to contiguous rows of the weight type, 16-byte aligned
static int64_t mm_float_row(const MulMatShape &s) { return align_up(s.K * float_size(s.wtype), 16); }
static int64_t mm_act_bytes(const MulMatShape &s) {
    if (s.flt) return align_up(s.act_rows * mm_float_row(s), 256);
    return act_layout(s.act_type, s.K, s.act_rows, act_has_f16(s.wtype, s.N)).total;
}
static FloatMM float_mm(const tlh_op *op, const MulMatShape &s, const void *src0, const void *x, int xtype,
                        const int64_t (&x_nb)[4], void *dst) {
    const tlh_tensor &a = op->t[0], &d = op->t[4];
    FloatMM f{};
    f.wtype = a.ty, f.xtype = xtype;
    f.w = (const char *)src0, f.w_nb1 = a.nb[1], f.w_nb2 = a.nb[2], f.w_nb3 = a.nb[3];
    f.x = (const char *)x, f.x_nb1 = x_nb[1], f.x_nb2 = x_nb[2], f.x_nb3 = x_nb[3];
    f.d = (float *)dst, f.d_nb1 = d.nb[1], f.d_nb2 = d.nb[2], f.d_nb3 = d.nb[3];
    f.M = s.M, f.K = s.K, f.N = s.N, f.ne12 = s.ne12, f.ne13 = s.ne13, f.r2 = s.r2, f.r3 = s.r3;
    return f;
}
static int64_t mm_partial_bytes(const MulMatShape &s) {
    if (s.flt) return 0;
    int ksplit, upw;
    const bool reg = s.N <= 2 && gemv_reg_geometry(s.K, ksplit, upw);
    if (s.N > 16 && has_gemm(s.wtype)) return align_up(gemm_partial_bytes(s.wtype, s.M, s.N, s.K, s.ne12 * s.ne13), 256);
    // (q4_0 at N <= 2 takes the MFMA form when its weights are not 4-byte
    // aligned, which only the pointers tell: reserve its partials too)
    const bool mfma = s.N <= 16 ? (!reg || s.wtype == TLH_TYPE_Q4_0) : true;
    return mfma ? align_up(gemv_mfma_partial_bytes(s.K, s.M, s.N, s.ne12 * s.ne13), 256) : 0;
}

tlh_status tlh_mul_mat_scratch_bytes(const tlh_op *op, size_t *bytes) {
    if (!bytes) return set_error(TLH_INVALID, "mul_mat_scratch_bytes: null pointer");
    MulMatShape s;
    const tlh_status st = check_mul_mat(op, s);
    if (st != TLH_OK) return st;
    *bytes = (size_t)(mm_act_bytes(s) + mm_partial_bytes(s));
    return TLH_OK;
}

static tlh_status mm_check_scratch(const MulMatShape &s, const void *scratch, size_t scratch_bytes) {
    const size_t need = (size_t)(mm_act_bytes(s) + mm_partial_bytes(s));
    if (!scratch || scratch_bytes < need)
        return set_error(TLH_INVALID, "mul_mat: scratch of %zu bytes, need %zu", scratch_bytes, need);
    if ((uintptr_t)scratch & 255) return set_error(TLH_INVALID, "mul_mat: scratch must be 256-byte aligned");
    return TLH_OK;
}

// Phase 1: src1 -> vec_dot-type codes in scratch (the CPU's wdata, ggml-cpu.c:1318-1359).
static tlh_status mm_quantize(const tlh_op *op, const MulMatShape &s, const void *src1, void *scratch,
                              hipStream_t hs) {
    const tlh_tensor &a = op->t[0], &b = op->t[1];
    if (s.flt) {
        if ((uintptr_t)src1 % float_size(b.ty)) return set_error(TLH_INVALID, "mul_mat: misaligned src1");
        const FloatMM f = float_mm(op, s, nullptr, src1, b.ty, b.nb, nullptr);
        return launch_mm_float_convert(f, scratch, mm_float_row(s), hs);
    }
    if ((uintptr_t)src1 & 3) return set_error(TLH_INVALID, "mul_mat: src1 must be 4-byte aligned");
    const bool packed = b.nb[2] == b.nb[1] * s.N && b.nb[3] == b.nb[2] * s.ne12;
    if (packed)
        return launch_quantize_act(a.ty, (const float *)src1, s.K, s.act_rows, b.nb[1], scratch, false, 0,
                                   s.act_rows, act_has_f16(s.wtype, s.N), hs);
    for (int64_t i13 = 0; i13 < s.ne13; ++i13)
        for (int64_t i12 = 0; i12 < s.ne12; ++i12) {
            const float *x = (const float *)((const char *)src1 + i12 * b.nb[2] + i13 * b.nb[3]);
            const tlh_status st = launch_quantize_act(a.ty, x, s.K, s.N, b.nb[1], scratch, false,
                                                      s.N * (i12 + s.ne12 * i13), s.act_rows, act_has_f16(s.wtype, s.N), hs);
            if (st != TLH_OK) return st;
        }
    return TLH_OK;
}

static MatmulArgs mm_args(const tlh_op *op, const MulMatShape &s, const void *src0, const void *scratch, void *dst) {
    const tlh_tensor &a = op->t[0], &d = op->t[4];
    MatmulArgs m{};
    m.wtype = a.ty;
    m.w = (const uint8_t *)src0;
    m.w_nb1 = a.nb[1];
    m.w_nb2 = a.nb[2];
    m.w_nb3 = a.nb[3];
    m.M = s.M;
    m.K = s.K;
    m.N = s.N;
    m.n0 = 0;
    m.N_total = s.N;
    m.ne12 = s.ne12;
    m.ne13 = s.ne13;
    m.r2 = s.r2;
    m.r3 = s.r3;
    m.act = scratch;
    m.dst = (float *)dst;
    m.d_nb1 = d.nb[1];
    m.d_nb2 = d.nb[2];
    m.d_nb3 = d.nb[3];
    m.part = mm_partial_bytes(s) > 0 ? (float *)((char *)scratch + mm_act_bytes(s)) : nullptr;
    return m;
}

// Phase 2: the products from the scratch, N <= 8 -> GEMV, else GEMM.
static tlh_status mm_compute(const tlh_op *op, const MulMatShape &s, const void *src0, const void *scratch,
                             void *dst, hipStream_t hs) {
    if (((uintptr_t)src0 & 1) || ((uintptr_t)dst & 3))
        return set_error(TLH_INVALID, "mul_mat: misaligned src0 (2 bytes) or dst (4 bytes)");
    if (s.flt) {
        if ((uintptr_t)src0 % float_size(s.wtype)) return set_error(TLH_INVALID, "mul_mat: misaligned src0");
        const int64_t row = mm_float_row(s);
        const int64_t x_nb[4] = {float_size(s.wtype), row, row * s.N, row * s.N * s.ne12};
        return launch_mm_float(float_mm(op, s, src0, scratch, s.wtype, x_nb, dst), hs);
    }
    const MatmulArgs m = mm_args(op, s, src0, scratch, dst);
    return s.N <= 16 ? launch_gemv(m, nullptr, 0, hs) : launch_gemm(m, hs);
}

static bool mm_empty(const MulMatShape &s) { return s.M == 0 || s.N == 0 || s.ne12 == 0 || s.ne13 == 0; }

}  // extern "C"

// Up to three MUL_MAT nodes at N = 1 (one batch slice) reading one activation
// with weights of one type and K, as one register-GEMV launch that quantizes
// the activation once. mul_mat_multi_ok checks the shapes; mul_mat_multi
// returns TLH_UNSUPPORTED when the pointers do not allow the fused launch
// (the caller then runs the nodes one by one).
// Up to three MUL_MATs with 3..16 columns reading one quantized activation
// (the same scratch a tlh_mul_mat_quantize filled), weights of one type, K
// (one chunk: K <= 4096) and row stride, as one int8-MFMA few-column launch
// over their concatenated rows (each a multiple of 16 but the last).
bool tlh::mul_mat_compute_multi_ok(const tlh_op *const *ops, int n) {
    if (n < 2 || n > 3) return false;
    MulMatShape first;
    for (int i = 0; i < n; ++i) {
        MulMatShape s;
        if (check_mul_mat(ops[i], s) != TLH_OK || mm_empty(s) || s.flt || s.N < 3 || s.ne12 * s.ne13 != 1)
            return false;
        // more than 16 columns: the q4_K / q5_K GEMM over the segments' rows
        // (each but the last a whole number of its 128-row tiles)
        const bool gemm = s.N > 16;
        if (gemm ? !(s.wtype == TLH_TYPE_Q4_K || s.wtype == TLH_TYPE_Q5_K)
                 : gemv_mfma_partial_bytes(s.K, s.M, s.N, 1) != 0)
            return false;
        if (i < n - 1 && s.M % (gemm ? 128 : 16) != 0) return false;
        if (i == 0) first = s;
        else if (s.K != first.K || s.wtype != first.wtype || s.N != first.N ||
                 ops[i]->t[0].nb[1] != ops[0]->t[0].nb[1] || ops[i]->t[1].nb[1] != ops[0]->t[1].nb[1])
            return false;
    }
    return true;
}

// The quantized activation of the first node plus, for the GEMM form, the
// partial sums of its K chunks over all the nodes' rows.
size_t tlh::mul_mat_compute_multi_scratch_bytes(const tlh_op *const *ops, int n) {
    if (!mul_mat_compute_multi_ok(ops, n)) return 0;
    MulMatShape s;
    check_mul_mat(ops[0], s);
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) rows += ops[i]->t[0].ne[1];
    const int64_t part = s.N > 16 ? align_up(gemm_partial_bytes(s.wtype, rows, s.N, s.K, 1), 256) : 0;
    return (size_t)(mm_act_bytes(s) + part);
}

// With epi (the executor's batched Q / K / V projection): the few-column
// kernel stores through the epilogue (N <= 16, one K chunk), or above 16
// columns the q4_K / q5_K GEMM's K-chunk reduce does (the GEMM must split K);
// TLH_UNSUPPORTED when neither can take the shapes or pointers (the executor
// then runs the absorbed dispatches after a plain launch).
tlh_status tlh::mul_mat_compute_multi(const tlh_op *const *ops, const void *const *w, void *const *dst, int n,
                                      const void *scratch, size_t scratch_bytes, hipStream_t stream,
                                      const GemvEpi *epi) {
    if (!mul_mat_compute_multi_ok(ops, n)) return set_error(TLH_UNSUPPORTED, "mul_mat_compute_multi: shapes");
    if (epi) {
        for (int i = 0; i < n; ++i) {
            if (epi->layout[i] == EPI_F32) continue;
            const uintptr_t es = epi->f16[i] ? 2 : 4, is = epi->idx_i64[i] ? 8 : 4;
            if (((uintptr_t)epi->dst[i] | (uintptr_t)epi->row_nb[i]) % es || (epi->idx[i] && (uintptr_t)epi->idx[i] % is) ||
                (epi->rope[i] && (((uintptr_t)epi->pos & 3) || ((uintptr_t)epi->ff & 3))))
                return set_error(TLH_UNSUPPORTED, "mul_mat_compute_multi: epilogue pointer alignment");
        }
    }
    MulMatShape s;
    check_mul_mat(ops[0], s);
    const size_t need = mul_mat_compute_multi_scratch_bytes(ops, n);
    if (!scratch || scratch_bytes < need)
        return set_error(TLH_INVALID, "mul_mat_compute_multi: scratch of %zu bytes, need %zu", scratch_bytes, need);
    if ((uintptr_t)scratch & 255) return set_error(TLH_INVALID, "mul_mat_compute_multi: scratch must be 256-byte aligned");
    MatmulArgs m = mm_args(ops[0], s, w[0], scratch, dst[0]);
    m.part = s.N > 16 ? (float *)((char *)scratch + mm_act_bytes(s)) : nullptr;
    m.nseg = n;
    int64_t rows = 0;
    for (int i = 0; i < 3; ++i) {
        m.seg_m0[i] = rows;
        if (i < n) {
            if (!w[i] || !dst[i] || ((uintptr_t)w[i] & 1) || ((uintptr_t)dst[i] & 3))
                return set_error(TLH_INVALID, "mul_mat_compute_multi: null or misaligned pointer");
            m.seg_w[i] = (const uint8_t *)w[i];
            m.seg_w_nb1[i] = ops[i]->t[0].nb[1];
            m.seg_dst[i] = (float *)dst[i];
            m.seg_d_nb1[i] = ops[i]->t[4].nb[1];
            rows += ops[i]->t[0].ne[1];
        }
    }
    m.seg_m0[3] = rows;
    for (int i = n; i < 3; ++i) m.seg_m0[i] = rows;
    m.M = rows;
    if (epi)  // few columns: the GEMV's own stores; many: the K-split GEMM's reduce
        return s.N > 16 ? launch_gemm_epi(m, *epi, stream) : launch_gemv_mfma_epi(m, *epi, stream);
    return s.N > 16 ? launch_gemm(m, stream) : launch_gemv_mfma(m, stream);
}

bool tlh::mul_mat_multi_ok(const tlh_op *const *ops, int n) {
    if (n < 1 || n > 3) return false;
    MulMatShape first;
    for (int i = 0; i < n; ++i) {
        MulMatShape s;
        // q4_1 / q5_0 / q5_1 / q2_K / q3_K have no segment or fused (prologue /
        // epilogue) register kernels
        if (check_mul_mat(ops[i], s) != TLH_OK || mm_empty(s) || s.flt || reg_plain_type(s.wtype) || s.N != 1 ||
            s.ne12 * s.ne13 != 1)
            return false;
        int ks, upw;
        if (s.K > 4096 || !gemv_reg_geometry(s.K, ks, upw)) return false;  // in-kernel quantization: K <= 4096
        if (i == 0) first = s;
        else if (s.K != first.K || s.wtype != first.wtype) return false;
    }
    return true;
}

tlh_status tlh::mul_mat_multi(const tlh_op *const *ops, const void *const *w, void *const *dst, int n,
                              const void *x, hipStream_t stream) {
    if (!mul_mat_multi_ok(ops, n)) return set_error(TLH_UNSUPPORTED, "mul_mat_multi: shapes");
    MulMatShape s;
    check_mul_mat(ops[0], s);
    MatmulArgs m = mm_args(ops[0], s, w[0], nullptr, dst[0]);
    m.nseg = n;
    int64_t rows = 0;
    for (int i = 0; i < 3; ++i) {
        m.seg_m0[i] = rows;
        if (i < n) {
            if (!w[i] || !dst[i] || ((uintptr_t)w[i] & 1) || ((uintptr_t)dst[i] & 3))
                return set_error(TLH_UNSUPPORTED, "mul_mat_multi: pointers");
            m.seg_w[i] = (const uint8_t *)w[i];
            m.seg_w_nb1[i] = ops[i]->t[0].nb[1];
            m.seg_dst[i] = (float *)dst[i];
            rows += ops[i]->t[0].ne[1];
        } else {
            m.seg_w[i] = nullptr;
            m.seg_w_nb1[i] = 0;
            m.seg_dst[i] = nullptr;
        }
    }
    m.seg_m0[3] = rows;
    m.M = rows;
    if (!x || !gemv_fuses_quantize(m, (const float *)x, ops[0]->t[1].nb[1]))
        return set_error(TLH_UNSUPPORTED, "mul_mat_multi: activation alignment");
    return launch_gemv_reg(m, (const float *)x, ops[0]->t[1].nb[1], stream);
}

// mul_mat_multi with a GemvPro prologue (the activation formed from an
// [ADD ->] RMS_NORM -> MUL chain; x is then null) and / or SwiGLU epilogue
// (two members: gate then up, equal rows; h goes to pro.glu). Shapes as
// mul_mat_multi_ok; TLH_UNSUPPORTED when the pointers or strides do not allow
// the fused launch (the executor then runs the pieces one by one).
tlh_status tlh::mul_mat_multi_pro(const tlh_op *const *ops, const void *const *w, void *const *dst, int n,
                                  const GemvPro &pro, const void *x, hipStream_t stream) {
    if (!mul_mat_multi_ok(ops, n)) return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: shapes");
    MulMatShape s;
    check_mul_mat(ops[0], s);
    const bool glu = pro.glu != nullptr;
    if (glu && (n != 2 || ops[0]->t[0].ne[1] != ops[1]->t[0].ne[1]))
        return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: SwiGLU takes a gate and an up matrix of equal rows");
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (pro.p) {
        if (s.K > 4096 || !a16(pro.p) || !a16(pro.w) || (pro.q && !a16(pro.q)) || (pro.s && !a16(pro.s)) ||
            ((pro.p_nb1 | pro.q_nb1 | pro.s_nb1) & 15))
            return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: norm rows (K <= 4096, 16-byte aligned)");
    } else if (!x || ((uintptr_t)x & 15) || (ops[0]->t[1].nb[1] & 15)) {
        return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: activation alignment");
    }
    if (glu && (((uintptr_t)pro.glu & 3) || (pro.glu_nb1 & 3)))
        return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: SwiGLU destination alignment");
    const GemvEpi &e = pro.epi;
    for (int i = 0; e.on && i < n; ++i) {
        if (e.layout[i] == EPI_F32) continue;
        const uintptr_t es = e.f16[i] ? 2 : 4, is = e.idx_i64[i] ? 8 : 4;
        if (((uintptr_t)e.dst[i] | (uintptr_t)e.row_nb[i]) % es || (e.idx[i] && (uintptr_t)e.idx[i] % is) ||
            (e.rope[i] && (((uintptr_t)e.pos & 3) || ((uintptr_t)e.ff & 3))))
            return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: epilogue pointer alignment");
    }
    MatmulArgs m = mm_args(ops[0], s, w[0], nullptr, dst[0]);
    m.nseg = n;
    int64_t rows = 0;
    for (int i = 0; i < 3; ++i) {
        m.seg_m0[i] = rows;
        if (i < n) {
            if (!w[i] || ((uintptr_t)w[i] & 1) || (!glu && (!dst[i] || ((uintptr_t)dst[i] & 3))))
                return set_error(TLH_UNSUPPORTED, "mul_mat_multi_pro: pointers");
            m.seg_w[i] = (const uint8_t *)w[i];
            m.seg_w_nb1[i] = ops[i]->t[0].nb[1];
            m.seg_dst[i] = (float *)dst[i];
            rows += ops[i]->t[0].ne[1];
        } else {
            m.seg_w[i] = nullptr;
            m.seg_w_nb1[i] = 0;
            m.seg_dst[i] = nullptr;
        }
    }
    m.seg_m0[3] = rows;
    m.M = rows;
    return launch_gemv_reg_pro(m, pro, (const float *)x, ops[0]->t[1].nb[1], stream);
}

extern "C" {

tlh_status tlh_mul_mat(const tlh_op *op, const void *src0, const void *src1, void *dst, void *scratch,
                       size_t scratch_bytes, void *stream) {
    MulMatShape s;
    tlh_status st = check_mul_mat(op, s);
    if (st != TLH_OK || mm_empty(s)) return st;
    if (!src0 || !src1 || !dst) return set_error(TLH_INVALID, "mul_mat: null tensor pointer");
    if ((st = mm_check_scratch(s, scratch, scratch_bytes)) != TLH_OK) return st;
    const hipStream_t hs = (hipStream_t)stream;
    const tlh_tensor &b = op->t[1];
    if (s.flt) {  // one launch that rounds src1 as it reads it
        if ((uintptr_t)src0 % float_size(s.wtype) || (uintptr_t)src1 % float_size(b.ty) || ((uintptr_t)dst & 3))
            return set_error(TLH_INVALID, "mul_mat: misaligned src0, src1 or dst");
        return launch_mm_float(float_mm(op, s, src0, src1, b.ty, b.nb, dst), hs);
    }
    // Decode with a small activation: the GEMV quantizes src1 itself (one launch).
    const bool packed = b.nb[2] == b.nb[1] * s.N && b.nb[3] == b.nb[2] * s.ne12;
    if (s.N <= 2 && packed && !((uintptr_t)src1 & 3)) {
        const MatmulArgs m = mm_args(op, s, src0, scratch, dst);
        if (gemv_fuses_quantize(m, (const float *)src1, b.nb[1])) {
            if (((uintptr_t)src0 & 1) || ((uintptr_t)dst & 3))
                return set_error(TLH_INVALID, "mul_mat: misaligned src0 (2 bytes) or dst (4 bytes)");
            return launch_gemv(m, (const float *)src1, b.nb[1], hs);
        }
    }
    if ((st = mm_quantize(op, s, src1, scratch, hs)) != TLH_OK) return st;
    return mm_compute(op, s, src0, scratch, dst, hs);
}

tlh_status tlh_mul_mat_quantize(const tlh_op *op, const void *src1, void *scratch, size_t scratch_bytes,
                                void *stream) {
    MulMatShape s;
    tlh_status st = check_mul_mat(op, s);
    if (st != TLH_OK || mm_empty(s)) return st;
    if (!src1) return set_error(TLH_INVALID, "mul_mat_quantize: null src1");
    if ((st = mm_check_scratch(s, scratch, scratch_bytes)) != TLH_OK) return st;
    return mm_quantize(op, s, src1, scratch, (hipStream_t)stream);
}

tlh_status tlh_mul_mat_compute(const tlh_op *op, const void *src0, const void *scratch, size_t scratch_bytes,
                               void *dst, void *stream);

}  // extern "C"

bool tlh::mul_mat_partials(const tlh_op *op, MmPartials &pp) {
    MulMatShape s;
    if (check_mul_mat(op, s) != TLH_OK || mm_empty(s) || s.flt || s.ne12 * s.ne13 != 1 || s.N < 3) return false;
    int64_t chunks;
    if (s.N > 16) {
        if (s.wtype != TLH_TYPE_Q8_0 && s.wtype != TLH_TYPE_Q4_0 && s.wtype != TLH_TYPE_Q4_K && s.wtype != TLH_TYPE_Q5_K)
            return false;
        chunks = gemm_ksplit(s.wtype, s.M, s.N, s.K, 1);
    } else {
        chunks = gemv_mfma_chunks(s.K);  // (the tall form takes K <= 4096: one chunk)
    }
    if (chunks < 2) return false;
    pp.off = mm_act_bytes(s);
    pp.chunks = (int)chunks;
    pp.cstride = s.N * s.M;
    return true;
}

tlh_status tlh::mul_mat_compute_keep(const tlh_op *op, const void *src0, const void *src1, void *scratch,
                                     size_t scratch_bytes, void *dst, hipStream_t hs) {
    MulMatShape s;
    tlh_status st = check_mul_mat(op, s);
    if (st != TLH_OK) return st;
    MmPartials pp;
    if (!mul_mat_partials(op, pp)) return set_error(TLH_UNSUPPORTED, "mul_mat_compute_keep: no K split here");
    if (!src0 || !dst) return set_error(TLH_INVALID, "mul_mat_compute_keep: null tensor pointer");
    if ((st = mm_check_scratch(s, scratch, scratch_bytes)) != TLH_OK) return st;
    if (((uintptr_t)src0 & 1) || ((uintptr_t)dst & 3))
        return set_error(TLH_INVALID, "mul_mat: misaligned src0 (2 bytes) or dst (4 bytes)");
    if (src1 && (st = mm_quantize(op, s, src1, scratch, hs)) != TLH_OK) return st;
    MatmulArgs m = mm_args(op, s, src0, scratch, dst);
    m.keep_part = 1;
    return s.N <= 16 ? launch_gemv(m, nullptr, 0, hs) : launch_gemm(m, hs);
}

extern "C" {

tlh_status tlh_mul_mat_compute(const tlh_op *op, const void *src0, const void *scratch, size_t scratch_bytes,
                               void *dst, void *stream) {
    MulMatShape s;
    tlh_status st = check_mul_mat(op, s);
    if (st != TLH_OK || mm_empty(s)) return st;
    if (!src0 || !dst) return set_error(TLH_INVALID, "mul_mat_compute: null tensor pointer");
    if ((st = mm_check_scratch(s, scratch, scratch_bytes)) != TLH_OK) return st;
    return mm_compute(op, s, src0, scratch, dst, (hipStream_t)stream);
}

}  // extern "C"

// ------------------------------------------------- MUL_MAT without allocation
// tlh_mul_mat_noalloc runs tlh_mul_mat's kernels with their scratch (the
// quantized activations and the K-chunk partial sums) in this file-scope
// device array instead of a caller buffer. Each GPU the library runs on holds
// its own copy for the life of the process. Host code must not pass the
// array's name to a kernel or a copy: on the host it is only a stand-in
// symbol. Its device address is looked up once per device with that device
// current (hipGetSymbolAddress) and kept in g_noalloc_ptr.
static __device__ __align__(256) uint8_t scratch[TLH_NOALLOC_SCRATCH_BYTES];

namespace tlh {

static std::mutex g_noalloc_mu;
static void *g_noalloc_ptr[kMaxDevices];

// The device address of `scratch` on the current device (resolved on first use).
static tlh_status noalloc_scratch(void **ptr) {
    int dev = 0;
    tlh_status st = hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (st != TLH_OK) return st;
    if (dev < 0 || dev >= kMaxDevices) return set_error(TLH_UNSUPPORTED, "mul_mat_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        st = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (st != TLH_OK) return st;
        if (!p || ((uintptr_t)p & 255))
            return set_error(TLH_EXECUTION, "mul_mat_noalloc: scratch address %p is not 256-byte aligned", p);
        g_noalloc_ptr[dev] = p;
    }
    *ptr = g_noalloc_ptr[dev];
    return TLH_OK;
}

// Set-up at device open, so a caller that opens its devices first never has
// the look-up happen inside a capture.
tlh_status noalloc_setup_current_device() {
    void *p = nullptr;
    return noalloc_scratch(&p);
}

}  // namespace tlh

extern "C" {

tlh_status tlh_mul_mat_noalloc(const tlh_op *op, const void *src0, const void *src1, void *dst, void *stream) {
    MulMatShape s;
    tlh_status st = check_mul_mat(op, s);
    if (st != TLH_OK || mm_empty(s)) return st;
    const size_t need = (size_t)(mm_act_bytes(s) + mm_partial_bytes(s));
    if (need > (size_t)TLH_NOALLOC_SCRATCH_BYTES)
        return set_error(TLH_INVALID,
                         "mul_mat_noalloc: this node needs %zu bytes of scratch, beyond the static %zu "
                         "(use tlh_mul_mat with a caller buffer)",
                         need, (size_t)TLH_NOALLOC_SCRATCH_BYTES);
    void *scr = nullptr;
    if ((st = noalloc_scratch(&scr)) != TLH_OK) return st;
    return tlh_mul_mat(op, src0, src1, dst, scr, (size_t)TLH_NOALLOC_SCRATCH_BYTES, stream);
}

// ------------------------------------------------------------ MUL_MAT_ID
// ggml_mul_mat_id (ggml.c:3329-3353) computed as the CPU backend does
// (ggml_compute_forward_mul_mat_id, ggml-cpu/ggml-cpu.c:1460-1640): src1 rows
// quantized to the vec_dot type once, then output column (e, t) is expert
// ids[e, t]'s matrix times quantized row (e % ne11) + ne11 * t, each element
// one vec_dot. Here every (e, t) pair is one batch slice of the int8-MFMA
// few-column kernel, which reads the expert id on the device.
struct MulMatIdShape {
    int64_t K, M, n_as, n_used, n_tok, n_b1;
    int wtype, act_type;
};

static tlh_status check_mul_mat_id(const tlh_op *op, MulMatIdShape &s) {
    if (!op) return set_error(TLH_INVALID, "mul_mat_id: null op");
    const tlh_tensor &a = op->t[0], &b = op->t[1], &ids = op->t[2], &d = op->t[4];
    if (!weight_type_ok(a.ty))
        return set_error(TLH_UNSUPPORTED,
                         "mul_mat_id: weights of ggml type %d (%s); have q4_0, q4_1, q5_0, q5_1, q8_0, q2_K, q3_K, "
                         "q4_K, q5_K, q6_K",
                         a.ty, type_name(a.ty));
    if (b.ty != TLH_TYPE_F32 || d.ty != TLH_TYPE_F32 || ids.ty != TLH_TYPE_I32)
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: f32 src1 and dst, i32 ids");
    for (int i = 0; i < 4; ++i)
        if (a.ne[i] < 0 || b.ne[i] < 0 || d.ne[i] < 0 || ids.ne[i] < 0)
            return set_error(TLH_INVALID, "mul_mat_id: negative extent");
    // ggml_mul_mat_id's asserts
    if (a.ne[3] != 1 || b.ne[3] != 1 || ids.ne[2] != 1 || ids.ne[3] != 1 || ids.ne[1] != b.ne[2] ||
        a.ne[0] != b.ne[0] || b.ne[1] == 0 || ids.ne[0] % b.ne[1] != 0)
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: shapes (as [K, M, n_as], b [K, n_b1, n_tokens], ids [n_used, "
                                          "n_tokens] with n_used %% n_b1 == 0)");
    if (d.ne[0] != a.ne[1] || d.ne[1] != ids.ne[0] || d.ne[2] != b.ne[2] || d.ne[3] != 1)
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: dst must be [M, n_used, n_tokens]");
    s.K = a.ne[0];
    s.M = a.ne[1];
    s.n_as = a.ne[2];
    s.n_used = ids.ne[0];
    s.n_tok = ids.ne[1];
    s.n_b1 = b.ne[1];
    const int be = block_elems(a.ty);
    if (s.K % be != 0)
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: K=%lld is not a multiple of the %s block (%d)", (long long)s.K,
                         type_name(a.ty), be);
    const int64_t rb = s.K / be * block_bytes(a.ty);
    if (a.nb[0] != block_bytes(a.ty) || a.nb[1] < rb || (a.nb[1] & 1) || a.nb[2] < a.nb[1] * s.M || (a.nb[2] & 1))
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: src0 must hold whole rows, 2-byte aligned, matrices apart");
    if (b.nb[0] != 4 || (b.nb[1] & 3) || (b.nb[2] & 3))
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: src1 must have contiguous f32 rows");
    if (ids.nb[0] != 4 || (ids.nb[1] & 3))
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: ids must be i32 with 4-byte strides");
    if (d.nb[0] != 4 || d.nb[1] < 4 * s.M || (d.nb[1] & 3) || d.nb[2] < d.nb[1] || (d.nb[2] & 3))
        return set_error(TLH_UNSUPPORTED, "mul_mat_id: dst must be f32 with ordered strides");
    if (s.n_used * s.n_tok > 65535) return set_error(TLH_UNSUPPORTED, "mul_mat_id: more than 65535 (expert, token) pairs");
    s.wtype = a.ty;
    s.act_type = vec_dot_type(a.ty);
    return TLH_OK;
}

static int64_t mmid_act_bytes(const MulMatIdShape &s) { return act_layout(s.act_type, s.K, s.n_b1 * s.n_tok).total; }
static int64_t mmid_partial_bytes(const MulMatIdShape &s) {
    return align_up(gemv_mfma_partial_bytes(s.K, s.M, 1, s.n_used * s.n_tok), 256);
}

tlh_status tlh_mul_mat_id_scratch_bytes(const tlh_op *op, size_t *bytes) {
    if (!bytes) return set_error(TLH_INVALID, "mul_mat_id_scratch_bytes: null pointer");
    MulMatIdShape s;
    const tlh_status st = check_mul_mat_id(op, s);
    if (st != TLH_OK) return st;
    *bytes = (size_t)(mmid_act_bytes(s) + mmid_partial_bytes(s));
    return TLH_OK;
}

tlh_status tlh_mul_mat_id(const tlh_op *op, const void *src0, const void *src1, const void *ids, void *dst,
                          void *scratch, size_t scratch_bytes, void *stream) {
    MulMatIdShape s;
    tlh_status st = check_mul_mat_id(op, s);
    if (st != TLH_OK) return st;
    if (s.M == 0 || s.n_used == 0 || s.n_tok == 0) return TLH_OK;
    if (!src0 || !src1 || !ids || !dst) return set_error(TLH_INVALID, "mul_mat_id: null tensor pointer");
    const size_t need = (size_t)(mmid_act_bytes(s) + mmid_partial_bytes(s));
    if (!scratch || scratch_bytes < need)
        return set_error(TLH_INVALID, "mul_mat_id: scratch of %zu bytes, need %zu", scratch_bytes, need);
    if (((uintptr_t)scratch & 255) || ((uintptr_t)src1 & 3) || ((uintptr_t)src0 & 1) || ((uintptr_t)dst & 3) ||
        ((uintptr_t)ids & 3))
        return set_error(TLH_INVALID, "mul_mat_id: misaligned pointer (scratch 256, src1/dst/ids 4, src0 2 bytes)");
    const tlh_tensor &a = op->t[0], &b = op->t[1], &it = op->t[2], &d = op->t[4];
    const hipStream_t hs = (hipStream_t)stream;
    const int64_t rows = s.n_b1 * s.n_tok;
    if (b.nb[2] == b.nb[1] * s.n_b1 || s.n_tok == 1) {
        st = launch_quantize_act(a.ty, (const float *)src1, s.K, rows, b.nb[1], scratch, false, 0, rows, false, hs);
    } else {
        for (int64_t t = 0; t < s.n_tok && st == TLH_OK; ++t)
            st = launch_quantize_act(a.ty, (const float *)((const char *)src1 + t * b.nb[2]), s.K, s.n_b1, b.nb[1],
                                     scratch, false, s.n_b1 * t, rows, false, hs);
    }
    if (st != TLH_OK) return st;
    MatmulArgs m{};
    m.wtype = a.ty;
    m.w = (const uint8_t *)src0;
    m.w_nb1 = a.nb[1];
    m.w_nb2 = a.nb[2];
    m.w_nb3 = a.nb[2] * s.n_as;
    m.M = s.M;
    m.K = s.K;
    m.N = 1;
    m.N_total = 1;
    m.ne12 = s.n_used;
    m.ne13 = s.n_tok;
    m.r2 = m.r3 = 1;
    m.act = scratch;
    m.dst = (float *)dst;
    m.d_nb1 = d.nb[1];
    m.d_nb2 = d.nb[1];
    m.d_nb3 = d.nb[2];
    m.part = mmid_partial_bytes(s) > 0 ? (float *)((char *)scratch + mmid_act_bytes(s)) : nullptr;
    m.ids = (const char *)ids;
    m.ids_nb0 = it.nb[0];
    m.ids_nb1 = it.nb[1];
    m.id_b1 = s.n_b1;
    m.id_nas = s.n_as;
    return launch_gemv_mfma(m, hs);
}

tlh_status tlh_quantize_act(int wtype, const float *x, int64_t k, int64_t rows, int64_t x_row_bytes, void *y,
                            void *stream) {
    if (!weight_type_ok(wtype)) return set_error(TLH_UNSUPPORTED, "quantize_act: weight type %d", wtype);
    if (k < 0 || rows < 0 || k % block_elems(vec_dot_type(wtype)) != 0)
        return set_error(TLH_INVALID, "quantize_act: k=%lld is not a multiple of the %s block", (long long)k,
                         type_name(vec_dot_type(wtype)));
    if ((!x || !y) && k * rows > 0) return set_error(TLH_INVALID, "quantize_act: null pointer");
    if (x_row_bytes < 4 * k || (x_row_bytes & 3) || ((uintptr_t)x & 3) || ((uintptr_t)y & 3))
        return set_error(TLH_INVALID, "quantize_act: rows must be 4-byte aligned f32 with stride >= 4k");
    return launch_quantize_act(wtype, x, k, rows, x_row_bytes, y, true, 0, rows, false, (hipStream_t)stream);
}

tlh_status tlh_dequantize(int type, const void *w, int64_t k, int64_t rows, int64_t w_row_bytes, float *y,
                          void *stream) {
    if (!weight_type_ok(type)) return set_error(TLH_UNSUPPORTED, "dequantize: type %d", type);
    if (k < 0 || rows < 0 || k % block_elems(type) != 0)
        return set_error(TLH_INVALID, "dequantize: k=%lld is not a multiple of the %s block", (long long)k,
                         type_name(type));
    if ((!w || !y) && k * rows > 0) return set_error(TLH_INVALID, "dequantize: null pointer");
    if (w_row_bytes < k / block_elems(type) * block_bytes(type) || (w_row_bytes & 1) || ((uintptr_t)w & 1))
        return set_error(TLH_INVALID, "dequantize: row stride too small or misaligned");
    return launch_dequantize(type, w, k, rows, w_row_bytes, y, (hipStream_t)stream);
}

static tlh_status check_paged(const tlh_paged_attention_args *a) {
    if (!a) return set_error(TLH_INVALID, "paged_attention: null args");
    static const int head_sizes[] = {64, 80, 96, 112, 128, 192, 256};
    bool hs_ok = false;
    for (int h : head_sizes) hs_ok |= a->head_size == h;
    if (!hs_ok) return set_error(TLH_INVALID, "paged_attention: unsupported head_size %d", a->head_size);
    if (a->block_size != 8 && a->block_size != 16 && a->block_size != 32)
        return set_error(TLH_INVALID, "paged_attention: unsupported block_size %d (have 8, 16, 32)", a->block_size);
    if (a->num_kv_heads <= 0 || a->num_heads <= 0 || a->num_heads % a->num_kv_heads != 0)
        return set_error(TLH_INVALID, "paged_attention: num_heads must be a multiple of num_kv_heads");
    if (a->num_seqs < 0 || a->max_blocks_per_seq < 0 || a->max_context_len < 0 ||
        (int64_t)a->max_blocks_per_seq * a->block_size < a->max_context_len)
        return set_error(TLH_INVALID, "paged_attention: max_blocks_per_seq * block_size < max_context_len");
    return TLH_OK;
}

tlh_status tlh_paged_attention_scratch_bytes(const tlh_paged_attention_args *a, size_t *bytes) {
    if (!bytes) return set_error(TLH_INVALID, "paged_attention_scratch_bytes: null pointer");
    const tlh_status st = check_paged(a);
    if (st != TLH_OK) return st;
    *bytes = paged_attention_scratch_bytes(*a);
    return TLH_OK;
}

tlh_status tlh_paged_attention(const tlh_paged_attention_args *a, void *scratch, size_t scratch_bytes,
                               void *stream) {
    const tlh_status st = check_paged(a);
    if (st != TLH_OK) return st;
    if (a->num_seqs == 0) return TLH_OK;
    if (!a->out || !a->q || !a->k_cache || !a->v_cache || !a->block_tables || !a->context_lens)
        return set_error(TLH_INVALID, "paged_attention: null pointer");
    const size_t need = paged_attention_scratch_bytes(*a);
    if (need > 0 && (!scratch || scratch_bytes < need))
        return set_error(TLH_INVALID, "paged_attention: scratch of %zu bytes, need %zu", scratch_bytes, need);
    return launch_paged_attention(*a, scratch, scratch_bytes, (hipStream_t)stream);
}

tlh_status tlh_reshape_and_cache(const void *key, const void *value, void *k_cache, void *v_cache,
                                 const int64_t *slots, int32_t num_tokens, int32_t num_kv_heads, int32_t head_size,
                                 int32_t block_size, int64_t num_blocks, void *stream) {
    if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || head_size % 8 != 0 || block_size <= 0 ||
        num_blocks < 0)
        return set_error(TLH_INVALID, "reshape_and_cache: bad geometry");
    if (num_tokens == 0) return TLH_OK;
    if (!key || !value || !k_cache || !v_cache || !slots) return set_error(TLH_INVALID, "reshape_and_cache: null pointer");
    return launch_reshape_and_cache(key, value, k_cache, v_cache, slots, num_tokens, num_kv_heads, head_size,
                                    block_size, num_blocks, (hipStream_t)stream);
}

tlh_status tlh_flash_attn_ext_scratch_bytes(const tlh_op *op, size_t *bytes) {
    if (!bytes) return set_error(TLH_INVALID, "flash_attn_ext_scratch_bytes: null pointer");
    FlashAttnDesc d;
    // a mask descriptor in slot 3 (OpBlob leaves it zeroed without a mask)
    const bool has_mask = op && op->t[3].ne[0] > 0;
    const tlh_status st = check_flash_attn(op, has_mask, d);
    if (st != TLH_OK) return st;
    *bytes = (size_t)flash_attn_scratch_bytes(d.DV, d.nq, d.nh, d.nhkv, d.nb, d.L, has_mask ? d.nq * d.m_ne2 * d.m_ne3 : 0);
    return TLH_OK;
}

tlh_status tlh_flash_attn_ext(const tlh_op *op, const void *q, const void *k, const void *v, const void *mask,
                              void *dst, void *scratch, size_t scratch_bytes, void *stream) {
    FlashAttnDesc d;
    const tlh_status st = check_flash_attn(op, mask != nullptr, d);
    if (st != TLH_OK) return st;
    if (d.max_bias > 0.0f && !mask) return set_error(TLH_INVALID, "flash_attn_ext: max_bias needs a mask");
    if (d.nq == 0 || d.nh == 0 || d.nb == 0 || d.DV == 0) return TLH_OK;
    if (!q || !dst || (d.L > 0 && (!k || !v))) return set_error(TLH_INVALID, "flash_attn_ext: null tensor pointer");
    if (((uintptr_t)k | (uintptr_t)v) & 15)
        return set_error(TLH_UNSUPPORTED, "flash_attn_ext: K/V must be 16-byte aligned");
    if (((uintptr_t)q | (uintptr_t)dst) & 3 || ((uintptr_t)mask & 1))
        return set_error(TLH_INVALID, "flash_attn_ext: misaligned q, dst or mask");
    const size_t need =
        (size_t)flash_attn_scratch_bytes(d.DV, d.nq, d.nh, d.nhkv, d.nb, d.L, mask ? d.nq * d.m_ne2 * d.m_ne3 : 0);
    if (need > 0 && (!scratch || scratch_bytes < need))
        return set_error(TLH_INVALID, "flash_attn_ext: scratch of %zu bytes, need %zu", scratch_bytes, need);
    if (need > 0 && ((uintptr_t)scratch & 7)) return set_error(TLH_INVALID, "flash_attn_ext: misaligned scratch");
    d.q = q, d.k = k, d.v = v, d.mask = mask, d.dst = dst, d.scratch = scratch;
    return launch_flash_attn(d, (hipStream_t)stream);
}

tlh_status tlh_core_check(int kind, const tlh_op *op, int has_src1, int has_src2) {
    return check_core(kind, op, has_src1 != 0, has_src2 != 0);
}

tlh_status tlh_core(int kind, const tlh_op *op, const void *src0, const void *src1, const void *src2, void *dst,
                    void *stream) {
    const tlh_status st = check_core(kind, op, src1 != nullptr, src2 != nullptr);
    if (st != TLH_OK) return st;
    if (nel(op->t[4]) == 0 || (kind == TLH_CORE_SET_ROWS && nel(op->t[0]) == 0)) return TLH_OK;  // nothing to do
    const bool needs1 = kind == TLH_CORE_BIN || kind == TLH_CORE_GET_ROWS || kind == TLH_CORE_SET_ROWS ||
                        kind == TLH_CORE_ROPE;
    if (!src0 || !dst || (needs1 && !src1)) return set_error(TLH_INVALID, "core: null tensor pointer");
    return launch_core(kind, *op, src0, src1, src2, dst, (hipStream_t)stream);
}

}  // extern "C"

// Test infrastructure only (never linked into the product library).
//
// A thin harness over the reference's own ggml CPU backend, compiled in place
// from /root/reference/vendor/ggml by oracle/Makefile. It runs one-op ggml
// graphs exactly as tensorlisp's Device::Cpu path does
// (crates/tensorlisp/src/model.rs:424-437 -> ggml_graph_compute,
// vendor/ggml/src/ggml-cpu/ggml-cpu.c:3355), so its outputs are the reference
// results the HIP path is checked against:
//
//   ref_mul_mat      GGML_OP_MUL_MAT, src0 = quantized weight [K, M],
//                    src1 = f32 activations [K, N] (ggml_mul_mat, ggml.c:3278;
//                    CPU kernel ggml-cpu.c:1254-1457).
//   ref_flash_attn   GGML_OP_FLASH_ATTN_EXT over dense f16 K/V (ops.cpp:8468),
//                    the dense-cache attention the paged kernel is compared to.
//   ref_flash_attn_ext  the same op in full: q [D, nq, nh, nb], K/V
//                    [D|DV, L, nhkv, nb], optional f16 mask [Lm, nqm, mne2,
//                    mne3], max_bias and logit softcap (ggml.c:5402-5444).
//
// Tensor data points at caller memory (no copies); the work buffer is
// allocated per call.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "ggml.h"
#include "ggml-cpu.h"

static struct ggml_context *meta_ctx(void) {
    ggml_cpu_init();  // fp16 tables and CPU feature probe; idempotent
    struct ggml_init_params p = {
        .mem_size = 64 * ggml_tensor_overhead() + ggml_graph_overhead() + 4096,
        .mem_buffer = NULL,
        .no_alloc = true,
    };
    return ggml_init(p);
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int compute(struct ggml_cgraph *gf, int nthreads, int reps, double *secs) {
    struct ggml_cplan plan = ggml_graph_plan(gf, nthreads, NULL);
    void *work = NULL;
    if (plan.work_size > 0) {
        work = malloc(plan.work_size);
        if (!work) return -2;
        plan.work_data = work;
    }
    int rc = 0;
    double t0 = now_s();
    for (int r = 0; r < reps && rc == 0; ++r) {
        if (ggml_graph_compute(gf, &plan) != GGML_STATUS_SUCCESS) rc = -3;
    }
    if (secs) *secs = now_s() - t0;
    free(work);
    return rc;
}

// y[n*M + m] = sum_k W[m, k] * x[n*K + k], W of ggml type `wtype` with rows of
// ggml_row_size(wtype, K) bytes. Runs `reps` times (>= 1); *secs receives the
// wall time of all of them when non-NULL.
int ref_mul_mat(int wtype, const void *w, int64_t M, int64_t K, const float *x, int64_t N, float *y,
                int nthreads, int reps, double *secs) {
    struct ggml_context *ctx = meta_ctx();
    if (!ctx) return -1;
    struct ggml_tensor *a = ggml_new_tensor_2d(ctx, (enum ggml_type)wtype, K, M);
    struct ggml_tensor *b = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, N);
    a->data = (void *)w;
    b->data = (void *)x;
    struct ggml_tensor *c = ggml_mul_mat(ctx, a, b);
    c->data = y;
    struct ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, c);
    int rc = compute(gf, nthreads, reps < 1 ? 1 : reps, secs);
    ggml_free(ctx);
    return rc;
}

// One decode query per head against dense caches of one sequence:
// q f32 [H][D], k/v f16 bits [Hkv][L][D], out f32 [H][D].
int ref_flash_attn(const float *q, const uint16_t *k, const uint16_t *v, int64_t D, int64_t L, int64_t H,
                   int64_t Hkv, float scale, float *out, int nthreads, int reps, double *secs) {
    struct ggml_context *ctx = meta_ctx();
    if (!ctx) return -1;
    struct ggml_tensor *tq = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, D, 1, H, 1);
    struct ggml_tensor *tk = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, D, L, Hkv, 1);
    struct ggml_tensor *tv = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, D, L, Hkv, 1);
    tq->data = (void *)q;
    tk->data = (void *)k;
    tv->data = (void *)v;
    struct ggml_tensor *o = ggml_flash_attn_ext(ctx, tq, tk, tv, NULL, scale, 0.0f, 0.0f);
    // result: [D, H, 1, 1] f32
    o->data = out;
    struct ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, o);
    int rc = compute(gf, nthreads, reps < 1 ? 1 : reps, secs);
    ggml_free(ctx);
    return rc;
}

size_t ref_row_size(int wtype, int64_t K) { return ggml_row_size((enum ggml_type)wtype, K); }

// Contiguous tensors; mask may be NULL. out: [DV, nh, nq, nb] f32.
int ref_flash_attn_ext(const float *q, const uint16_t *k, const uint16_t *v, const uint16_t *mask, int64_t D,
                       int64_t DV, int64_t nq, int64_t nh, int64_t nb, int64_t L, int64_t nhkv, int64_t Lm,
                       int64_t nqm, int64_t mne2, int64_t mne3, float scale, float max_bias, float softcap,
                       float *out, int nthreads, int reps, double *secs) {
    struct ggml_context *ctx = meta_ctx();
    if (!ctx) return -1;
    struct ggml_tensor *tq = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, D, nq, nh, nb);
    struct ggml_tensor *tk = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, D, L, nhkv, nb);
    struct ggml_tensor *tv = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, DV, L, nhkv, nb);
    struct ggml_tensor *tm = NULL;
    tq->data = (void *)q;
    tk->data = (void *)k;
    tv->data = (void *)v;
    if (mask) {
        tm = ggml_new_tensor_4d(ctx, GGML_TYPE_F16, Lm, nqm, mne2, mne3);
        tm->data = (void *)mask;
    }
    struct ggml_tensor *o = ggml_flash_attn_ext(ctx, tq, tk, tv, tm, scale, max_bias, softcap);
    o->data = out;
    struct ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, o);
    int rc = compute(gf, nthreads, reps < 1 ? 1 : reps, secs);
    ggml_free(ctx);
    return rc;
}

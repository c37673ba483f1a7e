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
//   ref_core         one of the ops around them in a decoder step (add/sub/
//                    mul/div, unary ops, norm/rms_norm, get_rows, set_rows,
//                    cpy of a permuted view, rope_ext, soft_max_ext, argmax,
//                    glu).
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

// One core op (kind numbering as tlh_core_kind) on contiguous caller buffers:
// tensor i (0 src0, 1 src1, 2 src2, 3 destination) has ggml type ty[i], extents
// ne[4*i .. 4*i+3] and data data[i] (NULL: absent). ip[] / fp[] hold the
// integer / float arguments of the ggml constructor:
//   BIN 1      ip0 = 0 add, 1 sub, 2 mul, 3 div
//   UNARY 2    ip0 = ggml_unary_op, or 100 scale_bias(fp0, fp1), 101 fill(fp0),
//              102 clamp(fp0, fp1), 103 leaky_relu(fp0), 104 sqr, 105 sqrt,
//              106 sin, 107 cos, 108 log
//   NORM 3     ip0 = 1 rms_norm / 0 norm, eps fp0
//   GET_ROWS 4 / SET_ROWS 5 (destination holds the rows not written)
//   CPY 6      src0 permuted by ip0..ip3 first when ip4 != 0
//   ROPE 7     n_dims ip0, mode ip1, n_ctx_orig ip2; freq_base, freq_scale,
//              ext_factor, attn_factor, beta_fast, beta_slow fp0..fp5
//   SOFT_MAX 8 scale fp0, max_bias fp1 (src1 mask optional)
//   ARGMAX 9
//   GLU 10     ip0 = ggml_glu_op, ip1 = swapped (src1 present: ggml_glu_split)
int ref_core(int kind, const int *ty, const int64_t *ne, void *const *data, const int32_t *ip, const float *fp,
             int nthreads) {
    struct ggml_context *ctx = meta_ctx();
    if (!ctx) return -1;
    struct ggml_tensor *t[4] = {NULL, NULL, NULL, NULL};
    for (int i = 0; i < 4; ++i) {
        if (!data[i]) continue;
        t[i] = ggml_new_tensor_4d(ctx, (enum ggml_type)ty[i], ne[4 * i], ne[4 * i + 1], ne[4 * i + 2], ne[4 * i + 3]);
        t[i]->data = data[i];
    }
    struct ggml_tensor *o = NULL;
    switch (kind) {
    case 1: {
        struct ggml_tensor *(*f[4])(struct ggml_context *, struct ggml_tensor *, struct ggml_tensor *) = {
            ggml_add, ggml_sub, ggml_mul, ggml_div};
        o = f[ip[0] & 3](ctx, t[0], t[1]);
        break;
    }
    case 2:
        switch (ip[0]) {
        case 100: o = ggml_scale_bias(ctx, t[0], fp[0], fp[1]); break;
        case 101: o = ggml_fill(ctx, t[0], fp[0]); break;
        case 102: o = ggml_clamp(ctx, t[0], fp[0], fp[1]); break;
        case 103: o = ggml_leaky_relu(ctx, t[0], fp[0], false); break;
        case 104: o = ggml_sqr(ctx, t[0]); break;
        case 105: o = ggml_sqrt(ctx, t[0]); break;
        case 106: o = ggml_sin(ctx, t[0]); break;
        case 107: o = ggml_cos(ctx, t[0]); break;
        case 108: o = ggml_log(ctx, t[0]); break;
        default: o = ggml_unary(ctx, t[0], (enum ggml_unary_op)ip[0]); break;
        }
        break;
    case 3: o = ip[0] ? ggml_rms_norm(ctx, t[0], fp[0]) : ggml_norm(ctx, t[0], fp[0]); break;
    case 4: o = ggml_get_rows(ctx, t[0], t[1]); break;
    case 5: o = ggml_set_rows(ctx, t[3], t[0], t[1]); break;
    case 6: {
        struct ggml_tensor *a = ip[4] ? ggml_permute(ctx, t[0], ip[0], ip[1], ip[2], ip[3]) : t[0];
        o = ggml_cpy(ctx, a, t[3]);
        break;
    }
    case 7:
        o = ggml_rope_ext(ctx, t[0], t[1], t[2], ip[0], ip[1], ip[2], fp[0], fp[1], fp[2], fp[3], fp[4], fp[5]);
        break;
    case 8: o = ggml_soft_max_ext(ctx, t[0], t[1], fp[0], fp[1]); break;
    case 9: o = ggml_argmax(ctx, t[0]); break;
    case 10:
        o = t[1] ? ggml_glu_split(ctx, t[0], t[1], (enum ggml_glu_op)ip[0])
                 : ggml_glu(ctx, t[0], (enum ggml_glu_op)ip[0], ip[1] != 0);
        break;
    default: ggml_free(ctx); return -4;
    }
    o->data = data[3];
    struct ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, o);
    int rc = compute(gf, nthreads, 1, NULL);
    ggml_free(ctx);
    return rc;
}

// ------------------------------------------------------------ IR graphs
// ref_ir_run: rebuilds a tlh_ir_tensor graph (include/tlhip.h) with the ggml
// constructors each record names, checks that ggml gives every tensor the same
// ne, nb and view placement as the record (so the IR is the graph ggml builds
// from those calls), and computes it on the CPU backend. Leaves point at the
// caller's host arrays by storage index (weights, states -- updated in place
// by SET_ROWS / CPY -- and inputs); `outs` receive copies of the tensors
// `out_ids` (contiguous). Returns 0, or -(1000 + id) for the first tensor whose
// shape, strides or placement differ, or -(2000 + id) for an op it cannot
// rebuild.
#include "../include/tlhip.h"

static int64_t ir_param_offset(const tlh_ir_tensor *r) {
    return (int64_t)(uint32_t)r->op_params[0] | ((int64_t)r->op_params[1] << 32);
}
static float ir_f(const tlh_ir_tensor *r, int i) {
    float f;
    memcpy(&f, &r->op_params[i], 4);
    return f;
}

int ref_ir_run(const tlh_ir_tensor *rec, int n, const int32_t *nodes, int n_nodes, void *const *weights,
               void *const *states, void *const *inputs, const int32_t *out_ids, void *const *outs, int n_outs,
               int nthreads) {
    ggml_cpu_init();
    size_t mem = ggml_graph_overhead_custom(4096 > n ? 4096 : (size_t)n * 2, false) + 1024 * 1024;
    for (int i = 0; i < n; ++i) {
        mem += ggml_tensor_overhead() + 64;
        if (rec[i].view_src < 0 && (strcmp(rec[i].op, "NONE") != 0 || rec[i].storage == TLH_STORE_TEMP)) {
            const int64_t ne = rec[i].ne[0] * rec[i].ne[1] * rec[i].ne[2] * rec[i].ne[3];
            mem += (size_t)(ne * 8 + 256);  // at most 8 bytes an element (i64)
        }
    }
    struct ggml_init_params ip = {.mem_size = mem, .mem_buffer = NULL, .no_alloc = false};
    struct ggml_context *ctx = ggml_init(ip);
    if (!ctx) return -1;
    struct ggml_tensor **t = calloc((size_t)n, sizeof *t);
    int rc = 0;
    for (int i = 0; i < n && rc == 0; ++i) {
        const tlh_ir_tensor *r = &rec[i];
        struct ggml_tensor *s0 = r->src[0] >= 0 ? t[r->src[0]] : NULL, *s1 = r->src[1] >= 0 ? t[r->src[1]] : NULL,
                           *s2 = r->src[2] >= 0 ? t[r->src[2]] : NULL, *s3 = r->src[3] >= 0 ? t[r->src[3]] : NULL;
        const char *op = r->op;
        struct ggml_tensor *x = NULL;
        if (!strcmp(op, "NONE") && r->storage == TLH_STORE_TEMP) {
            // a new tensor without a source (ggml_cast's destination): context memory
            x = ggml_new_tensor_4d(ctx, (enum ggml_type)r->ty, r->ne[0], r->ne[1], r->ne[2], r->ne[3]);
        } else if (!strcmp(op, "NONE")) {
            // leaves point at the caller's arrays: no context memory for their data
            ggml_set_no_alloc(ctx, true);
            x = ggml_new_tensor_4d(ctx, (enum ggml_type)r->ty, r->ne[0], r->ne[1], r->ne[2], r->ne[3]);
            ggml_set_no_alloc(ctx, false);
            void *const *leaf = r->storage == TLH_STORE_WEIGHT ? weights : r->storage == TLH_STORE_STATE ? states
                                : r->storage == TLH_STORE_INPUT ? inputs : NULL;
            if (!leaf) {
                rc = -(2000 + i);
                break;
            }
            x->data = leaf[r->storage_index];
        } else if (!strcmp(op, "VIEW")) {
            x = ggml_view_4d(ctx, s0, r->ne[0], r->ne[1], r->ne[2], r->ne[3], r->nb[1], r->nb[2], r->nb[3],
                             (size_t)ir_param_offset(r));
        } else if (!strcmp(op, "RESHAPE")) {
            x = ggml_reshape_4d(ctx, s0, r->ne[0], r->ne[1], r->ne[2], r->ne[3]);
        } else if (!strcmp(op, "PERMUTE")) {
            x = ggml_permute(ctx, s0, r->op_params[0], r->op_params[1], r->op_params[2], r->op_params[3]);
        } else if (!strcmp(op, "TRANSPOSE")) {
            x = ggml_transpose(ctx, s0);
        } else if (!strcmp(op, "CONT")) {
            x = ggml_cont_4d(ctx, s0, r->ne[0], r->ne[1], r->ne[2], r->ne[3]);
        } else if (!strcmp(op, "CPY")) {
            x = ggml_cpy(ctx, s0, s1);
        } else if (!strcmp(op, "MUL_MAT")) {
            x = ggml_mul_mat(ctx, s0, s1);
        } else if (!strcmp(op, "MUL_MAT_ID")) {
            x = ggml_mul_mat_id(ctx, s0, s1, s2);
        } else if (!strcmp(op, "ADD")) {
            x = r->view_src >= 0 ? ggml_add_inplace(ctx, s0, s1) : ggml_add(ctx, s0, s1);
        } else if (!strcmp(op, "SUB")) {
            x = ggml_sub(ctx, s0, s1);
        } else if (!strcmp(op, "MUL")) {
            x = ggml_mul(ctx, s0, s1);
        } else if (!strcmp(op, "DIV")) {
            x = ggml_div(ctx, s0, s1);
        } else if (!strcmp(op, "RMS_NORM")) {
            x = ggml_rms_norm(ctx, s0, ir_f(r, 0));
        } else if (!strcmp(op, "NORM")) {
            x = ggml_norm(ctx, s0, ir_f(r, 0));
        } else if (!strcmp(op, "UNARY")) {
            x = ggml_unary(ctx, s0, (enum ggml_unary_op)r->op_params[0]);
        } else if (!strcmp(op, "SCALE")) {
            x = ggml_scale_bias(ctx, s0, ir_f(r, 0), ir_f(r, 1));
        } else if (!strcmp(op, "GET_ROWS")) {
            x = ggml_get_rows(ctx, s0, s1);
        } else if (!strcmp(op, "SET_ROWS")) {
            x = ggml_set_rows(ctx, t[r->view_src], s0, s1);
        } else if (!strcmp(op, "ROPE")) {
            x = ggml_rope_ext(ctx, s0, s1, s2, r->op_params[1], r->op_params[2], r->op_params[4], ir_f(r, 5),
                              ir_f(r, 6), ir_f(r, 7), ir_f(r, 8), ir_f(r, 9), ir_f(r, 10));
        } else if (!strcmp(op, "SOFT_MAX")) {
            x = ggml_soft_max_ext(ctx, s0, s1, ir_f(r, 0), ir_f(r, 1));
        } else if (!strcmp(op, "FLASH_ATTN_EXT")) {
            x = ggml_flash_attn_ext(ctx, s0, s1, s2, s3, ir_f(r, 0), ir_f(r, 1), ir_f(r, 2));
        } else if (!strcmp(op, "GLU")) {
            x = s1 ? ggml_glu_split(ctx, s0, s1, (enum ggml_glu_op)r->op_params[0])
                   : ggml_glu(ctx, s0, (enum ggml_glu_op)r->op_params[0], r->op_params[1] != 0);
        } else if (!strcmp(op, "ARGMAX")) {
            x = ggml_argmax(ctx, s0);
        } else {
            rc = -(2000 + i);
            break;
        }
        t[i] = x;
        int same = x->type == (enum ggml_type)r->ty;
        for (int d = 0; d < 4; ++d) same = same && x->ne[d] == r->ne[d] && (int64_t)x->nb[d] == r->nb[d];
        if (r->view_src >= 0) same = same && x->view_src == t[r->view_src] && (int64_t)x->view_offs == r->view_offs;
        else same = same && x->view_src == NULL;
        if (!same) rc = -(1000 + i);
    }
    if (rc == 0) {
        struct ggml_cgraph *gf = ggml_new_graph_custom(ctx, 4096 > n ? 4096 : (size_t)n * 2, false);
        for (int k = 0; k < n_nodes; ++k) ggml_build_forward_expand(gf, t[nodes[k]]);
        rc = compute(gf, nthreads, 1, NULL);
        for (int k = 0; k < n_outs && rc == 0; ++k) memcpy(outs[k], t[out_ids[k]]->data, ggml_nbytes(t[out_ids[k]]));
    }
    free(t);
    ggml_free(ctx);
    return rc;
}

// ------------------------------------------------------------------ GGUF
// ggml's own GGUF reader and writer (vendor/ggml/src/gguf.cpp), to pin the
// product's reader: ref_gguf_* describe a file as ggml parses it, and
// ref_gguf_write_sample writes one with ggml's writer.
#include "gguf.h"

typedef struct {
    struct gguf_context *g;
    struct ggml_context *ctx;
} ref_gguf;

void *ref_gguf_open(const char *path) {
    ref_gguf *h = calloc(1, sizeof *h);
    struct gguf_init_params p = {.no_alloc = true, .ctx = &h->ctx};
    h->g = gguf_init_from_file(path, p);
    if (!h->g) {
        free(h);
        return NULL;
    }
    return h;
}
void ref_gguf_close(void *hp) {
    ref_gguf *h = hp;
    if (!h) return;
    gguf_free(h->g);
    if (h->ctx) ggml_free(h->ctx);
    free(h);
}
void ref_gguf_info(void *hp, int64_t *n_tensors, int64_t *n_kv, size_t *alignment, size_t *data_offset,
                   uint32_t *version) {
    ref_gguf *h = hp;
    *n_tensors = gguf_get_n_tensors(h->g);
    *n_kv = gguf_get_n_kv(h->g);
    *alignment = gguf_get_alignment(h->g);
    *data_offset = gguf_get_data_offset(h->g);
    *version = gguf_get_version(h->g);
}
void ref_gguf_tensor(void *hp, int64_t i, char *name, int *type, int64_t *ne, size_t *offset, size_t *bytes) {
    ref_gguf *h = hp;
    const char *n = gguf_get_tensor_name(h->g, i);
    strncpy(name, n, 63);
    name[63] = 0;
    *type = (int)gguf_get_tensor_type(h->g, i);
    *offset = gguf_get_tensor_offset(h->g, i);
    *bytes = gguf_get_tensor_size(h->g, i);
    const struct ggml_tensor *t = ggml_get_tensor(h->ctx, n);
    for (int d = 0; d < 4; ++d) ne[d] = t->ne[d];
}
const char *ref_gguf_key(void *hp, int64_t i, int *type, int *arr_type, size_t *n) {
    ref_gguf *h = hp;
    *type = (int)gguf_get_kv_type(h->g, i);
    *arr_type = *type == GGUF_TYPE_ARRAY ? (int)gguf_get_arr_type(h->g, i) : -1;
    *n = *type == GGUF_TYPE_ARRAY ? gguf_get_arr_n(h->g, i) : 1;
    return gguf_get_key(h->g, i);
}
const void *ref_gguf_data(void *hp, int64_t i) {
    ref_gguf *h = hp;
    return gguf_get_kv_type(h->g, i) == GGUF_TYPE_ARRAY ? gguf_get_arr_data(h->g, i) : gguf_get_val_data(h->g, i);
}
const char *ref_gguf_str(void *hp, int64_t i, int64_t j) {
    ref_gguf *h = hp;
    return gguf_get_kv_type(h->g, i) == GGUF_TYPE_ARRAY ? gguf_get_arr_str(h->g, i, j) : gguf_get_val_str(h->g, i);
}

// A file written by ggml's writer: every scalar type, strings, arrays of
// u32 / f32 / strings, general.alignment when `alignment` != 0, and tensors of
// several types and ranks with deterministic contents.
int ref_gguf_write_sample(const char *path, uint32_t alignment) {
    struct gguf_context *g = gguf_init_empty();
    gguf_set_val_u8(g, "t.u8", 200);
    gguf_set_val_i8(g, "t.i8", -100);
    gguf_set_val_u16(g, "t.u16", 60000);
    gguf_set_val_i16(g, "t.i16", -30000);
    gguf_set_val_u32(g, "t.u32", 4000000000u);
    gguf_set_val_i32(g, "t.i32", -2000000000);
    gguf_set_val_f32(g, "t.f32", 3.25f);
    gguf_set_val_bool(g, "t.bool", true);
    gguf_set_val_str(g, "t.str", "a string, unicode \\xc3\\xa9");
    gguf_set_val_u64(g, "t.u64", 18000000000000000000ull);
    gguf_set_val_i64(g, "t.i64", -9000000000000000000ll);
    gguf_set_val_f64(g, "t.f64", -1.0e300);
    const uint32_t au[5] = {1, 2, 3, 4, 5};
    gguf_set_arr_data(g, "t.arr_u32", GGUF_TYPE_UINT32, au, 5);
    const float af[3] = {0.5f, -1.5f, 1e-20f};
    gguf_set_arr_data(g, "t.arr_f32", GGUF_TYPE_FLOAT32, af, 3);
    const char *as[3] = {"x", "", "longer string"};
    gguf_set_arr_str(g, "t.arr_str", as, 3);
    if (alignment) gguf_set_val_u32(g, "general.alignment", alignment);
    struct ggml_init_params ip = {.mem_size = 1 << 20, .mem_buffer = NULL, .no_alloc = false};
    struct ggml_context *ctx = ggml_init(ip);
    const struct {
        const char *name;
        enum ggml_type ty;
        int nd;
        int64_t ne[4];
    } ts[] = {{"w.f32", GGML_TYPE_F32, 2, {7, 3}},    {"w.f16", GGML_TYPE_F16, 1, {64}},
              {"w.q4_0", GGML_TYPE_Q4_0, 2, {64, 2}}, {"w.q8_0", GGML_TYPE_Q8_0, 3, {32, 3, 2}},
              {"w.q4_K", GGML_TYPE_Q4_K, 2, {256, 2}}, {"w.q6_K", GGML_TYPE_Q6_K, 1, {512}},
              {"w.i32", GGML_TYPE_I32, 4, {5, 1, 1, 2}}};
    for (size_t k = 0; k < sizeof ts / sizeof ts[0]; ++k) {
        struct ggml_tensor *t = ggml_new_tensor(ctx, ts[k].ty, ts[k].nd, ts[k].ne);
        ggml_set_name(t, ts[k].name);
        uint8_t *d = t->data;
        for (size_t b = 0; b < ggml_nbytes(t); ++b) d[b] = (uint8_t)(b * 31 + k * 7);
        gguf_add_tensor(g, t);
    }
    const bool ok = gguf_write_to_file(g, path, false);
    ggml_free(ctx);
    gguf_free(g);
    return ok ? 0 : -1;
}

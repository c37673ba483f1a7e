/*
 * tlhip.h — C ABI of the MI355X (gfx950) executor for tensorlisp's quantized
 * hot path: GGML_OP_MUL_MAT over GGUF block-quantized weights (Q8_0, Q4_0,
 * Q4_K, Q5_K, Q6_K; decode GEMV for N <= 16 columns, MFMA GEMM for prefill),
 * paged-attention decode over an f16 block-table KV cache, and dense
 * GGML_OP_FLASH_ATTN_EXT over f16 K/V.
 *
 * This is the surface a `native-hip` feature binds from Rust
 * (crates/kernels/src/hip/ + crates/tensorlisp/src/native_hip.rs), in place of
 * the NVRTC launcher of crates/kernels/src/cuda/{mod,exec,lower}.rs. Plain C:
 * pointers, sizes and PODs; no torch or HIP types in the signatures (a stream
 * is an opaque `void*` that is a hipStream_t, NULL = the null stream).
 *
 * Conventions (mirroring crates/kernels/src/lib.rs:44-61 and
 * crates/kernels/src/cuda/mod.rs):
 *  - every call returns a tlh_status; tlh_last_error() gives this thread's
 *    text for the last failure;
 *  - work calls are stream-ordered and asynchronous; nothing allocates behind
 *    the caller's back except where a function says so (tlh_alloc);
 *  - device pointers are plain device addresses on the current device.
 */
#ifndef TLHIP_H
#define TLHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error kinds of tensorlisp_kernels::Error (crates/kernels/src/lib.rs:44-61):
 * NoDevice, Unsupported{op,node,why}, Invalid, Alloc(bytes), Execution(msg). */
typedef enum tlh_status {
    TLH_OK = 0,
    TLH_NO_DEVICE = 1,
    TLH_UNSUPPORTED = 2,
    TLH_INVALID = 3,
    TLH_ALLOC = 4,
    TLH_EXECUTION = 5
} tlh_status;

/* ggml type numbers (vendor/ggml/include/ggml.h:390-417). */
enum {
    TLH_TYPE_F32 = 0,
    TLH_TYPE_F16 = 1,
    TLH_TYPE_Q4_0 = 2,
    TLH_TYPE_Q4_1 = 3,
    TLH_TYPE_Q5_0 = 6,
    TLH_TYPE_Q5_1 = 7,
    TLH_TYPE_Q8_0 = 8,
    TLH_TYPE_Q8_1 = 9,
    TLH_TYPE_Q2_K = 10,
    TLH_TYPE_Q3_K = 11,
    TLH_TYPE_Q4_K = 12,
    TLH_TYPE_Q5_K = 13,
    TLH_TYPE_Q6_K = 14,
    TLH_TYPE_Q8_K = 15,
    TLH_TYPE_I32 = 26,
    TLH_TYPE_I64 = 27,
    TLH_TYPE_BF16 = 30
};

/* Thread-local text of the last failure on this thread ("" if none). */
const char *tlh_last_error(void);
const char *tlh_status_name(tlh_status s);
/* Library version string, e.g. "tlhip 0.1 gfx950". */
const char *tlh_version(void);

/* ------------------------------------------------------------------ device
 * Replaces Device::system_default / name (crates/kernels/src/cuda/mod.rs:244-277):
 * TLH_NO_DEVICE when no GPU is present (not fatal at probe time). Opening
 * makes the device current on the calling thread. */
typedef struct tlh_device_props {
    char name[64];
    char arch[32];       /* e.g. "gfx950" */
    int compute_units;
    int wave_size;       /* 64 on CDNA */
    int lds_bytes;       /* per workgroup */
    int clock_khz;
    int64_t hbm_bytes;
} tlh_device_props;

tlh_status tlh_device_count(int *count);
tlh_status tlh_device_open(int ordinal, tlh_device_props *props);

/* ------------------------------------------------------------------ memory
 * Replaces Buffer (crates/kernels/src/cuda/mod.rs:39-133): alloc/free and
 * blocking copies, plus a stream-ordered sync (mod.rs:544-548). */
tlh_status tlh_alloc(size_t bytes, void **ptr);
tlh_status tlh_free(void *ptr);
tlh_status tlh_h2d(void *dst, const void *src, size_t bytes);
tlh_status tlh_d2h(void *dst, const void *src, size_t bytes);
tlh_status tlh_stream_sync(void *stream);

/* ---------------------------------------------------------- op descriptor
 * struct T / struct Op of crates/kernels/src/cuda/native/common.cuh:14-26, as
 * packed by OpBlob (crates/kernels/src/cuda/lower.rs:67-99): 5 tensors (slots
 * 0..3 sources, 4 the destination) of ggml ne/nb/type, then 12 scalar slots
 * (ints, or floats as their bit pattern). 456 bytes. */
typedef struct tlh_tensor {
    int64_t ne[4];
    int64_t nb[4];
    int32_t ty;
    int32_t pad_;
} tlh_tensor;

typedef struct tlh_op {
    tlh_tensor t[5];
    int64_t x[12];
} tlh_op;

/* --------------------------------------------------------------- MUL_MAT
 * GGML_OP_MUL_MAT, replacing Ctx::mul_mat (crates/kernels/src/cuda/lower.rs:543-571)
 * and its mm_vec / mm_tile kernels (crates/kernels/src/cuda/native/mm.cu:16-103),
 * computed the way the ggml CPU backend does (vendor/ggml/src/ggml-cpu/ggml-cpu.c:1254-1457):
 *   op->t[0] src0: weights, type Q4_0 | Q4_1 | Q5_0 | Q5_1 | Q8_0 | Q4_K | Q5_K | Q6_K |
 *                  F32 | F16 | BF16,
 *                  ne [K, M, ne02, ne03], nb[0] = block (element) bytes (rows must
 *                  not be transposed);
 *   op->t[1] src1: f32 activations (or, for F16 / BF16 weights, already of the
 *                  weight type), ne [K, N, ne12, ne13], nb[0] = element bytes;
 *   op->t[4] dst:  f32 [M, N, ne12, ne13], nb[0] = 4;
 *   op->x[0] = r2 = ne12 / ne02, op->x[1] = r3 = ne13 / ne03 (broadcast).
 * src1 is first quantized to the weight type's vec_dot type (Q8_0 for Q4_0, Q5_0
 * and Q8_0, Q8_1 for Q4_1 and Q5_1, Q8_K for Q4_K, Q5_K and Q6_K) into `scratch`
 * (at least tlh_mul_mat_scratch_bytes);
 * then N <= 16 runs the decode GEMV (register kernel for N <= 2, int8-MFMA
 * few-column kernel above), larger N the MFMA GEMM. Integer block
 * sums are exact; the f32 result agrees with the CPU backend to rounding of
 * the f32 accumulation order. F32 / F16 / BF16 weights follow the CPU's float
 * rows (ggml-cpu.c:215-226, :394-399): src1 rounded to the weight type, f32
 * products summed in f32, one launch (tlh_mul_mat_scratch_bytes still counts
 * the converted src1 rows, which only the split form below writes).
 * TLH_UNSUPPORTED (with the reason in tlh_last_error) for any
 * other type or layout. */
tlh_status tlh_mul_mat_scratch_bytes(const tlh_op *op, size_t *bytes);
tlh_status tlh_mul_mat(const tlh_op *op, const void *src0, const void *src1, void *dst, void *scratch,
                       size_t scratch_bytes, void *stream);

/* tlh_mul_mat with no caller scratch and no allocation, for callers that
 * cannot allocate device memory per call: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. No counterpart in the
 * reference (its launcher allocates nothing per call but always passes
 * buffers it owns). Same kernels, descriptor and results as tlh_mul_mat; the
 * scratch is a static device array of TLH_NOALLOC_SCRATCH_BYTES that each GPU
 * holds for the life of the process, resolved on tlh_device_open (or on the
 * first call on a device). A node whose tlh_mul_mat_scratch_bytes exceeds it
 * is refused with TLH_INVALID (nothing is launched). The array keeps the last
 * call's contents and nothing in it has to start at zero; all calls on one GPU
 * share it, so calls that overlap in time on one GPU (other streams, other
 * threads) race: order them on one stream. Calls no hipMalloc/hipFree. */
#define TLH_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
tlh_status tlh_mul_mat_noalloc(const tlh_op *op, const void *src0, const void *src1, void *dst, void *stream);

/* The two phases of tlh_mul_mat, which the CPU backend separates with a
 * barrier (ggml-cpu.c:1318-1359 quantize src1 into wdata; :1366 barrier;
 * :1426-1451 the dot products). Splitting them lets an executor quantize an
 * activation once for several weights that consume it (e.g. Q, K and V
 * projections of one input: same src1 shape and weight type, one scratch).
 * tlh_mul_mat_compute reads the scratch a matching tlh_mul_mat_quantize
 * filled (same op shape for src1, same vec_dot type). */
tlh_status tlh_mul_mat_quantize(const tlh_op *op, const void *src1, void *scratch, size_t scratch_bytes,
                                void *stream);
tlh_status tlh_mul_mat_compute(const tlh_op *op, const void *src0, const void *scratch, size_t scratch_bytes,
                               void *dst, void *stream);

/* GGML_OP_MUL_MAT_ID (vendor/ggml/src/ggml.c:3329-3353; CPU
 * ggml_compute_forward_mul_mat_id, ggml-cpu/ggml-cpu.c:1460-1640), which the
 * reference's native lowering has no kernel for (docs/design/kernel-launcher.md:326)
 * and runs on the CPU backend. Descriptor slots: t[0] = as, the expert
 * matrices [K, M, n_as] (q4_0 | q8_0 | q4_K | q5_K | q6_K); t[1] = b f32
 * [K, n_b1, n_tokens] with n_used % n_b1 == 0; t[2] = ids i32 [n_used, n_tokens];
 * t[4] = dst f32 [M, n_used, n_tokens]. dst[:, e, t] = as[:, :, ids[e, t]] times
 * b row (e % n_b1, t), each element the CPU's vec_dot of the quantized row
 * (so within the MUL_MAT tolerance of the CPU backend). An id outside
 * [0, n_as) yields NaN in its column (the CPU backend aborts there). Decode
 * oriented: each (expert, token) pair streams its expert's matrix once. */
tlh_status tlh_mul_mat_id_scratch_bytes(const tlh_op *op, size_t *bytes);
tlh_status tlh_mul_mat_id(const tlh_op *op, const void *src0, const void *src1, const void *ids, void *dst,
                          void *scratch, size_t scratch_bytes, void *stream);

/* Activation quantizer alone: `rows` rows of `k` f32 (row stride x_row_bytes)
 * into ggml's block layout of the vec_dot type of `wtype` — the from_float the
 * CPU mul_mat applies (quantize_row_q8_0 / quantize_row_q8_K:
 * vendor/ggml/src/ggml-cpu/arch/x86/quants.c:302-398, :505-507), bit-exact.
 * Output: rows * row_size(vec_dot_type, k) bytes, rows packed. A block whose
 * values are all zero gets d = 0, zero codes and zero bsums (the reference
 * leaves a zero Q8_K block's bsums unwritten). */
tlh_status tlh_quantize_act(int wtype, const float *x, int64_t k, int64_t rows, int64_t x_row_bytes, void *y,
                            void *stream);

/* dequantize_row_{q4_0,q8_0,q4_K,q5_K,q6_K} (vendor/ggml/src/ggml-quants.c:459-476,
 * :553-565, :1529-1550, :1731-1756, :1939-1968), bit-exact: `rows` rows of `k` elements (row stride
 * w_row_bytes) into f32 [rows][k]. The to_f32 of DType (crates/tensorlisp/src/dtype.rs:80-95). */
tlh_status tlh_dequantize(int type, const void *w, int64_t k, int64_t rows, int64_t w_row_bytes, float *y,
                          void *stream);

/* ------------------------------------------------------- FLASH_ATTN_EXT
 * GGML_OP_FLASH_ATTN_EXT, replacing Ctx::flash_attn_ext and its fa_main /
 * fa_split + fa_reduce kernels (crates/kernels/src/cuda/lower.rs:575-657,
 * split plan :764-792; crates/kernels/src/cuda/native/fa.cu:21-232), computed
 * as the ggml CPU backend does (vendor/ggml/src/ggml-cpu/ops.cpp:8468-8700):
 *   op->t[0] q:    f32 [D, nq, nh, nb], nb[0] = 4;
 *   op->t[1] k:    f16 [D, L, nhkv, nbk], nb[0] = 2, nh % nhkv == 0, nb % nbk == 0;
 *   op->t[2] v:    f16 [DV, L, nhkv, nbk], nb[0] = 2;
 *   op->t[3] mask: f16 [>= L, >= nq, mne2, mne3] (read only when `mask` is
 *                  non-NULL), broadcast over heads (nh % mne2 == 0) and batch;
 *   op->t[4] dst:  f32 [DV, nh, nq, nb], nb[0] = 4;
 *   op->x[0] scale (divided by softcap when softcap != 0), x[1] max_bias,
 *   x[2] m0, x[3] m1 (floats as their bit pattern, sign-extended), x[4]
 *   n_head_log2, x[5] softcap: the OpBlob lower.rs:615-620 packs.
 * K/V base pointers and strides must be 16-byte multiples; head sizes D = DV
 * in {32, 40, 64, 72, 80, 96, 112, 128, 192, 256} or D = 192, DV = 128. No
 * attention sinks (the reference lowering refuses them too). q is rounded to
 * f16 (as the CPU backend does for f16 keys); scores and the softmax are f32,
 * P.V accumulates in f32 (the CPU backend accumulates P.V in f16), so the
 * result agrees with the CPU backend to f16 rounding. Keys with a -inf mask are
 * skipped; a row with every key masked gives 0. `scratch` holds split-key
 * partials (tlh_flash_attn_ext_scratch_bytes; may be NULL when that is 0). */
tlh_status tlh_flash_attn_ext_scratch_bytes(const tlh_op *op, size_t *bytes);
tlh_status tlh_flash_attn_ext(const tlh_op *op, const void *q, const void *k, const void *v, const void *mask,
                              void *dst, void *scratch, size_t scratch_bytes, void *stream);

/* ------------------------------------------------------------ core ops
 * The ggml ops around MUL_MAT and attention in a decoder step (token
 * embedding, norms, residuals, activations, RoPE, KV-cache writes, softmax,
 * greedy sampling), replacing the reference's core kernels
 * (crates/kernels/src/cuda/native/core.cu) as Ctx::lower dispatches them
 * (crates/kernels/src/cuda/lower.rs:175-213, 219-500), computed as the ggml CPU
 * backend does (vendor/ggml/src/ggml-cpu/binary-ops.cpp, unary-ops.cpp,
 * ops.cpp). `op` is the blob the reference's lowering packs: t[0..2] sources,
 * t[4] the destination, x[] the op's parameters (floats as their bit
 * pattern). Data types f32 / f16; index tensors i32 / i64. Results are
 * bit-exact for BIN, CPY, GET_ROWS, SET_ROWS, ARGMAX and the unary ops
 * without a transcendental function; NORM sums in double like the CPU (equal
 * up to the order of the double additions); the others use the GPU's
 * expf/sinf/... (within a few ulp of the CPU's libm; GELU and GELU_QUICK go
 * through f16 like the CPU's tables). A SOFT_MAX row whose every entry is -inf
 * gives zeros (the CPU gives NaN).
 * tlh_core_check validates a node without launching (for planning);
 * tlh_core runs it. A GET_ROWS index outside src0 reads the nearest row and a
 * SET_ROWS index outside dst writes nothing (ggml asserts instead). */
typedef enum tlh_core_kind {
    TLH_CORE_BIN = 1,      /* ADD/SUB/MUL/DIV: x0 = 0/1/2/3; t0 op t1, t1 repeated to t0's shape */
    TLH_CORE_UNARY = 2,    /* UNARY (x0 = ggml_unary_op) and SCALE 100 (x1 s, x2 b), FILL 101 (x1),
                              CLAMP 102 (x1, x2), LEAKY_RELU 103 (x1), SQR 104, SQRT 105, SIN 106,
                              COS 107, LOG 108 (lower.rs:250-290) */
    TLH_CORE_NORM = 3,     /* NORM (x0 = 0) / RMS_NORM (x0 = 1), x1 = eps; f32 rows, unit element stride */
    TLH_CORE_GET_ROWS = 4, /* t0 f32/f16/q4_0/q8_0/q4_K/q5_K/q6_K rows, t1 indices -> t4 f32/f16 */
    TLH_CORE_SET_ROWS = 5, /* t0 f32/f16 rows to the t4 rows named by t1 */
    TLH_CORE_CPY = 6,      /* DUP/CPY/CONT: equal element counts, any shapes/strides */
    TLH_CORE_ROPE = 7,     /* x0 n_dims, x1 mode (0 normal, 2 neox), x2 freq_scale, x3 ext_factor,
                              x4 attn_factor, x5 freq_base^(-2/n_dims), x6/x7 YaRN corr dims,
                              x8 = 1 with f32 frequency factors in src2; t1 i32 positions */
    TLH_CORE_SOFT_MAX = 8, /* x0 scale, x1 max_bias, x2 m0, x3 m1, x4 n_head_log2; t0 f32; mask src1
                              f32/f16, optional (lower.rs:314-341) */
    TLH_CORE_ARGMAX = 9,   /* t0 f32 [n, rows] -> t4 i32 [rows] (last index of the maximum) */
    TLH_CORE_GLU = 10      /* GGML_OP_GLU, f32: x0 = ggml_glu_op (0 reglu, 1 geglu, 2 swiglu, 4 geglu_erf,
                              5 geglu_quick), x1 = swapped; t0 [2n, ...] halves, or t0 and t1 [n, ...]
                              (split form). No counterpart in the reference's lowering, which leaves
                              GLU unsupported; computed as ops.cpp ggml_compute_forward_glu does */
} tlh_core_kind;

tlh_status tlh_core_check(int kind, const tlh_op *op, int has_src1, int has_src2);
tlh_status tlh_core(int kind, const tlh_op *op, const void *src0, const void *src1, const void *src2, void *dst,
                    void *stream);

/* ------------------------------------------------------- paged attention
 * The `paged-attention` custom node (crates/tensorlisp/src/scheme/core.ss:251-258),
 * lowered by Ctx::custom kind 1 (crates/kernels/src/cuda/lower.rs:672-731) to
 * vLLM's paged_attention_v1/v2 (crates/kernels/src/cuda/paged_attn.rs:326-417).
 * Layouts (f16 elements, x = 8):
 *   q        [num_seqs][num_heads][head_size] (contiguous)
 *   k_cache  [num_blocks][num_kv_heads][head_size/8][block_size][8]
 *   v_cache  [num_blocks][num_kv_heads][head_size][block_size]
 *   block_tables i32 [num_seqs][max_blocks_per_seq], context_lens i32 [num_seqs]
 *   out      [num_seqs][num_heads][head_size]
 * head_size in {64, 80, 96, 112, 128, 192, 256}, block_size in {8, 16, 32},
 * num_heads % num_kv_heads == 0, context lens <= max_context_len.
 * `scratch` holds split-context partials (tlh_paged_attention_scratch_bytes,
 * which never shrinks as num_seqs or max_context_len grow, so one buffer sized
 * for the largest batch and context serves every smaller call); it may be
 * NULL when that size is 0. */
typedef struct tlh_paged_attention_args {
    void *out;
    const void *q;
    const void *k_cache;
    const void *v_cache;
    const int32_t *block_tables;
    const int32_t *context_lens;
    int32_t num_seqs;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_size;
    int32_t block_size;
    int32_t max_blocks_per_seq;
    int32_t max_context_len;
    float scale;
} tlh_paged_attention_args;

tlh_status tlh_paged_attention_scratch_bytes(const tlh_paged_attention_args *a, size_t *bytes);
tlh_status tlh_paged_attention(const tlh_paged_attention_args *a, void *scratch, size_t scratch_bytes,
                               void *stream);

/* The `paged-cache-write` custom node (core.ss:265-272), Ctx::custom kind 2
 * (lower.rs:732-753) -> reshape_and_cache (crates/kernels/src/cuda/shaders/
 * reshape_and_cache_kernel.cu:31-84): key/value f16 [num_tokens][num_kv_heads*head_size]
 * into the caches at slot = block * block_size + offset; negative slots skip.
 * num_blocks is the pools' length in blocks (the caller's pool tensors give
 * it): a slot at or past num_blocks * block_size writes nothing, so a bad
 * slot cannot write outside the pools. */
tlh_status tlh_reshape_and_cache(const void *key, const void *value, void *k_cache, void *v_cache,
                                 const int64_t *slots, int32_t num_tokens, int32_t num_kv_heads, int32_t head_size,
                                 int32_t block_size, int64_t num_blocks, void *stream);

/* ------------------------------------------------------------ executor
 * A graph of ggml nodes compiled once into a recorded list of launches on this
 * library's kernels and replayed per run, replacing the reference's
 * Executor::compile / Program::run (crates/kernels/src/cuda/exec.rs:27-226)
 * over its IR (crates/kernels/src/graph.rs:72-229) and memory plan
 * (crates/kernels/src/plan.rs:56-189). The caller hands over the IR the
 * reference builds from a ggml graph (native_ir.rs lower_graph): one record
 * per tensor, the node order and the tensors that must outlive the run.
 *
 * Memory: weights stay where the caller put them (a device pointer per weight
 * index); state tensors live in one caller buffer at fixed byte offsets (per
 * state index), handed over per run so sessions can swap blocks; inputs live
 * in an io buffer and temporaries in an arena, both owned by the program. The
 * arena reuses a tensor's bytes once its last reader has run (first fit by
 * start position, 256-byte alignment), and holds each node's scratch.
 * MUL_MAT nodes that read the same activation with the same weight type
 * quantize it once: the first one writes the q8 blocks into a scratch block
 * that lives until the last of them has run (when the activation has more
 * than two columns; at one or two the GEMV quantizes on the fly, which saves
 * a launch).
 *
 * Lowering follows the reference's Ctx::lower (lower.rs:175-213): view ops
 * and empty tensors produce nothing; MUL_MAT, FLASH_ATTN_EXT and the core ops
 * go to the entry points above with the blobs Ctx packs. Every node is lowered
 * before failing, and one TLH_UNSUPPORTED names each missing op with a count
 * and an example, as exec.rs:39-58 reports them.
 *
 * Runs: tlh_program_run enqueues the launches on `stream`; with `graph` != 0
 * the launches are captured once into a hipGraph (per state buffer and stream)
 * and replayed with one hipGraphLaunch. Calls on one program must not overlap. */
typedef enum tlh_storage {
    TLH_STORE_TEMP = 0,   /* computed in the arena */
    TLH_STORE_WEIGHT = 1, /* weights[storage_index] */
    TLH_STORE_STATE = 2,  /* state buffer + state_offsets[storage_index] */
    TLH_STORE_INPUT = 3   /* input storage_index, in the program's io buffer */
} tlh_storage;

typedef struct tlh_ir_tensor {
    char op[24];            /* ggml op name ("MUL_MAT", "RMS_NORM", ...; "NONE" for leaves) */
    int32_t ty;             /* ggml type */
    int32_t storage;        /* tlh_storage; meaningful for roots */
    int32_t storage_index;
    int32_t view_src;       /* -1, or the root tensor whose storage this view aliases */
    int64_t view_offs;      /* byte offset into view_src */
    int64_t ne[4];
    int64_t nb[4];
    int32_t op_params[16];  /* as ggml stores them */
    int32_t src[10];        /* tensor ids, -1 = none */
} tlh_ir_tensor;

typedef struct tlh_program tlh_program;

/* Plans and lowers; allocates the arena and io buffer on the current device.
 * weights: n_weights device pointers; state_offsets: byte offset of each state
 * tensor in the state buffer given to tlh_program_run. */
tlh_status tlh_program_compile(const tlh_ir_tensor *tensors, int32_t n_tensors, const int32_t *nodes,
                               int32_t n_nodes, const int32_t *keep, int32_t n_keep, const void *const *weights,
                               int32_t n_weights, const int64_t *state_offsets, int32_t n_states,
                               tlh_program **program);
tlh_status tlh_program_destroy(tlh_program *p);
/* Stream-ordered copy between any two device (or pinned host) addresses. */
tlh_status tlh_copy(void *dst, const void *src, size_t bytes, void *stream);
/* Stream-ordered fill of `bytes` device bytes at dst with the low 8 bits of
   `value`, by a kernel (so it may be captured in a hipGraph). Replaces the
   CUDA backend's cuMemsetD8Async zero fill (Backend::zero,
   crates/kernels/src/cuda/backend.rs:334-343). */
tlh_status tlh_memset(void *dst, int value, size_t bytes, void *stream);
/* No counterpart in the reference: a plain streaming read of `bytes` bytes
   (16-byte aligned; `grid` workgroups of 256 lanes, `loads` = 1 or 4 16-byte
   loads in flight per lane) that writes nothing. For measurement only: the
   floor a kernel that must read the same bytes cannot beat, timed beside the
   GEMVs by bench.py. */
tlh_status tlh_read_floor(const void *src, size_t bytes, int32_t grid, int32_t loads, void *stream);
/* Device address and byte size of graph input i in the io buffer. */
tlh_status tlh_program_input(const tlh_program *p, int32_t i, void **ptr, size_t *bytes);
/* Device address of tensor `id` (any storage; `state` is the run's state buffer). */
tlh_status tlh_program_tensor(const tlh_program *p, int32_t id, void *state, void **ptr);
tlh_status tlh_program_run(tlh_program *p, void *state, void *stream, int32_t graph);
/* Sizes: arena bytes, io bytes, and the number of recorded dispatches (one
 * per lowered node, plus one quantization per MUL_MAT group; a dispatch may
 * launch more than one kernel). */
tlh_status tlh_program_stats(const tlh_program *p, size_t *arena_bytes, size_t *io_bytes, int32_t *launches);
/* Per-dispatch timing, in place of the reference's TL_NATIVE_PROFILE per-op
 * times (crates/kernels/src/cuda/exec.rs:186-216): one eager run of the program
 * on `stream` with an event after every dispatch; ms[i] = GPU milliseconds of
 * dispatch i (n >= the dispatch count of tlh_program_stats). Synchronous.
 * With the environment variable TLH_NATIVE_PROFILE set, every eager
 * tlh_program_run does the same and prints the ops with the most time to
 * stderr, as the reference does. */
tlh_status tlh_program_profile(tlh_program *p, void *state, void *stream, float *ms, int32_t n);
/* One eager run of the program on `stream` that records which kernels each
 * dispatch launched (no counterpart in the reference; its exec.rs labels
 * dispatches only by op). `text` receives one line per dispatch:
 * "<index>\t<ggml op of its first node>\t<launch labels, comma-separated>\n"
 * (labels as the launch sites name them: "gemv", "gemv_mfma", "gemv_cols",
 * "gemm_q4k", "gemm_q8", "flash_attn_ext", "flash_attn_ext (rows)",
 * "paged_attention", "norm_chain", ...), NUL-terminated and truncated to `cap`
 * bytes; *len (optional) = the bytes the whole text needs. Not synchronous. */
tlh_status tlh_program_trace(tlh_program *p, void *state, void *stream, char *text, size_t cap, size_t *len);
/* The plan without a device (for checking it): arena offset per tensor (-1 if
 * not in the arena), per-node scratch offset (-1 if none) and the arena size.
 * Scratch sizes come from the same entry points compile uses. */
tlh_status tlh_program_plan(const tlh_ir_tensor *tensors, int32_t n_tensors, const int32_t *nodes, int32_t n_nodes,
                            const int32_t *keep, int32_t n_keep, int64_t *tensor_offsets, int64_t *scratch_offsets,
                            size_t *arena_bytes);

/* ------------------------------------------------------------------ GGUF
 * Reading a GGUF model and loading its tensors into device memory, in place
 * of the reference's load for its native executors
 * (crates/tensorlisp/src/native_cuda.rs:44-82, reading through ggml's
 * gguf.cpp as crates/tensorlisp/src/gguf.rs:79-320 does). The file is checked
 * with ggml's rules (versions 2-3; general.alignment a u32 power of two,
 * default 32; tensor names under 64 bytes, unique; at most 4 dimensions; rows
 * of whole blocks; tensor offsets consecutive at the alignment); a refusal is
 * TLH_INVALID (TLH_UNSUPPORTED for a ggml type this loader cannot size) with
 * the reason. Key-value pairs keep their GGUF types (gguf_type numbering);
 * numeric values and arrays come back as their raw little-endian bytes.
 * tlh_gguf_layout places every tensor 256-byte aligned in one buffer of
 * `total` bytes; tlh_gguf_upload copies the file's tensor data there through
 * pinned staging buffers (a synchronous call on `stream`). */
typedef struct tlh_gguf tlh_gguf;
typedef struct tlh_gguf_tensor_info {
    char name[64];
    int32_t ty;      /* ggml type */
    int32_t n_dims;
    int64_t ne[4];
    uint64_t offset; /* in the data section */
    uint64_t bytes;
} tlh_gguf_tensor_info;

tlh_status tlh_gguf_open(const char *path, tlh_gguf **g);
tlh_status tlh_gguf_close(tlh_gguf *g);
tlh_status tlh_gguf_counts(const tlh_gguf *g, uint32_t *version, int64_t *n_tensors, int64_t *n_kv,
                           uint64_t *alignment, uint64_t *data_offset);
tlh_status tlh_gguf_tensor(const tlh_gguf *g, int64_t i, tlh_gguf_tensor_info *info);
tlh_status tlh_gguf_find_tensor(const tlh_gguf *g, const char *name, int64_t *i); /* -1 when absent */
tlh_status tlh_gguf_find_key(const tlh_gguf *g, const char *key, int64_t *i);     /* -1 when absent */
/* type: gguf_type of the value; for arrays (9) also the element type and count */
tlh_status tlh_gguf_key(const tlh_gguf *g, int64_t i, const char **key, int32_t *type, int32_t *arr_type,
                        uint64_t *n);
tlh_status tlh_gguf_value(const tlh_gguf *g, int64_t i, const void **data, size_t *bytes); /* numeric / bool */
tlh_status tlh_gguf_string(const tlh_gguf *g, int64_t i, uint64_t j, const char **s, uint64_t *len);
tlh_status tlh_gguf_layout(const tlh_gguf *g, uint64_t *offsets, uint64_t *total);
tlh_status tlh_gguf_upload(const tlh_gguf *g, void *dev, const uint64_t *offsets, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* TLHIP_H */

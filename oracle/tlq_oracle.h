// Test infrastructure only. The CPU oracle of the quantized MUL_MAT,
// FLASH_ATTN_EXT and paged-attention hot path: a plain-C restatement of the arithmetic the
// reference runs on its CPU backend (vendored ggml) and in its paged-attention
// kernels (vendored vLLM via crates/kernels/src/cuda/shaders). Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
// only as a checker: the product library never links or calls it.
//
// Every function cites the reference file:line it follows (paths relative to
// the reference repository root). How each one is pinned (against the compiled
// reference ggml in oracle/_ref, closed forms, invariants, brute force) is
// recorded next to its test under tests/.
#ifndef TLQ_ORACLE_H
#define TLQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ggml type numbers, vendor/ggml/include/ggml.h:390-405.
enum {
    TLQ_F32 = 0,
    TLQ_F16 = 1,
    TLQ_Q4_0 = 2,
    TLQ_Q4_1 = 3,
    TLQ_Q5_0 = 6,
    TLQ_Q5_1 = 7,
    TLQ_Q8_0 = 8,
    TLQ_Q8_1 = 9,
    TLQ_Q2_K = 10,
    TLQ_Q3_K = 11,
    TLQ_Q4_K = 12,
    TLQ_Q5_K = 13,
    TLQ_Q6_K = 14,
    TLQ_Q8_K = 15,
    TLQ_BF16 = 30,
};

// Block geometry, vendor/ggml/src/ggml-common.h:89-90,194-198,201-269 (q4_1, q5_0,
// q5_1, q8_1: 20, 22, 24, 36 bytes per 32),298-323 (q2_K, q3_K: 84, 110 bytes
// per 256),325-337,370-375.
int64_t tlq_block_elems(int type);
int64_t tlq_block_bytes(int type);
int64_t tlq_row_bytes(int type, int64_t k);
// vec_dot_type of a weight type on x86 (ggml-cpu.c:215-226,239-319,394-399):
// Q8_0 for Q4_0, Q5_0 and Q8_0 weights, Q8_1 for Q4_1 and Q5_1, Q8_K for the
// K-quants (q2_K..q6_K), the weight type itself for F32 / F16 / BF16; -1 otherwise.
int tlq_vec_dot_type(int wtype);

// IEEE binary16 <-> binary32 (round to nearest even), the semantics of
// ggml_compute_fp16_to_fp32 / ggml_compute_fp32_to_fp16 (ggml-impl.h:384-430).
float tlq_fp16_to_fp32(uint16_t h);
uint16_t tlq_fp32_to_fp16(float f);
void tlq_fp16_to_fp32_row(const uint16_t *h, float *f, int64_t n);
void tlq_fp32_to_fp16_row(const float *f, uint16_t *h, int64_t n);
// bfloat16 <-> binary32: ggml_compute_bf16_to_fp32 / ggml_compute_fp32_to_bf16
// (ggml-impl.h:590-624): round to nearest even, NaN kept and made quiet.
float tlq_bf16_to_fp32(uint16_t h);
uint16_t tlq_fp32_to_bf16(float f);

// Weight quantizers (offline, host only; ggml_quantize_chunk with imatrix NULL):
// quantize_row_q4_0_ref ggml-quants.c:113-147, quantize_row_q8_0_ref :276-297,
// quantize_row_q4_K_ref :1457-1527 (make_qkx2_quants :799-878).
void tlq_quantize_row_q4_0(const float *x, void *y, int64_t k);
void tlq_quantize_row_q4_K(const float *x, void *y, int64_t k);
// Activation quantizers the CPU mul_mat applies to src1
// (ggml-cpu.c:1318-1359 with from_float of type_traits_cpu):
// quantize_row_q8_0 -> _ref on x86 without AVX (arch/x86/quants.c:395-398,
// ggml-quants.c:276-297); quantize_row_q8_K -> _ref (arch/x86/quants.c:505-507,
// ggml-quants.c:2768-2804).
void tlq_quantize_row_q8_0(const float *x, void *y, int64_t k);
void tlq_quantize_row_q8_K(const float *x, void *y, int64_t k);
// quantize_row_q8_1 -> _ref on x86 without AVX (arch/x86/quants.c:400-501,
// ggml-quants.c:302-335): q8_0's d and codes plus s = f16(code sum * d).
void tlq_quantize_row_q8_1(const float *x, void *y, int64_t k);
// Quantize one activation row into the weight type's vec_dot type (for F32 /
// F16 / BF16 weights: from_float = copy / ggml_cpu_fp32_to_fp16 /
// ggml_cpu_fp32_to_bf16, ggml-cpu.c:3531-3536).
int tlq_quantize_act(int wtype, const float *x, void *y, int64_t k);

// Dequantizers: dequantize_row_q4_0 ggml-quants.c:459-476, _q8_0 :553-565,
// _q4_K :1529-1550, _q5_K :1731-1756, _q6_K :1939-1968; q8_K has no dequantizer on the path (d * q per element).
void tlq_dequantize_row_q4_0(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q8_0(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q4_K(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q5_K(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q6_K(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q8_K(const void *x, float *y, int64_t k);
// dequantize_row_q4_1 ggml-quants.c:479-498, _q5_0 :500-524, _q5_1 :526-551.
void tlq_dequantize_row_q4_1(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q5_0(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q5_1(const void *x, float *y, int64_t k);
// dequantize_row_q2_K ggml-quants.c:961-989, _q3_K :1305-1351.
void tlq_dequantize_row_q2_K(const void *x, float *y, int64_t k);
void tlq_dequantize_row_q3_K(const void *x, float *y, int64_t k);
int tlq_dequantize_row(int type, const void *x, float *y, int64_t k);

// Dot products of one weight row with one quantized activation row:
// ggml_vec_dot_q4_0_q8_0_generic ggml-cpu/quants.c:225-258,
// _q8_0_q8_0_generic :451-476, _q4_K_q8_K_generic :696-773,
// _q5_K_q8_K_generic :771-850, _q6_K_q8_K_generic :851-904.
float tlq_vec_dot_q4_0_q8_0(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q8_0_q8_0(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q4_K_q8_K(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q5_K_q8_K(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q6_K_q8_K(int64_t k, const void *x, const void *y);
// ggml_vec_dot_q4_1_q8_1_generic ggml-cpu/quants.c:262-296, _q5_0_q8_0_generic
// :365-406, _q5_1_q8_1_generic :408-449 (the x86 entries without AVX call them).
float tlq_vec_dot_q4_1_q8_1(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q5_0_q8_0(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q5_1_q8_1(int64_t k, const void *x, const void *y);
// ggml_vec_dot_q2_K_q8_K_generic ggml-cpu/quants.c:565-615, _q3_K_q8_K_generic
// :617-694 (the x86 entries without AVX call them, arch/x86/quants.c:1762, :2034).
float tlq_vec_dot_q2_K_q8_K(int64_t k, const void *x, const void *y);
float tlq_vec_dot_q3_K_q8_K(int64_t k, const void *x, const void *y);

// Exact integer parts of one block product (for pinning GPU partial sums):
// q4_K: *sum_q = sum_s sc_s * sum_{e in s} q4_e*q8_e, *sum_m = sum_s m_s * sum_{e in s} q8_e.
void tlq_block_ints_q4_K(const void *x_block, const void *y_block, int32_t *sum_q, int32_t *sum_m);

// Dot products of float rows as an x86-64 build without -march compiles them
// (no GGML_SIMD): each product in f32, the sum in double, rounded to f32 once
// (ggml_vec_dot_f32 vec.cpp:11-143 scalar branch, ggml_vec_dot_bf16
// :139-262 tail loop, ggml_vec_dot_f16 :264-352 scalar branch).
float tlq_vec_dot_f32(int64_t k, const void *x, const void *y);
float tlq_vec_dot_f16(int64_t k, const void *x, const void *y);
float tlq_vec_dot_bf16(int64_t k, const void *x, const void *y);

// GGML_OP_MUL_MAT on the CPU backend's algorithm (ggml-cpu.c:1254-1457 with
// the one-chunk loop :1164-1252): quantize every activation column to the
// vec_dot type, then y[n*M + m] = vec_dot(W row m, column n). `nthreads`
// splits rows; the result does not depend on it. Weights of F32 / F16 / BF16
// take the float dot products above on src1 converted to the weight type.
int tlq_mul_mat(int wtype, const void *w, int64_t M, int64_t K, const float *x, int64_t N, float *y,
                int nthreads);

// Paged-attention decode following the vLLM v1 kernel
// (crates/kernels/src/cuda/shaders/pagedattention.cuh:113-486, launched by
// crates/kernels/src/cuda/paged_attn.rs:326-417): f16 q [seqs][heads][hs],
// key cache [blocks][kvh][hs/8][bs][8] f16, value cache [blocks][kvh][hs][bs]
// f16, block tables i32 [seqs][max_blocks], context lens i32 [seqs]; out f16
// [seqs][heads][hs]. Logits scale*q.k in f32, softmax with 1/(sum + 1e-6),
// probabilities rounded to f16 before the f32 P.V accumulation, as the kernel
// does.
int tlq_paged_attention(uint16_t *out, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                        int num_kv_heads, float scale, const int32_t *block_tables, const int32_t *context_lens,
                        int max_blocks, int num_seqs, int num_heads, int head_size, int block_size);

// GGML_OP_FLASH_ATTN_EXT on the CPU backend's vec path
// (vendor/ggml/src/ggml-cpu/ops.cpp:8468-8700, ggml_compute_forward_flash_attn_ext_f16_one_chunk)
// for f32 q and f16 K/V, with the scalar helpers an x86-64 build without
// -march compiles (vec.h:570-580 ggml_vec_mad_f16, :845-850 ggml_vec_scale_f16,
// vec.cpp:264-352 ggml_vec_dot_f16): q rounded to f16, q.k summed in double,
// the P.V accumulator kept in f16 and rounded after every key. Shapes and
// byte strides are ggml's: q [D, nq, nh, nb], k [D, L, nhkv, nbk],
// v [DV, L, nhkv, nbk], mask [>= L, >= nq, mne2, mne3] (NULL = none),
// dst [DV, nh, nq, nb]. m0, m1 and n_head_log2 are derived from max_bias as
// ops.cpp:8527-8533 does. One query per batch with L >= 512 keys takes the
// backend's split-KV decode path instead (ops.cpp:9115-9145, reduce
// :8996-9063): `nthreads` key chunks with their own f16 accumulators, merged
// in f32 in chunk order, so the result depends on nthreads there as it does
// in the backend. (The backend's tiled path for >= 64 queries,
// ops.cpp:8706, accumulates in f32 and is not restated: its results are
// compared within f16 tolerance.)
int tlq_flash_attn_ext(const void *q, const int64_t q_ne[4], const int64_t q_nb[4], const void *k,
                       const int64_t k_ne[4], const int64_t k_nb[4], const void *v, const int64_t v_ne[4],
                       const int64_t v_nb[4], const void *mask, const int64_t m_ne[4], const int64_t m_nb[4],
                       void *dst, const int64_t d_nb[4], float scale, float max_bias, float softcap, int nthreads);

// Core ops of a decoder step, as the ggml CPU backend computes them
// (vendor/ggml/src/ggml-cpu/binary-ops.cpp, unary-ops.cpp, ops.cpp; each
// function in tlq_oracle.c cites its lines). Tensors as ggml describes them:
// data, ne[4], byte strides nb[4], type (f32, f16; i32 = 26 / i64 = 27 indices;
// GET_ROWS / CPY sources also q4_0, q8_0, q4_K, q5_K, q6_K).
typedef struct tlq_t {
    void *data;
    int64_t ne[4], nb[4];
    int ty;
} tlq_t;
void tlq_core_bin(int code, const tlq_t *a, const tlq_t *b, const tlq_t *d);
void tlq_core_unary(int code, float p1, float p2, const tlq_t *a, const tlq_t *d);
void tlq_core_norm(int rms, float eps, const tlq_t *a, const tlq_t *d);
void tlq_core_get_rows(const tlq_t *a, const tlq_t *idx, const tlq_t *d);
void tlq_core_set_rows(const tlq_t *a, const tlq_t *idx, const tlq_t *d);
void tlq_core_cpy(const tlq_t *a, const tlq_t *d);
void tlq_core_rope(int mode, int n_dims, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                   float attn_factor, float beta_fast, float beta_slow, const tlq_t *a, const int32_t *pos,
                   const float *ff, const tlq_t *d);
void tlq_core_soft_max(float scale, float max_bias, const tlq_t *a, const tlq_t *mask, const tlq_t *d);
void tlq_core_argmax(const tlq_t *a, int32_t *out);
void tlq_core_glu(int code, int swapped, const tlq_t *a, const tlq_t *b, const tlq_t *d);

// reshape_and_cache (crates/kernels/src/cuda/shaders/reshape_and_cache_kernel.cu:31-84):
// key/value f16 [tokens][kvh*hs] scattered to slot = block*bs + offset;
// negative slots are skipped.
void tlq_reshape_and_cache(const uint16_t *key, const uint16_t *value, uint16_t *k_cache, uint16_t *v_cache,
                           const int64_t *slots, int num_tokens, int num_kv_heads, int head_size, int block_size);
// The inverse read (gather_kv_cache_kernel.cu:40): dense f16 [kvh][L][hs] K and
// V of one sequence from its block table.
void tlq_gather_kv(const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *block_table, int context_len,
                   int num_kv_heads, int head_size, int block_size, uint16_t *k_out, uint16_t *v_out);

#ifdef __cplusplus
}
#endif
#endif

// Internal interface between the C ABI (tlhip.cpp) and the kernel files.
#pragma once

#include <atomic>
#include <string>

#include "common.hpp"

namespace tlh {

// Thread-local error text + status (defined in tlhip.cpp).
tlh_status set_error(tlh_status s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// hipGetLastError after a launch, mapped to TLH_EXECUTION with `what` in the text.
// While a trace is on (launch_trace with a sink), `what` is also appended to
// the sink, comma-separated: the launch labels of this thread.
tlh_status check_launch(const char *what);
void launch_trace(std::string *sink);
// Compute units of the current device (looked up once per device, thread-safe).
int device_cus();
// Workgroups of `kern` (block threads, dynamic LDS bytes) one CU holds at
// once, looked up once into `cache` (0: not yet; thread-safe).
template <typename Kern>
int blocks_per_cu(Kern kern, int threads, size_t lds, std::atomic<int> &cache) {
    int nb = cache.load(std::memory_order_relaxed);
    if (nb == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, threads, lds) != hipSuccess || nb < 1) {
            (void)hipGetLastError();
            nb = 1;
        }
        cache.store(nb, std::memory_order_relaxed);
    }
    return nb;
}

// rows of x (stride x_row_bytes) -> activation rows row_off.. of an output of
// total_rows rows, in ggml's block layout or the split scratch layout.
// f16: also write the codes as f16 (the scratch of a GEMM launch).
tlh_status launch_quantize_act(int wtype, const float *x, int64_t K, int64_t rows, int64_t x_row_bytes, void *out,
                               bool ggml_layout, int64_t row_off, int64_t total_rows, bool f16, hipStream_t stream);
tlh_status launch_dequantize(int type, const void *w, int64_t K, int64_t rows, int64_t w_row_bytes, float *y,
                             hipStream_t stream);

// One batch slice of MUL_MAT with pre-quantized activations:
//   dst[n*d_nb1 + m*4] = sum_k W[m][k] * act[n][k],  m < M, n < N
// over `batches` = ne12*ne13 slices (grid z), weights broadcast by r2/r3.
struct MatmulArgs {
    int wtype;
    const uint8_t *w;
    int64_t w_nb1, w_nb2, w_nb3;  // weight row / matrix strides (bytes)
    int64_t M, K, N;              // N: columns handled by this launch
    int64_t n0, N_total;          // first column; columns per batch slice in act/dst
    int64_t ne12, ne13, r2, r3;
    const void *act;              // split-layout scratch, N_total*ne12*ne13 rows:
                                  // column n of slice b is row n + N_total*b
    float *dst;
    int64_t d_nb1, d_nb2, d_nb3;  // dst strides (bytes), nb0 = 4
    float *part;                  // few-column kernel with K split in chunks: partial
                                  // sums [chunk][batch][N][M] (scratch), else null
    // Register GEMV at N = 1 and one batch slice only: with nseg > 0 the
    // launch's M rows are the rows of up to three weight matrices read with
    // the same activation -- rows seg_m0[s] .. seg_m0[s+1] come from seg_w[s]
    // (row stride seg_w_nb1[s]) and go to seg_dst[s]; w / dst above are unused.
    int nseg;
    const uint8_t *seg_w[3];
    int64_t seg_w_nb1[3];
    float *seg_dst[3];
    int64_t seg_m0[4];
    // the few-column MFMA kernel also takes segments (N <= 16, one K chunk,
    // segment row counts multiples of 16, one weight row stride): segment s's
    // outputs go to seg_dst[s] + column * seg_d_nb1[s] bytes
    int64_t seg_d_nb1[3];
    // MUL_MAT_ID (int8-MFMA few-column kernel only): with ids != null, batch
    // slice z = (e, t) = (z % ne12, z / ne12) multiplies weight matrix
    // ids[e * ids_nb0 + t * ids_nb1] (i32, w_nb2 apart; id_nas matrices) by
    // activation row (e % id_b1) + id_b1 * t of the id_b1 * ne13 quantized rows,
    // into dst + e * d_nb2 + t * d_nb3. An id outside [0, id_nas) gives NaN.
    const char *ids;
    int64_t ids_nb0, ids_nb1, id_b1, id_nas;
    // K-split launches leave their partials in `part` without the chunk-sum
    // launch (a consumer adds them: mul_mat_compute_keep)
    int keep_part;
};

// Batch slice z of a MUL_MAT launch: i12 = z % ne12, i13 = z / ne12 and the
// weight matrix it reads (broadcast by r2 / r3). Slice 0 -- the only one of a
// single-matrix MUL_MAT -- skips the integer divisions: they are a few hundred
// scalar instructions that every wave of the launch would otherwise issue
// before its first weight load. The counts fit 32 bits (grid z is below 2^16).
struct MmSlice {
    int64_t i12, i13;
    const uint8_t *w;
};
__device__ __forceinline__ MmSlice mm_slice(const MatmulArgs &a, uint32_t z) {
    MmSlice s{0, 0, a.w};
    if (z != 0) {
        const uint32_t ne12 = (uint32_t)a.ne12, i13 = z / ne12, i12 = z - i13 * ne12;
        s.i12 = i12;
        s.i13 = i13;
        s.w = a.w + (int64_t)(i12 / (uint32_t)a.r2) * a.w_nb2 + (int64_t)(i13 / (uint32_t)a.r3) * a.w_nb3;
    }
    return s;
}

// Rows of quantized activations a launch's scratch holds.
__host__ __device__ inline int64_t mm_act_rows(const MatmulArgs &a) {
    return a.ids ? a.id_b1 * a.ne13 : a.N_total * a.ne12 * a.ne13;
}

// Optional prologue and epilogue of the register GEMV (N <= 2, one batch
// slice), for the executor's fusions.
//  * Prologue (p != nullptr): activation column n is not read from src1 but
//    formed in the kernel as ggml's [ADD ->] RMS_NORM -> MUL chain does it:
//    x = p + q (q may be null), scale = 1/sqrtf((float)(sum x*x in double / K)
//    + eps), y = (x * scale) * w, then quantized like src1; the sum x goes to
//    s (written by one workgroup) when s is not null. Rows of p, q, s are
//    p_nb1, q_nb1, s_nb1 bytes apart.
//  * Epilogue (glu != nullptr): the launch's two segments are a gate and an
//    up matrix of equal rows; instead of their outputs the kernel stores
//    h = silu(gate) * up (ggml_vec_swiglu_f32) at glu + n * glu_nb1 bytes.
//  * Store epilogue (epi.on, N = 1, segments): segment s's row j goes out
//    through epi.layout[s] instead of seg_dst[s][j], rotated first when
//    epi.rope[s] (ROPE mode 0: rows 2p and 2p + 1 of a head of epi.ne0 rows
//    are a pair; a wave holds both) -- the ROPE, type cast, SET_ROWS and
//    one-token paged cache write that follow a Q / K / V projection.
enum { EPI_F32 = 0, EPI_CONTIG = 1, EPI_CACHE_ROW = 2, EPI_PAGED_KEY = 3, EPI_PAGED_VALUE = 4 };
struct GemvEpi {
    int on = 0;
    int layout[3] = {EPI_F32, EPI_F32, EPI_F32};
    int f16[3] = {0, 0, 0};   // destination element type f16 (else f32); the paged pools are f16
    int rope[3] = {0, 0, 0};
    char *dst[3] = {nullptr, nullptr, nullptr};  // contiguous rows, the cache, or the paged pool
    // EPI_CACHE_ROW: the row index (i32 or i64) and the cache's row stride and
    // rows (an index outside them writes nothing); paged: the token's i64 slot
    // and the pool's slots (a slot outside [0, slots) writes nothing)
    const char *idx[3] = {nullptr, nullptr, nullptr};
    int idx_i64[3] = {0, 0, 0};
    int64_t row_nb[3] = {0, 0, 0};
    int64_t rows[3] = {0, 0, 0};
    int kvh = 0, hs = 0, bs = 0;  // paged pools: kv heads, head size, block size
    // the rotation (one parameter set for every rotated segment): the token's
    // position, the per-pair frequency factors (or null) and the head size
    const int32_t *pos = nullptr;
    const float *ff = nullptr;
    int64_t ne0 = 0;
    RopeParams rp;
    // the few-column kernel (several tokens): the rotation's (cos, sin) per
    // (token, pair), [tokens][pairs][2], are the same for every layer of a
    // step. rt_mode 1: computed here and also written to rt; 2: read from rt
    // (a launch with mode 1 of the same positions and parameters ran before);
    // 0: computed here only
    float *rt = nullptr;
    int rt_mode = 0;
    // the K-split GEMM's reduce only: an EPI_CONTIG f16 segment also stored
    // into a paged pool (dual[s] = EPI_PAGED_KEY / EPI_PAGED_VALUE, dst2[s]
    // the pool, idx / rows / kvh / hs / bs as for a paged layout): a prefill's
    // keys and values, read as rows by its attention and kept in the pools
    int dual[3] = {0, 0, 0};
    char *dst2[3] = {nullptr, nullptr, nullptr};
};
struct GemvPro {
    const float *p = nullptr, *q = nullptr, *w = nullptr;
    float *s = nullptr;
    int64_t p_nb1 = 0, q_nb1 = 0, s_nb1 = 0;
    float eps = 0.0f;
    float *glu = nullptr;
    int64_t glu_nb1 = 0;
    GemvEpi epi;
};

// N <= 16. With x != nullptr (src1 rows in activation-row order, stride
// x_row_bytes) and a small N*K the GEMV quantizes x itself and the scratch is
// not read; otherwise it reads the scratch a quantize launch filled.
tlh_status launch_gemv(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream);
bool gemv_fuses_quantize(const MatmulArgs &a, const float *x, int64_t x_row_bytes);
bool gemv_reg_weights_ok(const MatmulArgs &a);
// register-resident GEMV (gemv_reg.hip): K <= 16384, K % 64 == 0
bool gemv_reg_geometry(int64_t K, int &ksplit, int &upw);
tlh_status launch_gemv_reg(const MatmulArgs &a, const float *x, int64_t x_row_bytes, hipStream_t stream);
// the register GEMV with a prologue and / or epilogue (GemvPro); quantizes in-kernel
// q4_1 / q5_0 / q5_1 / q2_K / q3_K register GEMV (gemv_reg_q.hip): plain stores only
tlh_status launch_gemv_reg_legacy(const MatmulArgs &a, const float *x, int64_t x_row_bytes, int ksplit, int upw,
                                  hipStream_t stream);
__host__ __device__ constexpr bool legacy_type(int t) {
    return t == TLH_TYPE_Q4_1 || t == TLH_TYPE_Q5_0 || t == TLH_TYPE_Q5_1;
}
// weight types whose register GEMV lives in gemv_reg_q.hip (plain stores, no
// prologue / epilogue forms): q4_1 / q5_0 / q5_1, q2_K / q3_K
__host__ __device__ constexpr bool reg_plain_type(int t) {
    return legacy_type(t) || t == TLH_TYPE_Q2_K || t == TLH_TYPE_Q3_K;
}
tlh_status launch_gemv_reg_pro(const MatmulArgs &a, const GemvPro &pro, const float *x, int64_t x_row_bytes,
                               hipStream_t stream);
// few-column GEMM on int8 MFMA (gemv_mfma.hip): 1 <= N <= 16, any K, from
// the scratch. K > 4096 needs a.part: gemv_mfma_partial_bytes of scratch.
bool gemv_mfma_supported(int64_t N);
int64_t gemv_mfma_partial_bytes(int64_t K, int64_t M, int64_t N, int64_t batches);
int64_t gemv_mfma_chunks(int64_t K);  // the few-column kernel's K chunks
tlh_status launch_gemv_mfma(const MatmulArgs &a, hipStream_t stream);
// launch_gemv_mfma with GemvEpi's store epilogue over the columns (token n =
// column n): segments, q4_K / q5_K / q6_K, one K chunk; TLH_UNSUPPORTED otherwise.
struct GemvEpi;
tlh_status launch_gemv_mfma_epi(const MatmulArgs &a, const GemvEpi &ep, hipStream_t stream);
// Tiled prefill GEMM for q8_0 / q4_0 weights (gemm_q8.hip), any N; with
// ksplit > 1 each K chunk writes a.part and a reduce launch sums them.
tlh_status launch_gemm_q8(const MatmulArgs &a, int ksplit, hipStream_t stream);
// dst (strided, columns n0..) = sum over `chunks` partials [chunk][batch][N][M] of a.part, in chunk order
tlh_status launch_partial_reduce(const MatmulArgs &a, int chunks, hipStream_t stream);
// the same through GemvEpi's store epilogue (segments, one batch slice);
// reduce_epi_check: TLH_OK when it takes a and ep
tlh_status launch_partial_reduce_epi(const MatmulArgs &a, int chunks, const GemvEpi &ep, hipStream_t stream);
tlh_status reduce_epi_check(const MatmulArgs &a, const GemvEpi &ep);
// K chunks of the tiled prefill GEMMs: a launch of fewer 128 x 128 tiles than
// CUs splits K into up to 512 / tiles chunks (whole stages per chunk, at least four super-blocks /
// sixteen q8_0 blocks each), and the bytes of its partial sums.
int gemm_ksplit(int wtype, int64_t M, int64_t N, int64_t K, int64_t batches);
int64_t gemm_partial_bytes(int wtype, int64_t M, int64_t N, int64_t K, int64_t batches);
tlh_status launch_gemm(const MatmulArgs &a, hipStream_t stream);  // any N, from the scratch
// q4_K / q5_K GEMM whose K chunks' reduce stores through ep (the launch must
// split K); TLH_UNSUPPORTED otherwise, before anything is launched
tlh_status launch_gemm_epi(const MatmulArgs &a, const GemvEpi &ep, hipStream_t stream);

// Dense FLASH_ATTN_EXT over f16 K/V (flash_attn.hip). Strides in bytes;
// scale already divided by softcap when softcap != 0; mask may be null.
struct FlashAttnDesc {
    const void *q, *k, *v, *mask;
    void *dst;
    void *scratch;  // flash_attn_scratch_bytes of partials (may be null when 0)
    int64_t D, DV, nq, nh, nb, L, nhkv, nbk;
    int64_t q_nb[4], k_nb[4], v_nb[4], m_nb[4], d_nb[4];
    int64_t m_ne2, m_ne3;
    float scale, max_bias, m0, m1, softcap;
    int n_head_log2;
};
bool flash_attn_head_sizes_ok(int64_t D, int64_t DV);
// split-key partials (mask_rows is not used: the kernels scan the mask)
int64_t flash_attn_scratch_bytes(int64_t DV, int64_t nq, int64_t nh, int64_t nhkv, int64_t nb, int64_t L,
                                 int64_t mask_rows);
tlh_status launch_flash_attn(const FlashAttnDesc &d, hipStream_t stream);

// core ops (core.hip): kind is a tlh_core_kind; op validated by the caller
// Up to three MUL_MAT nodes at N = 1 reading one activation with weights of one
// type and K as one register-GEMV launch (tlhip.cpp); TLH_UNSUPPORTED when the
// pointers do not allow it.
bool mul_mat_compute_multi_ok(const tlh_op *const *ops, int n);
size_t mul_mat_compute_multi_scratch_bytes(const tlh_op *const *ops, int n);
tlh_status mul_mat_compute_multi(const tlh_op *const *ops, const void *const *w, void *const *dst, int n,
                                 const void *scratch, size_t scratch_bytes, hipStream_t stream,
                                 const GemvEpi *epi = nullptr);
bool mul_mat_multi_ok(const tlh_op *const *ops, int n);
// Where a MUL_MAT's K-split product leaves its partial sums [chunk][N][M] in
// the node's scratch (byte offset, chunks > 1, chunk stride in floats), for a
// consumer that adds them itself; false when the node's product does not split
// K in a form this covers (N 3..16 few-column, or the q8_0 / q4_0 / q4_K /
// q5_K GEMM; one batch slice). mul_mat_compute_keep runs the node's product
// (after quantizing src1 into the scratch when src1 is given) without the
// chunk sum.
struct MmPartials {
    int64_t off = 0;
    int chunks = 1;
    int64_t cstride = 0;
};
bool mul_mat_partials(const tlh_op *op, MmPartials &pp);
tlh_status mul_mat_compute_keep(const tlh_op *op, const void *src0, const void *src1, void *scratch,
                                size_t scratch_bytes, void *dst, hipStream_t stream);
tlh_status mul_mat_multi(const tlh_op *const *ops, const void *const *w, void *const *dst, int n, const void *x,
                         hipStream_t stream);
// mul_mat_multi with a GemvPro prologue and / or SwiGLU epilogue (executor
// fusions; x is null with the prologue). TLH_UNSUPPORTED when the pointers do
// not allow it.
tlh_status mul_mat_multi_pro(const tlh_op *const *ops, const void *const *w, void *const *dst, int n,
                             const GemvPro &pro, const void *x, hipStream_t stream);
// A kernel's rows quantized as it writes them: the activation scratch of a
// MUL_MAT (split layout of `type` = q8_0 / q8_1 / q8_K for `rows` activation
// rows, f16 codes too when `f16`), row r of the kernel's output being
// activation row r.
struct ActQuantOut {
    void *out = nullptr;
    int type = 0;
    int64_t rows = 0;
    bool f16 = false;
};
// Longest row the norm chain quantizes (the row is held in registers).
constexpr int64_t NORM_CHAIN_QUANT_MAX = 4096;
// [ADD ->] RMS_NORM / NORM -> MUL(weight) in one kernel (core.hip k_norm_chain);
// op: t0 p (or x), t1 q, t2 w, t3 s, t4 y; x0 rms, x1 eps bits, x2 with the ADD.
// With qo, y is also quantized into qo's scratch (norm_chain_quantize_ok).
bool norm_chain_quantize_ok(const tlh_op &op, int act_type);
// qp (chunks > 1): q is not read; its rows are the sums, in chunk order, of the
// K-split partials a MUL_MAT left (mul_mat_compute_keep): row r element i at
// part + c * cstride + r * ne0 + i.
struct NormPartials {
    const float *part = nullptr;
    int chunks = 0;
    int64_t cstride = 0;
};
tlh_status launch_norm_chain(const tlh_op &op, const void *p, const void *q, const void *w, void *s, void *y,
                             hipStream_t stream, const ActQuantOut *qo = nullptr, const NormPartials *qp = nullptr);
// GGML_OP_GLU (the core op's operands, f32 rows of unit element stride) that
// also quantizes its output rows into qo (row length a multiple of qo's block).
bool glu_quantize_ok(const tlh_op &op, int act_type);
tlh_status launch_glu_quantize(const tlh_op &op, const void *src0, const void *src1, void *dst, const ActQuantOut &qo,
                               hipStream_t stream);
// ARGMAX of long rows in chunks over many workgroups (executor): scratch of
// argmax_split_scratch_bytes; same result as the core ARGMAX.
size_t argmax_split_scratch_bytes(const tlh_op &op);
tlh_status launch_argmax_split(const tlh_op &op, const void *x, void *dst, void *scratch, hipStream_t stream);
// Up to four independent element-wise core ops (BIN, UNARY, SET_ROWS, GLU,
// ROPE) in one launch; srcs[k] = s0, s1, s2 and, for a ROPE whose op has x9 =
// 1, the row index of each token (the result goes to those rows of the dst).
bool core_multi_kind(int kind);
// MUL_MAT with f32 / f16 / bf16 weights (mm_float.hip): w rows of wtype
// (w_nb* byte strides), x rows of xtype (f32, or already the weight type),
// f32 outputs; batch slice (i12, i13) reads weight slice (i12 / r2, i13 / r3).
struct FloatMM {
    int wtype, xtype;
    const char *w;
    int64_t w_nb1, w_nb2, w_nb3;
    const char *x;
    int64_t x_nb1, x_nb2, x_nb3;
    float *d;
    int64_t d_nb1, d_nb2, d_nb3;
    int64_t M, K, N, ne12, ne13, r2, r3;
};
tlh_status launch_mm_float(const FloatMM &f, hipStream_t stream);
// x rows -> contiguous rows of the weight type at out (out_row bytes apart)
tlh_status launch_mm_float_convert(const FloatMM &f, void *out, int64_t out_row, hipStream_t stream);
tlh_status launch_fill(void *dst, int value, size_t bytes, hipStream_t stream);
tlh_status launch_read_floor(const void *src, size_t bytes, int grid, int loads, hipStream_t stream);
tlh_status launch_core_multi(int n, const int *kinds, const tlh_op *ops, const void *const (*srcs)[4],
                             void *const *dsts, hipStream_t stream);
tlh_status launch_core(int kind, const tlh_op &op, const void *s0, const void *s1, const void *s2, void *dst,
                       hipStream_t stream);

// out32 != null: the f16 results are written widened to f32 there instead of
// a.out. counters != null: one launch that merges the partitions itself, on
// paged_attention_counters(a) zeroed counters it leaves zeroed (launches that
// share them must be stream-ordered); else a second launch merges them.
// qo (one-launch form, paged_attention_quantize_ok): the merging workgroup
// also quantizes its heads' outputs (as f32, whole q8_K blocks) into qo's
// split-layout scratch, activation row = sequence, K = heads x head size --
// the bytes the next MUL_MAT's quantize launch would write.
struct ActQuantOut;
tlh_status launch_paged_attention(const tlh_paged_attention_args &a, void *scratch, size_t scratch_bytes,
                                  hipStream_t stream, float *out32 = nullptr, unsigned *counters = nullptr,
                                  const ActQuantOut *qo = nullptr);
bool paged_attention_quantize_ok(const tlh_paged_attention_args &a, int act_type);
size_t paged_attention_scratch_bytes(const tlh_paged_attention_args &a);
size_t paged_attention_counters(const tlh_paged_attention_args &a);
// key_f32 / value_f32: that source is f32 and is rounded to f16 on the way
tlh_status launch_reshape_and_cache(const void *key, const void *value, void *k_cache, void *v_cache,
                                    const int64_t *slots, int num_tokens, int num_kv_heads, int head_size,
                                    int block_size, int64_t num_blocks, hipStream_t stream, bool key_f32 = false,
                                    bool value_f32 = false);

}  // namespace tlh

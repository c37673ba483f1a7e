// Paged-attention decode over an f16 block-table KV cache, gfx950.
//
// Computes what vLLM's paged_attention_v1/v2 kernels compute for tensorlisp's
// `paged-attention` node (crates/kernels/src/cuda/shaders/pagedattention.cuh:113-486,
// launched by crates/kernels/src/cuda/paged_attn.rs:326-417): per (sequence,
// query head) softmax(scale * q.k) over the sequence's context, then P.V, with
// the caches in vLLM's layouts
//   key   [blocks][kv_heads][head_size/8][block_size][8]
//   value [blocks][kv_heads][head_size][block_size]
// and the same 1/(sum + 1e-6) normalisation.
//
// Design (MI355X-first, not the vLLM structure):
//  * one workgroup (4 waves) per (sequence, kv head, 512-token partition);
//    it serves every query head of the GQA group from one read of each KV
//    page (vLLM v1 re-reads a kv head once per query head);
//  * each wave streams 16-token tiles of its partition's pages (the key and
//    value operands are 8-byte loads from the cache layouts, see the MFMA
//    operand notes below);
//  * q.k and p.v run on v_mfma_f32_16x16x16_f16 over 16-token tiles (below),
//    the softmax is online (running max / sum per head, f32) so a page is
//    touched once;
//  * waves merge their (max, sum, acc) through LDS; partitions are merged by
//    a second kernel (flash-decoding) into the f16 output.
#include <algorithm>

#include "kernels.hpp"

namespace tlh {

// tokens per partition (a multiple of every block size): 512; 256 when
// sequences x kv heads x 512-token partitions make fewer than 512
// workgroups; 64 when even 128-token ones would leave most of the 256 CUs
// idle (a short batch-1 context: one 16-token tile per wave)
constexpr int PA_PART = 512, PA_PART_SMALL = 64;
constexpr int PA_WAVES = 4;

// Scratch per (seq, head, partition): max, sum, acc[HS] (f32).
template <int HS>
__device__ __forceinline__ float *part_slot(float *scratch, int seq, int head, int part, int num_heads, int P) {
    return scratch + ((int64_t)(seq * num_heads + head) * P + part) * (HS + 2);
}

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16(half4_t a, half4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// One wave works on 16-token tiles with v_mfma_f32_16x16x16_f16 (lane l,
// g = l / 16, c = l % 16; A lane holds A[c][4g..4g+3], B lane B[4g..4g+3][c],
// D lane D[4g + r][c]):
//   S = K_tile (16 tokens x HS) . Q^T (HS x 16 heads), HS / 16 steps: the key
//       cache layout [HS/8][BS][8] makes the A operand (token c, dims
//       16s + 4g..+3) 8 contiguous bytes, and a step's 64 lanes read 512
//       contiguous bytes of the page;
//   P = softmax numerators, f16: lane (token 4g + r, head c) of S is exactly
//       the A operand (head c, tokens 4g..4g+3) of
//   O += P (16 heads x 16 tokens) . V_tile (16 tokens x 16 dims), HS / 16
//       tiles: the value layout [HS][BS] makes the B operand (tokens 4g..+3,
//       dim c) 8 contiguous bytes.
// Heads past the group (c >= gc) have zero q and are dropped; one MFMA serves
// up to 16 query heads of a kv head, so a page is read once per group.
// Merge partitions 0 .. np-1 of (seq, head) for output dim d, f16-rounded
// (the reduce kernel's loop, and the last partition's in the one-launch form).
template <int HS, bool COHERENT = false>
__device__ __forceinline__ uint16_t merge_parts(const float *base, int np, int d) {
    constexpr int CHUNK = 16;
    auto get = [](const float *p) {
        if constexpr (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else return *p;
    };
    float M = -INFINITY, lsum = 0.0f, a = 0.0f;
    for (int p0 = 0; p0 < np; p0 += CHUNK) {
        float m[CHUNK], l[CHUNK], v[CHUNK];
#pragma unroll
        for (int i = 0; i < CHUNK; ++i) {
            const int64_t o = (int64_t)(p0 + i < np ? p0 + i : p0) * (HS + 2);
            m[i] = get(base + o);
            l[i] = get(base + o + 1);
            v[i] = get(base + o + 2 + d);
        }
        float cm = -INFINITY;
#pragma unroll
        for (int i = 0; i < CHUNK; ++i) cm = fmaxf(cm, m[i]);  // repeats of p0 change nothing
        const float Mn = fmaxf(M, cm);
        if (Mn == -INFINITY) continue;
        const float so = __expf(M - Mn);  // 0 while M is -inf (then lsum and a are 0)
        lsum *= so;
        a *= so;
#pragma unroll
        for (int i = 0; i < CHUNK; ++i) {
            const float w = p0 + i < np ? __expf(m[i] - Mn) : 0.0f;
            lsum += w * l[i];
            a += w * v[i];
        }
        M = Mn;
    }
    return f2h(a * (1.0f / (lsum + 1e-6f)));
}

// The merged outputs of a workgroup's gc heads (f32 values of the f16
// results, in LDS) quantized to q8_K for the output projection: the heads'
// outputs are whole q8_K blocks of the sequence's row (the launcher's check);
// one wave per block, four consecutive values a lane, as the quantize launch
// takes them.
template <int HS, int W>
__device__ __forceinline__ void quantize_heads(const float *sq, int gc, int num_heads, int head0, int seq, void *qout,
                                               int64_t qrows) {
    const int64_t K = (int64_t)num_heads * HS;
    const ActLayout QL = act_layout(TLH_TYPE_Q8_K, K, qrows, false);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int b = wave; b < gc * HS / QKK; b += W) {
        float v[1][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[0][i] = sq[QKK * b + 4 * lane + i];
        uint32_t packed[1];
        int psum[1];
        float dq[1];
        q8K_waves<1>(v, lane, packed, psum, dq);
        q8K_store_split((char *)qout, QL, K, seq, (int64_t)head0 * HS / QKK + b, lane, packed[0], psum[0], dq[0],
                        false);
    }
}

// MERGE (one launch): after writing its partial, a workgroup counts itself
// in on its (sequence, head group) counter; the last of the sequence's
// partitions to arrive merges them all into the output and sets the counter
// back to zero. The counters start at zero (the caller's zeroed buffer) and
// launches that share them must be stream-ordered.
//
// WHOLE (W waves, one partition covering the whole context, PART >= every
// length): the workgroup's wave merge is the final merge, so the output is
// written straight from it (merge_parts of one partition gives the same
// value), with no scratch, counter or read-back round trip: for short
// contexts over few workgroups, where those round trips are most of the time.
template <int HS, int BS, bool PIPE, int PART, bool MERGE, int W = PA_WAVES, bool WHOLE = false>
__global__ void __launch_bounds__(64 * W) k_paged_attn(const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc,
                                                    const uint16_t *__restrict__ vc,
                                                    const int32_t *__restrict__ tables,
                                                    const int32_t *__restrict__ lens, int num_heads, int num_kv_heads,
                                                    int gc, int max_blocks, float scale, int P,
                                                    float *__restrict__ scratch, unsigned *__restrict__ counters,
                                                    uint16_t *__restrict__ out, float *__restrict__ out32,
                                                    void *__restrict__ qout, int64_t qrows) {
    constexpr int KS = HS / 16;  // QK steps = PV output tiles
    __shared__ int s_bt[PART / 8];
    constexpr int HR = WHOLE ? 4 : 16;  // head rows kept (the one-partition form takes gc <= 4)
    __shared__ float s_m[W][16], s_l[W][16];
    __shared__ float s_acc[W][HR][HS];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int G = num_heads / num_kv_heads;
    const int kvh = blockIdx.x / (G / gc);
    const int head0 = kvh * G + (blockIdx.x % (G / gc)) * gc;
    const int seq = blockIdx.y;
    const int part = blockIdx.z;
    const int t0 = part * PART;
    const int page0 = t0 / BS;
    // the partition's block ids are read together with the context length
    // (entries past the table are clamped to its last one and never used)
    if (max_blocks > 0)
        for (int i = threadIdx.x; i < PART / BS; i += blockDim.x)
            s_bt[i] = tables[(int64_t)seq * max_blocks + min(page0 + i, max_blocks - 1)];
    const int L = lens[seq];
    if (t0 >= L && !(part == 0 && L == 0)) return;  // the reduce kernel ignores partitions past the context
    const int t1 = min(L, t0 + PART);
    const int npages = (t1 + BS - 1) / BS - page0;
    __syncthreads();

    // Q^T operand: head c, dims 16s + 4g..+3 (zero past the group)
    half4_t qb[KS];
    {
        const uint16_t *qh = q + ((int64_t)seq * num_heads + head0 + (c < gc ? c : 0)) * HS + 4 * g;
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const uint2 v = *(const uint2 *)(qh + 16 * st);
            qb[st] = c < gc ? __builtin_bit_cast(half4_t, v) : (half4_t){};
        }
    }
    float m_run = -INFINITY, l_run = 0.0f;  // head c: running max; this lane's partial sum
    f32x4_t o[KS];
#pragma unroll
    for (int n = 0; n < KS; ++n) o[n] = (f32x4_t){};

    const int64_t kv_stride_blk = (int64_t)num_kv_heads * HS * BS;  // elements per block
    const int64_t head_off = (int64_t)kvh * HS * BS;
    const int ntiles = (t1 - t0 + 15) / 16;
    const int my_tiles = ntiles > wave ? (ntiles - wave + W - 1) / W : 0;
    // tile k of this wave: tokens t0 + 16 * (wave + W * k) ...
    auto load_tile = [&](int k, half4_t (&ka)[KS], half4_t (&vb)[KS]) {
        const int tk = 16 * (wave + W * k);  // first token of the tile, relative to t0
        // keys: token tk + c at slot (t0 + tk + c) % BS of partition page
        // (t0 % BS + tk + c) / BS. A tile's tokens past the context can lie on
        // a page past the sequence's last (block size 8): those read the last
        // page instead (their logits are masked, their values zeroed).
        const int kt = (t0 % BS) + tk + c;
        const int kpg = kt / BS < npages ? kt / BS : npages - 1;
        const uint16_t *kp = kc + (int64_t)s_bt[kpg] * kv_stride_blk + head_off + (kt % BS) * 8 + 4 * (g & 1);
#pragma unroll
        for (int st = 0; st < KS; ++st)
            ka[st] = __builtin_bit_cast(half4_t, *(const uint2 *)(kp + (2 * st + (g >> 1)) * BS * 8));
        // values: tokens tk + 4g..+3 (one 4-aligned run of slots), dim 16n + c
        const int vt = (t0 % BS) + tk + 4 * g;
        const int vpg = vt / BS < npages ? vt / BS : npages - 1;
        const uint16_t *vp = vc + (int64_t)s_bt[vpg] * kv_stride_blk + head_off + c * BS + (vt % BS);
#pragma unroll
        for (int n = 0; n < KS; ++n) vb[n] = __builtin_bit_cast(half4_t, *(const uint2 *)(vp + 16 * n * BS));
    };
    auto compute_tile = [&](int k, const half4_t (&ka)[KS], const half4_t (&vin)[KS]) {
        const int tk = t0 + 16 * (wave + W * k);
        f32x4_t S = (f32x4_t){};
#pragma unroll
        for (int st = 0; st < KS; ++st) S = mfma16(ka[st], qb[st], S);
        float x[4], mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            x[r] = tk + 4 * g + r < t1 ? S[r] * scale : -INFINITY;
            mx = fmaxf(mx, x[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);  // finite: every tile holds >= 1 valid token
        const float alpha = __expf(m_run - m_new);
        m_run = m_new;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = tk + 4 * g + r < t1 ? __expf(x[r] - m_new) : 0.0f;
        l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        const half4_t pa = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
        // O rows are heads 4g + r: their alphas live in lanes c = 4g + r
        float ao[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ao[r] = __shfl(alpha, 4 * g + r, 64);
        const bool partial = tk + 16 > t1;  // zero values past the context (they may be NaN)
#pragma unroll
        for (int n = 0; n < KS; ++n) {
            half4_t v = vin[n];
            if (partial) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (tk + 4 * g + r >= t1) v[r] = (_Float16)0.0f;
            }
            f32x4_t on = o[n];
#pragma unroll
            for (int r = 0; r < 4; ++r) on[r] *= ao[r];
            o[n] = mfma16(pa, v, on);
        }
    };
    half4_t ka[KS], va[KS];
    if (my_tiles > 0) load_tile(0, ka, va);
    if constexpr (PIPE) {
        // two register sets in turn: the next tile's loads are in flight while
        // this one is multiplied (past the last tile it rereads its own, a
        // cache hit, so the compiler can count the loads)
        half4_t kb[KS], vb[KS];
        for (int k = 0; k < my_tiles; k += 2) {
            load_tile(k + 1 < my_tiles ? k + 1 : k, kb, vb);
            compute_tile(k, ka, va);
            if (k + 1 >= my_tiles) break;
            load_tile(k + 2 < my_tiles ? k + 2 : k + 1, ka, va);
            compute_tile(k + 1, kb, vb);
        }
    } else {
        for (int k = 0; k < my_tiles; ++k) {
            compute_tile(k, ka, va);
            if (k + 1 < my_tiles) load_tile(k + 1, ka, va);
        }
    }

    // this wave's sum per head (over the 4 token groups), then merge the
    // waves through LDS: max, sum, acc[HS] per head
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (g == 0) {
        s_m[wave][c] = m_run;
        s_l[wave][c] = l_run;
    }
#pragma unroll
    for (int n = 0; n < KS; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (HR == 16 || g == 0) s_acc[wave][4 * g + r][16 * n + c] = o[n][r];
    __syncthreads();
    for (int e = threadIdx.x; e < gc * HS; e += blockDim.x) {
        const int h = e / HS, d = e % HS;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, s_m[w][h]);
        float lsum = 0.0f, a = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float f = s_m[w][h] == -INFINITY ? 0.0f : __expf(s_m[w][h] - M);
            lsum += f * s_l[w][h];
            a += f * s_acc[w][h][d];
        }
        if constexpr (WHOLE) {
            // merge_parts over one partition: exp(0) = 1 weighs it, so its
            // value is a * (1 / (lsum + 1e-6)) rounded to f16
            const uint16_t r = f2h(a * (1.0f / (lsum + 1e-6f)));
            const int64_t o = ((int64_t)seq * num_heads + head0 + h) * HS + d;
            if (out32) out32[o] = h2f(r);
            else out[o] = r;
            // s_acc[0][h][d], read above by this thread alone
            if (qout) s_acc[0][0][e] = h2f(r);
            continue;
        }
        float *slotp = part_slot<HS>(scratch, seq, head0 + h, part, num_heads, P);
        // the one-launch form's partials are agent-scope stores: coherent
        // across the XCDs' L2s without a write-back of the whole L2
        auto put = [&](float *p, float v) {
            if constexpr (MERGE) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else *p = v;
        };
        put(slotp + 2 + d, a);
        if (d == 0) {
            put(slotp, M);
            put(slotp + 1, lsum);
        }
    }
    if constexpr (WHOLE) {
        if (qout) {
            __syncthreads();
            quantize_heads<HS, W>(&s_acc[0][0][0], gc, num_heads, head0, seq, qout, qrows);
        }
        return;
    }
    if constexpr (MERGE) {
        // Every wave's partial stores complete before the barrier (the
        // barrier's wait), so the counter moves only after they have reached
        // the coherent level; the last workgroup reads them back with
        // agent-scope loads. No fence: an L2 write-back per wave, or an
        // invalidate that drops the pages the other workgroups are reading,
        // costs more than the merge saves.
        //
        // What this ordering rests on is gfx950's code generation, not the
        // HIP memory model: the partials, the counter and the read-back are
        // all relaxed atomics, which the model leaves unordered. It holds
        // because (1) relaxed agent-scope stores compile to stores that write
        // through to the device-coherent level (MALL / HBM) rather than stay
        // in one XCD's L2, (2) s_waitcnt(0) before the barrier makes every
        // wave's stores complete (acknowledged at that level) before thread 0
        // increments the counter, and (3) relaxed agent-scope loads bypass
        // the reading XCD's L2, so the last workgroup sees the partials the
        // counter accounts for. A target or compiler that cached agent-scope
        // relaxed stores or loads in a non-coherent L2 would need a release
        // fence before the increment and an acquire fence after it.
        __shared__ int s_last;
        const int np = min(P, L > 0 ? (L + PART - 1) / PART : 1);  // the partitions that get here
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned *cnt = counters + (int64_t)seq * gridDim.x + blockIdx.x;
            const unsigned before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = before + 1 == (unsigned)np;
            if (s_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!s_last) return;
        // with qout, the merged values also go to LDS (the partial sums' buffer
        // is free by now) for the quantization below
        float *sq = &s_acc[0][0][0];
        for (int e = threadIdx.x; e < gc * HS; e += blockDim.x) {
            const int h = e / HS, d = e % HS;
            const uint16_t r = merge_parts<HS, true>(
                scratch + (int64_t)(seq * num_heads + head0 + h) * P * (HS + 2), np, d);
            const int64_t o = ((int64_t)seq * num_heads + head0 + h) * HS + d;
            if (out32) out32[o] = h2f(r);
            else out[o] = r;
            if (qout) sq[e] = h2f(r);
        }
        if (qout) {
            __syncthreads();
            quantize_heads<HS, W>(sq, gc, num_heads, head0, seq, qout, qrows);
        }
    }
}

// Merge the partitions of one (sequence, head) and write f16 output. Each
// thread reads the maxima, sums and its dims of up to 16 partitions in one
// round of independent loads and folds them into a running (max, sum, acc)
// rescaled online; longer contexts take further rounds.
template <int HS, int PART>
__global__ void __launch_bounds__(256) k_paged_attn_reduce(uint16_t *__restrict__ out, float *__restrict__ out32,
                                                           const float *__restrict__ scratch,
                                                           const int32_t *__restrict__ lens, int num_heads, int P) {
    const int head = blockIdx.x, seq = blockIdx.y;
    const int L = lens[seq];
    // partitions holding this sequence's context (never more than were written)
    const int np = min(P, L > 0 ? (L + PART - 1) / PART : 1);
    const float *base = scratch + (int64_t)(seq * num_heads + head) * P * (HS + 2);
    for (int d = threadIdx.x; d < HS; d += blockDim.x) {
        const uint16_t h = merge_parts<HS>(base, np, d);
        const int64_t o = ((int64_t)seq * num_heads + head) * HS + d;
        if (out32) out32[o] = h2f(h);  // the f16 result widened (a cast to f32 fused into this store)
        else out[o] = h;
    }
}

static int64_t pa_workgroups(const tlh_paged_attention_args &a, int part) {
    return (int64_t)a.num_seqs * a.num_kv_heads * (a.max_context_len > 0 ? (a.max_context_len + part - 1) / part : 1);
}
static int pa_part(const tlh_paged_attention_args &a) {
    if (pa_workgroups(a, PA_PART) >= 512) return PA_PART;
    return pa_workgroups(a, 128) >= 256 ? PA_PART / 2 : PA_PART_SMALL;
}

// query heads per workgroup: a divisor of the group size, at most 16
static int pa_gc(const tlh_paged_attention_args &a) {
    const int G = a.num_kv_heads > 0 ? a.num_heads / a.num_kv_heads : 1;
    int gc = G < 16 ? G : 16;
    while (gc > 1 && G % gc) --gc;
    return gc > 0 ? gc : 1;
}

// The one-partition form: contexts up to PA_WHOLE tokens, one workgroup of
// PA_WHOLE_WAVES waves per (sequence, kv head), while those workgroups
// number 64 to 256 (fewer leave too few CUs pulling each context) and the
// group has at most 4 query heads.
constexpr int PA_WHOLE = 1024, PA_WHOLE_WAVES = 8;
static bool pa_whole(const tlh_paged_attention_args &a) {
    const int G = a.num_kv_heads > 0 ? a.num_heads / a.num_kv_heads : 1;
    const int64_t wgs = (int64_t)a.num_seqs * a.num_kv_heads * (G / pa_gc(a));
    return a.head_size <= 128 && a.max_context_len <= PA_WHOLE && pa_gc(a) <= 4 && wgs >= 64 && wgs <= 256;
}

static int pa_partitions(const tlh_paged_attention_args &a) {
    const int part = pa_part(a);
    return a.max_context_len > 0 ? (a.max_context_len + part - 1) / part : 1;
}

// Sized for the shorter (256-token) partitions whichever the launch picks, so
// the size grows with num_seqs and max_context_len: a caller may size its
// scratch once for its largest batch and context.
size_t paged_attention_scratch_bytes(const tlh_paged_attention_args &a) {
    auto bytes = [&](int part) {
        const int64_t parts = a.max_context_len > 0 ? (a.max_context_len + part - 1) / part : 1;
        return (int64_t)a.num_seqs * a.num_heads * parts * (a.head_size + 2) * (int64_t)sizeof(float);
    };
    // 64-token partitions only while sequences x kv heads x ceil(context /
    // 128) < 256, where sequences x heads x ceil(context / 64) <= 510 x the
    // group size: a bounded extra term keeps the size growing with the batch
    // and the context
    const int64_t G = a.num_kv_heads > 0 ? a.num_heads / a.num_kv_heads : 1;
    const int64_t bound = 510 * G * (a.head_size + 2) * (int64_t)sizeof(float);
    return (size_t)(bytes(PA_PART / 2) + std::min(bytes(PA_PART_SMALL), bound));
}

bool paged_attention_quantize_ok(const tlh_paged_attention_args &a, int act_type) {
    return act_type == TLH_TYPE_Q8_K && ((int64_t)pa_gc(a) * a.head_size) % QKK == 0 &&
           ((int64_t)a.num_heads * a.head_size) % QKK == 0;
}

template <int HS, int BS, int PART>
static void launch_pa3(const tlh_paged_attention_args &a, float *scratch, hipStream_t stream, float *out32,
                       unsigned *counters, const ActQuantOut *qo) {
    const int P = pa_partitions(a);
    const int G = a.num_heads / a.num_kv_heads;
    int gc = G < 16 ? G : 16;  // query heads per workgroup: a divisor of G, at most 16
    while (G % gc) --gc;
    constexpr bool PIPE = HS <= 128;  // two register sets fit
    const dim3 grid(a.num_kv_heads * (G / gc), a.num_seqs, P), rgrid(a.num_heads, a.num_seqs);
    const dim3 rblock(HS < 256 ? HS : 256);
    if (counters) {
        hipLaunchKernelGGL((k_paged_attn<HS, BS, PIPE, PART, true>), grid, dim3(256), 0, stream, (const uint16_t *)a.q,
                           (const uint16_t *)a.k_cache, (const uint16_t *)a.v_cache, a.block_tables, a.context_lens,
                           a.num_heads, a.num_kv_heads, gc, a.max_blocks_per_seq, a.scale, P, scratch, counters,
                           (uint16_t *)a.out, out32, qo ? qo->out : nullptr, qo ? qo->rows : (int64_t)0);
        return;
    }
    hipLaunchKernelGGL((k_paged_attn<HS, BS, PIPE, PART, false>), grid, dim3(256), 0, stream, (const uint16_t *)a.q,
                       (const uint16_t *)a.k_cache, (const uint16_t *)a.v_cache, a.block_tables, a.context_lens,
                       a.num_heads, a.num_kv_heads, gc, a.max_blocks_per_seq, a.scale, P, scratch, nullptr, nullptr,
                       nullptr, nullptr, (int64_t)0);
    hipLaunchKernelGGL((k_paged_attn_reduce<HS, PART>), rgrid, rblock, 0, stream, (uint16_t *)a.out, out32,
                       (const float *)scratch, a.context_lens, a.num_heads, P);
}

template <int HS, int BS>
static void launch_pa2(const tlh_paged_attention_args &a, float *scratch, hipStream_t stream, float *out32,
                       unsigned *counters, const ActQuantOut *qo) {
    if constexpr (HS <= 128) {
        if (pa_whole(a)) {  // no scratch or counters; both forms take it
            const int gc = pa_gc(a), G = a.num_heads / a.num_kv_heads;
            const dim3 grid(a.num_kv_heads * (G / gc), a.num_seqs, 1);
            hipLaunchKernelGGL((k_paged_attn<HS, BS, true, PA_WHOLE, false, PA_WHOLE_WAVES, true>), grid,
                               dim3(64 * PA_WHOLE_WAVES), 0, stream, (const uint16_t *)a.q,
                               (const uint16_t *)a.k_cache, (const uint16_t *)a.v_cache, a.block_tables,
                               a.context_lens, a.num_heads, a.num_kv_heads, gc, a.max_blocks_per_seq, a.scale, 1,
                               nullptr, nullptr, (uint16_t *)a.out, out32, qo ? qo->out : nullptr,
                               qo ? qo->rows : (int64_t)0);
            return;
        }
    }
    switch (pa_part(a)) {
    case PA_PART: launch_pa3<HS, BS, PA_PART>(a, scratch, stream, out32, counters, qo); break;
    case PA_PART / 2: launch_pa3<HS, BS, PA_PART / 2>(a, scratch, stream, out32, counters, qo); break;
    default: launch_pa3<HS, BS, PA_PART_SMALL>(a, scratch, stream, out32, counters, qo); break;
    }
}

template <int HS>
static void launch_pa1(const tlh_paged_attention_args &a, float *scratch, hipStream_t stream, float *out32,
                       unsigned *counters, const ActQuantOut *qo) {
    switch (a.block_size) {
    case 8: launch_pa2<HS, 8>(a, scratch, stream, out32, counters, qo); break;
    case 16: launch_pa2<HS, 16>(a, scratch, stream, out32, counters, qo); break;
    default: launch_pa2<HS, 32>(a, scratch, stream, out32, counters, qo); break;
    }
}

// Counters the one-launch form takes: one per (sequence, workgroup of a kv
// head's query heads).
size_t paged_attention_counters(const tlh_paged_attention_args &a) {
    const int G = a.num_kv_heads > 0 ? a.num_heads / a.num_kv_heads : 1;
    int gc = G < 16 ? G : 16;
    while (gc > 1 && G % gc) --gc;
    return (size_t)a.num_seqs * a.num_kv_heads * (G / (gc > 0 ? gc : 1));
}

tlh_status launch_paged_attention(const tlh_paged_attention_args &a, void *scratch, size_t, hipStream_t stream,
                                  float *out32, unsigned *counters, const ActQuantOut *qo) {
    float *s = (float *)scratch;
    if (qo && (!counters || !qo->out || !paged_attention_quantize_ok(a, qo->type) || qo->f16 ||
               qo->rows < a.num_seqs))
        return set_error(TLH_UNSUPPORTED, "paged_attention: the merge quantizes whole q8_K blocks of heads, "
                                          "one launch, no f16 codes");
    switch (a.head_size) {
    case 64: launch_pa1<64>(a, s, stream, out32, counters, qo); break;
    case 80: launch_pa1<80>(a, s, stream, out32, counters, qo); break;
    case 96: launch_pa1<96>(a, s, stream, out32, counters, qo); break;
    case 112: launch_pa1<112>(a, s, stream, out32, counters, qo); break;
    case 128: launch_pa1<128>(a, s, stream, out32, counters, qo); break;
    case 192: launch_pa1<192>(a, s, stream, out32, counters, qo); break;
    case 256: launch_pa1<256>(a, s, stream, out32, counters, qo); break;
    default: return set_error(TLH_INVALID, "paged_attention: head_size %d", a.head_size);
    }
    return check_launch("paged_attention");
}

// ------------------------------------------------------- reshape_and_cache
// reshape_and_cache_kernel.cu:31-84: one workgroup per token, 16-byte pieces
// of 8 dims; keys land as one contiguous piece, values scatter along slots.
// 8 consecutive elements as f16 bits: an f16 source as is, an f32 source
// rounded (the executor folds a preceding f32 -> f16 cast into the write)
template <bool F32> __device__ __forceinline__ uint4 load8_h(const void *base, int64_t e) {
    if constexpr (!F32) {
        return *(const uint4 *)((const uint16_t *)base + e);
    } else {
        const float4 a = *(const float4 *)((const float *)base + e), b = *(const float4 *)((const float *)base + e + 4);
        return make_uint4((uint32_t)f2h(a.x) | ((uint32_t)f2h(a.y) << 16), (uint32_t)f2h(a.z) | ((uint32_t)f2h(a.w) << 16),
                          (uint32_t)f2h(b.x) | ((uint32_t)f2h(b.y) << 16), (uint32_t)f2h(b.z) | ((uint32_t)f2h(b.w) << 16));
    }
}

template <bool K32, bool V32>
__global__ void __launch_bounds__(256) k_reshape_and_cache(const void *__restrict__ key, const void *__restrict__ value,
                                                           uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                           const int64_t *__restrict__ slots, int kvh, int hs,
                                                           int bs, int64_t pool_slots) {
    const int t = blockIdx.x;
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= pool_slots) return;  // negative: skip (the reference); past the pools: dropped
    const int64_t blk = slot / bs;
    const int off = (int)(slot % bs);
    const int chunks = kvh * hs / 8;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
        const int h = c / (hs / 8), ch = c % (hs / 8);
        const int64_t src = (int64_t)t * kvh * hs + 8 * (int64_t)c;
        const uint4 kk = load8_h<K32>(key, src);
        *(uint4 *)(kc + (((blk * kvh + h) * (hs / 8) + ch) * bs + off) * 8) = kk;
        const uint4 vv = load8_h<V32>(value, src);
        const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
        uint16_t *vdst = vc + ((blk * kvh + h) * (int64_t)hs + 8 * ch) * bs + off;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vdst[(2 * j) * bs] = (uint16_t)(w[j] & 0xffff);
            vdst[(2 * j + 1) * bs] = (uint16_t)(w[j] >> 16);
        }
    }
}

tlh_status launch_reshape_and_cache(const void *key, const void *value, void *k_cache, void *v_cache,
                                    const int64_t *slots, int num_tokens, int num_kv_heads, int head_size,
                                    int block_size, int64_t num_blocks, hipStream_t stream, bool key_f32,
                                    bool value_f32) {
    if (num_blocks < 0 || num_blocks > INT64_MAX / block_size)
        return set_error(TLH_INVALID, "reshape_and_cache: %lld blocks", (long long)num_blocks);
    if ((((uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache) & 15) != 0)
        return set_error(TLH_INVALID, "reshape_and_cache: key, value and key cache must be 16-byte aligned");
    auto k = key_f32 ? (value_f32 ? k_reshape_and_cache<true, true> : k_reshape_and_cache<true, false>)
                     : (value_f32 ? k_reshape_and_cache<false, true> : k_reshape_and_cache<false, false>);
    hipLaunchKernelGGL(k, dim3(num_tokens), dim3(128), 0, stream, key, value, (uint16_t *)k_cache,
                       (uint16_t *)v_cache, slots, num_kv_heads, head_size, block_size, num_blocks * block_size);
    return check_launch("reshape_and_cache");
}

}  // namespace tlh

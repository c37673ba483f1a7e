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
//  * each wave streams whole pages with 16-byte loads: a page of keys for one
//    kv head is head_size*block_size*2 contiguous bytes, lane l owns slot
//    l % block_size and 8-dim chunks l/block_size + (64/block_size)*i;
//    values are read the same way along [dim][slot];
//  * q.k and p.v run on v_dot2_f32_f16 (f16 pairs into f32), the softmax is
//    online (running max / sum per head, f32) so a page is touched once;
//  * waves merge their (max, sum, acc) through LDS; partitions are merged by
//    a second kernel (flash-decoding) into the f16 output.
#include "kernels.hpp"

namespace tlh {

constexpr int PA_PART = 512;  // tokens per partition (a multiple of every block size)
constexpr int PA_WAVES = 4;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
    return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
}

// Scratch per (seq, head, partition): max, sum, acc[HS] (f32).
template <int HS>
__device__ __forceinline__ float *part_slot(float *scratch, int seq, int head, int part, int num_heads, int P) {
    return scratch + ((int64_t)(seq * num_heads + head) * P + part) * (HS + 2);
}

template <int HS, int BS, int GC>
__global__ void __launch_bounds__(256) k_paged_attn(const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc,
                                                    const uint16_t *__restrict__ vc,
                                                    const int32_t *__restrict__ tables,
                                                    const int32_t *__restrict__ lens, int num_heads, int num_kv_heads,
                                                    int max_blocks, float scale, int P, float *__restrict__ scratch) {
    constexpr int CH = HS / 8;            // 8-dim chunks per key
    constexpr int PIECES = CH * BS;       // 16-byte pieces per page (keys or values)
    constexpr int NP = (PIECES + 63) / 64;  // pieces per lane
    constexpr int REP = 64 / BS;          // lanes sharing one slot (key layout)
    constexpr int SG = BS / 8;            // 8-slot groups per value row
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int seq = blockIdx.y;
    const int kvh = blockIdx.x / ((num_heads / num_kv_heads) / GC);
    const int hg = blockIdx.x % ((num_heads / num_kv_heads) / GC);
    const int head0 = kvh * (num_heads / num_kv_heads) + hg * GC;
    const int part = blockIdx.z;
    const int L = lens[seq];
    const int t0 = part * PA_PART;
    if (t0 >= L && !(part == 0 && L == 0)) return;  // the reduce kernel ignores partitions past the context
    const int t1 = min(L, t0 + PA_PART);
    const int pages0 = t0 / BS, pages1 = (t1 + BS - 1) / BS;

    // q chunks this lane multiplies: chunk c_i = lane / BS + REP * i (key layout).
    uint32_t qv[NP][GC][4];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int c = lane / BS + REP * i;
#pragma unroll
        for (int g = 0; g < GC; ++g) {
            const uint16_t *qh = q + ((int64_t)seq * num_heads + head0 + g) * HS;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (c < CH) v = *(const uint4 *)(qh + 8 * c);
            qv[i][g][0] = v.x;
            qv[i][g][1] = v.y;
            qv[i][g][2] = v.z;
            qv[i][g][3] = v.w;
        }
    }

    const int slot = lane % BS;     // key layout: this lane's slot
    const int vsg = lane % SG;      // value layout: this lane's 8-slot group
    float m_run[GC], l_run[GC], acc[NP][GC];
#pragma unroll
    for (int g = 0; g < GC; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < NP; ++i) acc[i][g] = 0.0f;
    }

    const int32_t *bt = tables + (int64_t)seq * max_blocks;
    const int64_t kv_stride_blk = (int64_t)num_kv_heads * HS * BS;  // elements per block (keys or values)
    for (int pg = pages0 + wave; pg < pages1; pg += PA_WAVES) {
        const int64_t blk = (int64_t)__builtin_amdgcn_readfirstlane(bt[pg]);
        const uint16_t *kp = kc + blk * kv_stride_blk + (int64_t)kvh * HS * BS;
        const uint16_t *vp = vc + blk * kv_stride_blk + (int64_t)kvh * HS * BS;
        uint4 kv[NP], vv[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = lane + 64 * i;
            kv[i] = make_uint4(0, 0, 0, 0);
            vv[i] = make_uint4(0, 0, 0, 0);
            if (p < PIECES) {
                kv[i] = *(const uint4 *)(kp + 8 * p);
                vv[i] = *(const uint4 *)(vp + 8 * p);
            }
        }
        // logits of slot `slot` for each head of the group
        float lg[GC];
#pragma unroll
        for (int g = 0; g < GC; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                s = fdot2(kv[i].x, qv[i][g][0], s);
                s = fdot2(kv[i].y, qv[i][g][1], s);
                s = fdot2(kv[i].z, qv[i][g][2], s);
                s = fdot2(kv[i].w, qv[i][g][3], s);
            }
#pragma unroll
            for (int m = BS; m < 64; m <<= 1) s += __shfl_xor(s, m, 64);
            lg[g] = s * scale;
        }
        const int tok = pg * BS + slot;
        const bool valid = tok < t1;
        float p[GC];
#pragma unroll
        for (int g = 0; g < GC; ++g) {
            float x = valid ? lg[g] : -INFINITY;
            float mx = x;
#pragma unroll
            for (int m = 1; m < BS; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
            const float m_new = fmaxf(m_run[g], mx);  // finite: every page holds >= 1 valid token
            const float alpha = __expf(m_run[g] - m_new);
            m_run[g] = m_new;
            p[g] = valid ? __expf(x - m_new) : 0.0f;
            l_run[g] = l_run[g] * alpha + p[g];  // per-lane partial sum over this lane's slot
#pragma unroll
            for (int i = 0; i < NP; ++i) acc[i][g] *= alpha;
        }
        // p for the 8 slots of this lane's value group, as f16 pairs, per head
        uint32_t pk[GC][4];
#pragma unroll
        for (int g = 0; g < GC; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float a = __shfl(p[g], 8 * vsg + 2 * j, 64);
                const float b = __shfl(p[g], 8 * vsg + 2 * j + 1, 64);
                pk[g][j] = pack_h2(a, b);
            }
        if (pg * BS + BS > t1) {  // last, partial page: zero values past the context (they may be NaN)
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                uint32_t w[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int s0 = pg * BS + 8 * vsg + 2 * j;
                    if (s0 >= t1) w[j] &= 0xffff0000u;
                    if (s0 + 1 >= t1) w[j] &= 0x0000ffffu;
                }
                vv[i] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
#pragma unroll
        for (int g = 0; g < GC; ++g)
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                float s = acc[i][g];
                s = fdot2(vv[i].x, pk[g][0], s);
                s = fdot2(vv[i].y, pk[g][1], s);
                s = fdot2(vv[i].z, pk[g][2], s);
                s = fdot2(vv[i].w, pk[g][3], s);
                acc[i][g] = s;
            }
    }

    // per-wave totals: sum over slots, acc over slot groups
#pragma unroll
    for (int g = 0; g < GC; ++g) {
#pragma unroll
        for (int m = 1; m < BS; m <<= 1) l_run[g] += __shfl_xor(l_run[g], m, 64);
#pragma unroll
        for (int i = 0; i < NP; ++i)
#pragma unroll
            for (int m = 1; m < SG; m <<= 1) acc[i][g] += __shfl_xor(acc[i][g], m, 64);
    }

    // merge the waves through LDS: max, sum, acc[HS] per head
    __shared__ float s_m[PA_WAVES][GC], s_l[PA_WAVES][GC];
    __shared__ float s_acc[PA_WAVES][GC][HS];
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < GC; ++g) {
            s_m[wave][g] = m_run[g];
            s_l[wave][g] = l_run[g];
        }
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int pidx = lane + 64 * i;
        const int d = pidx / SG;
        if (pidx < PIECES && vsg == 0)
#pragma unroll
            for (int g = 0; g < GC; ++g) s_acc[wave][g][d] = acc[i][g];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < GC * HS; e += blockDim.x) {
        const int g = e / HS, d = e % HS;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < PA_WAVES; ++w) M = fmaxf(M, s_m[w][g]);
        float lsum = 0.0f, a = 0.0f;
#pragma unroll
        for (int w = 0; w < PA_WAVES; ++w) {
            const float f = s_m[w][g] == -INFINITY ? 0.0f : __expf(s_m[w][g] - M);
            lsum += f * s_l[w][g];
            a += f * s_acc[w][g][d];
        }
        float *slotp = part_slot<HS>(scratch, seq, head0 + g, part, num_heads, P);
        slotp[2 + d] = a;
        if (d == 0) {
            slotp[0] = M;
            slotp[1] = lsum;
        }
    }
}

// Merge the partitions of one (sequence, head) and write f16 output.
template <int HS>
__global__ void __launch_bounds__(256) k_paged_attn_reduce(uint16_t *__restrict__ out, const float *__restrict__ scratch,
                                                           const int32_t *__restrict__ lens, int num_heads, int P) {
    const int head = blockIdx.x, seq = blockIdx.y;
    const int L = lens[seq];
    // partitions holding this sequence's context (never more than were written)
    const int np = min(P, L > 0 ? (L + PA_PART - 1) / PA_PART : 1);
    const float *base = scratch + (int64_t)(seq * num_heads + head) * P * (HS + 2);
    float M = -INFINITY;
    for (int p = 0; p < np; ++p) M = fmaxf(M, base[(int64_t)p * (HS + 2)]);
    float lsum = 0.0f;
    for (int p = 0; p < np; ++p) {
        const float m = base[(int64_t)p * (HS + 2)];
        lsum += m == -INFINITY ? 0.0f : __expf(m - M) * base[(int64_t)p * (HS + 2) + 1];
    }
    const float inv = 1.0f / (lsum + 1e-6f);
    for (int d = threadIdx.x; d < HS; d += blockDim.x) {
        float a = 0.0f;
        for (int p = 0; p < np; ++p) {
            const float m = base[(int64_t)p * (HS + 2)];
            if (m != -INFINITY) a += __expf(m - M) * base[(int64_t)p * (HS + 2) + 2 + d];
        }
        out[((int64_t)seq * num_heads + head) * HS + d] = f2h(a * inv);
    }
}

static int pa_partitions(const tlh_paged_attention_args &a) {
    return a.max_context_len > 0 ? (a.max_context_len + PA_PART - 1) / PA_PART : 1;
}

size_t paged_attention_scratch_bytes(const tlh_paged_attention_args &a) {
    return (size_t)a.num_seqs * a.num_heads * pa_partitions(a) * (a.head_size + 2) * sizeof(float);
}

template <int HS, int BS, int GC>
static void launch_pa3(const tlh_paged_attention_args &a, float *scratch, hipStream_t stream) {
    const int P = pa_partitions(a);
    const int groups = (a.num_heads / a.num_kv_heads) / GC;
    hipLaunchKernelGGL((k_paged_attn<HS, BS, GC>), dim3(a.num_kv_heads * groups, a.num_seqs, P), dim3(256), 0,
                       stream, (const uint16_t *)a.q, (const uint16_t *)a.k_cache, (const uint16_t *)a.v_cache,
                       a.block_tables, a.context_lens, a.num_heads, a.num_kv_heads, a.max_blocks_per_seq, a.scale, P,
                       scratch);
    hipLaunchKernelGGL((k_paged_attn_reduce<HS>), dim3(a.num_heads, a.num_seqs), dim3(HS < 256 ? HS : 256), 0, stream,
                       (uint16_t *)a.out, (const float *)scratch, a.context_lens, a.num_heads, P);
}

template <int HS, int BS>
static void launch_pa2(const tlh_paged_attention_args &a, float *scratch, hipStream_t stream) {
    const int G = a.num_heads / a.num_kv_heads;
    if (G % 4 == 0)
        launch_pa3<HS, BS, 4>(a, scratch, stream);
    else if (G % 2 == 0)
        launch_pa3<HS, BS, 2>(a, scratch, stream);
    else
        launch_pa3<HS, BS, 1>(a, scratch, stream);
}

template <int HS>
static void launch_pa1(const tlh_paged_attention_args &a, float *scratch, hipStream_t stream) {
    switch (a.block_size) {
    case 8: launch_pa2<HS, 8>(a, scratch, stream); break;
    case 16: launch_pa2<HS, 16>(a, scratch, stream); break;
    default: launch_pa2<HS, 32>(a, scratch, stream); break;
    }
}

tlh_status launch_paged_attention(const tlh_paged_attention_args &a, void *scratch, size_t, hipStream_t stream) {
    float *s = (float *)scratch;
    switch (a.head_size) {
    case 64: launch_pa1<64>(a, s, stream); break;
    case 80: launch_pa1<80>(a, s, stream); break;
    case 96: launch_pa1<96>(a, s, stream); break;
    case 112: launch_pa1<112>(a, s, stream); break;
    case 128: launch_pa1<128>(a, s, stream); break;
    case 192: launch_pa1<192>(a, s, stream); break;
    case 256: launch_pa1<256>(a, s, stream); break;
    default: return set_error(TLH_INVALID, "paged_attention: head_size %d", a.head_size);
    }
    return check_launch("paged_attention");
}

// ------------------------------------------------------- reshape_and_cache
// reshape_and_cache_kernel.cu:31-84: one workgroup per token, 16-byte pieces
// of 8 dims; keys land as one contiguous piece, values scatter along slots.
__global__ void __launch_bounds__(256) k_reshape_and_cache(const uint16_t *__restrict__ key,
                                                           const uint16_t *__restrict__ value,
                                                           uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                           const int64_t *__restrict__ slots, int kvh, int hs,
                                                           int bs) {
    const int t = blockIdx.x;
    const int64_t slot = slots[t];
    if (slot < 0) return;
    const int64_t blk = slot / bs;
    const int off = (int)(slot % bs);
    const int chunks = kvh * hs / 8;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
        const int h = c / (hs / 8), ch = c % (hs / 8);
        const int64_t src = (int64_t)t * kvh * hs + 8 * (int64_t)c;
        const uint4 kk = *(const uint4 *)(key + src);
        *(uint4 *)(kc + (((blk * kvh + h) * (hs / 8) + ch) * bs + off) * 8) = kk;
        const uint4 vv = *(const uint4 *)(value + src);
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
                                    int block_size, hipStream_t stream) {
    if ((((uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache) & 15) != 0)
        return set_error(TLH_INVALID, "reshape_and_cache: key, value and key cache must be 16-byte aligned");
    hipLaunchKernelGGL(k_reshape_and_cache, dim3(num_tokens), dim3(128), 0, stream, (const uint16_t *)key,
                       (const uint16_t *)value, (uint16_t *)k_cache, (uint16_t *)v_cache, slots, num_kv_heads,
                       head_size, block_size);
    return check_launch("reshape_and_cache");
}

}  // namespace tlh

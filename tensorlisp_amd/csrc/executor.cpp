// The graph executor (include/tlhip.h, "executor"): ggml IR in, a recorded
// list of launches on this library's entry points out, replayed per run
// eagerly or as one captured hipGraph. Host code only.
//
// It takes the place of the reference's Executor::compile / Program::run
// (crates/kernels/src/cuda/exec.rs:27-226) over its IR (graph.rs:72-229) and
// memory plan (plan.rs:56-189): lowering per node as Ctx::lower decides
// (lower.rs:175-213), then a liveness plan of one arena, then replay.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "kernels.hpp"

namespace tlh {
namespace {

constexpr int64_t ALIGN = 256;
int64_t align_up(int64_t n) { return (n + ALIGN - 1) / ALIGN * ALIGN; }

enum BufKind { B_NONE, B_ARENA, B_IO, B_STATE, B_WEIGHT };
struct Place {
    int buf = B_NONE;
    int32_t index = -1;  // weight index for B_WEIGHT
    int64_t off = 0;
};

enum DispatchKind { D_MUL_MAT, D_MM_QUANTIZE, D_MM_COMPUTE, D_FLASH_ATTN, D_CORE, D_NORM_CHAIN, D_MULTI_GEMV,
                    D_ARGMAX_SPLIT, D_CORE_MULTI, D_PAGED_ATTN, D_PAGED_WRITE, D_MUL_MAT_ID,
                    D_MM_COMPUTE_MULTI, D_GEMV_PRO };
constexpr int NSRC = 5;  // sources a dispatch reads (the paged nodes have five)
struct Dispatch {
    DispatchKind kind;
    int core_kind = 0;
    tlh_op op;
    Place src[NSRC];
    Place dst;
    int pos = 0;            // node position (the first one, for fused nodes)
    int pos_last = 0;       // last node position a fused dispatch covers
    int block = -1;         // scratch block index
    size_t scratch_bytes = 0;
    // D_MULTI_GEMV: the member MUL_MATs (shared activation in src[1])
    int nmem = 0;
    int mpos[3] = {0, 0, 0};  // D_MM_COMPUTE_MULTI: the members' node positions
    tlh_op mop[3];
    Place mw[3], mdst[3];
    // D_CORE_MULTI: independent element-wise ops in one launch
    int nsub = 0;
    int sub_kind[4];
    tlh_op sop[4];
    Place ssrc[4][4], sdst[4];
    // D_PAGED_ATTN: geometry and scale (pointers are set per launch);
    // D_PAGED_WRITE: tokens, kv heads, head size, block size
    tlh_paged_attention_args pa{};
    int pa_f32 = 0;  // D_PAGED_ATTN: dst is a fused cast's f32 tensor
    // D_GEMV_PRO: a register GEMV over the members (as D_MULTI_GEMV) that forms
    // its activation from the norm chain before it (has_norm: nop, the chain's
    // p, q, w, s in nsrc[0..3], its output y in ndst) and / or applies the
    // SwiGLU after it (has_glu: gop, h in gdst)
    int has_norm = 0, has_glu = 0;
    tlh_op nop, gop;
    Place nsrc[4], ndst, gdst;
    // D_CORE GLU, D_NORM_CHAIN: also quantizes its output for a MUL_MAT (type,
    // activation rows, f16 codes) into that MUL_MAT's scratch block
    int nq_type = 0, nq_f16 = 0;
    int64_t nq_rows = 0;
    int64_t rt_off = 0;  // batched epilogue: byte offset of its rotation table in the program's table buffer
    tlh_op nq_op;          // that MUL_MAT (its quantize launch, if the fused form is refused)
    size_t pa_own = 0;     // D_PAGED_ATTN with nq_type: its own scratch's offset in the shared block
    int32_t pw[4] = {0, 0, 0, 0};
    int64_t pw_blocks = 0;  // D_PAGED_WRITE: blocks in the smaller pool (slots past it are dropped)
    int pw_f32[2] = {0, 0};  // D_PAGED_WRITE: key / value read as f32 (a fused cast)
    // D_GEMV_PRO with has_epi: member rows leave through the store epilogue
    // (epi: layouts, types, geometry and rotation; its pointers come from
    // edst / eidx / epos / eff per launch) in place of the `absorbed`
    // dispatches, which run one by one after a plain GEMV when the fused
    // launch is refused
    int has_epi = 0;
    GemvEpi epi;
    Place edst[3], eidx[3], epos, eff;
    Place edst2[3];  // the second (paged pool) store of a dual segment
    // D_MUL_MAT / D_MM_COMPUTE: leave the K-split partials (no chunk-sum launch)
    // for the norm chain that adds them; D_NORM_CHAIN: q's rows are the partials
    // of dispatch pp_disp (pp_off bytes into its scratch; pp_chunks, pp_cstride)
    int keep_part = 0;
    int pp_disp = -1;
    int pp_chunks = 0;
    int64_t pp_off = 0, pp_cstride = 0;
    std::vector<Dispatch> absorbed;
};

// ggml type traits used for byte sizes: (block elements, block bytes)
bool type_traits(int ty, int64_t &blck, int64_t &size) {
    switch (ty) {
    case TLH_TYPE_F32: blck = 1, size = 4; return true;
    case TLH_TYPE_F16: blck = 1, size = 2; return true;
    case TLH_TYPE_Q4_0: blck = 32, size = 18; return true;
    case 3: blck = 32, size = 20; return true;   // q4_1
    case 6: blck = 32, size = 22; return true;   // q5_0
    case 7: blck = 32, size = 24; return true;   // q5_1
    case TLH_TYPE_Q8_0: blck = 32, size = 34; return true;
    case 9: blck = 32, size = 36; return true;   // q8_1
    case 10: blck = 256, size = 84; return true;   // q2_K
    case 11: blck = 256, size = 110; return true;  // q3_K
    case TLH_TYPE_Q4_K: blck = 256, size = 144; return true;
    case 13: blck = 256, size = 176; return true;  // q5_K
    case TLH_TYPE_Q6_K: blck = 256, size = 210; return true;
    case TLH_TYPE_Q8_K: blck = 256, size = 292; return true;
    case 24: blck = 1, size = 1; return true;  // i8
    case 25: blck = 1, size = 2; return true;  // i16
    case 26: blck = 1, size = 4; return true;  // i32
    case 27: blck = 1, size = 8; return true;  // i64
    case 28: blck = 1, size = 8; return true;  // f64
    case 30: blck = 1, size = 2; return true;  // bf16
    default: return false;
    }
}

int64_t nelements(const tlh_ir_tensor &t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }

// ggml_nbytes (graph.rs Tensor::nbytes)
int64_t nbytes(const tlh_ir_tensor &t) {
    if (nelements(t) == 0) return 0;
    int64_t blck = 1, size = 4;
    type_traits(t.ty, blck, size);
    int64_t n = blck == 1 ? size + (t.ne[0] - 1) * t.nb[0] : t.ne[0] * t.nb[0] / blck;
    for (int i = 1; i < 4; ++i) n += (t.ne[i] - 1) * t.nb[i];
    return n;
}

bool is_view_op(const tlh_ir_tensor &t) {
    return !strcmp(t.op, "NONE") || !strcmp(t.op, "RESHAPE") || !strcmp(t.op, "VIEW") || !strcmp(t.op, "TRANSPOSE") ||
           !strcmp(t.op, "PERMUTE");
}

float f32_of(int32_t bits) {
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
int64_t bits_of(float f) {
    int32_t b;
    memcpy(&b, &f, 4);
    return b;  // sign-extended, as OpBlob::float stores it
}

struct Graph {
    const tlh_ir_tensor *t = nullptr;
    int32_t n = 0;
    std::vector<int32_t> nodes, keep;

    int32_t root(int32_t id, int64_t &extra) const {
        extra = t[id].view_src >= 0 ? t[id].view_offs : 0;
        return t[id].view_src >= 0 ? t[id].view_src : id;
    }
    const char *name(int32_t id) const { return t[id].op; }
};

struct Unsupported {
    std::string op, example;
    int count = 0;
};

struct Block {
    int64_t first, last, size;
    int32_t tensor;  // arena root, or -1 for a scratch block
    int64_t off = 0;
};

// One program: the lowered launches and the plan.
struct Lowered {
    std::vector<Dispatch> d;
    std::vector<Block> blocks;        // arena blocks (tensor roots, then scratch)
    std::vector<int64_t> arena_off;   // per tensor root (-1: not in the arena)
    std::vector<int64_t> node_scratch;  // per node position (-1: none)
    std::vector<int32_t> node_ids;      // tensor id per node position
    int64_t arena = 0;
    int64_t rt_bytes = 0;  // the batched epilogues' rotation tables
};

class Lowering {
  public:
    Lowering(const Graph &g) : g_(g) {}

    tlh_status run(Lowered &out) {
        out.d.clear();
        out.node_ids = g_.nodes;
        for (size_t pos = 0; pos < g_.nodes.size(); ++pos) {
            const int32_t id = g_.nodes[pos];
            const tlh_ir_tensor &t = g_.t[id];
            if (is_view_op(t) || nelements(t) == 0) continue;
            std::string why;
            if (!lower_node((int)pos, id, out.d, why)) {
                bool found = false;
                for (auto &u : missing_)
                    if (u.op == t.op) {
                        ++u.count;
                        found = true;
                    }
                if (!found) missing_.push_back({t.op, "node " + std::to_string(id) + ": " + why, 1});
            }
        }
        if (!missing_.empty()) {
            std::string list;
            for (auto &u : missing_) {
                if (!list.empty()) list += "; ";
                list += u.op + " x" + std::to_string(u.count) + " (e.g. " + u.example + ")";
            }
            return set_error(TLH_UNSUPPORTED, "native HIP: not implemented: %s", list.c_str());
        }
        for (Dispatch &x : out.d) x.pos_last = x.pos;
        fuse_norm_chains(out.d);
        fuse_multi_gemv(out.d);
        fuse_gemv_pro(out.d);
        fuse_rope_rows(out.d);
        fuse_rope_cast(out.d);
        fuse_paged_cast(out.d);
        fuse_cache_write_cast(out.d);
        fuse_gemv_epilogue(out.d, false);
        group_mul_mats(out.d);
        merge_mm_computes(out.d);
        fuse_gemv_epilogue(out.d, true);  // the batched Q / K / V projection's merged compute
        group_elementwise(out.d);
        fuse_act_quantize(out.d);
        group_elementwise(out.d);  // merged computes can leave element-wise launches adjacent
        fuse_partials_into_norm(out.d);  // last: it refers to dispatches by index
        plan(out);
        return TLH_OK;
    }

  private:
    const Graph &g_;
    std::vector<Unsupported> missing_;

    static tlh_tensor desc(const tlh_ir_tensor &t) {
        tlh_tensor d;
        memset(&d, 0, sizeof d);
        for (int i = 0; i < 4; ++i) d.ne[i] = t.ne[i], d.nb[i] = t.nb[i];
        d.ty = t.ty;
        return d;
    }

    Place place_of(int32_t id) const {
        int64_t extra = 0;
        const int32_t r = g_.root(id, extra);
        Place p;
        p.off = extra;
        switch (g_.t[r].storage) {
        case TLH_STORE_WEIGHT: p.buf = B_WEIGHT, p.index = g_.t[r].storage_index; break;
        case TLH_STORE_STATE: p.buf = B_STATE, p.index = g_.t[r].storage_index; break;
        case TLH_STORE_INPUT: p.buf = B_IO, p.index = g_.t[r].storage_index; break;
        default: p.buf = B_ARENA, p.index = r; break;
        }
        return p;
    }

    Dispatch base(int pos, int32_t id, std::initializer_list<int> srcs) const {
        Dispatch d;
        memset(&d.op, 0, sizeof d.op);
        int i = 0;
        for (int s : srcs) {
            const int32_t sid = s >= 0 ? g_.t[id].src[s] : -1;
            if (sid >= 0) {
                d.op.t[i] = desc(g_.t[sid]);
                d.src[i] = place_of(sid);
            }
            ++i;
        }
        d.op.t[4] = desc(g_.t[id]);
        d.dst = place_of(id);
        d.pos = pos;
        return d;
    }

    bool core(std::vector<Dispatch> &out, Dispatch d, int kind, std::string &why) {
        d.kind = D_CORE;
        d.core_kind = kind;
        const tlh_status st = tlh_core_check(kind, &d.op, d.src[1].buf != B_NONE, d.src[2].buf != B_NONE);
        if (st != TLH_OK) {
            why = tlh_last_error();
            return false;
        }
        out.push_back(d);
        return true;
    }

    // A ggml CUSTOM node without a function names a paged-attention kernel in
    // its userdata (op_params[4..5] as one u64, low to high bits: kind 4,
    // kv heads 4, block size 8, max context 16, scale f32), as Ctx::custom
    // decodes it (crates/kernels/src/cuda/lower.rs:660-753):
    //  kind 1: paged attention, sources q f16 [hs, heads, seqs] (contiguous),
    //          key pool, value pool (f16), block tables i32 [max_blocks, seqs],
    //          context lengths i32 [seqs]; the node is f16 [hs, heads, seqs];
    //  kind 2: cache write, sources key and value f16 [hs * kv_heads, tokens]
    //          (contiguous rows), the two pools, slots (one i64 per token, as
    //          two i32); the node is a dummy.
    bool custom(int pos, int32_t id, std::vector<Dispatch> &out, std::string &why) {
        const tlh_ir_tensor &t = g_.t[id];
        const uint64_t ud = (uint64_t)(uint32_t)t.op_params[4] | (uint64_t)(uint32_t)t.op_params[5] << 32;
        const int kind = (int)(ud & 15), kvh = (int)((ud >> 4) & 15), bs = (int)((ud >> 8) & 255),
                  max_ctx = (int)((ud >> 16) & 0xffff);
        const float scale = f32_of((int32_t)(uint32_t)(ud >> 32));
        for (int i = 0; i < 5; ++i)
            if (t.src[i] < 0) return why = "a paged node takes five sources", false;
        auto T = [&](int i) -> const tlh_ir_tensor & { return g_.t[t.src[i]]; };
        auto is_f16 = [](const tlh_ir_tensor &x) { return x.ty == TLH_TYPE_F16; };
        Dispatch d = base(pos, id, {0, 1, 2, 3});
        d.src[4] = place_of(t.src[4]);
        if (kind == 1) {
            const tlh_ir_tensor &q = T(0);
            if (!(is_f16(q) && is_f16(T(1)) && is_f16(T(2)) && is_f16(t)))
                return why = "paged attention takes f16 q, caches and output", false;
            if (q.nb[0] != 2 || q.nb[1] != q.ne[0] * 2 || q.nb[2] != q.ne[0] * q.ne[1] * 2 || t.ne[0] != q.ne[0] ||
                t.ne[1] != q.ne[1] || t.ne[2] != q.ne[2] || t.nb[1] != t.ne[0] * 2 || t.nb[2] != t.ne[0] * t.ne[1] * 2)
                return why = "paged attention takes a contiguous q and an output of its shape", false;
            if (T(3).ty != TLH_TYPE_I32 || T(4).ty != TLH_TYPE_I32 || T(3).ne[1] < q.ne[2] || T(4).ne[0] < q.ne[2])
                return why = "paged attention takes i32 block tables [max_blocks, seqs] and lengths [seqs]", false;
            tlh_paged_attention_args &a = d.pa;
            a.num_seqs = (int32_t)q.ne[2];
            a.num_heads = (int32_t)q.ne[1];
            a.num_kv_heads = kvh;
            a.head_size = (int32_t)q.ne[0];
            a.block_size = bs;
            a.max_blocks_per_seq = (int32_t)T(3).ne[0];
            a.max_context_len = max_ctx;
            a.scale = scale;
            const int64_t pool = (int64_t)kvh * a.head_size * bs * 2;  // bytes per block of each pool
            if (kvh < 1 || nbytes(T(1)) < pool || nbytes(T(2)) < pool || nbytes(T(1)) % pool || nbytes(T(2)) % pool)
                return why = "paged attention: pools are not whole blocks of kv_heads x head_size x block_size", false;
            size_t bytes = 0;
            if (tlh_paged_attention_scratch_bytes(&a, &bytes) != TLH_OK) return why = tlh_last_error(), false;
            d.kind = D_PAGED_ATTN;
            d.scratch_bytes = bytes;
        } else if (kind == 2) {
            const tlh_ir_tensor &k = T(0), &v = T(1);
            if (!(is_f16(k) && is_f16(v) && is_f16(T(2)) && is_f16(T(3))))
                return why = "the cache write takes f16 keys, values and caches", false;
            const int64_t tokens = k.ne[1];
            int64_t ns = 1;
            for (int i = 0; i < 4; ++i) ns *= T(4).ne[i];
            if (ns != 2 * tokens || T(4).ty != TLH_TYPE_I32 || k.nb[1] != k.ne[0] * 2 || v.nb[1] != v.ne[0] * 2 ||
                v.ne[0] != k.ne[0] || v.ne[1] != tokens || k.nb[0] != 2 || v.nb[0] != 2)
                return why = "the cache write takes contiguous keys and one i64 slot per token", false;
            if (kvh < 1 || k.ne[0] % kvh) return why = "the cache write: rows are not kv_heads x head_size", false;
            d.pw[0] = (int32_t)tokens;
            d.pw[1] = kvh;
            d.pw[2] = (int32_t)(k.ne[0] / kvh);
            d.pw[3] = bs;
            if (d.pw[2] % 8 || !(bs == 8 || bs == 16 || bs == 32))
                return why = "the cache write: head size a multiple of 8, block size 8, 16 or 32", false;
            const int64_t block_bytes = (int64_t)kvh * d.pw[2] * bs * 2;
            d.pw_blocks = std::min(nbytes(T(2)), nbytes(T(3))) / block_bytes;
            d.kind = D_PAGED_WRITE;
        } else {
            return why = "unknown custom op", false;
        }
        out.push_back(d);
        return true;
    }

    // Ctx::lower's table (lower.rs:188-211) for the ops this library runs.
    bool lower_node(int pos, int32_t id, std::vector<Dispatch> &out, std::string &why) {
        const tlh_ir_tensor &t = g_.t[id];
        const std::string op = t.op;
        const int32_t *p = t.op_params;
        auto src = [&](int i) { return t.src[i]; };
        if (op == "MUL_MAT") {
            if (src(0) < 0 || src(1) < 0) return why = "missing source", false;
            Dispatch d = base(pos, id, {0, 1});
            const tlh_ir_tensor &a = g_.t[src(0)];
            d.op.x[0] = a.ne[2] ? t.ne[2] / a.ne[2] : 0;  // r2, r3 (lower.rs:556-559)
            d.op.x[1] = a.ne[3] ? t.ne[3] / a.ne[3] : 0;
            size_t bytes = 0;
            if (tlh_mul_mat_scratch_bytes(&d.op, &bytes) != TLH_OK) return why = tlh_last_error(), false;
            d.kind = D_MUL_MAT;
            d.scratch_bytes = bytes;
            out.push_back(d);
            return true;
        }
        if (op == "MUL_MAT_ID") {
            if (src(0) < 0 || src(1) < 0 || src(2) < 0) return why = "missing source", false;
            Dispatch d = base(pos, id, {0, 1, 2});
            size_t bytes = 0;
            if (tlh_mul_mat_id_scratch_bytes(&d.op, &bytes) != TLH_OK) return why = tlh_last_error(), false;
            d.kind = D_MUL_MAT_ID;
            d.scratch_bytes = bytes;
            out.push_back(d);
            return true;
        }
        if (op == "FLASH_ATTN_EXT") {
            if (src(4) >= 0) return why = "attention sinks", false;
            Dispatch d = base(pos, id, {0, 1, 2, 3});
            float scale = f32_of(p[0]);
            const float max_bias = f32_of(p[1]), softcap = f32_of(p[2]);
            if (softcap != 0.0f) scale /= softcap;
            const int64_t nh = g_.t[src(0)].ne[2];
            const uint32_t nhl2 = 1u << (uint32_t)floorf(log2f((float)nh));
            d.op.x[0] = bits_of(scale);
            d.op.x[1] = bits_of(max_bias);
            d.op.x[2] = bits_of(powf(2.0f, -max_bias / (float)nhl2));
            d.op.x[3] = bits_of(powf(2.0f, -(max_bias / 2.0f) / (float)nhl2));
            d.op.x[4] = nhl2;
            d.op.x[5] = bits_of(softcap);
            size_t bytes = 0;
            if (tlh_flash_attn_ext_scratch_bytes(&d.op, &bytes) != TLH_OK) return why = tlh_last_error(), false;
            d.kind = D_FLASH_ATTN;
            d.scratch_bytes = bytes;
            out.push_back(d);
            return true;
        }
        if (op == "CUSTOM") return custom(pos, id, out, why);
        if (op == "ADD" || op == "SUB" || op == "MUL" || op == "DIV") {
            Dispatch d = base(pos, id, {0, 1});
            d.op.x[0] = op == "ADD" ? 0 : op == "SUB" ? 1 : op == "MUL" ? 2 : 3;
            return core(out, d, TLH_CORE_BIN, why);
        }
        static const std::map<std::string, int> unary = {{"SCALE", 100}, {"FILL", 101}, {"CLAMP", 102},
                                                         {"LEAKY_RELU", 103}, {"SQR", 104}, {"SQRT", 105},
                                                         {"SIN", 106}, {"COS", 107}, {"LOG", 108}, {"UNARY", -1}};
        if (auto u = unary.find(op); u != unary.end()) {  // lower.rs:253-290
            Dispatch d = base(pos, id, {0});
            int code = u->second;
            if (code == -1) {
                code = p[0];
                if (code == 17) return why = "xielu", false;
            }
            if (code == 100 || code == 102) d.op.x[1] = bits_of(f32_of(p[0])), d.op.x[2] = bits_of(f32_of(p[1]));
            if (code == 101 || code == 103) d.op.x[1] = bits_of(f32_of(p[0]));
            d.op.x[0] = code;
            return core(out, d, TLH_CORE_UNARY, why);
        }
        if (op == "NORM" || op == "RMS_NORM") {
            Dispatch d = base(pos, id, {0});
            d.op.x[0] = op == "RMS_NORM";
            d.op.x[1] = bits_of(f32_of(p[0]));
            return core(out, d, TLH_CORE_NORM, why);
        }
        if (op == "GET_ROWS") return core(out, base(pos, id, {0, 1}), TLH_CORE_GET_ROWS, why);
        if (op == "SET_ROWS") return core(out, base(pos, id, {0, 1}), TLH_CORE_SET_ROWS, why);
        if (op == "CPY" || op == "DUP" || op == "CONT") return core(out, base(pos, id, {0}), TLH_CORE_CPY, why);
        if (op == "ARGMAX") {
            Dispatch d = base(pos, id, {0});
            if (!core(out, d, TLH_CORE_ARGMAX, why)) return false;
            if (d.op.t[0].ne[0] >= 8192) {  // a vocabulary: chunks over many workgroups
                out.back().kind = D_ARGMAX_SPLIT;
                out.back().scratch_bytes = argmax_split_scratch_bytes(d.op);
            }
            return true;
        }
        if (op == "GLU") {
            Dispatch d = base(pos, id, {0, 1});
            d.op.x[0] = p[0];
            d.op.x[1] = p[1];
            return core(out, d, TLH_CORE_GLU, why);
        }
        if (op == "SOFT_MAX") {  // lower.rs:314-341
            if (src(2) >= 0) return why = "sinks are not supported by the soft_max lowering", false;
            Dispatch d = base(pos, id, {0, 1});
            const float scale = f32_of(p[0]), max_bias = f32_of(p[1]);
            const uint32_t nhl2 = 1u << (uint32_t)floorf(log2f((float)g_.t[src(0)].ne[2]));
            d.op.x[0] = bits_of(scale);
            d.op.x[1] = bits_of(max_bias);
            d.op.x[2] = bits_of(powf(2.0f, -max_bias / (float)nhl2));
            d.op.x[3] = bits_of(powf(2.0f, -(max_bias / 2.0f) / (float)nhl2));
            d.op.x[4] = nhl2;
            return core(out, d, TLH_CORE_SOFT_MAX, why);
        }
        if (op == "ROPE") {  // lower.rs:422-466 with ggml_rope_yarn_corr_dims (ggml.c:4369-4381)
            Dispatch d = base(pos, id, {0, 1, 2});
            const int n_dims = p[1], mode = p[2], n_ctx_orig = p[4];
            const float freq_base = f32_of(p[5]), freq_scale = f32_of(p[6]), ext_factor = f32_of(p[7]);
            const float attn_factor = f32_of(p[8]), beta_fast = f32_of(p[9]), beta_slow = f32_of(p[10]);
            auto corr = [&](float beta) {
                return n_dims * logf(n_ctx_orig / (beta * 2 * 3.14159265358979323846f)) / (2 * logf(freq_base));
            };
            const float start = floorf(corr(beta_fast)), end = ceilf(corr(beta_slow));
            const float c0 = 0.0f > start ? 0.0f : start;
            const float c1 = (float)(n_dims - 1) < end ? (float)(n_dims - 1) : end;
            d.op.x[0] = n_dims;
            d.op.x[1] = mode;
            d.op.x[2] = bits_of(freq_scale);
            d.op.x[3] = bits_of(ext_factor);
            d.op.x[4] = bits_of(attn_factor);
            d.op.x[5] = bits_of(powf(freq_base, -2.0f / n_dims));
            d.op.x[6] = bits_of(c0);
            d.op.x[7] = bits_of(c1);
            d.op.x[8] = src(2) >= 0;
            return core(out, d, TLH_CORE_ROPE, why);
        }
        why = "op not implemented in the native HIP executor";
        return false;
    }

    int32_t node_of(const Dispatch &x) const { return g_.nodes[x.pos]; }

    void count_readers() {
        readers_.assign(g_.n, 0);
        reader_.assign(g_.n, -1);
        for (int32_t id : g_.nodes)
            for (int s = 0; s < 10; ++s)
                if (g_.t[id].src[s] >= 0) ++readers_[g_.t[id].src[s]], reader_[g_.t[id].src[s]] = id;
        for (int32_t id : g_.keep) ++readers_[id];
    }
    std::vector<int> readers_;
    std::vector<int32_t> reader_;  // the (last) node reading each tensor

    static bool f32_rows(const tlh_tensor &t) { return t.ty == TLH_TYPE_F32 && t.nb[0] == 4; }
    static bool same_ne(const tlh_tensor &a, const tlh_tensor &b) {
        return a.ne[0] == b.ne[0] && a.ne[1] == b.ne[1] && a.ne[2] == b.ne[2] && a.ne[3] == b.ne[3];
    }

    // [ADD ->] RMS_NORM / NORM -> MUL(weight) -> one k_norm_chain launch, when the
    // norm's result has no other reader, the MUL broadcasts a weight row over
    // it, and the ADD (if fused) feeds the norm directly with operands of its
    // own shape. The ADD's result is still written (it is read again later).
    void fuse_norm_chains(std::vector<Dispatch> &d) {
        count_readers();
        std::vector<Dispatch> out;
        out.reserve(d.size());
        for (size_t i = 0; i < d.size(); ++i) {
            const Dispatch &x = d[i];
            const bool is_norm = x.kind == D_CORE && x.core_kind == TLH_CORE_NORM;
            if (!is_norm || i + 1 >= d.size()) {
                out.push_back(x);
                continue;
            }
            const Dispatch &m = d[i + 1];
            const int32_t nid = node_of(x);
            const bool mul_ok = m.kind == D_CORE && m.core_kind == TLH_CORE_BIN && m.op.x[0] == 2 &&
                                g_.t[node_of(m)].src[0] == nid && readers_[nid] == 1 && f32_rows(m.op.t[1]) &&
                                m.op.t[1].ne[0] == x.op.t[0].ne[0] && f32_rows(m.op.t[4]) && same_ne(m.op.t[4], x.op.t[0]);
            if (!mul_ok) {
                out.push_back(x);
                continue;
            }
            // The fused kernel reads the row's tail (past its register cache)
            // from the sources again after writing the ADD's sum and the
            // output, so no destination may share storage with a source: an
            // in-place ADD (add-inplace) keeps its own launch.
            if (same_root(m.dst, x.src[0]) || same_root(m.dst, m.src[1])) {
                out.push_back(x);
                continue;
            }
            bool with_add = false;
            if (!out.empty()) {
                const Dispatch &a = out.back();
                with_add = a.kind == D_CORE && a.core_kind == TLH_CORE_BIN && a.op.x[0] == 0 &&
                           node_of(a) == g_.t[nid].src[0] && f32_rows(a.op.t[0]) && f32_rows(a.op.t[1]) &&
                           f32_rows(a.op.t[4]) && same_ne(a.op.t[0], a.op.t[4]) && same_ne(a.op.t[1], a.op.t[4]) &&
                           !same_root(a.dst, a.src[0]) && !same_root(a.dst, a.src[1]) &&
                           !same_root(m.dst, a.src[0]) && !same_root(m.dst, a.src[1]);
            }
            Dispatch f;
            f.kind = D_NORM_CHAIN;
            memset(&f.op, 0, sizeof f.op);
            if (with_add) {
                const Dispatch a = out.back();
                out.pop_back();
                f.op.t[0] = a.op.t[0], f.op.t[1] = a.op.t[1], f.op.t[3] = a.op.t[4];
                f.src[0] = a.src[0], f.src[1] = a.src[1], f.src[3] = a.dst;
                f.pos = a.pos;
            } else {
                f.op.t[0] = x.op.t[0];
                f.src[0] = x.src[0];
                f.pos = x.pos;
            }
            f.op.t[2] = m.op.t[1];
            f.src[2] = m.src[1];
            f.op.t[4] = m.op.t[4];
            f.dst = m.dst;
            f.op.x[0] = x.op.x[0];
            f.op.x[1] = x.op.x[1];
            f.op.x[2] = with_add;
            f.pos_last = m.pos;
            out.push_back(f);
            ++i;  // the MUL is part of it
        }
        d.swap(out);
    }

    // MUL_MATs at N = 1 that read the same activation with weights of one type
    // and K -> one multi-segment register GEMV at the first one's place (up to
    // three: Q, K and V, or gate and up). Later members move up: their weights
    // are leaves and their activation is the first one's, so only their
    // outputs' lifetimes grow, which the plan sees through the dispatch's
    // position range. A write into the activation's storage ends the search.
    void fuse_multi_gemv(std::vector<Dispatch> &d) {
        auto single_ok = [&](const Dispatch &x) {
            const tlh_op *o = &x.op;
            return x.kind == D_MUL_MAT && x.src[0].buf == B_WEIGHT && x.dst.buf == B_ARENA && mul_mat_multi_ok(&o, 1);
        };
        std::vector<char> taken(d.size(), 0);
        std::vector<Dispatch> out;
        out.reserve(d.size());
        for (size_t i = 0; i < d.size(); ++i) {
            if (taken[i]) continue;
            const Dispatch &x = d[i];
            if (!single_ok(x)) {
                out.push_back(x);
                continue;
            }
            std::vector<size_t> mem{i};
            const Place &a = x.src[1];
            for (size_t j = i + 1; j < d.size() && mem.size() < 3; ++j) {
                const Dispatch &y = d[j];
                if (y.dst.buf == a.buf && y.dst.index == a.index) break;  // the activation is overwritten
                if (y.kind == D_NORM_CHAIN && y.src[3].buf == a.buf && y.src[3].index == a.index) break;
                if (taken[j] || !single_ok(y)) continue;
                const tlh_tensor &b0 = x.op.t[1], &b1 = y.op.t[1];
                bool same = y.src[1].buf == a.buf && y.src[1].index == a.index && y.src[1].off == a.off &&
                            y.op.t[0].ty == x.op.t[0].ty && same_ne(b0, b1);
                for (int k = 0; k < 4 && same; ++k) same = b0.nb[k] == b1.nb[k];
                if (!same) continue;
                const tlh_op *ops[3];
                for (size_t k = 0; k < mem.size(); ++k) ops[k] = &d[mem[k]].op;
                ops[mem.size()] = &y.op;
                if (mul_mat_multi_ok(ops, (int)mem.size() + 1)) mem.push_back(j);
            }
            if (mem.size() < 2) {
                out.push_back(x);
                continue;
            }
            Dispatch f = x;
            f.kind = D_MULTI_GEMV;
            f.nmem = (int)mem.size();
            f.scratch_bytes = 0;
            for (size_t k = 0; k < mem.size(); ++k) {
                const Dispatch &y = d[mem[k]];
                f.mop[k] = y.op;
                f.mw[k] = y.src[0];
                f.mdst[k] = y.dst;
                f.scratch_bytes = std::max(f.scratch_bytes, y.scratch_bytes);
                f.pos_last = std::max(f.pos_last, y.pos_last);
                taken[mem[k]] = 1;
            }
            out.push_back(f);
        }
        d.swap(out);
    }

    // A single-column GEMV (D_MULTI_GEMV, or one D_MUL_MAT the register GEMV
    // runs) takes in its neighbours, in one launch:
    //  * the [ADD ->] RMS_NORM -> MUL chain right before it when the chain's
    //    output is read by these MUL_MATs only (K <= 4096): each workgroup forms
    //    the normalized row itself (the ADD's sum is still written once);
    //  * a SwiGLU right after a gate / up pair when it alone reads their
    //    outputs: h = silu(gate) * up is stored instead of the pair.
    // The pieces' own tensors stay planned: a launch whose pointers the fused
    // kernel cannot take runs them one by one.
    static bool same_place(const Place &a, const Place &b) {
        return a.buf == b.buf && a.index == b.index && a.off == b.off;
    }
    void fuse_gemv_pro(std::vector<Dispatch> &d) {
        count_readers();
        auto gemv_ok = [&](const Dispatch &x) {
            if (x.kind == D_MULTI_GEMV) return true;
            const tlh_op *o = &x.op;
            return x.kind == D_MUL_MAT && x.src[0].buf == B_WEIGHT && mul_mat_multi_ok(&o, 1);
        };
        std::vector<Dispatch> out;
        out.reserve(d.size());
        for (size_t i = 0; i < d.size(); ++i) {
            if (!gemv_ok(d[i])) {
                out.push_back(d[i]);
                continue;
            }
            Dispatch f = d[i];
            if (f.kind == D_MUL_MAT) {  // one member
                f.nmem = 1;
                f.mop[0] = f.op;
                f.mw[0] = f.src[0];
                f.mdst[0] = f.dst;
            }
            bool fused = false;
            // the norm chain before it
            if (!out.empty()) {
                const Dispatch &c = out.back();
                const int32_t y = g_.nodes[c.pos_last];
                bool ok = c.kind == D_NORM_CHAIN && c.op.x[0] == 1 && readers_[y] == f.nmem &&
                          std::find(g_.keep.begin(), g_.keep.end(), y) == g_.keep.end() &&
                          same_place(f.src[1], c.dst) && f.mop[0].t[1].ne[0] <= 4096 &&
                          f.mop[0].t[1].ne[1] == 1 && c.op.t[0].ne[1] == 1 && c.op.t[0].ne[2] == 1 &&
                          c.op.t[0].ne[3] == 1;
                if (ok) {
                    f.has_norm = 1;
                    f.nop = c.op;
                    for (int k = 0; k < 4; ++k) f.nsrc[k] = c.src[k];
                    f.ndst = c.dst;
                    f.pos = c.pos;
                    f.pos_last = std::max(f.pos_last, c.pos_last);
                    out.pop_back();
                    fused = true;
                }
            }
            // the SwiGLU after a gate / up pair
            if (f.nmem == 2 && i + 1 < d.size()) {
                const Dispatch &gl = d[i + 1];
                const int32_t m0 = f.mdst[0].index, m1 = f.mdst[1].index;  // arena places: root tensor ids
                bool ok = f.mdst[0].buf == B_ARENA && f.mdst[1].buf == B_ARENA && gl.kind == D_CORE && gl.core_kind == TLH_CORE_GLU && gl.op.x[0] == 2 && gl.op.x[1] == 0 &&
                          gl.src[1].buf != B_NONE && f32_rows(gl.op.t[4]) && gl.op.t[4].ne[1] == 1 &&
                          gl.op.t[4].ne[2] == 1 && gl.op.t[4].ne[3] == 1 &&
                          f.mop[0].t[0].ne[1] == f.mop[1].t[0].ne[1] && gl.op.t[4].ne[0] == f.mop[0].t[0].ne[1];
                int gate = -1;
                if (ok && same_place(gl.src[0], f.mdst[0]) && same_place(gl.src[1], f.mdst[1])) gate = 0;
                if (ok && same_place(gl.src[0], f.mdst[1]) && same_place(gl.src[1], f.mdst[0])) gate = 1;
                ok = gate >= 0 && readers_[m0] == 1 && readers_[m1] == 1 &&
                     std::find(g_.keep.begin(), g_.keep.end(), m0) == g_.keep.end() &&
                     std::find(g_.keep.begin(), g_.keep.end(), m1) == g_.keep.end();
                if (ok) {
                    if (gate == 1) {  // members in gate, up order
                        std::swap(f.mop[0], f.mop[1]);
                        std::swap(f.mw[0], f.mw[1]);
                        std::swap(f.mdst[0], f.mdst[1]);
                    }
                    f.has_glu = 1;
                    f.gop = gl.op;
                    f.gdst = gl.dst;
                    f.pos_last = std::max(f.pos_last, gl.pos_last);
                    ++i;  // the SwiGLU is part of it
                    fused = true;
                }
            }
            if (fused) f.kind = D_GEMV_PRO;
            out.push_back(fused ? f : d[i]);
        }
        d.swap(out);
    }

    static bool same_root(const Place &a, const Place &b) {
        return a.buf != B_NONE && a.buf != B_WEIGHT && a.buf == b.buf && a.index == b.index;
    }
    // every place a dispatch reads, and the ones it writes
    static void places(const Dispatch &x, std::vector<Place> &rd, std::vector<Place> &wr) {
        rd.clear(), wr.clear();
        for (int k = 0; k < NSRC; ++k) rd.push_back(x.src[k]);
        wr.push_back(x.dst);
        if (x.kind == D_PAGED_WRITE) wr.push_back(x.src[2]), wr.push_back(x.src[3]);  // the two pools
        for (int k = 0; k < x.nmem; ++k) rd.push_back(x.mw[k]), wr.push_back(x.mdst[k]);
        for (int k = 0; k < x.nsub; ++k) {
            for (int j = 0; j < 4; ++j) rd.push_back(x.ssrc[k][j]);
            wr.push_back(x.sdst[k]);
        }
        if (x.kind == D_NORM_CHAIN) wr.push_back(x.src[3]);  // the ADD's result
        if (x.has_norm) {
            for (int k = 0; k < 3; ++k) rd.push_back(x.nsrc[k]);
            wr.push_back(x.nsrc[3]), wr.push_back(x.ndst);
        }
        if (x.has_glu) wr.push_back(x.gdst);
        if (x.has_epi) {
            for (int k = 0; k < 3; ++k) wr.push_back(x.edst[k]), wr.push_back(x.edst2[k]), rd.push_back(x.eidx[k]);
            rd.push_back(x.epos), rd.push_back(x.eff);
            std::vector<Place> r2, w2;
            for (const Dispatch &a : x.absorbed) {
                places(a, r2, w2);
                rd.insert(rd.end(), r2.begin(), r2.end());
                wr.insert(wr.end(), w2.begin(), w2.end());
            }
        }
    }
    static bool independent(const Dispatch &a, const Dispatch &b) {
        std::vector<Place> ra, wa, rb, wb;
        places(a, ra, wa);
        places(b, rb, wb);
        for (const Place &w : wa) {
            for (const Place &r : rb)
                if (same_root(w, r)) return false;
            for (const Place &w2 : wb)
                if (same_root(w, w2)) return false;
        }
        for (const Place &w : wb)
            for (const Place &r : ra)
                if (same_root(w, r)) return false;
        return true;
    }

    // ROPE whose result is only reshaped into the rows a SET_ROWS writes (a
    // K cache write): the rotation writes those cache rows itself, in the
    // cache's type, and the SET_ROWS goes away. Nothing in between may touch
    // the cache.
    static bool contiguous(const tlh_tensor &t) {
        const int64_t es = t.ty == TLH_TYPE_F32 ? 4 : t.ty == TLH_TYPE_F16 ? 2 : 0;
        return es && t.nb[0] == es && t.nb[1] == t.nb[0] * t.ne[0] && t.nb[2] == t.nb[1] * t.ne[1] &&
               t.nb[3] == t.nb[2] * t.ne[2];
    }
    // ROPE whose only reader is a type cast (CPY of its f32 result, possibly
    // through a RESHAPE, into a new contiguous f32 / f16 tensor): the rope
    // writes the cast's destination itself, in its own shape. The values are
    // the same: the rope's f32 result rounded once to the destination type.
    void fuse_rope_cast(std::vector<Dispatch> &d) {
        std::vector<char> gone(d.size(), 0);
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &r = d[i];
            if (!(r.kind == D_CORE && r.core_kind == TLH_CORE_ROPE) || r.op.x[9]) continue;
            const int32_t rn = node_of(r);
            if (readers_[rn] != 1) continue;
            int32_t v = reader_[rn], from = rn;
            if (v >= 0 && strcmp(g_.t[v].op, "RESHAPE") == 0 && readers_[v] == 1) from = v, v = reader_[v];
            if (v < 0 || strcmp(g_.t[v].op, "CPY") != 0 || g_.t[v].src[0] != from) continue;
            size_t j = i + 1;
            while (j < d.size() && !(d[j].kind == D_CORE && node_of(d[j]) == v)) ++j;
            if (j == d.size()) continue;
            const Dispatch &w = d[j];
            const tlh_tensor &y = r.op.t[4], &c = w.op.t[4];
            bool ok = y.ty == TLH_TYPE_F32 && contiguous(y) && contiguous(c) &&
                      y.ne[0] * y.ne[1] * y.ne[2] * y.ne[3] == c.ne[0] * c.ne[1] * c.ne[2] * c.ne[3];
            for (size_t k = i + 1; k < j && ok; ++k) {
                std::vector<Place> rd, wr;
                places(d[k], rd, wr);
                for (const Place &p : rd) ok = ok && !same_root(p, w.dst);
                for (const Place &p : wr) ok = ok && !same_root(p, w.dst);
            }
            if (!ok) continue;
            tlh_tensor out = y;  // the rope's shape, the cast's type and bytes
            out.ty = c.ty;
            out.nb[0] = c.nb[0];
            for (int k = 1; k < 4; ++k) out.nb[k] = out.nb[k - 1] * out.ne[k - 1];
            r.op.t[4] = out;
            r.dst = w.dst;
            r.pos_last = std::max(r.pos_last, w.pos_last);
            gone[j] = 1;
        }
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i)
            if (!gone[i]) out.push_back(d[i]);
        d.swap(out);
    }

    // A cache write whose key or value is a cast (CPY) of a contiguous f32
    // tensor read by nothing else: the write reads the f32 source and rounds it
    // to f16 itself (the same rounding the cast does).
    void fuse_cache_write_cast(std::vector<Dispatch> &d) {
        std::vector<char> gone(d.size(), 0);
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &w = d[i];
            if (w.kind != D_PAGED_WRITE) continue;
            const int32_t wn = node_of(w);  // (w.pos moves to the first fused node below)
            for (int s = 0; s < 2; ++s) {
                const int32_t cn = g_.t[wn].src[s];
                if (cn < 0 || strcmp(g_.t[cn].op, "CPY") != 0 || readers_[cn] != 1) continue;
                size_t j = 0;
                while (j < i && !(d[j].kind == D_CORE && !gone[j] && node_of(d[j]) == cn)) ++j;
                if (j == i) continue;
                const Dispatch &c = d[j];
                const tlh_tensor &a = c.op.t[0], &b = c.op.t[4];
                bool ok = c.core_kind == TLH_CORE_CPY && a.ty == TLH_TYPE_F32 && b.ty == TLH_TYPE_F16 &&
                          contiguous(a) && contiguous(b) &&
                          a.ne[0] * a.ne[1] * a.ne[2] * a.ne[3] == b.ne[0] * b.ne[1] * b.ne[2] * b.ne[3];
                for (size_t k = j + 1; k < i && ok; ++k) {  // nothing in between writes the f32 source
                    std::vector<Place> rd, wr;
                    places(d[k], rd, wr);
                    for (const Place &p : wr) ok = ok && !same_root(p, c.src[0]);
                }
                if (!ok) continue;
                w.src[s] = c.src[0];
                w.pw_f32[s] = 1;
                w.pos = std::min(w.pos, c.pos);
                gone[j] = 1;
            }
        }
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i)
            if (!gone[i]) out.push_back(d[i]);
        d.swap(out);
    }

    // paged attention whose only reader is a cast of its f16 result to a
    // contiguous f32 tensor (possibly through a RESHAPE): the attention's
    // merge launch writes the widened values there.
    void fuse_paged_cast(std::vector<Dispatch> &d) {
        std::vector<char> gone(d.size(), 0);
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &r = d[i];
            if (r.kind != D_PAGED_ATTN) continue;
            const int32_t rn = node_of(r);
            if (readers_[rn] != 1) continue;
            int32_t v = reader_[rn], from = rn;
            if (v >= 0 && strcmp(g_.t[v].op, "RESHAPE") == 0 && readers_[v] == 1) from = v, v = reader_[v];
            if (v < 0 || strcmp(g_.t[v].op, "CPY") != 0 || g_.t[v].src[0] != from) continue;
            size_t j = i + 1;
            while (j < d.size() && !(d[j].kind == D_CORE && node_of(d[j]) == v)) ++j;
            if (j == d.size()) continue;
            const Dispatch &w = d[j];
            const tlh_tensor &c = w.op.t[4];
            bool ok = c.ty == TLH_TYPE_F32 && contiguous(c) && contiguous(r.op.t[4]) &&
                      c.ne[0] * c.ne[1] * c.ne[2] * c.ne[3] ==
                          r.op.t[4].ne[0] * r.op.t[4].ne[1] * r.op.t[4].ne[2] * r.op.t[4].ne[3];
            for (size_t k = i + 1; k < j && ok; ++k) {
                std::vector<Place> rd, wr;
                places(d[k], rd, wr);
                for (const Place &p : rd) ok = ok && !same_root(p, w.dst);
                for (const Place &p : wr) ok = ok && !same_root(p, w.dst);
            }
            if (!ok) continue;
            r.pa_f32 = 1;
            r.dst = w.dst;
            r.pos_last = std::max(r.pos_last, w.pos_last);
            gone[j] = 1;
        }
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i)
            if (!gone[i]) out.push_back(d[i]);
        d.swap(out);
    }

    void fuse_rope_rows(std::vector<Dispatch> &d) {
        std::vector<char> gone(d.size(), 0);
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &r = d[i];
            if (!(r.kind == D_CORE && r.core_kind == TLH_CORE_ROPE)) continue;
            const int32_t rn = node_of(r);
            if (readers_[rn] != 1) continue;
            const int32_t v = reader_[rn];
            if (v < 0 || strcmp(g_.t[v].op, "RESHAPE") != 0 || readers_[v] != 1) continue;
            const int32_t sr = reader_[v];
            if (sr < 0 || strcmp(g_.t[sr].op, "SET_ROWS") != 0 || g_.t[sr].src[0] != v) continue;
            size_t j = i + 1;
            while (j < d.size() && !(d[j].kind == D_CORE && node_of(d[j]) == sr)) ++j;
            if (j == d.size()) continue;
            const Dispatch &w = d[j];
            const tlh_tensor &x = r.op.t[0], &y = r.op.t[4], &cache = w.op.t[4], &ix = w.op.t[1];
            bool ok = x.ne[3] == 1 && same_ne(x, y) && y.nb[0] == (y.ty == TLH_TYPE_F32 ? 4 : 2) &&
                      y.nb[1] == y.nb[0] * y.ne[0] && y.nb[2] == y.nb[1] * y.ne[1] &&
                      w.op.t[0].ne[0] == y.ne[0] * y.ne[1] && w.op.t[0].ne[1] == y.ne[2] && w.op.t[0].ne[2] == 1 &&
                      w.op.t[0].ne[3] == 1 && ix.ne[0] == y.ne[2] && cache.ne[0] == y.ne[0] * y.ne[1] &&
                      cache.nb[0] == (cache.ty == TLH_TYPE_F32 ? 4 : 2) && cache.ne[2] == 1 && cache.ne[3] == 1;
            for (size_t k = i + 1; k < j && ok; ++k) {
                std::vector<Place> rd, wr;
                places(d[k], rd, wr);
                for (const Place &p : rd) ok = ok && !same_root(p, w.dst);
                for (const Place &p : wr) ok = ok && !same_root(p, w.dst);
            }
            if (!ok) continue;
            r.op.t[3] = ix;
            r.op.t[4] = cache;
            r.op.x[9] = 1;
            r.src[3] = w.src[1];
            r.dst = w.dst;
            r.pos_last = std::max(r.pos_last, w.pos_last);
            gone[j] = 1;
        }
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i)
            if (!gone[i]) out.push_back(d[i]);
        d.swap(out);
    }

    // The stores of a single-column GEMV over Q / K / V (D_MULTI_GEMV or a
    // norm-fused D_GEMV_PRO, K <= 4096) take in the dispatches that alone read
    // its member outputs, so that the projection and the cache writes of a
    // decode step are one launch:
    //  * a ROPE in mode 0 of a member (one token), written as f32 / f16 rows
    //    or into the rows of a cache (a fused SET_ROWS);
    //  * a SET_ROWS of a member (one row) into a cache;
    //  * a one-token paged cache write whose key (a member, or the f16 result
    //    of a ROPE of one) and value (a member read as f32) both come from
    //    the GEMV.
    // The member's f32 output is then not written. An absorbed dispatch moves
    // up to the GEMV's position, so nothing between may read what it writes
    // or write what it reads.
    // batched: the same for the merged compute of a few-column projection
    // (D_MM_COMPUTE_MULTI, 3..16 columns = tokens, K <= 4096, q4_K / q5_K /
    // q6_K: the int8-MFMA kernel's store epilogue, token n in column n), for
    // the rotated / cast outputs and paged K / V writes (not cache rows); and
    // for a prefill's (more columns, q4_K / q5_K) when the merged GEMM splits
    // K, through its reduce launch.
    void fuse_gemv_epilogue(std::vector<Dispatch> &d, bool batched) {
        count_readers();
        std::vector<char> gone(d.size(), 0);
        auto kept = [&](int32_t id) { return std::find(g_.keep.begin(), g_.keep.end(), id) != g_.keep.end(); };
        auto readers_after = [&](size_t i, const Place &p) {
            std::vector<size_t> who;
            std::vector<Place> rd, wr;
            for (size_t j = i + 1; j < d.size(); ++j) {
                if (gone[j]) continue;
                places(d[j], rd, wr);
                for (const Place &r : rd)
                    if (same_root(r, p)) {
                        who.push_back(j);
                        break;
                    }
            }
            return who;
        };
        auto is_core = [](const Dispatch &x, int kind) { return x.kind == D_CORE && x.core_kind == kind; };
        auto elems = [](const tlh_tensor &t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; };
        auto idx_ty = [](const tlh_tensor &t) { return t.ty == TLH_TYPE_I32 || t.ty == 27 /* i64 */; };
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &f = d[i];
            if (gone[i]) continue;
            if (batched ? !(f.kind == D_MM_COMPUTE_MULTI && !f.has_epi)
                        : !(f.kind == D_MULTI_GEMV || (f.kind == D_GEMV_PRO && !f.has_glu && !f.has_epi)))
                continue;
            const tlh_tensor &b = f.mop[0].t[1];
            const int wty = f.mop[0].t[0].ty;
            bool many = false;  // a prefill's merged GEMM: its reduce stores (second paged stores allowed)
            if (batched) {
                // 3..16 columns: the few-column kernel's stores; more (a
                // prefill): the reduce of a q4_K / q5_K GEMM that splits K
                int64_t rows = 0;
                for (int k = 0; k < f.nmem; ++k) rows += f.mop[k].t[0].ne[1];
                const bool few = b.ne[1] >= 3 && b.ne[1] <= 16 &&
                                 (wty == TLH_TYPE_Q4_K || wty == TLH_TYPE_Q5_K || wty == TLH_TYPE_Q6_K);
                many = b.ne[1] > 16 && (wty == TLH_TYPE_Q4_K || wty == TLH_TYPE_Q5_K) &&
                       gemm_ksplit(wty, rows, b.ne[1], b.ne[0], 1) > 1;
                if (!few && !many) continue;
            }
            const int64_t T = batched ? b.ne[1] : 1;  // tokens = columns
            if (b.ne[0] > 4096 || b.ne[1] != T || b.ne[2] != 1 || b.ne[3] != 1) continue;
            GemvEpi e;
            Place edst[3], eidx[3], epos, eff, edst2[3];
            std::vector<size_t> take[3];  // absorbed dispatch indices per member
            const tlh_op *rope = nullptr;  // the first rotation's op (parameters shared)
            Place rpos, rff;
            int paged_w = -1;             // index of the absorbed paged write
            int paged_have = 0;           // 1: key member found, 2: value member found
            // many columns: an f16 result `out` (rotated keys, cast values)
            // that the attention reads as rows and one paged write of these
            // tokens also reads (side 0 key, 1 value): that write becomes a
            // second store of the segment
            auto dual_write = [&](size_t j, const Place &out, int side) -> int {
                if (!many || out.buf != B_ARENA || kept(out.index)) return -1;
                const std::vector<size_t> w2 = readers_after(j, out);
                int found = -1;
                for (size_t q : w2)
                    if (d[q].kind == D_PAGED_WRITE && d[q].pw[0] == T && !d[q].pw_f32[side] &&
                        same_place(d[q].src[side], out) && !same_place(d[q].src[side ^ 1], out)) {
                        if (found >= 0) return -1;
                        found = (int)q;
                    }
                if (found < 0 || w2.size() < 2 || (paged_w >= 0 && paged_w != found)) return -1;
                return found;
            };
            int dual_w[3] = {-1, -1, -1};  // per member: the paged write taken as its second store
            for (int k = 0; k < f.nmem; ++k) {
                const Place P = f.mdst[k];
                const int64_t M = f.mop[k].t[0].ne[1];
                const tlh_tensor &y = f.mop[k].t[4];
                if (P.buf != B_ARENA || P.off != 0 || kept(P.index) || !contiguous(y) || y.ty != TLH_TYPE_F32)
                    continue;
                const std::vector<size_t> who = readers_after(i, P);
                if (who.size() != 1) continue;
                const size_t j = who[0];
                const Dispatch &c = d[j];
                if (c.scratch_bytes != 0) continue;
                if (is_core(c, TLH_CORE_ROPE) && same_place(c.src[0], P)) {
                    const tlh_tensor &x = c.op.t[0], &o = c.op.t[4];
                    bool ok = c.op.x[1] == 0 && x.ty == TLH_TYPE_F32 && contiguous(x) && x.ne[2] == T &&
                              x.ne[3] == 1 && x.ne[0] * x.ne[1] == M && c.op.t[1].ne[0] >= T &&
                              c.op.t[1].ty == TLH_TYPE_I32 && !(batched && c.op.x[9]);
                    if (ok && rope)
                        ok = memcmp(rope->x, c.op.x, 9 * sizeof c.op.x[0]) == 0 && rope->t[0].ne[0] == x.ne[0] &&
                             same_place(rpos, c.src[1]) && same_place(rff, c.src[2]);
                    if (!ok) continue;
                    int lay = EPI_CONTIG;
                    std::vector<size_t> t = {j};
                    if (c.op.x[9]) {  // into cache rows
                        if (!idx_ty(c.op.t[3]) || o.ne[0] != M || o.nb[0] != (o.ty == TLH_TYPE_F16 ? 2 : 4)) continue;
                        lay = EPI_CACHE_ROW;
                        eidx[k] = c.src[3];
                        e.idx_i64[k] = c.op.t[3].ty != TLH_TYPE_I32;
                        e.rows[k] = o.ne[1];
                        e.row_nb[k] = o.nb[1];
                    } else {
                        if (!contiguous(o) || elems(o) != M * T) continue;
                        // a rotated key that only a paged write of these tokens reads
                        const std::vector<size_t> w2 = readers_after(j, c.dst);
                        if (o.ty == TLH_TYPE_F16 && w2.size() == 1 && d[w2[0]].kind == D_PAGED_WRITE &&
                            d[w2[0]].pw[0] == T && !d[w2[0]].pw_f32[0] && same_place(d[w2[0]].src[0], c.dst) &&
                            c.dst.buf == B_ARENA && !kept(c.dst.index) && (paged_w < 0 || paged_w == (int)w2[0])) {
                            lay = EPI_PAGED_KEY;
                            paged_w = (int)w2[0];
                            paged_have |= 1;
                            t.push_back(w2[0]);
                        } else if (o.ty == TLH_TYPE_F16) {
                            const int q = dual_write(j, c.dst, 0);
                            if (q >= 0) {
                                e.dual[k] = EPI_PAGED_KEY;
                                dual_w[k] = q;
                                paged_w = q;
                                paged_have |= 1;
                                t.push_back((size_t)q);
                            }
                        }
                    }
                    e.layout[k] = lay;
                    e.rope[k] = 1;
                    e.f16[k] = lay == EPI_PAGED_KEY || o.ty == TLH_TYPE_F16;
                    if (lay != EPI_PAGED_KEY) edst[k] = c.dst;
                    if (!rope) rope = &c.op, rpos = c.src[1], rff = c.src[2];
                    take[k] = t;
                } else if (batched && is_core(c, TLH_CORE_CPY) && same_place(c.src[0], P)) {
                    // an f32 -> f16 cast of the member (a prefill's values, also
                    // read as rows by the attention): contiguous f16 rows
                    const tlh_tensor &x = c.op.t[0], &o = c.op.t[4];
                    if (!(x.ty == TLH_TYPE_F32 && o.ty == TLH_TYPE_F16 && contiguous(x) && contiguous(o) &&
                          elems(x) == M * T && elems(o) == M * T))
                        continue;
                    std::vector<size_t> t = {j};
                    e.layout[k] = EPI_CONTIG;
                    e.f16[k] = 1;
                    edst[k] = c.dst;
                    const int q = dual_write(j, c.dst, 1);
                    if (q >= 0) {
                        e.dual[k] = EPI_PAGED_VALUE;
                        dual_w[k] = q;
                        paged_w = q;
                        paged_have |= 2;
                        t.push_back((size_t)q);
                    }
                    take[k] = t;
                } else if (!batched && is_core(c, TLH_CORE_SET_ROWS) && same_place(c.src[0], P)) {
                    const tlh_tensor &x = c.op.t[0], &o = c.op.t[4];
                    if (!(x.ne[0] == M && x.ne[1] == 1 && x.ne[2] == 1 && x.ne[3] == 1 && idx_ty(c.op.t[1]) &&
                          o.ne[0] == M && (o.ty == TLH_TYPE_F16 || o.ty == TLH_TYPE_F32) &&
                          o.nb[0] == (o.ty == TLH_TYPE_F16 ? 2 : 4)))
                        continue;
                    e.layout[k] = EPI_CACHE_ROW;
                    e.f16[k] = o.ty == TLH_TYPE_F16;
                    edst[k] = c.dst;
                    eidx[k] = c.src[1];
                    e.idx_i64[k] = c.op.t[1].ty != TLH_TYPE_I32;
                    e.rows[k] = o.ne[1];
                    e.row_nb[k] = o.nb[1];
                    take[k] = {j};
                } else if (c.kind == D_PAGED_WRITE && c.pw[0] == T && (paged_w < 0 || paged_w == (int)j)) {
                    int side = -1;
                    if (same_place(c.src[1], P) && c.pw_f32[1]) side = 1;
                    else if (same_place(c.src[0], P) && c.pw_f32[0]) side = 0;
                    if (side < 0) continue;
                    e.layout[k] = side ? EPI_PAGED_VALUE : EPI_PAGED_KEY;
                    e.f16[k] = 1;
                    paged_w = (int)j;
                    paged_have |= side ? 2 : 1;
                    take[k] = {j};
                }
            }
            // a paged write goes only with both of its operands
            if (paged_w >= 0) {
                const Dispatch &w = d[paged_w];
                bool ok = paged_have == 3;
                for (int k = 0; k < f.nmem && ok; ++k) {
                    const int pl = e.dual[k] ? e.dual[k] : e.layout[k];
                    if (pl == EPI_PAGED_KEY || pl == EPI_PAGED_VALUE) {
                        ok = f.mop[k].t[0].ne[1] == (int64_t)w.pw[1] * w.pw[2];
                        (e.dual[k] ? edst2[k] : edst[k]) = pl == EPI_PAGED_KEY ? w.src[2] : w.src[3];
                        eidx[k] = w.src[4];
                        e.idx_i64[k] = 1;
                        e.rows[k] = w.pw_blocks * w.pw[3];
                    }
                }
                if (!ok)
                    for (int k = 0; k < f.nmem; ++k) {
                        if (e.dual[k]) {  // keep the contiguous rows, leave the paged write out
                            e.dual[k] = 0;
                            take[k].erase(std::remove(take[k].begin(), take[k].end(), (size_t)dual_w[k]), take[k].end());
                            eidx[k] = Place{}, e.idx_i64[k] = 0, e.rows[k] = 0;
                        } else if (e.layout[k] == EPI_PAGED_KEY || e.layout[k] == EPI_PAGED_VALUE) {
                            e.layout[k] = EPI_F32, e.rope[k] = 0, e.f16[k] = 0;
                            take[k].clear();
                        }
                    }
                e.kvh = w.pw[1], e.hs = w.pw[2], e.bs = w.pw[3];
            }
            // nothing between the GEMV and an absorbed dispatch touches what
            // the dispatch writes or writes what it reads
            std::vector<size_t> all;
            for (int k = 0; k < f.nmem; ++k) all.insert(all.end(), take[k].begin(), take[k].end());
            std::sort(all.begin(), all.end());
            all.erase(std::unique(all.begin(), all.end()), all.end());
            if (all.empty()) continue;
            bool ok = true;
            std::vector<Place> rd, wr, r2, w2;
            for (size_t j : all) {
                places(d[j], rd, wr);
                for (size_t t = i + 1; t < j && ok; ++t) {
                    if (gone[t] || std::binary_search(all.begin(), all.end(), t)) continue;
                    places(d[t], r2, w2);
                    for (const Place &p : w2)
                        for (const Place &q : rd) ok = ok && !same_root(p, q);
                    for (const Place &p : wr) {
                        for (const Place &q : r2) ok = ok && !same_root(p, q);
                        for (const Place &q : w2) ok = ok && !same_root(p, q);
                    }
                }
            }
            if (!ok) continue;
            if (rope) {
                e.ne0 = rope->t[0].ne[0];
                e.rp.n_dims = (int)rope->x[0];
                e.rp.mode = (int)rope->x[1];
                e.rp.freq_scale = __builtin_bit_cast(float, (int32_t)rope->x[2]);
                e.rp.ext_factor = __builtin_bit_cast(float, (int32_t)rope->x[3]);
                e.rp.attn_factor = __builtin_bit_cast(float, (int32_t)rope->x[4]);
                e.rp.theta_scale = __builtin_bit_cast(float, (int32_t)rope->x[5]);
                e.rp.corr0 = __builtin_bit_cast(float, (int32_t)rope->x[6]);
                e.rp.corr1 = __builtin_bit_cast(float, (int32_t)rope->x[7]);
                epos = rpos;
                if (rope->x[8]) eff = rff;
                if (batched && T <= 16) {  // one (cos, sin) table per positions and parameters, the first launch writes it
                    std::vector<int64_t> key = {rpos.buf, rpos.index, rpos.off, rff.buf, rff.index, rff.off, e.ne0, T};
                    for (int q = 0; q < 9; ++q) key.push_back(rope->x[q]);
                    auto it = rt_tables_.find(key);
                    const int64_t pairs = std::min<int64_t>(e.rp.n_dims, e.ne0) / 2;
                    if (it == rt_tables_.end()) {
                        f.rt_off = rt_bytes_;
                        rt_tables_[key] = rt_bytes_;
                        rt_bytes_ += align_up(T * pairs * 8);
                        e.rt_mode = 1;
                    } else {
                        f.rt_off = it->second;
                        e.rt_mode = 2;
                    }
                }
            }
            e.on = 1;
            Dispatch g = f;
            if (!batched) g.kind = D_GEMV_PRO;
            g.has_epi = 1;
            g.epi = e;
            for (int k = 0; k < 3; ++k) g.edst[k] = edst[k], g.eidx[k] = eidx[k], g.edst2[k] = edst2[k];
            g.epos = epos;
            g.eff = eff;
            for (size_t j : all) {
                g.absorbed.push_back(d[j]);
                g.pos_last = std::max(g.pos_last, d[j].pos_last);
                gone[j] = 1;
            }
            d[i] = g;
        }
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i)
            if (!gone[i]) out.push_back(d[i]);
        d.swap(out);
    }

    // consecutive independent element-wise dispatches -> one launch (up to 4)
    void group_elementwise(std::vector<Dispatch> &d) {
        // (a GLU that also quantizes for a MUL_MAT keeps its own launch)
        auto ew = [](const Dispatch &x) { return x.kind == D_CORE && core_multi_kind(x.core_kind) && !x.nq_type; };
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size();) {
            size_t j = i + 1;
            if (ew(d[i]))
                while (j < d.size() && j - i < 4 && ew(d[j])) {
                    bool ind = true;
                    for (size_t k = i; k < j && ind; ++k) ind = independent(d[k], d[j]);
                    if (!ind) break;
                    ++j;
                }
            if (j - i < 2) {
                out.push_back(d[i++]);
                continue;
            }
            Dispatch f = d[i];
            f.kind = D_CORE_MULTI;
            f.nsub = (int)(j - i);
            for (size_t k = i; k < j; ++k) {
                const int q = (int)(k - i);
                f.sub_kind[q] = d[k].core_kind;
                f.sop[q] = d[k].op;
                for (int m = 0; m < 4; ++m) f.ssrc[q][m] = d[k].src[m];
                f.sdst[q] = d[k].dst;
                f.pos_last = std::max(f.pos_last, d[k].pos_last);
            }
            for (int m = 0; m < 4; ++m) f.src[m] = Place();
            f.dst = Place();
            out.push_back(f);
            i = j;
        }
        d.swap(out);
    }

    // MUL_MAT nodes with more than two activation columns that read the same
    // bytes with the same weight type (so the same q8 layout) share one
    // quantization: the first of them writes the blocks into a scratch block
    // that lives until the last has run. A node that writes into the
    // activation's storage in between ends the group.
    void group_mul_mats(std::vector<Dispatch> &d) {
        using Key = std::tuple<int, int32_t, int64_t, int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                               int64_t, int64_t>;
        std::map<Key, int> open;  // key -> index of the group's first dispatch
        std::vector<Dispatch> out;
        out.reserve(d.size() * 2);
        std::vector<int> leader(d.size(), -1);
        for (size_t i = 0; i < d.size(); ++i) {
            const Dispatch &x = d[i];
            // a write into storage an open group reads closes that group
            for (auto it = open.begin(); it != open.end();) {
                const Place &s1 = d[it->second].src[1];
                if (x.dst.buf == s1.buf && x.dst.index == s1.index) it = open.erase(it);
                else ++it;
            }
            if (x.kind != D_MUL_MAT || x.op.t[1].ne[1] <= 2) continue;
            const tlh_tensor &b = x.op.t[1];
            const Key k{x.src[1].buf, x.src[1].index, x.src[1].off, x.op.t[0].ty, b.ty, b.ne[0], b.ne[1], b.ne[2],
                        b.ne[3], b.nb[1], b.nb[2], b.nb[3], x.op.t[0].ne[2]};
            auto it = open.find(k);
            if (it == open.end()) {
                open[k] = (int)i;
                leader[i] = (int)i;
            } else {
                leader[i] = it->second;
            }
        }
        // members per leader
        std::map<int, std::vector<int>> members;
        for (size_t i = 0; i < d.size(); ++i)
            if (leader[i] >= 0) members[leader[i]].push_back((int)i);
        group_of_.assign(d.size(), -1);
        groups_.clear();
        for (auto &[l, m] : members) {
            if (m.size() < 2) continue;
            Group gr;
            gr.first = d[m.front()].pos;
            gr.last = d[m.back()].pos;
            for (int i : m) gr.bytes = std::max(gr.bytes, d[i].scratch_bytes);
            for (int i : m) group_of_[i] = (int)groups_.size();
            gr.leader = l;
            groups_.push_back(gr);
        }
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch x = d[i];
            const int gi = group_of_[i];
            if (gi < 0) {
                out.push_back(x);
                continue;
            }
            x.scratch_bytes = groups_[gi].bytes;
            x.block = -2 - gi;  // resolved to the group's block by plan()
            if (groups_[gi].leader == (int)i) {
                Dispatch q = x;
                q.kind = D_MM_QUANTIZE;
                out.push_back(q);
            }
            x.kind = D_MM_COMPUTE;
            out.push_back(x);
        }
        d.swap(out);
    }

    // Compute halves of one quantization group become one launch over their
    // rows, at the first one's place: 3..16 columns with K <= 4096 the
    // few-column MFMA kernel, more columns of q4_K / q5_K weights the GEMM
    // (whose K-chunk partials over all the rows can outgrow the members'
    // scratch: the group's block grows to fit). A later member moves up only if nothing in between reads or
    // writes its destination (its weights and the group's activation scratch
    // are written by nobody else).
    void merge_mm_computes(std::vector<Dispatch> &d) {
        std::vector<char> taken(d.size(), 0);
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i) {
            if (taken[i]) continue;
            if (d[i].kind != D_MM_COMPUTE) {
                out.push_back(d[i]);
                continue;
            }
            std::vector<size_t> mem{i};
            const tlh_op *ops[3] = {&d[i].op, nullptr, nullptr};
            for (size_t j = i + 1; j < d.size() && j < i + 24 && mem.size() < 3; ++j) {
                if (taken[j] || d[j].kind != D_MM_COMPUTE || d[j].block != d[i].block) continue;
                bool ok = true;
                for (size_t k = i + 1; k < j && ok; ++k) {
                    if (taken[k]) continue;
                    std::vector<Place> rd, wr;
                    places(d[k], rd, wr);
                    for (const Place &p : rd) ok = ok && !same_root(p, d[j].dst);
                    for (const Place &p : wr) ok = ok && !same_root(p, d[j].dst);
                }
                ops[mem.size()] = &d[j].op;
                if (ok && mul_mat_compute_multi_ok(ops, (int)mem.size() + 1)) mem.push_back(j);
            }
            if (mem.size() < 2) {
                out.push_back(d[i]);
                continue;
            }
            Dispatch f = d[i];
            f.kind = D_MM_COMPUTE_MULTI;
            f.nmem = (int)mem.size();
            for (size_t k = 0; k < mem.size(); ++k) {
                const Dispatch &y = d[mem[k]];
                f.mop[k] = y.op;
                f.mpos[k] = y.pos;
                f.mw[k] = y.src[0];
                f.mdst[k] = y.dst;
                f.pos_last = std::max(f.pos_last, y.pos_last);
                taken[mem[k]] = 1;
            }
            const tlh_op *mops[3] = {&f.mop[0], &f.mop[1], &f.mop[2]};
            const size_t need = mul_mat_compute_multi_scratch_bytes(mops, f.nmem);
            if (need > f.scratch_bytes) {
                f.scratch_bytes = need;
                if (f.block <= -2) {
                    Group &gr = groups_[-2 - f.block];
                    gr.bytes = std::max(gr.bytes, need);
                }
            }
            out.push_back(f);
        }
        d.swap(out);
    }

    // A MUL_MAT of 3 or more columns whose activation is a GLU's output (the
    // SwiGLU before the down projection), a norm chain's output over at least
    // NQ_MIN_ROWS rows (the RMS_NORM before Q / K / V and gate / up in a
    // prefill) or the one-launch paged attention's f32 output (the output
    // projection of a batched decode step, the merge quantizing whole q8_K
    // blocks of heads): that launch also writes the quantized rows (the bytes the
    // quantize launch would write) into the MUL_MAT's scratch, and the MUL_MAT
    // keeps only its compute launch; a quantization group's leader quantize
    // goes the same way. Needs: src1 is the producer's whole output,
    // contiguous f32 rows (a multiple of the block) in the same order, and
    // nothing between the two writes that storage. The scratch then lives from
    // the producer on. (A norm chain over few rows -- a batched decode step --
    // spreads each row over its 1024-element groups, so the quantization does
    // not lengthen one workgroup's path by a whole row's.)
    static constexpr int64_t NQ_MIN_ROWS = 3;
    void fuse_act_quantize(std::vector<Dispatch> &d) {
        auto contiguous_f32 = [](const tlh_tensor &t) {
            return t.ty == TLH_TYPE_F32 && t.nb[0] == 4 && t.nb[1] == 4 * t.ne[0] && t.nb[2] == t.nb[1] * t.ne[1] &&
                   t.nb[3] == t.nb[2] * t.ne[2];
        };
        std::vector<char> gone(d.size(), 0);
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &q = d[i];
            const bool leader = q.kind == D_MM_QUANTIZE && q.block <= -2;
            const bool single = q.kind == D_MUL_MAT && q.block == -1 && q.scratch_bytes > 0;
            if (!leader && !single) continue;
            const tlh_tensor &b = q.op.t[1];
            const int wt = q.op.t[0].ty;
            if (wt == TLH_TYPE_F32 || wt == TLH_TYPE_F16 || wt == TLH_TYPE_BF16) continue;
            const int at = vec_dot_type(wt);
            const int64_t K = b.ne[0], rows = b.ne[1] * b.ne[2] * b.ne[3];
            if (!contiguous_f32(b) || rows == 0) continue;
            // the GLU that wrote src1, with nothing writing it since
            int gi = -1;
            std::vector<Place> rd, wr;
            for (int j = (int)i - 1; j >= 0; --j) {
                if (gone[j]) continue;
                const Dispatch &c = d[j];
                if (((c.kind == D_CORE && c.core_kind == TLH_CORE_GLU) || c.kind == D_NORM_CHAIN ||
                     (c.kind == D_PAGED_ATTN && c.pa_f32)) &&
                    same_place(c.dst, q.src[1])) {
                    gi = j;
                    break;
                }
                places(c, rd, wr);
                bool touches = false;
                for (const Place &p : wr) touches = touches || same_root(p, q.src[1]);
                if (touches) break;
            }
            if (gi < 0) continue;
            Dispatch &g = d[gi];
            // paged attention (one launch, f32 output): its merge quantizes the
            // heads it holds. Like the others only for 3 or more columns: below
            // that the MUL_MAT quantizes in its own launch, which costs less
            // than the merge's extra work (bs 1 decode: 1.85 -> 1.90 ms a step)
            const bool pa = g.kind == D_PAGED_ATTN;
            if (b.ne[1] < 3) continue;
            if (pa) {
                const int64_t per = (int64_t)g.pa.num_heads * g.pa.head_size;
                if (g.block != -1 || K != per || rows != g.pa.num_seqs || !contiguous_f32(b) ||
                    act_has_f16(wt, b.ne[1]) || !paged_attention_quantize_ok(g.pa, at))
                    continue;
            } else {
                const tlh_tensor &y = g.op.t[4];
                if (g.block != -1 || !contiguous_f32(y) || y.ne[0] != K ||
                    y.ne[1] * y.ne[2] * y.ne[3] != rows)
                    continue;
                if (g.kind == D_NORM_CHAIN ? rows < NQ_MIN_ROWS || !norm_chain_quantize_ok(g.op, at)
                                           : !glu_quantize_ok(g.op, at))
                    continue;
            }
            if (single) {  // a group of one: its scratch block spans GLU .. MUL_MAT
                Group gr;
                gr.first = q.pos;
                gr.last = q.pos_last;
                gr.bytes = q.scratch_bytes;
                gr.leader = (int)i;
                q.block = -2 - (int)groups_.size();
                groups_.push_back(gr);
                q.kind = D_MM_COMPUTE;
            } else {
                gone[i] = 1;
            }
            g.nq_type = at;
            g.nq_rows = rows;
            g.nq_f16 = act_has_f16(wt, b.ne[1]);
            g.nq_op = q.op;
            g.block = q.block;
            Group &gr = groups_[-2 - q.block];
            if (pa) {  // the block holds the MUL_MAT's scratch, then the attention's own
                g.pa_own = (size_t)align_up((int64_t)q.scratch_bytes);
                g.scratch_bytes = g.pa_own + g.scratch_bytes;
                gr.bytes = std::max(gr.bytes, g.scratch_bytes);
            } else {
                g.scratch_bytes = q.scratch_bytes;
            }
            gr.first = std::min<int64_t>(gr.first, g.pos);
        }
        std::vector<Dispatch> out;
        for (size_t i = 0; i < d.size(); ++i)
            if (!gone[i]) out.push_back(d[i]);
        d.swap(out);
    }

    // A K-split MUL_MAT product whose only reader is the ADD of a norm chain
    // (a layer's output or down projection at a batched decode step or a
    // prefill, then the residual ADD and the next RMS_NORM): the product leaves
    // its chunk partials in its scratch and the norm chain adds them in chunk
    // order as it reads q (the bits the chunk-sum launch would have written),
    // so that launch goes. The MUL_MAT's scratch then lives until the norm
    // chain; the MUL_MAT's own output is never written.
    void fuse_partials_into_norm(std::vector<Dispatch> &d) {
        count_readers();
        for (size_t i = 0; i < d.size(); ++i) {
            Dispatch &nc = d[i];
            if (nc.kind != D_NORM_CHAIN || nc.op.x[2] == 0 || nc.pp_disp >= 0) continue;
            const int32_t add_id = node_of(nc);
            for (int k = 0; k < 2; ++k) {
                // the producer of operand k, with nothing in between writing it
                int j = -1;
                std::vector<Place> rd, wr;
                for (int jj = (int)i - 1; jj >= 0; --jj) {
                    const Dispatch &c = d[jj];
                    if ((c.kind == D_MUL_MAT || c.kind == D_MM_COMPUTE) && same_place(c.dst, nc.src[k])) {
                        j = jj;
                        break;
                    }
                    places(c, rd, wr);
                    bool touches = false;
                    for (const Place &p : wr) touches = touches || same_root(p, nc.src[k]);
                    if (touches) break;
                }
                if (j < 0) continue;
                Dispatch &mm = d[j];
                const int32_t mm_id = node_of(mm);
                MmPartials pp;
                if (mm.keep_part || mm.scratch_bytes == 0 || readers_[mm_id] != 1 || reader_[mm_id] != add_id ||
                    !mul_mat_partials(&mm.op, pp))
                    continue;
                const tlh_tensor &y = mm.op.t[4];
                if (y.nb[0] != 4 || y.nb[1] != 4 * y.ne[0] || y.ne[0] != nc.op.t[0].ne[0] ||
                    y.ne[1] != nc.op.t[0].ne[1] * nc.op.t[0].ne[2] * nc.op.t[0].ne[3] || y.ne[2] != 1 || y.ne[3] != 1 ||
                    nc.op.t[0].ne[0] % 4 != 0)
                    continue;
                if (k == 0) {  // the partials become q: p + q is q + p, bit for bit
                    std::swap(nc.src[0], nc.src[1]);
                    std::swap(nc.op.t[0], nc.op.t[1]);
                }
                mm.keep_part = 1;
                nc.pp_disp = j;
                nc.pp_off = pp.off;
                nc.pp_chunks = pp.chunks;
                nc.pp_cstride = pp.cstride;
                // the MUL_MAT's scratch lives until the norm chain
                if (mm.block <= -2) {
                    Group &gr = groups_[-2 - mm.block];
                    gr.last = std::max<int64_t>(gr.last, nc.pos_last);
                } else {
                    Group gr;
                    gr.first = mm.pos;
                    gr.last = nc.pos_last;
                    gr.bytes = mm.scratch_bytes;
                    gr.leader = j;
                    mm.block = -2 - (int)groups_.size();
                    groups_.push_back(gr);
                }
                break;
            }
        }
    }

    std::map<std::vector<int64_t>, int64_t> rt_tables_;  // rotation table offset per key
    int64_t rt_bytes_ = 0;

    struct Group {
        int64_t first = 0, last = 0;
        size_t bytes = 0;
        int leader = -1;
    };
    std::vector<Group> groups_;
    std::vector<int> group_of_;

    // plan.rs:63-189: liveness of arena roots by node position, then first
    // fit by start position over the lowest free offset.
    void plan(Lowered &out) {
        const int64_t n = (int64_t)g_.nodes.size();
        std::vector<int64_t> first(g_.n, INT64_MAX), last(g_.n, -1);
        auto touch = [&](int32_t id, int64_t pos) {
            int64_t extra;
            const int32_t r = g_.root(id, extra);
            first[r] = std::min(first[r], pos);
            last[r] = std::max(last[r], pos);
        };
        for (int64_t pos = 0; pos < n; ++pos) {
            const int32_t id = g_.nodes[pos];
            touch(id, pos);
            for (int s = 0; s < 10; ++s)
                if (g_.t[id].src[s] >= 0) touch(g_.t[id].src[s], pos);
        }
        for (int32_t id : g_.keep) {
            int64_t extra;
            const int32_t r = g_.root(id, extra);
            if (first[r] == INT64_MAX) first[r] = n;
            last[r] = n;
        }
        // a fused dispatch reads and writes all its tensors over its whole
        // position range: none of them may share bytes with another there
        auto touch_place = [&](const Place &p, int64_t pos) {
            if (p.buf != B_ARENA) return;
            first[p.index] = std::min(first[p.index], pos);
            last[p.index] = std::max(last[p.index], pos);
        };
        for (const Dispatch &x : out.d) {
            if (x.pos_last == x.pos) continue;
            std::vector<Place> rd, wr;
            places(x, rd, wr);
            for (int64_t pos : {(int64_t)x.pos, (int64_t)x.pos_last}) {
                for (const Place &p : rd) touch_place(p, pos);
                for (const Place &p : wr) touch_place(p, pos);
            }
        }
        out.blocks.clear();
        out.arena_off.assign(g_.n, -1);
        for (int32_t id = 0; id < g_.n; ++id)
            if (g_.t[id].view_src < 0 && g_.t[id].storage == TLH_STORE_TEMP && first[id] != INT64_MAX)
                out.blocks.push_back({first[id], last[id], align_up(std::max<int64_t>(nbytes(g_.t[id]), 1)), id});
        const size_t n_tensor_blocks = out.blocks.size();
        // scratch: one block per ungrouped dispatch that asks for it, one per group
        std::vector<int> disp_block(out.d.size(), -1);
        for (size_t i = 0; i < out.d.size(); ++i) {
            Dispatch &x = out.d[i];
            if (x.block <= -2 || x.scratch_bytes == 0) continue;
            disp_block[i] = (int)out.blocks.size();
            out.blocks.push_back({x.pos, x.pos, align_up((int64_t)x.scratch_bytes), -1});
        }
        std::vector<int> group_block(groups_.size());
        for (size_t gi = 0; gi < groups_.size(); ++gi) {
            group_block[gi] = (int)out.blocks.size();
            out.blocks.push_back({groups_[gi].first, groups_[gi].last, align_up((int64_t)groups_[gi].bytes), -1});
        }
        for (size_t i = 0; i < out.d.size(); ++i) {
            Dispatch &x = out.d[i];
            if (x.block <= -2) x.block = group_block[-2 - x.block];
            else if (disp_block[i] >= 0) x.block = disp_block[i];
        }
        // order: (first, tensor blocks before scratch, index)
        std::vector<int> order(out.blocks.size());
        for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
        std::sort(order.begin(), order.end(), [&](int a, int b) {
            const bool sa = (size_t)a >= n_tensor_blocks, sb = (size_t)b >= n_tensor_blocks;
            return std::make_tuple(out.blocks[a].first, sa, a) < std::make_tuple(out.blocks[b].first, sb, b);
        });
        struct Live {
            int64_t off, size, last;
        };
        std::vector<Live> live;
        int64_t arena = 0;
        for (int bi : order) {
            Block &b = out.blocks[bi];
            live.erase(std::remove_if(live.begin(), live.end(), [&](const Live &l) { return l.last < b.first; }),
                       live.end());
            std::sort(live.begin(), live.end(), [](const Live &x, const Live &y) { return x.off < y.off; });
            int64_t off = 0;
            for (const Live &l : live) {
                if (l.off >= off + b.size) break;
                off = std::max(off, l.off + l.size);
            }
            b.off = off;
            live.push_back({off, b.size, b.last});
            arena = std::max(arena, off + b.size);
        }
        for (size_t i = 0; i < n_tensor_blocks; ++i) out.arena_off[out.blocks[i].tensor] = out.blocks[i].off;
        out.node_scratch.assign(n, -1);
        for (const Dispatch &x : out.d) {
            if (x.block >= 0 && !x.nq_type) out.node_scratch[x.pos] = out.blocks[x.block].off;
            if (x.block >= 0 && x.kind == D_MM_COMPUTE_MULTI)
                for (int k = 0; k < x.nmem; ++k) out.node_scratch[x.mpos[k]] = out.blocks[x.block].off;
        }
        out.arena = arena;
        out.rt_bytes = rt_bytes_;
    }
};

tlh_status read_graph(const tlh_ir_tensor *tensors, int32_t n_tensors, const int32_t *nodes, int32_t n_nodes,
                      const int32_t *keep, int32_t n_keep, Graph &g) {
    if (!tensors || n_tensors < 0 || n_nodes < 0 || n_keep < 0 || (n_nodes && !nodes) || (n_keep && !keep))
        return set_error(TLH_INVALID, "program: null or negative graph arrays");
    g.t = tensors;
    g.n = n_tensors;
    g.nodes.assign(nodes, nodes + n_nodes);
    g.keep.assign(keep, keep + n_keep);
    for (int32_t id = 0; id < n_tensors; ++id) {
        const tlh_ir_tensor &t = tensors[id];
        if (memchr(t.op, 0, sizeof t.op) == nullptr) return set_error(TLH_INVALID, "tensor %d: op name not terminated", id);
        for (int s = 0; s < 10; ++s)
            if (t.src[s] < -1 || t.src[s] >= n_tensors) return set_error(TLH_INVALID, "tensor %d: source %d out of range", id, s);
        if (t.view_src >= n_tensors || t.view_src < -1 || (t.view_src >= 0 && tensors[t.view_src].view_src >= 0))
            return set_error(TLH_INVALID, "tensor %d: view_src must be a root tensor", id);
        if (t.view_src < 0 && (t.storage < TLH_STORE_TEMP || t.storage > TLH_STORE_INPUT))
            return set_error(TLH_INVALID, "tensor %d: storage %d", id, t.storage);
        for (int i = 0; i < 4; ++i)
            if (t.ne[i] < 0 || t.nb[i] < 0) return set_error(TLH_INVALID, "tensor %d: negative extent or stride", id);
        int64_t blck, size;
        if (!type_traits(t.ty, blck, size)) return set_error(TLH_UNSUPPORTED, "tensor %d: ggml type %d", id, t.ty);
    }
    for (int32_t id : g.nodes)
        if (id < 0 || id >= n_tensors) return set_error(TLH_INVALID, "program: node id %d out of range", id);
    for (int32_t id : g.keep)
        if (id < 0 || id >= n_tensors) return set_error(TLH_INVALID, "program: kept id %d out of range", id);
    return TLH_OK;
}

}  // namespace
}  // namespace tlh

using namespace tlh;

struct tlh_program {
    std::vector<tlh_ir_tensor> tensors;
    Lowered low;
    std::vector<const void *> weights;
    std::vector<int64_t> state_offsets;
    std::vector<std::pair<int64_t, int64_t>> inputs;  // (io offset, bytes) per input index
    int64_t io_bytes = 0;
    char *arena = nullptr, *io = nullptr;
    // zeroed counters the one-launch paged attention leaves zeroed (its
    // dispatches run in stream order, so they share them)
    unsigned *counters = nullptr;
    float *rtab = nullptr;  // the batched epilogues' rotation tables (low.rt_bytes)
    // per table offset: its writing launch took the epilogue (else its readers
    // compute the rotation themselves); set as the dispatches are enqueued in order
    mutable std::map<int64_t, bool> rt_ok;
    hipGraphExec_t exec = nullptr;
    void *exec_state = nullptr;
    hipStream_t exec_stream = nullptr;
    int device = 0;

    void *resolve(const Place &p, void *state) const {
        switch (p.buf) {
        case B_ARENA: return arena + low.arena_off[p.index] + p.off;
        case B_IO: return io + inputs[p.index].first + p.off;
        case B_STATE: return (char *)state + state_offsets[p.index] + p.off;
        case B_WEIGHT: return (char *)weights[p.index] + p.off;
        default: return nullptr;
        }
    }

    // The ggml op of a dispatch's first node (its label in errors, traces and profiles).
    const char *op_of(const Dispatch &x) const { return tensors[low.node_ids[x.pos]].op; }

    tlh_status enqueue(void *state, hipStream_t s) const {
        for (size_t i = 0; i < low.d.size(); ++i) {
            const tlh_status st = enqueue_one(i, state, s);
            if (st != TLH_OK) return st;
        }
        return TLH_OK;
    }

    tlh_status enqueue_one(size_t i, void *state, hipStream_t s) const {
        const Dispatch &x = low.d[i];
        const tlh_status st = launch_one(x, state, s);
        if (st != TLH_OK) {
            const int32_t id = low.node_ids[x.pos];
            const std::string msg = tlh_last_error();
            return set_error(st, "launching `%s` (tensor %d): %s", op_of(x), id, msg.c_str());
        }
        return TLH_OK;
    }

    // Every dispatch between two events on `s` (eager launches); ms[i] is the
    // GPU time of dispatch i. The events are created and destroyed here.
    tlh_status profile(void *state, hipStream_t s, float *ms) const {
        const size_t n = low.d.size();
        std::vector<hipEvent_t> ev(n + 1, nullptr);
        tlh_status st = TLH_OK;
        size_t made = 0;
        for (; made <= n && st == TLH_OK; ++made)
            if (hipEventCreate(&ev[made]) != hipSuccess) st = set_error(TLH_EXECUTION, "profile: hipEventCreate");
        if (st == TLH_OK && hipEventRecord(ev[0], s) != hipSuccess) st = set_error(TLH_EXECUTION, "profile: record");
        for (size_t i = 0; i < n && st == TLH_OK; ++i) {
            st = enqueue_one(i, state, s);
            if (st == TLH_OK && hipEventRecord(ev[i + 1], s) != hipSuccess)
                st = set_error(TLH_EXECUTION, "profile: record");
        }
        if (st == TLH_OK && hipEventSynchronize(ev[n]) != hipSuccess)
            st = set_error(TLH_EXECUTION, "profile: hipEventSynchronize: %s", hipGetErrorString(hipGetLastError()));
        for (size_t i = 0; i < n && st == TLH_OK; ++i)
            if (hipEventElapsedTime(&ms[i], ev[i], ev[i + 1]) != hipSuccess)
                st = set_error(TLH_EXECUTION, "profile: hipEventElapsedTime");
        for (size_t i = 0; i < made && i <= n; ++i)
            if (ev[i]) (void)hipEventDestroy(ev[i]);
        return st;
    }

    tlh_status launch_one(const Dispatch &x, void *state, hipStream_t s) const {
        {
            void *src[NSRC];
            for (int i = 0; i < NSRC; ++i) src[i] = resolve(x.src[i], state);
            void *dst = resolve(x.dst, state);
            void *scratch = x.block >= 0 ? arena + low.blocks[x.block].off : nullptr;
            tlh_status st;
            switch (x.kind) {
            case D_MUL_MAT:
                st = x.keep_part ? mul_mat_compute_keep(&x.op, src[0], src[1], scratch, x.scratch_bytes, dst, s)
                                 : tlh_mul_mat(&x.op, src[0], src[1], dst, scratch, x.scratch_bytes, s);
                break;
            case D_MM_QUANTIZE: st = tlh_mul_mat_quantize(&x.op, src[1], scratch, x.scratch_bytes, s); break;
            case D_MM_COMPUTE:
                st = x.keep_part ? mul_mat_compute_keep(&x.op, src[0], nullptr, scratch, x.scratch_bytes, dst, s)
                                 : tlh_mul_mat_compute(&x.op, src[0], scratch, x.scratch_bytes, dst, s);
                break;
            case D_FLASH_ATTN:
                st = tlh_flash_attn_ext(&x.op, src[0], src[1], src[2], src[3], dst, scratch, x.scratch_bytes, s);
                break;
            case D_NORM_CHAIN: {
                ActQuantOut qo;
                if (x.nq_type) {
                    qo.out = scratch;
                    qo.type = x.nq_type;
                    qo.rows = x.nq_rows;
                    qo.f16 = x.nq_f16 != 0;
                }
                NormPartials qp;
                if (x.pp_disp >= 0) {
                    const Dispatch &mm = low.d[x.pp_disp];
                    qp.part = (const float *)(arena + low.blocks[mm.block].off + x.pp_off);
                    qp.chunks = x.pp_chunks;
                    qp.cstride = x.pp_cstride;
                }
                st = launch_norm_chain(x.op, src[0], src[1], src[2], src[3], dst, s, x.nq_type ? &qo : nullptr,
                                       x.pp_disp >= 0 ? &qp : nullptr);
                break;
            }
            case D_PAGED_ATTN: {
                tlh_paged_attention_args a = x.pa;
                a.out = dst;
                a.q = src[0];
                a.k_cache = src[1];
                a.v_cache = src[2];
                a.block_tables = (const int32_t *)src[3];
                a.context_lens = (const int32_t *)src[4];
                if (x.pa_f32) a.out = nullptr;
                if (a.num_seqs == 0) break;
                if (x.nq_type) {  // and the next MUL_MAT's quantized activation, at the block's start
                    ActQuantOut qo;
                    qo.out = scratch;
                    qo.type = x.nq_type;
                    qo.rows = x.nq_rows;
                    qo.f16 = x.nq_f16 != 0;
                    char *own = (char *)scratch + x.pa_own;
                    st = launch_paged_attention(a, own, x.scratch_bytes - x.pa_own, s, (float *)dst, counters, &qo);
                    if (st == TLH_UNSUPPORTED) {
                        st = launch_paged_attention(a, own, x.scratch_bytes - x.pa_own, s, (float *)dst, counters);
                        if (st == TLH_OK) st = tlh_mul_mat_quantize(&x.nq_op, dst, scratch, x.pa_own, s);
                    }
                    break;
                }
                st = launch_paged_attention(a, scratch, x.scratch_bytes, s, x.pa_f32 ? (float *)dst : nullptr,
                                            counters);
                break;
            }
            case D_MM_COMPUTE_MULTI: {
                const tlh_op *ops[3];
                const void *w[3];
                void *dsts[3];
                for (int k = 0; k < x.nmem; ++k) {
                    ops[k] = &x.mop[k];
                    w[k] = resolve(x.mw[k], state);
                    dsts[k] = resolve(x.mdst[k], state);
                }
                if (x.has_epi) {  // the absorbed rotations / casts / paged writes at the store
                    GemvEpi e = x.epi;
                    for (int k = 0; k < 3; ++k) {
                        e.dst[k] = (char *)resolve(x.edst[k], state);
                        e.idx[k] = (const char *)resolve(x.eidx[k], state);
                        e.dst2[k] = (char *)resolve(x.edst2[k], state);
                    }
                    e.pos = (const int32_t *)resolve(x.epos, state);
                    e.ff = (const float *)resolve(x.eff, state);
                    if (e.rt_mode) e.rt = (float *)((char *)rtab + x.rt_off);
                    if (e.rt_mode == 2 && !rt_ok[x.rt_off]) e.rt_mode = 0;
                    st = mul_mat_compute_multi(ops, w, dsts, x.nmem, scratch, x.scratch_bytes, s, &e);
                    if (e.rt_mode == 1) rt_ok[x.rt_off] = st == TLH_OK;
                    if (st != TLH_UNSUPPORTED) break;
                    st = mul_mat_compute_multi(ops, w, dsts, x.nmem, scratch, x.scratch_bytes, s);
                    for (size_t k = 0; k < x.absorbed.size() && st == TLH_OK; ++k) st = launch_one(x.absorbed[k], state, s);
                    break;
                }
                st = mul_mat_compute_multi(ops, w, dsts, x.nmem, scratch, x.scratch_bytes, s);
                break;
            }
            case D_MUL_MAT_ID:
                st = tlh_mul_mat_id(&x.op, src[0], src[1], src[2], dst, scratch, x.scratch_bytes, s);
                break;
            case D_PAGED_WRITE:
                if (x.pw_f32[0] || x.pw_f32[1])
                    st = x.pw[0] == 0 ? TLH_OK
                                      : launch_reshape_and_cache(src[0], src[1], src[2], src[3], (const int64_t *)src[4],
                                                                 x.pw[0], x.pw[1], x.pw[2], x.pw[3], x.pw_blocks, s,
                                                                 x.pw_f32[0] != 0, x.pw_f32[1] != 0);
                else
                    st = tlh_reshape_and_cache(src[0], src[1], src[2], src[3], (const int64_t *)src[4], x.pw[0],
                                               x.pw[1], x.pw[2], x.pw[3], x.pw_blocks, s);
                break;
            case D_ARGMAX_SPLIT: st = launch_argmax_split(x.op, src[0], dst, scratch, s); break;
            case D_CORE_MULTI: {
                const void *ss[4][4];
                void *dd[4];
                for (int k = 0; k < x.nsub; ++k) {
                    for (int m = 0; m < 4; ++m) ss[k][m] = resolve(x.ssrc[k][m], state);
                    dd[k] = resolve(x.sdst[k], state);
                }
                st = launch_core_multi(x.nsub, x.sub_kind, x.sop, ss, dd, s);
                break;
            }
            case D_MULTI_GEMV: {
                const tlh_op *ops[3];
                const void *w[3];
                void *dsts[3];
                for (int k = 0; k < x.nmem; ++k) {
                    ops[k] = &x.mop[k];
                    w[k] = resolve(x.mw[k], state);
                    dsts[k] = resolve(x.mdst[k], state);
                }
                st = mul_mat_multi(ops, w, dsts, x.nmem, src[1], s);
                if (st == TLH_UNSUPPORTED)  // pointers the fused launch cannot take: one launch per node
                    for (int k = 0; k < x.nmem && (k == 0 || st == TLH_OK); ++k)
                        st = tlh_mul_mat(ops[k], w[k], src[1], dsts[k], scratch, x.scratch_bytes, s);
                break;
            }
            case D_GEMV_PRO: {
                const tlh_op *ops[3];
                const void *w[3];
                void *dsts[3];
                for (int k = 0; k < x.nmem; ++k) {
                    ops[k] = &x.mop[k];
                    w[k] = resolve(x.mw[k], state);
                    dsts[k] = resolve(x.mdst[k], state);
                }
                GemvPro pro;
                if (x.has_norm) {
                    pro.p = (const float *)resolve(x.nsrc[0], state);
                    pro.q = x.nop.x[2] ? (const float *)resolve(x.nsrc[1], state) : nullptr;
                    pro.w = (const float *)resolve(x.nsrc[2], state);
                    pro.s = x.nop.x[2] ? (float *)resolve(x.nsrc[3], state) : nullptr;
                    pro.p_nb1 = x.nop.t[0].nb[1];
                    pro.q_nb1 = x.nop.t[1].nb[1];
                    pro.s_nb1 = x.nop.t[3].nb[1];
                    pro.eps = __builtin_bit_cast(float, (int32_t)x.nop.x[1]);
                }
                if (x.has_glu) {
                    pro.glu = (float *)resolve(x.gdst, state);
                    pro.glu_nb1 = x.gop.t[4].nb[1];
                }
                if (x.has_epi) {
                    pro.epi = x.epi;
                    for (int k = 0; k < 3; ++k) {
                        pro.epi.dst[k] = (char *)resolve(x.edst[k], state);
                        pro.epi.idx[k] = (const char *)resolve(x.eidx[k], state);
                    }
                    pro.epi.pos = (const int32_t *)resolve(x.epos, state);
                    pro.epi.ff = (const float *)resolve(x.eff, state);
                }
                st = mul_mat_multi_pro(ops, w, dsts, x.nmem, pro, x.has_norm ? nullptr : src[1], s);
                if (st == TLH_UNSUPPORTED) {  // the pieces one by one
                    const void *act = src[1];
                    st = TLH_OK;
                    if (x.has_norm) {
                        void *y = resolve(x.ndst, state);
                        st = launch_norm_chain(x.nop, pro.p, pro.q, pro.w, pro.s, y, s);
                        act = y;
                    }
                    if (st == TLH_OK) st = mul_mat_multi(ops, w, dsts, x.nmem, act, s);
                    if (st == TLH_UNSUPPORTED)
                        for (int k = 0; k < x.nmem && (k == 0 || st == TLH_OK); ++k)
                            st = tlh_mul_mat(ops[k], w[k], act, dsts[k], scratch, x.scratch_bytes, s);
                    if (st == TLH_OK && x.has_glu)
                        st = tlh_core(TLH_CORE_GLU, &x.gop, dsts[0], dsts[1], nullptr, resolve(x.gdst, state), s);
                    for (size_t k = 0; k < x.absorbed.size() && st == TLH_OK; ++k)
                        st = launch_one(x.absorbed[k], state, s);
                }
                break;
            }
            default:
                if (x.core_kind == TLH_CORE_ROPE && x.op.x[9]) {  // rope into cache rows
                    const void *ss[1][4] = {{src[0], src[1], src[2], src[3]}};
                    st = launch_core_multi(1, &x.core_kind, &x.op, ss, &dst, s);
                } else if (x.core_kind == TLH_CORE_GLU && x.nq_type) {  // and the next MUL_MAT's quantization
                    ActQuantOut qo;
                    qo.out = scratch;
                    qo.type = x.nq_type;
                    qo.rows = x.nq_rows;
                    qo.f16 = x.nq_f16 != 0;
                    st = launch_glu_quantize(x.op, src[0], src[1], dst, qo, s);
                } else {
                    st = tlh_core(x.core_kind, &x.op, src[0], src[1], src[2], dst, s);
                }
                break;
            }
            return st;
        }
    }

    void drop_graph() {
        if (exec) (void)hipGraphExecDestroy(exec);
        exec = nullptr;
        exec_state = nullptr;
        exec_stream = nullptr;
    }
};

namespace {

tlh_status hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return TLH_OK;
    (void)hipGetLastError();
    if (e == hipErrorOutOfMemory) return set_error(TLH_ALLOC, "%s: %s", what, hipGetErrorString(e));
    return set_error(TLH_EXECUTION, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" {

tlh_status tlh_program_plan(const tlh_ir_tensor *tensors, int32_t n_tensors, const int32_t *nodes, int32_t n_nodes,
                            const int32_t *keep, int32_t n_keep, int64_t *tensor_offsets, int64_t *scratch_offsets,
                            size_t *arena_bytes) {
    Graph g;
    tlh_status st = read_graph(tensors, n_tensors, nodes, n_nodes, keep, n_keep, g);
    if (st != TLH_OK) return st;
    Lowered low;
    if ((st = Lowering(g).run(low)) != TLH_OK) return st;
    if (tensor_offsets)
        for (int32_t id = 0; id < n_tensors; ++id) {
            int64_t extra = 0;
            const int32_t r = g.root(id, extra);
            tensor_offsets[id] = low.arena_off[r] >= 0 ? low.arena_off[r] + extra : -1;
        }
    if (scratch_offsets)
        for (int32_t i = 0; i < n_nodes; ++i) scratch_offsets[i] = low.node_scratch[i];
    if (arena_bytes) *arena_bytes = (size_t)low.arena;
    return TLH_OK;
}

tlh_status tlh_program_compile(const tlh_ir_tensor *tensors, int32_t n_tensors, const int32_t *nodes,
                               int32_t n_nodes, const int32_t *keep, int32_t n_keep, const void *const *weights,
                               int32_t n_weights, const int64_t *state_offsets, int32_t n_states,
                               tlh_program **program) {
    if (!program) return set_error(TLH_INVALID, "program_compile: null result pointer");
    *program = nullptr;
    if (n_weights < 0 || n_states < 0 || (n_weights && !weights) || (n_states && !state_offsets))
        return set_error(TLH_INVALID, "program_compile: null or negative leaf arrays");
    Graph g;
    tlh_status st = read_graph(tensors, n_tensors, nodes, n_nodes, keep, n_keep, g);
    if (st != TLH_OK) return st;
    // leaves must exist for every root that names them
    int32_t n_inputs = 0;
    for (int32_t id = 0; id < n_tensors; ++id) {
        const tlh_ir_tensor &t = tensors[id];
        if (t.view_src >= 0) continue;
        const int32_t k = t.storage_index;
        if (t.storage == TLH_STORE_WEIGHT && (k < 0 || k >= n_weights))
            return set_error(TLH_INVALID, "tensor %d: weight index %d of %d", id, k, n_weights);
        if (t.storage == TLH_STORE_STATE && (k < 0 || k >= n_states))
            return set_error(TLH_INVALID, "tensor %d: state index %d of %d", id, k, n_states);
        if (t.storage == TLH_STORE_INPUT) {
            if (k < 0 || k >= n_tensors) return set_error(TLH_INVALID, "tensor %d: input index %d", id, k);
            n_inputs = std::max(n_inputs, k + 1);
        }
    }
    tlh_program *p = new tlh_program;
    p->tensors.assign(tensors, tensors + n_tensors);
    g.t = p->tensors.data();
    if ((st = Lowering(g).run(p->low)) != TLH_OK) {
        delete p;
        return st;
    }
    p->weights.assign(weights, weights + n_weights);
    p->state_offsets.assign(state_offsets, state_offsets + n_states);
    // inputs live in the io buffer, by input index (plan.rs:155-167)
    p->inputs.assign(n_inputs, {0, 0});
    std::vector<int64_t> in_bytes(n_inputs, -1);
    for (int32_t id = 0; id < n_tensors; ++id) {
        const tlh_ir_tensor &t = tensors[id];
        if (t.view_src < 0 && t.storage == TLH_STORE_INPUT) in_bytes[t.storage_index] = nbytes(t);
    }
    for (int32_t i = 0; i < n_inputs; ++i) {
        p->inputs[i] = {p->io_bytes, std::max<int64_t>(in_bytes[i], 0)};
        p->io_bytes += align_up(std::max<int64_t>(in_bytes[i], 1));
    }
    size_t n_counters = 0;
    for (const Dispatch &x : p->low.d)
        if (x.kind == D_PAGED_ATTN) n_counters = std::max(n_counters, paged_attention_counters(x.pa));
    (void)hipGetDevice(&p->device);
    if ((st = hip_ok(hipMalloc((void **)&p->arena, (size_t)std::max<int64_t>(p->low.arena, ALIGN)), "arena")) !=
            TLH_OK ||
        (st = hip_ok(hipMalloc((void **)&p->io, (size_t)std::max<int64_t>(p->io_bytes, ALIGN)), "io buffer")) !=
            TLH_OK ||
        (p->low.rt_bytes &&
         (st = hip_ok(hipMalloc((void **)&p->rtab, (size_t)p->low.rt_bytes), "rotation tables")) != TLH_OK) ||
        (n_counters &&
         ((st = hip_ok(hipMalloc((void **)&p->counters, n_counters * sizeof(unsigned)), "counters")) != TLH_OK ||
          (st = hip_ok(hipMemset(p->counters, 0, n_counters * sizeof(unsigned)), "counters")) != TLH_OK ||
          (st = hip_ok(hipStreamSynchronize(nullptr), "counters")) != TLH_OK))) {  // zero before any run's stream
        tlh_program_destroy(p);
        return st;
    }
    *program = p;
    return TLH_OK;
}

tlh_status tlh_program_destroy(tlh_program *p) {
    if (!p) return TLH_OK;
    p->drop_graph();
    if (p->arena) (void)hipFree(p->arena);
    if (p->io) (void)hipFree(p->io);
    if (p->counters) (void)hipFree(p->counters);
    if (p->rtab) (void)hipFree(p->rtab);
    delete p;
    return TLH_OK;
}

tlh_status tlh_copy(void *dst, const void *src, size_t bytes, void *stream) {
    if (!bytes) return TLH_OK;
    if (!dst || !src) return set_error(TLH_INVALID, "copy: null pointer");
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, (hipStream_t)stream), "copy");
}

tlh_status tlh_memset(void *dst, int value, size_t bytes, void *stream) {
    if (!bytes) return TLH_OK;
    if (!dst) return set_error(TLH_INVALID, "memset: null pointer");
    return launch_fill(dst, value, bytes, (hipStream_t)stream);
}

tlh_status tlh_read_floor(const void *src, size_t bytes, int32_t grid, int32_t loads, void *stream) {
    if (!src || (uintptr_t)src % 16 || bytes % 16) return set_error(TLH_INVALID, "read_floor: 16-byte aligned bytes");
    if (grid < 1 || grid > 65536 || (loads != 1 && loads != 4))
        return set_error(TLH_INVALID, "read_floor: grid 1..65536, 1 or 4 loads per lane");
    if (!bytes) return TLH_OK;
    return launch_read_floor(src, bytes, grid, loads, (hipStream_t)stream);
}

tlh_status tlh_program_input(const tlh_program *p, int32_t i, void **ptr, size_t *bytes) {
    if (!p || !ptr) return set_error(TLH_INVALID, "program_input: null pointer");
    if (i < 0 || i >= (int32_t)p->inputs.size()) return set_error(TLH_INVALID, "program_input: no graph input %d", i);
    *ptr = p->io + p->inputs[i].first;
    if (bytes) *bytes = (size_t)p->inputs[i].second;
    return TLH_OK;
}

tlh_status tlh_program_tensor(const tlh_program *p, int32_t id, void *state, void **ptr) {
    if (!p || !ptr) return set_error(TLH_INVALID, "program_tensor: null pointer");
    if (id < 0 || id >= (int32_t)p->tensors.size()) return set_error(TLH_INVALID, "program_tensor: id %d", id);
    const tlh_ir_tensor &t = p->tensors[id];
    const int32_t r = t.view_src >= 0 ? t.view_src : id;
    const int64_t extra = t.view_src >= 0 ? t.view_offs : 0;
    const tlh_ir_tensor &rt = p->tensors[r];
    switch (rt.storage) {
    case TLH_STORE_WEIGHT: *ptr = (char *)p->weights[rt.storage_index] + extra; break;
    case TLH_STORE_STATE:
        if (!state) return set_error(TLH_INVALID, "program_tensor: tensor %d is state; pass the state buffer", id);
        *ptr = (char *)state + p->state_offsets[rt.storage_index] + extra;
        break;
    case TLH_STORE_INPUT: *ptr = p->io + p->inputs[rt.storage_index].first + extra; break;
    default:
        if (p->low.arena_off[r] < 0) return set_error(TLH_INVALID, "program_tensor: tensor %d is never computed", id);
        *ptr = p->arena + p->low.arena_off[r] + extra;
    }
    return TLH_OK;
}

// TLH_NATIVE_PROFILE set: an eager run times every dispatch and prints the
// ops with the most GPU time to stderr, as the reference's executor does under
// TL_NATIVE_PROFILE (crates/kernels/src/cuda/exec.rs:186-216; events here, not
// a host clock around a synchronize).
static tlh_status run_profiled(tlh_program *p, void *state, hipStream_t s) {
    const size_t n = p->low.d.size();
    std::vector<float> ms(n, 0.0f);
    const tlh_status st = p->profile(state, s, ms.data());
    if (st != TLH_OK) return st;
    std::vector<std::tuple<std::string, double, int>> by_op;
    double total = 0;
    for (size_t i = 0; i < n; ++i) {
        const std::string op = p->op_of(p->low.d[i]);
        auto it = std::find_if(by_op.begin(), by_op.end(), [&](const auto &e) { return std::get<0>(e) == op; });
        if (it == by_op.end()) by_op.emplace_back(op, ms[i], 1);
        else std::get<1>(*it) += ms[i], ++std::get<2>(*it);
        total += ms[i];
    }
    std::stable_sort(by_op.begin(), by_op.end(), [](const auto &a, const auto &b) { return std::get<1>(a) > std::get<1>(b); });
    std::string list;
    for (size_t i = 0; i < by_op.size() && i < 6; ++i) {
        char buf[96];
        snprintf(buf, sizeof buf, "%s%s %.3fms/%d", i ? ", " : "", std::get<0>(by_op[i]).c_str(), std::get<1>(by_op[i]),
                 std::get<2>(by_op[i]));
        list += buf;
    }
    fprintf(stderr, "profile: %zu launches %.3f ms (events): %s\n", n, total, list.c_str());
    return TLH_OK;
}

tlh_status tlh_program_run(tlh_program *p, void *state, void *stream, int32_t graph) {
    if (!p) return set_error(TLH_INVALID, "program_run: null program");
    if (!p->state_offsets.empty() && !state) return set_error(TLH_INVALID, "program_run: the graph has state; pass its buffer");
    const hipStream_t s = (hipStream_t)stream;
    if (!graph) return getenv("TLH_NATIVE_PROFILE") ? run_profiled(p, state, s) : p->enqueue(state, s);
    if (!s) return set_error(TLH_INVALID, "program_run: graph replay needs a stream other than the null stream");
    if (!p->exec || p->exec_state != state || p->exec_stream != s) {
        p->drop_graph();
        tlh_status st = hip_ok(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
        if (st != TLH_OK) return st;
        st = p->enqueue(state, s);
        hipGraph_t gr = nullptr;
        const hipError_t e = hipStreamEndCapture(s, &gr);
        if (st != TLH_OK) {
            if (gr) (void)hipGraphDestroy(gr);
            return st;
        }
        if ((st = hip_ok(e, "hipStreamEndCapture")) != TLH_OK) return st;
        hipGraphExec_t ex = nullptr;
        st = hip_ok(hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0), "hipGraphInstantiate");
        (void)hipGraphDestroy(gr);
        if (st != TLH_OK) return st;
        p->exec = ex;
        p->exec_state = state;
        p->exec_stream = s;
    }
    return hip_ok(hipGraphLaunch(p->exec, s), "hipGraphLaunch");
}

tlh_status tlh_program_profile(tlh_program *p, void *state, void *stream, float *ms, int32_t n) {
    if (!p || (!ms && !p->low.d.empty())) return set_error(TLH_INVALID, "program_profile: null pointer");
    if (n < (int32_t)p->low.d.size())
        return set_error(TLH_INVALID, "program_profile: room for %d of %zu dispatches", n, p->low.d.size());
    if (!p->state_offsets.empty() && !state)
        return set_error(TLH_INVALID, "program_profile: the graph has state; pass its buffer");
    return p->profile(state, (hipStream_t)stream, ms);
}

tlh_status tlh_program_trace(tlh_program *p, void *state, void *stream, char *text, size_t cap, size_t *len) {
    if (!p || (!text && cap)) return set_error(TLH_INVALID, "program_trace: null pointer");
    if (!p->state_offsets.empty() && !state)
        return set_error(TLH_INVALID, "program_trace: the graph has state; pass its buffer");
    std::string out, labels;
    tlh_status st = TLH_OK;
    for (size_t i = 0; i < p->low.d.size() && st == TLH_OK; ++i) {
        labels.clear();
        launch_trace(&labels);
        st = p->enqueue_one(i, state, (hipStream_t)stream);
        launch_trace(nullptr);
        const Dispatch &x = p->low.d[i];
        char head[64];
        snprintf(head, sizeof head, "%zu\t%s\t", i, p->op_of(x));
        out += head;
        out += labels;
        out.push_back('\n');
    }
    if (st != TLH_OK) return st;
    if (len) *len = out.size() + 1;
    if (cap) {
        const size_t k = std::min(cap - 1, out.size());
        memcpy(text, out.data(), k);
        text[k] = 0;
    }
    return TLH_OK;
}

tlh_status tlh_program_stats(const tlh_program *p, size_t *arena_bytes, size_t *io_bytes, int32_t *launches) {
    if (!p) return set_error(TLH_INVALID, "program_stats: null program");
    if (arena_bytes) *arena_bytes = (size_t)p->low.arena;
    if (io_bytes) *io_bytes = (size_t)p->io_bytes;
    if (launches) *launches = (int32_t)p->low.d.size();
    return TLH_OK;
}

}  // extern "C"

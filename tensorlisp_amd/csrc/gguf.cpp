// GGUF reading and loading (include/tlhip.h, "GGUF"). Host code only.
//
// Takes the place of the reference's model load for its native executors
// (crates/tensorlisp/src/native_cuda.rs:44-82 over ggml's reader,
// vendor/ggml/src/gguf.cpp:450-800 via crates/tensorlisp/src/gguf.rs:79-320):
// the header, key-value pairs and tensor infos are parsed and checked with
// the rules ggml applies (versions 2 and 3, general.alignment a power of two
// of type u32, names under 64 bytes and unique, at most 4 dimensions, rows of
// whole blocks, tensor offsets consecutive at the alignment), then every
// tensor is copied from the file into one device buffer at offsets the caller
// plans (tlh_gguf_layout: each tensor 256-byte aligned, as the kernels like
// their rows), through two pinned staging buffers so disk reads and copies
// overlap.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace {

using tlh::set_error;

constexpr uint32_t GG_STRING = 8, GG_ARRAY = 9;

// byte size of a scalar GGUF value type (0 for string / array / unknown)
size_t scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;   // u8, i8, bool
    case 2: case 3: return 2;           // u16, i16
    case 4: case 5: case 6: return 4;   // u32, i32, f32
    case 10: case 11: case 12: return 8;  // u64, i64, f64
    default: return 0;
    }
}

// ggml type traits for sizes: block elements, block bytes (types the loader sizes)
bool ggml_traits(int ty, int64_t &blck, int64_t &size) {
    static const int64_t t[][3] = {{0, 1, 4},     {1, 1, 2},      {2, 32, 18},    {3, 32, 20},   {6, 32, 22},
                                   {7, 32, 24},   {8, 32, 34},    {9, 32, 36},    {10, 256, 84}, {11, 256, 110},
                                   {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {24, 1, 1},
                                   {25, 1, 2},    {26, 1, 4},     {27, 1, 8},     {28, 1, 8},    {30, 1, 2}};
    for (const auto &e : t)
        if (e[0] == ty) {
            blck = e[1], size = e[2];
            return true;
        }
    return false;
}

struct Kv {
    std::string key;
    uint32_t type = 0, arr_type = 0;
    uint64_t n = 0;                      // array length
    std::vector<uint8_t> data;           // scalar or numeric array bytes
    std::vector<std::string> strs;       // string value (one) or string array
};

struct Reader {
    int fd;
    uint64_t pos = 0, size = 0;
    bool read(void *dst, size_t n) {
        if (pos + n > size) return false;
        size_t done = 0;
        while (done < n) {
            const ssize_t r = pread(fd, (char *)dst + done, n - done, (off_t)(pos + done));
            if (r <= 0) return false;
            done += (size_t)r;
        }
        pos += n;
        return true;
    }
    template <typename T> bool get(T &v) { return read(&v, sizeof v); }
    bool str(std::string &s) {
        uint64_t n;
        if (!get(n) || n > size - pos) return false;
        s.resize(n);
        return read(&s[0], n);
    }
};

}  // namespace

struct tlh_gguf {
    int fd = -1;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0, file_size = 0;
    std::vector<Kv> kv;
    std::vector<tlh_gguf_tensor_info> tensors;
    std::map<std::string, int64_t> by_name, key_id;
};

namespace {

tlh_status bad(tlh_gguf *g, const char *fmt, const std::string &a = "", long long b = 0) {
    char buf[384];
    snprintf(buf, sizeof buf, fmt, a.c_str(), b);
    if (g) {
        if (g->fd >= 0) close(g->fd);
        delete g;
    }
    return set_error(TLH_INVALID, "gguf: %s", buf);
}

}  // namespace

extern "C" {

tlh_status tlh_gguf_open(const char *path, tlh_gguf **out) {
    if (!path || !out) return set_error(TLH_INVALID, "gguf_open: null pointer");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return set_error(TLH_INVALID, "gguf_open: cannot open %s", path);
    tlh_gguf *g = new tlh_gguf;
    g->fd = fd;
    Reader r{fd};
    r.size = (uint64_t)lseek(fd, 0, SEEK_END);
    g->file_size = r.size;
    char magic[4];
    if (!r.read(magic, 4) || memcmp(magic, "GGUF", 4) != 0) return bad(g, "%s: not a GGUF file", path);
    if (!r.get(g->version)) return bad(g, "%struncated header", "");
    if (g->version == 0 || (g->version & 0xFFFF) == 0)
        return bad(g, "%sversion %lld: corrupt, or the other byte order", "", g->version);
    if (g->version == 1) return bad(g, "%sGGUF version 1 is no longer supported", "");
    if (g->version > 3) return bad(g, "%sGGUF version %lld is newer than 3", "", g->version);
    int64_t n_tensors, n_kv;
    if (!r.get(n_tensors) || !r.get(n_kv) || n_tensors < 0 || n_kv < 0)
        return bad(g, "%sbad tensor or key count", "");
    for (int64_t i = 0; i < n_kv; ++i) {
        Kv k;
        int32_t t;
        if (!r.str(k.key) || !r.get(t)) return bad(g, "%struncated key-value pair %lld", "", i);
        k.type = (uint32_t)t;
        if (g->key_id.count(k.key)) return bad(g, "duplicate key '%s'", k.key);
        bool ok = true;
        if (k.type == GG_STRING) {
            std::string s;
            ok = r.str(s);
            k.strs.push_back(s);
        } else if (k.type == GG_ARRAY) {
            int32_t at;
            ok = r.get(at) && r.get(k.n);
            k.arr_type = (uint32_t)at;
            if (ok && k.arr_type == GG_STRING) {
                for (uint64_t j = 0; ok && j < k.n; ++j) {
                    std::string s;
                    ok = r.str(s);
                    k.strs.push_back(s);
                }
            } else if (ok) {
                const size_t es = scalar_size(k.arr_type);
                if (es == 0) return bad(g, "key '%s': array of unsupported type %lld", k.key, k.arr_type);
                if (k.n > (r.size - r.pos) / es) return bad(g, "key '%s': array past the end of the file", k.key);
                k.data.resize(k.n * es);
                ok = r.read(k.data.data(), k.data.size());
            }
        } else {
            const size_t es = scalar_size(k.type);
            if (es == 0) return bad(g, "key '%s' has invalid GGUF type %lld", k.key, k.type);
            k.data.resize(es);
            ok = r.read(k.data.data(), es);
        }
        if (!ok) return bad(g, "key '%s': truncated value", k.key);
        g->key_id[k.key] = (int64_t)g->kv.size();
        g->kv.push_back(std::move(k));
    }
    if (g->key_id.count("general.alignment")) {
        const Kv &k = g->kv[g->key_id["general.alignment"]];
        if (k.type != 4) return bad(g, "%sgeneral.alignment must be a u32", "");
        uint32_t a;
        memcpy(&a, k.data.data(), 4);
        if (a == 0 || (a & (a - 1))) return bad(g, "%salignment %lld is not a power of 2", "", a);
        g->alignment = a;
    }
    uint64_t expect = 0;
    for (int64_t i = 0; i < n_tensors; ++i) {
        tlh_gguf_tensor_info ti;
        memset(&ti, 0, sizeof ti);
        std::string name;
        uint32_t n_dims;
        if (!r.str(name) || !r.get(n_dims)) return bad(g, "%struncated tensor info %lld", "", i);
        if (name.size() >= sizeof ti.name) return bad(g, "tensor name '%s' is too long (64 bytes at most)", name);
        if (g->by_name.count(name)) return bad(g, "duplicate tensor name '%s'", name);
        if (n_dims > 4) return bad(g, "tensor '%s' has %lld dimensions", name, n_dims);
        memcpy(ti.name, name.c_str(), name.size() + 1);
        ti.n_dims = (int32_t)n_dims;
        for (int d = 0; d < 4; ++d) {
            ti.ne[d] = 1;
            if ((uint32_t)d < n_dims && !r.get(ti.ne[d])) return bad(g, "tensor '%s': truncated shape", name);
            if (ti.ne[d] < 0) return bad(g, "tensor '%s' has a negative dimension", name);
        }
        int32_t ty;
        if (!r.get(ty) || !r.get(ti.offset)) return bad(g, "tensor '%s': truncated info", name);
        ti.ty = ty;
        int64_t blck, size;
        if (!ggml_traits(ty, blck, size)) {
            if (g->fd >= 0) close(g->fd);
            delete g;
            return set_error(TLH_UNSUPPORTED, "gguf: tensor '%s' has ggml type %d, which this loader does not size",
                             name.c_str(), ty);
        }
        if (ti.ne[0] % blck) return bad(g, "tensor '%s': rows are not whole blocks", name);
        // The element count must be an int64, as ggml's reader demands
        // (vendor/ggml/src/gguf.cpp:691-702); each partial product is
        // checked before it is formed. Then the byte count and the running
        // offset must not wrap either.
        int64_t nel = ti.ne[0];
        for (int d = 1; d < 4 && nel > 0; ++d) {
            if (ti.ne[d] > 0 && nel >= INT64_MAX / ti.ne[d])
                return bad(g, "tensor '%s' has more elements than an int64 holds", name);
            nel *= ti.ne[d];
        }
        if (ti.ne[1] == 0 || ti.ne[2] == 0 || ti.ne[3] == 0) nel = 0;
        const uint64_t nblocks = (uint64_t)(nel / blck);
        if (size > 0 && nblocks > UINT64_MAX / 2 / (uint64_t)size)
            return bad(g, "tensor '%s' has more bytes than a size holds", name);
        ti.bytes = nblocks * (uint64_t)size;
        if (ti.offset != expect) return bad(g, "tensor '%s' has offset %lld, expected the next aligned slot", name, (long long)ti.offset);
        const uint64_t padded = (ti.bytes + g->alignment - 1) / g->alignment * g->alignment;
        if (padded > g->file_size || expect > g->file_size - padded)
            return bad(g, "tensor '%s': data past the end of the file", name);
        expect += padded;
        g->by_name[name] = (int64_t)g->tensors.size();
        g->tensors.push_back(ti);
    }
    g->data_offset = n_tensors > 0 ? (r.pos + g->alignment - 1) / g->alignment * g->alignment : r.pos;
    for (const tlh_gguf_tensor_info &t : g->tensors)  // every tensor, offsets and sizes already bounded above
        if (g->data_offset > g->file_size || t.offset + t.bytes > g->file_size - g->data_offset)
            return bad(g, "tensor '%s': data past the end of the file", std::string(t.name));
    *out = g;
    return TLH_OK;
}

tlh_status tlh_gguf_close(tlh_gguf *g) {
    if (g) {
        if (g->fd >= 0) close(g->fd);
        delete g;
    }
    return TLH_OK;
}

tlh_status tlh_gguf_counts(const tlh_gguf *g, uint32_t *version, int64_t *n_tensors, int64_t *n_kv, uint64_t *alignment,
                           uint64_t *data_offset) {
    if (!g) return set_error(TLH_INVALID, "gguf: null handle");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
    if (n_kv) *n_kv = (int64_t)g->kv.size();
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    return TLH_OK;
}

tlh_status tlh_gguf_tensor(const tlh_gguf *g, int64_t i, tlh_gguf_tensor_info *info) {
    if (!g || !info) return set_error(TLH_INVALID, "gguf: null pointer");
    if (i < 0 || i >= (int64_t)g->tensors.size()) return set_error(TLH_INVALID, "gguf: no tensor %lld", (long long)i);
    *info = g->tensors[i];
    return TLH_OK;
}

tlh_status tlh_gguf_find_tensor(const tlh_gguf *g, const char *name, int64_t *i) {
    if (!g || !name || !i) return set_error(TLH_INVALID, "gguf: null pointer");
    auto it = g->by_name.find(name);
    *i = it == g->by_name.end() ? -1 : it->second;
    return TLH_OK;
}

tlh_status tlh_gguf_find_key(const tlh_gguf *g, const char *key, int64_t *i) {
    if (!g || !key || !i) return set_error(TLH_INVALID, "gguf: null pointer");
    auto it = g->key_id.find(key);
    *i = it == g->key_id.end() ? -1 : it->second;
    return TLH_OK;
}

tlh_status tlh_gguf_key(const tlh_gguf *g, int64_t i, const char **key, int32_t *type, int32_t *arr_type,
                        uint64_t *n) {
    if (!g) return set_error(TLH_INVALID, "gguf: null handle");
    if (i < 0 || i >= (int64_t)g->kv.size()) return set_error(TLH_INVALID, "gguf: no key %lld", (long long)i);
    const Kv &k = g->kv[i];
    if (key) *key = k.key.c_str();
    if (type) *type = (int32_t)k.type;
    if (arr_type) *arr_type = (int32_t)k.arr_type;
    if (n) *n = k.type == GG_ARRAY ? k.n : 1;
    return TLH_OK;
}

tlh_status tlh_gguf_value(const tlh_gguf *g, int64_t i, const void **data, size_t *bytes) {
    if (!g || !data) return set_error(TLH_INVALID, "gguf: null pointer");
    if (i < 0 || i >= (int64_t)g->kv.size()) return set_error(TLH_INVALID, "gguf: no key %lld", (long long)i);
    const Kv &k = g->kv[i];
    if (k.type == GG_STRING || (k.type == GG_ARRAY && k.arr_type == GG_STRING))
        return set_error(TLH_INVALID, "gguf: key '%s' holds strings", k.key.c_str());
    *data = k.data.data();
    if (bytes) *bytes = k.data.size();
    return TLH_OK;
}

tlh_status tlh_gguf_string(const tlh_gguf *g, int64_t i, uint64_t j, const char **s, uint64_t *len) {
    if (!g || !s) return set_error(TLH_INVALID, "gguf: null pointer");
    if (i < 0 || i >= (int64_t)g->kv.size()) return set_error(TLH_INVALID, "gguf: no key %lld", (long long)i);
    const Kv &k = g->kv[i];
    if (j >= k.strs.size()) return set_error(TLH_INVALID, "gguf: key '%s' has no string %llu", k.key.c_str(),
                                             (unsigned long long)j);
    *s = k.strs[j].c_str();
    if (len) *len = k.strs[j].size();
    return TLH_OK;
}

tlh_status tlh_gguf_layout(const tlh_gguf *g, uint64_t *offsets, uint64_t *total) {
    if (!g || !total) return set_error(TLH_INVALID, "gguf: null pointer");
    uint64_t off = 0;
    for (size_t i = 0; i < g->tensors.size(); ++i) {
        if (offsets) offsets[i] = off;
        off += (g->tensors[i].bytes + 255) / 256 * 256;
    }
    *total = off;
    return TLH_OK;
}

tlh_status tlh_gguf_upload(const tlh_gguf *g, void *dev, const uint64_t *offsets, void *stream) {
    if (!g || (!dev && !g->tensors.empty()) || (!offsets && !g->tensors.empty()))
        return set_error(TLH_INVALID, "gguf_upload: null pointer");
    constexpr size_t CHUNK = 64u << 20;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    const hipStream_t s = (hipStream_t)stream;
    tlh_status st = TLH_OK;
    for (int b = 0; b < 2 && st == TLH_OK; ++b) {
        if (hipHostMalloc(&stage[b], CHUNK, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess)
            st = set_error(TLH_ALLOC, "gguf_upload: pinned staging buffers");
    }
    bool used[2] = {false, false};
    int b = 0;
    for (size_t i = 0; i < g->tensors.size() && st == TLH_OK; ++i) {
        const tlh_gguf_tensor_info &t = g->tensors[i];
        for (uint64_t o = 0; o < t.bytes && st == TLH_OK; o += CHUNK) {
            const size_t n = (size_t)(t.bytes - o < CHUNK ? t.bytes - o : CHUNK);
            if (used[b] && hipEventSynchronize(done[b]) != hipSuccess) {  // the copy out of this buffer is done
                st = set_error(TLH_EXECUTION, "gguf_upload: waiting for a copy");
                break;
            }
            size_t got = 0;
            while (got < n) {
                const ssize_t r = pread(g->fd, (char *)stage[b] + got, n - got,
                                        (off_t)(g->data_offset + t.offset + o + got));
                if (r <= 0) break;
                got += (size_t)r;
            }
            if (got != n) {
                st = set_error(TLH_INVALID, "gguf_upload: short read of tensor '%s'", t.name);
                break;
            }
            if (hipMemcpyAsync((char *)dev + offsets[i] + o, stage[b], n, hipMemcpyHostToDevice, s) != hipSuccess ||
                hipEventRecord(done[b], s) != hipSuccess) {
                st = set_error(TLH_EXECUTION, "gguf_upload: copy of tensor '%s'", t.name);
                break;
            }
            used[b] = true;
            b ^= 1;
        }
    }
    if (hipStreamSynchronize(s) != hipSuccess && st == TLH_OK) st = set_error(TLH_EXECUTION, "gguf_upload: sync");
    for (int k = 0; k < 2; ++k) {
        if (done[k]) (void)hipEventDestroy(done[k]);
        if (stage[k]) (void)hipHostFree(stage[k]);
    }
    return st;
}

}  // extern "C"

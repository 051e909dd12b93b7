// gguf_reader.cpp -- GGUF (v2/v3) runtime-pack reader over a read-only
// memory mapping, the container of OpenASR's `.oasr` v1 packs
// (docs/format/OASR_PACKAGE_CONTRACT_V1.md: standard GGUF bytes, GGUF magic
// accepted, the reserved OASR magic and anything else refused). It stands in
// for the fork's gguf_init_from_file + the host's tensor-data reader
// (crates/openasr-core/src/ggml_runtime/gguf_metadata.rs,
// gguf_tensor_data.rs): metadata by key, tensor infos by name, and tensor
// bytes as views into the mapping (no copy), so weights go from the page
// cache straight into the device's WEIGHTS buffer.
//
// Every read is bounds-checked against the file; counts, string lengths and
// array sizes are capped by what the file can hold; tensor ranges must lie in
// the data section, be aligned, and match their type's row size. A malformed
// file fails closed with a message.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "ggml_host.h"
#include "openasr_models.h"

namespace {

enum gguf_vtype : uint32_t {
    GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64,
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case GV_U8: case GV_I8: case GV_BOOL: return 1;
        case GV_U16: case GV_I16: return 2;
        case GV_U32: case GV_I32: case GV_F32: return 4;
        case GV_U64: case GV_I64: case GV_F64: return 8;
        default: return 0;
    }
}

struct kv_entry {
    uint32_t type = 0;
    uint32_t arr_type = 0;
    uint64_t arr_n = 0;
    size_t off = 0;  // file offset of the value (of the first element for arrays)
    std::string str;  // GV_STR values
};

struct tensor_info {
    std::string name;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    int type = 0;
    uint64_t offset = 0;  // within the data section
    size_t nbytes = 0;
};

}  // namespace

struct oa_gguf {
    int fd = -1;
    const uint8_t * base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    size_t alignment = 32;
    size_t data_off = 0;
    std::unordered_map<std::string, kv_entry> kv;
    std::vector<tensor_info> tensors;
    std::unordered_map<std::string, int64_t> by_name;
};

namespace {

struct cursor {
    const oa_gguf * g;
    size_t pos;
    std::string err;

    bool fail(const char * fmt, ...) {
        if (err.empty()) {
            char buf[256];
            va_list ap;
            va_start(ap, fmt);
            std::vsnprintf(buf, sizeof(buf), fmt, ap);
            va_end(ap);
            err = buf;
        }
        return false;
    }
    bool need(size_t n) {
        if (n > g->size || pos > g->size - n) return fail("truncated at byte %zu (need %zu more)", pos, n);
        return true;
    }
    template <typename T>
    bool rd(T & v) {
        if (!need(sizeof(T))) return false;
        std::memcpy(&v, g->base + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool str(std::string & s) {
        uint64_t n = 0;
        if (!rd(n)) return false;
        if (n > (1u << 24)) return fail("string of %llu bytes at byte %zu", (unsigned long long) n, pos);
        if (!need((size_t) n)) return false;
        s.assign((const char *) g->base + pos, (size_t) n);
        pos += (size_t) n;
        return true;
    }
    bool skip(size_t n) {
        if (!need(n)) return false;
        pos += n;
        return true;
    }
};

void set_err(char * err, size_t cap, const std::string & msg) {
    if (err && cap) std::snprintf(err, cap, "%s", msg.c_str());
}

bool parse(oa_gguf * g, std::string & err) {
    cursor c{g, 0, {}};
    uint32_t magic = 0;
    if (!c.rd(magic)) {
        err = "not a GGUF file: " + c.err;
        return false;
    }
    if (std::memcmp(g->base, "OASR", 4) == 0) {
        err = "the OASR container magic is reserved and not supported by v1 readers";
        return false;
    }
    if (std::memcmp(g->base, "GGUF", 4) != 0) {
        err = "unknown magic: not a GGUF runtime pack";
        return false;
    }
    if (!c.rd(g->version)) {
        err = c.err;
        return false;
    }
    if (g->version != 2 && g->version != 3) {
        err = "unsupported GGUF version " + std::to_string(g->version);
        return false;
    }
    uint64_t n_tensors = 0, n_kv = 0;
    if (!c.rd(n_tensors) || !c.rd(n_kv)) {
        err = c.err;
        return false;
    }
    // every kv needs at least 13 bytes, every tensor info at least 28
    if (n_kv > g->size / 13 || n_tensors > g->size / 28) {
        err = "metadata counts exceed what the file can hold";
        return false;
    }
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        kv_entry e;
        if (!c.str(key) || !c.rd(e.type)) {
            err = c.err;
            return false;
        }
        if (e.type == GV_STR) {
            e.off = c.pos;
            if (!c.str(e.str)) {
                err = c.err;
                return false;
            }
        } else if (e.type == GV_ARR) {
            if (!c.rd(e.arr_type) || !c.rd(e.arr_n)) {
                err = c.err;
                return false;
            }
            e.off = c.pos;
            if (e.arr_type == GV_STR) {
                if (e.arr_n > g->size / 8) {
                    err = "string array larger than the file";
                    return false;
                }
                for (uint64_t k = 0; k < e.arr_n; k++) {
                    uint64_t n = 0;
                    if (!c.rd(n) || !c.skip((size_t) std::min<uint64_t>(n, g->size))) {
                        err = c.err;
                        return false;
                    }
                }
            } else {
                const size_t es = scalar_size(e.arr_type);
                if (!es || e.arr_n > g->size / es) {
                    err = "array of type " + std::to_string(e.arr_type) + " in key '" + key + "' is malformed";
                    return false;
                }
                if (!c.skip((size_t) (e.arr_n * es))) {
                    err = c.err;
                    return false;
                }
            }
        } else {
            const size_t es = scalar_size(e.type);
            if (!es) {
                err = "key '" + key + "' has unknown value type " + std::to_string(e.type);
                return false;
            }
            e.off = c.pos;
            if (!c.skip(es)) {
                err = c.err;
                return false;
            }
        }
        if (!g->kv.emplace(key, std::move(e)).second) {
            err = "duplicate metadata key '" + key + "'";
            return false;
        }
    }
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end()) {
        if (al->second.type != GV_U32) {
            err = "general.alignment is not a u32";
            return false;
        }
        uint32_t a = 0;
        std::memcpy(&a, g->base + al->second.off, 4);
        if (a == 0 || (a & (a - 1))) {
            err = "general.alignment " + std::to_string(a) + " is not a power of two";
            return false;
        }
        g->alignment = a;
    }
    g->tensors.resize((size_t) n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        tensor_info & t = g->tensors[(size_t) i];
        uint32_t nd = 0, type = 0;
        if (!c.str(t.name) || !c.rd(nd)) {
            err = c.err;
            return false;
        }
        if (nd < 1 || nd > 4) {
            err = "tensor '" + t.name + "' has " + std::to_string(nd) + " dimensions";
            return false;
        }
        t.n_dims = (int) nd;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v = 0;
            if (!c.rd(v)) {
                err = c.err;
                return false;
            }
            if (v == 0 || v > (1ull << 40)) {
                err = "tensor '" + t.name + "' has dimension " + std::to_string(v);
                return false;
            }
            t.ne[d] = (int64_t) v;
        }
        if (!c.rd(type) || !c.rd(t.offset)) {
            err = c.err;
            return false;
        }
        if (type >= GGML_TYPE_COUNT || ggml_type_size((ggml_type) type) == 0) {
            err = "tensor '" + t.name + "' has unsupported type " + std::to_string(type);
            return false;
        }
        t.type = (int) type;
        if (t.ne[0] % ggml_blck_size((ggml_type) type) != 0) {
            err = "tensor '" + t.name + "' rows are not whole blocks of its type";
            return false;
        }
        const size_t row = ggml_row_size((ggml_type) type, t.ne[0]);
        const double total = (double) row * (double) t.ne[1] * (double) t.ne[2] * (double) t.ne[3];
        if (total > (double) g->size) {
            err = "tensor '" + t.name + "' is larger than the file";
            return false;
        }
        t.nbytes = row * (size_t) (t.ne[1] * t.ne[2] * t.ne[3]);
        if (!g->by_name.emplace(t.name, (int64_t) i).second) {
            err = "duplicate tensor '" + t.name + "'";
            return false;
        }
    }
    g->data_off = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_off > g->size && n_tensors > 0) {
        err = "data section starts past the end of the file";
        return false;
    }
    for (const tensor_info & t : g->tensors) {
        if (t.offset % g->alignment != 0) {
            err = "tensor '" + t.name + "' data is not aligned to " + std::to_string(g->alignment);
            return false;
        }
        if (t.offset > g->size - g->data_off || t.nbytes > g->size - g->data_off - t.offset) {
            err = "tensor '" + t.name + "' data runs past the end of the file";
            return false;
        }
    }
    return true;
}

const kv_entry * find_kv(const oa_gguf * g, const char * key) {
    auto it = g->kv.find(key);
    return it == g->kv.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

oa_gguf * oa_gguf_open(const char * path, char * err, size_t err_cap) {
    oa_gguf * g = new oa_gguf;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0) {
        set_err(err, err_cap, std::string("cannot open ") + path);
        oa_gguf_close(g);
        return nullptr;
    }
    g->size = (size_t) st.st_size;
    if (g->size < 24) {
        set_err(err, err_cap, "file too small for a GGUF header");
        oa_gguf_close(g);
        return nullptr;
    }
    void * p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (p == MAP_FAILED) {
        set_err(err, err_cap, std::string("cannot map ") + path);
        oa_gguf_close(g);
        return nullptr;
    }
    g->base = (const uint8_t *) p;
    std::string e;
    if (!parse(g, e)) {
        set_err(err, err_cap, e);
        oa_gguf_close(g);
        return nullptr;
    }
    return g;
}

void oa_gguf_close(oa_gguf * g) {
    if (!g) return;
    if (g->base) munmap((void *) g->base, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

uint32_t oa_gguf_version(const oa_gguf * g) { return g->version; }
size_t oa_gguf_alignment(const oa_gguf * g) { return g->alignment; }
int64_t oa_gguf_n_tensors(const oa_gguf * g) { return (int64_t) g->tensors.size(); }
int64_t oa_gguf_n_kv(const oa_gguf * g) { return (int64_t) g->kv.size(); }

int64_t oa_gguf_find_tensor(const oa_gguf * g, const char * name) {
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : it->second;
}

const char * oa_gguf_tensor_name(const oa_gguf * g, int64_t i) {
    return i >= 0 && i < (int64_t) g->tensors.size() ? g->tensors[(size_t) i].name.c_str() : nullptr;
}

int oa_gguf_tensor_info(const oa_gguf * g, int64_t i, int * type, int64_t ne[4]) {
    if (i < 0 || i >= (int64_t) g->tensors.size()) return -1;
    const tensor_info & t = g->tensors[(size_t) i];
    if (type) *type = t.type;
    if (ne) std::memcpy(ne, t.ne, sizeof(t.ne));
    return t.n_dims;
}

const void * oa_gguf_tensor_data(const oa_gguf * g, int64_t i, size_t * nbytes) {
    if (i < 0 || i >= (int64_t) g->tensors.size()) return nullptr;
    const tensor_info & t = g->tensors[(size_t) i];
    if (nbytes) *nbytes = t.nbytes;
    return g->base + g->data_off + t.offset;
}

int oa_gguf_kv_type(const oa_gguf * g, const char * key) {
    const kv_entry * e = find_kv(g, key);
    return e ? (int) e->type : -1;
}

const char * oa_gguf_get_str(const oa_gguf * g, const char * key) {
    const kv_entry * e = find_kv(g, key);
    return e && e->type == GV_STR ? e->str.c_str() : nullptr;
}

bool oa_gguf_get_i64(const oa_gguf * g, const char * key, int64_t * out) {
    const kv_entry * e = find_kv(g, key);
    if (!e) return false;
    const uint8_t * p = g->base + e->off;
    switch (e->type) {
        case GV_U8: *out = *p; return true;
        case GV_I8: *out = (int8_t) *p; return true;
        case GV_U16: { uint16_t v; std::memcpy(&v, p, 2); *out = v; return true; }
        case GV_I16: { int16_t v; std::memcpy(&v, p, 2); *out = v; return true; }
        case GV_U32: { uint32_t v; std::memcpy(&v, p, 4); *out = v; return true; }
        case GV_I32: { int32_t v; std::memcpy(&v, p, 4); *out = v; return true; }
        case GV_U64: {
            uint64_t v;
            std::memcpy(&v, p, 8);
            if (v > (uint64_t) INT64_MAX) return false;
            *out = (int64_t) v;
            return true;
        }
        case GV_I64: { int64_t v; std::memcpy(&v, p, 8); *out = v; return true; }
        default: return false;
    }
}

bool oa_gguf_get_f64(const oa_gguf * g, const char * key, double * out) {
    const kv_entry * e = find_kv(g, key);
    if (!e) return false;
    const uint8_t * p = g->base + e->off;
    if (e->type == GV_F32) {
        float v;
        std::memcpy(&v, p, 4);
        *out = v;
        return true;
    }
    if (e->type == GV_F64) {
        std::memcpy(out, p, 8);
        return true;
    }
    int64_t i;
    if (!oa_gguf_get_i64(g, key, &i)) return false;
    *out = (double) i;
    return true;
}

}  // extern "C"

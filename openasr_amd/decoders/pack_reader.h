// pack_reader.h -- typed access to the tensors and keys of a mapped runtime
// pack (oa_gguf_*), shared by the model loaders of libopenasr-models.so.
// Mirrors the checks of the reference's binding (ggml_runtime/
// gguf_tensor_data.rs, models/*/ggml_tensor_binding.rs): a tensor must exist
// with the exact shape and one of the expected types; keys must be present
// positive integers.
#pragma once
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <string>
#include <vector>

#include "ggml_host.h"
#include "openasr_models.h"

namespace oa_pack {

// weight bytes: owned (synthesised, or assembled such as the fused QKV) or
// a view into a mapped runtime pack
struct blob {
    std::vector<uint8_t> own;
    const uint8_t * view = nullptr;
    size_t n = 0;
    blob & operator=(std::vector<uint8_t> && v) {
        own = std::move(v);
        view = nullptr;
        n = 0;
        return *this;
    }
    void set_view(const void * p, size_t bytes) {
        own.clear();
        view = (const uint8_t *) p;
        n = bytes;
    }
    const uint8_t * data() const { return view ? view : own.data(); }
    size_t size() const { return view ? n : own.size(); }
};

struct pack_reader {
    oa_gguf * g;
    std::string err;

    bool fail(const std::string & msg) {
        if (err.empty()) err = msg;
        return false;
    }
    bool key_i(const char * key, int & out) {
        int64_t v = 0;
        if (!oa_gguf_get_i64(g, key, &v)) return fail(std::string("missing or non-integer key ") + key);
        if (v <= 0 || v > (1 << 30)) return fail(std::string("key ") + key + " out of range");
        out = (int) v;
        return true;
    }
    // tensor `name` of type in `types` with ne = (ne0, ne1); returns its index
    int64_t tensor(const std::string & name, int64_t ne0, int64_t ne1, std::initializer_list<int> types, int & type) {
        const int64_t i = oa_gguf_find_tensor(g, name.c_str());
        if (i < 0) {
            fail("missing tensor " + name);
            return -1;
        }
        int64_t ne[4];
        const int nd = oa_gguf_tensor_info(g, i, &type, ne);
        if (ne[0] != ne0 || ne[1] != ne1 || ne[2] != 1 || ne[3] != 1 || nd > 2) {
            fail("tensor " + name + " has shape [" + std::to_string(ne[0]) + ", " + std::to_string(ne[1]) +
                 "], expected [" + std::to_string(ne0) + ", " + std::to_string(ne1) + "]");
            return -1;
        }
        bool ok = false;
        for (int t : types) ok |= t == type;
        if (!ok) {
            fail("tensor " + name + " has unsupported type " + std::string(ggml_type_name((ggml_type) type)));
            return -1;
        }
        return i;
    }
    // an f32 tensor of ne = (n, rows), copied
    bool vec(const std::string & name, int64_t n, std::vector<float> & out, int64_t rows = 1) {
        int type = 0;
        const int64_t i = tensor(name, n, rows, {GGML_TYPE_F32}, type);
        if (i < 0) return false;
        size_t nb = 0;
        const float * p = (const float *) oa_gguf_tensor_data(g, i, &nb);
        out.assign(p, p + n * rows);
        return true;
    }
    bool mat(const std::string & name, int64_t k, int64_t rows, int wtype, blob & out) {
        int type = 0;
        const int64_t i = tensor(name, k, rows, {GGML_TYPE_Q8_0, GGML_TYPE_Q4_K}, type);
        if (i < 0) return false;
        if (type != wtype) return fail("tensor " + name + " is " + ggml_type_name((ggml_type) type) +
                                       ", the pack's matrices are " + ggml_type_name((ggml_type) wtype));
        size_t nb = 0;
        const void * p = oa_gguf_tensor_data(g, i, &nb);
        out.set_view(p, nb);
        return true;
    }
};

}  // namespace oa_pack

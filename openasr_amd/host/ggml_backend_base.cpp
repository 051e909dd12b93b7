// ggml_backend_base.cpp -- backend front end, tensor allocation, graph
// allocator and verified plugin loading of this build's ggml-base.
//
// Mirrors the host-side calls in crates/openasr-core/src/ggml_runtime/ffi.rs
// (buffer / tensor transfer 520-564, gallocr 565-600, device and registry
// 600-628, verified loading 415-434) and the load/probe contract the host
// drives in ggml_runtime/backend.rs:1290-1444: a plugin is accepted only
// when its openasr_ggml_backend_{abi,provider,probe}_v1 exports attest the
// host ABI fingerprint, the provider label and the device target.

#include "ggml_host.h"

#include <dlfcn.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#ifndef OPENASR_HOST_ABI_FINGERPRINT
#define OPENASR_HOST_ABI_FINGERPRINT "unset"
#endif

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct registry_state {
    std::mutex mu;
    std::vector<ggml_backend_reg_t> regs;
    std::vector<void *> handles;  // parallel to regs; null for statically registered
};

registry_state & registry() {
    static registry_state r;
    return r;
}

ggml_backend_buffer_t tensor_buffer(const ggml_tensor * t) { return t->view_src ? t->view_src->buffer : t->buffer; }

}  // namespace

extern "C" {

const char * ggml_backend_host_abi_fingerprint(void) { return OPENASR_HOST_ABI_FINGERPRINT; }

// ---------------------------------------------------------------- buffers --

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void * context, size_t size) {
    ggml_backend_buffer * b = new ggml_backend_buffer;
    b->iface = iface;
    b->buft = buft;
    b->context = context;
    b->size = size;
    b->usage = GGML_BACKEND_BUFFER_USAGE_ANY;
    return b;
}

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) return;
    if (buffer->iface.free_buffer) buffer->iface.free_buffer(buffer);
    delete buffer;
}

void * ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer) {
    if (buffer->size == 0) return nullptr;
    return buffer->iface.get_base(buffer);
}

size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer->size; }

size_t ggml_backend_buffer_get_alignment(ggml_backend_buffer_t buffer) {
    return ggml_backend_buft_get_alignment(buffer->buft);
}

size_t ggml_backend_buffer_get_alloc_size(ggml_backend_buffer_t buffer, const struct ggml_tensor * t) {
    return ggml_backend_buft_get_alloc_size(buffer->buft, t);
}

bool ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer) { return ggml_backend_buft_is_host(buffer->buft); }

void ggml_backend_buffer_set_usage(ggml_backend_buffer_t buffer, enum ggml_backend_buffer_usage usage) {
    buffer->usage = usage;
}

enum ggml_backend_buffer_usage ggml_backend_buffer_get_usage(ggml_backend_buffer_t buffer) { return buffer->usage; }

void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    if (buffer->size == 0) return;
    buffer->iface.clear(buffer, value);
}

ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) { return buffer->buft; }

enum ggml_status ggml_backend_buffer_init_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t) {
    if (buffer->iface.init_tensor) return buffer->iface.init_tensor(buffer, t);
    return GGML_STATUS_SUCCESS;
}

// ----------------------------------------------------------- buffer types --

const char * ggml_backend_buft_name(ggml_backend_buffer_type_t buft) { return buft->iface.get_name(buft); }

ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    return buft->iface.alloc_buffer(buft, size);
}

size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft) { return buft->iface.get_alignment(buft); }

size_t ggml_backend_buft_get_max_size(ggml_backend_buffer_type_t buft) {
    return buft->iface.get_max_size ? buft->iface.get_max_size(buft) : SIZE_MAX;
}

size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor * t) {
    if (buft->iface.get_alloc_size) return buft->iface.get_alloc_size(buft, t);
    return ggml_nbytes(t);
}

bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft) {
    return buft->iface.is_host ? buft->iface.is_host(buft) : false;
}

ggml_backend_dev_t ggml_backend_buft_get_device(ggml_backend_buffer_type_t buft) { return buft->device; }

// ------------------------------------------------------- tensor transfers --

int ggml_backend_tensor_set(struct ggml_tensor * t, const void * data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor_buffer(t);
    if (size == 0) return 0;
    if (!buf || !t->data || offset + size > ggml_nbytes(t) || !buf->iface.set_tensor) return 1;
    buf->iface.set_tensor(buf, t, data, offset, size);
    return 0;
}

int ggml_backend_tensor_get(const struct ggml_tensor * t, void * data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor_buffer(t);
    if (size == 0) return 0;
    if (!buf || !t->data || offset + size > ggml_nbytes(t) || !buf->iface.get_tensor) return 1;
    buf->iface.get_tensor(buf, t, data, offset, size);
    return 0;
}

int ggml_backend_tensor_memset(struct ggml_tensor * t, uint8_t value, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor_buffer(t);
    if (size == 0) return 0;
    if (!buf || !t->data || offset + size > ggml_nbytes(t) || !buf->iface.memset_tensor) return 1;
    buf->iface.memset_tensor(buf, t, value, offset, size);
    return 0;
}

int ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, struct ggml_tensor * t, void * addr) {
    if (t->buffer != nullptr || t->data != nullptr || t->view_src != nullptr) return 1;
    char * base = (char *) ggml_backend_buffer_get_base(buffer);
    if ((char *) addr < base || (char *) addr + ggml_backend_buffer_get_alloc_size(buffer, t) > base + buffer->size)
        return 1;
    t->buffer = buffer;
    t->data = addr;
    return ggml_backend_buffer_init_tensor(buffer, t) == GGML_STATUS_SUCCESS ? 0 : 1;
}

int ggml_backend_view_init(struct ggml_tensor * t) {
    if (!t->view_src || !t->view_src->buffer || !t->view_src->data) return 1;
    t->buffer = t->view_src->buffer;
    t->data = (char *) t->view_src->data + t->view_offs;
    return ggml_backend_buffer_init_tensor(t->buffer, t) == GGML_STATUS_SUCCESS ? 0 : 1;
}

struct ggml_tallocr ggml_tallocr_new(ggml_backend_buffer_t buffer) {
    ggml_tallocr t;
    t.buffer = buffer;
    t.base = ggml_backend_buffer_get_base(buffer);
    t.alignment = ggml_backend_buffer_get_alignment(buffer);
    t.offset = align_up((size_t) t.base, t.alignment) - (size_t) t.base;
    return t;
}

int ggml_tallocr_alloc(struct ggml_tallocr * talloc, struct ggml_tensor * t) {
    const size_t size = align_up(ggml_backend_buffer_get_alloc_size(talloc->buffer, t), talloc->alignment);
    if (talloc->offset + size > ggml_backend_buffer_get_size(talloc->buffer)) return 1;
    void * addr = (char *) talloc->base + talloc->offset;
    talloc->offset += size;
    return ggml_backend_tensor_alloc(talloc->buffer, t, addr);
}

static size_t ctx_unallocated_bytes(ggml_context * ctx, ggml_backend_buffer_type_t buft) {
    const size_t align = ggml_backend_buft_get_alignment(buft);
    size_t total = 0;
    for (ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data == nullptr && t->view_src == nullptr) {
            total += align_up(ggml_backend_buft_get_alloc_size(buft, t), align);
        }
    }
    return total;
}

size_t ggml_backend_alloc_ctx_tensors_from_buft_size(struct ggml_context * ctx, ggml_backend_buffer_type_t buft) {
    return ctx_unallocated_bytes(ctx, buft);
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context * ctx,
                                                               ggml_backend_buffer_type_t buft) {
    const size_t total = ctx_unallocated_bytes(ctx, buft);
    if (total == 0) return nullptr;
    ggml_backend_buffer_t buffer = ggml_backend_buft_alloc_buffer(buft, total);
    if (!buffer) return nullptr;
    ggml_tallocr ta = ggml_tallocr_new(buffer);
    for (ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data == nullptr && t->view_src == nullptr) {
            if (ggml_tallocr_alloc(&ta, t) != 0) {
                ggml_backend_buffer_free(buffer);
                return nullptr;
            }
        }
    }
    for (ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->view_src && t->data == nullptr && t->view_src->data) ggml_backend_view_init(t);
    }
    return buffer;
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context * ctx, ggml_backend_t backend) {
    return ggml_backend_alloc_ctx_tensors_from_buft(ctx, ggml_backend_get_default_buffer_type(backend));
}

// ---------------------------------------------------------------- backend --

const char * ggml_backend_name(ggml_backend_t backend) { return backend ? backend->iface.get_name(backend) : "NULL"; }

void ggml_backend_free(ggml_backend_t backend) {
    if (backend) backend->iface.free(backend);
}

ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend) { return backend->device; }

ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend) {
    return ggml_backend_dev_buffer_type(backend->device);
}

ggml_backend_buffer_t ggml_backend_alloc_buffer(ggml_backend_t backend, size_t size) {
    return ggml_backend_buft_alloc_buffer(ggml_backend_get_default_buffer_type(backend), size);
}

void ggml_backend_synchronize(ggml_backend_t backend) {
    if (backend->iface.synchronize) backend->iface.synchronize(backend);
}

enum ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    return backend->iface.graph_compute(backend, cgraph);
}

enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    enum ggml_status st = ggml_backend_graph_compute_async(backend, cgraph);
    ggml_backend_synchronize(backend);
    return st;
}

static void * backend_proc(ggml_backend_t backend, const char * name) {
    if (!backend->device || !backend->device->reg) return nullptr;
    return ggml_backend_reg_get_proc_address(backend->device->reg, name);
}

// Cooperative cancellation (docs/design/graph-cancellation.md:9-35): a backend
// with a native abort hook gets the callback for this compute only; otherwise
// the graph runs in synchronized views of at most 32 nodes, polling between.
enum ggml_status ggml_backend_graph_compute_with_abort(ggml_backend_t backend, struct ggml_cgraph * cgraph,
                                                       ggml_abort_callback abort_callback,
                                                       void * abort_callback_data,
                                                       struct ggml_backend_graph_cancel_capability * cap) {
    if (cap) {
        cap->mechanism = GGML_BACKEND_GRAPH_CANCEL_DISABLED;
        cap->observation_granularity = GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_NONE;
    }
    if (!abort_callback) return ggml_backend_graph_compute(backend, cgraph);
    auto set_cb = (ggml_backend_set_abort_callback_t) backend_proc(backend, "ggml_backend_set_abort_callback");
    if (set_cb) {
        auto get_obs = (ggml_backend_get_cancel_observation_t) backend_proc(backend,
                                                                             "ggml_backend_get_cancel_observation");
        set_cb(backend, abort_callback, abort_callback_data);
        enum ggml_status st = ggml_backend_graph_compute(backend, cgraph);
        set_cb(backend, nullptr, nullptr);
        if (cap) {
            cap->mechanism = GGML_BACKEND_GRAPH_CANCEL_NATIVE;
            cap->observation_granularity =
                get_obs ? get_obs(backend) : GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_SUBMISSION_CHECKPOINT;
        }
        return st;
    }
    if (cap) {
        cap->mechanism = GGML_BACKEND_GRAPH_CANCEL_SEGMENTED;
        cap->observation_granularity = GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_SUBMISSION_CHECKPOINT;
    }
    const int kSegment = 32;
    for (int start = 0; start < cgraph->n_nodes; start += kSegment) {
        if (abort_callback(abort_callback_data)) return GGML_STATUS_ABORTED;
        ggml_cgraph view = *cgraph;
        view.nodes = cgraph->nodes + start;
        view.n_nodes = cgraph->n_nodes - start < kSegment ? cgraph->n_nodes - start : kSegment;
        view.n_leafs = 0;
        enum ggml_status st = ggml_backend_graph_compute(backend, &view);
        if (st != GGML_STATUS_SUCCESS) return st;
    }
    return abort_callback(abort_callback_data) ? GGML_STATUS_ABORTED : GGML_STATUS_SUCCESS;
}

bool ggml_backend_supports_op(ggml_backend_t backend, const struct ggml_tensor * op) {
    return ggml_backend_dev_supports_op(backend->device, op);
}

// ---------------------------------------------------------------- devices --

const char * ggml_backend_dev_name(ggml_backend_dev_t dev) { return dev->iface.get_name(dev); }
const char * ggml_backend_dev_description(ggml_backend_dev_t dev) { return dev->iface.get_description(dev); }
void ggml_backend_dev_memory(ggml_backend_dev_t dev, size_t * free, size_t * total) {
    dev->iface.get_memory(dev, free, total);
}
enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t dev) { return dev->iface.get_type(dev); }
void ggml_backend_dev_get_props(ggml_backend_dev_t dev, struct ggml_backend_dev_props * props) {
    std::memset(props, 0, sizeof(*props));
    dev->iface.get_props(dev, props);
}
ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t dev) { return dev->reg; }
ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t dev, const char * params) {
    return dev->iface.init_backend(dev, params);
}
ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t dev) {
    return dev->iface.get_buffer_type(dev);
}
ggml_backend_buffer_type_t ggml_backend_dev_host_buffer_type(ggml_backend_dev_t dev) {
    return dev->iface.get_host_buffer_type ? dev->iface.get_host_buffer_type(dev) : nullptr;
}
ggml_backend_buffer_t ggml_backend_dev_buffer_from_host_ptr(ggml_backend_dev_t dev, void * ptr, size_t size,
                                                            size_t max_tensor_size) {
    return dev->iface.buffer_from_host_ptr ? dev->iface.buffer_from_host_ptr(dev, ptr, size, max_tensor_size)
                                           : nullptr;
}
bool ggml_backend_dev_supports_op(ggml_backend_dev_t dev, const struct ggml_tensor * op) {
    return dev->iface.supports_op(dev, op);
}
bool ggml_backend_dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft) {
    return dev->iface.supports_buft(dev, buft);
}
bool ggml_backend_dev_offload_op(ggml_backend_dev_t dev, const struct ggml_tensor * op) {
    return dev->iface.offload_op ? dev->iface.offload_op(dev, op) : false;
}

// --------------------------------------------------------------- registry --

const char * ggml_backend_reg_name(ggml_backend_reg_t reg) { return reg->iface.get_name(reg); }
size_t ggml_backend_reg_dev_count(ggml_backend_reg_t reg) { return reg->iface.get_device_count(reg); }
ggml_backend_dev_t ggml_backend_reg_dev_get(ggml_backend_reg_t reg, size_t index) {
    return reg->iface.get_device(reg, index);
}
void * ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char * name) {
    return reg->iface.get_proc_address ? reg->iface.get_proc_address(reg, name) : nullptr;
}

static void register_with_handle(ggml_backend_reg_t reg, void * handle) {
    registry_state & r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    for (ggml_backend_reg_t existing : r.regs) {
        if (existing == reg) return;
    }
    r.regs.push_back(reg);
    r.handles.push_back(handle);
}

void ggml_backend_register(ggml_backend_reg_t reg) { register_with_handle(reg, nullptr); }

size_t ggml_backend_reg_count(void) {
    registry_state & r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    return r.regs.size();
}

ggml_backend_reg_t ggml_backend_reg_get(size_t index) {
    registry_state & r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    return index < r.regs.size() ? r.regs[index] : nullptr;
}

size_t ggml_backend_dev_count(void) {
    size_t n = 0;
    for (size_t i = 0; i < ggml_backend_reg_count(); i++) n += ggml_backend_reg_dev_count(ggml_backend_reg_get(i));
    return n;
}

ggml_backend_dev_t ggml_backend_dev_get(size_t index) {
    for (size_t i = 0; i < ggml_backend_reg_count(); i++) {
        ggml_backend_reg_t reg = ggml_backend_reg_get(i);
        const size_t n = ggml_backend_reg_dev_count(reg);
        if (index < n) return ggml_backend_reg_dev_get(reg, index);
        index -= n;
    }
    return nullptr;
}

ggml_backend_t ggml_backend_init_by_type(enum ggml_backend_dev_type type, const char * params) {
    for (size_t i = 0; i < ggml_backend_dev_count(); i++) {
        ggml_backend_dev_t dev = ggml_backend_dev_get(i);
        if (ggml_backend_dev_type(dev) == type) return ggml_backend_dev_init(dev, params);
    }
    return nullptr;
}

ggml_backend_t ggml_backend_init_best(void) {
    ggml_backend_t b = ggml_backend_init_by_type(GGML_BACKEND_DEVICE_TYPE_GPU, nullptr);
    return b ? b : ggml_backend_init_by_type(GGML_BACKEND_DEVICE_TYPE_CPU, nullptr);
}

typedef const char * (*openasr_abi_fn)(void);
typedef const char * (*openasr_provider_fn)(void);
typedef bool (*openasr_probe_fn)(const char * device_target, const char * minimum_driver, char * driver_out,
                                 size_t driver_out_capacity);

namespace {

// Opens the plugin and checks its attestation exports. On success returns the
// dlopen handle (caller owns it); on any mismatch closes it and returns null.
void * open_attested(const char * path, const char * abi, const char * provider, const char * target,
                     const char * min_driver, char * driver_out, size_t driver_cap) {
    if (!path) return nullptr;
    void * h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        std::fprintf(stderr, "ggml-base: cannot load %s: %s\n", path, dlerror());
        return nullptr;
    }
    auto abi_fn = (openasr_abi_fn) dlsym(h, "openasr_ggml_backend_abi_v1");
    auto prov_fn = (openasr_provider_fn) dlsym(h, "openasr_ggml_backend_provider_v1");
    auto probe_fn = (openasr_probe_fn) dlsym(h, "openasr_ggml_backend_probe_v1");
    auto init_fn = dlsym(h, "ggml_backend_init");
    bool ok = abi_fn && prov_fn && probe_fn && init_fn;
    if (ok && abi && std::strcmp(abi_fn(), abi) != 0) {
        std::fprintf(stderr, "ggml-base: %s attests ABI %s, host expects %s\n", path, abi_fn(), abi);
        ok = false;
    }
    if (ok && provider && std::strcmp(prov_fn(), provider) != 0) {
        std::fprintf(stderr, "ggml-base: %s provides '%s', host expects '%s'\n", path, prov_fn(), provider);
        ok = false;
    }
    char local[64];
    if (!driver_out) {
        driver_out = local;
        driver_cap = sizeof(local);
    }
    if (ok && !probe_fn(target ? target : "", min_driver ? min_driver : "", driver_out, driver_cap)) {
        std::fprintf(stderr, "ggml-base: %s probe failed for target '%s'\n", path, target ? target : "");
        ok = false;
    }
    if (!ok) {
        dlclose(h);
        return nullptr;
    }
    return h;
}

}  // namespace

bool ggml_backend_probe_verified_v3_utf8(const char * path_utf8, const char * const * dependency_dirs_utf8,
                                         size_t dependency_dir_count, const char * expected_openasr_abi_v1,
                                         const char * expected_provider_v1, const char * expected_device_target,
                                         const char * minimum_driver_version, char * driver_out,
                                         size_t driver_out_capacity) {
    (void) dependency_dirs_utf8;
    (void) dependency_dir_count;
    if (driver_out && driver_out_capacity) driver_out[0] = '\0';
    void * h = open_attested(path_utf8, expected_openasr_abi_v1, expected_provider_v1, expected_device_target,
                             minimum_driver_version, driver_out, driver_out_capacity);
    if (!h) return false;
    dlclose(h);
    return driver_out == nullptr || driver_out[0] != '\0';
}

ggml_backend_reg_t ggml_backend_load_verified_v3_utf8(const char * path_utf8, const char * const * dependency_dirs_utf8,
                                                      size_t dependency_dir_count,
                                                      const char * expected_openasr_abi_v1,
                                                      const char * expected_provider_v1,
                                                      const char * expected_device_target,
                                                      const char * minimum_driver_version) {
    (void) dependency_dirs_utf8;
    (void) dependency_dir_count;
    void * h = open_attested(path_utf8, expected_openasr_abi_v1, expected_provider_v1, expected_device_target,
                             minimum_driver_version, nullptr, 0);
    if (!h) return nullptr;
    auto init_fn = (ggml_backend_init_t) dlsym(h, "ggml_backend_init");
    ggml_backend_reg_t reg = init_fn();
    if (!reg || reg->api_version != GGML_BACKEND_API_VERSION) {
        std::fprintf(stderr, "ggml-base: %s registry API version mismatch\n", path_utf8);
        dlclose(h);
        return nullptr;
    }
    register_with_handle(reg, h);
    return reg;
}

ggml_backend_reg_t ggml_backend_load(const char * path) {
    return ggml_backend_load_verified_v3_utf8(path, nullptr, 0, OPENASR_HOST_ABI_FINGERPRINT, nullptr, nullptr,
                                              nullptr);
}

void ggml_backend_unload(ggml_backend_reg_t reg) {
    registry_state & r = registry();
    void * handle = nullptr;
    {
        std::lock_guard<std::mutex> lock(r.mu);
        for (size_t i = 0; i < r.regs.size(); i++) {
            if (r.regs[i] == reg) {
                handle = r.handles[i];
                r.regs.erase(r.regs.begin() + (long) i);
                r.handles.erase(r.handles.begin() + (long) i);
                break;
            }
        }
    }
    // The plugin keeps device state for the life of the process (HIP contexts
    // cannot be torn down safely while other threads may hold streams), so the
    // module stays mapped; only the registry entry is removed.
    (void) handle;
}

// -------------------------------------------------------- graph allocator --

struct ggml_gallocr {
    ggml_backend_buffer_type_t buft;
    ggml_backend_buffer_t buffer;
};

ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft) {
    ggml_gallocr * g = new ggml_gallocr;
    g->buft = buft;
    g->buffer = nullptr;
    return g;
}

void ggml_gallocr_free(ggml_gallocr_t galloc) {
    if (!galloc) return;
    ggml_backend_buffer_free(galloc->buffer);
    delete galloc;
}

size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t galloc, int buffer_id) {
    (void) buffer_id;
    return galloc->buffer ? ggml_backend_buffer_get_size(galloc->buffer) : 0;
}

// Every graph tensor without storage gets its own slot in one buffer (no
// lifetime-based reuse: an MI355X holds 288 GB and the decoder graphs here
// need at most a few GB of intermediates). The buffer is kept and reused
// while the next graph fits.
bool ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph * graph) {
    const size_t align = ggml_backend_buft_get_alignment(galloc->buft);
    std::vector<ggml_tensor *> todo;
    auto consider = [&](ggml_tensor * t) {
        if (t && t->data == nullptr && t->view_src == nullptr) {
            for (ggml_tensor * seen : todo) {
                if (seen == t) return;
            }
            todo.push_back(t);
        }
    };
    for (int i = 0; i < graph->n_leafs; i++) consider(graph->leafs[i]);
    for (int i = 0; i < graph->n_nodes; i++) {
        for (int s = 0; s < GGML_MAX_SRC; s++) consider(graph->nodes[i]->src[s]);
        // a view node whose base is not a graph node (set_rows into a cache
        // tensor of the same context) still needs the base to have storage
        consider(graph->nodes[i]->view_src);
        consider(graph->nodes[i]);
    }
    size_t total = 0;
    for (ggml_tensor * t : todo) total += align_up(ggml_backend_buft_get_alloc_size(galloc->buft, t), align);
    if (total == 0) total = align;
    if (!galloc->buffer || ggml_backend_buffer_get_size(galloc->buffer) < total) {
        ggml_backend_buffer_free(galloc->buffer);
        galloc->buffer = ggml_backend_buft_alloc_buffer(galloc->buft, total);
        if (!galloc->buffer) return false;
        ggml_backend_buffer_set_usage(galloc->buffer, GGML_BACKEND_BUFFER_USAGE_COMPUTE);
    }
    ggml_tallocr ta = ggml_tallocr_new(galloc->buffer);
    for (ggml_tensor * t : todo) {
        if (ggml_tallocr_alloc(&ta, t) != 0) return false;
    }
    auto init_view = [](ggml_tensor * t) {
        if (t && t->view_src && t->data == nullptr && t->view_src->data) ggml_backend_view_init(t);
    };
    for (int i = 0; i < graph->n_leafs; i++) init_view(graph->leafs[i]);
    for (int i = 0; i < graph->n_nodes; i++) {
        for (int s = 0; s < GGML_MAX_SRC; s++) init_view(graph->nodes[i]->src[s]);
        init_view(graph->nodes[i]);
    }
    return true;
}

}  // extern "C"

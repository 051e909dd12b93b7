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
#include <unordered_map>
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

// ------------------------------------------------------ host buffer type --
// Plain host memory (ggml-base's CPU buffer type): what a graph allocated
// without a device runs in, e.g. to inspect an allocation plan on a machine
// with no GPU.

namespace {

void hostbuf_free(ggml_backend_buffer_t b) {
    std::free(b->context);
}
void * hostbuf_base(ggml_backend_buffer_t b) { return b->context; }
void hostbuf_memset(ggml_backend_buffer_t, struct ggml_tensor * t, uint8_t v, size_t off, size_t n) {
    std::memset((char *) t->data + off, v, n);
}
void hostbuf_set(ggml_backend_buffer_t, struct ggml_tensor * t, const void * d, size_t off, size_t n) {
    std::memcpy((char *) t->data + off, d, n);
}
void hostbuf_get(ggml_backend_buffer_t, const struct ggml_tensor * t, void * d, size_t off, size_t n) {
    std::memcpy(d, (const char *) t->data + off, n);
}
void hostbuf_clear(ggml_backend_buffer_t b, uint8_t v) { std::memset(b->context, v, b->size); }

const char * hostbuft_name(ggml_backend_buffer_type_t) { return "CPU"; }
ggml_backend_buffer_t hostbuft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    const size_t n = align_up(size ? size : 64, 64);
    void * p = std::aligned_alloc(64, n);
    if (!p) return nullptr;
    static const ggml_backend_buffer_i iface = {hostbuf_free, hostbuf_base, nullptr, hostbuf_memset,
                                                hostbuf_set, hostbuf_get, nullptr, hostbuf_clear, nullptr};
    return ggml_backend_buffer_init(buft, iface, p, size);
}
size_t hostbuft_align(ggml_backend_buffer_type_t) { return 64; }
size_t hostbuft_max(ggml_backend_buffer_type_t) { return SIZE_MAX; }
size_t hostbuft_alloc_size(ggml_backend_buffer_type_t, const struct ggml_tensor * t) { return ggml_nbytes(t); }
bool hostbuft_is_host(ggml_backend_buffer_type_t) { return true; }

}  // namespace

ggml_backend_buffer_type_t ggml_backend_cpu_buffer_type(void) {
    static ggml_backend_buffer_type buft = {
        {hostbuft_name, hostbuft_alloc, hostbuft_align, hostbuft_max, hostbuft_alloc_size, hostbuft_is_host},
        nullptr, nullptr};
    return &buft;
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

// Graph allocation by lifetime, as ggml-alloc does it (the allocator the
// host's graph runner uses, reached through ggml_gallocr_alloc_graph,
// crates/openasr-core/src/ggml_runtime/ffi.rs): every node counts its
// consumers and the views of it; inputs are placed first and live for the
// whole graph; each node then takes a block, or -- when its op can run in
// place and a source of the same layout has no other consumer and no view --
// that source's block; a source's block returns to the free list when its
// last consumer has been placed (outputs and inputs are never freed). Blocks
// are carved best-fit from one buffer whose size is the high-water mark of
// the walk; adjacent free blocks merge.
namespace {

bool op_can_inplace(enum ggml_op op) {
    switch (op) {
        case GGML_OP_SCALE:
        case GGML_OP_ADD:
        case GGML_OP_SUB:
        case GGML_OP_MUL:
        case GGML_OP_DIV:
        case GGML_OP_UNARY:
        case GGML_OP_ROPE:
        case GGML_OP_RMS_NORM:
        case GGML_OP_SOFT_MAX:
            return true;
        default:
            return false;
    }
}

bool same_layout(const ggml_tensor * a, const ggml_tensor * b) {
    if (a->type != b->type) return false;
    for (int d = 0; d < GGML_MAX_DIMS; d++)
        if (a->ne[d] != b->ne[d] || a->nb[d] != b->nb[d]) return false;
    return true;
}

struct block_pool {
    struct blk {
        size_t off, size;
    };
    std::vector<blk> free_list;  // sorted by offset, disjoint, merged
    size_t top = 0;              // end of the highest block ever used

    size_t alloc(size_t size) {
        int best = -1;
        for (int k = 0; k < (int) free_list.size(); k++) {
            if (free_list[(size_t) k].size >= size &&
                (best < 0 || free_list[(size_t) k].size < free_list[(size_t) best].size))
                best = k;
        }
        if (best >= 0) {
            blk & b = free_list[(size_t) best];
            const size_t off = b.off;
            b.off += size;
            b.size -= size;
            if (b.size == 0) free_list.erase(free_list.begin() + best);
            return off;
        }
        // grow: a free block at the end is extended
        if (!free_list.empty() && free_list.back().off + free_list.back().size == top) {
            const size_t off = free_list.back().off;
            top = off + size;
            free_list.pop_back();
            return off;
        }
        const size_t off = top;
        top += size;
        return off;
    }

    void release(size_t off, size_t size) {
        size_t k = 0;
        while (k < free_list.size() && free_list[k].off < off) k++;
        free_list.insert(free_list.begin() + (long) k, blk{off, size});
        if (k + 1 < free_list.size() && free_list[k].off + free_list[k].size == free_list[k + 1].off) {
            free_list[k].size += free_list[k + 1].size;
            free_list.erase(free_list.begin() + (long) k + 1);
        }
        if (k > 0 && free_list[k - 1].off + free_list[k - 1].size == free_list[k].off) {
            free_list[k - 1].size += free_list[k].size;
            free_list.erase(free_list.begin() + (long) k);
        }
    }
};

struct galloc_plan {
    struct info {
        int n_children = 0, n_views = 0;
        bool own = false;        // placed by this allocator
        bool pinned = false;     // an output, or the base of an output view: never freed or taken over
        bool allocated = false;  // holds a block that will be freed at last use
        size_t off = 0, size = 0;
    };
    std::unordered_map<const ggml_tensor *, info> tab;
    std::vector<ggml_tensor *> order;  // tensors placed, in placement order
    block_pool pool;
    size_t align = 256;
    ggml_backend_buffer_type_t buft = nullptr;

    info & at(const ggml_tensor * t) { return tab[t]; }

    void place(ggml_tensor * t) {
        info & in = at(t);
        if (in.own || t->data || t->view_src) return;
        in.own = true;
        in.size = align_up(ggml_backend_buft_get_alloc_size(buft, t), align);
        if (in.size == 0) in.size = align;
        order.push_back(t);
        if (op_can_inplace(t->op) && !(t->flags & GGML_TENSOR_FLAG_INPUT)) {
            for (int s = 0; s < GGML_MAX_SRC; s++) {
                ggml_tensor * p = t->src[s];
                if (!p) continue;
                const bool view = p->view_src != nullptr;
                ggml_tensor * base = view ? p->view_src : p;
                info & pb = at(base);
                info & pi = at(p);
                if (!pb.own || !pb.allocated) continue;
                if ((base->flags & (GGML_TENSOR_FLAG_OUTPUT | GGML_TENSOR_FLAG_INPUT)) ||
                    (p->flags & GGML_TENSOR_FLAG_OUTPUT) || pb.pinned)
                    continue;
                if (!same_layout(t, p) || pi.n_children != 1 || pi.n_views != 0) continue;
                if (view && (pb.n_views != 1 || pb.n_children != 0 || p->view_offs != 0)) continue;
                if (pb.size < in.size) continue;
                // take over the source's block
                in.off = pb.off;
                in.size = pb.size;
                in.allocated = true;
                pb.allocated = false;
                return;
            }
        }
        in.off = pool.alloc(in.size);
        in.allocated = true;
    }

    void release_if_dead(const ggml_tensor * t) {
        info & in = at(t);
        if (!in.own || !in.allocated) return;
        if (in.n_children != 0 || in.n_views != 0) return;
        if ((t->flags & (GGML_TENSOR_FLAG_OUTPUT | GGML_TENSOR_FLAG_INPUT)) || in.pinned) return;
        pool.release(in.off, in.size);
        in.allocated = false;
    }

    void run(ggml_cgraph * g) {
        for (int i = 0; i < g->n_nodes; i++) {
            ggml_tensor * n = g->nodes[i];
            if (n->view_src) {
                at(n->view_src).n_views++;
                if (n->flags & GGML_TENSOR_FLAG_OUTPUT) at(n->view_src).pinned = true;
            }
            for (int s = 0; s < GGML_MAX_SRC; s++)
                if (n->src[s]) at(n->src[s]).n_children++;
        }
        // inputs first: they hold what the host sets before the compute
        for (int i = 0; i < g->n_leafs; i++)
            if (g->leafs[i]->flags & GGML_TENSOR_FLAG_INPUT) place(g->leafs[i]);
        for (int i = 0; i < g->n_nodes; i++) {
            ggml_tensor * n = g->nodes[i];
            if (n->flags & GGML_TENSOR_FLAG_INPUT) place(n);
            for (int s = 0; s < GGML_MAX_SRC; s++)
                if (n->src[s] && (n->src[s]->flags & GGML_TENSOR_FLAG_INPUT)) place(n->src[s]);
        }
        for (int i = 0; i < g->n_nodes; i++) {
            ggml_tensor * n = g->nodes[i];
            // sources not placed yet (leafs: constants of the graph) live on
            for (int s = 0; s < GGML_MAX_SRC; s++) {
                ggml_tensor * p = n->src[s];
                if (p && !p->data && !p->view_src && !at(p).own) {
                    place(p);
                    at(p).allocated = false;  // never freed
                }
            }
            if (n->view_src && !n->view_src->data && !at(n->view_src).own) {
                place(n->view_src);
                at(n->view_src).allocated = false;
            }
            place(n);
            for (int s = 0; s < GGML_MAX_SRC; s++) {
                ggml_tensor * p = n->src[s];
                if (!p) continue;
                info & pi = at(p);
                pi.n_children--;
                if (pi.n_children != 0 || pi.n_views != 0) continue;
                if (p->view_src) {
                    info & vb = at(p->view_src);
                    vb.n_views--;
                    release_if_dead(p->view_src);
                } else {
                    release_if_dead(p);
                }
            }
        }
        // leafs the nodes never read (kept by the host for later graphs)
        for (int i = 0; i < g->n_leafs; i++) {
            ggml_tensor * l = g->leafs[i];
            if (!l->data && !l->view_src && !at(l).own) {
                place(l);
                at(l).allocated = false;
            }
        }
    }
};

}  // namespace

bool ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph * graph) {
    galloc_plan plan;
    plan.align = ggml_backend_buft_get_alignment(galloc->buft);
    plan.buft = galloc->buft;
    plan.run(graph);
    size_t total = align_up(plan.pool.top, plan.align);
    if (total == 0) total = plan.align;
    if (!galloc->buffer || ggml_backend_buffer_get_size(galloc->buffer) < total) {
        ggml_backend_buffer_free(galloc->buffer);
        galloc->buffer = ggml_backend_buft_alloc_buffer(galloc->buft, total);
        if (!galloc->buffer) return false;
        ggml_backend_buffer_set_usage(galloc->buffer, GGML_BACKEND_BUFFER_USAGE_COMPUTE);
    }
    char * base = (char *) ggml_backend_buffer_get_base(galloc->buffer);
    for (ggml_tensor * t : plan.order) {
        if (ggml_backend_tensor_alloc(galloc->buffer, t, base + plan.at(t).off) != 0) return false;
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

// mi355x_backend.cpp -- the ggml backend plugin for MI355X (gfx950): registry,
// device, buffer type, buffer and backend vtables (ggml-backend-impl.h, API
// version 3), plus the OpenASR attestation exports the verified loader checks
// before it calls ggml_backend_init (.github/workflows/release-binaries.yml:
// 823-835; loader: crates/openasr-core/src/ggml_runtime/backend.rs:1290-1444).
//
// Device memory is plain hipMalloc'd HBM. Q8_0 tensors are stored row-split
// ([quants][scales] per row) and converted in set/get_tensor, so the host
// always sees ggml's byte layout.

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ggml_backend_memory.h"
#include "ggml_host.h"
#include "ggml_mi355x.h"
#include "mi355x_exec.h"
#include "ops.h"

#ifndef OPENASR_HOST_ABI_FINGERPRINT
#define OPENASR_HOST_ABI_FINGERPRINT "unset"
#endif

namespace mi355x {

static thread_local std::atomic<int> * tl_error_sink = nullptr;

void note_hip_error(hipError_t err) {
    if (err == hipSuccess || !tl_error_sink) return;
    int expected = 0;
    tl_error_sink->compare_exchange_strong(expected, (int) err);
}

error_scope::error_scope(std::atomic<int> * sink) : prev_(tl_error_sink) { tl_error_sink = sink; }
error_scope::~error_scope() { tl_error_sink = prev_; }

struct registry_ctx {
    std::once_flag once;
    std::vector<device_state *> devices;
    ggml_backend_reg reg{};
};

static registry_ctx & reg_ctx() {
    static registry_ctx r;
    return r;
}

// ------------------------------------------------------- Q8_0 conversion --

void q8_0_to_split_rows(const uint8_t * src, uint8_t * dst, int64_t rows, int64_t k) {
    const int64_t nb = k / 32;
    const size_t rb = q8_0_row_bytes(k);
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t * s = src + (size_t) r * rb;
        uint8_t * q = dst + (size_t) r * rb;
        uint8_t * d = q + k;
        for (int64_t b = 0; b < nb; b++) {
            std::memcpy(d + 2 * b, s + 34 * b, 2);
            std::memcpy(q + 32 * b, s + 34 * b + 2, 32);
        }
    }
}

void q8_0_from_split_rows(const uint8_t * src, uint8_t * dst, int64_t rows, int64_t k) {
    const int64_t nb = k / 32;
    const size_t rb = q8_0_row_bytes(k);
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t * q = src + (size_t) r * rb;
        const uint8_t * d = q + k;
        uint8_t * o = dst + (size_t) r * rb;
        for (int64_t b = 0; b < nb; b++) {
            std::memcpy(o + 34 * b, d + 2 * b, 2);
            std::memcpy(o + 34 * b + 2, q + 32 * b, 32);
        }
    }
}

// --------------------------------------------------------------- buffers --

struct buffer_ctx {
    device_state * dev;
    char * base;
    size_t size;
};

static void buf_free(ggml_backend_buffer_t buffer) {
    buffer_ctx * c = (buffer_ctx *) buffer->context;
    error_scope scope(&c->dev->transfer_error);
    MI_CHECK(hipSetDevice(c->dev->hip_id));
    flush_uploads(c->dev, nullptr, true);  // queued writes into this buffer land before it is freed
    MI_CHECK(hipFree(c->base));
    ledger_sub(c->dev, c->size, false);
    delete c;
}

static void * buf_get_base(ggml_backend_buffer_t buffer) { return ((buffer_ctx *) buffer->context)->base; }

static enum ggml_status buf_init_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t) {
    (void) buffer;
    (void) t;
    return GGML_STATUS_SUCCESS;
}

static void buf_set_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t, const void * data, size_t offset,
                           size_t size);

static void buf_memset_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t, uint8_t value, size_t offset,
                              size_t size) {
    buffer_ctx * c = (buffer_ctx *) buffer->context;
    error_scope scope(&c->dev->transfer_error);
    MI_CHECK(hipSetDevice(c->dev->hip_id));
    flush_uploads(c->dev, nullptr, true);
    if (t->type == GGML_TYPE_Q8_0) {
        // stored row-split on the device: ggml-layout bytes go through the
        // same row conversion as set_tensor
        std::vector<uint8_t> bytes(size, value);
        buf_set_tensor(buffer, t, bytes.data(), offset, size);
        return;
    }
    MI_CHECK(hipMemset((char *) t->data + offset, value, size));
}

// Q8_0 transfers work on whole rows; a partial-row range is widened to the
// rows it touches (read-modify-write through the host).
static bool q8_0_rows(const ggml_tensor * t, size_t offset, size_t size, int64_t & r0, int64_t & r1, size_t & rb) {
    rb = q8_0_row_bytes(t->ne[0]);
    if ((size_t) t->nb[1] != rb) return false;
    r0 = (int64_t) (offset / rb);
    r1 = (int64_t) ((offset + size + rb - 1) / rb);
    return true;
}

static void buf_set_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t, const void * data, size_t offset,
                           size_t size) {
    buffer_ctx * c = (buffer_ctx *) buffer->context;
    error_scope scope(&c->dev->transfer_error);
    MI_CHECK(hipSetDevice(c->dev->hip_id));
    if (t->type != GGML_TYPE_Q8_0) {
        // small writes wait in pinned memory for the next device use
        if (stage_upload(c->dev, (char *) t->data + offset, data, size)) return;
        flush_uploads(c->dev, nullptr, true);
        MI_CHECK(hipMemcpy((char *) t->data + offset, data, size, hipMemcpyHostToDevice));
        return;
    }
    flush_uploads(c->dev, nullptr, true);
    int64_t r0, r1;
    size_t rb;
    if (!q8_0_rows(t, offset, size, r0, r1, rb)) {
        std::fprintf(stderr, "mi355x: Q8_0 tensor '%s' has non-packed rows\n", t->name);
        note_hip_error(hipErrorInvalidValue);
        return;
    }
    const size_t span = (size_t) (r1 - r0) * rb;
    std::vector<uint8_t> ggml_rows(span), split(span);
    char * dev_rows = (char *) t->data + (size_t) r0 * rb;
    if (offset != (size_t) r0 * rb || size != span) {
        MI_CHECK(hipMemcpy(split.data(), dev_rows, span, hipMemcpyDeviceToHost));
        q8_0_from_split_rows(split.data(), ggml_rows.data(), r1 - r0, t->ne[0]);
    }
    std::memcpy(ggml_rows.data() + (offset - (size_t) r0 * rb), data, size);
    q8_0_to_split_rows(ggml_rows.data(), split.data(), r1 - r0, t->ne[0]);
    MI_CHECK(hipMemcpy(dev_rows, split.data(), span, hipMemcpyHostToDevice));
}

static void buf_get_tensor(ggml_backend_buffer_t buffer, const struct ggml_tensor * t, void * data, size_t offset,
                           size_t size) {
    buffer_ctx * c = (buffer_ctx *) buffer->context;
    error_scope scope(&c->dev->transfer_error);
    MI_CHECK(hipSetDevice(c->dev->hip_id));
    flush_uploads(c->dev, nullptr, true);
    if (t->type != GGML_TYPE_Q8_0) {
        MI_CHECK(hipMemcpy(data, (const char *) t->data + offset, size, hipMemcpyDeviceToHost));
        return;
    }
    int64_t r0, r1;
    size_t rb;
    if (!q8_0_rows(t, offset, size, r0, r1, rb)) {
        std::fprintf(stderr, "mi355x: Q8_0 tensor '%s' has non-packed rows\n", t->name);
        note_hip_error(hipErrorInvalidValue);
        return;
    }
    const size_t span = (size_t) (r1 - r0) * rb;
    std::vector<uint8_t> split(span), ggml_rows(span);
    MI_CHECK(hipMemcpy(split.data(), (const char *) t->data + (size_t) r0 * rb, span, hipMemcpyDeviceToHost));
    q8_0_from_split_rows(split.data(), ggml_rows.data(), r1 - r0, t->ne[0]);
    std::memcpy(data, ggml_rows.data() + (offset - (size_t) r0 * rb), size);
}

static const char * buft_get_name(ggml_backend_buffer_type_t buft);

static bool buf_cpy_tensor(ggml_backend_buffer_t buffer, const struct ggml_tensor * src, struct ggml_tensor * dst) {
    ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    if (!sb || sb->buft->iface.get_name != buft_get_name) return false;
    buffer_ctx * c = (buffer_ctx *) buffer->context;
    error_scope scope(&c->dev->transfer_error);
    MI_CHECK(hipSetDevice(c->dev->hip_id));
    flush_uploads(c->dev, nullptr, true);
    MI_CHECK(hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice));
    return true;
}

static void buf_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    buffer_ctx * c = (buffer_ctx *) buffer->context;
    error_scope scope(&c->dev->transfer_error);
    MI_CHECK(hipSetDevice(c->dev->hip_id));
    flush_uploads(c->dev, nullptr, true);
    MI_CHECK(hipMemset(c->base, value, c->size));
}

static const ggml_backend_buffer_i kBufferIface = {
    buf_free, buf_get_base, buf_init_tensor, buf_memset_tensor, buf_set_tensor,
    buf_get_tensor, buf_cpy_tensor, buf_clear, nullptr,
};

// ---------------------------------------------------------- buffer type ---

static const char * buft_get_name(ggml_backend_buffer_type_t buft) {
    return ((device_state *) buft->context)->name.c_str();
}

static ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    device_state * dev = (device_state *) buft->context;
    MI_CHECK(hipSetDevice(dev->hip_id));
    void * p = nullptr;
    const size_t alloc = std::max<size_t>(size, 256);
    if (hipMalloc(&p, alloc) != hipSuccess) {
        (void) hipGetLastError();
        ledger_failure(dev);
        std::fprintf(stderr, "mi355x: cannot allocate %zu bytes on %s\n", size, dev->name.c_str());
        return nullptr;
    }
    ledger_add(dev, alloc, false);
    buffer_ctx * c = new buffer_ctx{dev, (char *) p, alloc};
    return ggml_backend_buffer_init(buft, kBufferIface, c, size);
}

static size_t buft_get_alignment(ggml_backend_buffer_type_t) { return 256; }
static size_t buft_get_max_size(ggml_backend_buffer_type_t buft) {
    return ((device_state *) buft->context)->total_mem;
}
static size_t buft_get_alloc_size(ggml_backend_buffer_type_t, const struct ggml_tensor * t) { return ggml_nbytes(t); }
static bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

static const ggml_backend_buffer_type_i kBuftIface = {
    buft_get_name, buft_alloc_buffer, buft_get_alignment, buft_get_max_size, buft_get_alloc_size, buft_is_host,
};

// --------------------------------------------------------------- backend --

static const char * be_get_name(ggml_backend_t backend) {
    return ((backend_state *) backend->context)->name.c_str();
}

static void be_free(ggml_backend_t backend) {
    backend_state * be = (backend_state *) backend->context;
    MI_CHECK(hipSetDevice(be->dev->hip_id));
    release_scratch(be);
    MI_CHECK(hipStreamDestroy(be->stream));
    delete be;
}

static void be_set_tensor_async(ggml_backend_t backend, struct ggml_tensor * t, const void * data, size_t offset,
                                size_t size) {
    (void) backend;
    ggml_backend_tensor_set(t, data, offset, size);
}

static void be_get_tensor_async(ggml_backend_t backend, const struct ggml_tensor * t, void * data, size_t offset,
                                size_t size) {
    (void) backend;
    ggml_backend_tensor_get(t, data, offset, size);
}

static void be_synchronize(ggml_backend_t backend) {
    backend_state * be = (backend_state *) backend->context;
    MI_CHECK(hipSetDevice(be->dev->hip_id));
    flush_uploads(be->dev, be->stream, false);
    MI_CHECK(hipStreamSynchronize(be->stream));
}

static enum ggml_status be_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    backend_state * be = (backend_state *) backend->context;
    const enum ggml_status st = graph_compute(be, cgraph);
    be->last_status = (int) st;
    return st;
}

static const ggml_backend_i kBackendIface = {
    be_get_name, be_free, be_set_tensor_async, be_get_tensor_async, nullptr, be_synchronize, nullptr, nullptr,
    nullptr, nullptr, be_graph_compute, nullptr, nullptr, nullptr,
};

// ---------------------------------------------------------------- device --

static const char * dev_get_name(ggml_backend_dev_t d) { return ((device_state *) d->context)->name.c_str(); }
static const char * dev_get_description(ggml_backend_dev_t d) {
    return ((device_state *) d->context)->description.c_str();
}

static void dev_get_memory(ggml_backend_dev_t d, size_t * free, size_t * total) {
    device_state * dev = (device_state *) d->context;
    MI_CHECK(hipSetDevice(dev->hip_id));
    size_t f = 0, t = 0;
    MI_CHECK(hipMemGetInfo(&f, &t));
    *free = f;
    *total = t;
}

static enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

static void dev_get_props(ggml_backend_dev_t d, struct ggml_backend_dev_props * props) {
    device_state * dev = (device_state *) d->context;
    props->name = dev->name.c_str();
    props->description = dev->description.c_str();
    props->type = GGML_BACKEND_DEVICE_TYPE_GPU;
    props->device_id = dev->pci_id.c_str();
    dev_get_memory(d, &props->memory_free, &props->memory_total);
    props->caps.async = false;
    props->caps.host_buffer = false;
    props->caps.buffer_from_host_ptr = false;
    props->caps.events = false;
}

static ggml_guid g_guid = {{0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x00,
                            0x00, 0x01}};

static ggml_backend_t dev_init_backend(ggml_backend_dev_t d, const char * params) {
    (void) params;
    device_state * dev = (device_state *) d->context;
    MI_CHECK(hipSetDevice(dev->hip_id));
    backend_state * be = new backend_state;
    be->dev = dev;
    be->name = dev->name;
    if (hipStreamCreateWithFlags(&be->stream, hipStreamNonBlocking) != hipSuccess) {
        delete be;
        return nullptr;
    }
    const char * env = std::getenv("OPENASR_MI355X_HIP_GRAPHS");
    if (env && env[0] == '0') be->use_graphs = false;
    be->guid = g_guid;
    be->backend.guid = &be->guid;
    be->backend.iface = kBackendIface;
    be->backend.device = d;
    be->backend.context = be;
    return &be->backend;
}

static ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t d) {
    return &((device_state *) d->context)->buft;
}

static bool dev_supports_op(ggml_backend_dev_t d, const struct ggml_tensor * op) {
    return supports_op((device_state *) d->context, op);
}

static bool dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return buft == &((device_state *) d->context)->buft;
}

static bool dev_offload_op(ggml_backend_dev_t, const struct ggml_tensor * op) {
    // worth moving to the GPU when the batch is wide enough to amortise the copy
    return op->op == GGML_OP_MUL_MAT && op->src[1] && op->src[1]->ne[1] >= 32;
}

static const ggml_backend_device_i kDeviceIface = {
    dev_get_name, dev_get_description, dev_get_memory, dev_get_type, dev_get_props, dev_init_backend,
    dev_get_buffer_type, nullptr, nullptr, dev_supports_op, dev_supports_buft, dev_offload_op,
    nullptr, nullptr, nullptr,
};

// -------------------------------------------------------------- registry --

static float host_gelu(float x) {
    const float c = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + 0.044715f * x * x)));
}

static uint16_t host_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t) (sign | (uint32_t) std::nearbyint(a * 16777216.0f));
    }
    const uint32_t mant = ax & 0x7fffffu, rem = mant & 0x1fffu;
    uint32_t h = (((ax >> 23) - 112u) << 10) | (mant >> 13);
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t) (sign | h);
}

static float host_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float) m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

static void init_devices() {
    registry_ctx & r = reg_ctx();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void) hipGetLastError();
        n = 0;
    }
    std::vector<uint16_t> table(65536);
    for (uint32_t i = 0; i < 65536; i++) table[i] = host_f32_to_f16(host_gelu(host_f16_to_f32((uint16_t) i)));
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        const std::string arch = p.gcnArchName;
        if (arch.rfind("gfx950", 0) != 0) continue;  // kernels are built for gfx950 only
        device_state * dev = new device_state;
        dev->hip_id = i;
        dev->n_cu = p.multiProcessorCount;
        int wc = 0;
        if (hipDeviceGetAttribute(&wc, hipDeviceAttributeWallClockRate, i) == hipSuccess && wc > 0)
            dev->wall_clock_khz = wc;
        dev->total_mem = p.totalGlobalMem;
        dev->arch = arch;
        dev->name = "ROCm" + std::to_string(r.devices.size());
        dev->description = std::string(p.name) + " (" + arch + ", MI355X-native)";
        char pci[32];
        std::snprintf(pci, sizeof(pci), "%04x:%02x:%02x.0", p.pciDomainID, p.pciBusID, p.pciDeviceID);
        dev->pci_id = pci;
        MI_CHECK(hipSetDevice(i));
        hipUUID uuid;
        if (hipDeviceGetUuid(&uuid, i) == hipSuccess) std::memcpy(dev->uuid, uuid.bytes, 16);
        MI_CHECK(hipMalloc((void **) &dev->gelu_table, table.size() * 2));
        ledger_add(dev, table.size() * 2, false);
        // the fixed scratch array of the allocation-free compute is device
        // memory the plugin holds on every device until the process ends
        // (mapped with the code object, not by hipMalloc)
        ledger_add(dev, static_scratch_bytes(), false);
        MI_CHECK(hipMemcpy(dev->gelu_table, table.data(), table.size() * 2, hipMemcpyHostToDevice));
        dev->buft.iface = kBuftIface;
        dev->buft.device = &dev->dev;
        dev->buft.context = dev;
        dev->dev.iface = kDeviceIface;
        dev->dev.reg = &r.reg;
        dev->dev.context = dev;
        r.devices.push_back(dev);
    }
}

static const char * reg_get_name(ggml_backend_reg_t) { return "ROCm-MI355X"; }
static size_t reg_get_device_count(ggml_backend_reg_t) { return reg_ctx().devices.size(); }
static ggml_backend_dev_t reg_get_device(ggml_backend_reg_t, size_t index) {
    registry_ctx & r = reg_ctx();
    return index < r.devices.size() ? &r.devices[index]->dev : nullptr;
}

static void set_abort_callback(ggml_backend_t backend, ggml_abort_callback cb, void * data) {
    backend_state * be = (backend_state *) backend->context;
    be->abort_cb = cb;
    be->abort_data = data;
}

static int get_cancel_observation(ggml_backend_t backend) {
    return ((backend_state *) backend->context)->last_observation;
}

static uint32_t pci_vendor_id(ggml_backend_dev_t) { return 0x1002u; }

static void * reg_get_proc_address(ggml_backend_reg_t, const char * name) {
    if (std::strcmp(name, "ggml_backend_set_abort_callback") == 0) return (void *) set_abort_callback;
    if (std::strcmp(name, "ggml_backend_get_cancel_observation") == 0) return (void *) get_cancel_observation;
    if (std::strcmp(name, "ggml_backend_device_pci_vendor_id") == 0) return (void *) pci_vendor_id;
    if (std::strcmp(name, "ggml_backend_mi355x_profile_graph") == 0) return (void *) ggml_backend_mi355x_profile_graph;
    if (std::strcmp(name, "ggml_backend_mi355x_set_hip_graphs") == 0) return (void *) ggml_backend_mi355x_set_hip_graphs;
    if (std::strcmp(name, "ggml_backend_mi355x_refuse_next_launch") == 0)
        return (void *) ggml_backend_mi355x_refuse_next_launch;
    if (std::strcmp(name, "ggml_backend_memory_get_api_v1") == 0) return (void *) ggml_backend_memory_get_api_v1;
    return nullptr;
}

static const ggml_backend_reg_i kRegIface = {reg_get_name, reg_get_device_count, reg_get_device,
                                             reg_get_proc_address};

device_state * device_of(ggml_backend_dev_t d) {
    return d && d->iface.get_name == dev_get_name ? (device_state *) d->context : nullptr;
}

device_state * device_of_buft(ggml_backend_buffer_type_t buft) {
    return buft && buft->iface.get_name == buft_get_name ? (device_state *) buft->context : nullptr;
}

backend_state * backend_of(ggml_backend_t backend) {
    return backend && backend->iface.get_name == be_get_name ? (backend_state *) backend->context : nullptr;
}

}  // namespace mi355x

using namespace mi355x;

extern "C" {

ggml_backend_reg_t ggml_backend_mi355x_reg(void) {
    registry_ctx & r = reg_ctx();
    std::call_once(r.once, [&] {
        r.reg.api_version = GGML_BACKEND_API_VERSION;
        r.reg.iface = kRegIface;
        r.reg.context = nullptr;
        init_devices();
    });
    return &r.reg;
}

ggml_backend_reg_t ggml_backend_init(void) { return ggml_backend_mi355x_reg(); }

ggml_backend_t ggml_backend_mi355x_init(int device) {
    ggml_backend_reg_t reg = ggml_backend_mi355x_reg();
    ggml_backend_dev_t d = reg_get_device(reg, (size_t) device);
    return d ? dev_init_backend(d, nullptr) : nullptr;
}

bool ggml_backend_is_mi355x(ggml_backend_t backend) {
    return backend && backend->guid && std::memcmp(backend->guid, &g_guid, sizeof(ggml_guid)) == 0;
}

const char * openasr_ggml_backend_abi_v1(void) { return OPENASR_HOST_ABI_FINGERPRINT; }

const char * openasr_ggml_backend_provider_v1(void) { return "hip"; }

bool openasr_ggml_backend_probe_v1(const char * device_target, const char * minimum_driver_version,
                                   char * driver_out, size_t driver_out_capacity) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        (void) hipGetLastError();
        return false;
    }
    bool found = false;
    for (int i = 0; i < n && !found; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        const std::string arch = p.gcnArchName;
        found = arch.rfind("gfx950", 0) == 0 &&
                (!device_target || !device_target[0] || arch.rfind(device_target, 0) == 0);
    }
    if (!found) return false;
    int drv = 0;
    if (hipDriverGetVersion(&drv) != hipSuccess) return false;
    if (minimum_driver_version && minimum_driver_version[0]) {
        const long need = std::strtol(minimum_driver_version, nullptr, 10);
        if (drv < need) return false;
    }
    if (driver_out && driver_out_capacity) std::snprintf(driver_out, driver_out_capacity, "hip-%d", drv);
    return true;
}

int ggml_backend_mi355x_profile_graph(ggml_backend_t backend, struct ggml_cgraph * cgraph, int iters,
                                      float * step_ms, int max_steps, char * labels, int label_cap) {
    if (!ggml_backend_is_mi355x(backend)) return -1;
    return profile_graph((backend_state *) backend->context, cgraph, iters, step_ms, max_steps, labels, label_cap);
}

void ggml_backend_mi355x_set_hip_graphs(ggml_backend_t backend, bool enabled) {
    if (!ggml_backend_is_mi355x(backend)) return;
    backend_state * be = (backend_state *) backend->context;
    be->use_graphs = enabled;
    if (!enabled) release_graph_cache(be);
}

void ggml_backend_mi355x_refuse_next_launch(ggml_backend_t backend) {
    if (!ggml_backend_is_mi355x(backend)) return;
    ((backend_state *) backend->context)->fail_next_launch = true;
}

int ggml_backend_mi355x_device_count(void) { return (int) ggml_backend_mi355x_reg()->iface.get_device_count(nullptr); }

}  // extern "C"

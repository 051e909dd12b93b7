// mi355x_memory.cpp -- the optional physical-memory ABI v1
// (ggml_backend_memory_get_api_v1; layouts in include/ggml_backend_memory.h,
// restating crates/openasr-core/src/ggml_runtime/ffi.rs:144-332; host side:
// ggml_runtime/backend_memory.rs and backend_memory_admission.rs).
//
// One DEVICE_LOCAL domain per device. The numbers come from the device's
// allocation ledger (every hipMalloc the plugin makes: buffers, executor
// arenas, its own tables) and hipMemGetInfo. The ledger generation advances
// with every allocation and release, so a quote taken at generation g is
// still valid for reserve_private exactly while nothing was allocated or
// released in between.

#include <time.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>

#include "ggml_backend_memory.h"
#include "mi355x_exec.h"

namespace mi355x {
namespace {

constexpr uint64_t kGranule = 2ull << 20;  // device allocations are rounded up to 2 MiB pages

std::atomic<uint64_t> g_quote_token{1};

uint64_t round_granule(uint64_t v) { return (v + kGranule - 1) / kGranule * kGranule; }

ggml_backend_memory_domain_id_v1 domain_id(const device_state * dev) {
    ggml_backend_memory_domain_id_v1 id{};
    std::memcpy(id.physical_device_uuid, dev->uuid, 16);
    id.heap_index = 0;
    id.kind = GGML_BACKEND_MEMORY_DOMAIN_DEVICE_LOCAL;
    return id;
}

struct ledger_view {
    uint64_t live, workspace, high_water, allocs, failures, generation;
};

ledger_view read_ledger(device_state * dev) {
    std::lock_guard<std::mutex> lk(dev->mem_mu);
    return {dev->live_bytes, dev->workspace_bytes, dev->high_water, dev->alloc_count, dev->alloc_failures,
            dev->generation};
}

// FNV-1a over the fields that decide a quote
uint64_t fingerprint(const ggml_backend_memory_request_v1 * r, uint32_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    auto mix = [&](uint64_t v) {
        for (int i = 0; i < 8; i++) {
            h ^= (v >> (8 * i)) & 0xFF;
            h *= 0x100000001b3ull;
        }
    };
    mix(n);
    for (uint32_t i = 0; i < n; i++) {
        mix(r[i].kind);
        mix(r[i].flags);
        mix(r[i].usage);
        mix(r[i].request_id);
        mix((uint64_t) (uintptr_t) r[i].backend);
        mix((uint64_t) (uintptr_t) r[i].buft);
        mix((uint64_t) (uintptr_t) r[i].graph);
        mix(r[i].requested_bytes);
        mix(r[i].currently_allocated_bytes);
        mix(r[i].max_tensor_bytes);
    }
    return h;
}

// the device a request lands on: its backend's, else its buffer type's
device_state * request_device(const ggml_backend_memory_request_v1 & r) {
    if (backend_state * be = backend_of(r.backend)) return be->dev;
    return device_of_buft(r.buft);
}

struct planned_claim {
    ggml_backend_memory_claim_v1 claim;
    bool provisional;
};

// Claims of a request list (one per request). Returns a ggml_status.
// GRAPH_PRIVATE requests of one backend share its arena: the arena grows to
// the largest need once, charged to the request that needs the most.
int plan_claims(const ggml_backend_memory_request_v1 * req, uint32_t n, std::vector<planned_claim> & out,
                uint32_t & quote_flags, uint64_t & generation) {
    out.clear();
    quote_flags = 0;
    generation = 0;
    device_state * gen_dev = nullptr;
    std::map<backend_state *, std::pair<uint64_t, uint32_t>> arena;  // backend -> (largest need, request)
    std::vector<uint64_t> need(n, 0);
    std::vector<bool> need_known(n, true);
    for (uint32_t i = 0; i < n; i++) {
        const ggml_backend_memory_request_v1 & r = req[i];
        if (r.struct_size < sizeof(ggml_backend_memory_request_v1)) return GGML_STATUS_FAILED;
        device_state * dev = request_device(r);
        if (!dev) return GGML_STATUS_FAILED;
        if (gen_dev && gen_dev != dev) return GGML_STATUS_FAILED;  // one device per transaction
        gen_dev = dev;
        if (r.kind == GGML_BACKEND_MEMORY_REQUEST_GRAPH_PRIVATE) {
            backend_state * be = backend_of(r.backend);
            if (!be || !r.graph) return GGML_STATUS_FAILED;
            size_t bytes = 0;
            if (!graph_arena_bytes(be, r.graph, &bytes)) {
                // a graph the executor cannot plan yet: the default arena, provisionally
                bytes = 64u << 20;
                need_known[i] = false;
            }
            need[i] = bytes;
            auto & a = arena[be];
            if (bytes > a.first) a = {bytes, i};
        } else if (r.kind == GGML_BACKEND_MEMORY_REQUEST_HOST_IMPORT) {
            return GGML_STATUS_FAILED;  // no buffer_from_host_ptr on this device
        } else if (r.kind != GGML_BACKEND_MEMORY_REQUEST_BUFFER && r.kind != GGML_BACKEND_MEMORY_REQUEST_TRANSFER) {
            return GGML_STATUS_FAILED;
        }
    }
    if (!gen_dev) return GGML_STATUS_SUCCESS;
    const ledger_view lv = read_ledger(gen_dev);
    generation = lv.generation;
    uint64_t committed = lv.live + lv.workspace;
    for (uint32_t i = 0; i < n; i++) {
        const ggml_backend_memory_request_v1 & r = req[i];
        planned_claim pc{};
        ggml_backend_memory_claim_v1 & c = pc.claim;
        c.struct_size = sizeof(ggml_backend_memory_claim_v1);
        c.request_id = r.request_id;
        c.domain = domain_id(gen_dev);
        c.payload_requested_bytes = r.requested_bytes;
        c.committed_before_bytes = committed;
        uint64_t extra = 0, retained_extra = 0, releasable = 0;
        if (r.kind == GGML_BACKEND_MEMORY_REQUEST_BUFFER) {
            const uint64_t want = round_granule(std::max<uint64_t>(r.requested_bytes, 256));
            extra = want > r.currently_allocated_bytes ? want - r.currently_allocated_bytes : 0;
            retained_extra = extra;
            c.flags = GGML_BACKEND_MEMORY_CLAIM_CONSERVATIVE_UPPER;
        } else if (r.kind == GGML_BACKEND_MEMORY_REQUEST_GRAPH_PRIVATE) {
            backend_state * be = backend_of(r.backend);
            c.payload_requested_bytes = need[i];
            const auto & a = arena[be];
            const uint64_t cur = be->scratch_cap;
            if (a.second == i && a.first > cur) {
                // the arena is freed, then allocated at the new size
                extra = a.first - cur;
                retained_extra = extra;
            }
            releasable = std::max<uint64_t>(cur, a.first);
            c.flags = need_known[i] ? GGML_BACKEND_MEMORY_CLAIM_EXACT : GGML_BACKEND_MEMORY_CLAIM_PROVISIONAL;
            if (!need_known[i]) pc.provisional = true;
            // instantiated HIP graphs hold driver memory beyond the arena
            quote_flags |= GGML_BACKEND_MEMORY_QUOTE_OPAQUE_DRIVER_COSTS_REQUIRE_DOMAIN_HEADROOM;
        } else {
            c.flags = GGML_BACKEND_MEMORY_CLAIM_EXACT;  // TRANSFER: synchronous copies, no device staging
        }
        c.commit_peak_extra_upper_bytes = extra;
        c.committed_after_upper_bytes = committed + extra;
        c.resident_after_upper_bytes = committed + extra;
        c.retained_after_use_upper_bytes = committed + retained_extra;
        c.releasable_after_use_upper_bytes = releasable;
        committed += extra;
        if (pc.provisional) quote_flags |= GGML_BACKEND_MEMORY_QUOTE_PROVISIONAL;
        out.push_back(pc);
    }
    return GGML_STATUS_SUCCESS;
}

int mem_get_domains(ggml_backend_dev_t device, ggml_backend_memory_domain_v1 * domains, uint32_t * count) {
    device_state * dev = device_of(device);
    if (!dev || !count) return GGML_STATUS_FAILED;
    if (!domains) {
        *count = 1;
        return GGML_STATUS_SUCCESS;
    }
    if (*count < 1) return GGML_STATUS_FAILED;
    ggml_backend_memory_domain_v1 & d = domains[0];
    if (d.struct_size < sizeof(ggml_backend_memory_domain_v1)) return GGML_STATUS_FAILED;
    d.flags = 0;
    d.id = domain_id(dev);
    std::memset(d.name, 0, sizeof(d.name));
    std::snprintf(d.name, sizeof(d.name), "%s HBM3E", dev->name.c_str());
    *count = 1;
    return GGML_STATUS_SUCCESS;
}

int mem_quote(const ggml_backend_memory_request_v1 * requests, uint32_t n, ggml_backend_memory_quote_v1 * quote,
              ggml_backend_memory_claim_v1 * claims, uint32_t * count) {
    if (!quote || !count || (n && !requests)) return GGML_STATUS_FAILED;
    if (quote->struct_size < sizeof(ggml_backend_memory_quote_v1)) return GGML_STATUS_FAILED;
    std::vector<planned_claim> pcs;
    uint32_t qflags = 0;
    uint64_t generation = 0;
    const int st = plan_claims(requests, n, pcs, qflags, generation);
    if (st != GGML_STATUS_SUCCESS) return st;
    const uint32_t need = (uint32_t) pcs.size();
    if (claims) {
        if (*count < need) return GGML_STATUS_FAILED;
        for (uint32_t i = 0; i < need; i++) {
            if (claims[i].struct_size < sizeof(ggml_backend_memory_claim_v1)) return GGML_STATUS_FAILED;
            claims[i] = pcs[i].claim;
        }
    }
    *count = need;
    quote->flags = qflags;
    quote->residual_flags = 0;
    quote->residual_request_count = 0;
    quote->provisional_requested_upper_bytes = 0;
    quote->stats_generation = generation;
    quote->quote_token = g_quote_token.fetch_add(1);
    quote->request_fingerprint = fingerprint(requests, n);
    return GGML_STATUS_SUCCESS;
}

int mem_reserve_private(const ggml_backend_memory_request_v1 * requests, uint32_t n,
                        const ggml_backend_memory_quote_v1 * quote, ggml_backend_memory_claim_v1 * claims,
                        uint32_t * count) {
    if (!quote || !count || (n && !requests)) return GGML_STATUS_FAILED;
    if (quote->quote_token == 0 || quote->request_fingerprint != fingerprint(requests, n)) return GGML_STATUS_FAILED;
    std::vector<planned_claim> pcs;
    uint32_t qflags = 0;
    uint64_t generation = 0;
    int st = plan_claims(requests, n, pcs, qflags, generation);
    if (st != GGML_STATUS_SUCCESS) return st;
    if (generation != 0 && generation != quote->stats_generation) return GGML_STATUS_FAILED;  // stale quote
    std::vector<uint32_t> priv;
    for (uint32_t i = 0; i < n; i++) {
        if (requests[i].kind == GGML_BACKEND_MEMORY_REQUEST_GRAPH_PRIVATE) priv.push_back(i);
    }
    if (!claims) {  // sizing call: no state change
        *count = (uint32_t) priv.size();
        return GGML_STATUS_SUCCESS;
    }
    if (*count < priv.size()) return GGML_STATUS_FAILED;
    for (uint32_t k = 0; k < priv.size(); k++) {
        if (claims[k].struct_size < sizeof(ggml_backend_memory_claim_v1)) return GGML_STATUS_FAILED;
    }
    // commit: grow each backend's arena. Failure-atomic as the host requires
    // of a non-success status: the arenas grown by this call are released
    // again, so no private reservation outlives the failed call.
    std::vector<backend_state *> grown;
    for (uint32_t i : priv) {
        backend_state * be = backend_of(requests[i].backend);
        const size_t before = be->scratch_cap;
        if (!reserve_graph_arena(be, requests[i].graph)) {
            for (backend_state * g : grown) release_scratch(g);
            return GGML_STATUS_ALLOC_FAILED;
        }
        if (be->scratch_cap != before) grown.push_back(be);
    }
    for (uint32_t k = 0; k < priv.size(); k++) {
        ggml_backend_memory_claim_v1 c = pcs[priv[k]].claim;
        backend_state * be = backend_of(requests[priv[k]].backend);
        c.flags = GGML_BACKEND_MEMORY_CLAIM_EXACT;
        c.payload_requested_bytes = be->scratch_cap;
        claims[k] = c;
    }
    *count = (uint32_t) priv.size();
    return GGML_STATUS_SUCCESS;
}

int mem_get_stats(ggml_backend_dev_t device, ggml_backend_t backend, ggml_backend_memory_stats_v1 * stats,
                  uint32_t * count) {
    backend_state * be = backend_of(backend);
    device_state * dev = device ? device_of(device) : (be ? be->dev : nullptr);
    if (!dev || !count || (backend && !be) || (be && be->dev != dev)) return GGML_STATUS_FAILED;
    if (!stats) {
        *count = 1;
        return GGML_STATUS_SUCCESS;
    }
    if (*count < 1 || stats[0].struct_size < sizeof(ggml_backend_memory_stats_v1)) return GGML_STATUS_FAILED;
    ggml_backend_memory_stats_v1 & s = stats[0];
    const uint32_t size = s.struct_size;
    std::memset(&s, 0, sizeof(s));
    s.struct_size = size;
    s.domain = domain_id(dev);
    const ledger_view lv = read_ledger(dev);
    s.generation = lv.generation;
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    s.timestamp_monotonic_ns = (uint64_t) ts.tv_sec * 1000000000ull + (uint64_t) ts.tv_nsec;
    size_t free_b = 0, total_b = 0;
    if (hipSetDevice(dev->hip_id) != hipSuccess || hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        (void) hipGetLastError();
        s.flags |= GGML_BACKEND_MEMORY_STATS_BUDGET_UNAVAILABLE;
        total_b = dev->total_mem;
        free_b = 0;
    }
    s.total_bytes = total_b;
    s.budget_bytes = total_b;
    s.device_free_bytes = free_b;
    s.device_used_bytes = total_b - std::min(total_b, free_b);
    s.backend_owned_live_bytes = lv.live;
    s.backend_owned_cached_bytes = 0;
    s.backend_owned_workspace_bytes = lv.workspace;
    s.backend_owned_high_water_bytes = lv.high_water;
    s.allocation_count = lv.allocs;
    s.allocation_failure_count = lv.failures;
    s.health = GGML_BACKEND_MEMORY_HEALTHY;
    if (be) {
        if (be->quarantined) s.health = GGML_BACKEND_MEMORY_QUARANTINED;
        else if (be->poisoned) s.health = GGML_BACKEND_MEMORY_DEVICE_LOST;
        s.last_ggml_status = be->last_status;
        s.last_native_error = be->last_native_error;
        s.quarantine_generation = be->quarantine_generation;
    }
    *count = 1;
    return GGML_STATUS_SUCCESS;
}

int mem_trim(ggml_backend_t backend, uint64_t flags) {
    (void) flags;
    backend_state * be = backend_of(backend);
    if (!be) return GGML_STATUS_FAILED;
    if (hipSetDevice(be->dev->hip_id) != hipSuccess || hipStreamSynchronize(be->stream) != hipSuccess) {
        (void) hipGetLastError();
        return GGML_STATUS_FAILED;
    }
    release_scratch(be);
    return GGML_STATUS_SUCCESS;
}

int mem_quarantine(ggml_backend_t backend, const ggml_backend_memory_quarantine_v1 * q) {
    backend_state * be = backend_of(backend);
    if (!be || !q || q->struct_size < sizeof(ggml_backend_memory_quarantine_v1)) return GGML_STATUS_FAILED;
    be->quarantined = true;
    be->poisoned = true;  // graph_compute now fails closed
    be->quarantine_generation++;
    be->last_status = q->ggml_status;
    be->last_native_error = q->native_error;
    return GGML_STATUS_SUCCESS;
}

const ggml_backend_memory_api_v1 kMemoryApi = {
    sizeof(ggml_backend_memory_api_v1),
    GGML_BACKEND_MEMORY_ABI_V1,
    0,
    mem_get_domains,
    mem_quote,
    mem_reserve_private,
    mem_get_stats,
    mem_trim,
    mem_quarantine,
};

}  // namespace
}  // namespace mi355x

extern "C" const ggml_backend_memory_api_v1 * ggml_backend_memory_get_api_v1(void) { return &mi355x::kMemoryApi; }

/*
 * ggml_backend_memory.h -- the optional physical-memory ABI v1 of OpenASR's
 * ggml fork, served by libggml-mi355x.so through the registry proc
 * "ggml_backend_memory_get_api_v1".
 *
 * The layouts restate the host's #[repr(C)] mirror
 * (crates/openasr-core/src/ggml_runtime/ffi.rs:144-332): the fork's own header
 * is absent, so the Rust side is the contract. The host resolves the proc from
 * the backend's registry (ggml_runtime/backend_memory.rs:140-190), requires
 * struct_size >= sizeof(api), abi_version == 1 and non-null get_domains,
 * quote, reserve_private and get_stats, and drives every list-returning call
 * twice: first with a null array to learn the count (which must not change
 * backend state), then with an array of that capacity
 * (backend_memory.rs:193-330). Every function returns a ggml_status value
 * (0 = success).
 *
 * What the MI355X plugin reports:
 *   one DEVICE_LOCAL domain per device (heap 0, the device's HBM), named by
 *   the HIP device UUID;
 *   quotes for BUFFER requests (hipMalloc of the request rounded up to the
 *   2 MiB allocation granule) and GRAPH_PRIVATE requests (the executor's
 *   scratch arena for that graph, found by planning it), TRANSFER requests
 *   costing no device memory (copies are synchronous from host memory);
 *   HOST_IMPORT is not supported (the device has no buffer_from_host_ptr);
 *   reserve_private grows the backend's scratch arena for the quoted graphs;
 *   stats from hipMemGetInfo plus the plugin's own allocation ledger;
 *   trim releases the scratch arena and the HIP-graph cache;
 *   quarantine poisons the backend (its graph_compute then fails closed).
 */
#ifndef OPENASR_GGML_BACKEND_MEMORY_H
#define OPENASR_GGML_BACKEND_MEMORY_H

#include <stdint.h>

#include "ggml_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* constants: ffi.rs:144-172 */
#define GGML_BACKEND_MEMORY_ABI_V1 1u
#define GGML_BACKEND_MEMORY_DOMAIN_DEVICE_LOCAL 1u
#define GGML_BACKEND_MEMORY_DOMAIN_HOST_PAGEABLE 2u
#define GGML_BACKEND_MEMORY_DOMAIN_HOST_PINNED 3u
#define GGML_BACKEND_MEMORY_DOMAIN_UNIFIED 4u
#define GGML_BACKEND_MEMORY_DOMAIN_FILE_BACKED 5u
#define GGML_BACKEND_MEMORY_REQUEST_BUFFER 1u
#define GGML_BACKEND_MEMORY_REQUEST_HOST_IMPORT 2u
#define GGML_BACKEND_MEMORY_REQUEST_GRAPH_PRIVATE 3u
#define GGML_BACKEND_MEMORY_REQUEST_TRANSFER 4u
#define GGML_BACKEND_MEMORY_QUOTE_PROVISIONAL (1u << 0)
#define GGML_BACKEND_MEMORY_QUOTE_HAS_RESIDUAL_UNCERTAINTY (1u << 1)
#define GGML_BACKEND_MEMORY_QUOTE_OPAQUE_DRIVER_COSTS_REQUIRE_DOMAIN_HEADROOM (1u << 2)
#define GGML_BACKEND_MEMORY_RESIDUAL_BACKEND_PRIVATE (1u << 0)
#define GGML_BACKEND_MEMORY_STATS_BUDGET_UNAVAILABLE (1u << 0)
#define GGML_BACKEND_MEMORY_CLAIM_EXACT (1u << 0)
#define GGML_BACKEND_MEMORY_CLAIM_CONSERVATIVE_UPPER (1u << 1)
#define GGML_BACKEND_MEMORY_CLAIM_DRIVER_ESTIMATE (1u << 2)
#define GGML_BACKEND_MEMORY_CLAIM_FILE_BACKED (1u << 5)
#define GGML_BACKEND_MEMORY_CLAIM_PROVISIONAL (1u << 6)
#define GGML_BACKEND_MEMORY_HEALTHY 0u
#define GGML_BACKEND_MEMORY_DEGRADED 1u
#define GGML_BACKEND_MEMORY_QUARANTINED 2u
#define GGML_BACKEND_MEMORY_DEVICE_LOST 3u

/* GgmlBackendMemoryDomainIdV1, ffi.rs:174-179 */
typedef struct ggml_backend_memory_domain_id_v1 {
    uint8_t physical_device_uuid[16];
    uint32_t heap_index;
    uint32_t kind;
} ggml_backend_memory_domain_id_v1;

/* GgmlBackendMemoryDomainV1, ffi.rs:181-188 */
typedef struct ggml_backend_memory_domain_v1 {
    uint32_t struct_size;
    uint32_t flags;
    ggml_backend_memory_domain_id_v1 id;
    char name[48];
} ggml_backend_memory_domain_v1;

/* GgmlBackendMemoryRequestV1, ffi.rs:190-205 */
typedef struct ggml_backend_memory_request_v1 {
    uint32_t struct_size;
    uint32_t kind;
    uint32_t flags;
    uint32_t usage; /* ggml_backend_buffer_usage for BUFFER requests */
    uint64_t request_id;
    ggml_backend_t backend;
    ggml_backend_t peer_backend;
    ggml_backend_buffer_type_t buft;
    struct ggml_cgraph * graph;
    const void * host_ptr;
    uint64_t requested_bytes;
    uint64_t currently_allocated_bytes;
    uint64_t max_tensor_bytes;
} ggml_backend_memory_request_v1;

/* GgmlBackendMemoryClaimV1, ffi.rs:227-241 */
typedef struct ggml_backend_memory_claim_v1 {
    uint32_t struct_size;
    uint32_t flags;
    uint64_t request_id;
    ggml_backend_memory_domain_id_v1 domain;
    uint64_t payload_requested_bytes;
    uint64_t committed_before_bytes;
    uint64_t committed_after_upper_bytes;
    uint64_t commit_peak_extra_upper_bytes;
    uint64_t resident_after_upper_bytes;
    uint64_t retained_after_use_upper_bytes;
    uint64_t releasable_after_use_upper_bytes;
} ggml_backend_memory_claim_v1;

/* GgmlBackendMemoryQuoteV1, ffi.rs:243-254 */
typedef struct ggml_backend_memory_quote_v1 {
    uint32_t struct_size;
    uint32_t flags;
    uint32_t residual_flags;
    uint32_t residual_request_count;
    uint64_t provisional_requested_upper_bytes;
    uint64_t stats_generation;
    uint64_t quote_token;
    uint64_t request_fingerprint;
} ggml_backend_memory_quote_v1;

/* GgmlBackendMemoryStatsV1, ffi.rs:256-279 */
typedef struct ggml_backend_memory_stats_v1 {
    uint32_t struct_size;
    uint32_t flags;
    ggml_backend_memory_domain_id_v1 domain;
    uint64_t generation;
    uint64_t timestamp_monotonic_ns;
    uint64_t total_bytes;
    uint64_t budget_bytes;
    uint64_t device_used_bytes;
    uint64_t device_free_bytes;
    uint64_t backend_owned_live_bytes;
    uint64_t backend_owned_cached_bytes;
    uint64_t backend_owned_workspace_bytes;
    uint64_t backend_owned_high_water_bytes;
    uint64_t allocation_count;
    uint64_t allocation_failure_count;
    uint32_t health;
    int32_t last_ggml_status;
    int64_t last_native_error;
    uint64_t quarantine_generation;
} ggml_backend_memory_stats_v1;

/* GgmlBackendMemoryQuarantineV1, ffi.rs:281-290 */
typedef struct ggml_backend_memory_quarantine_v1 {
    uint32_t struct_size;
    uint32_t flags;
    uint32_t reason;
    int32_t ggml_status;
    int64_t native_error;
    char message[96];
} ggml_backend_memory_quarantine_v1;

/* function table, ffi.rs:292-330 */
typedef struct ggml_backend_memory_api_v1 {
    uint32_t struct_size;
    uint32_t abi_version;
    uint64_t capabilities;
    int (*get_domains)(ggml_backend_dev_t device, ggml_backend_memory_domain_v1 * domains, uint32_t * count);
    int (*quote)(const ggml_backend_memory_request_v1 * requests, uint32_t n_requests,
                 ggml_backend_memory_quote_v1 * quote, ggml_backend_memory_claim_v1 * claims, uint32_t * count);
    int (*reserve_private)(const ggml_backend_memory_request_v1 * requests, uint32_t n_requests,
                           const ggml_backend_memory_quote_v1 * quote, ggml_backend_memory_claim_v1 * claims,
                           uint32_t * count);
    int (*get_stats)(ggml_backend_dev_t device, ggml_backend_t backend, ggml_backend_memory_stats_v1 * stats,
                     uint32_t * count);
    int (*trim)(ggml_backend_t backend, uint64_t flags);
    int (*quarantine)(ggml_backend_t backend, const ggml_backend_memory_quarantine_v1 * request);
} ggml_backend_memory_api_v1;

/* The registry proc "ggml_backend_memory_get_api_v1" (ffi.rs:332,
 * backend_memory.rs:17): returns the plugin's static table. Also exported
 * directly for hosts that link the plugin. */
const ggml_backend_memory_api_v1 * ggml_backend_memory_get_api_v1(void);

#ifdef __cplusplus
}
#endif

#endif

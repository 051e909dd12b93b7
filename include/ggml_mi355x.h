/*
 * ggml_mi355x.h -- entry points of libggml-mi355x.so, the MI355X (gfx950)
 * ggml backend plugin for OpenASR's quantized decoder step.
 *
 * The first four are what OpenASR's verified plugin loader resolves; they
 * replace the exports of the fork's ggml-hip plugin:
 *   ggml_backend_init                  -- ggml DL convention, returns the registry
 *                                         (required export list:
 *                                         .github/workflows/release-binaries.yml:823-829)
 *   openasr_ggml_backend_abi_v1        -- host ABI fingerprint the plugin was built
 *                                         against (compared with the value baked
 *                                         by crates/openasr-core/build.rs:1145-1256;
 *                                         passed as expected_openasr_abi_v1 at
 *                                         ggml_runtime/ffi.rs:415-423)
 *   openasr_ggml_backend_provider_v1   -- provider label, "hip"
 *                                         (ggml_runtime/backend.rs:1366-1380)
 *   openasr_ggml_backend_probe_v1      -- live device check for the catalog's device
 *                                         target and driver floor; writes the driver
 *                                         version string (ffi.rs:424-434,
 *                                         backend.rs:1382-1444)
 * The registry's name is "ROCm-MI355X" (the host requires "hip" or "rocm" in
 * it, backend.rs:1347-1350).
 *
 * Registry procs served through get_proc_address:
 *   "ggml_backend_set_abort_callback"     -- native cancellation hook
 *                                            (docs/design/graph-cancellation.md:9-35)
 *   "ggml_backend_get_cancel_observation" -- observation boundary of the last compute
 *   "ggml_backend_device_pci_vendor_id"   -- 0x1002 (backend.rs:1678-1694)
 *   "ggml_backend_mi355x_profile_graph", "ggml_backend_mi355x_set_hip_graphs",
 *   "ggml_backend_mi355x_refuse_next_launch"
 *                                         -- the three functions below
 */
#ifndef OPENASR_GGML_MI355X_H
#define OPENASR_GGML_MI355X_H

#include "ggml_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

ggml_backend_reg_t ggml_backend_init(void);
const char * openasr_ggml_backend_abi_v1(void);
const char * openasr_ggml_backend_provider_v1(void);
bool openasr_ggml_backend_probe_v1(const char * device_target, const char * minimum_driver_version,
                                   char * driver_out, size_t driver_out_capacity);

/* direct-link helpers, the ggml-hip equivalents of ggml_backend_cuda_reg / _init */
ggml_backend_reg_t ggml_backend_mi355x_reg(void);
ggml_backend_t ggml_backend_mi355x_init(int device);
bool ggml_backend_is_mi355x(ggml_backend_t backend);
int ggml_backend_mi355x_device_count(void);

/* Measurement: plan `cgraph` and run its launches eagerly `iters` times with a
 * HIP event pair around each launch group on the backend's own stream; fills
 * the mean milliseconds per group and "<kernel>:<node name>" labels
 * (label_cap bytes each). Returns the number of groups, or -1. No reference
 * counterpart: it exists for the benchmark's roofline figures. */
int ggml_backend_mi355x_profile_graph(ggml_backend_t backend, struct ggml_cgraph * cgraph, int iters,
                                      float * step_ms, int max_steps, char * labels, int label_cap);

/* Turn HIP-graph capture of repeated graphs on or off (default on; the
 * environment variable OPENASR_MI355X_HIP_GRAPHS=0 also turns it off). */
void ggml_backend_mi355x_set_hip_graphs(ggml_backend_t backend, bool enabled);

/* Test seam: the first launch of the backend's next graph_compute is refused
 * on the host (as a launcher refuses a shape it cannot run) and no kernel of
 * it runs; that compute then fails closed with GGML_STATUS_FAILED and caches
 * no HIP graph. It plays the role of the host's injected compute status
 * (crates/openasr-core/src/ggml_runtime/cpu_graph.rs:7926-7947). */
void ggml_backend_mi355x_refuse_next_launch(ggml_backend_t backend);

/* Graph compute that allocates no device memory. No counterpart in the
 * reference: it is for callers that cannot call hipMalloc (code under their
 * own HIP-graph capture, tight serving loops, harnesses that forbid
 * allocation). Same plan, kernels and results as ggml_backend_graph_compute
 * on this backend, launched eagerly (no HIP-graph capture), with the plan's
 * scratch in a fixed 64 MiB device array (one per device, held until the
 * process ends; ggml_backend_mi355x_static_scratch_bytes reports its size).
 * A graph whose plan needs more scratch returns GGML_STATUS_ALLOC_FAILED with
 * a message. Calls that overlap on one device race on the shared array. */
enum ggml_status ggml_backend_mi355x_graph_compute_static(ggml_backend_t backend, struct ggml_cgraph * cgraph);
size_t ggml_backend_mi355x_static_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif

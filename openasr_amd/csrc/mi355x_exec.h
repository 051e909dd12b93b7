// mi355x_exec.h -- device / backend state and the graph executor interface.
#pragma once

#include <atomic>
#include <cstdint>
#include <functional>
#include <mutex>
#include <string>
#include <vector>

#include "ggml_abi.h"
#include "mi355x_common.h"
#include "ops.h"

namespace mi355x {

// small host uploads waiting in pinned memory (mi355x_upload.cpp)
struct upload_queue {
    std::mutex mu;
    char * pinned = nullptr;  // two halves of kUploadHalf bytes, hipHostMalloc'd
    bool tried = false;       // allocation attempted (on failure uploads stay synchronous)
    int cur = 0;              // the half new uploads go to
    size_t used = 0;
    std::vector<upload_entry> pending;
    hipEvent_t done[2] = {nullptr, nullptr};  // recorded after the launch that read each half
    bool busy[2] = {false, false};
};

struct device_state {
    int hip_id = -1;
    int n_cu = 0;
    size_t total_mem = 0;
    std::string name;
    std::string description;
    std::string pci_id;
    std::string arch;
    uint16_t * gelu_table = nullptr;  // device copy of the f16 GELU table
    int wall_clock_khz = 100000;      // constant-rate device clock (hipDeviceAttributeWallClockRate)
    uint8_t uuid[16] = {};            // hipDeviceGetUuid
    ggml_backend_device dev{};
    ggml_backend_buffer_type buft{};
    // allocation ledger of the memory ABI: every device allocation the plugin
    // makes on this device (buffers, executor arenas, its own tables)
    std::mutex mem_mu;
    uint64_t live_bytes = 0;       // buffers and tables
    uint64_t workspace_bytes = 0;  // executor scratch arenas
    uint64_t high_water = 0;       // largest live + workspace seen
    uint64_t alloc_count = 0, alloc_failures = 0;
    uint64_t generation = 1;       // advances with every allocation and release
    // first HIP error of a tensor transfer (set/get/memset/copy/clear) since
    // the last graph_compute on this device; that compute consumes it and
    // fails with it
    std::atomic<int> transfer_error{0};
    // the device's copy of the fixed scratch array (mi355x_static.cpp), looked
    // up once on first use
    std::once_flag static_once;
    char * static_scratch = nullptr;
    hipError_t static_err = hipSuccess;
    upload_queue uploads;
};

// Staged uploads. stage_upload copies n bytes for dst into pinned memory
// and queues them (false: not staged -- too large, or no pinned memory --
// and the caller copies synchronously). flush_uploads applies everything
// queued, on stream s (null: the null stream), before any device work that
// may read it; with wait it returns once the writes are done. Every buffer
// operation and every compute on the device flushes first, so the queue is
// invisible to the host except in time.
bool stage_upload(device_state * dev, char * dst, const void * src, size_t n);
void flush_uploads(device_state * dev, hipStream_t s, bool wait);
void release_uploads(device_state * dev);

// Errors noted while an error_scope is active on the calling thread go to
// its sink (the first one is kept): a backend's launch_error while it plans,
// captures or launches a graph, the device's transfer_error inside a buffer
// operation. Scopes nest; the innermost one receives the error.
struct error_scope {
    explicit error_scope(std::atomic<int> * sink);
    ~error_scope();
    error_scope(const error_scope &) = delete;
    error_scope & operator=(const error_scope &) = delete;

  private:
    std::atomic<int> * prev_;
};

// this plugin's objects behind ggml handles (null for another backend's)
device_state * device_of(ggml_backend_dev_t d);
device_state * device_of_buft(ggml_backend_buffer_type_t buft);
struct backend_state;
backend_state * backend_of(ggml_backend_t backend);

// ledger updates (thread-safe)
void ledger_add(device_state * dev, uint64_t bytes, bool workspace);
void ledger_sub(device_state * dev, uint64_t bytes, bool workspace);
void ledger_failure(device_state * dev);
// size of the fixed scratch array every device holds (mi355x_static.cpp)
size_t static_scratch_bytes();

// one planned launch: a closure that enqueues kernels on a stream
struct step {
    std::function<void(hipStream_t)> run;
    const ggml_tensor * node;  // the last graph node this step produces
    std::string label;
    int pos = -1;  // graph position of the node being planned when the step was made (where it runs)
    std::vector<std::pair<uintptr_t, uintptr_t>> writes;  // byte ranges [lo, hi) the step writes
};

struct cache_entry {
    uint64_t key = 0;
    int seen = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t last_use = 0;
};

struct backend_state {
    device_state * dev = nullptr;
    hipStream_t stream = nullptr;
    char * scratch = nullptr;
    size_t scratch_cap = 0;
    size_t gen_off = 0;  // offset of the general region inside the arena
    std::vector<cache_entry> cache;
    uint64_t use_clock = 0;
    bool use_graphs = true;
    ggml_abort_callback abort_cb = nullptr;
    void * abort_data = nullptr;
    int last_observation = 0;
    bool poisoned = false;
    bool quarantined = false;          // by the memory ABI's quarantine call
    uint64_t quarantine_generation = 0;
    int last_status = 0;               // ggml_status of the last graph_compute
    int64_t last_native_error = 0;     // hipError_t behind it
    std::atomic<int> launch_error{0};  // first error noted during the current graph_compute
    bool fail_next_launch = false;     // test seam: the next compute's first launch is refused
    char * scratch_override = nullptr; // while graph_compute_in runs: the caller's scratch
    size_t override_gen_off = 0;       // offset of its general region
    ggml_guid guid{};
    ggml_backend backend{};
    std::string name;
};

enum ggml_status graph_compute(backend_state * be, ggml_cgraph * cg);

// graph_compute with the plan's scratch in [scratch, scratch + cap) instead of
// the backend's arena: eager launches only (no HIP-graph capture), no device
// allocation; GGML_STATUS_ALLOC_FAILED if the plan needs more than cap
enum ggml_status graph_compute_in(backend_state * be, ggml_cgraph * cg, char * scratch, size_t cap);

// executor scratch arena: the bytes running `cg` needs (false if the graph
// cannot be planned), growing the arena to it, and releasing it (with the
// HIP-graph cache that points into it)
bool graph_arena_bytes(backend_state * be, ggml_cgraph * cg, size_t * bytes);
bool reserve_graph_arena(backend_state * be, ggml_cgraph * cg);
void release_scratch(backend_state * be);
bool supports_op(const device_state * dev, const ggml_tensor * op);
void release_graph_cache(backend_state * be);

// measurement hook: runs the graph's planned steps eagerly `iters` times with
// a HIP event pair around every step; fills per-step mean milliseconds
int profile_graph(backend_state * be, ggml_cgraph * cg, int iters, float * step_ms, int max_steps, char * labels,
                  int label_cap);

}  // namespace mi355x

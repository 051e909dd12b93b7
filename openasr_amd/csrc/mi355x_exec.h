// mi355x_exec.h -- device / backend state and the graph executor interface.
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "ggml_abi.h"
#include "mi355x_common.h"

namespace mi355x {

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
    ggml_backend_device dev{};
    ggml_backend_buffer_type buft{};
};

// one planned launch: a closure that enqueues kernels on a stream
struct step {
    std::function<void(hipStream_t)> run;
    const ggml_tensor * node;  // the last graph node this step produces
    std::string label;
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
    ggml_guid guid{};
    ggml_backend backend{};
    std::string name;
};

enum ggml_status graph_compute(backend_state * be, ggml_cgraph * cg);
bool supports_op(const device_state * dev, const ggml_tensor * op);
void release_graph_cache(backend_state * be);

// measurement hook: runs the graph's planned steps eagerly `iters` times with
// a HIP event pair around every step; fills per-step mean milliseconds
int profile_graph(backend_state * be, ggml_cgraph * cg, int iters, float * step_ms, int max_steps, char * labels,
                  int label_cap);

}  // namespace mi355x

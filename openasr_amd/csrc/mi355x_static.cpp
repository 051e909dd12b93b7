// mi355x_static.cpp -- a graph compute that allocates no device memory.
//
// ggml_backend_graph_compute runs a graph's launches with their scratch
// (quantized activations of the MUL_MATs, attention chunk partials, the decode
// step's rope table, argmax partials) in an arena the backend allocates and
// grows with hipMalloc. Callers that cannot allocate -- code under HIP graph
// capture of their own, tight serving loops, harnesses that forbid it -- call
// ggml_backend_mi355x_graph_compute_static instead: the same plan and
// kernels, launched eagerly, with the scratch in the fixed device array below.
//
// Every device the library runs on holds its own copy of the array (64 MiB)
// until the process ends. Calls on one device share it and it keeps the last
// call's contents: calls that overlap on one device race. No kernel of a plan
// relies on scratch starting at zero (every region is written before it is
// read in the same compute), so nothing is cleared between calls.
#include <mutex>

#include "ggml_mi355x.h"
#include "mi355x_exec.h"

static constexpr size_t kStaticScratchBytes = 64u << 20;

static __device__ __align__(256) char scratch[kStaticScratchBytes];

namespace mi355x {

// this device's address of `scratch` (the name is a host-side stand-in, not a
// device address); looked up once per device with the device current
static char * device_scratch(device_state * dev) {
    std::call_once(dev->static_once, [dev] {
        void * ptr = nullptr;
        hipError_t e = hipSetDevice(dev->hip_id);
        if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            (void) hipGetLastError();
            std::fprintf(stderr, "mi355x: no address for the fixed scratch array on %s: %s\n", dev->name.c_str(),
                         hipGetErrorString(e));
            dev->static_err = e;
            return;
        }
        dev->static_scratch = (char *) ptr;
    });
    return dev->static_scratch;
}

size_t static_scratch_bytes() { return kStaticScratchBytes; }

}  // namespace mi355x

using namespace mi355x;

extern "C" enum ggml_status ggml_backend_mi355x_graph_compute_static(ggml_backend_t backend,
                                                                     struct ggml_cgraph * cgraph) {
    backend_state * be = backend_of(backend);
    if (!be || !cgraph) return GGML_STATUS_FAILED;
    char * base = device_scratch(be->dev);
    if (!base) return GGML_STATUS_FAILED;
    const enum ggml_status st = graph_compute_in(be, cgraph, base, kStaticScratchBytes);
    be->last_status = (int) st;
    return st;
}

extern "C" size_t ggml_backend_mi355x_static_scratch_bytes(void) { return kStaticScratchBytes; }

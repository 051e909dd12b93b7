// sync_latency.hip -- what it costs, on one MI355X, to order dependent work
// inside a decode step. A decode step of the Qwen3-0.6B-shaped decoder is a
// chain of ~145 dependent launches whose data (1-4 MB of weights each) takes
// well under a microsecond of HBM time, so the price of the ordering itself
// decides the step time. Measured here:
//
//   boundary   a chain of dependent kernels replayed from a HIP graph
//              (time per kernel, tiny and 256..1024-workgroup grids)
//   barrier    a grid barrier inside one cooperatively launched persistent
//              kernel: one counter (relaxed, or release/acquire at agent
//              scope), or one counter per XCD group then a global one
//   flag       a point-to-point flag between two workgroups, on different
//              XCDs and on the same XCD (one round trip per two hops)
//   exchange   a barrier that also publishes 1 KB per workgroup which the
//              next workgroup reads back and checks: plain stores behind
//              release/acquire fences, or agent-coherent relaxed atomic
//              stores/loads with only a wait for the stores before the arrive
//   overlap    a barrier whose workgroups first request a 16 KB slice of a
//              1 GiB buffer (the next phase's weights) and consume it after
//              the wait, against the same stream with no barrier
//
// Every wait polls a wall clock and gives up after 50 ms, raising an abort
// flag that every other wait also watches, so every wave always exits; the
// persistent kernels are launched cooperatively (the runtime refuses a grid
// that cannot be co-resident). Output: a markdown table on stdout.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                             \
    do {                                                                                     \
        hipError_t e_ = (x);                                                                 \
        if (e_ != hipSuccess) {                                                              \
            std::fprintf(stderr, "%s failed at line %d: %s\n", #x, __LINE__, hipGetErrorString(e_)); \
            std::exit(1);                                                                    \
        }                                                                                    \
    } while (0)

namespace {

constexpr uint64_t kTimeoutTicks = 5000000;  // 50 ms of the 100 MHz wall clock
constexpr int kThreads = 256;

struct sync_state {
    unsigned * ctr;      // [0] global counter, [16 * (1 + g)] group counters (own 64 B lines)
    unsigned * abort;    // set by a wait that timed out
    unsigned * errors;   // mismatches seen by the exchange check
    unsigned * xcc;      // XCC id of each workgroup
};

__device__ __forceinline__ unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xF;
}

__device__ __forceinline__ unsigned ld_relaxed(const unsigned * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_acquire(const unsigned * p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

// wait until *p >= target (or the abort flag rises / 50 ms pass); false on give-up
template <bool ACQ>
__device__ bool wait_ge(const unsigned * p, unsigned target, unsigned * abort) {
    const uint64_t t0 = wall_clock64();
    for (;;) {
        const unsigned v = ACQ ? ld_acquire(p) : ld_relaxed(p);
        if (v >= target) return true;
        if (ld_relaxed(abort)) return false;
        if (wall_clock64() - t0 > kTimeoutTicks) {
            __hip_atomic_store(abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
}

// MODE 0: one counter, relaxed; 1: one counter, release arrive / acquire wait;
// 2: per-group counters (workgroup i in group i % 8, the XCD it is dealt to)
// then the global counter, relaxed
template <int MODE>
__device__ __forceinline__ bool grid_barrier(const sync_state & s, unsigned round) {
    bool ok = true;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned G = gridDim.x;
        if (MODE == 0) {
            __hip_atomic_fetch_add(s.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = wait_ge<false>(s.ctr, round * G, s.abort);
        } else if (MODE == 1) {
            __hip_atomic_fetch_add(s.ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            ok = wait_ge<true>(s.ctr, round * G, s.abort);
        } else {
            const unsigned grp = blockIdx.x & 7;
            const unsigned members = (G - grp + 7) / 8;
            unsigned * gc = s.ctr + 16 * (1 + grp);
            const unsigned old = __hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old + 1 == round * members) __hip_atomic_fetch_add(s.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned groups = G < 8 ? G : 8;
            ok = wait_ge<false>(s.ctr, round * groups, s.abort);
        }
    }
    __shared__ int s_ok;
    if (threadIdx.x == 0) s_ok = ok;
    __syncthreads();
    return s_ok;
}

__global__ void k_tiny(unsigned * buf) {
    if (threadIdx.x == 0) buf[blockIdx.x] += 1u;
}

template <int MODE>
__global__ void k_barrier(sync_state s, int rounds) {
    if (threadIdx.x == 0) s.xcc[blockIdx.x] = xcc_id();
    for (int r = 1; r <= rounds; r++) {
        if (!grid_barrier<MODE>(s, (unsigned) r)) return;
    }
}

// workgroups a and b bounce a flag `rounds` times; the others exit at once
__global__ void k_pingpong(sync_state s, int a, int b, int rounds) {
    if (threadIdx.x == 0) s.xcc[blockIdx.x] = xcc_id();
    const int me = (int) blockIdx.x;
    if ((me != a && me != b) || threadIdx.x != 0) return;
    unsigned * flag = s.ctr;
    for (int r = 0; r < rounds; r++) {
        const unsigned want = 2u * (unsigned) r + (me == a ? 0u : 1u);
        if (!wait_ge<false>(flag, want, s.abort)) return;
        __hip_atomic_store(flag, want + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// publish kThreads floats per workgroup each round, barrier, read the next
// workgroup's slab back and count stale values
template <bool COHERENT>
__global__ void k_exchange(sync_state s, unsigned * slab, int rounds) {
    const unsigned G = gridDim.x, me = blockIdx.x, nb = (me + 1) % G;
    for (int r = 1; r <= rounds; r++) {
        const unsigned val = ((unsigned) r << 12) | me;
        unsigned * mine = slab + ((size_t) (r & 1) * G + me) * kThreads + threadIdx.x;
        const unsigned * theirs = slab + ((size_t) (r & 1) * G + nb) * kThreads + threadIdx.x;
        if (COHERENT) {
            __hip_atomic_store(mine, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);  // the store is acknowledged before this wave arrives
            if (!grid_barrier<0>(s, (unsigned) r)) return;
            const unsigned got = ld_relaxed(theirs);
            if (got != (((unsigned) r << 12) | nb)) atomicAdd(s.errors, 1u);
        } else {
            *mine = val;
            if (!grid_barrier<1>(s, (unsigned) r)) return;
            const unsigned got = *(volatile const unsigned *) theirs;
            if (got != (((unsigned) r << 12) | nb)) atomicAdd(s.errors, 1u);
        }
    }
}

// each round every workgroup requests its 16 KB slice of round r, then
// (BARRIER) waits at the grid barrier, then consumes the slice
template <bool BARRIER>
__global__ void k_overlap(sync_state s, const uint4 * big, size_t slices, int rounds, unsigned * sink) {
    const unsigned G = gridDim.x;
    unsigned acc = 0;
    for (int r = 1; r <= rounds; r++) {
        const size_t slice = ((size_t) r * G + blockIdx.x) % slices;
        const uint4 * p = big + slice * (16384 / 16);
        uint4 v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = p[i * kThreads + threadIdx.x];
        if (BARRIER && !grid_barrier<0>(s, (unsigned) r)) return;
#pragma unroll
        for (int i = 0; i < 4; i++) acc += v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads
}

struct bench {
    sync_state s{};
    unsigned * d_mem = nullptr;
    hipEvent_t e0, e1;
    int n_cu = 0;

    bench() {
        hipDeviceProp_t p;
        CHECK(hipGetDeviceProperties(&p, 0));
        n_cu = p.multiProcessorCount;
        std::printf("device: %s, %d CUs, cooperative launch %d\n\n", p.gcnArchName, n_cu, p.cooperativeLaunch);
        // ctr (16 x 9 lines) | abort | errors | xcc[4096]
        CHECK(hipMalloc(&d_mem, (size_t) (16 * 9 + 64 + 64 + 4096) * sizeof(unsigned)));
        s.ctr = d_mem;
        s.abort = d_mem + 16 * 9;
        s.errors = s.abort + 64;
        s.xcc = s.errors + 64;
        CHECK(hipEventCreate(&e0));
        CHECK(hipEventCreate(&e1));
    }
    void reset() {
        CHECK(hipMemset(d_mem, 0, (size_t) (16 * 9 + 64 + 64) * sizeof(unsigned)));
        CHECK(hipDeviceSynchronize());
    }
    unsigned host_word(const unsigned * p) {
        unsigned v;
        CHECK(hipMemcpy(&v, p, sizeof(v), hipMemcpyDeviceToHost));
        return v;
    }
    template <typename F>
    float time_ms(F && launch) {
        CHECK(hipEventRecord(e0, 0));
        launch();
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        return ms;
    }
    // cooperative launch of `kern` with `grid` workgroups; false if refused
    template <typename... A>
    bool coop(void (*kern)(A...), int grid, A... args) {
        void * argv[] = {(void *) &args...};
        const hipError_t e =
            hipLaunchCooperativeKernel((const void *) kern, dim3(grid), dim3(kThreads), argv, 0, 0);
        if (e != hipSuccess) {
            (void) hipGetLastError();
            return false;
        }
        return true;
    }
};

void row(const char * what, int grid, double us, const char * note) {
    std::printf("| %s | %d | %.3f | %s |\n", what, grid, us, note);
}

}  // namespace

int main() {
    bench b;
    std::printf("| measurement | workgroups | us per event | note |\n|---|---|---|---|\n");

    // kernel boundaries inside a HIP graph
    for (int grid : {1, b.n_cu, 4 * b.n_cu}) {
        const int chain = 200;
        hipStream_t st;
        CHECK(hipStreamCreate(&st));
        hipGraph_t g;
        hipGraphExec_t ge;
        CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < chain; i++) hipLaunchKernelGGL(k_tiny, dim3(grid), dim3(kThreads), 0, st, b.s.xcc);
        CHECK(hipStreamEndCapture(st, &g));
        CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        for (int w = 0; w < 3; w++) CHECK(hipGraphLaunch(ge, st));
        CHECK(hipStreamSynchronize(st));
        const int reps = 10;
        CHECK(hipEventRecord(b.e0, st));
        for (int w = 0; w < reps; w++) CHECK(hipGraphLaunch(ge, st));
        CHECK(hipEventRecord(b.e1, st));
        CHECK(hipEventSynchronize(b.e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, b.e0, b.e1));
        row("boundary: dependent kernel in a HIP graph", grid, 1000.0 * ms / (reps * chain), "200-kernel chain, 10 replays");
        CHECK(hipGraphExecDestroy(ge));
        CHECK(hipGraphDestroy(g));
        CHECK(hipStreamDestroy(st));
    }

    const int rounds = 2000;
    struct mode_t {
        void (*k)(sync_state, int);
        const char * name;
    } modes[] = {{k_barrier<0>, "barrier: one counter, relaxed"},
                 {k_barrier<1>, "barrier: one counter, release/acquire (agent)"},
                 {k_barrier<2>, "barrier: 8 group counters, then global, relaxed"}};
    for (const mode_t & m : modes) {
        for (int grid : {b.n_cu / 8, b.n_cu, 2 * b.n_cu, 4 * b.n_cu}) {
            b.reset();
            (void) b.coop(m.k, grid, b.s, 10);  // warm-up
            CHECK(hipDeviceSynchronize());
            b.reset();
            bool launched = false;
            const float ms = b.time_ms([&] { launched = b.coop(m.k, grid, b.s, rounds); });
            if (!launched) {
                row(m.name, grid, 0.0, "cooperative launch refused");
                continue;
            }
            const unsigned ab = b.host_word(b.s.abort);
            row(m.name, grid, 1000.0 * ms / rounds, ab ? "TIMED OUT (aborted)" : "2000 rounds");
        }
    }

    // point-to-point flag between two workgroups (one hop = half a round)
    {
        const int grid = 16, pp_rounds = 4000;
        std::vector<unsigned> x(grid);
        for (int pair = 0; pair < 2; pair++) {
            const int a = 0, bb = pair == 0 ? 1 : 8;
            b.reset();
            bool launched = false;
            const float ms = b.time_ms([&] { launched = b.coop(k_pingpong, grid, b.s, a, bb, pp_rounds); });
            CHECK(hipMemcpy(x.data(), b.s.xcc, grid * sizeof(unsigned), hipMemcpyDeviceToHost));
            char note[128];
            std::snprintf(note, sizeof(note), "workgroups %d and %d on XCC %u and %u%s", a, bb, x[a], x[bb],
                          b.host_word(b.s.abort) ? ", TIMED OUT" : "");
            if (!launched) std::snprintf(note, sizeof(note), "cooperative launch refused");
            row("flag: one hop between two workgroups", 2, 1000.0 * ms / (2.0 * pp_rounds), note);
        }
        // which XCC each of the first 16 workgroups of a grid ran on
        std::printf("\nworkgroup -> XCC of a 16-workgroup grid:");
        for (int i = 0; i < grid; i++) std::printf(" %u", x[i]);
        std::printf("\n\n| measurement | workgroups | us per event | note |\n|---|---|---|---|\n");
    }

    // barrier with 1 KB per workgroup published and checked
    {
        unsigned * slab;
        const int maxg = 4 * b.n_cu;
        CHECK(hipMalloc(&slab, (size_t) 2 * maxg * kThreads * sizeof(unsigned)));
        CHECK(hipMemset(slab, 0, (size_t) 2 * maxg * kThreads * sizeof(unsigned)));
        for (int coherent = 0; coherent < 2; coherent++) {
            for (int grid : {b.n_cu, 2 * b.n_cu}) {
                b.reset();
                bool launched = false;
                auto k = coherent ? k_exchange<true> : k_exchange<false>;
                const float ms = b.time_ms([&] { launched = b.coop(k, grid, b.s, slab, rounds); });
                char note[160];
                std::snprintf(note, sizeof(note), "%u stale values of %llu read%s", b.host_word(b.s.errors),
                              (unsigned long long) rounds * grid * kThreads, b.host_word(b.s.abort) ? ", TIMED OUT" : "");
                if (!launched) std::snprintf(note, sizeof(note), "cooperative launch refused");
                row(coherent ? "exchange: relaxed agent-coherent stores/loads, relaxed barrier"
                             : "exchange: plain stores/loads, release/acquire barrier",
                    grid, 1000.0 * ms / rounds, note);
            }
        }
        CHECK(hipFree(slab));
    }

    // does a request issued before the barrier hide under it?
    {
        const size_t bytes = (size_t) 1 << 30, slices = bytes / 16384;
        uint4 * big;
        unsigned * sink;
        CHECK(hipMalloc(&big, bytes));
        CHECK(hipMalloc(&sink, 64));
        CHECK(hipMemset(big, 1, bytes));
        const int orounds = 256;
        for (int grid : {b.n_cu, 2 * b.n_cu}) {
            for (int withb = 0; withb < 2; withb++) {
                b.reset();
                bool launched = false;
                auto k = withb ? k_overlap<true> : k_overlap<false>;
                const uint4 * cbig = big;
                const float ms = b.time_ms([&] { launched = b.coop(k, grid, b.s, cbig, slices, orounds, sink); });
                char note[160];
                std::snprintf(note, sizeof(note), "16 KB per workgroup per round = %.2f MB a round, %.0f GB/s%s",
                              grid * 16384.0 / 1e6, (double) grid * 16384.0 * orounds / (ms * 1e6),
                              b.host_word(b.s.abort) ? ", TIMED OUT" : "");
                if (!launched) std::snprintf(note, sizeof(note), "cooperative launch refused");
                row(withb ? "overlap: slice requested, barrier, slice consumed" : "overlap: slices streamed, no barrier",
                    grid, 1000.0 * ms / orounds, note);
            }
        }
        CHECK(hipFree(big));
        CHECK(hipFree(sink));
    }
    CHECK(hipFree(b.d_mem));
    return 0;
}

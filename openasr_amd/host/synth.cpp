// synth.cpp -- deterministic synthetic inputs for the decoder workloads:
// random-init weights N(0, 0.02), N(0, 1) audio prefixes and encoder states.
// The generator is counter based (splitmix64 of (seed, stream, index) feeding
// Box-Muller), so any slice of any tensor can be produced independently and
// in parallel, and every run on every machine sees the same values.

#include <cmath>
#include <cstdint>

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ULL;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
    return x ^ (x >> 31);
}

// uniform in (0, 1], 53-bit resolution
inline double unit(uint64_t r) { return ((double) (r >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

}  // namespace

extern "C" {

// out[i] = mean + std * N(0,1) for i in [0, n), values indexed from `first`
void oa_synth_normal(uint64_t seed, uint64_t stream, int64_t first, int64_t n, float mean, float std_dev,
                     float * out) {
    const uint64_t key = splitmix64(seed ^ splitmix64(stream * 0x632be59bd9b4e019ULL + 1));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const int64_t g = first + i;
        const uint64_t pair = (uint64_t) (g >> 1);
        const uint64_t r1 = splitmix64(key ^ (2 * pair));
        const uint64_t r2 = splitmix64(key ^ (2 * pair + 1));
        const double rad = std::sqrt(-2.0 * std::log(unit(r1)));
        const double ang = 6.283185307179586476925286766559 * unit(r2);
        const double z = (g & 1) ? rad * std::sin(ang) : rad * std::cos(ang);
        out[i] = (float) (mean + std_dev * z);
    }
}

// uniform integers in [0, bound)
void oa_synth_uniform_i32(uint64_t seed, uint64_t stream, int64_t n, int32_t bound, int32_t * out) {
    const uint64_t key = splitmix64(seed ^ splitmix64(stream * 0x632be59bd9b4e019ULL + 7));
    for (int64_t i = 0; i < n; i++) out[i] = (int32_t) (splitmix64(key ^ (uint64_t) i) % (uint64_t) bound);
}

}  // extern "C"

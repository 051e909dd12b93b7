// mi355x_common.h -- shared definitions for the gfx950 backend: error
// handling, tensor views passed to kernels, block formats and device helpers.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "ggml_abi.h"

#define MI_CHECK(expr)                                                                                   \
    do {                                                                                                 \
        hipError_t err__ = (expr);                                                                       \
        if (err__ != hipSuccess) {                                                                       \
            std::fprintf(stderr, "mi355x: %s failed at %s:%d: %s\n", #expr, __FILE__, __LINE__,         \
                         hipGetErrorString(err__));                                                      \
            mi355x::note_hip_error(err__);                                                               \
        }                                                                                                \
    } while (0)

namespace mi355x {

void note_hip_error(hipError_t err);

constexpr int kWave = 64;

// A tensor as a kernel sees it: base pointer plus element counts and byte
// strides in ggml order (dim 0 innermost).
struct tview {
    char * data;
    int64_t ne[4];
    int64_t nb[4];
};

inline tview make_view(const ggml_tensor * t) {
    tview v;
    v.data = (char *) t->data;
    for (int i = 0; i < 4; i++) {
        v.ne[i] = t->ne[i];
        v.nb[i] = (int64_t) t->nb[i];
    }
    return v;
}

// Q8_0 weights are stored per row as [K int8 quants][K/32 f16 scales]
// (same byte count as ggml's interleaved 34-byte blocks) so a lane can issue
// aligned 16-byte loads of quants. Conversion happens in set/get_tensor.
inline size_t q8_0_row_bytes(int64_t k) { return (size_t) (k / 32) * 34; }

// Activations quantized for a Q8_0 weight: per column K int8 + K/32 f32
// scales (the f32 value of the f16-rounded scale ggml stores).
// Activations quantized for a Q4_K weight (ggml's Q8_K): per column K int8,
// K/256 f32 scales and K/16 int16 partial sums.
struct act_layout {
    int64_t q_stride;   // bytes between columns of quants
    int64_t d_stride;   // floats between columns of scales
    int64_t ss_stride;  // int16 between columns of 32-element sums (Q8_K only)
};

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float round_to_half(float f) { return __half2float(__float2half_rn(f)); }

__device__ __forceinline__ int dot4_i8(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, W);
    return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, W));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<kWave>(v); }

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// exp and sin/cos as a fixed sequence of IEEE double operations rounded once
// to f32 (the library is built without FMA contraction). The CPU reference
// evaluates the identical sequence, so host and device agree bit for bit and
// both are within one rounding of the exact value.
__device__ __forceinline__ float expf_det(float x) {
    if (x != x) return x;
    if (x > 88.72284f) return INFINITY;
    if (x < -103.97208f) return 0.0f;
    const double xd = (double) x;
    const double k = rint(xd * 1.4426950408889634074);
    const double r = (xd - k * 0.69314718055994528623) - k * 2.3190468138462996154e-17;
    double p = 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return (float) ldexp(p, (int) k);
}

// erf(x) as a fixed sequence of IEEE double operations rounded once to f32:
// the Maclaurin series 2/sqrt(pi) x sum_{n < 64} a_n (x^2)^n, a_n = (-1)^n /
// (n! (2n+1)) rounded to the nearest double, by Horner's rule from n = 63
// down with separate multiplies and adds, for |x| < 4 (the largest partial
// value there is ~1e5, so the double result is good to ~1e-10 absolute, far
// inside half an f32 ulp); +-1 beyond, where the exact value rounds to +-1
// in f32. The CPU reference runs the same table and steps.
static constexpr double kErfCoef[64] = {
    0x1.0000000000000p+0, -0x1.5555555555555p-2, 0x1.999999999999ap-4, -0x1.8618618618618p-6,
    0x1.2f684bda12f68p-8, -0x1.8d3018d3018d3p-11, 0x1.c01c01c01c01cp-14, -0x1.bbd779334ef0bp-17,
    0x1.87a00187a0018p-20, -0x1.3777c55568ccdp-23, 0x1.c2e3054870b38p-27, -0x1.2b67310aa9f3ap-30,
    0x1.6f448e13e85e1p-34, -0x1.a289ee7e40f74p-38, 0x1.bd577e658d020p-42, -0x1.bc6250fb14231p-46,
    0x1.a173a167fba4dp-50, -0x1.7271cbe5863ecp-54, 0x1.377c2110f2083p-58, -0x1.f1b4073b34a68p-63,
    0x1.7abd72258fb6ep-67, -0x1.13246abce1bddp-71, 0x1.7e6b81382cd42p-76, -0x1.fd6bebd65107ap-81,
    0x1.45c0a838efe59p-85, -0x1.909c9de3a31c5p-90, 0x1.da7460554e5dbp-95, -0x1.0eef30fa10d2cp-99,
    0x1.2ac65385f79acp-104, -0x1.3e81bb5701ac5p-109, 0x1.4899fcdef0a8dp-114, -0x1.486eea20c2656p-119,
    0x1.3e53defc4e233p-124, -0x1.2b778acc3dedfp-129, 0x1.11ae81077a49ep-134, -0x1.e6597092ccbf0p-140,
    0x1.a47767f2a3c32p-145, -0x1.61f30bc3acd1ap-150, 0x1.22521d98f98a9p-155, -0x1.d05cc9e3507c9p-161,
    0x1.6a513f56f8a2fp-166, -0x1.13f85fc9e143ep-171, 0x1.9aa19d4d16643p-177, -0x1.2a8fa59ffec31p-182,
    0x1.a8830736a5123p-188, -0x1.273d8edcec957p-193, 0x1.91ef82b367a95p-199, -0x1.0be5a4cd94283p-204,
    0x1.5dd4c9219115ap-210, -0x1.bfb10e0f68c50p-216, 0x1.18d952ef00889p-221, -0x1.59982b2e94840p-227,
    0x1.a13ec00b39f6fp-233, -0x1.ee6cefaa5a158p-239, 0x1.1f9dec94da5f8p-244, -0x1.48a6b3820b441p-250,
    0x1.70f41ac13e2a1p-256, -0x1.970f1cb2ad53fp-262, 0x1.b97d90d3e603bp-268, -0x1.d6db2a7c68dcbp-274,
    0x1.edf1e6e4658a9p-280, -0x1.fdcf88bbf71dbp-286, 0x1.02eb04e5f82f5p-291, -0x1.02e2bc1b5790ep-297,
};

__device__ __forceinline__ float erff_det(float x) {
    if (x != x) return x;
    const double xd = (double) x;
    if (xd >= 4.0) return 1.0f;
    if (xd <= -4.0) return -1.0f;
    const double t = xd * xd;
    double p = kErfCoef[63];
#pragma unroll
    for (int n = 62; n >= 0; n--) p = p * t + kErfCoef[n];
    return (float) (xd * p * 1.1283791670955125739);
}

// GELU_ERF (ggml_vec_gelu_erf_f32): 0.5 x (1 + erf(x / sqrt 2)) in f32
__device__ __forceinline__ float gelu_erf_det(float x) { return 0.5f * x * (1.0f + erff_det(x * 0.70710678118654752440f)); }

// gelu_erf_det of NV values at once: the same operations per value (so the
// same bits), the NV Horner chains interleaved step by step so that a lane
// has NV independent double operations in flight instead of one chain; the
// series is evaluated for every value and the NaN / |x| >= 4 cases selected
// after it (their series result is discarded)
template <int NV>
__device__ __forceinline__ void gelu_erf_det_n(float (&x)[NV]) {
    double xd[NV], t[NV], p[NV];
#pragma unroll
    for (int e = 0; e < NV; e++) {
        xd[e] = (double) (x[e] * 0.70710678118654752440f);
        t[e] = xd[e] * xd[e];
        p[e] = kErfCoef[63];
    }
#pragma unroll
    for (int n = 62; n >= 0; n--)
#pragma unroll
        for (int e = 0; e < NV; e++) p[e] = p[e] * t[e] + kErfCoef[n];
#pragma unroll
    for (int e = 0; e < NV; e++) {
        const float a = x[e] * 0.70710678118654752440f;
        float er = (float) (xd[e] * p[e] * 1.1283791670955125739);
        if (xd[e] >= 4.0) er = 1.0f;
        if (xd[e] <= -4.0) er = -1.0f;
        if (a != a) er = a;
        x[e] = 0.5f * x[e] * (1.0f + er);
    }
}

__device__ __forceinline__ void sincosf_det(float x, float & s_out, float & c_out) {
    const double xd = (double) x;
    const double k = rint(xd * 0.63661977236758134308);
    const double r = (xd - k * 1.5707963267341256458) - k * 6.0771005065061922341e-11;
    const double r2 = r * r;
    double s = -1.0 / 355687428096000.0;
    s = s * r2 + 1.0 / 1307674368000.0;
    s = s * r2 - 1.0 / 6227020800.0;
    s = s * r2 + 1.0 / 39916800.0;
    s = s * r2 - 1.0 / 362880.0;
    s = s * r2 + 1.0 / 5040.0;
    s = s * r2 - 1.0 / 120.0;
    s = s * r2 + 1.0 / 6.0;
    s = r - (r * r2) * s;
    double c = 1.0 / 6402373705728000.0;
    c = c * r2 - 1.0 / 20922789888000.0;
    c = c * r2 + 1.0 / 87178291200.0;
    c = c * r2 - 1.0 / 479001600.0;
    c = c * r2 + 1.0 / 3628800.0;
    c = c * r2 - 1.0 / 40320.0;
    c = c * r2 + 1.0 / 720.0;
    c = c * r2 - 1.0 / 24.0;
    c = c * r2 + 0.5;
    c = 1.0 - r2 * c;
    const int q = (int) (((long long) k) & 3);
    double so, co;
    if (q == 0) {
        so = s;
        co = c;
    } else if (q == 1) {
        so = c;
        co = -s;
    } else if (q == 2) {
        so = -s;
        co = -c;
    } else {
        so = -c;
        co = s;
    }
    s_out = (float) so;
    c_out = (float) co;
}

}  // namespace mi355x

// GGML_OP_IM2COL: the column matrix of a 2-D (or 1-D) convolution, the
// first half of ggml_conv_2d as the Qwen audio encoder's stem uses it
// (nn/conv.rs:82-110, cpu_graph.rs:5191-5246). Pure index work, bound by
// HBM. The line form: a workgroup takes one output line (image n, output row
// oh: OW column rows) and a block of input channels, reads the KH input rows
// the line's taps touch for those channels into LDS (consecutive lanes,
// consecutive input elements) and writes each column row's run of
// channels x taps (consecutive lanes, consecutive output elements; a 16-byte
// f32 or 8-byte f16 store of four when the runs allow). The element form
// (any shape): a lane writes V consecutive elements of one column row,
// splitting its first flat index once by multiply-and-shift division and
// stepping the taps by carries. A tap in the padding is written as zero; an
// in-range tap is copied (f32) or rounded to nearest-even (f16),
// bit-identical to ggml-cpu.

#include <algorithm>
#include <type_traits>

#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {
namespace {

// n / d for n < 2^31: m = ceil(2^(31 + l) / d), l = ceil(log2 d), so that
// m d - 2^(31 + l) < d <= 2^l and floor(n / d) = floor(n m / 2^(31 + l))
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", 1994, theorem 4.2 with N = 31); n m < 2^64.
struct fast_div {
    uint64_t m;
    uint32_t d;
    int sh;
};

fast_div make_fast_div(uint32_t d) {
    int l = 0;
    while ((1ull << l) < d) l++;
    fast_div f;
    f.d = d;
    f.sh = 31 + l;
    f.m = ((1ull << f.sh) + d - 1) / d;
    return f;
}

__device__ __forceinline__ uint32_t div_by(uint32_t n, const fast_div & f) {
    return (uint32_t) (((uint64_t) n * f.m) >> f.sh);
}

struct im2col_divs {
    fast_div K, OW, OH, KW, KH;
};

template <typename DT>
__device__ __forceinline__ void im2col_store(DT * p, const float (&v)[1]) {
    *p = (DT) v[0];
}
__device__ __forceinline__ void im2col_store(float * p, const float (&v)[4]) {
    *(float4 *) p = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void im2col_store(_Float16 * p, const float (&v)[4]) {
    const uint32_t lo = (uint32_t) float_to_half_bits(v[0]) | ((uint32_t) float_to_half_bits(v[1]) << 16);
    const uint32_t hi = (uint32_t) float_to_half_bits(v[2]) | ((uint32_t) float_to_half_bits(v[3]) << 16);
    *(uint2 *) p = make_uint2(lo, hi);
}

// the split layout (im2col_args::split): flat element f of the column matrix
// (K % 8 == 0, so a row starts a group) goes to bf16 hi at byte 32 (f / 8) +
// 2 (f % 8) and lo 16 bytes further; V = 4 values start on a 4-element boundary
template <int V>
__device__ __forceinline__ void im2col_split_store(float * dst, int64_t f, const float (&v)[V]) {
    uint16_t h[V], l[V];
#pragma unroll
    for (int e = 0; e < V; e++) {
        const __bf16 xh = (__bf16) v[e];
        h[e] = __builtin_bit_cast(uint16_t, xh);
        l[e] = __builtin_bit_cast(uint16_t, (__bf16) (v[e] - (float) xh));
    }
    char * p = (char *) dst + (f >> 3) * 32 + (f & 7) * 2;
    if constexpr (V == 4) {
        *(uint2 *) p = make_uint2(h[0] | ((uint32_t) h[1] << 16), h[2] | ((uint32_t) h[3] << 16));
        *(uint2 *) (p + 16) = make_uint2(l[0] | ((uint32_t) l[1] << 16), l[2] | ((uint32_t) l[3] << 16));
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) {
            ((uint16_t *) p)[e] = h[e];
            ((uint16_t *) (p + 16))[e] = l[e];
        }
    }
}
template <typename DT, int V>
__device__ __forceinline__ void im2col_put(DT * dst, int64_t f, const float (&v)[V], bool split) {
    if constexpr (std::is_same<DT, float>::value) {
        if (split) {
            im2col_split_store<V>(dst, f, v);
            return;
        }
    }
    im2col_store(dst + f, v);
}

// total < 2^31 and K % V == 0: lane t writes elements V t .. V t + V - 1
template <typename DT, int V>
__global__ __launch_bounds__(256) void k_im2col_v(DT * __restrict__ dst, const char * __restrict__ src, im2col_args a,
                                                  im2col_divs dv) {
    const uint32_t nt = (uint32_t) (a.total / V);
    const uint32_t stride = gridDim.x * 256u;
    for (uint32_t t = blockIdx.x * 256u + threadIdx.x; t < nt; t += stride) {
        const uint32_t i = t * V;
        const uint32_t r = div_by(i, dv.K), k = i - r * dv.K.d;
        const uint32_t r2 = div_by(r, dv.OW), ow = r - r2 * dv.OW.d;
        const uint32_t n = div_by(r2, dv.OH), oh = r2 - n * dv.OH.d;
        const uint32_t t2 = div_by(k, dv.KW);
        int kw = (int) (k - t2 * dv.KW.d);
        const uint32_t ic0 = div_by(t2, dv.KH);
        int kh = (int) (t2 - ic0 * dv.KH.d);
        int64_t ic = ic0;
        const char * img = src + (int64_t) n * a.nb_n;
        const int64_t iw0 = (int64_t) ow * a.s0 - a.p0, ih0 = (int64_t) oh * a.s1 - a.p1;
        float raw[V];
        bool in[V];
#pragma unroll
        for (int e = 0; e < V; e++) {
            const int64_t iw = iw0 + (int64_t) kw * a.d0, ih = ih0 + (int64_t) kh * a.d1;
            in[e] = iw >= 0 && iw < a.IW && ih >= 0 && ih < a.IH;
            const int64_t cw = in[e] ? iw : 0, ch = in[e] ? ih : 0;
            raw[e] = *(const float *) (img + ic * a.nb_c + ch * a.nb_h + cw * 4);
            if (++kw == a.KW) {
                kw = 0;
                if (++kh == a.KH) {
                    kh = 0;
                    ic++;
                }
            }
        }
        float v[V];
#pragma unroll
        for (int e = 0; e < V; e++) v[e] = in[e] ? raw[e] : 0.0f;
        im2col_put<DT, V>(dst, i, v, a.split);
    }
}

// The line form. Block b: line = b / nblk (n = line / OH, oh = line % OH),
// channels c0 = (b % nblk) cb .. + cb - 1 (fewer in the last block). LDS:
// tile[kh][c][iw], zeros for an input row outside the image. Output: row
// line OW + ow, elements c0 KH KW + j for j < run = cbn KH KW.
struct im2col_line {
    int cb, nblk, ic;
    fast_div run, taps, KW;  // run: cb KH KW (the full block's run); taps: KH KW
};

template <typename DT, int V>
__global__ __launch_bounds__(256) void k_im2col_line(DT * __restrict__ dst, const char * __restrict__ src, im2col_args a,
                                                     im2col_line L) {
    extern __shared__ float tile[];
    const int64_t line = blockIdx.x / L.nblk;
    const int c0 = (int) (blockIdx.x % L.nblk) * L.cb;
    const int cbn = L.ic - c0 < L.cb ? L.ic - c0 : L.cb;
    const int64_t n = line / a.OH, oh = line % a.OH;
    const int IW = (int) a.IW;
    const char * img = src + n * a.nb_n;
    // the taps' input rows into LDS
    for (int e = threadIdx.x; e < a.KH * cbn * IW; e += 256) {
        const int iw = e % IW, r = e / IW;
        const int c = r % cbn, kh = r / cbn;
        const int64_t ih = oh * a.s1 - a.p1 + (int64_t) kh * a.d1;
        float v = 0.0f;
        if (ih >= 0 && ih < a.IH) v = *(const float *) (img + (int64_t) (c0 + c) * a.nb_c + ih * a.nb_h + iw * 4);
        tile[(kh * L.cb + c) * IW + iw] = v;
    }
    __syncthreads();
    const uint32_t run = (uint32_t) cbn * L.taps.d;
    const uint32_t total = (uint32_t) a.OW * run;
    const int64_t out0 = line * a.OW * a.K + (int64_t) c0 * L.taps.d;  // flat index of the line's first element
    for (uint32_t i = threadIdx.x * V; i < total; i += 256 * V) {
        // run == the full block's run except in the last block: divide by it
        const uint32_t ow = run == L.run.d ? div_by(i, L.run) : i / run;
        const uint32_t j = i - ow * run;
        uint32_t c = div_by(j, L.taps);
        const uint32_t t = j - c * L.taps.d;
        const uint32_t khu = div_by(t, L.KW);
        int kh = (int) khu, kw = (int) (t - khu * L.KW.d);
        const int64_t iw0 = (int64_t) ow * a.s0 - a.p0;
        float v[V];
#pragma unroll
        for (int e = 0; e < V; e++) {
            const int64_t iw = iw0 + (int64_t) kw * a.d0;
            const bool in = iw >= 0 && iw < IW;
            const float x = tile[(kh * L.cb + (int) c) * IW + (in ? (int) iw : 0)];
            v[e] = in ? x : 0.0f;
            if (++kw == a.KW) {
                kw = 0;
                if (++kh == a.KH) {
                    kh = 0;
                    c++;
                }
            }
        }
        im2col_put<DT, V>(dst, out0 + (int64_t) ow * a.K + j, v, a.split);
    }
}

// any size: one lane per element, 64-bit index arithmetic
template <typename DT>
__global__ __launch_bounds__(256) void k_im2col(DT * __restrict__ dst, const char * __restrict__ src, im2col_args a) {
    const int64_t stride = (int64_t) gridDim.x * 256;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < a.total; i += stride) {
        const int64_t k = i % a.K;
        int64_t r = i / a.K;
        const int64_t ow = r % a.OW;
        r /= a.OW;
        const int64_t oh = r % a.OH;
        const int64_t n = r / a.OH;
        const int kw = (int) (k % a.KW);
        const int64_t t = k / a.KW;
        const int kh = (int) (t % a.KH);
        const int64_t ic = t / a.KH;
        const int64_t iw = ow * a.s0 + (int64_t) kw * a.d0 - a.p0;
        const int64_t ih = oh * a.s1 + (int64_t) kh * a.d1 - a.p1;
        float v[1] = {0.0f};
        if (iw >= 0 && iw < a.IW && ih >= 0 && ih < a.IH)
            v[0] = *(const float *) (src + n * a.nb_n + ic * a.nb_c + ih * a.nb_h + iw * 4);
        im2col_put<DT, 1>(dst, i, v, a.split);
    }
}

constexpr int kLineTileFloats = 8192;  // 32 KB of LDS a workgroup

template <typename DT>
void im2col_launch(DT * dst, const char * src, const im2col_args & a, hipStream_t s) {
    constexpr int64_t kMaxBlocks = 65536;
    const int64_t taps = (int64_t) a.KH * a.KW, ic = a.K / taps;
    const int64_t lines = (a.total / a.K) / a.OW;  // N OH
    int64_t cb = kLineTileFloats / std::max<int64_t>(1, a.KH * a.IW);
    if (cb >= 4) cb = cb / 4 * 4;
    cb = std::min<int64_t>(cb, ic);
    const int64_t nblk = cb > 0 ? (ic + cb - 1) / cb : 0;
    if (a.total < (1LL << 31) && cb >= 1 && lines * nblk < (1LL << 31) && a.OW * cb * taps < (1LL << 31)) {
        im2col_line L;
        L.cb = (int) cb;
        L.nblk = (int) nblk;
        L.ic = (int) ic;
        L.run = make_fast_div((uint32_t) (cb * taps));
        L.taps = make_fast_div((uint32_t) taps);
        L.KW = make_fast_div((uint32_t) a.KW);
        const bool vec = a.K % 4 == 0 && (cb * taps) % 4 == 0 && (uintptr_t) dst % (4 * sizeof(DT)) == 0;
        const size_t lds = (size_t) a.KH * cb * a.IW * sizeof(float);
        const dim3 grid((unsigned) (lines * nblk));
        if (vec) hipLaunchKernelGGL((k_im2col_line<DT, 4>), grid, dim3(256), lds, s, dst, src, a, L);
        else hipLaunchKernelGGL((k_im2col_line<DT, 1>), grid, dim3(256), lds, s, dst, src, a, L);
        return;
    }
    if (a.total < (1LL << 31)) {
        const im2col_divs dv{make_fast_div((uint32_t) a.K), make_fast_div((uint32_t) a.OW),
                             make_fast_div((uint32_t) a.OH), make_fast_div((uint32_t) a.KW),
                             make_fast_div((uint32_t) a.KH)};
        const bool vec = a.K % 4 == 0 && (uintptr_t) dst % (4 * sizeof(DT)) == 0;
        const int64_t nt = vec ? a.total / 4 : a.total;
        const dim3 grid((unsigned) std::min<int64_t>((nt + 255) / 256, kMaxBlocks));
        if (vec) hipLaunchKernelGGL((k_im2col_v<DT, 4>), grid, dim3(256), 0, s, dst, src, a, dv);
        else hipLaunchKernelGGL((k_im2col_v<DT, 1>), grid, dim3(256), 0, s, dst, src, a, dv);
    } else {
        const dim3 grid((unsigned) std::min<int64_t>((a.total + 255) / 256, kMaxBlocks));
        hipLaunchKernelGGL(k_im2col<DT>, grid, dim3(256), 0, s, dst, src, a);
    }
}

}  // namespace

void launch_im2col(void * dst, int dst_f16, const char * src, const im2col_args & a, hipStream_t s) {
    if (a.total <= 0) return;
    if (a.split && (dst_f16 || a.K % 8 != 0 || (uintptr_t) dst % 16 != 0)) {
        note_hip_error(hipErrorInvalidValue);
        return;
    }
    if (dst_f16) im2col_launch((_Float16 *) dst, src, a, s);
    else im2col_launch((float *) dst, src, a, s);
}

}  // namespace mi355x

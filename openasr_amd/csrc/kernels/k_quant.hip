// k_quant.hip -- activation quantizers that feed the integer dot products of
// MUL_MAT on Q8_0 / Q4_K weights (ggml-cpu converts src1 to the weight's
// vec_dot type before the dot: Q8_0 -> Q8_0, Q4_K -> Q8_K; the mul_mat call
// site is crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686).
//
// One wave covers 256 consecutive elements of one column, four per lane, so
// a Q8_0 block is an 8-lane group and a Q8_K block is the whole wave; the
// reductions stay inside the wave (no LDS, no barriers).
#include "../mi355x_common.h"
#include "../ops.h"
#include "../quant_dev.h"

namespace mi355x {

// Q8_0: one 8-lane group per 32-element block (quantize_q8_0_group).
// Output quants [col][K], scales [col][K/32] as the f32 value of the f16 scale.
__global__ __launch_bounds__(256) void k_quantize_q8_0(const char * __restrict__ src, int64_t K, int64_t ncols,
                                                       int64_t ne1, int64_t nb1, int64_t nb2,
                                                       int8_t * __restrict__ q, float * __restrict__ d) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t) blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    const int64_t chunks = (K + 255) / 256;
    const int64_t col = wave / chunks;
    if (col >= ncols) return;
    const int64_t e = (wave % chunks) * 256 + lane * 4;
    const int64_t i1 = col % ne1, i2 = col / ne1;
    const float * x = (const float *) (src + i1 * nb1 + i2 * nb2);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e < K) v = *(const float4 *) (x + e);
    const q8_0_lane o = quantize_q8_0_group(v);
    if (e < K) {
        *(char4 *) (q + col * K + e) = o.q;
        if ((lane & 7) == 0) d[col * (K / 32) + e / 32] = o.d;
    }
}

// Q8_K: one wave per 256-element block (quantize_q8_K_wave); sums over 32.
__global__ __launch_bounds__(256) void k_quantize_q8_K(const char * __restrict__ src, int64_t K, int64_t ncols,
                                                       int64_t ne1, int64_t nb1, int64_t nb2,
                                                       int8_t * __restrict__ q, float * __restrict__ d,
                                                       int16_t * __restrict__ ssum) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t) blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    const int64_t chunks = K / 256;
    const int64_t col = wave / chunks;
    if (col >= ncols) return;
    const int64_t blk = wave % chunks;
    const int64_t e = blk * 256 + lane * 4;
    const int64_t i1 = col % ne1, i2 = col / ne1;
    const float * x = (const float *) (src + i1 * nb1 + i2 * nb2);
    const q8_K_lane o = quantize_q8_K_wave(*(const float4 *) (x + e), lane);
    *(char4 *) (q + col * K + e) = o.q;
    if ((lane & 7) == 0) ssum[col * (K / 32) + e / 32] = (int16_t) o.ssum;
    if (lane == 0) d[col * chunks + blk] = o.d;
}

static size_t al256(size_t v) { return (v + 255) / 256 * 256; }

size_t act_bytes(int wtype, int64_t K, int64_t ncols) {
    const size_t q = al256((size_t) (K * ncols));
    if (wtype == GGML_TYPE_Q8_0) return q + al256((size_t) (K / 32 * ncols) * 4);
    return q + al256((size_t) (K / 256 * ncols) * 4) + al256((size_t) (K / 32 * ncols) * 2);
}

act_buffers act_carve(int wtype, char * base, int64_t K, int64_t ncols) {
    act_buffers a;
    const size_t q = al256((size_t) (K * ncols));
    a.q = (int8_t *) base;
    a.d = (float *) (base + q);
    if (wtype == GGML_TYPE_Q8_0) {
        a.ssum = nullptr;
    } else {
        a.ssum = (int16_t *) (base + q + al256((size_t) (K / 256 * ncols) * 4));
    }
    return a;
}

void launch_quantize_act(const tview & src, int wtype, const act_buffers & out, hipStream_t stream) {
    const int64_t K = src.ne[0];
    const int64_t ncols = src.ne[1] * src.ne[2] * src.ne[3];
    const int64_t chunks = (K + 255) / 256;
    const int64_t waves = chunks * ncols;
    const int64_t blocks = (waves + 3) / 4;
    // columns are addressed as (i1, i2) with i2 folding dims 2 and 3; a
    // contiguous-rows source has nb3 == nb2 * ne2 in every graph we plan.
    if (wtype == GGML_TYPE_Q8_0) {
        hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned) blocks), dim3(256), 0, stream, src.data, K, ncols,
                           src.ne[1], src.nb[1], src.nb[2], out.q, out.d);
    } else {
        hipLaunchKernelGGL(k_quantize_q8_K, dim3((unsigned) blocks), dim3(256), 0, stream, src.data, K, ncols,
                           src.ne[1], src.nb[1], src.nb[2], out.q, out.d, out.ssum);
    }
}

}  // namespace mi355x

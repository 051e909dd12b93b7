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

namespace mi355x {

// Q8_0 (x86 ggml-cpu rule): d = amax/127 stored as f16, multiplier 127/amax,
// quants rounded half to even. Output quants [col][K], scales [col][K/32] as
// the f32 value of the f16 scale.
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
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = group_max<8>(amax);
    const float dd = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    if (e < K) {
        char4 o;
        o.x = (signed char) __float2int_rn(v.x * id);
        o.y = (signed char) __float2int_rn(v.y * id);
        o.z = (signed char) __float2int_rn(v.z * id);
        o.w = (signed char) __float2int_rn(v.w * id);
        *(char4 *) (q + col * K + e) = o;
        if ((lane & 7) == 0) d[col * (K / 32) + e / 32] = round_to_half(dd);
    }
}

// Q8_K (quantize_row_q8_K_ref): the signed value of largest magnitude (first
// one on ties) sets iscale = -127/max; d = 1/iscale; bsums over 16 quants.
__global__ __launch_bounds__(256) void k_quantize_q8_K(const char * __restrict__ src, int64_t K, int64_t ncols,
                                                       int64_t ne1, int64_t nb1, int64_t nb2,
                                                       int8_t * __restrict__ q, float * __restrict__ d,
                                                       int16_t * __restrict__ bsums) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t) blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    const int64_t chunks = K / 256;
    const int64_t col = wave / chunks;
    if (col >= ncols) return;
    const int64_t blk = wave % chunks;
    const int64_t e = blk * 256 + lane * 4;
    const int64_t i1 = col % ne1, i2 = col / ne1;
    const float * x = (const float *) (src + i1 * nb1 + i2 * nb2);
    const float4 v = *(const float4 *) (x + e);
    // per-lane winner: first of the four with the largest |x|
    float best = v.x, ab = fabsf(v.x);
    int bidx = lane * 4;
    if (fabsf(v.y) > ab) { ab = fabsf(v.y); best = v.y; bidx = lane * 4 + 1; }
    if (fabsf(v.z) > ab) { ab = fabsf(v.z); best = v.z; bidx = lane * 4 + 2; }
    if (fabsf(v.w) > ab) { ab = fabsf(v.w); best = v.w; bidx = lane * 4 + 3; }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float oab = __shfl_xor(ab, off);
        const float obest = __shfl_xor(best, off);
        const int oidx = __shfl_xor(bidx, off);
        if (oab > ab || (oab == ab && oidx < bidx)) {
            ab = oab;
            best = obest;
            bidx = oidx;
        }
    }
    int8_t * qo = q + col * K + e;
    if (ab == 0.0f) {
        *(char4 *) qo = make_char4(0, 0, 0, 0);
        if ((lane & 3) == 0) bsums[col * (K / 16) + e / 16] = 0;
        if (lane == 0) d[col * chunks + blk] = 0.0f;
        return;
    }
    const float iscale = -127.0f / best;
    const int a = min(127, __float2int_rn(iscale * v.x));
    const int b = min(127, __float2int_rn(iscale * v.y));
    const int c = min(127, __float2int_rn(iscale * v.z));
    const int w = min(127, __float2int_rn(iscale * v.w));
    *(char4 *) qo = make_char4((signed char) a, (signed char) b, (signed char) c, (signed char) w);
    int s = a + b + c + w;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) bsums[col * (K / 16) + e / 16] = (int16_t) s;
    if (lane == 0) d[col * chunks + blk] = 1.0f / iscale;
}

static size_t al256(size_t v) { return (v + 255) / 256 * 256; }

size_t act_bytes(int wtype, int64_t K, int64_t ncols) {
    const size_t q = al256((size_t) (K * ncols));
    if (wtype == GGML_TYPE_Q8_0) return q + al256((size_t) (K / 32 * ncols) * 4);
    return q + al256((size_t) (K / 256 * ncols) * 4) + al256((size_t) (K / 16 * ncols) * 2);
}

act_buffers act_carve(int wtype, char * base, int64_t K, int64_t ncols) {
    act_buffers a;
    const size_t q = al256((size_t) (K * ncols));
    a.q = (int8_t *) base;
    a.d = (float *) (base + q);
    if (wtype == GGML_TYPE_Q8_0) {
        a.bsums = nullptr;
    } else {
        a.bsums = (int16_t *) (base + q + al256((size_t) (K / 256 * ncols) * 4));
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
                           src.ne[1], src.nb[1], src.nb[2], out.q, out.d, out.bsums);
    }
}

}  // namespace mi355x

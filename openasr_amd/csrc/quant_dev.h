// quant_dev.h -- device-side activation quantizers shared by the stand-alone
// quantize kernels and by kernels that emit quantized activations for the
// next MUL_MAT in their epilogue. Both paths call these functions, so a
// column quantized in an epilogue carries the same bytes as one quantized by
// k_quantize_q8_0 / k_quantize_q8_K.
#pragma once

#include "mi355x_common.h"

namespace mi355x {

struct q8_0_lane {
    char4 q;
    float d;  // f32 value of the f16 block scale
};

// Q8_0 (x86 ggml-cpu rule) for 32 values held four per lane by an aligned
// 8-lane group: d = amax/127 stored as f16, multiplier 127/amax, quants
// rounded half to even.
__device__ __forceinline__ q8_0_lane quantize_q8_0_group(float4 v) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = group_max<8>(amax);
    const float dd = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    q8_0_lane o;
    o.q.x = (signed char) __float2int_rn(v.x * id);
    o.q.y = (signed char) __float2int_rn(v.y * id);
    o.q.z = (signed char) __float2int_rn(v.z * id);
    o.q.w = (signed char) __float2int_rn(v.w * id);
    o.d = round_to_half(dd);
    return o;
}

struct q8_K_lane {
    char4 q;
    int ssum;  // sum of the 32 quants of this lane's 8-lane group (same in all eight lanes)
    float d;   // block scale, uniform over the wave
};

// Q8_K (quantize_row_q8_K_ref) for 256 values held four per lane by a whole
// wave (lane l holds elements 4l..4l+3): the signed value of largest
// magnitude, first one on ties, sets iscale = -127/max; d = 1/iscale.
__device__ __forceinline__ q8_K_lane quantize_q8_K_wave(float4 v, int lane) {
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
    q8_K_lane o;
    if (ab == 0.0f) {
        o.q = make_char4(0, 0, 0, 0);
        o.ssum = 0;
        o.d = 0.0f;
        return o;
    }
    const float iscale = -127.0f / best;
    const int a = min(127, __float2int_rn(iscale * v.x));
    const int b = min(127, __float2int_rn(iscale * v.y));
    const int c = min(127, __float2int_rn(iscale * v.z));
    const int w = min(127, __float2int_rn(iscale * v.w));
    o.q = make_char4((signed char) a, (signed char) b, (signed char) c, (signed char) w);
    int s = a + b + c + w;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    o.ssum = s;
    o.d = 1.0f / iscale;
    return o;
}

}  // namespace mi355x

// mfma_units.h -- the integer-exact MFMA arithmetic of one quantized block
// unit, shared by the decode GEMVs (k_gemv_mfma.hip) and the tile GEMM
// (k_mmq.hip) so that every launch form forms the same f64 block sums.
//
// Orientation: activations are the A operand of v_mfma_i32_16x16x32_i8 (16
// columns x 32 k), a 16-row weight tile the B operand (32 k x 16 rows); lane l
// ends with weight row l % 16 and activation columns 4 (l / 16) + i. Call
// site of the op: crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
#pragma once
#include "mi355x_common.h"

namespace mi355x {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

typedef float v4f __attribute__((ext_vector_type(4)));

// the A operand of the min correction: the 32-element sums of sub-blocks g
// and g + 4 (g = lane / 16) of the lane's activation column, as floats
__device__ __forceinline__ void q4k_ssum_operand(const int16_t * col_ss, bool ok, int g, float (&ssa)[2]) {
    const int s0 = col_ss[g], s1 = col_ss[g + 4];
    ssa[0] = ok ? (float) s0 : 0.0f;
    ssa[1] = ok ? (float) s1 : 0.0f;
}

// one Q4_K super-block of a 16-row tile against four activation columns per
// lane: integer MFMA sums per sub-block, scaled by the 6-bit scales (exact
// 24-bit products), then d * isum - dmin * msum added to acc in f64. The min
// correction msum = sum over sub-blocks of min(row) * ssum(column) runs on
// two f32 MFMAs (16x16x4, sub-blocks g and g + 4 of lane group g): every
// product is below 2^18 and every partial sum below 2^21, so the f32 result
// is the exact integer. NCL: the lane's columns in use (1 when the launch
// has one column: lanes hold columns 4g + i, so only i = 0 can be live).
template <int NCL = 4>
__device__ __forceinline__ void q4k_unit(const uint4 & hdr, const long (&q)[4], const long (&af)[8],
                                         const float (&ad)[4], const float (&ssa)[2], double (&acc)[4]) {
    const int g = (threadIdx.x & 63) >> 4;
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;  // bytes 0-3, 4-7, 8-11 of scales[12]
    // B operand of the min correction: this row's mins of sub-blocks g and g + 4
    const float m0 = (float) ((s1 >> (8 * g)) & 63);
    const float m1 = (float) (((s2 >> (8 * g + 4)) & 0xF) | (((s1 >> (8 * g + 6)) & 3) << 4));
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    const v4f mlo = __builtin_amdgcn_mfma_f32_16x16x4f32(ssa[0], m0, z, 0, 0, 0);
    const v4f msum = __builtin_amdgcn_mfma_f32_16x16x4f32(ssa[1], m1, mlo, 0, 0, 0);
    int sc[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        sc[j] = (s0 >> (8 * j)) & 63;
        sc[j + 4] = ((s2 >> (8 * j)) & 0xF) | (((s0 >> (8 * j + 6)) & 3) << 4);
    }
    int isum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const long lo = q[c] & 0x0F0F0F0F0F0F0F0FL;
        const long hi = (q[c] >> 4) & 0x0F0F0F0F0F0F0F0FL;
        const v4i zi = {0, 0, 0, 0};
        const v4i c0v = mfma_i8(af[2 * c], lo, zi);
        const v4i c1v = mfma_i8(af[2 * c + 1], hi, zi);
#pragma unroll
        for (int i = 0; i < NCL; i++) isum[i] += __mul24(sc[2 * c], c0v[i]) + __mul24(sc[2 * c + 1], c1v[i]);
    }
    const float dw = half_bits_to_float((uint16_t) (hdr.x & 0xFFFF));
    const float dmw = half_bits_to_float((uint16_t) (hdr.x >> 16));
#pragma unroll
    for (int i = 0; i < NCL; i++) {
        const double da = (double) ad[i];
        const double d = (double) dw * da;
        const double dmin = (double) dmw * da;
        acc[i] += d * (double) isum[i] - dmin * (double) msum[i];
    }
}

// Q8_0 weights in the row-split layout [K quants][K/32 f16 scales]; a unit
// is a group of 8 blocks
constexpr int kQ8Group = 8;

// one Q8_0 block of a 16-row tile against four activation columns per lane:
// the MFMA's integer sum (|sum| < 2^19) times d_w * d_a (two halves: 22
// significant bits, exact in f32) is exact in f64, so one fused multiply-add
// rounds acc + term exactly as the separate product and sum do (NCL as for
// q4k_unit)
template <int NCL = 4>
__device__ __forceinline__ void q8_0_block(long af, long q, uint16_t ds, const float (&da)[4], double (&acc)[4]) {
    const v4i z = {0, 0, 0, 0};
    const v4i cc = mfma_i8(af, q, z);
    const float dw = half_bits_to_float(ds);
#pragma unroll
    for (int i = 0; i < NCL; i++) acc[i] = fma((double) cc[i], (double) (dw * da[i]), acc[i]);
}

// the first nb (<= kQ8Group) blocks of a group, in order
template <int NCL = 4>
__device__ __forceinline__ void q8_0_unit(const long (&q)[kQ8Group], const uint16_t (&ds)[kQ8Group],
                                          const long (&af)[kQ8Group], const float4 (&ad)[4][kQ8Group / 4], int nb,
                                          double (&acc)[4]) {
#pragma unroll
    for (int u = 0; u < kQ8Group; u++) {
        if (u < nb) {
            float da[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 d4 = ad[i][u / 4];
                da[i] = (u & 3) == 0 ? d4.x : (u & 3) == 1 ? d4.y : (u & 3) == 2 ? d4.z : d4.w;
            }
            q8_0_block<NCL>(af[u], q[u], ds[u], da, acc);
        }
    }
}

}  // namespace mi355x

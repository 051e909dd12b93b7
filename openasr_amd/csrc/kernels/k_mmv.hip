// k_mmv.hip -- GGML_OP_MUL_MAT on block-quantized weights for a few
// activation columns (decode, N <= 2 here; wider N goes to the MFMA path):
// a dequant-in-register GEMV with integer dot products (v_dot4_i32_i8).
// Call site: crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
//
// Mapping: a "row team" of LPR lanes (a power of two, <= 64) owns one weight
// row at a time; every lane streams CPL 16-byte chunks of the row with
// 128-bit loads, the team reduces its partial sums with cross-lane shuffles,
// and waves walk the rows grid-stride. Rows of one wave are adjacent, so a
// wave reads one contiguous run of weight memory per step.
//
// Block dots are exact integers; the scaled block terms are summed in f64 and
// rounded to f32 once, so the result does not depend on the lane / team
// split -- the CPU reference sums the same terms sequentially and gets the
// same f32 value.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

__device__ __forceinline__ int dot16(const int4 & w, const int4 & a) {
    int s = dot4_i8(w.x, a.x, 0);
    s = dot4_i8(w.y, a.y, s);
    s = dot4_i8(w.z, a.z, s);
    return dot4_i8(w.w, a.w, s);
}

// Q8_0 weights in the row-split layout: [K quants][K/32 f16 scales].
template <int NC>
__global__ __launch_bounds__(256) void k_mmv_q8_0(const char * __restrict__ W, int64_t row_bytes, int64_t M,
                                                  int64_t K, const int8_t * __restrict__ aq,
                                                  const float * __restrict__ ad, char * __restrict__ dst,
                                                  int64_t dst_nb1, int lpr_log2, int cpl) {
    const int lane = threadIdx.x & 63;
    const int LPR = 1 << lpr_log2;
    const int li = lane & (LPR - 1);
    const int teams_per_wave = 64 >> lpr_log2;
    const int64_t team = ((int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * teams_per_wave +
                         (lane >> lpr_log2);
    const int64_t team_stride = (int64_t) gridDim.x * (blockDim.x >> 6) * teams_per_wave;
    const int64_t nblk = K / 32;
    for (int64_t row = team; row < M; row += team_stride) {
        const char * wr = W + row * row_bytes;
        const uint16_t * ws = (const uint16_t *) (wr + K);
        double acc[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) acc[n] = 0.0;
        for (int c = 0; c < cpl; c++) {
            const int64_t e = (int64_t) (li + c * LPR) * 16;
            const int64_t b = e >> 5;
            const int4 w = *(const int4 *) (wr + e);
            const float dw = half_bits_to_float(ws[b]);
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const int4 a = *(const int4 *) (aq + n * K + e);
                const int s = dot16(w, a);
                // d_w * d_a of two halves is exact in f32, the term exact in f64
                acc[n] += (double) s * (double) (dw * ad[n * nblk + b]);
            }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            double v = acc[n];
            for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (li == 0) *(float *) (dst + n * dst_nb1 + row * 4) = (float) v;
        }
    }
}

// Q4_K weights (ggml layout, 144-byte super-blocks: f16 d, f16 dmin,
// 12 bytes of 6-bit scales/mins, 128 bytes of nibbles) against Q8_K
// activations. A chunk is 16 bytes of nibbles = 16 weights of sub-block 2g
// (low nibbles) and 16 of sub-block 2g+1 (high nibbles).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t * s, int & sc, int & m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Q4_K: a chunk is one sub-block pair c of a super-block (32 bytes of
// nibbles: low nibbles = sub-block 2c, high nibbles = sub-block 2c+1), so the
// min correction needs the activations' 32-element sums.
template <int NC>
__global__ __launch_bounds__(256) void k_mmv_q4_K(const char * __restrict__ W, int64_t row_bytes, int64_t M,
                                                  int64_t K, const int8_t * __restrict__ aq,
                                                  const float * __restrict__ ad, const int16_t * __restrict__ ass,
                                                  char * __restrict__ dst, int64_t dst_nb1, int lpr_log2, int cpl) {
    const int lane = threadIdx.x & 63;
    const int LPR = 1 << lpr_log2;
    const int li = lane & (LPR - 1);
    const int teams_per_wave = 64 >> lpr_log2;
    const int64_t team = ((int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * teams_per_wave +
                         (lane >> lpr_log2);
    const int64_t team_stride = (int64_t) gridDim.x * (blockDim.x >> 6) * teams_per_wave;
    const int64_t nsb = K / 256;
    for (int64_t row = team; row < M; row += team_stride) {
        const char * wr = W + row * row_bytes;
        double acc[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) acc[n] = 0.0;
        for (int c = 0; c < cpl; c++) {
            const int ci = li + c * LPR;
            const int sb = ci >> 2;
            const int g = ci & 3;
            const char * blk = wr + (int64_t) sb * 144;
            const uint4 hdr = *(const uint4 *) blk;
            const int4 q0 = *(const int4 *) (blk + 16 + 32 * g);
            const int4 q1 = *(const int4 *) (blk + 32 + 32 * g);
            const float dw = half_bits_to_float((uint16_t) (hdr.x & 0xFFFF));
            const float dmw = half_bits_to_float((uint16_t) (hdr.x >> 16));
            uint8_t sc8[12];
            *(uint32_t *) (sc8 + 0) = hdr.y;
            *(uint32_t *) (sc8 + 4) = hdr.z;
            *(uint32_t *) (sc8 + 8) = hdr.w;
            int sc_lo, m_lo, sc_hi, m_hi;
            scale_min_k4(2 * g, sc8, sc_lo, m_lo);
            scale_min_k4(2 * g + 1, sc8, sc_hi, m_hi);
            const int4 lo0 = make_int4(q0.x & 0x0F0F0F0F, q0.y & 0x0F0F0F0F, q0.z & 0x0F0F0F0F, q0.w & 0x0F0F0F0F);
            const int4 lo1 = make_int4(q1.x & 0x0F0F0F0F, q1.y & 0x0F0F0F0F, q1.z & 0x0F0F0F0F, q1.w & 0x0F0F0F0F);
            const int4 hi0 = make_int4((q0.x >> 4) & 0x0F0F0F0F, (q0.y >> 4) & 0x0F0F0F0F, (q0.z >> 4) & 0x0F0F0F0F,
                                       (q0.w >> 4) & 0x0F0F0F0F);
            const int4 hi1 = make_int4((q1.x >> 4) & 0x0F0F0F0F, (q1.y >> 4) & 0x0F0F0F0F, (q1.z >> 4) & 0x0F0F0F0F,
                                       (q1.w >> 4) & 0x0F0F0F0F);
            const int64_t e_lo = (int64_t) sb * 256 + 64 * g;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const int8_t * acol = aq + n * K + e_lo;
                const int isum = (dot16(lo0, *(const int4 *) acol) + dot16(lo1, *(const int4 *) (acol + 16))) * sc_lo +
                                 (dot16(hi0, *(const int4 *) (acol + 32)) + dot16(hi1, *(const int4 *) (acol + 48))) * sc_hi;
                const int16_t * ss = ass + n * (K / 32) + sb * 8 + 2 * g;
                const int msum = (int) ss[0] * m_lo + (int) ss[1] * m_hi;
                const double da = (double) ad[n * nsb + sb];
                acc[n] += ((double) dw * da) * (double) isum - ((double) dmw * da) * (double) msum;
            }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            double v = acc[n];
            for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (li == 0) *(float *) (dst + n * dst_nb1 + row * 4) = (float) v;
        }
    }
}

// Q3_K weights (ggml layout, 110-byte super-blocks: hmask[32], qs[64],
// scales[12], f16 d; rows only 2-byte aligned). A chunk is one 32-weight
// group g = 4h + j of a super-block: weights 128h + 32j + l (l < 32) with
// quants ((qs[32h + l] >> 2j) & 3) - 4, the 4 dropped where bit 4h + j of
// hmask[l] is set, scaled by 6-bit scales 8h + 2j (l < 16) and 8h + 2j + 1,
// each stored plus 32. Used by ggml-cpu's MUL_MAT for the host's q3_k pack
// policy (models/pack_quant.rs:205-207).
__device__ __forceinline__ uint32_t ld32_a2(const char * p) {
    const uint16_t * h = (const uint16_t *) p;
    return (uint32_t) h[0] | ((uint32_t) h[1] << 16);
}
__device__ __forceinline__ int q3_K_scale(const uint8_t * sc, int i) {
    const int lo = (sc[i % 8] >> (4 * (i / 8))) & 0xF;
    const int hi = (sc[8 + i % 4] >> (2 * (i / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}

template <int NC>
__global__ __launch_bounds__(256) void k_mmv_q3_K(const char * __restrict__ W, int64_t row_bytes, int64_t M,
                                                  int64_t K, const int8_t * __restrict__ aq,
                                                  const float * __restrict__ ad, char * __restrict__ dst,
                                                  int64_t dst_nb1, int lpr_log2, int cpl) {
    const int lane = threadIdx.x & 63;
    const int LPR = 1 << lpr_log2;
    const int li = lane & (LPR - 1);
    const int teams_per_wave = 64 >> lpr_log2;
    const int64_t team = ((int64_t) blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * teams_per_wave +
                         (lane >> lpr_log2);
    const int64_t team_stride = (int64_t) gridDim.x * (blockDim.x >> 6) * teams_per_wave;
    const int64_t nsb = K / 256;
    for (int64_t row = team; row < M; row += team_stride) {
        const char * wr = W + row * row_bytes;
        double acc[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) acc[n] = 0.0;
        for (int c = 0; c < cpl; c++) {
            const int ci = li + c * LPR;
            const int sb = ci >> 3, g = ci & 7, h = g >> 2, j = g & 3;
            const char * blk = wr + (int64_t) sb * 110;
            // the 32 signed quants as eight words of four int8: two low bits
            // plus 0xFC (-4) in bytes whose hmask bit is clear (at most
            // 3 + 0xFC, no carry between bytes)
            int q[8];
#pragma unroll
            for (int w = 0; w < 8; w++) {
                const uint32_t lo = (ld32_a2(blk + 32 + 32 * h + 4 * w) >> (2 * j)) & 0x03030303u;
                const uint32_t hb = (ld32_a2(blk + 4 * w) >> (4 * h + j)) & 0x01010101u;
                q[w] = (int) (lo + (hb ^ 0x01010101u) * 0xFCu);
            }
            const int s0 = q3_K_scale((const uint8_t *) (blk + 96), 8 * h + 2 * j);
            const int s1 = q3_K_scale((const uint8_t *) (blk + 96), 8 * h + 2 * j + 1);
            const float dw = half_bits_to_float(*(const uint16_t *) (blk + 108));
            const int64_t e0 = (int64_t) sb * 256 + 128 * h + 32 * j;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const int8_t * acol = aq + n * K + e0;
                const int isum = dot16(make_int4(q[0], q[1], q[2], q[3]), *(const int4 *) acol) * s0 +
                                 dot16(make_int4(q[4], q[5], q[6], q[7]), *(const int4 *) (acol + 16)) * s1;
                acc[n] += ((double) dw * (double) ad[n * nsb + sb]) * (double) isum;
            }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            double v = acc[n];
            for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (li == 0) *(float *) (dst + n * dst_nb1 + row * 4) = (float) v;
        }
    }
}

// Split the row's chunks over a power-of-two team so each lane owns a whole
// number of chunks: chunks = LPR * CPL with LPR = min(64, largest power of
// two dividing chunks).
static void pick_team(int64_t chunks, int & lpr_log2, int & cpl) {
    int l2 = 0;
    while (l2 < 6 && chunks % (2LL << l2) == 0) l2++;
    lpr_log2 = l2;
    cpl = (int) (chunks >> l2);
}

template <int NC>
static void mmv_dispatch(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K,
                         const act_buffers & act, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu) {
    const int64_t chunks = wtype == GGML_TYPE_Q8_0 ? K / 16 : wtype == GGML_TYPE_Q3_K ? K / 32 : K / 64;
    int lpr_log2, cpl;
    pick_team(chunks, lpr_log2, cpl);
    const int64_t teams = M;
    const int64_t teams_per_block = 4LL * (64 >> lpr_log2);
    int64_t blocks = (teams + teams_per_block - 1) / teams_per_block;
    const int64_t cap = (int64_t) n_cu * 8;
    if (blocks > cap) blocks = cap;
    if (wtype == GGML_TYPE_Q8_0) {
        hipLaunchKernelGGL(k_mmv_q8_0<NC>, dim3((unsigned) blocks), dim3(256), 0, stream, W, row_bytes, M, K, act.q,
                           act.d, dst, dst_nb1, lpr_log2, cpl);
    } else if (wtype == GGML_TYPE_Q3_K) {
        hipLaunchKernelGGL(k_mmv_q3_K<NC>, dim3((unsigned) blocks), dim3(256), 0, stream, W, row_bytes, M, K, act.q,
                           act.d, dst, dst_nb1, lpr_log2, cpl);
    } else {
        hipLaunchKernelGGL(k_mmv_q4_K<NC>, dim3((unsigned) blocks), dim3(256), 0, stream, W, row_bytes, M, K, act.q,
                           act.d, act.ssum, dst, dst_nb1, lpr_log2, cpl);
    }
}

void launch_mmv(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu) {
    int64_t done = 0;
    while (done < N) {
        const int64_t n = N - done > 8 ? 8 : N - done;
        act_buffers a = act;
        a.q += done * K;
        a.d += done * (wtype == GGML_TYPE_Q8_0 ? K / 32 : K / 256);
        if (a.ssum) a.ssum += done * (K / 32);
        char * d = dst + done * dst_nb1;
        switch (n) {
            case 1: mmv_dispatch<1>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            case 2: mmv_dispatch<2>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            case 3: mmv_dispatch<3>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            case 4: mmv_dispatch<4>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            case 5: mmv_dispatch<5>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            case 6: mmv_dispatch<6>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            case 7: mmv_dispatch<7>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
            default: mmv_dispatch<8>(wtype, W, row_bytes, M, K, a, d, dst_nb1, stream, n_cu); break;
        }
        done += n;
    }
}

}  // namespace mi355x

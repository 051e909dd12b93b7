// k_mmq.hip -- GGML_OP_MUL_MAT on Q4_K / Q8_0 weights for wide activation
// batches (prefill, the audio prefix, N > 16) on the int8 matrix cores.
// Call site: crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
//
// A workgroup computes a 64-row x 64-column output tile: each of its four
// waves owns 16 weight rows and all 64 columns (four 16-column MFMA groups),
// so every weight fragment a wave loads feeds four v_mfma_i32_16x16x32_i8.
// The activations of the current 256-element K slice (quants, scales and
// 32-element sums of 64 columns) are staged once per slice in LDS and shared
// by the four waves. The operand orientation is the GEMV's (activations A,
// weight tile B: one weight row and four columns per lane), and each lane
// walks K in order, so the f64 block sums are formed exactly as the CPU
// reference forms them.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8_mmq(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

constexpr int kMmqRows = 64;
constexpr int kMmqCols = 64;
constexpr int kMmqPad = 16;  // bytes of padding per staged column (LDS banks)

struct mmq_args {
    const char * W;
    int64_t row_bytes, M, K;
    const int8_t * aq;
    const float * ad;
    const int16_t * ass;
    int N;
    char * dst;
    int64_t dst_nb1;
};

// stage 256 quants of each of the tile's columns (K slice ks) into LDS
__device__ __forceinline__ void mmq_stage_q(const mmq_args & a, int n0, int ncol, int64_t ks,
                                            int8_t (*s_q)[256 + kMmqPad]) {
    for (int idx = (int) threadIdx.x; idx < kMmqCols * 16; idx += 256) {
        const int col = idx / 16, piece = idx % 16;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (col < ncol) {
            const int8_t * src = a.aq + (int64_t) (n0 + col) * a.K + ks * 256 + piece * 16;
            if (ks * 256 + piece * 16 < a.K) v = *(const uint4 *) src;
        }
        *(uint4 *) &s_q[col][piece * 16] = v;
    }
}

__device__ __forceinline__ void mmq_store(const mmq_args & a, double (&acc)[4][4], int64_t row, int n0) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int grp = 0; grp < 4; grp++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + grp * 16 + 4 * g + i;
            if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + row * 4) = (float) acc[grp][i];
        }
    }
}

__global__ __launch_bounds__(256) void k_mmq_q4_K(mmq_args a) {
    __shared__ __align__(16) int8_t s_q[kMmqCols][256 + kMmqPad];
    __shared__ float s_d[kMmqCols];
    __shared__ __align__(16) int16_t s_ss[kMmqCols][8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t row = (int64_t) blockIdx.x * kMmqRows + wave * 16 + r;
    const bool row_ok = (int64_t) blockIdx.x * kMmqRows + wave * 16 < a.M;  // uniform per wave
    const int n0 = (int) blockIdx.y * kMmqCols;
    const int ncol = min(kMmqCols, a.N - n0);
    const int64_t nsb = a.K / 256;
    const char * wrow = a.W + (row_ok ? row : 0) * a.row_bytes;
    double acc[4][4];
#pragma unroll
    for (int grp = 0; grp < 4; grp++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[grp][i] = 0.0;
    for (int64_t sb = 0; sb < nsb; sb++) {
        __syncthreads();  // the previous slice's LDS reads are done
        mmq_stage_q(a, n0, ncol, sb, s_q);
        if (threadIdx.x < kMmqCols) {
            const int col = threadIdx.x;
            s_d[col] = col < ncol ? a.ad[(int64_t) (n0 + col) * nsb + sb] : 0.0f;
            *(uint4 *) s_ss[col] =
                col < ncol ? *(const uint4 *) (a.ass + ((int64_t) (n0 + col) * nsb + sb) * 8) : make_uint4(0, 0, 0, 0);
        }
        const char * blk = wrow + sb * 144;
        const uint4 hdr = *(const uint4 *) blk;
        long q[4];
#pragma unroll
        for (int c = 0; c < 4; c++) q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
        __syncthreads();
        if (!row_ok) continue;
        int sc[8], mn[8];
        {
            const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sc[j] = (s0 >> (8 * j)) & 63;
                mn[j] = (s1 >> (8 * j)) & 63;
                sc[j + 4] = ((s2 >> (8 * j)) & 0xF) | (((s0 >> (8 * j + 6)) & 3) << 4);
                mn[j + 4] = ((s2 >> (8 * j + 4)) & 0xF) | (((s1 >> (8 * j + 6)) & 3) << 4);
            }
        }
        const float dw = half_bits_to_float((uint16_t) (hdr.x & 0xFFFF));
        const float dmw = half_bits_to_float((uint16_t) (hdr.x >> 16));
#pragma unroll
        for (int grp = 0; grp < 4; grp++) {
            const int8_t * acol = &s_q[grp * 16 + r][0];
            int isum[4] = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const long lo = q[c] & 0x0F0F0F0F0F0F0F0FL;
                const long hi = (q[c] >> 4) & 0x0F0F0F0F0F0F0F0FL;
                const long a0 = *(const long *) (acol + 64 * c + 8 * g);
                const long a1 = *(const long *) (acol + 64 * c + 32 + 8 * g);
                const v4i z = {0, 0, 0, 0};
                const v4i c0 = mfma_i8_mmq(a0, lo, z);
                const v4i c1 = mfma_i8_mmq(a1, hi, z);
#pragma unroll
                for (int i = 0; i < 4; i++) isum[i] += __mul24(sc[2 * c], c0[i]) + __mul24(sc[2 * c + 1], c1[i]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = grp * 16 + 4 * g + i;
                int msum = 0;
#pragma unroll
                for (int j = 0; j < 8; j++) msum += __mul24(mn[j], (int) s_ss[n][j]);  // 6 x 13 bits
                const double da = (double) s_d[n];
                const double d = (double) dw * da;
                const double dmin = (double) dmw * da;
                acc[grp][i] += d * (double) isum[i] - dmin * (double) msum;
            }
        }
    }
    if (row_ok) mmq_store(a, acc, row, n0);
}

// Q8_0 weights in the row-split layout [K quants][K/32 f16 scales]; K is
// walked in 256-element slices of eight blocks (the last may be partial)
__global__ __launch_bounds__(256) void k_mmq_q8_0(mmq_args a) {
    __shared__ __align__(16) int8_t s_q[kMmqCols][256 + kMmqPad];
    __shared__ float s_d[kMmqCols][8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t row = (int64_t) blockIdx.x * kMmqRows + wave * 16 + r;
    const bool row_ok = (int64_t) blockIdx.x * kMmqRows + wave * 16 < a.M;
    const int n0 = (int) blockIdx.y * kMmqCols;
    const int ncol = min(kMmqCols, a.N - n0);
    const int64_t nblk = a.K / 32;
    const int64_t nks = (a.K + 255) / 256;
    const char * wrow = a.W + (row_ok ? row : 0) * a.row_bytes;
    const uint16_t * wsc = (const uint16_t *) (wrow + a.K);
    double acc[4][4];
#pragma unroll
    for (int grp = 0; grp < 4; grp++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[grp][i] = 0.0;
    for (int64_t ks = 0; ks < nks; ks++) {
        const int nb = (int) min((int64_t) 8, nblk - ks * 8);
        __syncthreads();
        mmq_stage_q(a, n0, ncol, ks, s_q);
        for (int idx = (int) threadIdx.x; idx < kMmqCols * 8; idx += 256) {
            const int col = idx / 8, bb = idx % 8;
            s_d[col][bb] = col < ncol && bb < nb ? a.ad[(int64_t) (n0 + col) * nblk + ks * 8 + bb] : 0.0f;
        }
        long q[8];
        uint16_t ds[8];
#pragma unroll
        for (int bb = 0; bb < 8; bb++) {
            q[bb] = bb < nb ? *(const long *) (wrow + (ks * 8 + bb) * 32 + 8 * g) : 0;
            ds[bb] = bb < nb ? wsc[ks * 8 + bb] : 0;
        }
        __syncthreads();
        if (!row_ok) continue;
#pragma unroll
        for (int bb = 0; bb < 8; bb++) {
            if (bb >= nb) break;
            const float dw = half_bits_to_float(ds[bb]);
#pragma unroll
            for (int grp = 0; grp < 4; grp++) {
                const long av = *(const long *) (&s_q[grp * 16 + r][32 * bb + 8 * g]);
                const v4i z = {0, 0, 0, 0};
                const v4i cc = mfma_i8_mmq(av, q[bb], z);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = grp * 16 + 4 * g + i;
                    // d_w * d_a of two halves is exact in f32, the term exact in f64
                    acc[grp][i] += (double) cc[i] * (double) (dw * s_d[n][bb]);
                }
            }
        }
    }
    if (row_ok) mmq_store(a, acc, row, n0);
}

bool mmq_supported(int wtype, int64_t M, int64_t K) {
    if (M % 16 != 0) return false;
    if (wtype == GGML_TYPE_Q4_K) return K % 256 == 0;
    if (wtype == GGML_TYPE_Q8_0) return K % 32 == 0;
    return false;
}

void launch_mmq(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu) {
    (void) n_cu;
    mmq_args a;
    a.W = W;
    a.row_bytes = row_bytes;
    a.M = M;
    a.K = K;
    a.aq = act.q;
    a.ad = act.d;
    a.ass = act.ssum;
    a.N = (int) N;
    a.dst = dst;
    a.dst_nb1 = dst_nb1;
    const dim3 grid((unsigned) ((M + kMmqRows - 1) / kMmqRows), (unsigned) ((N + kMmqCols - 1) / kMmqCols));
    if (wtype == GGML_TYPE_Q4_K) hipLaunchKernelGGL(k_mmq_q4_K, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(k_mmq_q8_0, grid, dim3(256), 0, stream, a);
}

}  // namespace mi355x

// k_gemv_mfma.hip -- GGML_OP_MUL_MAT on Q4_K / Q8_0 weights for up to 16
// activation columns per launch (the decode step: batch 1..8 tokens) on the
// int8 matrix cores (v_mfma_i32_16x16x32_i8).
// Call site: crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
//
// Orientation: activations are the MFMA A operand (16 columns x 32 k) and a
// 16-row weight tile is the B operand (32 k x 16 rows), so the 16x16 int32
// result lands with one weight row per lane (row = lane % 16) and four
// activation columns per lane (n = 4 * (lane / 16) + i). Each lane therefore
// needs the 6-bit scales / f16 super-block scales of exactly one row, and
// holds the complete integer sum of every (row, column, sub-block) -- the
// scale products are applied per super-block to exact integers and summed in
// f64, the same terms the CPU reference sums.
//
// B-operand loads: lane (row r, group g) reads 8 bytes of nibbles at
// qs + 32c + 8g for c = 0..3, which hold elements 8g..8g+7 of sub-block 2c
// (low nibbles) and of sub-block 2c+1 (high nibbles); the A operand takes
// the matching 8 activation bytes, so the k order inside a sub-block is the
// same on both sides. A workgroup's four waves either cover four row tiles
// or split one tile's K range (reduced through LDS in f64) when the matrix
// has too few tiles to occupy the chip.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

struct gemv_args {
    const char * W;
    int64_t row_bytes, M, K;
    const int8_t * aq;
    const float * ad;
    const int16_t * abs_;
    int N;  // columns in this launch (<= 16)
    char * dst;
    int64_t dst_nb1;
    int ksplit;  // waves sharing one row tile (1, 2 or 4)
};

// per-lane scale / min of sub-blocks 0..7 of one Q4_K super-block header
__device__ __forceinline__ void q4k_scales(const uint4 & hdr, int * sc, int * mn) {
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;  // bytes 0-3, 4-7, 8-11 of scales[12]
#pragma unroll
    for (int j = 0; j < 4; j++) {
        sc[j] = (s0 >> (8 * j)) & 63;
        mn[j] = (s1 >> (8 * j)) & 63;
        sc[j + 4] = ((s2 >> (8 * j)) & 0xF) | (((s0 >> (8 * j + 6)) & 3) << 4);
        mn[j + 4] = ((s2 >> (8 * j + 4)) & 0xF) | (((s1 >> (8 * j + 6)) & 3) << 4);
    }
}

__global__ __launch_bounds__(256) void k_gemv_q4_K(gemv_args a) {
    __shared__ double s_red[4][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ks = a.ksplit, tiles_per_block = 4 / ks;
    const int slot = wave / ks, kslice = wave % ks;
    const int r = lane & 15, g = lane >> 4;
    const int64_t nsb = a.K / 256;
    const int64_t sb0 = nsb * kslice / ks, sb1 = nsb * (kslice + 1) / ks;
    const int64_t tiles = a.M / 16;
    const int na = lane & 15;  // A-operand column of this lane
    const bool a_ok = na < a.N;
    const int8_t * acol = a.aq + (int64_t) na * a.K;
    for (int64_t base = (int64_t) blockIdx.x * tiles_per_block; base < tiles; base += (int64_t) gridDim.x * tiles_per_block) {
        const int64_t tile = base + slot;
        const bool tile_ok = tile < tiles;  // uniform per wave
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
        if (tile_ok) {
            const char * wrow = a.W + (tile * 16 + r) * a.row_bytes;
            for (int64_t sb = sb0; sb < sb1; sb++) {
                const char * blk = wrow + sb * 144;
                const uint4 hdr = *(const uint4 *) blk;
                long q[4];
#pragma unroll
                for (int c = 0; c < 4; c++) q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
                long af[8];
#pragma unroll
                for (int j = 0; j < 8; j++) af[j] = a_ok ? *(const long *) (acol + sb * 256 + 32 * j + 8 * g) : 0;
                int sc[8], mn[8];
                q4k_scales(hdr, sc, mn);
                int isum[4] = {0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const long lo = q[c] & 0x0F0F0F0F0F0F0F0FL;
                    const long hi = (q[c] >> 4) & 0x0F0F0F0F0F0F0F0FL;
                    const v4i z = {0, 0, 0, 0};
                    const v4i c0 = mfma_i8(af[2 * c], lo, z);
                    const v4i c1 = mfma_i8(af[2 * c + 1], hi, z);
#pragma unroll
                    for (int i = 0; i < 4; i++) isum[i] += sc[2 * c] * c0[i] + sc[2 * c + 1] * c1[i];
                }
                const float dw = half_bits_to_float((uint16_t) (hdr.x & 0xFFFF));
                const float dmw = half_bits_to_float((uint16_t) (hdr.x >> 16));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = 4 * g + i;
                    if (n < a.N) {
                        const int16_t * bs = a.abs_ + (int64_t) n * (a.K / 16) + sb * 16;
                        int msum = 0;
#pragma unroll
                        for (int j = 0; j < 8; j++) msum += mn[j] * ((int) bs[2 * j] + (int) bs[2 * j + 1]);
                        const double da = (double) a.ad[(int64_t) n * nsb + sb];
                        const double d = (double) dw * da;
                        const double dmin = (double) dmw * da;
                        acc[i] += d * (double) isum[i] - dmin * (double) msum;
                    }
                }
            }
        }
        if (ks > 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) s_red[wave][lane][i] = acc[i];
            __syncthreads();
            if (kslice == 0 && tile_ok) {
                for (int w = 1; w < ks; w++) {
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i] += s_red[wave + w][lane][i];
                }
            }
            __syncthreads();
        }
        if (kslice == 0 && tile_ok) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = 4 * g + i;
                if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + (tile * 16 + r) * 4) = (float) acc[i];
            }
        }
    }
}

// Q8_0 weights in the row-split layout: [K quants][K/32 f16 scales] per row
__global__ __launch_bounds__(256) void k_gemv_q8_0(gemv_args a) {
    __shared__ double s_red[4][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ks = a.ksplit, tiles_per_block = 4 / ks;
    const int slot = wave / ks, kslice = wave % ks;
    const int r = lane & 15, g = lane >> 4;
    const int64_t nblk = a.K / 32;
    const int64_t b0 = nblk * kslice / ks, b1 = nblk * (kslice + 1) / ks;
    const int64_t tiles = a.M / 16;
    const int na = lane & 15;
    const bool a_ok = na < a.N;
    const int8_t * acol = a.aq + (int64_t) na * a.K;
    for (int64_t base = (int64_t) blockIdx.x * tiles_per_block; base < tiles; base += (int64_t) gridDim.x * tiles_per_block) {
        const int64_t tile = base + slot;
        const bool tile_ok = tile < tiles;
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
        if (tile_ok) {
            const char * wrow = a.W + (tile * 16 + r) * a.row_bytes;
            const uint16_t * wsc = (const uint16_t *) (wrow + a.K);
            int64_t b = b0;
            for (; b + 4 <= b1; b += 4) {
                long q[4], af[4];
                uint16_t ds[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    q[u] = *(const long *) (wrow + (b + u) * 32 + 8 * g);
                    af[u] = a_ok ? *(const long *) (acol + (b + u) * 32 + 8 * g) : 0;
                    ds[u] = wsc[b + u];
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const v4i z = {0, 0, 0, 0};
                    const v4i cc = mfma_i8(af[u], q[u], z);
                    const float dw = half_bits_to_float(ds[u]);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int n = 4 * g + i;
                        if (n < a.N) acc[i] += (double) cc[i] * (double) (dw * a.ad[(int64_t) n * nblk + b + u]);
                    }
                }
            }
            for (; b < b1; b++) {
                const long q = *(const long *) (wrow + b * 32 + 8 * g);
                const long af = a_ok ? *(const long *) (acol + b * 32 + 8 * g) : 0;
                const v4i z = {0, 0, 0, 0};
                const v4i cc = mfma_i8(af, q, z);
                const float dw = half_bits_to_float(wsc[b]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = 4 * g + i;
                    if (n < a.N) acc[i] += (double) cc[i] * (double) (dw * a.ad[(int64_t) n * nblk + b]);
                }
            }
        }
        if (ks > 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) s_red[wave][lane][i] = acc[i];
            __syncthreads();
            if (kslice == 0 && tile_ok) {
                for (int w = 1; w < ks; w++) {
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i] += s_red[wave + w][lane][i];
                }
            }
            __syncthreads();
        }
        if (kslice == 0 && tile_ok) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = 4 * g + i;
                if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + (tile * 16 + r) * 4) = (float) acc[i];
            }
        }
    }
}

bool gemv_mfma_supported(int wtype, int64_t M, int64_t K) {
    (void) K;
    return (wtype == GGML_TYPE_Q4_K || wtype == GGML_TYPE_Q8_0) && M % 16 == 0;
}

void launch_gemv_mfma(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                      int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu) {
    const int64_t units = wtype == GGML_TYPE_Q4_K ? K / 256 : K / 32;
    const int64_t tiles = M / 16;
    int ks = 1;
    if (tiles < (int64_t) n_cu * 16) ks = units >= 4 ? 4 : (units >= 2 ? 2 : 1);
    const int64_t tiles_per_block = 4 / ks;
    int64_t blocks = (tiles + tiles_per_block - 1) / tiles_per_block;
    const int64_t cap = (int64_t) n_cu * 8;
    if (blocks > cap) blocks = cap;
    for (int64_t n0 = 0; n0 < N; n0 += 16) {
        gemv_args a;
        a.W = W;
        a.row_bytes = row_bytes;
        a.M = M;
        a.K = K;
        a.aq = act.q + n0 * K;
        a.ad = act.d + n0 * (wtype == GGML_TYPE_Q4_K ? K / 256 : K / 32);
        a.abs_ = act.bsums ? act.bsums + n0 * (K / 16) : nullptr;
        a.N = (int) (N - n0 < 16 ? N - n0 : 16);
        a.dst = dst + n0 * dst_nb1;
        a.dst_nb1 = dst_nb1;
        a.ksplit = ks;
        if (wtype == GGML_TYPE_Q4_K) hipLaunchKernelGGL(k_gemv_q4_K, dim3((unsigned) blocks), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(k_gemv_q8_0, dim3((unsigned) blocks), dim3(256), 0, stream, a);
    }
}

}  // namespace mi355x

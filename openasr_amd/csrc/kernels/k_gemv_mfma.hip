// k_gemv_mfma.hip -- GGML_OP_MUL_MAT on Q4_K / Q8_0 weights for the decode
// step (a few activation columns) on the int8 matrix cores
// (v_mfma_i32_16x16x32_i8). Call site:
// crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
//
// Orientation: activations are the MFMA A operand (16 columns x 32 k) and a
// 16-row weight tile is the B operand (32 k x 16 rows), so the 16x16 int32
// result lands with one weight row per lane (row = lane % 16) and four
// activation columns per lane (n = 4 * (lane / 16) + i). Each lane therefore
// needs the scales of exactly one row and holds the complete integer sum of
// every (row, column, sub-block); the scale products are applied to exact
// integers and summed in f64 -- the terms the CPU reference sums.
//
// Launch shape: one workgroup per 16-row tile (and per 16-column chunk of the
// activations); its up to 16 waves split the K range, every wave issues all
// loads of a unit (a Q4_K super-block, eight Q8_0 blocks) before its first
// MFMA -- one memory round trip per unit, one unit per wave at decode sizes --
// and the waves' f64 partials are added in wave order through LDS. Decode
// matrices are a few MB, so the whole matrix is in flight at once; the kernel
// is latency-bound by construction, not issue-bound.
//
// Q4_K B-operand loads: lane (row r, group g) reads 8 bytes of nibbles at
// qs + 32c + 8g for c = 0..3, which hold elements 8g..8g+7 of sub-block 2c
// (low nibbles) and of sub-block 2c+1 (high nibbles); the A operand takes the
// matching 8 activation bytes, so the k order inside a sub-block is the same
// on both sides. The min correction uses the activations' 32-element sums.
//
// Optional epilogue: a residual of the output's shape is added to the
// rounded product (the ADD that follows the output projections,
// nn/decoder.rs:2107-2145) -- the same two f32 roundings as the unfused ops.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

struct gemv_args {
    const char * W;
    const char * W2;  // optional second matrix of the same shape (gate + up)
    int64_t row_bytes, M, K;
    const int8_t * aq;
    const float * ad;
    const int16_t * ass;  // Q8_K 32-element sums
    int N;                // activation columns
    char * dst;
    int64_t dst_nb1;
    const char * res;  // optional residual, same layout as dst
    int64_t res_nb1;
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

// wave partials summed in wave order by wave 0, then stored. Waves
// [0, half) hold W's partials, waves [half, nw) W2's when there is a second
// matrix; the epilogue then writes silu(W x) * (W2 x) -- the SwiGLU gate of
// nn/ffn.rs:64-91 with the same roundings as MUL_MAT, SILU and MUL apart.
// A residual, when given, is added to the rounded product.
__device__ __forceinline__ void gemv_finish(const gemv_args & a, double (&acc)[4], double (*s_red)[64][4], int64_t row,
                                            int n0, int half) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int g = lane >> 4;
    double acc2[4] = {0.0, 0.0, 0.0, 0.0};
    if (nw > 1) {
        if (wave > 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) s_red[wave][lane][i] = acc[i];
        }
        __syncthreads();
        if (wave != 0) return;
        for (int w = 1; w < half; w++) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] += s_red[w][lane][i];
        }
        for (int w = half; w < nw; w++) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc2[i] += s_red[w][lane][i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int n = n0 + 4 * g + i;
        if (n < a.N) {
            float v = (float) acc[i];
            if (a.W2) {
                const float u = (float) acc2[i];
                v = (v / (1.0f + expf_det(-v))) * u;
            }
            if (a.res) v = *(const float *) (a.res + (int64_t) n * a.res_nb1 + row * 4) + v;
            *(float *) (a.dst + (int64_t) n * a.dst_nb1 + row * 4) = v;
        }
    }
}

// waves of the workgroup take super-blocks round-robin (wave w: sb = w,
// w + nw, ...); each super-block's loads are issued together
__global__ __launch_bounds__(1024) void k_gemv_q4_K(gemv_args a) {
    __shared__ double s_red[16][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int half = a.W2 ? nw / 2 : nw;
    const int second = wave >= half;
    const int wv = wave - (second ? half : 0);
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile = blockIdx.x;
    const int n0 = (int) blockIdx.y * 16;
    const int64_t nsb = a.K / 256;
    const int64_t row = tile * 16 + r;
    const char * wrow = (second ? a.W2 : a.W) + row * a.row_bytes;
    const bool a_ok = n0 + r < a.N;  // this lane's A-operand column
    const int8_t * acol = a.aq + (int64_t) (n0 + r) * a.K;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t sb = wv; sb < nsb; sb += half) {
        const char * blk = wrow + sb * 144;
        const uint4 hdr = *(const uint4 *) blk;
        long q[4], af[8];
        float ad[4];
        uint4 ss[4];
#pragma unroll
        for (int c = 0; c < 4; c++) q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
#pragma unroll
        for (int j = 0; j < 8; j++) af[j] = a_ok ? *(const long *) (acol + sb * 256 + 32 * j + 8 * g) : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + 4 * g + i;
            const bool ok = n < a.N;
            ad[i] = ok ? a.ad[(int64_t) n * nsb + sb] : 0.0f;
            ss[i] = ok ? *(const uint4 *) (a.ass + ((int64_t) n * nsb + sb) * 8) : make_uint4(0, 0, 0, 0);
        }
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
            const uint32_t w4[4] = {ss[i].x, ss[i].y, ss[i].z, ss[i].w};
            int msum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                msum += mn[2 * j] * (int) (int16_t) (w4[j] & 0xFFFF);
                msum += mn[2 * j + 1] * (int) (int16_t) (w4[j] >> 16);
            }
            const double da = (double) ad[i];
            const double d = (double) dw * da;
            const double dmin = (double) dmw * da;
            acc[i] += d * (double) isum[i] - dmin * (double) msum;
        }
    }
    gemv_finish(a, acc, s_red, row, n0, half);
}

// Q8_0 weights in the row-split layout [K quants][K/32 f16 scales]; the waves
// take groups of 8 blocks round-robin, each group's loads issued together
constexpr int kQ8Group = 8;

__global__ __launch_bounds__(1024) void k_gemv_q8_0(gemv_args a) {
    __shared__ double s_red[16][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int half = a.W2 ? nw / 2 : nw;
    const int second = wave >= half;
    const int wv = wave - (second ? half : 0);
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile = blockIdx.x;
    const int n0 = (int) blockIdx.y * 16;
    const int64_t nblk = a.K / 32;
    const int64_t row = tile * 16 + r;
    const char * wrow = (second ? a.W2 : a.W) + row * a.row_bytes;
    const uint16_t * wsc = (const uint16_t *) (wrow + a.K);
    const bool a_ok = n0 + r < a.N;
    const int8_t * acol = a.aq + (int64_t) (n0 + r) * a.K;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int64_t b0 = (int64_t) wv * kQ8Group; b0 < nblk; b0 += (int64_t) half * kQ8Group) {
        long q[kQ8Group], af[kQ8Group];
        uint16_t ds[kQ8Group];
        float4 ad[4][kQ8Group / 4];
#pragma unroll
        for (int u = 0; u < kQ8Group; u++) {
            const int64_t b = b0 + u;
            const bool ok = b < nblk;
            q[u] = ok ? *(const long *) (wrow + b * 32 + 8 * g) : 0;
            af[u] = ok && a_ok ? *(const long *) (acol + b * 32 + 8 * g) : 0;
            ds[u] = ok ? wsc[b] : 0;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + 4 * g + i;
#pragma unroll
            for (int v = 0; v < kQ8Group / 4; v++) {
                const int64_t b = b0 + 4 * v;
                ad[i][v] = n < a.N && b < nblk ? *(const float4 *) (a.ad + (int64_t) n * nblk + b)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int u = 0; u < kQ8Group; u++) {
            if (b0 + u < nblk) {
                const v4i z = {0, 0, 0, 0};
                const v4i cc = mfma_i8(af[u], q[u], z);
                const float dw = half_bits_to_float(ds[u]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 d4 = ad[i][u / 4];
                    const float da = (u & 3) == 0 ? d4.x : (u & 3) == 1 ? d4.y : (u & 3) == 2 ? d4.z : d4.w;
                    // d_w * d_a of two halves is exact in f32, the term exact in f64
                    acc[i] += (double) cc[i] * (double) (dw * da);
                }
            }
        }
    }
    gemv_finish(a, acc, s_red, row, n0, half);
}

bool gemv_mfma_supported(int wtype, int64_t M, int64_t K) {
    if (M % 16 != 0) return false;
    if (wtype == GGML_TYPE_Q4_K) return K % 256 == 0;
    if (wtype == GGML_TYPE_Q8_0) return K % 128 == 0;
    return false;
}

void launch_gemv_mfma(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                      int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu, const char * res,
                      int64_t res_nb1, const char * W2) {
    (void) n_cu;
    gemv_args a;
    a.W = W;
    a.W2 = W2;
    a.row_bytes = row_bytes;
    a.M = M;
    a.K = K;
    a.aq = act.q;
    a.ad = act.d;
    a.ass = act.ssum;
    a.N = (int) N;
    a.dst = dst;
    a.dst_nb1 = dst_nb1;
    a.res = res;
    a.res_nb1 = res_nb1;
    const dim3 grid((unsigned) (M / 16), (unsigned) ((N + 15) / 16));
    const int64_t units = wtype == GGML_TYPE_Q4_K ? K / 256 : (K / 32 + kQ8Group - 1) / kQ8Group;
    const int64_t per = W2 ? 8 : 16;  // waves per matrix
    const unsigned waves = (unsigned) ((units < per ? units : per) * (W2 ? 2 : 1));
    if (wtype == GGML_TYPE_Q4_K) hipLaunchKernelGGL(k_gemv_q4_K, grid, dim3(64 * waves), 0, stream, a);
    else hipLaunchKernelGGL(k_gemv_q8_0, grid, dim3(64 * waves), 0, stream, a);
}

}  // namespace mi355x

// k_mmq.hip -- GGML_OP_MUL_MAT on Q4_K / Q8_0 weights for wide activation
// batches (prefill, the audio prefix, N > 16) on the int8 matrix cores.
// Call site: crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
//
// A workgroup computes a 64-row x 64-column output tile: each of its four
// waves owns 16 weight rows and all 64 columns (four 16-column MFMA groups),
// so every weight fragment a wave loads feeds four column groups; where the
// 64-column tiles would leave CUs idle, 32-column tiles (two groups). K is walked
// in 256-element slices. A slice's activations (quants, scales and, for Q4_K,
// the 32-element sums of the 64 columns) are staged in LDS, double-buffered:
// right after a slice's barrier the workgroup requests the next slice's
// activations and weights into registers, computes the current slice from
// LDS, and stores the next slice into the other buffer at the top of the
// next iteration -- one barrier a slice, the next slice's loads in flight
// under this slice's arithmetic. A buffer is written again only after the
// following barrier, which every wave reaches after its reads of it.
//
// The arithmetic of a block unit is the GEMV's (mfma_units.h) and each lane
// walks K in order, so the f64 block sums are the ones the CPU reference
// forms and the bits equal the GEMV's.
//
// Tiles are dealt to the XCDs in contiguous runs (workgroup i runs on XCD
// i % 8): XCD x takes tiles [x P, (x + 1) P), the column blocks of a row tile
// adjacent, so a weight tile is fetched into one XCD's L2 and read there by
// all of its column blocks.
#include "../mi355x_common.h"
#include "../ops.h"
#include "../mfma_units.h"

namespace mi355x {

constexpr int kMmqRows = 64;
constexpr int kMmqCols = 64;
constexpr int kMmqPad = 16;  // bytes of padding per staged column (LDS banks)
constexpr int kMmqXcds = 8;

struct mmq_args {
    const char * W;
    int64_t row_bytes, M, K;
    const int8_t * aq;
    const float * ad;
    const int16_t * ass;
    int N;
    char * dst;
    int64_t dst_nb1;
    int64_t col_blocks, tiles, per_xcd;
    gemm_float_epi epi;  // bias, residual (laid out as dst), GELU_ERF
    // sibling products of the same activations (rows [sub_m0[i],
    // sub_m0[i + 1]) are product i: weights, contiguous output, bias)
    int nsub;
    int64_t sub_m0[kGemmFloatMaxSubs + 2];
    const char * sub_W[kGemmFloatMaxSubs + 1];
    char * sub_dst[kGemmFloatMaxSubs + 1];
    const float * sub_bias[kGemmFloatMaxSubs + 1];
};

// the activations of one K slice of the tile's 64 columns
struct mmq_slice {
    int8_t q[kMmqCols][256 + kMmqPad];
    float d[8][kMmqCols];     // Q4_K: [0][col] the super-block scale; Q8_0: [block][col]
    int16_t ss[kMmqCols][8];  // Q4_K: the 32-element sums
};

// this thread's share of a slice, held in registers between its request and
// its store into LDS
struct mmq_act {
    uint4 q[4];
    float d[4];
    uint4 ss;
};

template <int WT, int GRPS>
__device__ __forceinline__ void mmq_act_load(const mmq_args & a, int n0, int ncol, int64_t ks, mmq_act & r) {
    const int t = (int) threadIdx.x;
#pragma unroll
    for (int u = 0; u < GRPS; u++) {
        const int idx = t + 256 * u, col = idx >> 4, piece = idx & 15;
        const int64_t kk = ks * 256 + piece * 16;
        const bool ok = col < ncol && kk < a.K;
        // clamped address, unconditional load: masked when stored
        r.q[u] = *(const uint4 *) (a.aq + (int64_t) (n0 + (ok ? col : 0)) * a.K + (ok ? kk : 0));
    }
    if constexpr (WT == GGML_TYPE_Q4_K) {
        const int64_t nsb = a.K / 256;
        const int col = t < ncol ? t : 0;
        if (t < 16 * GRPS) {
            r.d[0] = a.ad[(int64_t) (n0 + col) * nsb + ks];
            r.ss = *(const uint4 *) (a.ass + ((int64_t) (n0 + col) * nsb + ks) * 8);
        }
    } else {
        const int64_t nblk = a.K / 32;
        const int col = (t >> 1) < ncol ? (t >> 1) : 0, h = t & 1;
        if (t < 32 * GRPS) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t b = ks * 8 + 4 * h + j;
                r.d[j] = a.ad[(int64_t) (n0 + col) * nblk + (b < nblk ? b : nblk - 1)];
            }
        }
    }
}

template <int WT, int GRPS>
__device__ __forceinline__ void mmq_act_store(const mmq_args & a, int ncol, int64_t ks, const mmq_act & r,
                                              mmq_slice & S) {
    const int t = (int) threadIdx.x;
#pragma unroll
    for (int u = 0; u < GRPS; u++) {
        const int idx = t + 256 * u, col = idx >> 4, piece = idx & 15;
        const bool ok = col < ncol && ks * 256 + piece * 16 < a.K;
        *(uint4 *) &S.q[col][piece * 16] = ok ? r.q[u] : make_uint4(0, 0, 0, 0);
    }
    if constexpr (WT == GGML_TYPE_Q4_K) {
        if (t < 16 * GRPS) {
            const bool ok = t < ncol;
            S.d[0][t] = ok ? r.d[0] : 0.0f;
            *(uint4 *) &S.ss[t][0] = ok ? r.ss : make_uint4(0, 0, 0, 0);
        }
    } else {
        const int64_t nblk = a.K / 32;
        if (t < 32 * GRPS) {
            const int col = t >> 1, h = t & 1;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool ok = col < ncol && ks * 8 + 4 * h + j < nblk;
                S.d[4 * h + j][col] = ok ? r.d[j] : 0.0f;
            }
        }
    }
}

// this lane's weights of one slice: Q4_K one super-block of its row, Q8_0
// eight blocks (past the end of K: the row's last block, never used)
struct mmq_w4 {
    uint4 hdr;
    long q[4];
};
struct mmq_w8 {
    long q[kQ8Group];
    uint16_t ds[kQ8Group];
};

__device__ __forceinline__ void mmq_w_load(const mmq_args & a, const char * wrow, int64_t ks, int g, mmq_w4 & w) {
    (void) a;
    const char * blk = wrow + ks * 144;
    w.hdr = *(const uint4 *) blk;
#pragma unroll
    for (int c = 0; c < 4; c++) w.q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
}

__device__ __forceinline__ void mmq_w_load(const mmq_args & a, const char * wrow, int64_t ks, int g, mmq_w8 & w) {
    const int64_t nblk = a.K / 32;
    const uint16_t * wsc = (const uint16_t *) (wrow + a.K);
#pragma unroll
    for (int bb = 0; bb < kQ8Group; bb++) {
        const int64_t b = ks * 8 + bb < nblk ? ks * 8 + bb : nblk - 1;
        w.q[bb] = *(const long *) (wrow + b * 32 + 8 * g);
        w.ds[bb] = wsc[b];
    }
}

template <int GRPS>
__device__ __forceinline__ void mmq_compute(const mmq_args & a, const mmq_slice & S, const mmq_w4 & w, int64_t ks,
                                            int r, int g, double (&acc)[4][4]) {
    (void) a;
    (void) ks;
#pragma unroll
    for (int grp = 0; grp < GRPS; grp++) {
        const int8_t * acol = &S.q[grp * 16 + r][0];
        long af[8];
#pragma unroll
        for (int j = 0; j < 8; j++) af[j] = *(const long *) (acol + 32 * j + 8 * g);
        const float4 d4 = *(const float4 *) &S.d[0][grp * 16 + 4 * g];
        const float ad[4] = {d4.x, d4.y, d4.z, d4.w};
        float ssa[2];
        q4k_ssum_operand(&S.ss[grp * 16 + r][0], true, g, ssa);  // columns past N were staged as zeros
        q4k_unit(w.hdr, w.q, af, ad, ssa, acc[grp]);
    }
}

template <int GRPS>
__device__ __forceinline__ void mmq_compute(const mmq_args & a, const mmq_slice & S, const mmq_w8 & w, int64_t ks,
                                            int r, int g, double (&acc)[4][4]) {
    const int64_t nblk = a.K / 32;
    const int nb = (int) (nblk - ks * 8 < kQ8Group ? nblk - ks * 8 : kQ8Group);
    // block by block (each (row, column) sum still takes its blocks in order),
    // the column groups inner: a block's weights and scale serve four groups
#pragma unroll
    for (int u = 0; u < kQ8Group; u++) {
        if (u >= nb) break;
#pragma unroll
        for (int grp = 0; grp < GRPS; grp++) {
            const long af = *(const long *) (&S.q[grp * 16 + r][32 * u + 8 * g]);
            const float4 d4 = *(const float4 *) &S.d[u][grp * 16 + 4 * g];
            const float da[4] = {d4.x, d4.y, d4.z, d4.w};
            q8_0_block(af, w.q[u], w.ds[u], da, acc[grp]);
        }
    }
}

template <int WT, int GRPS>
__global__ __launch_bounds__(256) void k_mmq(mmq_args a) {
    __shared__ __align__(16) mmq_slice s_buf[2];
    using wregs = typename std::conditional<WT == GGML_TYPE_Q4_K, mmq_w4, mmq_w8>::type;
    // contiguous runs of tiles per XCD
    const int64_t id = blockIdx.x;
    const int64_t t = (id % kMmqXcds) * a.per_xcd + id / kMmqXcds;
    if (t >= a.tiles) return;  // before any barrier: the whole workgroup leaves
    int64_t row_tile = t / a.col_blocks;
    const int64_t col_block = t % a.col_blocks;
    // sibling products: this tile's product, selected with constant indices
    // (an index into the argument arrays would put them in scratch memory)
    static_assert(kGemmFloatMaxSubs == 2, "product selection below");
    if (a.nsub > 0) {
        const int64_t r0 = row_tile * kMmqRows;
        int64_t base = 0, mend = a.sub_m0[1];
        const char * sw = a.sub_W[0];
        char * sd = a.sub_dst[0];
        const float * sb = a.sub_bias[0];
        if (r0 >= a.sub_m0[1]) {
            base = a.sub_m0[1], mend = a.sub_m0[2];
            sw = a.sub_W[1], sd = a.sub_dst[1], sb = a.sub_bias[1];
        }
        if (a.nsub >= 2 && r0 >= a.sub_m0[2]) {
            base = a.sub_m0[2], mend = a.sub_m0[3];
            sw = a.sub_W[2], sd = a.sub_dst[2], sb = a.sub_bias[2];
        }
        row_tile -= base / kMmqRows;
        a.M = mend - base;
        a.W = sw;
        a.dst = sd;
        a.dst_nb1 = a.M * 4;  // each product's output is contiguous
        a.epi.bias = sb;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t row = row_tile * kMmqRows + wave * 16 + r;
    const bool row_ok = row_tile * kMmqRows + wave * 16 < a.M;  // uniform per wave
    const int n0 = (int) (col_block * 16 * GRPS);
    const int ncol = min(16 * GRPS, a.N - n0);
    const int64_t nks = (a.K + 255) / 256;
    const char * wrow = a.W + (row_ok ? row : 0) * a.row_bytes;
    double acc[4][4];
#pragma unroll
    for (int grp = 0; grp < 4; grp++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[grp][i] = 0.0;
    mmq_act act;
    wregs wn;
    mmq_act_load<WT, GRPS>(a, n0, ncol, 0, act);
    mmq_w_load(a, wrow, 0, g, wn);
    for (int64_t ks = 0; ks < nks; ks++) {
        mmq_slice & S = s_buf[ks & 1];
        mmq_act_store<WT, GRPS>(a, ncol, ks, act, S);
        const wregs w = wn;
        __syncthreads();
        if (ks + 1 < nks) {
            mmq_act_load<WT, GRPS>(a, n0, ncol, ks + 1, act);
            mmq_w_load(a, wrow, ks + 1, g, wn);
        }
        if (row_ok) mmq_compute<GRPS>(a, S, w, ks, r, g, acc);
    }
    if (!row_ok) return;
    // the adds, then (GELU_ERF) the lane's GELUs together, then the stores
    float o[4 * GRPS];
#pragma unroll
    for (int grp = 0; grp < GRPS; grp++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + grp * 16 + 4 * g + i;
            float v = (float) acc[grp][i];
            if (n < a.N) {
                if (a.epi.bias) v = v + a.epi.bias[row];
                if (a.epi.res) v = v + *(const float *) ((const char *) a.epi.res + (int64_t) n * a.dst_nb1 + row * 4);
            }
            o[grp * 4 + i] = v;
        }
    }
    if (a.epi.gelu_erf) gelu_erf_det_n<4 * GRPS>(o);
#pragma unroll
    for (int grp = 0; grp < GRPS; grp++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + grp * 16 + 4 * g + i;
            if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + row * 4) = o[grp * 4 + i];
        }
    }
}

bool mmq_supported(int wtype, int64_t M, int64_t K) {
    if (M % 16 != 0) return false;
    if (wtype == GGML_TYPE_Q4_K) return K % 256 == 0;
    if (wtype == GGML_TYPE_Q8_0) return K % 32 == 0;
    return false;
}

void launch_mmq(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu, const gemm_float_epi & epi,
                const gemm_float_sub * subs, int nsub) {
    mmq_args a;
    a.nsub = 0;
    int64_t m_all = M;
    if (nsub > 0 && nsub <= kGemmFloatMaxSubs && M % kMmqRows == 0 && !epi.res && !epi.gelu_erf) {
        a.nsub = nsub;
        a.sub_m0[0] = 0;
        a.sub_W[0] = W;
        a.sub_dst[0] = dst;
        a.sub_bias[0] = epi.bias;
        for (int i = 0; i < nsub; i++) {
            a.sub_m0[i + 1] = m_all;
            a.sub_W[i + 1] = subs[i].a;
            a.sub_dst[i + 1] = subs[i].d;
            a.sub_bias[i + 1] = subs[i].bias;
            m_all += subs[i].M;
        }
        a.sub_m0[nsub + 1] = m_all;
    } else if (nsub > 0) {
        // not joinable: each product on its own
        launch_mmq(wtype, W, row_bytes, M, K, act, N, dst, dst_nb1, stream, n_cu, epi);
        for (int i = 0; i < nsub; i++) {
            gemm_float_epi ei;
            ei.bias = subs[i].bias;
            launch_mmq(wtype, subs[i].a, row_bytes, subs[i].M, K, act, N, subs[i].d, subs[i].M * 4, stream, n_cu, ei);
        }
        return;
    }
    a.epi = epi;
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
    // 32-column tiles where 64-column tiles leave CUs idle (the audio
    // encoder's 896-row projections over 390 positions: 98 -> 182 tiles)
    const int64_t row_tiles = (m_all + kMmqRows - 1) / kMmqRows;
    const bool narrow = N > 32 && row_tiles * ((N + kMmqCols - 1) / kMmqCols) < n_cu;
    const int cols = narrow ? 32 : kMmqCols;
    a.col_blocks = (N + cols - 1) / cols;
    a.tiles = row_tiles * a.col_blocks;
    a.per_xcd = (a.tiles + kMmqXcds - 1) / kMmqXcds;
    const dim3 grid((unsigned) (a.per_xcd * kMmqXcds));
    if (wtype == GGML_TYPE_Q4_K) {
        if (narrow) hipLaunchKernelGGL((k_mmq<GGML_TYPE_Q4_K, 2>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((k_mmq<GGML_TYPE_Q4_K, 4>), grid, dim3(256), 0, stream, a);
    } else {
        if (narrow) hipLaunchKernelGGL((k_mmq<GGML_TYPE_Q8_0, 2>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((k_mmq<GGML_TYPE_Q8_0, 4>), grid, dim3(256), 0, stream, a);
    }
}

}  // namespace mi355x

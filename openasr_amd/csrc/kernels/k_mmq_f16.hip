// k_mmq_f16.hip -- GGML_OP_MUL_MAT on Q4_K / Q8_0 weights for wide
// activation batches (prefill chunks) at the default precision, on the f16
// matrix cores. Call site of the op:
// crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686; a quantized
// MUL_MAT is built at the default precision (GGML_PREC_F32 is set only on
// F16 x F32 products a backend flags, cpu_graph.rs:156-165, 3683), the
// contract under which a backend takes its fastest validated form.
// GGML_PREC_F32 keeps the exact int8 tile GEMM of k_mmq.hip.
//
// Arithmetic (float tolerance): the activations are quantized exactly as
// for the exact path (Q8_K for Q4_K weights, Q8_0 for Q8_0 weights: the
// same int8 values and scales), then dequantized once per launch into an f16
// copy d_a * q_a (one rounding); the weights are dequantized while they are
// staged -- Q4_K: (d * sc_j) * q - dmin * m_j with the two scale products
// rounded to f16 and one f16 fused multiply-add; Q8_0: d * q, one rounding --
// and the products run on v_mfma_f32_16x16x32_f16 with f32 sums. Each
// operand element carries at most a few f16 roundings (2^-11 relative); the
// result is held to 2e-3 of the exact product.
//
// Why: the exact tile GEMM spends 14-25 VALU instructions on every int8
// MFMA forming f64 block sums (VALU 80 % busy, MFMA 27 %). Here the scaling
// happens once per staged weight element (shared by the tile's 128 columns)
// and the inner loop is LDS reads and MFMAs only.
//
// Work: a workgroup of four waves owns a 128 (weight rows) x 128
// (activation columns) output tile and walks K in 64-wide steps. A step's
// weights and activations are requested into registers while the previous
// step is multiplied, then dequantized into the other of two LDS buffers
// (16-byte pieces XOR-swizzled by row: conflict-free fragment reads, 64 KB
// of LDS a workgroup); one barrier a
// step (174 VGPRs + 88 AGPRs: one workgroup a CU; held to two a CU, 256
// registers a lane, the compiler fits without spills but the GEMM measured
// 1-5 % slower). Wave (wr, wc) multiplies the 64 x 64 quarter (wr: rows, wc:
// columns) as 4 x 4 blocks of 16 x 16: the activations are the MFMA A
// operand (lane l: column l % 16, k 8 (l / 16) .. + 7), the weights the B
// operand, so lane l ends with weight row l % 16 of four consecutive
// columns and a tile's stores are 64-byte runs of an output column. Tiles
// are dealt to the XCDs in contiguous runs (workgroup i on XCD i % 8), the
// column blocks of a row tile adjacent, so a weight tile is fetched into one
// L2.
#include <type_traits>

#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

namespace {

constexpr int kHM = 128, kHN = 128, kHK = 64;
constexpr int kHRow = kHK;  // staged row: 64 halves, its 16-byte pieces XOR-swizzled by the row

// the staged row's 16-byte piece p (eight halves): stored at slot p ^ (row %
// 8), so that the fragment reads (16 rows, one piece each) spread over the
// banks
__device__ __forceinline__ uint4 * hq_slot(uint16_t (*a)[kHRow], int row, int piece) {
    return (uint4 *) &a[row][8 * (piece ^ (row & 7))];
}
constexpr int kHThreads = 256;
constexpr int kHXcds = 8;

typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
typedef _Float16 hh8 __attribute__((ext_vector_type(8)));
typedef float hf4 __attribute__((ext_vector_type(4)));

struct mmqh_args {
    const char * W;
    const char * W2;  // SwiGLU form: the up matrix (W the gate), same shape
    int64_t row_bytes, M, K;
    const uint16_t * x16;  // the dequantized activations, f16 [N][K]
    int N;
    char * dst;
    int64_t dst_nb1;
    int64_t col_blocks, tiles, per_xcd;
    gemm_float_epi epi;
    // sibling products of the same activations (rows [sub_m0[i], sub_m0[i +
    // 1]) are product i: weights, contiguous output, bias); each a multiple
    // of 128 rows
    int nsub;
    int64_t sub_m0[kGemmFloatMaxSubs + 2];
    const char * sub_W[kGemmFloatMaxSubs + 1];
    char * sub_dst[kGemmFloatMaxSubs + 1];
    const float * sub_bias[kGemmFloatMaxSubs + 1];
};

// bytes b0 .. b3 of v as f16 values 1024 + b (the byte in the mantissa under
// the exponent of 1024): (b0, b1) and (b2, b3)
__device__ __forceinline__ void hq_bytes(uint32_t v, hh2 & p01, hh2 & p23) {
    p01 = __builtin_bit_cast(hh2, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
    p23 = __builtin_bit_cast(hh2, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
}

__device__ __forceinline__ uint32_t hq_u32(hh2 v) { return __builtin_bit_cast(uint32_t, v); }

// eight nibbles-in-bytes (each < 16) of two words, as x * s + nm in f16
__device__ __forceinline__ uint4 hq_nibbles(uint32_t w0, uint32_t w1, hh2 s, hh2 nm) {
    const hh2 k1024 = {(_Float16) 1024.0f, (_Float16) 1024.0f};
    hh2 a, b, c, d;
    hq_bytes(w0, a, b);
    hq_bytes(w1, c, d);
    a = __builtin_elementwise_fma(a - k1024, s, nm);
    b = __builtin_elementwise_fma(b - k1024, s, nm);
    c = __builtin_elementwise_fma(c - k1024, s, nm);
    d = __builtin_elementwise_fma(d - k1024, s, nm);
    return make_uint4(hq_u32(a), hq_u32(b), hq_u32(c), hq_u32(d));
}

// eight signed bytes of two words, as q * s in f16 (q + 128 in the mantissa
// under the exponent of 1024, then 1152 taken off: exact)
__device__ __forceinline__ uint4 hq_int8(uint32_t w0, uint32_t w1, hh2 s) {
    const hh2 k1152 = {(_Float16) 1152.0f, (_Float16) 1152.0f};
    hh2 a, b, c, d;
    hq_bytes(w0 ^ 0x80808080u, a, b);
    hq_bytes(w1 ^ 0x80808080u, c, d);
    a = (a - k1152) * s;
    b = (b - k1152) * s;
    c = (c - k1152) * s;
    d = (d - k1152) * s;
    return make_uint4(hq_u32(a), hq_u32(b), hq_u32(c), hq_u32(d));
}

// a thread's share of one K step, held in registers between its request and
// its store: weights of row r = t / 2, half h = t % 2 (Q4_K: the 16 bytes
// holding sub-blocks 2c and 2c + 1 at elements 16 h .. 16 h + 15, plus the
// super-block header; Q8_0: the 32 quants of block 2 s + h and its scale);
// activations: 16-byte piece t % 8 of columns t / 8 + 32 i (i = 0 .. 3). Only
// 16-byte members: a narrower one leaves padding that keeps the struct in
// scratch memory.
struct hq_regs {
    uint4 w0, w1;
    uint4 hdr;  // Q4_K: the super-block header; Q8_0: .x the block's f16 scale
    uint4 x0, x1, x2, x3;
};

template <int WT>
__device__ __forceinline__ void hq_load(const mmqh_args & a, const char * wrow, int n0, int64_t k0, hq_regs & r) {
    const int t = (int) threadIdx.x, h = t & 1;
    if constexpr (WT == GGML_TYPE_Q4_K) {
        const char * blk = wrow + (k0 / 256) * 144;
        const int c = (int) ((k0 % 256) / 64);
        r.hdr = *(const uint4 *) blk;
        r.w0 = *(const uint4 *) (blk + 16 + 32 * c + 16 * h);
    } else {
        const int64_t bk = k0 / 32 + h;
        r.w0 = *(const uint4 *) (wrow + bk * 32);
        r.w1 = *(const uint4 *) (wrow + bk * 32 + 16);
        r.hdr = make_uint4(((const uint16_t *) (wrow + a.K))[bk], 0, 0, 0);
    }
    // activations: piece q = t + 256 i (i = 0 .. 3) is 16-byte piece q % 8 of
    // column q / 8, so eight consecutive lanes read one column's whole 128
    // bytes of the step
    const uint16_t * xs = a.x16 + k0 + 8 * (t & 7);
    auto xcol = [&](int i) { return (int64_t) min(n0 + (t >> 3) + 32 * i, a.N - 1) * a.K; };
    r.x0 = *(const uint4 *) (xs + xcol(0));
    r.x1 = *(const uint4 *) (xs + xcol(1));
    r.x2 = *(const uint4 *) (xs + xcol(2));
    r.x3 = *(const uint4 *) (xs + xcol(3));
}

template <int WT>
__device__ __forceinline__ void hq_store(const hq_regs & r, int64_t k0, uint16_t (*sw)[kHRow],
                                         uint16_t (*sx)[kHRow]) {
    const int t = (int) threadIdx.x, row = t >> 1, h = t & 1;
    if constexpr (WT == GGML_TYPE_Q4_K) {
        // sub-blocks j = 2c (low nibbles) and 2c + 1 (high nibbles):
        // get_scale_min_k4 of the header's 12 scale bytes
        const int c = (int) ((k0 % 256) / 64);
        const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
        auto scale_min = [&](int j, float & sc, float & mn) {
            if (j < 4) {
                sc = (float) ((s0 >> (8 * j)) & 63);
                mn = (float) ((s1 >> (8 * j)) & 63);
            } else {
                const int q = j - 4;
                sc = (float) (((s2 >> (8 * q)) & 0xF) | (((s0 >> (8 * q + 6)) & 3) << 4));
                mn = (float) (((s2 >> (8 * q + 4)) & 0xF) | (((s1 >> (8 * q + 6)) & 3) << 4));
            }
        };
        const float d = half_bits_to_float((uint16_t) (r.hdr.x & 0xFFFF));
        const float dmin = half_bits_to_float((uint16_t) (r.hdr.x >> 16));
        float sc0, mn0, sc1, mn1;
        scale_min(2 * c, sc0, mn0);
        scale_min(2 * c + 1, sc1, mn1);
        const _Float16 a0 = (_Float16) (d * sc0), b0 = (_Float16) (-(dmin * mn0));
        const _Float16 a1 = (_Float16) (d * sc1), b1 = (_Float16) (-(dmin * mn1));
        const hh2 sl = {a0, a0}, ml = {b0, b0}, sh = {a1, a1}, mh = {b1, b1};
        const uint32_t q[4] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = q[i] & 0x0F0F0F0Fu;
            hi[i] = (q[i] >> 4) & 0x0F0F0F0Fu;
        }
        *hq_slot(sw, row, 2 * h) = hq_nibbles(lo[0], lo[1], sl, ml);
        *hq_slot(sw, row, 2 * h + 1) = hq_nibbles(lo[2], lo[3], sl, ml);
        *hq_slot(sw, row, 4 + 2 * h) = hq_nibbles(hi[0], hi[1], sh, mh);
        *hq_slot(sw, row, 4 + 2 * h + 1) = hq_nibbles(hi[2], hi[3], sh, mh);
    } else {
        const _Float16 ds = (_Float16) half_bits_to_float((uint16_t) r.hdr.x);
        const hh2 s = {ds, ds};
        *hq_slot(sw, row, 4 * h) = hq_int8(r.w0.x, r.w0.y, s);
        *hq_slot(sw, row, 4 * h + 1) = hq_int8(r.w0.z, r.w0.w, s);
        *hq_slot(sw, row, 4 * h + 2) = hq_int8(r.w1.x, r.w1.y, s);
        *hq_slot(sw, row, 4 * h + 3) = hq_int8(r.w1.z, r.w1.w, s);
    }
    const int xc = t >> 3, xp = t & 7;
    *hq_slot(sx, xc, xp) = r.x0;
    *hq_slot(sx, xc + 32, xp) = r.x1;
    *hq_slot(sx, xc + 64, xp) = r.x2;
    *hq_slot(sx, xc + 96, xp) = r.x3;
}

// SWI (the SwiGLU pair, MUL(SILU(W x), W2 x)): a tile holds 64 gate rows
// (tile rows 0 .. 63) and the same 64 rows of the up matrix (64 .. 127); the
// up waves hand their sums to the gate waves through LDS, which store
// silu(g) * u for the 64 rows -- the roundings of MUL_MAT, SILU and MUL apart.
template <int WT, bool SWI>
__global__ __launch_bounds__(kHThreads) void k_mmq_f16(mmqh_args a) {
    __shared__ __align__(16) uint16_t s_w[2][kHM][kHRow];
    __shared__ __align__(16) uint16_t s_x[2][kHN][kHRow];
    const int64_t id = blockIdx.x;
    const int64_t t = (id % kHXcds) * a.per_xcd + id / kHXcds;
    if (t >= a.tiles) return;  // before any barrier: the whole workgroup leaves
    int64_t row_tile = t / a.col_blocks;
    const int64_t col_block = t % a.col_blocks;
    // sibling products: this tile's product, selected with constant indices
    static_assert(kGemmFloatMaxSubs == 2, "product selection below");
    if (a.nsub > 0) {
        const int64_t r0 = row_tile * kHM;
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
        row_tile -= base / kHM;
        a.M = mend - base;
        a.W = sw;
        a.dst = sd;
        a.dst_nb1 = a.M * 4;  // each product's output is contiguous
        a.epi.bias = sb;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = wave & 1, wc = wave >> 1;
    const int64_t m0 = row_tile * (SWI ? kHM / 2 : kHM);  // the tile's first output row
    const int n0 = (int) (col_block * kHN);
    // this thread's staging row (rows past M repeat the last one; their
    // outputs are not stored)
    const int sr = (int) (threadIdx.x >> 1);
    const char * wrow = SWI ? (sr < kHM / 2 ? a.W : a.W2) + min(m0 + (sr & (kHM / 2 - 1)), a.M - 1) * a.row_bytes
                            : a.W + min(m0 + sr, a.M - 1) * a.row_bytes;
    const int64_t nsteps = a.K / kHK;
    hf4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = hf4{0.f, 0.f, 0.f, 0.f};
    // two register sets, step j in set j % 2: a step's loads are issued two
    // steps before its rows are stored into LDS, so two steps of MFMAs cover
    // their latency
    // (loads past the last step repeat it: unconditional, in bounds, unused)
    auto kstep = [&](int64_t j) { return (j < nsteps ? j : nsteps - 1) * kHK; };
    hq_regs ra, rb;
    hq_load<WT>(a, wrow, n0, 0, ra);
    hq_load<WT>(a, wrow, n0, kstep(1), rb);
    hq_store<WT>(ra, 0, s_w[0], s_x[0]);
    hq_load<WT>(a, wrow, n0, kstep(2), ra);
    __syncthreads();
    const int fr = lane & 15, fp = lane >> 4;  // fragment row, 16-byte piece
    auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            uint4 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = *hq_slot(s_x[buf], wc * 64 + 16 * i + fr, 4 * ks + fp);
#pragma unroll
            for (int j = 0; j < 4; j++) bf[j] = *hq_slot(s_w[buf], wr * 64 + 16 * j + fr, 4 * ks + fp);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(hh8, af[i]),
                                                                        __builtin_bit_cast(hh8, bf[j]), acc[i][j], 0,
                                                                        0, 0);
        }
    };
    // step s (set and buffer s % 2): multiply buffer s % 2, store step s + 1
    // into the other buffer -- last read in step s - 1, before the barrier
    // that ended it -- and reload that set with step s + 3
    // an even number of steps (K % 128 == 0): no conditions in the loop (the
    // last stores repeat the last step into a buffer nobody reads again)
    for (int64_t s = 0; s < nsteps; s += 2) {
        compute(0);
        hq_store<WT>(rb, kstep(s + 1), s_w[1], s_x[1]);
        hq_load<WT>(a, wrow, n0, kstep(s + 3), rb);
        __syncthreads();
        compute(1);
        hq_store<WT>(ra, kstep(s + 2), s_w[0], s_x[0]);
        hq_load<WT>(a, wrow, n0, kstep(s + 4), ra);
        __syncthreads();
    }
    if constexpr (SWI) {
        // the up waves' sums through the staging buffers (free after the
        // loop's last barrier): lane, block (i, j) of wave column wc
        hf4 * s_up = (hf4 *) &s_w[0][0][0];
        static_assert(sizeof(s_w) >= 2 * 16 * 64 * sizeof(hf4), "staging buffers hold the up sums");
        if (wr == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) s_up[(wc * 16 + 4 * i + j) * 64 + lane] = acc[i][j];
        }
        __syncthreads();
        if (wr == 0) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t m = m0 + 16 * j + fr;
                if (m >= a.M) continue;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const hf4 up = s_up[(wc * 16 + 4 * i + j) * 64 + lane];
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int n = n0 + wc * 64 + 16 * i + 4 * (lane >> 4) + v;
                        const float g = acc[i][j][v];
                        if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + m * 4) = (g / (1.0f + expf_det(-g))) * up[v];
                    }
                }
            }
        }
        return;
    }
    // lane: weight row m0 + 64 wr + 16 j + lane % 16 of columns n0 + 64 wc +
    // 16 i + 4 (lane / 16) + v; the adds, then (GELU_ERF) the lane's values
    // together, then the stores
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t m = m0 + wr * 64 + 16 * j + fr;
        float o[16];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int n = n0 + wc * 64 + 16 * i + 4 * (lane >> 4) + v;
                float x = acc[i][j][v];
                if (m < a.M && n < a.N) {
                    if (a.epi.bias) x = x + a.epi.bias[m];
                    if (a.epi.res) x = x + *(const float *) ((const char *) a.epi.res + (int64_t) n * a.dst_nb1 + m * 4);
                }
                o[4 * i + v] = x;
            }
        if (a.epi.gelu_erf) gelu_erf_det_n<16>(o);
        if (m < a.M) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int n = n0 + wc * 64 + 16 * i + 4 * (lane >> 4) + v;
                    if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + m * 4) = o[4 * i + v];
                }
        }
    }
}

// the quantized activations dequantized to f16: x16[n][k] = f16(d * q), eight
// elements a thread
template <int WT>
__global__ __launch_bounds__(256) void k_act_f16(act_buffers act, int64_t K, int64_t N, uint16_t * __restrict__ x16) {
    const int64_t i = ((int64_t) blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= K * N) return;
    const int64_t n = i / K, k = i % K;
    const uint2 q = *(const uint2 *) (act.q + i);
    const float d = WT == GGML_TYPE_Q4_K ? act.d[n * (K / 256) + k / 256] : act.d[n * (K / 32) + k / 32];
    const uint32_t qw[2] = {q.x, q.y};
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 2; w++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const float lo = d * (float) (int8_t) ((qw[w] >> (16 * b)) & 0xFF);
            const float hi = d * (float) (int8_t) ((qw[w] >> (16 * b + 8)) & 0xFF);
            o[2 * w + b] = (uint32_t) float_to_half_bits(lo) | ((uint32_t) float_to_half_bits(hi) << 16);
        }
    *(uint4 *) (x16 + i) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

bool mmq_f16_supported(int wtype, int64_t M, int64_t K, int64_t N, int n_cu) {
    if (wtype == GGML_TYPE_Q4_K) {
        if (K % 256 != 0) return false;
    } else if (wtype == GGML_TYPE_Q8_0) {
        if (K % (2 * kHK) != 0) return false;  // an even number of steps
    } else {
        return false;
    }
    // a workgroup for every CU at least (fewer, larger tiles than the exact
    // tile GEMM: below that the exact form keeps the product), and columns
    // that fill most of a tile (151936 x 1024 at 64 columns: Q4_K 78 us
    // here against 64 in the exact form, Q8_0 90 against 104)
    const int64_t tiles = (M + kHM - 1) / kHM * ((N + kHN - 1) / kHN);
    const int64_t min_n = wtype == GGML_TYPE_Q4_K ? kHN : kHN / 2;
    return M % 16 == 0 && N >= min_n && tiles >= n_cu;
}

size_t mmq_f16_scratch_bytes(int64_t K, int64_t N) { return (size_t) (K * N * 2 + 256); }

void launch_mmq_f16(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                    int64_t N, char * dst, int64_t dst_nb1, void * scratch, hipStream_t stream,
                    const gemm_float_epi & epi, const gemm_float_sub * subs, int nsub, const char * W2) {
    uint16_t * x16 = (uint16_t *) scratch;
    const int64_t n8 = K * N / 8;
    if (wtype == GGML_TYPE_Q4_K)
        hipLaunchKernelGGL(k_act_f16<GGML_TYPE_Q4_K>, dim3((unsigned) ((n8 + 255) / 256)), dim3(256), 0, stream, act, K,
                           N, x16);
    else
        hipLaunchKernelGGL(k_act_f16<GGML_TYPE_Q8_0>, dim3((unsigned) ((n8 + 255) / 256)), dim3(256), 0, stream, act, K,
                           N, x16);
    if (W2) {
        // the SwiGLU pair: 64 output rows a tile, no epilogue adds or siblings
        if (nsub != 0 || epi.bias || epi.res || epi.gelu_erf || M % (kHM / 2) != 0) {
            note_hip_error(hipErrorInvalidValue);
            return;
        }
        mmqh_args b = mmqh_args{};
        b.W = W, b.W2 = W2, b.row_bytes = row_bytes, b.M = M, b.K = K, b.x16 = x16, b.N = (int) N, b.dst = dst;
        b.dst_nb1 = dst_nb1;
        b.nsub = 0;
        b.col_blocks = (N + kHN - 1) / kHN;
        b.tiles = M / (kHM / 2) * b.col_blocks;
        b.per_xcd = (b.tiles + kHXcds - 1) / kHXcds;
        const dim3 grid((unsigned) (b.per_xcd * kHXcds));
        if (wtype == GGML_TYPE_Q4_K) hipLaunchKernelGGL((k_mmq_f16<GGML_TYPE_Q4_K, true>), grid, dim3(kHThreads), 0, stream, b);
        else hipLaunchKernelGGL((k_mmq_f16<GGML_TYPE_Q8_0, true>), grid, dim3(kHThreads), 0, stream, b);
        return;
    }
    mmqh_args a;
    a.W2 = nullptr;
    a.nsub = 0;
    int64_t m_all = M;
    bool joined = nsub == 0;
    if (nsub > 0 && nsub <= kGemmFloatMaxSubs && M % kHM == 0 && !epi.res && !epi.gelu_erf) {
        joined = true;
        for (int i = 0; i < nsub; i++) joined = joined && subs[i].M % kHM == 0;
    }
    if (!joined) {
        // not joinable: each product on its own (the activations converted once)
        gemm_float_sub none[1];
        (void) none;
        mmqh_args b;
        auto one = [&](const char * w, int64_t m, char * d, int64_t nb1, const gemm_float_epi & e) {
            b = mmqh_args{};
            b.W = w, b.row_bytes = row_bytes, b.M = m, b.K = K, b.x16 = x16, b.N = (int) N, b.dst = d, b.dst_nb1 = nb1;
            b.epi = e;
            b.nsub = 0;
            b.col_blocks = (N + kHN - 1) / kHN;
            b.tiles = (m + kHM - 1) / kHM * b.col_blocks;
            b.per_xcd = (b.tiles + kHXcds - 1) / kHXcds;
            const dim3 grid((unsigned) (b.per_xcd * kHXcds));
            if (wtype == GGML_TYPE_Q4_K)
                hipLaunchKernelGGL((k_mmq_f16<GGML_TYPE_Q4_K, false>), grid, dim3(kHThreads), 0, stream, b);
            else hipLaunchKernelGGL((k_mmq_f16<GGML_TYPE_Q8_0, false>), grid, dim3(kHThreads), 0, stream, b);
        };
        one(W, M, dst, dst_nb1, epi);
        for (int i = 0; i < nsub; i++) {
            gemm_float_epi ei;
            ei.bias = subs[i].bias;
            one(subs[i].a, subs[i].M, subs[i].d, subs[i].M * 4, ei);
        }
        return;
    }
    if (nsub > 0) {
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
    }
    a.epi = epi;
    a.W = W;
    a.row_bytes = row_bytes;
    a.M = M;
    a.K = K;
    a.x16 = x16;
    a.N = (int) N;
    a.dst = dst;
    a.dst_nb1 = dst_nb1;
    a.col_blocks = (N + kHN - 1) / kHN;
    a.tiles = (m_all + kHM - 1) / kHM * a.col_blocks;
    a.per_xcd = (a.tiles + kHXcds - 1) / kHXcds;
    const dim3 grid((unsigned) (a.per_xcd * kHXcds));
    if (wtype == GGML_TYPE_Q4_K) hipLaunchKernelGGL((k_mmq_f16<GGML_TYPE_Q4_K, false>), grid, dim3(kHThreads), 0, stream, a);
    else hipLaunchKernelGGL((k_mmq_f16<GGML_TYPE_Q8_0, false>), grid, dim3(kHThreads), 0, stream, a);
}

}  // namespace mi355x

// k_gemm_float.hip -- GGML_OP_MUL_MAT with float weights (F16 or F32 src0)
// over many columns, on the matrix cores: the dense projections and the
// convolution GEMM of the audio encoders (crates/openasr-core/src/nn/conv.rs:
// 82-110, nn/encoder.rs:678-870, models/qwen/audio_encoder.rs:520-668) and
// the score / context products of the unfused attention chain
// (nn/decoder.rs:2154-2200). Call site of the op:
// crates/openasr-core/src/ggml_runtime/cpu_graph.rs:3652-3686.
//
// Operand types follow ggml-cpu's vec_dot_type rule: an F16 src0 takes its
// columns rounded to f16 (f16 x f16 products, exact in f32, summed in f32 on
// v_mfma_f32_16x16x32_f16); an F32 src0 takes f32 columns (an F16 src1 is
// widened) on v_mfma_f32_16x16x4f32. The sums are f32 in the matrix core's
// order: the result is within float tolerance of the reference, not bit
// for bit (the CPU's own SIMD reduction order differs by ISA as well).
//
// Tiling: a workgroup of four waves owns a 64 (rows of src0) x 64 (columns)
// output tile and walks K in 32-wide slabs staged through LDS, the next
// slab's global loads in flight while the current one is multiplied. The
// columns are the MFMA A operand and the weight rows the B operand, so each
// lane ends with one output row (lane % 16) of four columns, and a store of
// the tile writes 64-byte runs of consecutive rows.
#include <algorithm>
#include <type_traits>

#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

namespace {

constexpr int kGfBM = 64, kGfBN = 64, kGfBK = 32;
constexpr int kGfDepth = 4;  // slabs in flight in the aligned form (even: slab s is in LDS buffer s % 2)
constexpr int kGfThreads = 256;

typedef float gf_v4f __attribute__((ext_vector_type(4)));
typedef _Float16 gf_v8h __attribute__((ext_vector_type(8)));

// element k of a row of type f16 (t16) or f32, as float
__device__ __forceinline__ float gf_elem(const char * row, int64_t k, bool t16) {
    return t16 ? half_bits_to_float(((const uint16_t *) row)[k]) : ((const float *) row)[k];
}

// eight consecutive elements k0 .. k0 + 7 of a row (zero past K), as floats;
// vec: the row and k0 are 16-byte aligned for this type (one or two vector loads)
__device__ __forceinline__ void gf_load8(const char * row, int64_t k0, int64_t K, bool t16, bool vec, bool live,
                                         float (&v)[8]) {
    if (live && vec && k0 + 8 <= K) {
        if (t16) {
            const uint4 w = *(const uint4 *) (row + 2 * k0);
            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[2 * i] = half_bits_to_float((uint16_t) (u[i] & 0xFFFF));
                v[2 * i + 1] = half_bits_to_float((uint16_t) (u[i] >> 16));
            }
        } else {
            const float4 a = *(const float4 *) (row + 4 * k0), b = *(const float4 *) (row + 4 * k0 + 16);
            v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = live && k0 + i < K ? gf_elem(row, k0 + i, t16) : 0.0f;
}

}  // namespace

// the epilogue of output (m, n) with accumulated value o, into dst
__device__ __forceinline__ void gf_epi_store(const gemm_float_args & g, float o, int64_t m, int64_t n, char * dbase) {
    if (g.epi.bias) o = o + g.epi.bias[m];
    if (g.epi.bias_col) o = o + g.epi.bias_col[n];
    // the residual has the output's layout (contiguous, same batch offsets)
    if (g.epi.res) o = o + ((const float *) ((const char *) g.epi.res + (dbase - g.d) + n * g.d_nb1))[m];
    if (g.epi.gelu_erf) o = gelu_erf_det(o);
    if (g.epi.perm_rows) {
        const int64_t pr = g.epi.perm_rows;
        ((float *) g.d)[m % pr + pr * n + pr * g.N * (m / pr)] = o;
    } else {
        ((float *) (dbase + n * g.d_nb1))[m] = o;
    }
}

// the wave's 32 x 32 outputs (lane: row wr + 16 i + (lane % 16), columns wc
// + 16 j + 4 (lane / 16) + v) through the epilogue into dst, or as they are
// into a split's partials (part: column-major M x N)
__device__ __forceinline__ void gf_store(const gemm_float_args & g, const gf_v4f (&acc)[2][2], int64_t m0, int64_t n0,
                                         int wr, int wc, int lane, char * dbase, float * part = nullptr) {
    const int r16 = lane & 15, cg = lane >> 4;
    if (part || !g.epi.gelu_erf) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int64_t m = m0 + wr + 16 * i + r16;
            if (m >= g.M) continue;
#pragma unroll
            for (int j = 0; j < 2; j++) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int64_t n = n0 + wc + 16 * j + 4 * cg + v;
                    if (n >= g.N) continue;
                    if (part) part[n * g.M + m] = acc[i][j][v];
                    else gf_epi_store(g, acc[i][j][v], m, n, dbase);
                }
            }
        }
        return;
    }
    // with GELU_ERF: the lane's 16 values through the adds, then the 16
    // GELUs together (interleaved chains), then the stores
    gemm_float_epi e2 = g.epi;
    e2.gelu_erf = false;
    gemm_float_args g2 = g;
    g2.epi = e2;
    float o[16];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int64_t m = m0 + wr + 16 * i + r16, n = n0 + wc + 16 * j + 4 * cg + v;
                float x = acc[i][j][v];
                if (m < g.M && n < g.N) {
                    if (g.epi.bias) x = x + g.epi.bias[m];
                    if (g.epi.bias_col) x = x + g.epi.bias_col[n];
                    if (g.epi.res) x = x + ((const float *) ((const char *) g.epi.res + (dbase - g.d) + n * g.d_nb1))[m];
                }
                o[(i * 2 + j) * 4 + v] = x;
            }
    gelu_erf_det_n<16>(o);
    g2.epi.bias = g2.epi.bias_col = g2.epi.res = nullptr;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int64_t m = m0 + wr + 16 * i + r16;
        if (m >= g.M) continue;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int64_t n = n0 + wc + 16 * j + 4 * cg + v;
                if (n < g.N) gf_epi_store(g2, o[(i * 2 + j) * 4 + v], m, n, dbase);
            }
    }
}

// one slab's MFMAs from LDS (sa, sb) into the wave's 32 x 32 outputs
template <bool F16, typename T, int PADE>
__device__ __forceinline__ void gf_mfma(const T (*sa)[kGfBK + PADE], const T (*sb)[kGfBK + PADE], int wr, int wc,
                                        int lane, gf_v4f (&acc)[2][2]) {
    const int r16 = lane & 15, kg = lane >> 4;
    if constexpr (F16) {
        // A: column wc + 16 j + r16, k 8 kg .. + 7; B: row wr + 16 i + r16, same k
        gf_v8h bo[2], ao[2];
#pragma unroll
        for (int j = 0; j < 2; j++) bo[j] = *(const gf_v8h *) &sb[wc + 16 * j + r16][8 * kg];
#pragma unroll
        for (int i = 0; i < 2; i++) ao[i] = *(const gf_v8h *) &sa[wr + 16 * i + r16][8 * kg];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bo[j], ao[i], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
        for (int kk = 0; kk < kGfBK; kk += 4) {
            float bo[2], ao[2];
#pragma unroll
            for (int j = 0; j < 2; j++) bo[j] = sb[wc + 16 * j + r16][kk + kg];
#pragma unroll
            for (int i = 0; i < 2; i++) ao[i] = sa[wr + 16 * i + r16][kk + kg];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bo[j], ao[i], acc[i][j], 0, 0, 0);
        }
    }
}

// eight elements k0 .. k0 + 7 of a 16-byte aligned row of a K % 8 == 0
// operand, raw (one 16-byte load for f16, two for f32) with whether they are
// live (inside K and a live row). The load is always made (clamped to the
// row start) and the mask applied only when the slab is staged: a load
// behind a branch, or a value used right after its load, would make the step
// wait for every load in flight.
struct gf_raw {
    uint4 r[2];
    bool ok;
};
template <bool T16>
__device__ __forceinline__ void gf_load_raw(const char * row, int64_t k0, int64_t K, bool live, gf_raw & v) {
    v.ok = live && k0 < K;
    const int64_t kc = v.ok ? k0 : 0;
    if constexpr (T16) {
        v.r[0] = *(const uint4 *) (row + 2 * kc);
    } else {
        v.r[0] = *(const uint4 *) (row + 4 * kc);
        v.r[1] = *(const uint4 *) (row + 4 * kc + 16);
    }
}

// a raw operand piece as eight f16 (T16 source: as is; f32: rounded to
// nearest even) or eight f32 values, zeros when not live
template <bool T16>
__device__ __forceinline__ uint4 gf_as_f16(const gf_raw & v) {
    if constexpr (T16) return v.ok ? v.r[0] : make_uint4(0, 0, 0, 0);
    const uint32_t f[8] = {v.r[0].x, v.r[0].y, v.r[0].z, v.r[0].w, v.r[1].x, v.r[1].y, v.r[1].z, v.r[1].w};
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = (uint32_t) float_to_half_bits(__uint_as_float(f[2 * i])) |
               ((uint32_t) float_to_half_bits(__uint_as_float(f[2 * i + 1])) << 16);
    return v.ok ? make_uint4(w[0], w[1], w[2], w[3]) : make_uint4(0, 0, 0, 0);
}
template <bool T16>
__device__ __forceinline__ void gf_as_f32(const gf_raw & v, uint4 & lo, uint4 & hi) {
    if constexpr (T16) {
        const uint32_t u[4] = {v.r[0].x, v.r[0].y, v.r[0].z, v.r[0].w};
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            f[2 * i] = half_bits_to_float((uint16_t) (u[i] & 0xFFFF));
            f[2 * i + 1] = half_bits_to_float((uint16_t) (u[i] >> 16));
        }
        lo = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
        hi = make_uint4(__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]), __float_as_uint(f[7]));
    } else {
        lo = v.r[0];
        hi = v.r[1];
    }
    if (!v.ok) lo = hi = make_uint4(0, 0, 0, 0);
}

// a slab's pieces into LDS (sa, sb): f16 operands for an F16 src0 (the
// columns rounded to f16, as ggml-cpu converts src1 to the weight's
// vec_dot type), else f32; one or two 16-byte stores a piece (the padded
// rows stay 16-byte aligned)
template <bool F16, bool BF16, typename T, int PADE>
__device__ __forceinline__ void gf_stage_raw(const gf_raw & a, const gf_raw & b, int srow, int sk,
                                             T (*sa)[kGfBK + PADE], T (*sb)[kGfBK + PADE]) {
    if constexpr (F16) {
        *(uint4 *) &sa[srow][sk] = gf_as_f16<true>(a);
        *(uint4 *) &sb[srow][sk] = gf_as_f16<BF16>(b);
    } else {
        uint4 lo, hi;
        gf_as_f32<false>(a, lo, hi);
        *(uint4 *) &sa[srow][sk] = lo;
        *(uint4 *) &sa[srow][sk + 4] = hi;
        gf_as_f32<BF16>(b, lo, hi);
        *(uint4 *) &sb[srow][sk] = lo;
        *(uint4 *) &sb[srow][sk + 4] = hi;
    }
}

// X3 staging: eight f32 elements (zeros when not live) as bf16 hi (rounded to
// nearest even) and lo = bf16(x - hi): hi + lo carries ~17 of the 24 bits
typedef __bf16 gf_v8b __attribute__((ext_vector_type(8)));
__device__ __forceinline__ void gf_split8(const gf_raw & v, uint4 & hi, uint4 & lo) {
    const uint32_t f[8] = {v.r[0].x, v.r[0].y, v.r[0].z, v.r[0].w, v.r[1].x, v.r[1].y, v.r[1].z, v.r[1].w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t hb[2], lb[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float x = v.ok ? __uint_as_float(f[2 * i + e]) : 0.0f;
            const __bf16 xh = (__bf16) x;
            const __bf16 xl = (__bf16) (x - (float) xh);
            hb[e] = __builtin_bit_cast(uint16_t, xh);
            lb[e] = __builtin_bit_cast(uint16_t, xl);
        }
        h[i] = hb[0] | (hb[1] << 16);
        l[i] = lb[0] | (lb[1] << 16);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// The aligned form (16-byte aligned rows of both operands, K % 8 == 0):
// kGfDepth slabs in flight, slab j in register slot j % kGfDepth from its
// request until it is staged, and the LDS double-buffered -- step s
// multiplies slab s (buffer s % 2), stages slab s + 1 into the other buffer
// and requests slab s + 1 + kGfDepth into the slot it left; one barrier a
// step (a buffer is staged again only after the barrier that follows every
// wave's reads of it). Every load is unconditional (past K: clamped, zeros),
// so each step waits for its own slab only, not for all loads in flight. The
// steps are padded to a multiple of kGfDepth; the extra slabs are zeros.
template <bool F16, bool BF16>
__global__ __launch_bounds__(kGfThreads) void k_gemm_float_v(gemm_float_args g) {
    constexpr int PADE = F16 ? 8 : 4;
    using T = typename std::conditional<F16, _Float16, float>::type;
    __shared__ __align__(16) T sa[2][kGfBM][kGfBK + PADE];
    __shared__ __align__(16) T sb[2][kGfBN][kGfBK + PADE];
    const int tid = (int) threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t m0 = (int64_t) blockIdx.x * kGfBM;
    const int64_t n0 = (int64_t) blockIdx.y * kGfBN;
    // sibling products: this tile's product (rows, weights, output, bias)
    // (selects with constant indices: an index into the argument arrays
    // would put the arguments in scratch memory)
    static_assert(kGemmFloatMaxSubs == 2, "product selection below");
    if (g.nsub > 0) {
        int64_t base = 0, mend = g.sub_m0[1];
        const char * sa = g.sub_a[0];
        char * sd = g.sub_d[0];
        const float * sbias = g.sub_bias[0];
        if (m0 >= g.sub_m0[1]) {
            base = g.sub_m0[1], mend = g.sub_m0[2];
            sa = g.sub_a[1], sd = g.sub_d[1], sbias = g.sub_bias[1];
        }
        if (g.nsub >= 2 && m0 >= g.sub_m0[2]) {
            base = g.sub_m0[2], mend = g.sub_m0[3];
            sa = g.sub_a[2], sd = g.sub_d[2], sbias = g.sub_bias[2];
        }
        m0 -= base;
        g.M = mend - base;
        g.a = sa;
        g.d = sd;
        g.d_nb1 = g.M * 4;  // each product's output is contiguous
        g.epi.bias = sbias;
    }
    // split: blockIdx.z is the split (one batch); else the batch
    const int zb = g.splits > 1 ? 0 : (int) blockIdx.z, ks = g.splits > 1 ? (int) blockIdx.z : 0;
    const int i2 = zb % g.ne2, i3 = zb / g.ne2;
    const int64_t kb = (int64_t) ks * g.k_span;
    const int64_t K = g.splits > 1 ? (g.K - kb < g.k_span ? g.K - kb : g.k_span) : g.K;
    const char * abase = g.a + (int64_t) (i2 / g.r2) * g.a_nb2 + (int64_t) (i3 / g.r3) * g.a_nb3 + kb * (F16 ? 2 : 4);
    const char * bbase = g.b + (int64_t) i2 * g.b_nb2 + (int64_t) i3 * g.b_nb3 + kb * (BF16 ? 2 : 4);
    char * dbase = g.d + (int64_t) i2 * g.d_nb2 + (int64_t) i3 * g.d_nb3;
    const int srow = tid >> 2, sk = (tid & 3) * 8;
    const bool a_live = m0 + srow < g.M, b_live = n0 + srow < g.N;
    const char * arow = abase + (a_live ? m0 + srow : 0) * g.a_nb1;
    const char * brow = bbase + (b_live ? n0 + srow : 0) * g.b_nb1;
    const int64_t S = ((K + kGfBK - 1) / kGfBK + kGfDepth - 1) / kGfDepth * kGfDepth;
    gf_raw av[kGfDepth], bv[kGfDepth];
#pragma unroll
    for (int p = 0; p < kGfDepth; p++) {
        gf_load_raw<F16>(arow, (int64_t) p * kGfBK + sk, K, a_live, av[p]);
        gf_load_raw<BF16>(brow, (int64_t) p * kGfBK + sk, K, b_live, bv[p]);
    }
    gf_stage_raw<F16, BF16, T, PADE>(av[0], bv[0], srow, sk, sa[0], sb[0]);
    gf_load_raw<F16>(arow, (int64_t) kGfDepth * kGfBK + sk, K, a_live, av[0]);
    gf_load_raw<BF16>(brow, (int64_t) kGfDepth * kGfBK + sk, K, b_live, bv[0]);
    __syncthreads();
    // wave w: rows (w & 1) * 32 .. + 31, columns (w >> 1) * 32 .. + 31 of the tile
    const int wr = (wave & 1) * 32, wc = (wave >> 1) * 32;
    gf_v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = gf_v4f{0.f, 0.f, 0.f, 0.f};
    for (int64_t s0 = 0; s0 < S; s0 += kGfDepth) {
#pragma unroll
        for (int p = 0; p < kGfDepth; p++) {
            const int q = (p + 1) % kGfDepth;
            gf_mfma<F16, T, PADE>(sa[p & 1], sb[p & 1], wr, wc, lane, acc);
            gf_stage_raw<F16, BF16, T, PADE>(av[q], bv[q], srow, sk, sa[(p + 1) & 1], sb[(p + 1) & 1]);
            const int64_t kn = (s0 + p + 1 + kGfDepth) * kGfBK + sk;
            gf_load_raw<F16>(arow, kn, K, a_live, av[q]);
            gf_load_raw<BF16>(brow, kn, K, b_live, bv[q]);
            __syncthreads();
        }
    }
    gf_store(g, acc, m0, n0, wr, wc, lane, dbase, g.splits > 1 ? g.part + ks * g.M * g.N : nullptr);
}

// The aligned form for an F32 x F32 product at the default precision (x3):
// the same tiles, slabs in flight and barriers as k_gemm_float_v, the slab
// staged as bf16 hi / lo halves of each f32 element and each 16 x 16 block
// advanced by three bf16 MFMAs a 32-wide slab (lo hi, hi lo, then hi hi; the
// lo lo term, ~2^-16 of the product, dropped) instead of eight f32 ones.
template <int PADE>
__device__ __forceinline__ void gf_mfma_x3(const uint16_t (*sah)[kGfBK + PADE], const uint16_t (*sal)[kGfBK + PADE],
                                           const uint16_t (*sbh)[kGfBK + PADE], const uint16_t (*sbl)[kGfBK + PADE],
                                           int wr, int wc, int lane, gf_v4f (&acc)[2][2]) {
    const int r16 = lane & 15, kg = lane >> 4;
    gf_v8b bh[2], bl[2], ah[2], al[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        bh[j] = *(const gf_v8b *) &sbh[wc + 16 * j + r16][8 * kg];
        bl[j] = *(const gf_v8b *) &sbl[wc + 16 * j + r16][8 * kg];
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        ah[i] = *(const gf_v8b *) &sah[wr + 16 * i + r16][8 * kg];
        al[i] = *(const gf_v8b *) &sal[wr + 16 * i + r16][8 * kg];
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl[j], ah[i], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[j], al[i], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[j], ah[i], acc[i][j], 0, 0, 0);
        }
}

// ASPLIT: src0 already holds the hi / lo halves (im2col_args::split: each
// 8-element group of a row as 8 bf16 hi then 8 lo, the bytes its 8 f32 would
// take), staged as loaded
template <bool ASPLIT>
__global__ __launch_bounds__(kGfThreads) void k_gemm_float_x3(gemm_float_args g) {
    constexpr int PADE = 8;
    __shared__ __align__(16) uint16_t sah[2][kGfBM][kGfBK + PADE], sal[2][kGfBM][kGfBK + PADE];
    __shared__ __align__(16) uint16_t sbh[2][kGfBN][kGfBK + PADE], sbl[2][kGfBN][kGfBK + PADE];
    const int tid = (int) threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the tile: contiguous runs of tiles a XCD, a row tile's column tiles
    // adjacent (dispatched together, so the row tile's columns are fetched
    // into one L2)
    const int64_t t = (int64_t) (blockIdx.x % 8) * g.per_xcd + blockIdx.x / 8;
    if (t >= g.tiles) return;  // the grid's padding, before any barrier
    int64_t m0 = t / g.col_blocks * kGfBM;
    const int64_t n0 = t % g.col_blocks * kGfBN;
    static_assert(kGemmFloatMaxSubs == 2, "product selection below");
    if (g.nsub > 0) {
        int64_t base = 0, mend = g.sub_m0[1];
        const char * sa = g.sub_a[0];
        char * sd = g.sub_d[0];
        const float * sbias = g.sub_bias[0];
        if (m0 >= g.sub_m0[1]) {
            base = g.sub_m0[1], mend = g.sub_m0[2];
            sa = g.sub_a[1], sd = g.sub_d[1], sbias = g.sub_bias[1];
        }
        if (g.nsub >= 2 && m0 >= g.sub_m0[2]) {
            base = g.sub_m0[2], mend = g.sub_m0[3];
            sa = g.sub_a[2], sd = g.sub_d[2], sbias = g.sub_bias[2];
        }
        m0 -= base;
        g.M = mend - base;
        g.a = sa;
        g.d = sd;
        g.d_nb1 = g.M * 4;
        g.epi.bias = sbias;
    }
    const int zb = g.splits > 1 ? 0 : (int) blockIdx.z, ks = g.splits > 1 ? (int) blockIdx.z : 0;
    const int i2 = zb % g.ne2, i3 = zb / g.ne2;
    const int64_t kb = (int64_t) ks * g.k_span;
    const int64_t K = g.splits > 1 ? (g.K - kb < g.k_span ? g.K - kb : g.k_span) : g.K;
    const char * abase = g.a + (int64_t) (i2 / g.r2) * g.a_nb2 + (int64_t) (i3 / g.r3) * g.a_nb3 + kb * 4;
    const char * bbase = g.b + (int64_t) i2 * g.b_nb2 + (int64_t) i3 * g.b_nb3 + kb * 4;
    char * dbase = g.d + (int64_t) i2 * g.d_nb2 + (int64_t) i3 * g.d_nb3;
    const int srow = tid >> 2, sk = (tid & 3) * 8;
    const bool a_live = m0 + srow < g.M, b_live = n0 + srow < g.N;
    const char * arow = abase + (a_live ? m0 + srow : 0) * g.a_nb1;
    const char * brow = bbase + (b_live ? n0 + srow : 0) * g.b_nb1;
    const int64_t S = ((K + kGfBK - 1) / kGfBK + kGfDepth - 1) / kGfDepth * kGfDepth;
    auto stage = [&](const gf_raw & a, const gf_raw & b, int buf) {
        uint4 hi, lo;
        if constexpr (ASPLIT) {
            hi = a.ok ? a.r[0] : make_uint4(0, 0, 0, 0);
            lo = a.ok ? a.r[1] : make_uint4(0, 0, 0, 0);
        } else {
            gf_split8(a, hi, lo);
        }
        *(uint4 *) &sah[buf][srow][sk] = hi;
        *(uint4 *) &sal[buf][srow][sk] = lo;
        gf_split8(b, hi, lo);
        *(uint4 *) &sbh[buf][srow][sk] = hi;
        *(uint4 *) &sbl[buf][srow][sk] = lo;
    };
    gf_raw av[kGfDepth], bv[kGfDepth];
#pragma unroll
    for (int p = 0; p < kGfDepth; p++) {
        gf_load_raw<false>(arow, (int64_t) p * kGfBK + sk, K, a_live, av[p]);
        gf_load_raw<false>(brow, (int64_t) p * kGfBK + sk, K, b_live, bv[p]);
    }
    stage(av[0], bv[0], 0);
    gf_load_raw<false>(arow, (int64_t) kGfDepth * kGfBK + sk, K, a_live, av[0]);
    gf_load_raw<false>(brow, (int64_t) kGfDepth * kGfBK + sk, K, b_live, bv[0]);
    __syncthreads();
    const int wr = (wave & 1) * 32, wc = (wave >> 1) * 32;
    gf_v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = gf_v4f{0.f, 0.f, 0.f, 0.f};
    for (int64_t s0 = 0; s0 < S; s0 += kGfDepth) {
#pragma unroll
        for (int p = 0; p < kGfDepth; p++) {
            const int q = (p + 1) % kGfDepth;
            gf_mfma_x3<PADE>(sah[p & 1], sal[p & 1], sbh[p & 1], sbl[p & 1], wr, wc, lane, acc);
            stage(av[q], bv[q], (p + 1) & 1);
            const int64_t kn = (s0 + p + 1 + kGfDepth) * kGfBK + sk;
            gf_load_raw<false>(arow, kn, K, a_live, av[q]);
            gf_load_raw<false>(brow, kn, K, b_live, bv[q]);
            __syncthreads();
        }
    }
    gf_store(g, acc, m0, n0, wr, wc, lane, dbase, g.splits > 1 ? g.part + ks * g.M * g.N : nullptr);
}

// the splits' partials of each output added in split order, then the epilogue
__global__ __launch_bounds__(256) void k_gemm_float_reduce(gemm_float_args g) {
    const int64_t total = g.M * g.N;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        float o = g.part[i];
        for (int s = 1; s < g.splits; s++) o = o + g.part[s * total + i];
        gf_epi_store(g, o, i % g.M, i / g.M, g.d);
    }
}

// F16 = true: f16 operands (an F16 src0), else f32 operands
template <bool F16>
__global__ __launch_bounds__(kGfThreads) void k_gemm_float(gemm_float_args g) {
    constexpr int PADE = F16 ? 8 : 4;  // row padding of the LDS slabs, in elements
    using T = typename std::conditional<F16, _Float16, float>::type;
    __shared__ __align__(16) T sa[kGfBM][kGfBK + PADE];  // weight rows x k
    __shared__ __align__(16) T sb[kGfBN][kGfBK + PADE];  // columns x k
    const int tid = (int) threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t m0 = (int64_t) blockIdx.x * kGfBM, n0 = (int64_t) blockIdx.y * kGfBN;
    const int i2 = (int) blockIdx.z % g.ne2, i3 = (int) blockIdx.z / g.ne2;
    const char * abase = g.a + (int64_t) (i2 / g.r2) * g.a_nb2 + (int64_t) (i3 / g.r3) * g.a_nb3;
    const char * bbase = g.b + (int64_t) i2 * g.b_nb2 + (int64_t) i3 * g.b_nb3;
    char * dbase = g.d + (int64_t) i2 * g.d_nb2 + (int64_t) i3 * g.d_nb3;

    // staging: thread t loads row / column t / 4, elements 8 (t % 4) .. + 7 of the slab
    const int srow = tid >> 2, sk = (tid & 3) * 8;
    const bool a_live = m0 + srow < g.M, b_live = n0 + srow < g.N;
    const char * arow = abase + (a_live ? m0 + srow : 0) * g.a_nb1;
    const char * brow = bbase + (b_live ? n0 + srow : 0) * g.b_nb1;
    float av[8], bv[8];
    gf_load8(arow, sk, g.K, g.a_f16, g.a_vec, a_live, av);
    gf_load8(brow, sk, g.K, g.b_f16, g.b_vec, b_live, bv);

    // wave w: rows (w & 1) * 32 .. + 31, columns (w >> 1) * 32 .. + 31 of the tile
    const int wr = (wave & 1) * 32, wc = (wave >> 1) * 32;
    gf_v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = gf_v4f{0.f, 0.f, 0.f, 0.f};

    for (int64_t k0 = 0; k0 < g.K; k0 += kGfBK) {
        // the slab into LDS (columns rounded to f16 for an F16 src0, as
        // ggml-cpu converts src1 to the weight's vec_dot type)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sa[srow][sk + i] = (T) av[i];
            sb[srow][sk + i] = F16 ? (T) round_to_half(bv[i]) : (T) bv[i];
        }
        __syncthreads();
        // the next slab's loads, in flight under this slab's MFMAs
        if (k0 + kGfBK < g.K) {
            gf_load8(arow, k0 + kGfBK + sk, g.K, g.a_f16, g.a_vec, a_live, av);
            gf_load8(brow, k0 + kGfBK + sk, g.K, g.b_f16, g.b_vec, b_live, bv);
        }
        gf_mfma<F16, T, PADE>(sa, sb, wr, wc, lane, acc);
        __syncthreads();
    }

    gf_store(g, acc, m0, n0, wr, wc, lane, dbase);
}

namespace {

// one weight matrix for every batch and columns that continue across the
// batch dims (as in dst): the batches are more columns of one product
bool batches_are_columns(const tview & d, const tview & a, const tview & b) {
    return a.ne[2] == 1 && a.ne[3] == 1 && b.nb[2] == b.nb[1] * b.ne[1] && b.nb[3] == b.nb[2] * b.ne[2] &&
           d.nb[2] == d.nb[1] * d.ne[1] && d.nb[3] == d.nb[2] * d.ne[2];
}

}  // namespace

bool gemm_float_supported(const tview & d, const tview & a, int atype, const tview & b, int btype) {
    const int ea = atype == GGML_TYPE_F16 ? 2 : 4, eb = btype == GGML_TYPE_F16 ? 2 : 4;
    if (atype != GGML_TYPE_F16 && atype != GGML_TYPE_F32) return false;
    if (btype != GGML_TYPE_F16 && btype != GGML_TYPE_F32) return false;
    if (a.nb[0] != ea || b.nb[0] != eb || d.nb[0] != 4) return false;
    if (a.ne[0] != b.ne[0] || d.ne[0] != a.ne[1] || d.ne[1] != b.ne[1]) return false;
    if (d.ne[2] != b.ne[2] || d.ne[3] != b.ne[3] || d.ne[2] % a.ne[2] != 0 || d.ne[3] % a.ne[3] != 0) return false;
    const bool fold = batches_are_columns(d, a, b);
    const int64_t n = fold ? d.ne[1] * d.ne[2] * d.ne[3] : d.ne[1], batches = fold ? 1 : d.ne[2] * d.ne[3];
    // the matrix cores pay off once a 64 x 64 tile is mostly live, or a long
    // K makes even a narrow tile cheaper than a wave per output
    return d.ne[0] >= 16 && (n >= 16 || a.ne[0] >= 256) && batches <= 65535 && (n + kGfBN - 1) / kGfBN <= 65535;
}

namespace {

bool row_aligned(const tview & t) {
    return ((uintptr_t) t.data | (uintptr_t) t.nb[1] | (uintptr_t) t.nb[2] | (uintptr_t) t.nb[3]) % 16 == 0;
}

// the product with batches that continue the columns folded into one batch
void fold_batches(const tview & d, const tview & b, tview & d2, tview & b2) {
    d2 = d, b2 = b;
    d2.ne[1] = d.ne[1] * d.ne[2] * d.ne[3];
    b2.ne[1] = d2.ne[1];
    d2.ne[2] = d2.ne[3] = b2.ne[2] = b2.ne[3] = 1;
    d2.nb[2] = d2.nb[3] = d2.nb[1] * d2.ne[1];
    b2.nb[2] = b2.nb[3] = b2.nb[1] * b2.ne[1];
}

}  // namespace

// Split K only where the aligned form runs one batch on fewer 64 x 64 tiles
// than CUs: about two workgroups a CU, each with a whole number of kGfDepth
// slab groups (the 896 x 390 projections of a 30 s audio encode: 98 tiles,
// K = 896 in 4 splits, K = 3584 in 6).
int gemm_float_splits(const tview & d, const tview & a, int atype, const tview & b, int btype, int n_cu) {
    tview dd = d, bb = b;
    if (batches_are_columns(d, a, b)) fold_batches(d, b, dd, bb);
    if (dd.ne[2] * dd.ne[3] != 1) return 1;
    const int64_t K = a.ne[0];
    (void) atype, (void) btype;
    if (!row_aligned(a) || !row_aligned(bb) || K % 8 != 0) return 1;
    const int64_t tiles = (dd.ne[0] + kGfBM - 1) / kGfBM * ((dd.ne[1] + kGfBN - 1) / kGfBN);
    const int64_t slabs = (K + kGfBK - 1) / kGfBK;
    if (tiles >= n_cu || slabs < 2 * kGfDepth) return 1;
    const int64_t want = (2 * n_cu + tiles - 1) / tiles;
    const int64_t per = ((slabs + want - 1) / want + kGfDepth - 1) / kGfDepth * kGfDepth;
    return (int) std::min<int64_t>((slabs + per - 1) / per, 16);
}

bool gemm_float_siblings_ok(const tview & d, const tview & a, const tview & b) {
    return d.ne[2] * d.ne[3] == 1 && a.ne[2] * a.ne[3] == 1 && row_aligned(a) && row_aligned(b) && a.ne[0] % 8 == 0 &&
           d.ne[0] % kGfBM == 0;
}

size_t gemm_float_split_bytes(const tview & d, int splits) {
    return splits > 1 ? (size_t) splits * d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3] * sizeof(float) : 0;
}

bool gemm_float_x3_aligned(const tview & a, const tview & b) {
    return row_aligned(a) && row_aligned(b) && a.ne[0] % 8 == 0;
}

void launch_gemm_float(const tview & d, const tview & a, int atype, const tview & b, int btype, hipStream_t s,
                       const gemm_float_epi & epi, int splits, float * part, const gemm_float_sub * subs, int nsub,
                       bool x3, bool a_split) {
    if (a_split && (!x3 || atype != GGML_TYPE_F32 || btype != GGML_TYPE_F32 || nsub > 0 ||
                    !gemm_float_x3_aligned(a, b))) {
        note_hip_error(hipErrorInvalidValue);  // only the aligned bf16 form reads the split layout
        return;
    }
    if (batches_are_columns(d, a, b) && d.ne[2] * d.ne[3] > 1) {
        tview d2, b2;
        fold_batches(d, b, d2, b2);
        launch_gemm_float(d2, a, atype, b2, btype, s, epi, splits, part, subs, nsub, x3, a_split);
        return;
    }
    gemm_float_args g{};
    g.epi = epi;
    g.a = a.data;
    g.a_nb1 = a.nb[1];
    g.a_nb2 = a.nb[2];
    g.a_nb3 = a.nb[3];
    g.a_f16 = atype == GGML_TYPE_F16;
    g.b = b.data;
    g.b_nb1 = b.nb[1];
    g.b_nb2 = b.nb[2];
    g.b_nb3 = b.nb[3];
    g.b_f16 = btype == GGML_TYPE_F16;
    g.d = d.data;
    g.d_nb1 = d.nb[1];
    g.d_nb2 = d.nb[2];
    g.d_nb3 = d.nb[3];
    g.M = d.ne[0];
    g.N = d.ne[1];
    g.K = a.ne[0];
    g.ne2 = (int) d.ne[2];
    g.ne3 = (int) d.ne[3];
    g.r2 = (int) (d.ne[2] / a.ne[2]);
    g.r3 = (int) (d.ne[3] / a.ne[3]);
    // 16-byte vector loads where every row start is 16-byte aligned
    g.a_vec = row_aligned(a);
    g.b_vec = row_aligned(b);
    g.splits = 1;
    g.k_span = g.K;
    g.part = nullptr;
    g.nsub = 0;
    const bool aligned = g.a_vec && g.b_vec && g.K % 8 == 0;
    int64_t m_all = g.M;
    if (nsub > 0 && aligned && g.ne2 * g.ne3 == 1 && g.M % kGfBM == 0 && nsub <= kGemmFloatMaxSubs) {
        // sibling products: their row ranges follow the first product's
        g.nsub = nsub;
        g.sub_m0[0] = 0;
        g.sub_a[0] = g.a;
        g.sub_d[0] = g.d;
        g.sub_bias[0] = epi.bias;
        for (int i = 0; i < nsub; i++) {
            g.sub_m0[i + 1] = m_all;
            g.sub_a[i + 1] = subs[i].a;
            g.sub_d[i + 1] = subs[i].d;
            g.sub_bias[i + 1] = subs[i].bias;
            m_all += subs[i].M;
        }
        g.sub_m0[nsub + 1] = m_all;
        splits = 1;
    } else if (nsub > 0) {
        // not joinable here: each product on its own
        launch_gemm_float(d, a, atype, b, btype, s, epi, splits, part, nullptr, 0, x3);
        for (int i = 0; i < nsub; i++) {
            tview ai = a, di = d;
            ai.data = (char *) subs[i].a;
            ai.ne[1] = subs[i].M;
            di.data = subs[i].d;
            di.ne[0] = subs[i].M;
            di.nb[1] = di.nb[0] * subs[i].M;
            di.nb[2] = di.nb[3] = di.nb[1] * di.ne[1];
            gemm_float_epi ei;
            ei.bias = subs[i].bias;
            launch_gemm_float(di, ai, atype, b, btype, s, ei, 1, nullptr, nullptr, 0, x3);
        }
        return;
    }
    if (splits > 1 && part && aligned && g.ne2 * g.ne3 == 1) {
        // every split but the last takes k_span (whole kGfDepth slab groups)
        const int64_t slabs = (g.K + kGfBK - 1) / kGfBK;
        const int64_t per = ((slabs + splits - 1) / splits + kGfDepth - 1) / kGfDepth * kGfDepth;
        g.k_span = per * kGfBK;
        g.splits = (int) ((slabs + per - 1) / per);
        g.part = part;
    }
    const dim3 grid((unsigned) ((m_all + kGfBM - 1) / kGfBM), (unsigned) ((g.N + kGfBN - 1) / kGfBN),
                    (unsigned) (g.splits > 1 ? g.splits : g.ne2 * g.ne3));
    if (aligned) {
        if (g.a_f16 && g.b_f16) hipLaunchKernelGGL((k_gemm_float_v<true, true>), grid, dim3(kGfThreads), 0, s, g);
        else if (g.a_f16) hipLaunchKernelGGL((k_gemm_float_v<true, false>), grid, dim3(kGfThreads), 0, s, g);
        else if (g.b_f16) hipLaunchKernelGGL((k_gemm_float_v<false, true>), grid, dim3(kGfThreads), 0, s, g);
        else if (x3) {
            // one dim of tiles, dealt to the XCDs in contiguous runs
            g.tiles = (int64_t) grid.x * grid.y;
            g.col_blocks = grid.y;
            g.per_xcd = (g.tiles + 7) / 8;
            const dim3 g1((unsigned) (g.per_xcd * 8), 1u, grid.z);
            if (a_split) hipLaunchKernelGGL(k_gemm_float_x3<true>, g1, dim3(kGfThreads), 0, s, g);
            else hipLaunchKernelGGL(k_gemm_float_x3<false>, g1, dim3(kGfThreads), 0, s, g);
        }
        else hipLaunchKernelGGL((k_gemm_float_v<false, false>), grid, dim3(kGfThreads), 0, s, g);
        if (g.splits > 1) {
            const int64_t blocks = std::min<int64_t>((g.M * g.N + 255) / 256, 4096);
            hipLaunchKernelGGL(k_gemm_float_reduce, dim3((unsigned) blocks), dim3(256), 0, s, g);
        }
    } else if (g.a_f16) hipLaunchKernelGGL(k_gemm_float<true>, grid, dim3(kGfThreads), 0, s, g);
    else hipLaunchKernelGGL(k_gemm_float<false>, grid, dim3(kGfThreads), 0, s, g);
    note_hip_error(hipGetLastError());
}

}  // namespace mi355x

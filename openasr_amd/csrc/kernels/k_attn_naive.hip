// k_attn_naive.hip -- the unfused attention chain of the discrete-GPU prefill
// as one launch. For prefill chunks of more than two queries over a span of
// more than 32 positions the host builds llm_naive_masked_attention
// (crates/openasr-core/src/nn/decoder.rs:2154-2200; the choice:
// models/qwen/llm_transformer.rs:7864-7877) over K/V that expand_attention_kv
// has REPEAT-expanded to the query heads (nn/decoder.rs:1799-1841):
//   S = MUL_MAT(K, Q), P = SOFT_MAX_EXT(S, mask, scale),
//   C = MUL_MAT(CONT(TRANSPOSE(V)), P), O = CONT(PERMUTE(C, 0, 2, 1, 3)).
// The launch reads K and V where the caches hold them (query head h reads kv
// head h / (Hq / Hkv): the REPEAT and the V transpose are never
// materialised), keeps S and P per workgroup in scratch, and writes O. Its
// arithmetic is the ops' in a fixed order:
//   score  one f32 fma chain over the dims in order from +0, then
//          s * scale + mask (two roundings); a masked position is -inf;
//   softmax M = max s; e = exp(s - M) (the deterministic exp); the f64 sum
//          of each 64-position chunk's e by a pairwise tree over the chunk
//          (positions past the span add +0), then of the chunk sums in
//          chunk order from 0; P = e * (float) (1 / sum);
//   context out[d] = fma(P[t], v[t][d], out[d]) over the positions in
//          order from +0, terms with P = 0 skipped (the sum is never -0, so
//          such a term would leave it unchanged).
// With GGML_PREC_F32 on a product (the host sets it on CUDA/HIP backends,
// ggml_runtime/cpu_graph.rs:157-165, 202-228) its f32 operand (Q, P) stays
// f32; without it, it is rounded to f16 as ggml-cpu converts src1 to an F16
// src0's vec_dot type.
//
// Work: a workgroup owns the query heads of one kv head for a tile of
// queries (up to 16 rows) of one sequence and walks the span in 64-position
// chunks: (1) stages the chunk's K rows in LDS (16-byte pieces swizzled so
// that lane p reading row p hits distinct banks) and computes the rows'
// scores, lane = position; (2) exponentials and the per-chunk tree sums in
// registers (butterfly over the wave); (3) stages each chunk's V rows and P
// and runs the context chains, one thread per row and eight dims. Chunks
// masked for every row of the workgroup are skipped.
#include <cmath>

#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

namespace {

constexpr int kNaRows = 16;
constexpr int kNaChunk = 64;
constexpr int kNaThreads = 256;

__device__ __forceinline__ void unpack8(const uint4 w, float (&f)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = half_bits_to_float((uint16_t) (u[i] & 0xFFFF));
        f[2 * i + 1] = half_bits_to_float((uint16_t) (u[i] >> 16));
    }
}

// pairwise sum over the 64 lanes: level k adds the lane groups of 2^k
// consecutive lanes two by two (a + b == b + a, so every lane ends with the
// same tree's value)
__device__ __forceinline__ double tree_sum64(double v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = v + __shfl_xor(v, m);
    return v;
}

}  // namespace

template <int D>
__global__ __launch_bounds__(kNaThreads) void k_attn_naive(naive_attn_args a) {
    constexpr int P16 = D / 8;  // 16-byte pieces of a K/V row
    __shared__ __align__(16) float s_q[kNaRows][D];
    __shared__ __align__(16) uint16_t s_kv[kNaChunk][D];
    __shared__ __align__(16) float s_p[kNaRows][kNaChunk];
    __shared__ float s_max[kNaRows], s_inv[kNaRows];
    __shared__ unsigned char s_live[kNaMaxChunks];

    const int tid = (int) threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = a.hq / a.hkv, qt = a.qt, R = g * qt;
    const int kvh = (int) blockIdx.y, seq = (int) blockIdx.z;
    const int i0 = (int) blockIdx.x * qt;
    const int n_kv = a.n_kv, nch = (n_kv + kNaChunk - 1) / kNaChunk, tp = nch * kNaChunk;
    float * work = a.work + ((size_t) (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * kNaRows * tp;
    const char * kb = a.k + (int64_t) kvh * a.k_nb2 + (int64_t) (seq / a.rk3) * a.k_nb3;
    const char * vb = a.v + (int64_t) kvh * a.v_nb2 + (int64_t) (seq / a.rk3) * a.v_nb3;

    // row r: query head kvh * g + r / qt, query i0 + r % qt
    auto row_head = [&](int r) { return kvh * g + r / qt; };
    auto row_query = [&](int r) { return i0 + r % qt; };
    auto row_live = [&](int r) { return r < R && row_query(r) < a.n_q; };
    auto mask_row = [&](int r) -> const uint16_t * {
        return (const uint16_t *) (a.mask + (int64_t) row_query(r) * a.m_nb1 +
                                   (int64_t) (row_head(r) % a.m_ne2) * a.m_nb2 + (int64_t) (seq % a.m_ne3) * a.m_nb3);
    };

    for (int e = tid; e < kNaRows * D; e += kNaThreads) {
        const int r = e / D, d = e % D;
        float v = 0.0f;
        if (row_live(r)) {
            v = ((const float *) (a.q + (int64_t) row_query(r) * a.q_nb1 + (int64_t) row_head(r) * a.q_nb2 +
                                  (int64_t) seq * a.q_nb3))[d];
            if (!a.q_f32) v = round_to_half(v);
        }
        s_q[r][d] = v;
    }

    // (1) scores: wave w owns rows w, w + 4, w + 8, w + 12; lane = position
    float rmax[4];
#pragma unroll
    for (int j = 0; j < 4; j++) rmax[j] = -INFINITY;
    for (int c = 0; c < nch; c++) {
        const int t = c * kNaChunk + lane;
        float mv[4];
        int any = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = wave + 4 * j;
            mv[j] = -INFINITY;
            if (row_live(r) && t < n_kv) mv[j] = a.mask ? half_bits_to_float(mask_row(r)[t]) : 0.0f;
            any |= mv[j] != -INFINITY;
        }
        any = __syncthreads_or(any);
        if (tid == 0) s_live[c] = (unsigned char) (any != 0);
        if (!any) continue;
        for (int e = tid; e < kNaChunk * P16; e += kNaThreads) {
            const int p = e / P16, j = e % P16;
            const int tt = c * kNaChunk + p;
            uint4 w = make_uint4(0, 0, 0, 0);
            if (tt < n_kv) w = *(const uint4 *) (kb + (int64_t) tt * a.k_nb1 + 16 * j);
            *(uint4 *) &s_kv[p][8 * (j ^ (p % P16))] = w;
        }
        __syncthreads();
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int jp = 0; jp < P16; jp++) {
            float kf[8];
            unpack8(*(const uint4 *) &s_kv[lane][8 * (jp ^ (lane % P16))], kf);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = wave + 4 * j;
                if (r >= R) continue;  // uniform in the wave
                const float4 qa = *(const float4 *) &s_q[r][8 * jp];
                const float4 qb = *(const float4 *) &s_q[r][8 * jp + 4];
                float x = acc[j];
                x = fmaf(kf[0], qa.x, x);
                x = fmaf(kf[1], qa.y, x);
                x = fmaf(kf[2], qa.z, x);
                x = fmaf(kf[3], qa.w, x);
                x = fmaf(kf[4], qb.x, x);
                x = fmaf(kf[5], qb.y, x);
                x = fmaf(kf[6], qb.z, x);
                x = fmaf(kf[7], qb.w, x);
                acc[j] = x;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = wave + 4 * j;
            if (!row_live(r) || t >= n_kv) continue;
            const float s = mv[j] == -INFINITY ? -INFINITY : acc[j] * a.scale + mv[j];
            work[(size_t) r * tp + t] = s;
            rmax[j] = fmaxf(rmax[j], s);
        }
        __syncthreads();  // the next chunk's K replaces this one's in LDS
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = wave + 4 * j;
        const float m = wave_max(rmax[j]);
        if (lane == 0 && r < kNaRows) s_max[r] = m;
    }
    __syncthreads();

    // (2) e = exp(s - M) in place (each lane rewrites what it wrote) and the
    // sum: per chunk the pairwise tree, the chunk sums in order
    double total[4] = {0.0, 0.0, 0.0, 0.0};
    for (int c = 0; c < nch; c++) {
        if (!s_live[c]) continue;
        const int t = c * kNaChunk + lane;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = wave + 4 * j;
            if (r >= R) continue;  // uniform in the wave
            float e = 0.0f;
            if (row_live(r) && t < n_kv) {
                float* wp = work + (size_t) r * tp + t;
                e = expf_det(*wp - s_max[r]);
                *wp = e;
            }
            total[j] = total[j] + tree_sum64((double) e);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = wave + 4 * j;
        if (lane == 0 && r < kNaRows) s_inv[r] = (float) (1.0 / total[j]);
    }
    __threadfence_block();
    __syncthreads();

    // (3) context: thread (row tid / P16, dims 8 (tid % P16) .. + 7)
    const int r3 = tid / P16, dg = tid % P16;
    float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = 0; c < nch; c++) {
        if (!s_live[c]) continue;
        for (int e = tid; e < kNaChunk * P16; e += kNaThreads) {
            const int p = e / P16, j = e % P16;
            const int tt = c * kNaChunk + p;
            uint4 w = make_uint4(0, 0, 0, 0);
            if (tt < n_kv) w = *(const uint4 *) (vb + (int64_t) tt * a.v_nb1 + 16 * j);
            *(uint4 *) &s_kv[p][8 * j] = w;
        }
        for (int e = tid; e < kNaRows * kNaChunk; e += kNaThreads) {
            const int r = e / kNaChunk, j = e % kNaChunk;
            const int tt = c * kNaChunk + j;
            float pv = 0.0f;
            if (row_live(r) && tt < n_kv) {
                pv = work[(size_t) r * tp + tt] * s_inv[r];
                // P is the f32 product, then rounded to f16: the empty asm
                // keeps the multiply and the conversion from being folded
                // into one mixed-precision fma (v_fma_mixlo_f16), which
                // would round the exact product to f16 once
                asm volatile("" : "+v"(pv));
                if (!a.p_f32) pv = round_to_half(pv);
            }
            s_p[r][j] = pv;
        }
        __syncthreads();
        if (r3 < kNaRows && r3 < R) {
            for (int j = 0; j < kNaChunk; j++) {
                const float p = s_p[r3][j];
                float vf[8];
                unpack8(*(const uint4 *) &s_kv[j][8 * dg], vf);
#pragma unroll
                for (int k = 0; k < 8; k++) o[k] = p != 0.0f ? fmaf(p, vf[k], o[k]) : o[k];
            }
        }
        __syncthreads();
    }
    if (r3 < kNaRows && row_live(r3)) {
        // a row with no live position: the ops give NaN (exp(-inf - -inf))
        const bool dead = s_max[r3] == -INFINITY;
        float * op = a.out + (((int64_t) seq * a.n_q + row_query(r3)) * a.hq + row_head(r3)) * D + 8 * dg;
#pragma unroll
        for (int k = 0; k < 8; k++) op[k] = dead ? __builtin_nanf("") : o[k];
    }
}

bool attn_naive_supported(int d, int hq, int hkv, int64_t n_kv) {
    return (d == 64 || d == 128) && hkv > 0 && hq % hkv == 0 && hq / hkv <= kNaRows && n_kv > 0 &&
           n_kv <= (int64_t) kNaMaxChunks * kNaChunk;
}

static int naive_qt(const naive_attn_args & a) { return kNaRows / (a.hq / a.hkv); }

size_t attn_naive_scratch_bytes(const naive_attn_args & a) {
    const int qt = naive_qt(a);
    const int64_t tiles = (a.n_q + qt - 1) / qt;
    const int64_t tp = (a.n_kv + kNaChunk - 1) / kNaChunk * kNaChunk;
    return (size_t) (tiles * a.hkv * a.n_seq) * kNaRows * tp * sizeof(float);
}

void launch_attn_naive(const naive_attn_args & args, float * work, hipStream_t s) {
    naive_attn_args a = args;
    a.qt = naive_qt(a);
    a.work = work;
    const dim3 grid((unsigned) ((a.n_q + a.qt - 1) / a.qt), (unsigned) a.hkv, (unsigned) a.n_seq);
    if (a.d == 128) hipLaunchKernelGGL(k_attn_naive<128>, grid, dim3(kNaThreads), 0, s, a);
    else hipLaunchKernelGGL(k_attn_naive<64>, grid, dim3(kNaThreads), 0, s, a);
    note_hip_error(hipGetLastError());
}

}  // namespace mi355x

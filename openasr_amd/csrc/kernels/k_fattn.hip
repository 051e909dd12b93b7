// k_fattn.hip -- GGML_OP_FLASH_ATTN_EXT over an f16 KV cache with grouped
// query heads (call site crates/openasr-core/src/ggml_runtime/cpu_graph.rs:
// 4144-4215; graph built in crates/openasr-core/src/nn/decoder.rs:2031-2105).
//
// Split-KV, two passes, order-independent sums:
//   scores   one workgroup per (KV chunk, kv head, sequence, query tile)
//            computes s = (q . k) * scale + mask for every query head that
//            shares the kv head (K is read once per kv head) and the per-chunk
//            row maxima. A chunk whose mask is -inf for every row of the tile
//            is skipped without touching K (the graph always passes the full
//            fixed span, nn/decoder.rs:1295-1301).
//   accum    the same grid takes the row's global max M, forms
//            p = exp(s - M), and accumulates sum(p) and sum(p * V) in f64
//            per chunk (V read once per kv head; masked positions skipped).
//   combine  sums the chunk partials in f64 and divides once.
// Q is rounded to f16 before the dot with f16 K, as ggml-cpu does; products
// of two halves are exact in f32 and every sum is carried in f64, so the
// result does not depend on how positions are split across lanes, waves or
// chunks -- the CPU reference computes the same value sequentially.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

constexpr int kFaThreads = 256;
constexpr int kFaMaxChunk = 256;
constexpr int kFaRows = 8;  // query rows (heads x positions) per workgroup

struct fa_tile {
    int kvh, seq, g, q0, nrows, c0, clen, kv_seq;
};

__device__ __forceinline__ fa_tile fa_tile_of(const fattn_args & a) {
    fa_tile t;
    t.kvh = blockIdx.y % a.hkv;
    t.seq = blockIdx.y / a.hkv;
    t.g = a.hq / a.hkv;
    const int tq_per_tile = kFaRows / t.g;
    t.q0 = blockIdx.z * tq_per_tile;
    t.nrows = min(tq_per_tile, a.n_q - t.q0) * t.g;
    t.c0 = blockIdx.x * a.chunk;
    t.clen = min(a.chunk, a.n_kv - t.c0);
    t.kv_seq = t.seq / a.rk3;
    return t;
}

// output row index of tile row r (= query position q0 + r / g, head kvh*g + r % g)
__device__ __forceinline__ int64_t fa_orow(const fattn_args & a, const fa_tile & t, int r) {
    return ((int64_t) t.seq * a.n_q + t.q0 + r / t.g) * a.hq + (int64_t) t.kvh * t.g + r % t.g;
}

__device__ __forceinline__ const uint16_t * fa_mask_row(const fattn_args & a, const fa_tile & t, int tq) {
    return (const uint16_t *) (a.mask + (int64_t) (t.q0 + tq) * a.m_nb1 + (int64_t) (t.seq % a.m_ne3) * a.m_nb3);
}

__device__ __forceinline__ double dsum_group(double v, int width) {
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, width);
    return v;
}

template <int D>
__global__ __launch_bounds__(kFaThreads) void k_fattn_scores(fattn_args a, float * __restrict__ S,
                                                             float * __restrict__ cmax) {
    constexpr int LPP = D / 8;     // lanes per key position
    constexpr int PPW = 64 / LPP;  // positions per wave per step
    __shared__ float s_max[4][kFaRows];
    __shared__ int s_any;
    const fa_tile t = fa_tile_of(a);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int chunk = blockIdx.x;

    if (tid == 0) s_any = a.mask ? 0 : 1;
    __syncthreads();
    if (a.mask) {
        int any = 0;
        for (int idx = tid; idx < t.clen * (t.nrows / t.g); idx += kFaThreads) {
            if (fa_mask_row(a, t, idx / t.clen)[t.c0 + idx % t.clen] != 0xFC00) any = 1;
        }
        if (any) s_any = 1;
    }
    __syncthreads();
    if (!s_any) {
        if (tid < t.nrows) cmax[fa_orow(a, t, tid) * a.n_chunks + chunk] = -INFINITY;
        return;
    }

    const char * kbase = a.k + (int64_t) t.kvh * a.k_nb2 + (int64_t) t.kv_seq * a.k_nb3;
    const int dl = (lane % LPP) * 8;
    float qr[kFaRows][8];
#pragma unroll
    for (int r = 0; r < kFaRows; r++) {
        const bool ok = r < t.nrows;
        const float * qp = (const float *) (a.q + (int64_t) (t.q0 + (ok ? r / t.g : 0)) * a.q_nb1 +
                                            (int64_t) (t.kvh * t.g + r % t.g) * a.q_nb2 + (int64_t) t.seq * a.q_nb3);
#pragma unroll
        for (int i = 0; i < 8; i++) qr[r][i] = ok ? round_to_half(qp[dl + i]) : 0.0f;
    }
    float rmax[kFaRows];
#pragma unroll
    for (int r = 0; r < kFaRows; r++) rmax[r] = -INFINITY;
    for (int base = wave * PPW; base < t.clen; base += 4 * PPW) {
        const int p = base + lane / LPP;
        const bool valid = p < t.clen;
        float kf[8];
        if (valid) {
            const uint4 kv4 = *(const uint4 *) (kbase + (int64_t) (t.c0 + p) * a.k_nb1 + dl * 2);
            const uint32_t w[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kf[2 * i] = half_bits_to_float((uint16_t) (w[i] & 0xFFFF));
                kf[2 * i + 1] = half_bits_to_float((uint16_t) (w[i] >> 16));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) kf[i] = 0.0f;
        }
#pragma unroll
        for (int r = 0; r < kFaRows; r++) {
            if (r >= t.nrows) break;
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < 8; i++) acc += (double) (kf[i] * qr[r][i]);  // exact products
            acc = dsum_group(acc, LPP);
            if (valid && (lane % LPP) == 0) {
                const float mv = a.mask ? half_bits_to_float(fa_mask_row(a, t, r / t.g)[t.c0 + p]) : 0.0f;
                // a masked position is skipped outright, as ggml-cpu does, so
                // whatever an unwritten cache slot holds never reaches the sums
                const float s = mv == -INFINITY ? -INFINITY : (float) acc * a.scale + mv;
                S[fa_orow(a, t, r) * a.n_kv + t.c0 + p] = s;
                rmax[r] = fmaxf(rmax[r], s);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kFaRows; r++) {
        const float m = wave_max(rmax[r]);
        if (lane == 0) s_max[wave][r] = m;
    }
    __syncthreads();
    if (tid < t.nrows) {
        const float m = fmaxf(fmaxf(s_max[0][tid], s_max[1][tid]), fmaxf(s_max[2][tid], s_max[3][tid]));
        cmax[fa_orow(a, t, tid) * a.n_chunks + chunk] = m;
    }
}

template <int D>
__global__ __launch_bounds__(kFaThreads) void k_fattn_accum(fattn_args a, const float * __restrict__ S,
                                                            const float * __restrict__ cmax,
                                                            double * __restrict__ part_acc,
                                                            double * __restrict__ part_l) {
    constexpr int DPL = D / 64;                // dims per lane
    constexpr int PG = kFaThreads / (D / DPL);  // position groups
    __shared__ float s_p[kFaRows][kFaMaxChunk];
    __shared__ float s_M[kFaRows];
    __shared__ int s_live[kFaRows];
    __shared__ double s_red[PG][kFaRows][D];
    __shared__ double s_l[kFaRows];
    const fa_tile t = fa_tile_of(a);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int chunk = blockIdx.x;

    if (tid < kFaRows) {
        float M = -INFINITY;
        int live = 0;
        if (tid < t.nrows) {
            const float * cm = cmax + fa_orow(a, t, tid) * a.n_chunks;
            for (int i = 0; i < a.n_chunks; i++) M = fmaxf(M, cm[i]);
            live = cm[chunk] != -INFINITY;
        }
        s_M[tid] = M;
        s_live[tid] = live;
    }
    __syncthreads();
    int any = 0;
    for (int r = 0; r < t.nrows; r++) any |= s_live[r];
    if (!any) {
        for (int idx = tid; idx < t.nrows * (D + 1); idx += kFaThreads) {
            const int r = idx / (D + 1), d = idx % (D + 1);
            const int64_t o = fa_orow(a, t, r) * a.n_chunks + chunk;
            if (d < D) part_acc[o * D + d] = 0.0;
            else part_l[o] = 0.0;
        }
        return;
    }
    // p = exp(s - M) with the row's global max, one wave per row
    for (int r = wave; r < t.nrows; r += 4) {
        const float * sr = S + fa_orow(a, t, r) * a.n_kv + t.c0;
        double l = 0.0;
        for (int p = lane; p < t.clen; p += 64) {
            float e = 0.0f;
            if (s_live[r]) {
                const float s = sr[p];
                e = s == -INFINITY ? 0.0f : expf_det(s - s_M[r]);
            }
            s_p[r][p] = e;
            l += (double) e;
        }
        l = dsum_group(l, 64);
        if (lane == 0) s_l[r] = l;
    }
    __syncthreads();
    const char * vbase = a.v + (int64_t) t.kvh * a.v_nb2 + (int64_t) t.kv_seq * a.v_nb3;
    const int dslot = tid % (D / DPL);
    const int pg = tid / (D / DPL);
    double acc[kFaRows][DPL];
#pragma unroll
    for (int r = 0; r < kFaRows; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) acc[r][i] = 0.0;
    for (int p = pg; p < t.clen; p += PG) {
        bool need = false;
#pragma unroll
        for (int r = 0; r < kFaRows; r++) need |= (r < t.nrows) && s_p[r][p] != 0.0f;
        if (!need) continue;
        const char * vp = vbase + (int64_t) (t.c0 + p) * a.v_nb1 + dslot * DPL * 2;
        float vf[DPL];
        if (DPL == 2) {
            const uint32_t w = *(const uint32_t *) vp;
            vf[0] = half_bits_to_float((uint16_t) (w & 0xFFFF));
            vf[DPL - 1] = half_bits_to_float((uint16_t) (w >> 16));
        } else {
            vf[0] = half_bits_to_float(*(const uint16_t *) vp);
        }
#pragma unroll
        for (int r = 0; r < kFaRows; r++) {
            if (r >= t.nrows) break;
            const float pr = s_p[r][p];
            if (pr == 0.0f) continue;
#pragma unroll
            for (int i = 0; i < DPL; i++) acc[r][i] += (double) pr * (double) vf[i];  // exact products
        }
    }
#pragma unroll
    for (int r = 0; r < kFaRows; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) s_red[pg][r][dslot * DPL + i] = acc[r][i];
    __syncthreads();
    for (int idx = tid; idx < t.nrows * D; idx += kFaThreads) {
        const int r = idx / D, d = idx % D;
        double v = 0.0;
#pragma unroll
        for (int q = 0; q < PG; q++) v += s_red[q][r][d];
        const int64_t o = fa_orow(a, t, r) * a.n_chunks + chunk;
        part_acc[o * D + d] = v;
        if (d == 0) part_l[o] = s_l[r];
    }
}

template <int D>
__global__ __launch_bounds__(D) void k_fattn_combine(const double * __restrict__ part_acc,
                                                     const double * __restrict__ part_l, int n_chunks,
                                                     float * __restrict__ out) {
    const int64_t orow = blockIdx.x;
    const int d = threadIdx.x;
    double L = 0.0, acc = 0.0;
    for (int i = 0; i < n_chunks; i++) {
        L += part_l[orow * n_chunks + i];
        acc += part_acc[(orow * n_chunks + i) * D + d];
    }
    out[orow * D + d] = L == 0.0 ? 0.0f : (float) (acc / L);
}

static int64_t fa_rows(const fattn_args & a) { return (int64_t) a.n_seq * a.n_q * a.hq; }

size_t fattn_scratch_bytes(const fattn_args & a) {
    const int64_t rows = fa_rows(a);
    return (size_t) rows * a.n_kv * sizeof(float) + (size_t) rows * a.n_chunks * sizeof(float) +
           (size_t) rows * a.n_chunks * (a.d + 1) * sizeof(double) + 1024;
}

void fattn_plan(fattn_args & a, int n_cu) {
    const int g = a.hq / a.hkv;
    const int tq_per_tile = kFaRows / g;
    a.q_tiles = (a.n_q + tq_per_tile - 1) / tq_per_tile;
    const int64_t groups = (int64_t) a.hkv * a.n_seq * a.q_tiles;
    int chunk = kFaMaxChunk;
    while (chunk > 32 && groups * ((a.n_kv + chunk - 1) / chunk) < 2LL * n_cu) chunk >>= 1;
    a.chunk = chunk;
    a.n_chunks = (a.n_kv + chunk - 1) / chunk;
}

bool fattn_supported(int d, int hq, int hkv) {
    if (d != 64 && d != 128) return false;
    if (hkv <= 0 || hq % hkv != 0) return false;
    return kFaRows % (hq / hkv) == 0;
}

void launch_fattn(const fattn_args & a, float * scratch, float * out, hipStream_t stream) {
    const int64_t rows = fa_rows(a);
    float * S = scratch;
    float * cmax = S + rows * a.n_kv;
    char * p = (char *) (cmax + rows * a.n_chunks);
    p = (char *) (((uintptr_t) p + 255) & ~(uintptr_t) 255);
    double * part_acc = (double *) p;
    double * part_l = part_acc + rows * a.n_chunks * a.d;
    const dim3 grid((unsigned) a.n_chunks, (unsigned) (a.hkv * a.n_seq), (unsigned) a.q_tiles);
    if (a.d == 128) {
        hipLaunchKernelGGL(k_fattn_scores<128>, grid, dim3(kFaThreads), 0, stream, a, S, cmax);
        hipLaunchKernelGGL(k_fattn_accum<128>, grid, dim3(kFaThreads), 0, stream, a, S, cmax, part_acc, part_l);
        hipLaunchKernelGGL(k_fattn_combine<128>, dim3((unsigned) rows), dim3(128), 0, stream, part_acc, part_l,
                           a.n_chunks, out);
    } else {
        hipLaunchKernelGGL(k_fattn_scores<64>, grid, dim3(kFaThreads), 0, stream, a, S, cmax);
        hipLaunchKernelGGL(k_fattn_accum<64>, grid, dim3(kFaThreads), 0, stream, a, S, cmax, part_acc, part_l);
        hipLaunchKernelGGL(k_fattn_combine<64>, dim3((unsigned) rows), dim3(64), 0, stream, part_acc, part_l,
                           a.n_chunks, out);
    }
}

}  // namespace mi355x

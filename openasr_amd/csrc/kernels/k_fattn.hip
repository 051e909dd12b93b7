// k_fattn.hip -- GGML_OP_FLASH_ATTN_EXT over an f16 KV cache with grouped
// query heads (call site crates/openasr-core/src/ggml_runtime/cpu_graph.rs:
// 4144-4215; graph built in crates/openasr-core/src/nn/decoder.rs:2031-2105).
//
// Split-KV design: the KV span is cut into chunks; one workgroup owns one
// (chunk, kv head, sequence, query tile) and every query head that shares the
// kv head, so K/V bytes are fetched once per kv head. A chunk whose mask is
// -inf for every row is skipped without touching K/V (the reference graph
// always passes the full fixed span, nn/decoder.rs:1295-1301). Each
// workgroup leaves (max, sum, unnormalised V accumulator) per query row; a
// second kernel merges the chunks. Numerics follow ggml-cpu where it is
// cheap to do so: Q is rounded to f16 before the dot with f16 K, scores are
// scaled then masked, and V is accumulated in f32.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

constexpr int kFaThreads = 256;
constexpr int kFaMaxChunk = 256;

template <int D, int RMAX>
__global__ __launch_bounds__(kFaThreads) void k_fattn_partial(fattn_args a, float * __restrict__ part_acc,
                                                              float * __restrict__ part_ml) {
    constexpr int LPP = D / 8;        // lanes per key position in the score phase
    constexpr int PPW = 64 / LPP;     // positions per wave per step
    constexpr int DPL = D / 64;       // dims per lane in the V phase (1 or 2)
    constexpr int PG = kFaThreads / (D / DPL);  // position groups in the V phase
    __shared__ float s_sc[RMAX][kFaMaxChunk];
    __shared__ float s_m[RMAX], s_l[RMAX];
    __shared__ float s_red[PG][RMAX][D];
    __shared__ int s_any;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int chunk = blockIdx.x;
    const int kvh = blockIdx.y % a.hkv;
    const int seq = blockIdx.y / a.hkv;
    const int qtile = blockIdx.z;
    const int g = a.hq / a.hkv;
    const int tq_per_tile = RMAX / g;
    const int q0 = qtile * tq_per_tile;
    const int nrows = min(tq_per_tile, a.n_q - q0) * g;
    const int c0 = chunk * a.chunk;
    const int clen = min(a.chunk, a.n_kv - c0);
    const int kv_seq = seq / a.rk3;
    const char * kbase = a.k + (int64_t) kvh * a.k_nb2 + (int64_t) kv_seq * a.k_nb3;
    const char * vbase = a.v + (int64_t) kvh * a.v_nb2 + (int64_t) kv_seq * a.v_nb3;

    // mask rows of this tile; skip the chunk when every entry is -inf
    if (tid == 0) s_any = 0;
    __syncthreads();
    if (a.mask) {
        int any = 0;
        for (int idx = tid; idx < clen * (nrows / g); idx += kFaThreads) {
            const int tq = idx / clen, p = idx % clen;
            const uint16_t mv = *(const uint16_t *) (a.mask + (int64_t) (q0 + tq) * a.m_nb1 +
                                                     (int64_t) (kvh * g % a.m_ne2) * a.m_nb2 +
                                                     (int64_t) (seq % a.m_ne3) * a.m_nb3 + (int64_t) (c0 + p) * 2);
            if (mv != 0xFC00) any = 1;
        }
        if (any) s_any = 1;
    } else if (tid == 0) {
        s_any = 1;
    }
    __syncthreads();
    const int64_t row_base = ((int64_t) seq * a.n_q + q0) * a.hq + (int64_t) kvh * g;  // output row of (tq=0, gi=0)
    if (!s_any) {
        for (int r = tid; r < nrows; r += kFaThreads) {
            const int tq = r / g, gi = r % g;
            const int64_t orow = row_base + (int64_t) tq * a.hq + gi;
            float * ml = part_ml + (orow * a.n_chunks + chunk) * 2;
            ml[0] = -INFINITY;
            ml[1] = 0.0f;
        }
        return;
    }

    // ---- scores: LPP lanes per key position, Q slice in registers ----
    const int dl = (lane % LPP) * 8;
    float qr[RMAX][8];
#pragma unroll
    for (int r = 0; r < RMAX; r++) {
        const int tq = r / g, gi = r % g;
        const bool ok = r < nrows;
        const float * qp = (const float *) (a.q + (int64_t) (q0 + (ok ? tq : 0)) * a.q_nb1 +
                                            (int64_t) (kvh * g + gi) * a.q_nb2 + (int64_t) seq * a.q_nb3);
#pragma unroll
        for (int i = 0; i < 8; i++) qr[r][i] = ok ? round_to_half(qp[dl + i]) : 0.0f;
    }
    for (int base = wave * PPW; base < clen; base += 4 * PPW) {
        const int p = base + lane / LPP;
        const bool valid = p < clen;
        float kf[8];
        if (valid) {
            const uint4 kv4 = *(const uint4 *) (kbase + (int64_t) (c0 + p) * a.k_nb1 + dl * 2);
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
        for (int r = 0; r < RMAX; r++) {
            if (r >= nrows) break;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) s += kf[i] * qr[r][i];
            s = group_sum<LPP>(s);
            if (valid && (lane % LPP) == 0) {
                const int tq = r / g;
                float mv = 0.0f;
                if (a.mask) {
                    mv = half_bits_to_float(*(const uint16_t *) (a.mask + (int64_t) (q0 + tq) * a.m_nb1 +
                                                                 (int64_t) (kvh * g % a.m_ne2) * a.m_nb2 +
                                                                 (int64_t) (seq % a.m_ne3) * a.m_nb3 +
                                                                 (int64_t) (c0 + p) * 2));
                }
                // a masked position is skipped outright, as ggml-cpu does, so
                // whatever an unwritten cache slot holds never reaches the sums
                s_sc[r][p] = mv == -INFINITY ? -INFINITY : s * a.scale + mv;
            }
        }
    }
    __syncthreads();

    // ---- softmax statistics per row (one wave per row) ----
    for (int r = wave; r < nrows; r += 4) {
        float m = -INFINITY;
        for (int p = lane; p < clen; p += 64) m = fmaxf(m, s_sc[r][p]);
        m = wave_max(m);
        float l = 0.0f;
        for (int p = lane; p < clen; p += 64) {
            const float e = m == -INFINITY ? 0.0f : expf(s_sc[r][p] - m);
            s_sc[r][p] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            s_m[r] = m;
            s_l[r] = l;
        }
    }
    __syncthreads();

    // ---- V accumulation: threads over (dim slice, position group) ----
    const int dslot = tid % (D / DPL);
    const int pg = tid / (D / DPL);
    float acc[RMAX][DPL];
#pragma unroll
    for (int r = 0; r < RMAX; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) acc[r][i] = 0.0f;
    for (int p = pg; p < clen; p += PG) {
        const char * vp = vbase + (int64_t) (c0 + p) * a.v_nb1 + dslot * DPL * 2;
        float vf[DPL];
        if (DPL == 2) {
            const uint32_t w = *(const uint32_t *) vp;
            vf[0] = half_bits_to_float((uint16_t) (w & 0xFFFF));
            vf[DPL - 1] = half_bits_to_float((uint16_t) (w >> 16));
        } else {
            vf[0] = half_bits_to_float(*(const uint16_t *) vp);
        }
#pragma unroll
        for (int r = 0; r < RMAX; r++) {
            if (r >= nrows) break;
            const float pr = s_sc[r][p];
            if (pr == 0.0f) continue;
#pragma unroll
            for (int i = 0; i < DPL; i++) acc[r][i] += pr * vf[i];
        }
    }
#pragma unroll
    for (int r = 0; r < RMAX; r++)
#pragma unroll
        for (int i = 0; i < DPL; i++) s_red[pg][r][dslot * DPL + i] = acc[r][i];
    __syncthreads();
    for (int idx = tid; idx < nrows * D; idx += kFaThreads) {
        const int r = idx / D, d = idx % D;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < PG; q++) v += s_red[q][r][d];
        const int tq = r / g, gi = r % g;
        const int64_t orow = row_base + (int64_t) tq * a.hq + gi;
        part_acc[(orow * a.n_chunks + chunk) * D + d] = v;
        if (d == 0) {
            float * ml = part_ml + (orow * a.n_chunks + chunk) * 2;
            ml[0] = s_m[r];
            ml[1] = s_l[r];
        }
    }
}

// merge the per-chunk partials of one output row: out = sum_i acc_i e^(m_i-M) / sum_i l_i e^(m_i-M)
template <int D>
__global__ __launch_bounds__(D) void k_fattn_combine(const float * __restrict__ part_acc,
                                                     const float * __restrict__ part_ml, int n_chunks,
                                                     float * __restrict__ out) {
    const int64_t orow = blockIdx.x;
    const int d = threadIdx.x;
    const float * ml = part_ml + orow * n_chunks * 2;
    float M = -INFINITY;
    for (int i = 0; i < n_chunks; i++) M = fmaxf(M, ml[2 * i]);
    float L = 0.0f, acc = 0.0f;
    if (M != -INFINITY) {
        for (int i = 0; i < n_chunks; i++) {
            const float mi = ml[2 * i];
            if (mi == -INFINITY) continue;
            const float w = expf(mi - M);
            L += ml[2 * i + 1] * w;
            acc += part_acc[(orow * n_chunks + i) * D + d] * w;
        }
    }
    out[orow * D + d] = L == 0.0f ? 0.0f : acc / L;
}

size_t fattn_scratch_bytes(const fattn_args & a) {
    const int64_t rows = (int64_t) a.n_seq * a.n_q * a.hq;
    return (size_t) rows * a.n_chunks * (a.d + 2) * sizeof(float);
}

void fattn_plan(fattn_args & a, int n_cu) {
    const int g = a.hq / a.hkv;
    const int rmax = g <= 8 ? 8 : 16;
    const int tq_per_tile = rmax / g;
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
    return hq / hkv <= 16;
}

void launch_fattn(const fattn_args & a, float * scratch, float * out, hipStream_t stream) {
    float * part_acc = scratch;
    float * part_ml = scratch + (int64_t) a.n_seq * a.n_q * a.hq * a.n_chunks * a.d;
    const dim3 grid((unsigned) a.n_chunks, (unsigned) (a.hkv * a.n_seq), (unsigned) a.q_tiles);
    const int g = a.hq / a.hkv;
    if (a.d == 128) {
        if (g <= 8) hipLaunchKernelGGL((k_fattn_partial<128, 8>), grid, dim3(kFaThreads), 0, stream, a, part_acc, part_ml);
        else hipLaunchKernelGGL((k_fattn_partial<128, 16>), grid, dim3(kFaThreads), 0, stream, a, part_acc, part_ml);
        hipLaunchKernelGGL(k_fattn_combine<128>, dim3((unsigned) (a.n_seq * a.n_q * a.hq)), dim3(128), 0, stream,
                           part_acc, part_ml, a.n_chunks, out);
    } else {
        if (g <= 8) hipLaunchKernelGGL((k_fattn_partial<64, 8>), grid, dim3(kFaThreads), 0, stream, a, part_acc, part_ml);
        else hipLaunchKernelGGL((k_fattn_partial<64, 16>), grid, dim3(kFaThreads), 0, stream, a, part_acc, part_ml);
        hipLaunchKernelGGL(k_fattn_combine<64>, dim3((unsigned) (a.n_seq * a.n_q * a.hq)), dim3(64), 0, stream,
                           part_acc, part_ml, a.n_chunks, out);
    }
}

}  // namespace mi355x

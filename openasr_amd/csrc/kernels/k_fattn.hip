// k_fattn.hip -- GGML_OP_FLASH_ATTN_EXT over an f16 KV cache with grouped
// query heads (call site crates/openasr-core/src/ggml_runtime/cpu_graph.rs:
// 4144-4215; graph built in crates/openasr-core/src/nn/decoder.rs:2031-2105).
//
// The result is defined chunk-wise over fixed 64-position KV chunks, the
// same on every launch shape:
//   per chunk c   for each live (unmasked) position, in f32:
//                   s = fma-chain_d(k[d], f16(q)[d]) * scale + mask
//                 (the chain runs over the dims in order from 0; masked
//                 positions are skipped outright, as ggml-cpu does)
//                 m_c = max s, p = exp(s - m_c); over the live positions in
//                 order, l_c = l_c + p and a_c = fma(p, v, a_c) in f32
//   combine       M = max m_c; for c in order, in f64: w = exp(m_c - M),
//                 L += w * l_c, O += w * a_c; out = f32(O / L)
// Every chain is sequential in one thread, so each launch form below gives
// the same bits. The CPU reference evaluates the same definition (oracle
// fidelity 5).
//
// Three launch forms compute it:
//   decode one wave per (chunk, kv head, sequence) and query head (or
//          pair of the kv head's query heads) for a single query
//          position: mask first, then the chunk's K and V, no barriers;
//          partials to scratch, combined by a second launch.
//   split  one workgroup per (chunk, kv head, sequence, query tile): loads
//          the chunk's mask first and skips a fully masked chunk without
//          touching K/V (the graph always passes the full fixed span,
//          nn/decoder.rs:1295-1301), then issues all of its K and V loads at
//          once into LDS; partials go to scratch and a second launch combines
//          them per tile.
//   full   one workgroup per (kv head, sequence, query tile) walks every
//          chunk twice (chunk maxima, then sums). Used for prefill.
// In split and full, lane p of each wave takes position p for the scores
// (wave w the tile rows w, w + 4, ...) and each thread one row's run of dims
// for P * V. Both can quantize their output straight into the activation
// layout of the MUL_MAT that consumes it (the attention output projection),
// since a tile holds all query heads of one kv head: g*D consecutive
// elements of a column.
#include <type_traits>

#include "../mi355x_common.h"
#include "../ops.h"
#include "../quant_dev.h"
#include "../fattn_dev.h"

namespace mi355x {

constexpr int kFaThreads = 256;
constexpr int kFaChunk = 64;
constexpr int kFaMaxChunks = 256;  // 16384 KV positions
constexpr int kFaMaxRows = 8;      // query rows (positions x heads of one kv head) per tile


__device__ __forceinline__ fa_tile fa_tile_of(const fattn_args & a) {
    fa_tile t;
    t.kvh = (int) blockIdx.y % a.hkv;
    t.seq = (int) blockIdx.y / a.hkv;
    t.g = a.hq / a.hkv;
    t.tq0 = (int) blockIdx.z * a.tq;
    t.ntq = min(a.tq, a.n_q - t.tq0);
    t.nrows = t.ntq * t.g;
    t.kv_seq = t.seq / a.rk3;
    t.gti = (int) blockIdx.y * a.q_tiles + (int) blockIdx.z;
    return t;
}

// output row (ggml result layout [D, hq, n_q, n_seq]) of tile row r
__device__ __forceinline__ int64_t fa_orow(const fattn_args & a, const fa_tile & t, int r) {
    return ((int64_t) t.seq * a.n_q + t.tq0 + r / t.g) * a.hq + (int64_t) t.kvh * t.g + r % t.g;
}

template <int D, int R>
struct alignas(16) fa_smem {
    uint4 k[kFaChunk][D / 8 + 1];  // the chunk's K rows, padded: conflict-free row reads
    uint4 v[kFaChunk][D / 8];      // the chunk's V rows
    float q[R][D];                 // f16-rounded queries; after the combine, the output rows
    float s[R][kFaChunk];          // scores, then p
    float mask[R][kFaChunk];       // per query position of the tile
    uint64_t live[R];              // live positions of the chunk per row
    float m[R];
};

__device__ __forceinline__ void unpack8(const uint4 & u, float * f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = half_bits_to_float((uint16_t) (w[i] & 0xFFFF));
        f[2 * i + 1] = half_bits_to_float((uint16_t) (w[i] >> 16));
    }
}

// the score chain of one position: acc = fma(k[d], q[d], acc) over the dims
// in order, from 0, in f32 (k is f16, so the compiler may read it in place)
template <int D>
__device__ __forceinline__ float fa_dot(const uint4 (&kr)[D / 8], const float * q) {
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < D / 8; u++) {
        float kf[8];
        unpack8(kr[u], kf);
        const float4 q0 = *(const float4 *) (q + 8 * u);
        const float4 q1 = *(const float4 *) (q + 8 * u + 4);
        const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) acc = fmaf(kf[i], qv[i], acc);
    }
    return acc;
}

// the same chain with the query as f16 halves (its f16-rounded values), all
// D/8 16-byte pieces requested before the first step: the chain then waits
// on no LDS read (each step is one v_fma_mix_f32, both operands halves)
template <int D>
__device__ __forceinline__ float fa_dot_h(const uint4 (&kr)[D / 8], const uint4 * qh) {
    uint4 qv[D / 8];
#pragma unroll
    for (int u = 0; u < D / 8; u++) qv[u] = qh[u];
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < D / 8; u++) {
        float kf[8], qf[8];
        unpack8(kr[u], kf);
        unpack8(qv[u], qf);
#pragma unroll
        for (int i = 0; i < 8; i++) acc = fmaf(kf[i], qf[i], acc);
    }
    return acc;
}

// mask of chunk c for the tile's query positions; true if any entry is live
template <int D, int R>
__device__ __forceinline__ bool fa_load_mask(const fattn_args & a, const fa_tile & t, int c, fa_smem<D, R> & sm) {
    const int clen = min(kFaChunk, a.n_kv - c * kFaChunk);
    int live = 0;
    for (int idx = (int) threadIdx.x; idx < t.ntq * kFaChunk; idx += kFaThreads) {
        const int tql = idx / kFaChunk, p = idx % kFaChunk;
        float mv = -INFINITY;
        if (p < clen) {
            mv = 0.0f;
            if (a.mask) {
                const uint16_t * mr = (const uint16_t *) (a.mask + (int64_t) (t.tq0 + tql) * a.m_nb1 +
                                                          (int64_t) (t.seq % a.m_ne3) * a.m_nb3);
                mv = half_bits_to_float(mr[c * kFaChunk + p]);
            }
        }
        sm.mask[tql][p] = mv;
        live |= mv != -INFINITY;
    }
    return __syncthreads_or(live) != 0;
}

// the chunk's K (and V) rows into registers, all requested at once: thread t
// takes the 16-byte pieces t, t + 256, ... of the row-major chunk. Rows past
// the span repeat the chunk's last row (in bounds; such positions are masked).
template <int D, bool WITH_V>
struct fa_kv_regs {
    static constexpr int NP = kFaChunk * D / 8 / kFaThreads;
    uint4 k[NP];
    uint4 v[WITH_V ? NP : 1];
};

template <int D, bool WITH_V>
__device__ __forceinline__ void fa_load_kv(const fattn_args & a, const fa_tile & t, int c, fa_kv_regs<D, WITH_V> & r) {
    constexpr int RP = D / 8;
    const int clen = min(kFaChunk, a.n_kv - c * kFaChunk);
    const char * kb = a.k + (int64_t) t.kvh * a.k_nb2 + (int64_t) t.kv_seq * a.k_nb3 + (int64_t) c * kFaChunk * a.k_nb1;
    const char * vb = a.v + (int64_t) t.kvh * a.v_nb2 + (int64_t) t.kv_seq * a.v_nb3 + (int64_t) c * kFaChunk * a.v_nb1;
#pragma unroll
    for (int i = 0; i < fa_kv_regs<D, WITH_V>::NP; i++) {
        const int piece = (int) threadIdx.x + i * kFaThreads, row = min(piece / RP, clen - 1), col = piece % RP;
        r.k[i] = *(const uint4 *) (kb + (int64_t) row * a.k_nb1 + 16 * col);
        if constexpr (WITH_V) r.v[i] = *(const uint4 *) (vb + (int64_t) row * a.v_nb1 + 16 * col);
    }
}

template <int D, int R, bool WITH_V>
__device__ __forceinline__ void fa_store_kv(const fa_kv_regs<D, WITH_V> & r, fa_smem<D, R> & sm) {
    constexpr int RP = D / 8;
#pragma unroll
    for (int i = 0; i < fa_kv_regs<D, WITH_V>::NP; i++) {
        const int piece = (int) threadIdx.x + i * kFaThreads;
        sm.k[piece / RP][piece % RP] = r.k[i];
        if constexpr (WITH_V) sm.v[piece / RP][piece % RP] = r.v[i];
    }
}

template <int D, int R>
__device__ __forceinline__ void fa_load_q(const fattn_args & a, const fa_tile & t, fa_smem<D, R> & sm) {
    for (int idx = (int) threadIdx.x; idx < t.nrows * D; idx += kFaThreads) {
        const int r = idx / D, d = idx % D;
        const float * qp = (const float *) (a.q + (int64_t) (t.tq0 + r / t.g) * a.q_nb1 +
                                            (int64_t) (t.kvh * t.g + r % t.g) * a.q_nb2 + (int64_t) t.seq * a.q_nb3);
        sm.q[r][d] = round_to_half(qp[d]);
    }
}

// scores of the chunk into sm.s: lane p of every wave takes position p (its
// K row from LDS), wave w the rows w, w + 4, ... (needs sm.k, sm.q, sm.mask;
// the caller syncs after)
template <int D, int R>
__device__ __forceinline__ void fa_scores(const fattn_args & a, const fa_tile & t, fa_smem<D, R> & sm) {
    const int p = (int) threadIdx.x & 63, wave = (int) threadIdx.x >> 6;
    if (wave >= t.nrows) return;
    uint4 kr[D / 8];
#pragma unroll
    for (int u = 0; u < D / 8; u++) kr[u] = sm.k[p][u];
    for (int r = wave; r < t.nrows; r += 4) {
        const float acc = fa_dot<D>(kr, &sm.q[r][0]);
        const float mv = sm.mask[r / t.g][p];
        sm.s[r][p] = mv == -INFINITY ? -INFINITY : acc * a.scale + mv;
    }
}

// chunk maximum m_c and (WITH_P) p = exp(s - m_c) in place and the live
// positions; one wave per row
template <int D, int R, bool WITH_P>
__device__ __forceinline__ void fa_softmax_chunk(const fa_tile & t, fa_smem<D, R> & sm) {
    const int lane = (int) threadIdx.x & 63, wave = (int) threadIdx.x >> 6;
    for (int r = wave; r < t.nrows; r += 4) {
        const float s = sm.s[r][lane];
        const float m = wave_max(s);
        const bool live = s != -INFINITY;
        if constexpr (WITH_P) sm.s[r][lane] = live ? expf_det(s - m) : 0.0f;
        const uint64_t bits = __ballot(live);
        if (lane == 0) {
            sm.m[r] = m;
            sm.live[r] = bits;
        }
    }
}

// P * V of one row's dims [d0, d0 + DPT): the live positions in order,
// l = l + p and acc = fma(p, v, acc) in f32 (needs sm.s, sm.v, sm.live)
template <int D, int R, int DPT>
__device__ __forceinline__ void fa_pv_row(const fa_smem<D, R> & sm, int r, int d0, float (&acc)[DPT], float & l) {
    const uint64_t live = sm.live[r];
    const uint16_t * vb = (const uint16_t *) &sm.v[0][0] + d0;
#pragma unroll
    for (int i = 0; i < DPT; i++) acc[i] = 0.0f;
    l = 0.0f;
    for (int j = 0; j < kFaChunk; j++) {
        if ((live >> j) & 1) {
            const float p = sm.s[r][j];
            l = l + p;
            const uint16_t * vr = vb + j * D;
#pragma unroll
            for (int i = 0; i < DPT; i++) acc[i] = fmaf(p, half_bits_to_float(vr[i]), acc[i]);
        }
    }
}

// dims per thread of the P * V step: every (row, dim) of the tile has one thread
template <int D, int R>
struct fa_pv_shape {
    static constexpr int DPT = R * D >= 2 * kFaThreads ? R * D / kFaThreads : 1;
    static constexpr int TPR = D / DPT;  // threads per row
};

template <int D, int R>
__global__ __launch_bounds__(kFaThreads) void k_fattn_split(fattn_args a, float * __restrict__ part_m,
                                                            float * __restrict__ part_l,
                                                            float * __restrict__ part_acc) {
    __shared__ fa_smem<D, R> sm;
    using PV = fa_pv_shape<D, R>;
    const fa_tile t = fa_tile_of(a);
    const int c = (int) blockIdx.x, tid = (int) threadIdx.x;
    const int64_t prow = (int64_t) t.gti * R;  // partial row of tile row 0

    if (fa_load_mask<D, R>(a, t, c, sm)) {
        fa_kv_regs<D, true> kv;
        fa_load_kv<D, true>(a, t, c, kv);
        fa_load_q<D, R>(a, t, sm);
        fa_store_kv<D, R, true>(kv, sm);
        __syncthreads();
        fa_scores<D, R>(a, t, sm);
        __syncthreads();
        fa_softmax_chunk<D, R, true>(t, sm);
        __syncthreads();
        const int r = tid / PV::TPR, d0 = (tid % PV::TPR) * PV::DPT;
        if (r < t.nrows) {
            float acc[PV::DPT], l;
            fa_pv_row<D, R, PV::DPT>(sm, r, d0, acc, l);
            float * pa = part_acc + ((prow + r) * a.n_chunks + c) * D + d0;
#pragma unroll
            for (int i = 0; i < PV::DPT; i++) pa[i] = acc[i];
            if (d0 == 0) {
                part_m[(prow + r) * a.n_chunks + c] = sm.m[r];
                part_l[(prow + r) * a.n_chunks + c] = l;
            }
        }
    } else if (tid < t.nrows) {
        part_m[(prow + tid) * a.n_chunks + c] = -INFINITY;
        part_l[(prow + tid) * a.n_chunks + c] = 0.0f;
    }
}

// combine of the split forms: one workgroup per tile, chunks in order, in
// f64. Each thread owns output elements of the tile; its partials for up to
// CB chunks are requested together with the chunk maxima and sums, so a span
// of up to CB chunks costs one memory round trip. The loads are unconditional
// (chunk index clamped to the span, row 0 for a thread without an element).
template <int D, int R, int CB0>
__global__ __launch_bounds__(kFaThreads) void k_fattn_combine(fattn_args a, const float * __restrict__ part_m,
                                                              const float * __restrict__ part_l,
                                                              const float * __restrict__ part_acc,
                                                              float * __restrict__ out) {
    constexpr int NE = (R * D + kFaThreads - 1) / kFaThreads;  // output elements per thread
    constexpr int CB = CB0 < 64 / NE ? CB0 : 64 / NE;          // chunks per batch of loads
    __shared__ __align__(16) float s_out[R][D];
    __shared__ double s_w[R][kFaMaxChunks];
    __shared__ double s_l[R][kFaMaxChunks];
    const fa_tile t = fa_tile_of(a);
    const int tid = (int) threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t prow = (int64_t) t.gti * R;
    const int nc = a.n_chunks;
    // the chunk maxima and sums of this wave's row first (clamped loads: up to
    // kFaMaxChunks / 64 per lane), then every partial this thread combines, so
    // that the weights are computed while the partials are still in flight
    constexpr int MPL = kFaMaxChunks / 64;
    const int r_w = wave < t.nrows ? wave : 0;  // rows >= 4 handled below
    float mreg[MPL], lreg[MPL];
#pragma unroll
    for (int q = 0; q < MPL; q++) {
        const int i = lane + 64 * q;
        const int ic = i < nc ? i : 0;
        mreg[q] = part_m[(prow + r_w) * nc + ic];
        lreg[q] = part_l[(prow + r_w) * nc + ic];
    }
    int er[NE], ed[NE];
    bool ev[NE];
    float pv[NE][CB];
#pragma unroll
    for (int e = 0; e < NE; e++) {
        const int idx = tid + e * kFaThreads;
        ev[e] = idx < t.nrows * D;
        er[e] = ev[e] ? idx / D : 0;
        ed[e] = idx % D;
        const float * pa = part_acc + (prow + er[e]) * nc * D + ed[e];
#pragma unroll
        for (int k = 0; k < CB; k++) pv[e][k] = pa[(int64_t) min(k, nc - 1) * D];
    }
    for (int r = wave; r < t.nrows; r += 4) {
        if (r != r_w) {  // a wave with a second row (tiles of more than 4 rows) loads it now
#pragma unroll
            for (int q = 0; q < MPL; q++) {
                const int i = lane + 64 * q;
                const int ic = i < nc ? i : 0;
                mreg[q] = part_m[(prow + r) * nc + ic];
                lreg[q] = part_l[(prow + r) * nc + ic];
            }
        }
        float M = -INFINITY;
#pragma unroll
        for (int q = 0; q < MPL; q++) M = lane + 64 * q < nc ? fmaxf(M, mreg[q]) : M;
        M = wave_max(M);
#pragma unroll
        for (int q = 0; q < MPL; q++) {
            const int i = lane + 64 * q;
            if (i < nc) {
                s_w[r][i] = mreg[q] == -INFINITY ? 0.0 : (double) expf_det(mreg[q] - M);
                s_l[r][i] = (double) lreg[q];
            }
        }
    }
    __syncthreads();
    // per element two chains (L, O), each in chunk order; every batch of
    // chunks requests the partials of all this thread's elements before any
    // is added, so a span of nc chunks costs nc / CB round trips, not NE times
    // as many
    double L[NE], O[NE];
#pragma unroll
    for (int e = 0; e < NE; e++) {
        L[e] = 0.0;
        O[e] = 0.0;
    }
    for (int c0 = 0; c0 < nc; c0 += CB) {
        if (c0 > 0) {
#pragma unroll
            for (int e = 0; e < NE; e++) {
                const float * pa = part_acc + ((prow + er[e]) * nc + c0) * D + ed[e];
#pragma unroll
                for (int k = 0; k < CB; k++) pv[e][k] = pa[(int64_t) (min(c0 + k, nc - 1) - c0) * D];
            }
        }
        // a chunk with w = 0 adds +0, which leaves a sum that starts at +0
        // unchanged, as skipping it would (its partials may be stale)
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int r = er[e];
#pragma unroll
            for (int k = 0; k < CB; k++) {
                if (c0 + k >= nc) break;
                const double w = s_w[r][c0 + k];
                const double tl = w * s_l[r][c0 + k], to = w * (double) pv[e][k];
                L[e] += w != 0.0 ? tl : 0.0;
                O[e] += w != 0.0 ? to : 0.0;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < NE; e++) {
        if (!ev[e]) continue;
        const float o = L[e] == 0.0 ? 0.0f : (float) (O[e] / L[e]);
        out[fa_orow(a, t, er[e]) * D + ed[e]] = o;
        s_out[er[e]][ed[e]] = o;
    }
    if (a.qtype >= 0) {
        __syncthreads();
        fa_quantize_out<D>(a, t, &s_out[0][0]);
    }
}

// The decode wave's K and V requests for one chunk; rows past the span
// repeat the last one. K goes straight to LDS (global_load_lds, 16 bytes a
// lane): instruction u fills slots u*64 .. u*64+63 of the wave's area, slot
// t holding piece (t % KU) ^ (row & 7) of row t / KU -- swizzled, so that
// the transposed reads (lane p: the pieces of row p) hit distinct banks. V
// goes to registers, lane = its dims of every position.
__device__ __forceinline__ int fa_kslot(int row, int piece, int KU) { return row * KU + (piece ^ (row & 7)); }

template <int D>
__device__ __forceinline__ void fa_issue_kv(const char * kc, const char * vb, int64_t k_nb1, int vs, int loff, int clen,
                                            int lane, uint4 * s_kw, uint32_t (&vr)[kFaChunk]) {
    constexpr int KU = D / 8, DL = D / 64;
#pragma unroll
    for (int u = 0; u < KU; u++) {
        const int t = u * 64 + lane, row = t / KU, piece = (t % KU) ^ (row & 7);
        const char * src = kc + (int64_t) min(row, clen - 1) * k_nb1 + 16 * piece;
        __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *) src,
                                         (void __attribute__((address_space(3))) *) (s_kw + u * 64), 16, 0, 0);
    }
    // every K request is issued ahead of every V request: the callers' "at
    // most 63 outstanding" waits rely on that order, which the scheduler must
    // not change
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kFaChunk; j++) {
        const int off = (j < clen ? j : clen - 1) * vs + loff;
        if (DL == 2) vr[j] = *(const uint32_t *) (vb + off);
        else vr[j] = (uint32_t) *(const uint16_t *) (vb + off);
    }
}

// s_waitcnt with only a vector-memory bound: at most n (< 64) requests of this
// wave outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// The decode form's item of workgroup b: a unit (chunk c, sequence s, kv
// head k) and one group hg of G query heads of the kv head's g (ng = g / G
// groups): item = u * ng + hg with unit u = c * nkt + s * hkv + k (or, for
// G = 2, u = (s * hkv + k) * n_chunks + c). Workgroups are dealt to the 8
// XCDs round-robin (b % 8); the ng groups of a unit are XCD b % 8's
// consecutive workgroups b, b + 8, ..., whose L2 serves the second read of
// the chunk's K/V rows, and consecutive units go to consecutive XCDs, so the
// masked tail of the span spreads over every XCD. A grid of
// fa_decode_grid(items, ng) workgroups covers every item once.
constexpr int kFaXcds = 8;
__device__ __forceinline__ int64_t fa_decode_item(int64_t b, int ng) {
    const int64_t r = b / kFaXcds;
    return ((r / ng) * kFaXcds + b % kFaXcds) * ng + r % ng;
}
static int64_t fa_decode_grid(int64_t items, int ng) {
    const int64_t blk = (int64_t) kFaXcds * ng;
    return (items + blk - 1) / blk * blk;
}
// query heads per decode wave (fattn_args::dheads): one, or two whose chains
// share each K piece; more would not fit the wave's registers next to the K
// row and the chunk's V
// The mask of the decode wave's position (lane < clen), -inf past the span.
// The load is unconditional (a null mask reads the K cache's first half and
// ignores it; lanes past the span read the chunk's last position): a branch
// around it would leave the first loads' completion unknown where the paths
// join, and the compiler would then wait for every later request there.
__device__ __forceinline__ float fa_decode_mask(const fattn_args & a, int seq, int pos, int clen, int lane) {
    const int pc = pos - lane + min(lane, clen - 1);
    const uint16_t * mp = a.mask ? (const uint16_t *) (a.mask + (int64_t) (seq % a.m_ne3) * a.m_nb3) + pc
                                 : (const uint16_t *) a.k;
    const uint16_t raw = *mp;
    return lane < clen ? (a.mask ? half_bits_to_float(raw) : 0.0f) : -INFINITY;
}

// The G score chains of one position (lane = position): for each query head
// h of the kv head, acc_h = fma(k[d], q_h[d], acc_h) over the dims in order
// from 0, in f32. One K piece feeds the G chains, which advance together; the
// queries are f16 halves in LDS (their f16-rounded values), so each step is
// one v_fma_mix_f32. The query pieces are read two 8-dim steps ahead of their
// use: held all at once they would take 4 * D / 8 registers a head.
template <int D, int G>
__device__ __forceinline__ void fa_dot_hg(const uint4 (&kr)[D / 8], const uint16_t (*sq)[D], float (&sc)[G]) {
    constexpr int KU = D / 8;
    uint4 q0[G], q1[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        sc[h] = 0.0f;
        q0[h] = *(const uint4 *) &sq[h][0];
        q1[h] = *(const uint4 *) &sq[h][8];
    }
#pragma unroll
    for (int u = 0; u < KU; u++) {
        uint4 q2[G];
#pragma unroll
        for (int h = 0; h < G; h++) q2[h] = *(const uint4 *) &sq[h][8 * (u + 2 < KU ? u + 2 : KU - 1)];
        // the reads above stay here: hoisted, every piece would be live at once
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < G; h++) {
            // each head converts the K halves inside its own fused
            // multiply-adds (v_fma_mix_f32): shared, the converted row would
            // take D registers
            uint4 kx = kr[u];
            if (h > 0) asm volatile("" : "+v"(kx.x), "+v"(kx.y), "+v"(kx.z), "+v"(kx.w));
            float kf[8], qf[8];
            unpack8(kx, kf);
            unpack8(q0[h], qf);
#pragma unroll
            for (int i = 0; i < 8; i++) sc[h] = fmaf(kf[i], qf[i], sc[h]);
            q0[h] = q1[h];
            q1[h] = q2[h];
        }
    }
}

// Decode form (one query position): one wave -- a workgroup of its own -- per
// (chunk, kv head, sequence) and group of G query heads of the kv head, so a
// kv head's K/V rows are requested once per G heads. For the scores lane p owns KV position p of the
// chunk (its whole K row, each query broadcast from LDS); for P*V lane l owns
// dims D/64*l.. of every position, the chunk's p values broadcast lane by
// lane. After the mask, K and V are requested in one burst. Each score chain
// runs over the dims in order in one lane, and each P*V chain over the
// positions in order in one lane, as the definition has them. A workgroup of
// one wave takes a CU's load and LDS bandwidth to itself where four queued
// behind each other (batch 1: 9.8 -> 8.7 us a launch).
//
// STEP (decode step, D = 128): the wave also derives its inputs from the
// fused QKV projection -- each query row's RMS norm * w and NEOX RoPE (the
// arithmetic of k_rms_norm_rope128), and, in the chunk holding this step's
// position, the new K row (same) and V row, which replace that cache row in
// the wave's registers; that wave also writes them into the f16 caches
// (SET_ROWS, after its outputs). No other wave reads the new row from the
// cache in this launch, so the write needs no ordering.
template <int D, bool STEP, int G>
__global__ __launch_bounds__(64) void k_fattn_decode(attn_step_args st, float * __restrict__ part_m,
                                                     float * __restrict__ part_l, float * __restrict__ part_acc) {
    constexpr int DL = D / 64;
    constexpr int KU = D / 8;  // 16-byte pieces of a K row
    static_assert(!STEP || D == 128, "the step form handles 128-wide heads");
    __shared__ __align__(16) uint16_t s_q[G][D];  // the query rows, f16
    __shared__ uint4 s_k[kFaChunk * KU];          // the chunk's K rows, swizzled (fa_kslot)
    __shared__ __align__(16) uint16_t s_vnew[D];  // STEP: the new V row
    const fattn_args & a = st.fa;
    const int lane = (int) threadIdx.x & 63;
    const int nc = a.n_chunks;
    const int64_t nkt = (int64_t) a.hkv * a.n_seq;
    const int g = a.hq / a.hkv, ng = g / G;
    const int64_t item = fa_decode_item(blockIdx.x, ng);
    if (item >= (int64_t) nc * nkt * ng) return;  // the grid's padding
    const int64_t unit = item / ng;
    // G = 2 (waves in several rounds): chunk-minor units, so waves resident
    // together stream neighbouring 16 KB K / V blocks rather than blocks 1 MB
    // apart (1.7B, 3000 positions: 2.44 -> 2.40 ms a step); G = 1 (one round):
    // chunk-major (0.6B, 640 positions: 1.24 -> 1.22 ms)
    const int c = (int) (G == 2 ? unit % nc : unit / nkt);
    const int kt = (int) (G == 2 ? unit / nc : unit % nkt);  // seq * hkv + kvh
    const int kvh = kt % a.hkv, seq = kt / a.hkv;
    const int head0 = kvh * g + (int) (item % ng) * G;
    const int kv_seq = seq / a.rk3;
    const int clen = min(kFaChunk, a.n_kv - c * kFaChunk);
    const int64_t prow0 = (int64_t) seq * a.hq + head0;  // partial rows prow0 + h
    const int pos = c * kFaChunk + lane;

    // the queries (f16-rounded) and the mask first; in the step form every
    // independent input is requested before any is used, and the queries'
    // norm and rotation wait until the chunk's K/V loads are in flight
    int jn = -1;  // STEP: the chunk row of this step's position, if in this chunk
    int64_t r_new = -1;
    float mv = -INFINITY;
    // STEP: the queries' inputs, normalised and rotated once the K/V loads are in flight
    float qx0[G], qx1[G], qw0 = 0.0f, qw1 = 0.0f;
    float2 qcs = make_float2(0.0f, 0.0f);
    // STEP: the new K / V row's inputs, requested with the queries' (every wave:
    // which one holds this step's position is known only with the index)
    float kx0 = 0.0f, kx1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f, vx0 = 0.0f, vx1 = 0.0f;
    uint16_t knew0 = 0, knew1 = 0, vnew0 = 0, vnew1 = 0;  // STEP: the new rows, f16
    if constexpr (STEP) {
        const char * ip = st.idx + (int64_t) (kvh % st.idx_ne1) * st.idx_nb1 + (int64_t) (seq % st.idx_ne2) * st.idx_nb2;
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float * qx = (const float *) (st.qsrc + (int64_t) (head0 + h) * st.q_nb1 + (int64_t) seq * st.q_nb2);
            qx0[h] = qx[lane];
            qx1[h] = qx[lane + 64];
        }
        qw0 = st.qw[lane];
        qw1 = st.qw[lane + 64];
        qcs = st.rope[seq * 64 + lane];
        const float * kxp = (const float *) (st.ksrc + (int64_t) kvh * st.k_nb1 + (int64_t) seq * st.k_nb2);
        kx0 = kxp[lane];
        kx1 = kxp[lane + 64];
        kw0 = st.kw[lane];
        kw1 = st.kw[lane + 64];
        const float * vxp = (const float *) (st.vsrc + (int64_t) kvh * st.v_nb1 + (int64_t) seq * st.v_nb2);
        vx0 = vxp[lane];
        vx1 = vxp[lane + 64];
        mv = fa_decode_mask(a, seq, pos, clen, lane);
        // the index as one or two 32-bit words, both requested whatever its
        // type (a branch here would make the compiler wait for every request
        // of the K/V burst before the queries' norm)
        const uint32_t lo = *(const uint32_t *) ip, hi = *(const uint32_t *) (ip + (st.idx_i64 ? 4 : 0));
        r_new = st.idx_i64 ? (int64_t) (((uint64_t) hi << 32) | lo) : (int64_t) (int32_t) lo;
        const int64_t j = r_new - (int64_t) c * kFaChunk;
        jn = j >= 0 && j < clen ? (int) j : -1;
    } else {
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float * qp = (const float *) (a.q + (int64_t) (head0 + h) * a.q_nb2 + (int64_t) seq * a.q_nb3);
            for (int d = lane; d < D; d += 64) s_q[h][d] = float_to_half_bits(qp[d]);
        }
        mv = fa_decode_mask(a, seq, pos, clen, lane);
    }
    const bool live = mv != -INFINITY;
    if (__ballot(live) == 0) {
        if (lane < G) {
            part_m[(prow0 + lane) * nc + c] = -INFINITY;
            part_l[(prow0 + lane) * nc + c] = 0.0f;
        }
        if constexpr (STEP) {
            // the cache row is written even when no query attends to it
            if (jn < 0) return;
        } else {
            return;
        }
    }
    // K (into LDS, for the transposed reads: lane p gets row p) and V (lane =
    // dims of every position) in one burst. Positions past the span read the
    // chunk's last valid row (always in bounds, loads stay unconditional);
    // they are masked.
    const char * kc = a.k + (int64_t) kvh * a.k_nb2 + (int64_t) kv_seq * a.k_nb3 + (int64_t) c * kFaChunk * a.k_nb1;
    const char * vb = a.v + (int64_t) kvh * a.v_nb2 + (int64_t) kv_seq * a.v_nb3 + (int64_t) c * kFaChunk * a.v_nb1;
    const int vs = (int) a.v_nb1, loff = lane * DL * 2;
    uint32_t vr[kFaChunk];
    fa_issue_kv<D>(kc, vb, a.k_nb1, vs, loff, clen, lane, &s_k[0], vr);
    if constexpr (STEP) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            float y0, y1;
            as_norm_rope(qx0[h], qx1[h], qw0, qw1, qcs, st.q_eps, y0, y1);
            s_q[h][lane] = float_to_half_bits(y0);
            s_q[h][lane + 64] = float_to_half_bits(y1);
        }
        if (jn >= 0) {
            // this step's K / V rows: K replaces the LDS row jn once the
            // chunk's K has landed (its requests precede the 64 V requests, so
            // at most 63 outstanding means every K request is done), V goes
            // through LDS to the dims layout
            float y0, y1;
            as_norm_rope(kx0, kx1, kw0, kw1, qcs, st.k_eps, y0, y1);
            knew0 = float_to_half_bits(y0);
            knew1 = float_to_half_bits(y1);
            vnew0 = float_to_half_bits(vx0);
            vnew1 = float_to_half_bits(vx1);
            uint16_t * krow = (uint16_t *) &s_k[0];
            wait_vmcnt<63>();
            krow[fa_kslot(jn, lane >> 3, KU) * 8 + (lane & 7)] = knew0;
            krow[fa_kslot(jn, (lane + 64) >> 3, KU) * 8 + (lane & 7)] = knew1;
            s_vnew[lane] = vnew0;
            s_vnew[lane + 64] = vnew1;
        }
        if (__ballot(live) == 0) {  // a fully masked chunk only has the cache row to write
            fa_decode_set_rows(st, jn, r_new, kvh, seq, lane, knew0, knew1, vnew0, vnew1);
            return;
        }
    }
    wait_vmcnt<63>();  // the K requests (ahead of the V ones) have landed
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint4 kr[KU];
#pragma unroll
    for (int u = 0; u < KU; u++) kr[u] = s_k[fa_kslot(lane, u, KU)];
    if constexpr (STEP) {
        if (jn >= 0) {
            const uint32_t vn = *(const uint32_t *) &s_vnew[lane * DL];
#pragma unroll
            for (int j = 0; j < kFaChunk; j++) vr[j] = j == jn ? vn : vr[j];
        }
    }

    // scores: lane = position, per query head the f32 fma chain over the dims in order
    float sc[G], p[G], m[G];
    fa_dot_hg<D, G>(kr, s_q, sc);
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float sv = live ? sc[h] * a.scale + mv : -INFINITY;
        m[h] = wave_max(sv);
        p[h] = sv == -INFINITY ? 0.0f : expf_det(sv - m[h]);
    }
    // P * V: lane = dims; per head l = l + p and acc = fma(p, v, acc) over the
    // live positions in order, p_j broadcast through a scalar register.
    // Masked positions (which may hold anything in the cache, even NaN) are
    // skipped by a scalar test of the live-position mask; with every position
    // live the loop runs without a test.
    const uint64_t live_bits = __ballot(live);
    float acc[G][DL], l[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        l[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < DL; i++) acc[h][i] = 0.0f;
    }
    auto pv_step = [&](int j) {
        const float v0 = half_bits_to_float((uint16_t) (vr[j] & 0xFFFF));
        const float v1 = DL == 2 ? half_bits_to_float((uint16_t) (vr[j] >> 16)) : 0.0f;
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[h]), j));
            l[h] = l[h] + pj;
            acc[h][0] = fmaf(pj, v0, acc[h][0]);
            if (DL == 2) acc[h][DL - 1] = fmaf(pj, v1, acc[h][DL - 1]);
        }
    };
    if (live_bits == ~0ull) {
#pragma unroll
        for (int j = 0; j < kFaChunk; j++) pv_step(j);
    } else {
#pragma unroll
        for (int j = 0; j < kFaChunk; j++) {
            if ((live_bits >> j) & 1) pv_step(j);
        }
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
        float * pa = part_acc + ((prow0 + h) * nc + c) * D + lane * DL;
#pragma unroll
        for (int i = 0; i < DL; i++) pa[i] = acc[h][i];
        if (lane == 0) {
            part_m[(prow0 + h) * nc + c] = m[h];
            part_l[(prow0 + h) * nc + c] = l[h];
        }
    }
    if constexpr (STEP) fa_decode_set_rows(st, jn, r_new, kvh, seq, lane, knew0, knew1, vnew0, vnew1);
}

template <int D, int R>
__global__ __launch_bounds__(kFaThreads) void k_fattn_full(fattn_args a, float * __restrict__ out) {
    __shared__ fa_smem<D, R> sm;
    __shared__ float s_mc[R][kFaMaxChunks];
    using PV = fa_pv_shape<D, R>;
    const fa_tile t = fa_tile_of(a);
    const int tid = (int) threadIdx.x;
    const int r = tid / PV::TPR, d0 = (tid % PV::TPR) * PV::DPT;  // this thread's output row and dims
    const bool owner = r < t.nrows;

    fa_load_q<D, R>(a, t, sm);
    // pass 1: chunk maxima
    for (int c = 0; c < a.n_chunks; c++) {
        const bool live = fa_load_mask<D, R>(a, t, c, sm);
        if (live) {
            fa_kv_regs<D, false> kv;
            fa_load_kv<D, false>(a, t, c, kv);
            fa_store_kv<D, R, false>(kv, sm);
            __syncthreads();
            fa_scores<D, R>(a, t, sm);
            __syncthreads();
            fa_softmax_chunk<D, R, false>(t, sm);
            __syncthreads();
        }
        if (tid < t.nrows) s_mc[tid][c] = live ? sm.m[tid] : -INFINITY;
        __syncthreads();
    }
    float M = -INFINITY;
    if (owner) {
        for (int c = 0; c < a.n_chunks; c++) M = fmaxf(M, s_mc[r][c]);
    }
    // pass 2: chunk sums combined in chunk order, in f64
    double O[PV::DPT], L = 0.0;
#pragma unroll
    for (int i = 0; i < PV::DPT; i++) O[i] = 0.0;
    for (int c = 0; c < a.n_chunks; c++) {
        int any = 0;
        for (int rr = 0; rr < t.nrows; rr++) any |= s_mc[rr][c] != -INFINITY;
        if (!any) continue;  // uniform
        fa_load_mask<D, R>(a, t, c, sm);
        fa_kv_regs<D, true> kv;
        fa_load_kv<D, true>(a, t, c, kv);
        fa_store_kv<D, R, true>(kv, sm);
        __syncthreads();
        fa_scores<D, R>(a, t, sm);
        __syncthreads();
        fa_softmax_chunk<D, R, true>(t, sm);
        __syncthreads();
        if (owner) {
            const float mc = s_mc[r][c];
            const float w = mc == -INFINITY ? 0.0f : expf_det(mc - M);
            if (w != 0.0f) {
                float acc[PV::DPT], l;
                fa_pv_row<D, R, PV::DPT>(sm, r, d0, acc, l);
                L += (double) w * (double) l;
#pragma unroll
                for (int i = 0; i < PV::DPT; i++) O[i] += (double) w * (double) acc[i];
            }
        }
        __syncthreads();
    }
    if (owner) {
#pragma unroll
        for (int i = 0; i < PV::DPT; i++) {
            const float o = L == 0.0 ? 0.0f : (float) (O[i] / L);
            out[fa_orow(a, t, r) * D + d0 + i] = o;
            sm.q[r][d0 + i] = o;
        }
    }
    if (a.qtype >= 0) {
        __syncthreads();
        fa_quantize_out<D>(a, t, &sm.q[0][0]);
    }
}

// ------------------------------------------------------------------ host --

static int64_t fa_tiles(const fattn_args & a) { return (int64_t) a.hkv * a.n_seq * a.q_tiles; }

size_t fattn_scratch_bytes(const fattn_args & a) {
    if (a.mfma) return fattn_mfma_scratch_bytes(a);
    if (a.dec) return fattn_dec_scratch_bytes(a);
    if (!a.split) return 0;
    const int64_t prows = fa_tiles(a) * a.rows * a.n_chunks;
    return (size_t) prows * (2 + (size_t) a.d) * sizeof(float) + 1024;
}

void fattn_plan(fattn_args & a, int n_cu) {
    const int g = a.hq / a.hkv;
    a.tq = a.n_q == 1 ? 1 : kFaMaxRows / g;
    a.rows = g * a.tq;
    a.q_tiles = (a.n_q + a.tq - 1) / a.tq;
    a.n_chunks = (a.n_kv + kFaChunk - 1) / kFaChunk;
    const int64_t tiles = fa_tiles(a);
    const int64_t part_bytes = tiles * a.rows * a.n_chunks * (8 + 4 * (int64_t) a.d);
    // split the KV span over workgroups when the tiles alone leave CUs idle.
    // Measured: 64-wide heads (the audio encoders' 390 x 390 self attention,
    // 686 tiles: 93 -> ~60 us a layer) gain from the split up to several
    // tiles a CU; 128-wide causal prefill chunks (1024 tiles) lose from it
    const bool fits = a.n_chunks <= kFaMaxChunks && part_bytes <= (256LL << 20);
    if (fits && a.n_q == 1) a.split = 2;  // wave per (chunk, kv head, query head group) of the one query
    else a.split = fits && tiles < (a.d == 64 ? 8LL : 2LL) * n_cu ? 1 : 0;
    // decode waves: one per query head while they all fit the CUs at once
    // (eight a CU: the LDS and registers of one allow that many); past that,
    // one wave takes two heads from one K/V read, halving the rounds of waves
    // behind each other
    const int64_t units = (int64_t) a.n_chunks * a.hkv * a.n_seq;
    a.dheads = g >= 2 && units * g > 8LL * n_cu ? 2 : 1;
}

template <int D, int R>
static void launch_combine(const fattn_args & a, const float * pm, const float * pl, const float * pa, float * out,
                           hipStream_t s) {
    const dim3 grid(1u, (unsigned) (a.hkv * a.n_seq), (unsigned) a.q_tiles);
    if (a.n_chunks <= 16) hipLaunchKernelGGL((k_fattn_combine<D, R, 16>), grid, dim3(kFaThreads), 0, s, a, pm, pl, pa, out);
    else hipLaunchKernelGGL((k_fattn_combine<D, R, 64>), grid, dim3(kFaThreads), 0, s, a, pm, pl, pa, out);
}

bool attn_step_supported(const fattn_args & a) {
    if (a.dec) return a.d == 128;  // the default-precision workgroup form
    return a.d == 128 && a.n_q == 1 && a.split == 2 && fattn_supported(a.d, a.hq, a.hkv);
}

size_t attn_step_scratch_bytes(const fattn_args & a) { return fattn_scratch_bytes(a); }

void launch_fattn_combine(const fattn_args & a, const float * pm, const float * pl, const float * pa, float * out,
                          hipStream_t s) {
    auto go = [&](auto d) {
        constexpr int D = decltype(d)::value;
        switch (a.rows) {
            case 1: launch_combine<D, 1>(a, pm, pl, pa, out, s); break;
            case 2: launch_combine<D, 2>(a, pm, pl, pa, out, s); break;
            case 4: launch_combine<D, 4>(a, pm, pl, pa, out, s); break;
            default: launch_combine<D, 8>(a, pm, pl, pa, out, s); break;
        }
    };
    if (a.d == 128) go(std::integral_constant<int, 128>{});
    else go(std::integral_constant<int, 64>{});
}

// one query position: rows = g query heads of a kv head, one decode wave per
// (chunk, kv head, sequence) for all of them
template <int R>
static void launch_attn_step_g(const attn_step_args & st, float * pm, float * pl, float * pa, hipStream_t s) {
    const fattn_args & a = st.fa;
    const int64_t units = (int64_t) a.n_chunks * a.hkv * a.n_seq;
    if (R >= 2 && a.dheads == 2) {
        constexpr int G = R >= 2 ? 2 : 1;
        hipLaunchKernelGGL((k_fattn_decode<128, true, G>), dim3((unsigned) fa_decode_grid(units * (R / G), R / G)),
                           dim3(64), 0, s, st, pm, pl, pa);
    } else {
        hipLaunchKernelGGL((k_fattn_decode<128, true, 1>), dim3((unsigned) fa_decode_grid(units * R, R)), dim3(64), 0,
                           s, st, pm, pl, pa);
    }
    launch_combine<128, R>(a, pm, pl, pa, st.out, s);
}

void launch_attn_step(const attn_step_args & st, void * scratch, hipStream_t s) {
    const fattn_args & a = st.fa;
    if (a.dec) {
        launch_fattn_dec(st, true, st.out, scratch, s);
        return;
    }
    const int64_t prows = fa_tiles(a) * a.rows * a.n_chunks;
    float * pm = (float *) scratch;
    float * pl = pm + prows;
    char * p = (char *) (pl + prows);
    float * pa = (float *) (((uintptr_t) p + 255) & ~(uintptr_t) 255);
    switch (a.rows) {
        case 1: launch_attn_step_g<1>(st, pm, pl, pa, s); break;
        case 2: launch_attn_step_g<2>(st, pm, pl, pa, s); break;
        case 4: launch_attn_step_g<4>(st, pm, pl, pa, s); break;
        default: launch_attn_step_g<8>(st, pm, pl, pa, s); break;
    }
}

bool fattn_supported(int d, int hq, int hkv) {
    if (d != 64 && d != 128) return false;
    if (hkv <= 0 || hq % hkv != 0) return false;
    const int g = hq / hkv;
    return g == 1 || g == 2 || g == 4 || g == 8;
}

bool fattn_fits(const fattn_args & a) { return a.n_chunks <= kFaMaxChunks; }

template <int D, int R>
static void launch_fa(const fattn_args & a, void * scratch, float * out, hipStream_t s) {
    static_assert(R >= 1 && R <= kFaMaxRows, "tile rows");
    if (a.split) {
        const int64_t prows = fa_tiles(a) * a.rows * a.n_chunks;
        float * pm = (float *) scratch;
        float * pl = pm + prows;
        char * p = (char *) (pl + prows);
        float * pa = (float *) (((uintptr_t) p + 255) & ~(uintptr_t) 255);
        if (a.split == 2) {
            // one query position: the tile rows are the g query heads (R = g)
            const int64_t units = (int64_t) a.n_chunks * a.hkv * a.n_seq;
            attn_step_args st{};
            st.fa = a;
            if (R >= 2 && a.dheads == 2) {
                constexpr int G = R >= 2 ? 2 : 1;
                hipLaunchKernelGGL((k_fattn_decode<D, false, G>), dim3((unsigned) fa_decode_grid(units * (R / G), R / G)),
                                   dim3(64), 0, s, st, pm, pl, pa);
            } else {
                hipLaunchKernelGGL((k_fattn_decode<D, false, 1>), dim3((unsigned) fa_decode_grid(units * R, R)), dim3(64),
                                   0, s, st, pm, pl, pa);
            }
        } else {
            const dim3 grid((unsigned) a.n_chunks, (unsigned) (a.hkv * a.n_seq), (unsigned) a.q_tiles);
            hipLaunchKernelGGL((k_fattn_split<D, R>), grid, dim3(kFaThreads), 0, s, a, pm, pl, pa);
        }
        launch_combine<D, R>(a, pm, pl, pa, out, s);
    } else {
        const dim3 grid(1u, (unsigned) (a.hkv * a.n_seq), (unsigned) a.q_tiles);
        hipLaunchKernelGGL((k_fattn_full<D, R>), grid, dim3(kFaThreads), 0, s, a, out);
    }
}

template <int D>
static void launch_fa_d(const fattn_args & a, void * scratch, float * out, hipStream_t s) {
    switch (a.rows) {
        case 1: launch_fa<D, 1>(a, scratch, out, s); break;
        case 2: launch_fa<D, 2>(a, scratch, out, s); break;
        case 4: launch_fa<D, 4>(a, scratch, out, s); break;
        default: launch_fa<D, 8>(a, scratch, out, s); break;
    }
}

void launch_fattn(const fattn_args & a, void * scratch, float * out, hipStream_t stream) {
    if (a.mfma) {
        launch_fattn_mfma(a, scratch, out, stream);
        return;
    }
    if (a.dec) {
        attn_step_args st{};
        st.fa = a;
        launch_fattn_dec(st, false, out, scratch, stream);
        return;
    }
    if (a.d == 128) launch_fa_d<128>(a, scratch, out, stream);
    else launch_fa_d<64>(a, scratch, out, stream);
}

}  // namespace mi355x

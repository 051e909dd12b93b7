// k_fattn_mfma.hip -- GGML_OP_FLASH_ATTN_EXT with more than one query
// position (prefill chunks, the audio encoders' self attention) at the
// default precision, on the matrix cores. Call site of the op:
// crates/openasr-core/src/ggml_runtime/cpu_graph.rs:4144-4215; the precision
// contract: Default is the backend's fastest validated implementation, F32
// ggml's full-precision contract (cpu_graph.rs:129-133, set per graph,
// models/qwen/llm_transformer.rs:3044-3053). F32 graphs and single-query
// (decode) steps keep the exact chunked form of k_fattn.hip.
//
// Arithmetic (float tolerance, the ggml GPU backends' flash attention): the
// query rows rounded to f16, S^T = K Q^T on v_mfma_f32_16x16x32_f16 (f16
// products, f32 sums), S * scale * log2(e) + mask * log2(e) in f32, an
// online softmax over 64-position tiles in f32 with exp2 (running max m, sum
// l, the output rescaled by 2^(m_old - m_new)), P rounded to f16 for
// O^T = V^T P^T on the same MFMA, out = O / l (0 for a row with no open
// position).
//
// Work: a workgroup of four waves owns 64 rows -- 64 / g queries times the
// g query heads of one kv head of one sequence -- so each K/V tile is read
// once for g heads; wave w owns rows 16 w .. 16 w + 15. MFMA operand layouts
// (16x16x32): A lane l = row l % 16, k 8 (l / 16) .. + 7; B lane l = k
// 8 (l / 16) .. + 7, column l % 16; result lane l = rows 4 (l / 16) .. + 3,
// column l % 16. The scores are computed transposed (rows = positions,
// columns = the wave's rows), so a lane holds 16 positions of one row: the
// softmax is lane-local but for two cross-lane steps, and its P values are
// the lane's own B operand of the P V product (the k slots ordered to match,
// V^T read in that order) -- P never goes through LDS. Per 64-position tile:
// K rows staged in LDS (rows padded against bank conflicts), V staged
// transposed ([dim][position]), the mask as f32.
#include <algorithm>
#include <cmath>

#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

namespace {

constexpr int kFmRows = 64;       // rows a workgroup owns
constexpr int kFmTile = 64;       // KV positions a tile
constexpr int kFmThreads = 256;
constexpr int kFmMaxSpan = 8192;  // positions one split covers (its live bits sit in LDS)
constexpr uint16_t kFmNegInf = 0xFC00u;

typedef _Float16 fm_h8 __attribute__((ext_vector_type(8)));
typedef float fm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t fm_u4 __attribute__((ext_vector_type(4)));  // 16 bytes (a native vector: copies stay in registers)

__device__ __forceinline__ fm_h8 fm_load8(const _Float16 * p) { return *(const fm_h8 *) p; }

// Mask entries pos .. pos + 7 of one mask row (f16 bits), in two steps so
// that a thread's loads issue back to back and are waited for only where the
// values are used. fm_mask_load: unconditional loads. MM (the mask form, one
// per kernel): 0 no mask (zeros); 1 16-byte rows -- the aligned 16-byte
// piece at pos, or the last piece holding an entry below n_kv when pos is
// past it (an aligned 16-byte piece holding a valid entry lies in that
// entry's page); 3 4-byte rows -- four word loads the same way; 2 other
// rows -- eight 2-byte loads, indexes clamped below n_kv. fm_mask_fix:
// positions at or past n_kv become -inf.
template <int MM>
__device__ __forceinline__ fm_u4 fm_mask_load(const uint16_t * row, int pos, int n_kv) {
    if constexpr (MM == 0) {
        return fm_u4{0, 0, 0, 0};
    } else if constexpr (MM == 1) {
        return *(const fm_u4 *) (row + min(pos, (n_kv - 1) & ~7));
    } else if constexpr (MM == 3) {
        // 4-byte rows: four word loads, clamped to the last word holding an
        // entry below n_kv (pos is even; a word holding a valid entry lies in
        // that entry's page)
        const uint32_t * w = (const uint32_t *) row;
        const int wi = pos >> 1, wl = (n_kv - 1) >> 1;
        return fm_u4{w[min(wi, wl)], w[min(wi + 1, wl)], w[min(wi + 2, wl)], w[min(wi + 3, wl)]};
    } else {
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 8; j++) h[j] = row[min(pos + j, n_kv - 1)];
        return fm_u4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
}

__device__ __forceinline__ fm_u4 fm_mask_fix(fm_u4 m, int pos, int n_kv) {
    if (pos + 8 <= n_kv) return m;
    uint32_t w[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (pos + 2 * j >= n_kv) w[j] = (w[j] & 0xFFFF0000u) | kFmNegInf;
        if (pos + 2 * j + 1 >= n_kv) w[j] = (w[j] & 0xFFFFu) | ((uint32_t) kFmNegInf << 16);
    }
    return fm_u4{w[0], w[1], w[2], w[3]};
}

// bit j set when entry j of the eight is not -inf
__device__ __forceinline__ uint32_t fm_open_bits(fm_u4 m) {
    const uint32_t w[4] = {m.x, m.y, m.z, m.w};
    uint32_t bits = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        bits |= ((w[j] & 0xFFFFu) != kFmNegInf ? 1u : 0u) << (2 * j);
        bits |= ((w[j] >> 16) != kFmNegInf ? 1u : 0u) << (2 * j + 1);
    }
    return bits;
}

}  // namespace

// Per workgroup: (1) the mask of its queries over its split of the span is
// scanned once into per-position "seen by some query" bits in LDS; tiles with
// none are skipped and V rows no query sees are staged as zeros (0 x V stays
// 0 whatever the cache holds there). (2) Live tiles are software-pipelined:
// the next live tile's K / V / mask are loaded into registers while the
// current one is on the matrix cores.
template <int D, int MM>
__global__ __launch_bounds__(kFmThreads) void k_fattn_mfma(fattn_args a, float * __restrict__ out,
                                                           float * __restrict__ part) {
    constexpr int KS = D / 32;  // k steps of the score MFMA
    constexpr int NT = D / 16;  // output column tiles
    constexpr int KP = D + 8;   // padded K row (halves)
    constexpr int VP = kFmTile + 8;
    constexpr int PC = D / 8;                                   // 16-byte pieces of a K / V row
    constexpr int KLD = kFmTile * PC / kFmThreads;              // K pieces a thread stages
    constexpr int VLD = (kFmTile / 2) * PC / kFmThreads;        // V piece pairs (two positions) a thread stages
    constexpr int MLD = kFmRows * (kFmTile / 8) / kFmThreads;   // 8-entry mask pieces a thread stages (at most)
    static_assert(KLD >= 1 && VLD >= 1 && MLD >= 1, "staging split");
    __shared__ __align__(16) _Float16 s_k[kFmTile][KP];
    __shared__ __align__(16) _Float16 s_vt[D][VP];
    __shared__ __align__(16) float s_m[kFmRows][kFmTile + 4];  // mask x log2(e), -inf kept
    __shared__ uint32_t s_open[kFmMaxSpan / 32];
    const int tid = (int) threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = a.hq / a.hkv, qpw = kFmRows / g;  // queries a workgroup
    // Workgroup b is dispatched to XCD b % 8: each XCD gets a contiguous run
    // of (query block, kv head / sequence, split) coordinates, query blocks
    // fastest, so the query blocks reading the same K / V tiles share an L2.
    const int q_blocks = (a.n_q + qpw - 1) / qpw, n_blk = (int) gridDim.x;
    int b = (int) blockIdx.x;
    if (n_blk % 8 == 0) b = (b % 8) * (n_blk / 8) + b / 8;
    const int qb = b % q_blocks, hs = (b / q_blocks) % (a.hkv * a.n_seq), z = b / (q_blocks * a.hkv * a.n_seq);
    const int kvh = hs % a.hkv, seq = hs / a.hkv;
    const int q0 = qb * qpw;
    const int nq_live = min(qpw, a.n_q - q0);
    const int kv_seq = seq / a.rk3;
    const int l16 = lane & 15, lg = lane >> 4;
    const char * kbase = a.k + (int64_t) kvh * a.k_nb2 + (int64_t) kv_seq * a.k_nb3;
    const char * vbase = a.v + (int64_t) kvh * a.v_nb2 + (int64_t) kv_seq * a.v_nb3;
    const char * mbase = MM ? a.mask + (int64_t) (seq % a.m_ne3) * a.m_nb3 : nullptr;
    auto mask_row = [&](int ql) { return (const uint16_t *) (mbase + (int64_t) (q0 + ql) * a.m_nb1); };
    // this workgroup's share of the span: tiles [t_begin, t_end) of split z
    const int n_tiles = (a.n_kv + kFmTile - 1) / kFmTile;
    const int per = (n_tiles + a.mfma_split - 1) / a.mfma_split;
    const int t_begin = z * per, t_end = min(n_tiles, t_begin + per);
    const int span0 = t_begin * kFmTile;

    // registers for one tile in flight
    fm_u4 kr[KLD], vr[VLD][2], mr[MLD];
    auto issue = [&](int tile) {
        const int p0 = tile * kFmTile;
        // every load unconditional (rows clamped into the span, the result
        // selected after), so they issue back to back
#pragma unroll
        for (int i = 0; i < KLD; i++) {
            const int e = tid + i * kFmThreads, p = e / PC, piece = e % PC;
            kr[i] = *(const fm_u4 *) (kbase + (int64_t) min(p0 + p, a.n_kv - 1) * a.k_nb1 + 16 * piece);
        }
#pragma unroll
        for (int i = 0; i < VLD; i++) {
            const int e = tid + i * kFmThreads, pair = e % (kFmTile / 2), piece = e / (kFmTile / 2);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int p = p0 + 2 * pair + h;
                vr[i][h] = *(const fm_u4 *) (vbase + (int64_t) min(p, a.n_kv - 1) * a.v_nb1 + 16 * piece);
            }
        }
#pragma unroll
        for (int i = 0; i < MLD; i++) {
            const int e = tid + i * kFmThreads, ql = e >> 3, c = e & 7;
            mr[i] = fm_mask_load<MM>(mask_row(min(ql, nq_live - 1)), p0 + 8 * c, a.n_kv);
        }
        // positions past the span: their K rows (copies of the last) meet a
        // -inf mask, their V rows are not open (staged as zeros)
    };
    // the split's first tile goes out with the query rows and the mask scan
    // (one memory round trip for all three)
    issue(t_begin);

    // this lane's query row (the score MFMA's A operand): row 16 wave + l16,
    // dims 8 lg .. + 7 of each 32-dim step, f16-rounded
    const int q_row = 16 * wave + l16;
    const bool q_live = q0 + q_row / g < a.n_q;
    float qv[KS][8];
    {
        const float * qp = (const float *) (a.q + (int64_t) (q_live ? q0 + q_row / g : 0) * a.q_nb1 +
                                            (int64_t) (kvh * g + q_row % g) * a.q_nb2 + (int64_t) seq * a.q_nb3);
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
#pragma unroll
            for (int j = 0; j < 8; j++) qv[kk][j] = qp[32 * kk + 8 * lg + j];  // a row of query 0 for a dead row
        }
    }

    // (1) positions of the split some query of the workgroup sees
    const int words = (t_end - t_begin) * (kFmTile / 32);
    for (int w = tid; w < words; w += kFmThreads) s_open[w] = 0;
    __syncthreads();
    {
        const int pieces = (t_end - t_begin) * (kFmTile / 8);  // 8-position pieces of a row
        const int total = nq_live * pieces;
        for (int e0 = tid; e0 < total; e0 += 4 * kFmThreads) {
            fm_u4 raw[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int e = min(e0 + u * kFmThreads, total - 1);
                raw[u] = fm_mask_load<MM>(mask_row(e / pieces), span0 + 8 * (e % pieces), a.n_kv);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int e = e0 + u * kFmThreads, c = e % pieces;
                if (e >= total) continue;
                const uint32_t bits = fm_open_bits(fm_mask_fix(raw[u], span0 + 8 * c, a.n_kv));
                if (bits) atomicOr(&s_open[c >> 2], bits << (8 * (c & 3)));
            }
        }
    }
    __syncthreads();
    auto tile_open = [&](int t) {
        const int w = (t - t_begin) * (kFmTile / 32);
        return (s_open[w] | s_open[w + 1]) != 0;
    };
    auto next_open = [&](int t) {
        while (t < t_end && !tile_open(t)) t++;
        return t;
    };

    // scores are taken to base-2 exponent units in f32 (exp2 on the softmax
    // side): s = S * scale * log2(e) + mask * log2(e)
    const float qscale = a.scale * 1.4426950408889634f;
    fm_h8 qa[KS];
#pragma unroll
    for (int kk = 0; kk < KS; kk++) {
#pragma unroll
        for (int j = 0; j < 8; j++) qa[kk][j] = q_live ? (_Float16) qv[kk][j] : (_Float16) 0.0f;
    }
    // this lane's row (query / head pair): 16 wave + l16; its running max,
    // sum and O^T columns (dims 16 ct + 4 lg + i)
    float m = -INFINITY, l = 0.0f;
    fm_f4 o[NT];
#pragma unroll
    for (int ct = 0; ct < NT; ct++) o[ct] = fm_f4{0.f, 0.f, 0.f, 0.f};

    // (2) the pipeline over the open tiles
    auto stage = [&](int tile) {
        const int rel = tile * kFmTile - span0;
#pragma unroll
        for (int i = 0; i < KLD; i++) {
            const int e = tid + i * kFmThreads, p = e / PC, piece = e % PC;
            *(fm_u4 *) &s_k[p][8 * piece] = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VLD; i++) {
            const int e = tid + i * kFmThreads, pair = e % (kFmTile / 2), piece = e / (kFmTile / 2);
            const int pr = rel + 2 * pair;  // even: both positions in one word
            const uint32_t open = s_open[pr >> 5] >> (pr & 31);
            const fm_u4 v0 = (open & 1u) ? vr[i][0] : fm_u4{0, 0, 0, 0};
            const fm_u4 v1 = (open & 2u) ? vr[i][1] : fm_u4{0, 0, 0, 0};
            const uint32_t w0[4] = {v0.x, v0.y, v0.z, v0.w}, w1[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                *(uint32_t *) &s_vt[8 * piece + 2 * j][2 * pair] = (w0[j] & 0xFFFFu) | (w1[j] << 16);
                *(uint32_t *) &s_vt[8 * piece + 2 * j + 1][2 * pair] = (w0[j] >> 16) | (w1[j] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int i = 0; i < MLD; i++) {
            const int e = tid + i * kFmThreads, ql = e >> 3, c = e & 7;
            if (ql >= qpw) continue;
            const fm_u4 mh = ql < nq_live ? fm_mask_fix(mr[i], tile * kFmTile + 8 * c, a.n_kv)
                                          : fm_u4{0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u};
            fm_f4 lo, hi;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t w = mh[j];
                const float e0 = half_bits_to_float((uint16_t) (w & 0xFFFFu)), e1 = half_bits_to_float((uint16_t) (w >> 16));
                const float f0 = e0 * 1.4426950408889634f, f1 = e1 * 1.4426950408889634f;
                if (j < 2) {
                    lo[2 * j] = f0;
                    lo[2 * j + 1] = f1;
                } else {
                    hi[2 * j - 4] = f0;
                    hi[2 * j - 3] = f1;
                }
            }
            *(fm_f4 *) &s_m[ql][8 * c] = lo;
            *(fm_f4 *) &s_m[ql][8 * c + 4] = hi;
        }
    };

    int tile = next_open(t_begin);
    if (tile < t_end && tile != t_begin) issue(tile);  // the first tile was not open
    while (tile < t_end) {
        __syncthreads();  // the previous tile's LDS reads are done
        stage(tile);
        __syncthreads();
        const int nxt = next_open(tile + 1);
        if (nxt < t_end) issue(nxt);
        // S^T = K Q^T for the tile's 64 positions and the wave's 16 rows:
        // lane (lg, l16) gets positions 16 t + 4 lg + i of row l16 (k steps
        // outer: four independent accumulations in flight)
        fm_f4 sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) sc[t] = fm_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KS; kk++) {
            fm_h8 kb[4];
#pragma unroll
            for (int t = 0; t < 4; t++) kb[t] = fm_load8(&s_k[16 * t + l16][32 * kk + 8 * lg]);
#pragma unroll
            for (int t = 0; t < 4; t++) sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[t], qa[kk], sc[t], 0, 0, 0);
        }
        // mask and online softmax of the lane's row: 16 of its 64 values in
        // the lane, the rest in lanes l16 + 16, + 32, + 48
        const int ql = (16 * wave + l16) / g;
        float sv[4][4], mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const fm_f4 mk = *(const fm_f4 *) &s_m[ql][16 * t + 4 * lg];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[t][i] = mk[i] == -INFINITY ? -INFINITY : fmaf(sc[t][i], qscale, mk[i]);
                mx = fmaxf(mx, sv[t][i]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float base = mn == -INFINITY ? 0.0f : mn;  // a row with nothing open yet
        const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - base);
        // P^T in registers as the P V product's B operand: k slot 8 lg + j of
        // step kk holds position 32 kk + 16 (j / 4) + 4 lg + j % 4 -- this
        // lane's own values; V^T is read in the same order
        fm_h8 pb[kFmTile / 32];
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv = sv[t][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[t][i] - base);
                const _Float16 ph = (_Float16) pv;
                ps += (float) ph;
                pb[t >> 1][4 * (t & 1) + i] = ph;
            }
        }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        l = l * alpha + ps;
        m = mn;
        // rescale the accumulators only when some row's maximum moved
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int ct = 0; ct < NT; ct++) o[ct] *= alpha;
        }
        // O^T += V^T P^T: A lane (lg, l16) = dim 16 ct + l16 at the k slots'
        // positions, two 4-position runs of V^T
#pragma unroll
        for (int kk = 0; kk < kFmTile / 32; kk++) {
#pragma unroll
            for (int ct = 0; ct < NT; ct++) {
                const _Float16 * vrow = &s_vt[16 * ct + l16][32 * kk + 4 * lg];
                typedef _Float16 fm_h4 __attribute__((ext_vector_type(4)));
                const fm_h4 v0 = *(const fm_h4 *) vrow, v1 = *(const fm_h4 *) (vrow + 16);
                const fm_h8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                o[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[kk], o[ct], 0, 0, 0);
            }
        }
        tile = nxt;
    }
    if (a.mfma_split > 1) {
        // partials of split z: O unnormalised, then (m, l), per workgroup row
        const int64_t blk = (int64_t) hs * q_blocks + qb;
        const int64_t all_rows = (int64_t) n_blk * kFmRows;
        const int64_t pr = (blk * a.mfma_split + z) * kFmRows + 16 * wave + l16;
#pragma unroll
        for (int ct = 0; ct < NT; ct++) *(fm_f4 *) &part[pr * D + 16 * ct + 4 * lg] = o[ct];
        if (lg == 0) {
            part[all_rows * D + 2 * pr] = m;
            part[all_rows * D + 2 * pr + 1] = l;
        }
        return;
    }
    // out = O / l, ggml's [D, hq, n_q, n_seq] layout
    const int r = 16 * wave + l16, i = q0 + r / g;
    if (i >= a.n_q) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float * op = out + (((int64_t) seq * a.n_q + i) * a.hq + kvh * g + r % g) * D;
#pragma unroll
    for (int ct = 0; ct < NT; ct++) *(fm_f4 *) &op[16 * ct + 4 * lg] = o[ct] * inv;
}

// the splits of a workgroup row: M = max m_s, L = sum l_s exp(m_s - M),
// out = sum O_s exp(m_s - M) / L (0 for a row with no live position).
// 256 threads: 256 / D rows, one dim a thread.
template <int D>
__global__ __launch_bounds__(kFmThreads) void k_fattn_mfma_combine(fattn_args a, const float * __restrict__ part,
                                                                   float * __restrict__ out, int q_blocks) {
    constexpr int RW = kFmThreads / D;
    const int dim = (int) threadIdx.x % D;
    const int64_t row = (int64_t) blockIdx.x * RW + (int) threadIdx.x / D;  // over blk * kFmRows
    const int64_t n_blk = (int64_t) q_blocks * a.hkv * a.n_seq;
    if (row >= n_blk * kFmRows) return;
    const int64_t blk = row / kFmRows;
    const int r = (int) (row % kFmRows);
    const int g = a.hq / a.hkv, qpw = kFmRows / g;
    const int bx = (int) (blk % q_blocks), by = (int) (blk / q_blocks);
    const int kvh = by % a.hkv, seq = by / a.hkv;
    const int i = bx * qpw + r / g, head = kvh * g + r % g;
    if (i >= a.n_q) return;
    const int ns = a.mfma_split;
    const int64_t all_rows = n_blk * ns * kFmRows;
    const float * ml = part + all_rows * D;
    // batches of kB splits: every load of a batch is requested before any is
    // used (indexes clamped to the last split, the extra terms masked), so a
    // batch costs one memory round trip
    constexpr int kB = 16;
    float mx = -INFINITY;
    for (int z0 = 0; z0 < ns; z0 += kB) {
        float mz[kB];
#pragma unroll
        for (int k = 0; k < kB; k++) mz[k] = ml[2 * ((blk * ns + min(z0 + k, ns - 1)) * kFmRows + r)];
#pragma unroll
        for (int k = 0; k < kB; k++) mx = z0 + k < ns ? fmaxf(mx, mz[k]) : mx;
    }
    float L = 0.0f, acc = 0.0f;
    if (mx != -INFINITY) {
        for (int z0 = 0; z0 < ns; z0 += kB) {
            float mz[kB], lz[kB], oz[kB];
#pragma unroll
            for (int k = 0; k < kB; k++) {
                const int64_t pr = (blk * ns + min(z0 + k, ns - 1)) * kFmRows + r;
                mz[k] = ml[2 * pr];
                lz[k] = ml[2 * pr + 1];
                oz[k] = part[pr * D + dim];
            }
#pragma unroll
            for (int k = 0; k < kB; k++) {
                if (z0 + k >= ns || mz[k] == -INFINITY) continue;
                const float w = __builtin_amdgcn_exp2f(mz[k] - mx);  // maxima in base-2 exponent units
                L += lz[k] * w;
                acc += oz[k] * w;
            }
        }
    }
    out[(((int64_t) seq * a.n_q + i) * a.hq + head) * D + dim] = L > 0.0f ? acc / L : 0.0f;
}

static int fm_q_blocks(const fattn_args & a) {
    const int qpw = kFmRows / (a.hq / a.hkv);
    return (a.n_q + qpw - 1) / qpw;
}

void fattn_mfma_plan(fattn_args & a, int n_cu) {
    // split the span when one sequence's query blocks leave CUs idle: up to
    // two workgroups a CU (their LDS and registers fit twice), at least four
    // tiles a split. Planned from one sequence's shape, so a sequence's rows
    // get the same bits batched or alone.
    const int64_t base = (int64_t) fm_q_blocks(a) * a.hkv;
    const int n_tiles = (a.n_kv + kFmTile - 1) / kFmTile;
    int split = 1;
    if (base < 2 * n_cu) split = (int) std::min<int64_t>((2 * n_cu + base - 1) / base, std::max(1, n_tiles / 4));
    // a split covers at most kFmMaxSpan positions (its live bits in LDS)
    split = std::max(split, (n_tiles + kFmMaxSpan / kFmTile - 1) / (kFmMaxSpan / kFmTile));
    // no empty split: every split owns at least one tile
    const int per = (n_tiles + split - 1) / split;
    a.mfma_split = (n_tiles + per - 1) / per;
}

size_t fattn_mfma_scratch_bytes(const fattn_args & a) {
    if (a.mfma_split <= 1) return 0;
    const int64_t rows = (int64_t) fm_q_blocks(a) * a.hkv * a.n_seq * a.mfma_split * kFmRows;
    return (size_t) rows * (a.d + 2) * sizeof(float);
}

bool fattn_mfma_supported(const fattn_args & a) {
    const int g = a.hkv > 0 ? a.hq / a.hkv : 0;
    // K / V rows, heads and sequences start on 16 bytes (16-byte row loads)
    const bool aligned = (a.k_nb1 | a.k_nb2 | a.k_nb3 | a.v_nb1 | a.v_nb2 | a.v_nb3) % 16 == 0;
    // one mask row for every head (the planner's FLASH_ATTN_EXT contract)
    return (a.d == 64 || a.d == 128) && a.n_q > 1 && g >= 1 && g <= 8 && kFmRows % g == 0 && a.n_kv > 0 && aligned &&
           (!a.mask || a.m_ne2 == 1);
}

void launch_fattn_mfma(const fattn_args & a, void * scratch, float * out, hipStream_t s) {
    const int qb = fm_q_blocks(a);
    const dim3 grid((unsigned) (qb * a.hkv * a.n_seq * std::max(1, a.mfma_split)));
    float * part = (float *) scratch;
    const uintptr_t mal = (uintptr_t) a.mask | (uintptr_t) a.m_nb1 | (uintptr_t) a.m_nb3;
    const int mm = !a.mask ? 0 : (mal & 15) == 0 ? 1 : (mal & 3) == 0 ? 3 : 2;
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kFmThreads), 0, s, a, out, part); };
    if (a.d == 128) {
        if (mm == 0) go(k_fattn_mfma<128, 0>);
        else if (mm == 1) go(k_fattn_mfma<128, 1>);
        else if (mm == 3) go(k_fattn_mfma<128, 3>);
        else go(k_fattn_mfma<128, 2>);
    } else {
        if (mm == 0) go(k_fattn_mfma<64, 0>);
        else if (mm == 1) go(k_fattn_mfma<64, 1>);
        else if (mm == 3) go(k_fattn_mfma<64, 3>);
        else go(k_fattn_mfma<64, 2>);
    }
    note_hip_error(hipGetLastError());
    if (a.mfma_split > 1) {
        const int64_t rows = (int64_t) qb * a.hkv * a.n_seq * kFmRows;
        const int rw = kFmThreads / a.d;
        const unsigned wgs = (unsigned) ((rows + rw - 1) / rw);
        if (a.d == 128) hipLaunchKernelGGL(k_fattn_mfma_combine<128>, dim3(wgs), dim3(kFmThreads), 0, s, a, part, out, qb);
        else hipLaunchKernelGGL(k_fattn_mfma_combine<64>, dim3(wgs), dim3(kFmThreads), 0, s, a, part, out, qb);
        note_hip_error(hipGetLastError());
    }
}

}  // namespace mi355x

// k_fattn_dec.hip -- GGML_OP_FLASH_ATTN_EXT with one query position (the
// decode step) at the default precision. Call site of the op:
// crates/openasr-core/src/ggml_runtime/cpu_graph.rs:4144-4215; the
// transcription decoders build it with GgmlFlashAttentionPrecision::Default
// (models/qwen/llm_transformer.rs:2748, 2999; nn/decoder.rs:3064-3728), the
// contract under which a backend runs its fastest validated form
// (cpu_graph.rs:129-133). GGML_PREC_F32 keeps the exact chunked form of
// k_fattn.hip.
//
// Arithmetic (float tolerance, like the ggml GPU backends' vector flash
// attention): the query rows rounded to f16; S^T = K q^T on
// v_mfma_f32_16x16x32_f16 (f16 products, f32 sums; the kv head's g query
// heads are the B operand's columns); s = S * scale * log2(e) + mask *
// log2(e) in f32; an online softmax over 64-position tiles with exp2 (running
// max m, sum l, output rescaled by 2^(m_old - m_new)); P * V in f32 (each f16
// V element widened inside its fused multiply-add); the waves' states merged
// in the workgroup; out = O / l (0 for a query with no open position).
// Masked positions are dropped outright: their scores are -inf and their V
// rows read as zeros (a cache row past the written ones may hold anything).
//
// Work: one workgroup of eight waves per (sequence, kv head, KV split), all
// g query heads of the kv head together, so a decode step's attention is one
// launch: the exact form's one-wave chunks need a second launch to combine,
// and a kernel boundary plus that launch cost more than the whole attention
// here. A split covers up to 16 tiles of 64 positions (1024); wave w takes
// the split's tiles w and w + 8. A wave reads its tiles' mask entries first
// (lane = position) and skips a tile with no open position without touching
// K / V. Longer spans split; each split writes (max, sum, unnormalised
// output) in the chunk-partial form k_fattn_combine merges.
//
// Layouts (MFMA 16x16x32: A lane l = row l % 16, k 8 (l / 16) .. + 7; B lane
// l = k 8 (l / 16) .. + 7, column l % 16; result lane l = rows 4 (l / 16) ..
// + 3, column l % 16): K rows are the A operand straight from memory (lane l:
// row 16 b + l % 16 of the tile, dims 32 s + 8 (l / 16) .. + 7, one 16-byte
// load), the query heads the B operand. For P * V lane l owns dims
// 8 (l % LPR) .. + 7 (LPR = D / 8 lanes a row) of the tile rows u RPI +
// l / LPR (RPI = 64 / LPR rows a load), the p values read back from a
// per-wave LDS row ordered to match; the row groups' partial sums are added
// across lanes once, after the last tile.
//
// STEP (the fused decode step, D = 128): every wave normalises and rotates
// the query rows (QK-norm * w, NEOX RoPE by the step's rope table); the wave
// whose tile holds this step's position also forms the new K row (same) and
// V row, puts them in its K / V registers in place of the cache row, and
// writes them into the f16 caches (SET_ROWS) after its reads. No other wave
// of the launch reads that cache row.
#include <algorithm>
#include <cmath>

#include "../fattn_dev.h"
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

namespace {

constexpr int kFdWaves = 8;
constexpr int kFdThreads = 64 * kFdWaves;
constexpr int kFdTile = 64;                                // positions a tile
constexpr int kFdSplitTiles = 16;                          // tiles a split
constexpr int kFdTilesPerWave = kFdSplitTiles / kFdWaves;  // 2
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;

typedef _Float16 fd_h8 __attribute__((ext_vector_type(8)));
typedef float fd_f4 __attribute__((ext_vector_type(4)));

struct fd_scores {
    fd_f4 v[4];  // lane l: positions 16 b + 4 (l / 16) + i of the tile, head l % 16
};

__device__ __forceinline__ fd_h8 fd_as_h8(const uint4 & u) { return __builtin_bit_cast(fd_h8, u); }

// 8 floats rounded to f16, packed
__device__ __forceinline__ uint4 fd_pack8(const float (&f)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = (uint32_t) float_to_half_bits(f[2 * i]) | ((uint32_t) float_to_half_bits(f[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// x = m ? y : x bit by bit (m all ones or zero): arithmetic, not a select,
// so that the registers of x never become a memory slot picked by address
__device__ __forceinline__ void fd_merge(uint4 & x, const uint4 & y, uint32_t m) {
    x.x = (x.x & ~m) | (y.x & m);
    x.y = (x.y & ~m) | (y.y & m);
    x.z = (x.z & ~m) | (y.z & m);
    x.w = (x.w & ~m) | (y.w & m);
}

__device__ __forceinline__ void fd_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D>
struct fd_shape {
    static constexpr int KS = D / 32;            // k steps of the score product
    static constexpr int LPR = D / 8;            // lanes a V row (8 dims a lane)
    static constexpr int RPI = 64 / LPR;         // V rows a load instruction
    static constexpr int NV = kFdTile / RPI;     // V load instructions a tile
};

// one tile's K (A operands) and V rows in registers
template <int D>
struct fd_tile_regs {
    uint4 k[4][fd_shape<D>::KS];
    uint4 v[fd_shape<D>::NV];
};

template <int D>
__device__ __forceinline__ void fd_load_k(const char * kb, int64_t k_nb1, int pos0, int n_kv, int lane,
                                          fd_tile_regs<D> & r) {
    using S = fd_shape<D>;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int row = min(pos0 + 16 * b + (lane & 15), n_kv - 1);
        const char * kr = kb + (int64_t) row * k_nb1 + 16 * (lane >> 4);
#pragma unroll
        for (int s = 0; s < S::KS; s++) r.k[b][s] = *(const uint4 *) (kr + 64 * s);
    }
}

template <int D>
__device__ __forceinline__ void fd_load_v(const char * vb, int64_t v_nb1, int pos0, int n_kv, int lane,
                                          fd_tile_regs<D> & r) {
    using S = fd_shape<D>;
#pragma unroll
    for (int u = 0; u < S::NV; u++) {
        const int row = min(pos0 + u * S::RPI + lane / S::LPR, n_kv - 1);
        r.v[u] = *(const uint4 *) (vb + (int64_t) row * v_nb1 + 16 * (lane % S::LPR));
    }
}

// position p of a tile in the per-wave p row: the order the P * V lanes read
template <int D>
__device__ __forceinline__ int fd_pidx(int p) {
    using S = fd_shape<D>;
    return (p % S::RPI) * S::NV + p / S::RPI;
}

template <int D, int G, bool STEP>
__global__ __launch_bounds__(kFdThreads) void k_fattn_dec(attn_step_args st, float * __restrict__ out,
                                                          float * __restrict__ part) {
    using S = fd_shape<D>;
    static_assert(!STEP || D == 128, "the step form handles 128-wide heads");
    static_assert(G == 1 || G == 2 || G == 4, "query heads a kv head");
    __shared__ __align__(16) float s_mask[kFdWaves][kFdTile];    // per wave: the tile's mask * log2(e)
    __shared__ __align__(16) float s_p[kFdWaves][G][kFdTile];    // per wave: the tile's p values
    __shared__ __align__(16) uint16_t s_q[kFdWaves][G][D];       // per wave: the f16 query rows
    __shared__ __align__(16) uint16_t s_new[2][D];               // STEP: the new K and V rows (f16)
    __shared__ float s_wm[kFdWaves][G], s_wl[kFdWaves][G];
    __shared__ __align__(16) float s_wacc[kFdWaves][G][D];
    __shared__ __align__(16) float s_out[G * D];
    const fattn_args & a = st.fa;
    const int lane = (int) threadIdx.x & 63, w = (int) threadIdx.x >> 6;
    const int nsp = a.dec;
    const int sp = (int) blockIdx.x % nsp, pair = (int) blockIdx.x / nsp;
    const int kvh = pair % a.hkv, seq = pair / a.hkv;
    const int head0 = kvh * G;
    const int kv_seq = seq / a.rk3;
    const int n_tiles = (a.n_kv + kFdTile - 1) / kFdTile;
    const int t0 = sp * kFdSplitTiles, t1 = min(n_tiles, t0 + kFdSplitTiles);
    const char * kb = a.k + (int64_t) kvh * a.k_nb2 + (int64_t) kv_seq * a.k_nb3;
    const char * vb = a.v + (int64_t) kvh * a.v_nb2 + (int64_t) kv_seq * a.v_nb3;

    // the mask entries of this wave's tiles (lane = position); every load
    // unconditional (a null mask reads the K cache's first row and drops it)
    const uint16_t * mrow = a.mask ? (const uint16_t *) (a.mask + (int64_t) (seq % a.m_ne3) * a.m_nb3)
                                   : (const uint16_t *) a.k;
    float mv[kFdTilesPerWave];
#pragma unroll
    for (int k = 0; k < kFdTilesPerWave; k++) {
        const int tile = t0 + w + k * kFdWaves;
        const int pos = tile * kFdTile + lane;
        const uint16_t raw = mrow[min(pos, a.n_kv - 1)];
        const float m = a.mask ? half_bits_to_float(raw) : 0.0f;
        mv[k] = tile < t1 && pos < a.n_kv ? m : -INFINITY;
    }
    // STEP: the query, new K and V rows' inputs, requested with the mask
    float qx0[G], qx1[G], qw0 = 0.0f, qw1 = 0.0f, kx0 = 0.0f, kx1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f, vx0 = 0.0f,
                                vx1 = 0.0f;
    float2 qcs = make_float2(0.0f, 0.0f);
    int64_t r_new = -1;
    float qp[S::KS][8];  // plain form: this lane's query elements (B operand)
    if constexpr (STEP) {
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
        const char * ip = st.idx + (int64_t) (kvh % st.idx_ne1) * st.idx_nb1 + (int64_t) (seq % st.idx_ne2) * st.idx_nb2;
        const uint32_t lo = *(const uint32_t *) ip, hi = *(const uint32_t *) (ip + (st.idx_i64 ? 4 : 0));
        r_new = st.idx_i64 ? (int64_t) (((uint64_t) hi << 32) | lo) : (int64_t) (int32_t) lo;
    } else {
        const int hl = (lane & 15) < G ? (lane & 15) : 0;
        const float * qr = (const float *) (a.q + (int64_t) (head0 + hl) * a.q_nb2 + (int64_t) seq * a.q_nb3);
#pragma unroll
        for (int s = 0; s < S::KS; s++)
#pragma unroll
            for (int i = 0; i < 8; i++) qp[s][i] = qr[32 * s + 8 * (lane >> 4) + i];
    }
    // the wave's first tile (tile w of the split: open in any decode step past
    // 64 w positions) is requested before its mask entries arrive; if none of
    // them is open the rows are dropped
    fd_tile_regs<D> r;
    const int pos_of[kFdTilesPerWave] = {(t0 + w) * kFdTile, (t0 + w + kFdWaves) * kFdTile};
    static_assert(kFdTilesPerWave == 2, "two tiles a wave");
    const bool in0 = t0 + w < t1;
    if (in0) {
        fd_load_k<D>(kb, a.k_nb1, pos_of[0], a.n_kv, lane, r);
        fd_load_v<D>(vb, a.v_nb1, pos_of[0], a.n_kv, lane, r);
    }
    uint64_t lb[kFdTilesPerWave];
#pragma unroll
    for (int k = 0; k < kFdTilesPerWave; k++) lb[k] = __ballot(mv[k] != -INFINITY);

    // STEP: the wave whose tiles hold this step's position (the cache row it
    // replaces): its tile k_new and row jn
    int k_new = -1, jn = 0;
    uint16_t knew0 = 0, knew1 = 0, vnew0 = 0, vnew1 = 0;
    uint4 qb[S::KS];
    if constexpr (STEP) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            float y0, y1;
            as_norm_rope(qx0[h], qx1[h], qw0, qw1, qcs, st.q_eps, y0, y1);
            s_q[w][h][lane] = float_to_half_bits(y0);
            s_q[w][h][lane + 64] = float_to_half_bits(y1);
        }
        if (r_new >= 0 && r_new < a.n_kv) {
            const int tn = (int) (r_new / kFdTile);
            if (tn >= t0 && tn < t1 && (tn - t0) % kFdWaves == w) {
                k_new = (tn - t0) / kFdWaves;
                jn = (int) (r_new - (int64_t) tn * kFdTile);
                float y0, y1;
                as_norm_rope(kx0, kx1, kw0, kw1, qcs, st.k_eps, y0, y1);
                knew0 = float_to_half_bits(y0);
                knew1 = float_to_half_bits(y1);
                vnew0 = float_to_half_bits(vx0);
                vnew1 = float_to_half_bits(vx1);
                s_new[0][lane] = knew0;
                s_new[0][lane + 64] = knew1;
                s_new[1][lane] = vnew0;
                s_new[1][lane + 64] = vnew1;
            }
        }
        fd_wave_sync();
        const int hl = lane & 15;
#pragma unroll
        for (int s = 0; s < S::KS; s++) {
            const uint4 v = *(const uint4 *) &s_q[w][hl < G ? hl : 0][32 * s + 8 * (lane >> 4)];
            qb[s] = hl < G ? v : make_uint4(0, 0, 0, 0);
        }
    } else {
        const bool hv = (lane & 15) < G;
#pragma unroll
        for (int s = 0; s < S::KS; s++) {
            float f[8];
#pragma unroll
            for (int i = 0; i < 8; i++) f[i] = hv ? qp[s][i] : 0.0f;
            qb[s] = fd_pack8(f);
        }
    }

    const float scl2 = a.scale * kLog2e;
    float m_run = -INFINITY, l_run = 0.0f;  // lanes l % 16 == h: head h's state
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < 8; i++) acc[h][i] = 0.0f;

    // one tile: its K rows (with this step's row in place) against the
    // queries, the online softmax, then P * V. The next tile's K is requested
    // once this tile's scores are formed and its V once the P * V is done (the
    // registers are reused), so its rows arrive under this tile's arithmetic.
    auto tile_scores = [&](int k) {
        s_mask[w][lane] = mv[k] * kLog2e;  // -inf stays -inf
        if constexpr (STEP) {
            if (k == k_new) {
                // this step's K row in place of the cache row jn. The register
                // each lane replaces is picked by a bit mask the compiler
                // cannot see through: a select on "b == jn / 16" becomes an
                // indexed store, which puts the whole tile in scratch memory
                uint32_t kbits = (lane & 15) == (jn & 15) ? 1u << (jn >> 4) : 0u;
                asm volatile("" : "+v"(kbits));
#pragma unroll
                for (int s = 0; s < S::KS; s++) {
                    const uint4 nv = *(const uint4 *) &s_new[0][32 * s + 8 * (lane >> 4)];
#pragma unroll
                    for (int b = 0; b < 4; b++) fd_merge(r.k[b][s], nv, 0u - ((kbits >> b) & 1u));
                }
            }
        }
        fd_wave_sync();
        // scores: S^T = K q^T, lane l: positions 16 b + 4 (l / 16) + i of head l % 16
        fd_scores sc;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            sc.v[b] = fd_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < S::KS; s++)
                sc.v[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fd_as_h8(r.k[b][s]), fd_as_h8(qb[s]), sc.v[b], 0, 0, 0);
        }
        return sc;
    };
    auto tile_softmax_pv = [&](int k, const fd_scores & sc) {
        float sv[4][4];
        float tmax = -INFINITY;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const fd_f4 mk = *(const fd_f4 *) &s_mask[w][16 * b + 4 * (lane >> 4)];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[b][i] = mk[i] == -INFINITY ? -INFINITY : fmaf(sc.v[b][i], scl2, mk[i]);
                tmax = fmaxf(tmax, sv[b][i]);
            }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float base = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - base);
        float tsum = 0.0f;
        const int hl = lane & 15;
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = sv[b][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[b][i] - base);
                tsum += p;
                if (hl < G) s_p[w][hl][fd_pidx<D>(16 * b + 4 * (lane >> 4) + i)] = p;
            }
        tsum += __shfl_xor(tsum, 16);
        tsum += __shfl_xor(tsum, 32);
        l_run = l_run * alpha + tsum;
        m_run = m_new;
        if constexpr (STEP) {
            if (k == k_new) {  // this step's V row in place of the cache row jn
                uint32_t vbits = lane / S::LPR == jn % S::RPI ? 1u << (jn / S::RPI) : 0u;
                asm volatile("" : "+v"(vbits));
                const uint4 nv = *(const uint4 *) &s_new[1][8 * (lane % S::LPR)];
#pragma unroll
                for (int u = 0; u < S::NV; u++) fd_merge(r.v[u], nv, 0u - ((vbits >> u) & 1u));
            }
        }
        if (lb[k] != ~0ull) {
            // V rows of closed positions read as zeros (p is 0 there, and the
            // row may hold anything)
#pragma unroll
            for (int u = 0; u < S::NV; u++) {
                const uint32_t open = 0u - (uint32_t) ((lb[k] >> (u * S::RPI + lane / S::LPR)) & 1);
                fd_merge(r.v[u], make_uint4(0, 0, 0, 0), ~open);
            }
        }
        fd_wave_sync();
        // P * V: lane = dims 8 (l % LPR) .. + 7 of rows u RPI + l / LPR
        const int rg = lane / S::LPR;
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float ah = __shfl(alpha, h);
#pragma unroll
            for (int i = 0; i < 8; i++) acc[h][i] *= ah;
            const float * ph = &s_p[w][h][rg * S::NV];
#pragma unroll
            for (int u0 = 0; u0 < S::NV; u0 += 4) {
                const fd_f4 pp = *(const fd_f4 *) (ph + u0);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint4 vv = r.v[u0 + j];
                    const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[h][2 * i] = fmaf(pp[j], half_bits_to_float((uint16_t) (vw[i] & 0xFFFF)), acc[h][2 * i]);
                        acc[h][2 * i + 1] = fmaf(pp[j], half_bits_to_float((uint16_t) (vw[i] >> 16)), acc[h][2 * i + 1]);
                    }
                }
            }
        }
    };
    if (lb[0]) {
        const auto sc = tile_scores(0);
        tile_softmax_pv(0, sc);
    }
    if (lb[1]) {
        fd_load_k<D>(kb, a.k_nb1, pos_of[1], a.n_kv, lane, r);
        fd_load_v<D>(vb, a.v_nb1, pos_of[1], a.n_kv, lane, r);
    }
    if (lb[1]) {
        const auto sc = tile_scores(1);
        tile_softmax_pv(1, sc);
    }
    // the row groups' sums of each dim, then the wave's state into LDS
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int off = S::LPR; off < 64; off <<= 1) acc[h][i] += __shfl_xor(acc[h][i], off);
    if (lane < S::LPR) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            *(fd_f4 *) &s_wacc[w][h][8 * lane] = fd_f4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
            *(fd_f4 *) &s_wacc[w][h][8 * lane + 4] = fd_f4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
        }
    }
    if (lane < G) {
        s_wm[w][lane] = m_run;
        s_wl[w][lane] = l_run;
    }
    __syncthreads();
    // the workgroup's merge: thread t = head t / D, dim t % D
    const int t = (int) threadIdx.x;
    if (t < G * D) {
        const int h = t / D, d = t % D;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < kFdWaves; v++) M = fmaxf(M, s_wm[v][h]);
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int v = 0; v < kFdWaves; v++) {
                const float mw = s_wm[v][h];
                const float c = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
                L = fmaf(c, s_wl[v][h], L);
                O = fmaf(c, s_wacc[v][h][d], O);
            }
        }
        if (nsp == 1) {
            const float o = L > 0.0f ? O / L : 0.0f;
            if (out) out[((int64_t) seq * a.hq + head0 + h) * D + d] = o;
            s_out[t] = o;
        } else {
            // the chunk-partial form of k_fattn_combine: natural-log maxima
            const int64_t prow = (int64_t) pair * G + h;
            float * pm = part;
            float * pl = pm + (int64_t) a.n_seq * a.hkv * G * nsp;
            float * pa = (float *) (((uintptr_t) (pl + (int64_t) a.n_seq * a.hkv * G * nsp) + 255) & ~(uintptr_t) 255);
            pa[(prow * nsp + sp) * D + d] = O;
            if (d == 0) {
                pm[prow * nsp + sp] = M == -INFINITY ? -INFINITY : M * kLn2;
                pl[prow * nsp + sp] = L;
            }
        }
    }
    if (nsp == 1 && a.qtype >= 0) {
        __syncthreads();
        fa_tile tt{};
        tt.kvh = kvh;
        tt.seq = seq;
        tt.g = G;
        tt.tq0 = 0;
        tt.ntq = 1;
        tt.nrows = G;
        fa_quantize_out<D, kFdWaves>(a, tt, s_out);
    }
    if constexpr (STEP) {
        if (k_new >= 0) fa_decode_set_rows(st, 0, r_new, kvh, seq, lane, knew0, knew1, vnew0, vnew1);
    }
}

}  // namespace

bool fattn_dec_supported(const fattn_args & a) {
    const int g = a.hkv > 0 ? a.hq / a.hkv : 0;
    // K / V rows, heads and sequences start on 16 bytes (16-byte row loads)
    const bool aligned = (a.k_nb1 | a.k_nb2 | a.k_nb3 | a.v_nb1 | a.v_nb2 | a.v_nb3) % 16 == 0 &&
                         ((uintptr_t) a.k | (uintptr_t) a.v) % 16 == 0;
    return a.n_q == 1 && (a.d == 64 || a.d == 128) && (g == 1 || g == 2 || g == 4) && a.hq == g * a.hkv &&
           a.n_kv > 0 && aligned && (!a.mask || a.m_ne2 == 1);
}

void fattn_dec_plan(fattn_args & a, int n_cu) {
    const int n_tiles = (a.n_kv + kFdTile - 1) / kFdTile;
    const int splits = (n_tiles + kFdSplitTiles - 1) / kFdSplitTiles;
    // A workgroup streams its K / V at a few tens of GB/s, so the form pays
    // only with a workgroup for every CU (n_seq * hkv * splits >= n_cu: the
    // 1.7B batch-8 decode over 4096 positions, 40.3 -> 32.6 us a layer) or
    // over short spans where one launch replaces two (Whisper self attention
    // over a 448-position arena, 8.5 -> 5.6 us). Elsewhere the chunked form
    // with its combine launch is faster (batch 8 over 1024 positions: 14.2 us
    // against 14.7; batch 1: 9.7 against 13.1) and takes the attention.
    const bool wide = (int64_t) a.n_seq * a.hkv * splits >= n_cu;
    a.dec = wide || a.n_kv <= 512 ? splits : 0;
}

size_t fattn_dec_scratch_bytes(const fattn_args & a) {
    if (a.dec <= 1) return 0;
    const int64_t prows = (int64_t) a.n_seq * a.hkv * (a.hq / a.hkv) * a.dec;
    return (size_t) prows * (2 + (size_t) a.d) * sizeof(float) + 1024;
}

template <int D, int G, bool STEP>
static void launch_dec_g(const attn_step_args & st, float * out, void * scratch, hipStream_t s) {
    const fattn_args & a = st.fa;
    const dim3 grid((unsigned) (a.n_seq * a.hkv * a.dec));
    hipLaunchKernelGGL((k_fattn_dec<D, G, STEP>), grid, dim3(kFdThreads), 0, s, st, a.dec == 1 ? out : nullptr,
                       (float *) scratch);
    if (a.dec > 1) {
        fattn_args c = a;
        c.n_chunks = a.dec;
        c.tq = 1;
        c.rows = G;
        c.q_tiles = 1;
        const int64_t prows = (int64_t) a.n_seq * a.hkv * G * a.dec;
        float * pm = (float *) scratch;
        float * pl = pm + prows;
        float * pa = (float *) (((uintptr_t) (pl + prows) + 255) & ~(uintptr_t) 255);
        launch_fattn_combine(c, pm, pl, pa, out, s);
    }
}

void launch_fattn_dec(const attn_step_args & st, bool step, float * out, void * scratch, hipStream_t s) {
    const fattn_args & a = st.fa;
    const int g = a.hq / a.hkv;
    if (step) {
        if (g == 1) launch_dec_g<128, 1, true>(st, out, scratch, s);
        else if (g == 2) launch_dec_g<128, 2, true>(st, out, scratch, s);
        else launch_dec_g<128, 4, true>(st, out, scratch, s);
        return;
    }
    if (a.d == 128) {
        if (g == 1) launch_dec_g<128, 1, false>(st, out, scratch, s);
        else if (g == 2) launch_dec_g<128, 2, false>(st, out, scratch, s);
        else launch_dec_g<128, 4, false>(st, out, scratch, s);
    } else {
        if (g == 1) launch_dec_g<64, 1, false>(st, out, scratch, s);
        else if (g == 2) launch_dec_g<64, 2, false>(st, out, scratch, s);
        else launch_dec_g<64, 4, false>(st, out, scratch, s);
    }
}

}  // namespace mi355x

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
// Activation prologue (optional): the workgroup reads the f32 activations,
// normalises them when the graph puts a norm in front of the MUL_MAT, and
// quantizes them into LDS; the main loop then reads its A operands from LDS.
// The first unit's weight loads are issued before the prologue, so the HBM
// round trip of the weights overlaps it, and the norm / quantize launches
// that would otherwise precede the GEMV disappear.
//
// The scale products are 24-bit multiplies: |MFMA sum| <= 32 * 127 * 15 and
// |32-element sum| <= 32 * 127, scales and mins 6-bit, all within 24 bits.
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
#include "../quant_dev.h"
#include "../mfma_units.h"

namespace mi355x {

struct gemv_args {
    const char * W;
    const char * W2;  // optional second matrix of the same shape (gate + up)
    int64_t row_bytes, M, K;
    const int8_t * aq;
    const float * ad;
    const int16_t * ass;  // Q8_K 32-element sums
    int N;                // activation columns
    int cw;               // columns a workgroup takes (16, fewer to spread a short matrix's prologue)
    char * dst;
    int64_t dst_nb1;
    const char * res;  // optional residual, same layout as dst
    int64_t res_nb1;
    gemv_prologue pro;
    gemv_epilogue epi;  // single-column form only
    // single-column form: matrices after the first, their workgroups following
    // the first's (sub_wg0[s] = the first workgroup of matrix s + 1)
    int nsub;
    gemv_sub sub[kGemvMaxSubs];
    int64_t sub_wg0[kGemvMaxSubs];
};

// prologue modes (template parameter)
constexpr int kProNone = 0;      // pre-quantized activations in global memory
constexpr int kProQuant = 1;     // quantize f32 activations into LDS
constexpr int kProNorm = 2;      // normalise (* w), then quantize into LDS
constexpr int kProNormBias = 3;  // normalise, * w, + b, then quantize into LDS
constexpr int kPadQ = 16;        // bytes of padding per staged column (LDS banks)

// Staging layout: a job is one 256-element span (column j / nspan, span
// j % nspan) held by one DPP row of 16 lanes, 16 consecutive elements per
// lane (lane li of the row: elements 16 li .. 16 li + 15). A wave works on a
// group of four jobs at once (one per row); wave w takes groups w, w + nw, ...
// The normalising prologue keeps kNormGroups groups per wave in registers
// across its statistics pass (launches give it one wave per group).
constexpr int kNormGroups = 1;

// LDS carve of the staged activations of nc columns
struct gemv_lds {
    int64_t q_stride;  // bytes between staged columns of quants
    int64_t d_stride;  // floats between columns of scales
    int64_t ss_stride;  // int16 between columns of 32-element sums
    int64_t q_off, d_off, ss_off, part_off, stat_off, total;
};

__host__ __device__ inline int64_t round16(int64_t v) { return (v + 15) & ~(int64_t) 15; }

__host__ __device__ inline gemv_lds gemv_lds_layout(int wtype, int64_t K, int nc) {
    gemv_lds L;
    const int64_t nspan = (K + 255) / 256;
    L.q_stride = K + kPadQ;
    L.d_stride = wtype == GGML_TYPE_Q4_K ? K / 256 : K / 32;
    L.ss_stride = wtype == GGML_TYPE_Q4_K ? K / 32 : 0;
    L.q_off = 0;
    L.d_off = round16(L.q_off + nc * L.q_stride);
    L.ss_off = round16(L.d_off + nc * L.d_stride * 4);
    L.part_off = round16(L.ss_off + nc * L.ss_stride * 2);
    L.stat_off = round16(L.part_off + 2 * nc * nspan * 8);
    L.total = round16(L.stat_off + nc * 8);
    return L;
}

// DPP moves inside a row of 16 lanes (VALU operations, no LDS traffic):
// xor 1 and xor 2 within quads, rotations by 4 and 8 across the row
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRor4 = 0x124, kDppRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    return __hiloint2double(dpp_i<CTRL>(__double2hiint(v)), dpp_i<CTRL>(__double2loint(v)));
}

// f64 sum over the 16 lanes of a row (lane 0's value is the one used)
__device__ __forceinline__ double row16_sum(double v) {
    v += dpp_d<kDppXor1>(v);
    v += dpp_d<kDppXor2>(v);
    v += dpp_d<kDppRor4>(v);
    v += dpp_d<kDppRor8>(v);
    return v;
}

// f32 max / min over the 16 lanes of a row (every lane gets the result)
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppRor4>(v));
    return fmaxf(v, dpp_f<kDppRor8>(v));
}
__device__ __forceinline__ float row16_min(float v) {
    v = fminf(v, dpp_f<kDppXor1>(v));
    v = fminf(v, dpp_f<kDppXor2>(v));
    v = fminf(v, dpp_f<kDppRor4>(v));
    return fminf(v, dpp_f<kDppRor8>(v));
}
__device__ __forceinline__ int row16_min_i(int v) {
    v = min(v, dpp_i<kDppXor1>(v));
    v = min(v, dpp_i<kDppXor2>(v));
    v = min(v, dpp_i<kDppRor4>(v));
    return min(v, dpp_i<kDppRor8>(v));
}

__device__ __forceinline__ float elem16(const float4 (&x)[4], int t) {
    const float4 & v = x[t >> 2];
    return (t & 3) == 0 ? v.x : (t & 3) == 1 ? v.y : (t & 3) == 2 ? v.z : v.w;
}

// Round-to-nearest-even of y (|y| < 2^22) by adding 1.5 * 2^23: the sum's
// low mantissa bits are the integer in two's complement (ggml's nearest_int
// does exactly this), so the low byte of the sum's bits is the int8 quant.
constexpr float kRneMagic = 12582912.0f;

// the low bytes of four such sums packed into one word, element a lowest
__device__ __forceinline__ uint32_t pack_low_bytes(float a, float b, float c, float d) {
    const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x04000c0cu);
    return lo | hi;
}

// quants of 16 elements times s, packed four to a word
__device__ __forceinline__ void quant16(const float4 (&x)[4], float s, uint32_t (&w)[4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        w[j] = pack_low_bytes(s * x[j].x + kRneMagic, s * x[j].y + kRneMagic, s * x[j].z + kRneMagic,
                              s * x[j].w + kRneMagic);
    }
}

// Quantize one row's span into LDS. Q8_K (quantize_row_q8_K_ref): the
// signed value of largest magnitude, first one on ties, sets iscale =
// -127/max, quants min(127, rne(iscale x)), d = 1/iscale, sums of each 32
// quants (two lanes). Q8_0 (x86 ggml-cpu rule): per 32 elements (two lanes)
// d = amax/127 stored as f16, quants rne(x * 127/amax). Same arithmetic as
// quantize_q8_K_wave / quantize_q8_0_group.
//
// The Q8_K maximum comes from the row's signed max and min: when only one of
// +amax / -amax occurs it is the value of largest magnitude whatever its
// position, so the first-on-ties search runs only for a row holding both.
// |iscale x| <= 127 (1 + 2^-24)^2 < 127.5, so the min(127, .) never binds
// and the quant is the rounded product alone.
template <int WT>
__device__ __forceinline__ void stage_quantize(const float4 (&x)[4], bool live, int col, int sp, int li, int64_t K,
                                               const gemv_lds & L, char * smem) {
    int8_t * s_q = (int8_t *) (smem + L.q_off);
    float * s_d = (float *) (smem + L.d_off);
    int16_t * s_ss = (int16_t *) (smem + L.ss_off);
    const int64_t e = (int64_t) sp * 256 + 16 * li;  // first element of this lane
    uint32_t w[4];
    if constexpr (WT == GGML_TYPE_Q4_K) {
        float hi = x[0].x, lo = x[0].x;
#pragma unroll
        for (int t = 1; t < 16; t++) {
            hi = fmaxf(hi, elem16(x, t));
            lo = fminf(lo, elem16(x, t));
        }
        hi = row16_max(hi);
        lo = row16_min(lo);
        const float amax = fmaxf(hi, -lo);
        float best = hi >= -lo ? hi : lo;
        if (hi == -lo && amax != 0.0f) {
            // both signs reach amax (uniform over the row): the first such
            // element in order decides; key = 2 * index + sign
            int key = 0x7fffffff;
#pragma unroll
            for (int t = 15; t >= 0; t--) {
                const float v = elem16(x, t);
                if (fabsf(v) == amax) key = 2 * (16 * li + t) + (v < 0.0f ? 1 : 0);
            }
            key = row16_min_i(key);
            best = (key & 1) ? lo : hi;
        }
        const float iscale = amax == 0.0f ? 0.0f : -127.0f / best;
        quant16(x, iscale, w);
        int ssum = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) ssum = __builtin_amdgcn_sdot4((int) w[j], 0x01010101, ssum, false);
        ssum += dpp_i<kDppXor1>(ssum);
        if (live) {
            if ((li & 1) == 0) s_ss[col * L.ss_stride + e / 32] = (int16_t) ssum;
            if (li == 0) s_d[col * L.d_stride + sp] = amax == 0.0f ? 0.0f : 1.0f / iscale;
        }
    } else {
        float amax = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; t++) amax = fmaxf(amax, fabsf(elem16(x, t)));
        amax = fmaxf(amax, dpp_f<kDppXor1>(amax));
        const float dd = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        quant16(x, id, w);
        live = live && e < K;  // Q8_0 spans may end early; whole lane pairs drop out
        if (live && (li & 1) == 0) s_d[col * L.d_stride + e / 32] = round_to_half(dd);
    }
    if (live) *(uint4 *) (s_q + col * L.q_stride + e) = make_uint4(w[0], w[1], w[2], w[3]);
}

// load this lane's 16 elements of job `job`; false outside the job range,
// where the values (element 0 of the chunk's first column) are not used: the
// users mask them, and the lanes that reduce together (a DPP row for Q8_K, a
// lane pair for Q8_0) are all in range or all out, so no reduction sees them.
// Masking here would make the load be waited for at once.
__device__ __forceinline__ bool stage_load(const gemv_args & a, int n0, int jobs, int nspan, int job, int li,
                                           float4 (&x)[4]) {
    const int col = job / nspan, sp = job - col * nspan;
    const int64_t e = (int64_t) sp * 256 + 16 * li;
    const bool ok = job < jobs && e < a.K;
    // clamped address, unconditional load: keeps the loads of a group in flight together
    const float * src = (const float *) ((const char *) a.pro.x + (int64_t) (n0 + (ok ? col : 0)) * a.pro.x_nb1) +
                        (ok ? e : 0);
#pragma unroll
    for (int j = 0; j < 4; j++) x[j] = ((const float4 *) src)[j];
    return ok;
}

// quantize-only staging: each wave streams its groups, two groups' loads in
// flight at a time. The first two groups are requested before `issue` runs
// (the caller's weight loads): loads return in issue order, so activations
// requested first never wait behind the weights' HBM round trip.
template <int WT, typename F>
__device__ __forceinline__ void gemv_stage_quant(const gemv_args & a, int n0, int nc, char * smem, F && issue) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int row = lane >> 4, li = lane & 15;
    const int64_t K = a.K;
    const int nspan = (int) ((K + 255) / 256);
    const int jobs = nc * nspan;
    const int groups = (jobs + 3) / 4;
    const gemv_lds L = gemv_lds_layout(WT, K, nc);
    float4 x0[4], x1[4];
    int gi = wave;
    // clamped, unconditional loads (a job past the end reads element 0)
    bool ok0 = stage_load(a, n0, jobs, nspan, 4 * gi + row, li, x0);
    bool ok1 = stage_load(a, n0, jobs, nspan, 4 * (gi + nw) + row, li, x1);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the caller's
    issue();
    for (; gi < groups; gi += 2 * nw) {
        const int j0 = 4 * gi + row, j1 = 4 * (gi + nw) + row;
        if (gi != wave) {
            ok0 = stage_load(a, n0, jobs, nspan, j0, li, x0);
            ok1 = stage_load(a, n0, jobs, nspan, j1, li, x1);
        }
        stage_quantize<WT>(x0, ok0, j0 / nspan, j0 % nspan, li, K, L, smem);
        if (gi + nw < groups) stage_quantize<WT>(x1, ok1, j1 / nspan, j1 % nspan, li, K, L, smem);
    }
    __syncthreads();
}

__device__ __forceinline__ double readlane_d(double v, int l) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), l),
                            __builtin_amdgcn_readlane(__double2loint(v), l));
}

// the sum over a column's spans, in span order from 0.0, when the column's
// nspan spans are rows first .. first + nspan - 1 of this wave's group: each
// row's row16_sum is read from its lane 0
__device__ __forceinline__ double group_col_sum(double v, int first, int nspan) {
    const double r0 = readlane_d(v, 0), r1 = readlane_d(v, 16), r2 = readlane_d(v, 32), r3 = readlane_d(v, 48);
    double t = 0.0;
#pragma unroll
    for (int sp = 0; sp < 4; sp++) {
        if (sp < nspan) {
            const int q = first + sp;
            t += q == 0 ? r0 : q == 1 ? r1 : q == 2 ? r2 : r3;
        }
    }
    return t;
}

// normalising staging: the statistics are f64 sums of the elements (layer
// norm) and of the centred squares -- per lane in element order, over the
// row by DPP, per column over the spans in order -- then
// mean = sum / K, scale = 1 / sqrt(var + eps); the normalised value is
// ((x - mean) * scale) * w (+ b), the roundings of NORM / RMS_NORM, MUL, ADD
template <int WT, bool BIAS, typename F>
__device__ __forceinline__ void gemv_stage_norm(const gemv_args & a, int n0, int nc, char * smem, F && issue) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int row = lane >> 4, li = lane & 15;
    const int64_t K = a.K;
    const int nspan = (int) ((K + 255) / 256);
    const int jobs = nc * nspan;
    const gemv_lds L = gemv_lds_layout(WT, K, nc);
    double * s_part = (double *) (smem + L.part_off);
    float2 * s_stat = (float2 *) (smem + L.stat_off);
    const gemv_prologue & p = a.pro;
    float4 x[kNormGroups][4], w[kNormGroups][4], b[BIAS ? kNormGroups : 1][4];
    bool ok[kNormGroups];
#pragma unroll
    for (int k = 0; k < kNormGroups; k++) {
        const int job = 4 * (wave + nw * k) + row;
        ok[k] = stage_load(a, n0, jobs, nspan, job, li, x[k]);
        const int64_t e = ok[k] ? (int64_t) (job % nspan) * 256 + 16 * li : 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            w[k][j] = p.w ? *(const float4 *) (p.w + e + 4 * j) : make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (BIAS) b[k][j] = *(const float4 *) (p.b + e + 4 * j);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the caller's
    issue();  // the caller's weight loads, behind the activations
    const double n = (double) K;
    if (kNormGroups == 1 && (nspan == 1 || nspan == 2 || nspan == 4)) {
        // every column's spans lie in one wave's group (rows first ..
        // first + nspan - 1): the statistics are summed inside the wave --
        // the same sums in the same order -- with no LDS round trip and no
        // barrier before the quantization
        const int job = 4 * wave + row;
        const int first = (row / nspan) * nspan;
        float mean = 0.0f;
        if (p.norm == 1) {
            double s = 0.0;
#pragma unroll
            for (int t = 0; t < 16; t++) s += ok[0] ? (double) elem16(x[0], t) : 0.0;
            mean = (float) (group_col_sum(row16_sum(s), first, nspan) / n);
        }
        double s2 = 0.0;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const float v = ok[0] ? elem16(x[0], t) - mean : 0.0f;
            s2 += (double) (v * v);
        }
        const float var = (float) (group_col_sum(row16_sum(s2), first, nspan) / n);
        const float scale = 1.0f / sqrtf(var + p.eps);
        if (4 * wave < jobs) {  // uniform: some row of the wave has a job
            const int col = ok[0] ? job / nspan : 0;
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float4 xs = x[0][j];
                if (p.norm == 1) xs = make_float4(xs.x - mean, xs.y - mean, xs.z - mean, xs.w - mean);
                v[j].x = (xs.x * scale) * w[0][j].x;
                v[j].y = (xs.y * scale) * w[0][j].y;
                v[j].z = (xs.z * scale) * w[0][j].z;
                v[j].w = (xs.w * scale) * w[0][j].w;
                if constexpr (BIAS) {
                    v[j].x += b[0][j].x;
                    v[j].y += b[0][j].y;
                    v[j].z += b[0][j].z;
                    v[j].w += b[0][j].w;
                }
            }
            stage_quantize<WT>(v, ok[0], col, job % nspan, li, K, L, smem);
        }
        __syncthreads();
        return;
    }
    if (p.norm == 1) {
#pragma unroll
        for (int k = 0; k < kNormGroups; k++) {
            double s = 0.0;
#pragma unroll
            for (int t = 0; t < 16; t++) s += ok[k] ? (double) elem16(x[k], t) : 0.0;
            s = row16_sum(s);
            const int job = 4 * (wave + nw * k) + row;
            if (li == 0 && job < jobs) s_part[job] = s;
        }
        __syncthreads();
        if ((int) threadIdx.x < nc) {
            double t = 0.0;
            for (int sp = 0; sp < nspan; sp++) t += s_part[threadIdx.x * nspan + sp];
            s_stat[threadIdx.x].x = (float) (t / n);
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < kNormGroups; k++) {
        const int job = 4 * (wave + nw * k) + row;
        const float mean = p.norm == 1 && ok[k] ? s_stat[job / nspan].x : 0.0f;
        double s2 = 0.0;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const float v = ok[k] ? elem16(x[k], t) - mean : 0.0f;
            s2 += (double) (v * v);
        }
        s2 = row16_sum(s2);
        if (li == 0 && job < jobs) s_part[jobs + job] = s2;
    }
    __syncthreads();
    if ((int) threadIdx.x < nc) {
        double t2 = 0.0;
        for (int sp = 0; sp < nspan; sp++) t2 += s_part[jobs + threadIdx.x * nspan + sp];
        const float var = (float) (t2 / n);
        s_stat[threadIdx.x].y = 1.0f / sqrtf(var + p.eps);
        if (p.norm != 1) s_stat[threadIdx.x].x = 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kNormGroups; k++) {
        const int job = 4 * (wave + nw * k) + row;
        if (4 * (wave + nw * k) >= jobs) break;  // uniform: no row of the wave has a job
        const int col = ok[k] ? job / nspan : 0;
        const float2 st = s_stat[col];
        float4 v[4];
        // RMS norm: x - 0 == x bit for bit, so the subtraction is skipped
        const float4 * xs = x[k];
        float4 xc[4];
        if (p.norm == 1) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                xc[j] = make_float4(x[k][j].x - st.x, x[k][j].y - st.x, x[k][j].z - st.x, x[k][j].w - st.x);
            xs = xc;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j].x = (xs[j].x * st.y) * w[k][j].x;
            v[j].y = (xs[j].y * st.y) * w[k][j].y;
            v[j].z = (xs[j].z * st.y) * w[k][j].z;
            v[j].w = (xs[j].w * st.y) * w[k][j].w;
            if constexpr (BIAS) {
                v[j].x += b[k][j].x;
                v[j].y += b[k][j].y;
                v[j].z += b[k][j].z;
                v[j].w += b[k][j].w;
            }
        }
        stage_quantize<WT>(v, ok[k], col, job % nspan, li, K, L, smem);
    }
    __syncthreads();
}

// Split-K finish. Every wave puts its partials in LDS; after one barrier
// each thread takes outputs o = tid, tid + 64 nw, ... of the tile (row o % 16,
// column o / 16) and sums that output's partials in wave order -- waves
// [0, half) hold W's, waves [half, nw) W2's when there is a second matrix,
// whose epilogue then writes silu(W x) * (W2 x), the SwiGLU gate of
// nn/ffn.rs:64-91 with the roundings of MUL_MAT, SILU and MUL apart. A
// residual, when given, is added to the rounded product. The sums run in the
// order a single wave would have added them, so the bits do not depend on
// which thread finishes an output.
constexpr int kFinishPerThread = 4;  // 16 x 16 outputs over at least one wave

// the residual of this thread's outputs, requested early. The loads are
// unconditional (clamped; without a residual they read the output tensor and
// the value is not used): a load behind a branch would make every later wait
// count it as outstanding on both paths.
__device__ __forceinline__ void gemv_res_prefetch(const gemv_args & a, int64_t tile, int n0, int nc,
                                                  float (&res)[kFinishPerThread]) {
    const int nt = (int) blockDim.x;
    const char * base = a.res ? a.res : a.dst;
    const int64_t nb1 = a.res ? a.res_nb1 : a.dst_nb1;
#pragma unroll
    for (int k = 0; k < kFinishPerThread; k++) {
        int o = (int) threadIdx.x + k * nt;
        o = o < 16 * nc ? o : 0;
        res[k] = *(const float *) (base + (int64_t) (n0 + (o >> 4)) * nb1 + (tile * 16 + (o & 15)) * 4);
    }
}

__device__ __forceinline__ void gemv_finish(const gemv_args & a, const double (&acc)[4], double (*s_red)[64][4],
                                            int64_t tile, int n0, int nc, int half, const float (&res)[kFinishPerThread]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int i = 0; i < 4; i++) s_red[wave][lane][i] = acc[i];
    __syncthreads();
    const int nt = 64 * nw;
#pragma unroll
    for (int k = 0; k < kFinishPerThread; k++) {
        const int o = (int) threadIdx.x + k * nt;
        if (o >= 16 * nc) break;
        const int r = o & 15, n = o >> 4;
        const int sl = r + 16 * (n >> 2), si = n & 3;  // the MFMA lane and slot holding (row r, column n)
        double v = s_red[0][sl][si];
#pragma unroll
        for (int w = 1; w < 16; w++) {
            const double pw = s_red[w][sl][si];  // in bounds for every w; added only for w < half
            v = w < half ? v + pw : v;
        }
        float f = (float) v;
        if (a.W2) {
            double v2 = 0.0;
#pragma unroll
            for (int w = 1; w < 16; w++) {
                const double pw = s_red[w][sl][si];
                v2 = w >= half && w < nw ? v2 + pw : v2;
            }
            const float u = (float) v2;
            f = (f / (1.0f + expf_det(-f))) * u;
        }
        if (a.res) f = res[k] + f;
        *(float *) (a.dst + (int64_t) (n0 + n) * a.dst_nb1 + (tile * 16 + r) * 4) = f;
    }
}

// waves of the workgroup take super-blocks round-robin (wave w: sb = w,
// w + nw, ...); the first unit's weights are requested at kernel start, each
// next unit's at the end of the current one
template <int PRO, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void k_gemv_q4_K(gemv_args a) {
    extern __shared__ __align__(16) char smem[];
    __shared__ double s_red[16][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int half = a.W2 ? nw / 2 : nw;
    const int second = wave >= half;
    const int wv = wave - (second ? half : 0);
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile = blockIdx.x;
    const int n0 = (int) blockIdx.y * a.cw;
    const int nc = min(a.cw, a.N - n0);
    const int64_t nsb = a.K / 256;
    const int64_t row = tile * 16 + r;
    const char * wrow = (second ? a.W2 : a.W) + row * a.row_bytes;
    uint4 hdr;
    long q[4];
    int64_t sb = wv;
    float res[kFinishPerThread];
    // the first unit's weights and the residual; with a prologue they are
    // requested right after the activations the prologue waits for
    auto issue = [&]() {
        gemv_res_prefetch(a, tile, n0, nc, res);
        // waves without a unit (staging helpers) read unit 0 and never use it
        const char * blk = wrow + (sb < nsb ? sb : 0) * 144;
        hdr = *(const uint4 *) blk;
#pragma unroll
        for (int c = 0; c < 4; c++) q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
    };
    // activation operands: LDS after the prologue, else the global buffers
    const int8_t * aq;
    const float * adp;
    const int16_t * asp;
    int64_t q_stride, d_stride, ss_stride;
    int c0;  // column index of the chunk's first column in the operand arrays
    if constexpr (PRO != kProNone) {
        if constexpr (PRO == kProQuant) gemv_stage_quant<GGML_TYPE_Q4_K>(a, n0, nc, smem, issue);
        else gemv_stage_norm<GGML_TYPE_Q4_K, PRO == kProNormBias>(a, n0, nc, smem, issue);
        const gemv_lds L = gemv_lds_layout(GGML_TYPE_Q4_K, a.K, nc);
        aq = (const int8_t *) (smem + L.q_off);
        adp = (const float *) (smem + L.d_off);
        asp = (const int16_t *) (smem + L.ss_off);
        q_stride = L.q_stride;
        d_stride = L.d_stride;
        ss_stride = L.ss_stride;
        c0 = 0;
    } else {
        issue();
        aq = a.aq;
        adp = a.ad;
        asp = a.ass;
        q_stride = a.K;
        d_stride = nsb;
        ss_stride = a.K / 32;
        c0 = n0;
    }
    const bool a_ok = r < nc;  // this lane's A-operand column
    const int8_t * acol = aq + (int64_t) (c0 + (a_ok ? r : 0)) * q_stride;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (; sb < nsb; sb += half) {
        long af[8];
        float ad[4], ssa[2];
        // every load unconditional (clamped to column 0 of the chunk, which
        // always exists) and masked afterwards: no load waits behind a branch
#pragma unroll
        for (int j = 0; j < 8; j++) af[j] = *(const long *) (acol + sb * 256 + 32 * j + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = 4 * g + i;
            const int nn = n < nc ? n : 0;
            ad[i] = adp[(int64_t) (c0 + nn) * d_stride + sb];
        }
        q4k_ssum_operand(asp + (int64_t) (c0 + (a_ok ? r : 0)) * ss_stride + sb * 8, a_ok, g, ssa);
#pragma unroll
        for (int j = 0; j < 8; j++) af[j] = a_ok ? af[j] : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) ad[i] = 4 * g + i < nc ? ad[i] : 0.0f;
        q4k_unit(hdr, q, af, ad, ssa, acc);
        // the next unit's weights
        if (sb + half < nsb) {
            const char * blk = wrow + (sb + half) * 144;
            hdr = *(const uint4 *) blk;
#pragma unroll
            for (int c = 0; c < 4; c++) q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
        }
    }
    gemv_finish(a, acc, s_red, tile, n0, nc, half, res);
}

// k_gemv_q4_K with TPW = 2 16-row tiles a workgroup, for launches where one
// tile a workgroup would take the CUs more than one round (the Qwen3-1.7B
// gate/up pair: 384 tiles of 16 waves, one workgroup a CU): the tiles share
// the staged activations and each unit's activation operands, their weights
// are requested together, and each tile's outputs are summed and stored in
// turn. No residual (the launcher keeps such products on k_gemv_q4_K).
template <int PRO, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void k_gemv_q4_K_pair(gemv_args a) {
    constexpr int TPW = 2;
    extern __shared__ __align__(16) char smem[];
    __shared__ double s_red[16][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int half = a.W2 ? nw / 2 : nw;
    const int second = wave >= half;
    const int wv = wave - (second ? half : 0);
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile0 = (int64_t) blockIdx.x * TPW;
    const int64_t ntile = a.M / 16;
    const int n0 = (int) blockIdx.y * a.cw;
    const int nc = min(a.cw, a.N - n0);
    const int64_t nsb = a.K / 256;
    const char * wrow[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int64_t tt = tile0 + t < ntile ? tile0 + t : tile0;  // a missing tile reads the first, never stored
        wrow[t] = (second ? a.W2 : a.W) + (tt * 16 + r) * a.row_bytes;
    }
    uint4 hdr[TPW];
    long q[TPW][4];
    int64_t sb = wv;
    const float res[kFinishPerThread] = {0.0f, 0.0f, 0.0f, 0.0f};  // no residual
    // the first unit's weights of tile t; with a prologue tile 0's are
    // requested right after the activations the prologue waits for, tile 1's
    // once the prologue's registers are free
    auto issue_tile = [&](int t) {
        // waves without a unit (staging helpers) read unit 0 and never use it
        const char * blk = wrow[t] + (sb < nsb ? sb : 0) * 144;
        hdr[t] = *(const uint4 *) blk;
#pragma unroll
        for (int c = 0; c < 4; c++) q[t][c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
    };
    auto issue = [&]() { issue_tile(0); };
    // activation operands: LDS after the prologue, else the global buffers
    const int8_t * aq;
    const float * adp;
    const int16_t * asp;
    int64_t q_stride, d_stride, ss_stride;
    int c0;  // column index of the chunk's first column in the operand arrays
    if constexpr (PRO != kProNone) {
        if constexpr (PRO == kProQuant) gemv_stage_quant<GGML_TYPE_Q4_K>(a, n0, nc, smem, issue);
        else gemv_stage_norm<GGML_TYPE_Q4_K, PRO == kProNormBias>(a, n0, nc, smem, issue);
        const gemv_lds L = gemv_lds_layout(GGML_TYPE_Q4_K, a.K, nc);
        aq = (const int8_t *) (smem + L.q_off);
        adp = (const float *) (smem + L.d_off);
        asp = (const int16_t *) (smem + L.ss_off);
        q_stride = L.q_stride;
        d_stride = L.d_stride;
        ss_stride = L.ss_stride;
        c0 = 0;
    } else {
        issue();
        aq = a.aq;
        adp = a.ad;
        asp = a.ass;
        q_stride = a.K;
        d_stride = nsb;
        ss_stride = a.K / 32;
        c0 = n0;
    }
    issue_tile(1);
    const bool a_ok = r < nc;  // this lane's A-operand column
    const int8_t * acol = aq + (int64_t) (c0 + (a_ok ? r : 0)) * q_stride;
    // the tiles one after the other (tile 1's first weights in flight
    // meanwhile), so only one tile's sums are live at a time
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        if (tile0 + t >= ntile) break;  // uniform
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
        for (int64_t u = wv; u < nsb; u += half) {
            long af[8];
            float ad[4], ssa[2];
            // every load unconditional (clamped to column 0 of the chunk,
            // which always exists) and masked afterwards
#pragma unroll
            for (int j = 0; j < 8; j++) af[j] = *(const long *) (acol + u * 256 + 32 * j + 8 * g);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = 4 * g + i;
                const int nn = n < nc ? n : 0;
                ad[i] = adp[(int64_t) (c0 + nn) * d_stride + u];
            }
            q4k_ssum_operand(asp + (int64_t) (c0 + (a_ok ? r : 0)) * ss_stride + u * 8, a_ok, g, ssa);
#pragma unroll
            for (int j = 0; j < 8; j++) af[j] = a_ok ? af[j] : 0;
#pragma unroll
            for (int i = 0; i < 4; i++) ad[i] = 4 * g + i < nc ? ad[i] : 0.0f;
            q4k_unit(hdr[t], q[t], af, ad, ssa, acc);
            // the tile's next unit
            if (u + half < nsb) {
                const char * blk = wrow[t] + (u + half) * 144;
                hdr[t] = *(const uint4 *) blk;
#pragma unroll
                for (int c = 0; c < 4; c++) q[t][c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
            }
        }
        if (t > 0) __syncthreads();  // the previous tile's sums have been read from s_red
        gemv_finish(a, acc, s_red, tile0 + t, n0, nc, half, res);
    }
}

// Q8_0 weights in the row-split layout [K quants][K/32 f16 scales]; the waves
// take groups of 8 blocks round-robin, each group's loads issued together
// (the first group's weights before the prologue)
template <int PRO, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void k_gemv_q8_0(gemv_args a) {
    extern __shared__ __align__(16) char smem[];
    __shared__ double s_red[16][64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int half = a.W2 ? nw / 2 : nw;
    const int second = wave >= half;
    const int wv = wave - (second ? half : 0);
    const int r = lane & 15, g = lane >> 4;
    const int64_t tile = blockIdx.x;
    const int n0 = (int) blockIdx.y * a.cw;
    const int nc = min(a.cw, a.N - n0);
    const int64_t nblk = a.K / 32;
    const int64_t row = tile * 16 + r;
    const char * wrow = (second ? a.W2 : a.W) + row * a.row_bytes;
    const uint16_t * wsc = (const uint16_t *) (wrow + a.K);
    long q[kQ8Group];
    uint16_t ds[kQ8Group];
    int64_t b0 = (int64_t) wv * kQ8Group;
    float res[kFinishPerThread];
    // the first group's weights and the residual, behind the prologue's activations
    auto issue = [&]() {
        gemv_res_prefetch(a, tile, n0, nc, res);
#pragma unroll
        for (int u = 0; u < kQ8Group; u++) {
            const int64_t b = b0 + u < nblk ? b0 + u : 0;  // clamped; past-the-end blocks are never used
            q[u] = *(const long *) (wrow + b * 32 + 8 * g);
            ds[u] = wsc[b];
        }
    };
    const int8_t * aq;
    const float * adp;
    int64_t q_stride, d_stride;
    int c0;
    if constexpr (PRO != kProNone) {
        if constexpr (PRO == kProQuant) gemv_stage_quant<GGML_TYPE_Q8_0>(a, n0, nc, smem, issue);
        else gemv_stage_norm<GGML_TYPE_Q8_0, PRO == kProNormBias>(a, n0, nc, smem, issue);
        const gemv_lds L = gemv_lds_layout(GGML_TYPE_Q8_0, a.K, nc);
        aq = (const int8_t *) (smem + L.q_off);
        adp = (const float *) (smem + L.d_off);
        q_stride = L.q_stride;
        d_stride = L.d_stride;
        c0 = 0;
    } else {
        issue();
        aq = a.aq;
        adp = a.ad;
        q_stride = a.K;
        d_stride = nblk;
        c0 = n0;
    }
    const bool a_ok = r < nc;
    const int8_t * acol = aq + (int64_t) (c0 + (a_ok ? r : 0)) * q_stride;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    const int64_t first = b0;
    for (; b0 < nblk; b0 += (int64_t) half * kQ8Group) {
        if (b0 != first) {
#pragma unroll
            for (int u = 0; u < kQ8Group; u++) {
                const int64_t b = b0 + u < nblk ? b0 + u : 0;
                q[u] = *(const long *) (wrow + b * 32 + 8 * g);
                ds[u] = wsc[b];
            }
        }
        // unconditional clamped loads, masked afterwards (no load behind a branch)
        long af[kQ8Group];
        float4 ad[4][kQ8Group / 4];
#pragma unroll
        for (int u = 0; u < kQ8Group; u++) {
            const int64_t b = b0 + u < nblk ? b0 + u : 0;
            af[u] = *(const long *) (acol + b * 32 + 8 * g);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = 4 * g + i;
            const int nn = n < nc ? n : 0;
#pragma unroll
            for (int v = 0; v < kQ8Group / 4; v++) {
                const int64_t b = b0 + 4 * v < nblk ? b0 + 4 * v : 0;
                ad[i][v] = *(const float4 *) (adp + (int64_t) (c0 + nn) * d_stride + b);
            }
        }
#pragma unroll
        for (int u = 0; u < kQ8Group; u++) af[u] = a_ok ? af[u] : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (4 * g + i >= nc) {
#pragma unroll
                for (int v = 0; v < kQ8Group / 4; v++) ad[i][v] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        q8_0_unit(q, ds, af, ad, (int) (nblk - b0 < kQ8Group ? nblk - b0 : kQ8Group), acc);
    }
    gemv_finish(a, acc, s_red, tile, n0, nc, half, res);
}

// Streaming form for tall matrices with pre-quantized activations (the
// vocabulary projection: thousands of tiles, one unit per wave). A workgroup
// of U waves (U = units of a row) keeps wave w's activation operands -- those
// of unit w, the same for every tile -- in registers and walks batches of
// kStreamTiles consecutive tiles, batch k + 1's weights requested before
// batch k's arithmetic. Each wave puts its unit's term of every tile of the
// batch in LDS; after one barrier wave j sums tile j's terms in wave order
// (the order of gemv_finish) and stores the rows. The LDS of consecutive
// batches alternates, so one barrier a batch suffices: a wave writes a
// buffer again only after the next batch's barrier, which every wave reaches
// after its reads of that buffer.
constexpr int kStreamTiles = 2;
constexpr int kStreamWgPerCu = 4;

template <int WT> struct stream_w;
template <> struct stream_w<GGML_TYPE_Q4_K> {
    uint4 hdr;
    long q[4];
};
template <> struct stream_w<GGML_TYPE_Q8_0> {
    long q[kQ8Group];
    uint16_t ds[kQ8Group];
};

// unit `u` of the rows of tiles base .. base + kStreamTiles - 1 (tiles past
// the end read tile 0, which always exists; their values are never stored)
template <int WT>
__device__ __forceinline__ void stream_load(const gemv_args & a, int64_t base, int u, int r, int g,
                                            stream_w<WT> (&w)[kStreamTiles]) {
    const int64_t ntiles = a.M / 16;
#pragma unroll
    for (int j = 0; j < kStreamTiles; j++) {
        const int64_t tile = base + j < ntiles ? base + j : 0;
        const char * wrow = a.W + (tile * 16 + r) * a.row_bytes;
        if constexpr (WT == GGML_TYPE_Q4_K) {
            const char * blk = wrow + (int64_t) u * 144;
            w[j].hdr = *(const uint4 *) blk;
#pragma unroll
            for (int c = 0; c < 4; c++) w[j].q[c] = *(const long *) (blk + 16 + 32 * c + 8 * g);
        } else {
            const uint16_t * wsc = (const uint16_t *) (wrow + a.K);
            const int64_t b0 = (int64_t) u * kQ8Group;
#pragma unroll
            for (int v = 0; v < kQ8Group; v++) {
                w[j].q[v] = *(const long *) (wrow + (b0 + v) * 32 + 8 * g);
                w[j].ds[v] = wsc[b0 + v];
            }
        }
    }
}

// NCL: the columns a lane keeps (1 for a one-column launch, else 4)
template <int WT, int NCL>
__global__ __launch_bounds__(512) void k_gemv_stream(gemv_args a) {
    extern __shared__ __align__(16) char smem[];
    double (*s_part)[64][4] = (double (*)[64][4]) smem;  // [tile of the batch * nw + wave][lane]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = (int) blockIdx.y * 16;
    const int nc = min(16, a.N - n0);
    const int64_t ntiles = a.M / 16;
    const int64_t step = (int64_t) gridDim.x * kStreamTiles;
    int64_t base = (int64_t) blockIdx.x * kStreamTiles;
    stream_w<WT> cur[kStreamTiles], nxt[kStreamTiles];
    stream_load<WT>(a, base, wave, r, g, cur);
    // this wave's activation operands (unit `wave`), clamped loads masked afterwards
    const bool a_ok = r < nc;
    const int8_t * acol = a.aq + (int64_t) (n0 + (a_ok ? r : 0)) * a.K;
    long af[8];
    float ad4[4], ssa[2];
    float4 ad8[4][kQ8Group / 4];
    if constexpr (WT == GGML_TYPE_Q4_K) {
        const int64_t sb = wave, nsb = a.K / 256;
#pragma unroll
        for (int j = 0; j < 8; j++) af[j] = *(const long *) (acol + sb * 256 + 32 * j + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = 4 * g + i;
            const int nn = n < nc ? n : 0;
            ad4[i] = a.ad[(int64_t) (n0 + nn) * nsb + sb];
        }
        q4k_ssum_operand(a.ass + (int64_t) (n0 + (a_ok ? r : 0)) * (a.K / 32) + sb * 8, a_ok, g, ssa);
#pragma unroll
        for (int i = 0; i < 4; i++) ad4[i] = 4 * g + i < nc ? ad4[i] : 0.0f;
    } else {
        const int64_t b0 = (int64_t) wave * kQ8Group, nblk = a.K / 32;
#pragma unroll
        for (int u = 0; u < kQ8Group; u++) af[u] = *(const long *) (acol + (b0 + u) * 32 + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = 4 * g + i;
            const int nn = n < nc ? n : 0;
#pragma unroll
            for (int v = 0; v < kQ8Group / 4; v++) {
                ad8[i][v] = *(const float4 *) (a.ad + (int64_t) (n0 + nn) * nblk + b0 + 4 * v);
                if (n >= nc) ad8[i][v] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) af[j] = a_ok ? af[j] : 0;
    for (int par = 0; base < ntiles; base += step, par ^= 1) {
        if (base + step < ntiles) stream_load<WT>(a, base + step, wave, r, g, nxt);
        double (*sp)[64][4] = s_part + par * kStreamTiles * nw;
#pragma unroll
        for (int j = 0; j < kStreamTiles; j++) {
            double acc[4] = {0.0, 0.0, 0.0, 0.0};
            if constexpr (WT == GGML_TYPE_Q4_K) q4k_unit<NCL>(cur[j].hdr, cur[j].q, af, ad4, ssa, acc);
            else q8_0_unit<NCL>(cur[j].q, cur[j].ds, af, ad8, kQ8Group, acc);
#pragma unroll
            for (int i = 0; i < NCL; i++) sp[j * nw + wave][lane][i] = acc[i];
        }
        __syncthreads();
        for (int j = wave; j < kStreamTiles; j += nw) {
            const int64_t tile = base + j;
            if (tile < ntiles) {
                double v[4];
#pragma unroll
                for (int i = 0; i < NCL; i++) v[i] = sp[j * nw][lane][i];
                for (int w = 1; w < nw; w++) {
#pragma unroll
                    for (int i = 0; i < NCL; i++) v[i] += sp[j * nw + w][lane][i];
                }
#pragma unroll
                for (int i = 0; i < NCL; i++) {
                    const int n = n0 + 4 * g + i;
                    if (n < a.N) *(float *) (a.dst + (int64_t) n * a.dst_nb1 + (tile * 16 + r) * 4) = (float) v[i];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kStreamTiles; j++) cur[j] = nxt[j];
    }
}

// Single-column form (batch 1, Q8_0 weights). At N = 1 the MFMA tile spends
// 15 of its 16 columns on padding and a short matrix gives few workgroups.
// Here a wave owns one weight row and walks K 1024 elements a pass: lane l
// takes 16 quants (half a block) against the column's 16 activation quants
// with four v_dot4_i32_i8, the two halves of a block add exactly (DPP), the
// even lane adds the block term isum * (d_w * d_a) -- exact in f64, one fused
// multiply-add -- to its f64 partial, and the row is the f64 sum of the
// partials (the CPU reference sums the same exact terms wide, so any order
// gives its bits). Workgroups of WV waves of R rows each; with a norm or
// quantize in front each workgroup stages the column itself, its weight
// pieces already requested.
constexpr int kG1Waves = 4;
constexpr int kG1MaxPasses = 8;  // K <= 8192

template <int PRO, int WV, int R>
__global__ __launch_bounds__(64 * WV) void k_gemv1_q8_0(gemv_args a) {
    extern __shared__ __align__(16) char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // which matrix of the launch this workgroup serves (constant indices:
    // the argument block stays in scalar registers)
    const char * Wm = a.W;
    int64_t M = a.M, blk = blockIdx.x;
    char * dst = a.dst;
    const char * resp = a.res;
    int si = -1;  // the sibling matrix this workgroup serves, if any
    if (a.nsub > 1 && (int64_t) blockIdx.x >= a.sub_wg0[1]) {
        Wm = a.sub[1].W, M = a.sub[1].M, dst = a.sub[1].dst, resp = a.sub[1].res, blk -= a.sub_wg0[1];
        si = 1;
    } else if (a.nsub > 0 && (int64_t) blockIdx.x >= a.sub_wg0[0]) {
        Wm = a.sub[0].W, M = a.sub[0].M, dst = a.sub[0].dst, resp = a.sub[0].res, blk -= a.sub_wg0[0];
        si = 0;
    }
    // a sibling's SET_ROWS: the cache row its column also goes to (null: none
    // or an index out of range)
    uint16_t * crow = nullptr;
    if (si >= 0 && a.sub[si].rows_dst) {
        const gemv_sub & sb = a.sub[si];
        const int64_t r = sb.rows_i64 ? *(const int64_t *) sb.rows_idx : (int64_t) *(const int32_t *) sb.rows_idx;
        crow = r >= 0 && r < sb.rows_n ? (uint16_t *) (sb.rows_dst + r * sb.rows_nb1) : nullptr;
    }
    const int64_t row0 = (blk * WV + wave) * R;  // this wave's R rows
    const bool wave_ok = row0 < M;                // uniform per wave
    const int64_t K = a.K;
    const int passes = (int) ((K + 1023) / 1024);
    uint4 wq[R][kG1MaxPasses], wq2[R][kG1MaxPasses];
    uint16_t ws[R][kG1MaxPasses], ws2[R][kG1MaxPasses];
    float res[R], res2[R];
    // the rows' weights and residuals; with a prologue they are requested
    // right after the column the prologue waits for (loads return in order)
    auto issue = [&]() {
#pragma unroll
        for (int j = 0; j < R; j++) {
            const int64_t rr = row0 + j < M ? row0 + j : 0;  // clamped, never stored
            const char * wrow = Wm + rr * a.row_bytes;
            const char * wrow2 = a.W2 ? a.W2 + rr * a.row_bytes : nullptr;
#pragma unroll
            for (int p = 0; p < kG1MaxPasses; p++) {
                if (p < passes) {
                    const int64_t e = (int64_t) p * 1024 + 16 * lane;
                    const int64_t ec = e < K ? e : 0;  // clamped, masked below
                    wq[j][p] = *(const uint4 *) (wrow + ec);
                    ws[j][p] = ((const uint16_t *) (wrow + K))[ec / 32];
                    if (wrow2) {
                        wq2[j][p] = *(const uint4 *) (wrow2 + ec);
                        ws2[j][p] = ((const uint16_t *) (wrow2 + K))[ec / 32];
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < R; j++) {
            const int64_t rr = row0 + j < M ? row0 + j : 0;
            res[j] = res2[j] = 0.0f;
            if (resp && lane == 0) res[j] = *(const float *) (resp + rr * 4);
            if (a.epi.res2 && lane == 0) res2[j] = *(const float *) (a.epi.res2 + rr * 4);
        }
    };
    const int8_t * aq;
    const float * adp;
    if constexpr (PRO != kProNone) {
        if constexpr (PRO == kProQuant) gemv_stage_quant<GGML_TYPE_Q8_0>(a, 0, 1, smem, issue);
        else gemv_stage_norm<GGML_TYPE_Q8_0, PRO == kProNormBias>(a, 0, 1, smem, issue);
        const gemv_lds L = gemv_lds_layout(GGML_TYPE_Q8_0, K, 1);
        aq = (const int8_t *) (smem + L.q_off);
        adp = (const float *) (smem + L.d_off);
    } else {
        issue();
        aq = a.aq;
        adp = a.ad;
    }
    if (!wave_ok) return;  // after the prologue's barriers
    double acc[R], acc2[R];
#pragma unroll
    for (int j = 0; j < R; j++) acc[j] = acc2[j] = 0.0;
#pragma unroll
    for (int p = 0; p < kG1MaxPasses; p++) {
        if (p < passes) {
            const int64_t e = (int64_t) p * 1024 + 16 * lane;
            const bool ok = e < K;
            const int64_t ec = ok ? e : 0;
            const uint4 av = *(const uint4 *) (aq + ec);
            const float da = adp[ec / 32];
            auto term = [&](const uint4 & w, uint16_t sc, double & s) {
                int h = dot4_i8((int) w.x, (int) av.x, 0);
                h = dot4_i8((int) w.y, (int) av.y, h);
                h = dot4_i8((int) w.z, (int) av.z, h);
                h = dot4_i8((int) w.w, (int) av.w, h);
                h = ok ? h : 0;
                const int isum = h + dpp_i<kDppXor1>(h);  // the block's two halves, exact
                // |isum| < 2^19 and d_w * d_a has 22 significant bits: the product is exact
                if ((lane & 1) == 0 && ok) s = fma((double) isum, (double) (half_bits_to_float(sc) * da), s);
            };
#pragma unroll
            for (int j = 0; j < R; j++) {
                term(wq[j][p], ws[j][p], acc[j]);
                if (a.W2) term(wq2[j][p], ws2[j][p], acc2[j]);
            }
        }
    }
    auto wave_total = [&](double v) {
        v = row16_sum(v);
        double t = 0.0;
#pragma unroll
        for (int q = 0; q < 4; q++)
            t += __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 16 * q),
                                  __builtin_amdgcn_readlane(__double2loint(v), 16 * q));
        return t;
    };
#pragma unroll
    for (int j = 0; j < R; j++) {
        const double sum = wave_total(acc[j]);
        const double sum2 = a.W2 ? wave_total(acc2[j]) : 0.0;
        if (lane == 0 && row0 + j < M) {
            float v = (float) sum;
            if (a.W2) {
                const float u = (float) sum2;
                v = (v / (1.0f + expf_det(-v))) * u;
            }
            if (resp) v = res[j] + v;
            if (a.epi.res2) v = res2[j] + v;
            if (a.epi.gelu) v = half_bits_to_float(a.epi.gelu[float_to_half_bits(v)]);
            if (dst) *(float *) (dst + (row0 + j) * 4) = v;  // null: a sibling with only its cache row
            if (crow) crow[row0 + j] = float_to_half_bits(v);
        }
    }
}

bool gemv_single_column(int wtype, int64_t K, int64_t N, bool norm) {
    if (wtype != GGML_TYPE_Q8_0 || N != 1 || K % 32 != 0 || K > 1024LL * kG1MaxPasses) return false;
    return !norm || (K + 255) / 256 <= 4LL * kG1Waves * kNormGroups;  // one staging group a wave
}

bool gemv_mfma_supported(int wtype, int64_t M, int64_t K) {
    if (M % 16 != 0) return false;
    if (wtype == GGML_TYPE_Q4_K) return K % 256 == 0;
    if (wtype == GGML_TYPE_Q8_0) return K % 128 == 0;
    return false;
}

namespace {

int64_t gemv_units(int wtype, int64_t K) { return wtype == GGML_TYPE_Q4_K ? K / 256 : (K / 32 + kQ8Group - 1) / kQ8Group; }

// the streaming form: pre-quantized activations, one matrix, no residual, at
// most 8 full units a row (the LDS of two batches stays within 64 KB), and enough
// tiles that every CU walks several batches
bool gemv_stream_eligible(int wtype, int64_t M, int64_t K, int mode, bool dual, bool res, int n_cu) {
    if (mode != kProNone || dual || res || n_cu <= 0 || M % 16 != 0) return false;
    if (wtype == GGML_TYPE_Q8_0 && (K / 32) % kQ8Group != 0) return false;
    const int64_t units = gemv_units(wtype, K);
    return units >= 1 && units <= 8 && M / 16 >= 8LL * n_cu;
}

// waves of a launch: one per unit up to 16 (8 per matrix with W2); with a
// prologue, up to one staging group (four spans) per wave as well -- every
// wave stages, W2's included
int gemv_waves(int wtype, int64_t K, int64_t N, bool dual, int pro) {
    const int64_t units = gemv_units(wtype, K);
    const int64_t per = dual ? 8 : 16;
    const int64_t mats = dual ? 2 : 1;
    int64_t w = units < per ? units : per;
    if (pro != kProNone) {
        const int64_t nc = N < 16 ? N : 16;
        const int64_t groups = (nc * ((K + 255) / 256) + 3) / 4;
        const int64_t need = groups < 16 ? groups : 16;
        const int64_t wm = (need + mats - 1) / mats;
        if (w < wm) w = wm;
    }
    return (int) (w * mats);
}

// columns a workgroup takes: 16, or half as many, again, while the
// workgroups still run in one round -- the column chunks of a short matrix's
// tile then load (and, with a prologue, stage) their activations in parallel
// and re-read the tile's weights from L2. One workgroup a CU is the round,
// except while a prologue still gives a wave more than one staging group:
// then as many workgroups as fit a CU at 16 waves (the down projection).
int gemv_cols(int wtype, int64_t M, int64_t K, int64_t N, bool dual, int mode, int n_cu) {
    int cw = (int) (N < 16 ? N : 16);
    const int64_t nspan = (K + 255) / 256;
    while (cw > 1) {
        const int half = (cw + 1) / 2;
        const int64_t wgs = (M / 16) * ((N + half - 1) / half);
        int64_t round = n_cu;
        if (mode != kProNone) {
            const int64_t groups = (cw * nspan + 3) / 4;
            const int64_t per_cu = 16 / gemv_waves(wtype, K, half, dual, mode);
            if (groups > gemv_waves(wtype, K, cw, dual, mode) && per_cu > 1) round *= per_cu;
        }
        if (wgs > round) break;
        cw = half;
    }
    return cw;
}

// kernels compiled for at most 8 waves get twice the registers per lane
template <int PRO, int MAXW, int TPW>
void launch_kernel_w(int wtype, const dim3 & grid, const dim3 & block, size_t lds, hipStream_t stream,
                     const gemv_args & a) {
    static_assert(TPW == 1 || TPW == 2, "tiles a workgroup");
    const void * fn = wtype != GGML_TYPE_Q4_K ? (const void *) k_gemv_q8_0<PRO, MAXW>
                      : TPW == 2               ? (const void *) k_gemv_q4_K_pair<PRO, MAXW>
                                               : (const void *) k_gemv_q4_K<PRO, MAXW>;
    if (lds > 48 * 1024) {
        // staged columns beyond the default dynamic-LDS limit: raise it once per kernel
        static bool raised[2] = {false, false};  // per instantiation: Q4_K, Q8_0
        const int idx = wtype == GGML_TYPE_Q4_K ? 0 : 1;
        if (!raised[idx]) {
            MI_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 32768));
            raised[idx] = true;
        }
    }
    if (wtype != GGML_TYPE_Q4_K) hipLaunchKernelGGL((k_gemv_q8_0<PRO, MAXW>), grid, block, lds, stream, a);
    else if (TPW == 2) hipLaunchKernelGGL((k_gemv_q4_K_pair<PRO, MAXW>), grid, block, lds, stream, a);
    else hipLaunchKernelGGL((k_gemv_q4_K<PRO, MAXW>), grid, block, lds, stream, a);
}

// tpw: 16-row tiles a workgroup (2 only for Q4_K)
template <int PRO>
void launch_kernel(int wtype, const dim3 & grid, const dim3 & block, size_t lds, hipStream_t stream,
                   const gemv_args & a, int tpw) {
    if (block.x <= 512) {
        if (tpw == 2) launch_kernel_w<PRO, 8, 2>(wtype, grid, block, lds, stream, a);
        else launch_kernel_w<PRO, 8, 1>(wtype, grid, block, lds, stream, a);
    } else {
        if (tpw == 2) launch_kernel_w<PRO, 16, 2>(wtype, grid, block, lds, stream, a);
        else launch_kernel_w<PRO, 16, 1>(wtype, grid, block, lds, stream, a);
    }
}

}  // namespace

bool gemv_prologue_supported(int wtype, int64_t M, int64_t K, int64_t N, bool norm) {
    if (!gemv_mfma_supported(wtype, M, K) || N < 1) return false;
    const int64_t nc = N < 16 ? N : 16;
    const int64_t groups = (nc * ((K + 255) / 256) + 3) / 4;
    // the normalising prologue holds at most kNormGroups groups per wave, 16 waves
    if (norm && groups > 16 * kNormGroups) return false;
    // LDS: the staged columns plus the 32 KB reduction buffer within 160 KB
    return gemv_lds_layout(wtype, K, (int) nc).total + 32768 <= 160 * 1024;
}

void launch_gemv_mfma(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                      int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu, const char * res,
                      int64_t res_nb1, const char * W2, const gemv_prologue * pro, const gemv_epilogue & epi,
                      const gemv_sub * subs, int nsub) {
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
    a.epi = epi;
    a.nsub = 0;
    const int mode = !pro ? kProNone : pro->norm < 0 ? kProQuant : pro->b ? kProNormBias : kProNorm;
    if (pro) a.pro = *pro;
    a.cw = 16;
    const bool single = gemv_single_column(wtype, K, N, mode == kProNorm || mode == kProNormBias) &&
                        !gemv_stream_eligible(wtype, M, K, mode, W2 != nullptr, res != nullptr, n_cu);
    if ((epi.res2 || epi.gelu || nsub > 0) && !single) {  // only the single-column form has these
        note_hip_error(hipErrorInvalidValue);
        return;
    }
    if (single) {
        // one column: v_dot4 on the VALU, a wave per row (two for tall
        // matrices with a prologue: fewer workgroups repeat the staging)
        const bool tall = mode != kProNone && M >= 2048 && !W2 && nsub == 0;  // a SwiGLU pair already has two rows a wave
        const int rows_wg = kG1Waves * (tall ? 2 : 1);
        int64_t wgs = (M + rows_wg - 1) / rows_wg;
        if (nsub > kGemvMaxSubs || W2 || epi.res2 || epi.gelu) nsub = nsub > 0 ? -1 : 0;
        if (nsub < 0) {  // further matrices only beside a plain first one
            note_hip_error(hipErrorInvalidValue);
            return;
        }
        for (int q = 0; q < nsub; q++) {
            a.sub[q] = subs[q];
            a.sub_wg0[q] = wgs;
            wgs += (subs[q].M + rows_wg - 1) / rows_wg;
        }
        a.nsub = nsub;
        const dim3 grid((unsigned) wgs), block(64 * kG1Waves);
        const size_t lds = mode == kProNone ? 0 : (size_t) gemv_lds_layout(wtype, K, 1).total;
        auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, lds, stream, a); };
        if (tall) {
            switch (mode) {
                case kProQuant: go(k_gemv1_q8_0<kProQuant, kG1Waves, 2>); break;
                case kProNorm: go(k_gemv1_q8_0<kProNorm, kG1Waves, 2>); break;
                default: go(k_gemv1_q8_0<kProNormBias, kG1Waves, 2>); break;
            }
        } else {
            switch (mode) {
                case kProNone: go(k_gemv1_q8_0<kProNone, kG1Waves, 1>); break;
                case kProQuant: go(k_gemv1_q8_0<kProQuant, kG1Waves, 1>); break;
                case kProNorm: go(k_gemv1_q8_0<kProNorm, kG1Waves, 1>); break;
                default: go(k_gemv1_q8_0<kProNormBias, kG1Waves, 1>); break;
            }
        }
        return;
    }
    if (M % 16 != 0) {  // the tile forms need whole 16-row tiles (gemv_mfma_supported)
        note_hip_error(hipErrorInvalidValue);
        return;
    }
    if (gemv_stream_eligible(wtype, M, K, mode, W2 != nullptr, res != nullptr, n_cu)) {
        // tall matrix: a persistent grid of kStreamWgPerCu workgroups per CU walks the tiles
        const int64_t units = gemv_units(wtype, K);
        const int64_t batches = (M / 16 + kStreamTiles - 1) / kStreamTiles;
        const int64_t cap = (int64_t) kStreamWgPerCu * n_cu;
        const dim3 grid((unsigned) (batches < cap ? batches : cap), (unsigned) ((N + 15) / 16));
        const size_t lds = 2 * (size_t) kStreamTiles * units * 64 * 4 * sizeof(double);
        const bool one = N == 1;  // one column: a lane keeps one of its four
        const int which = (wtype == GGML_TYPE_Q4_K ? 0 : 2) + (one ? 1 : 0);
        const void * fns[4] = {(const void *) k_gemv_stream<GGML_TYPE_Q4_K, 4>,
                               (const void *) k_gemv_stream<GGML_TYPE_Q4_K, 1>,
                               (const void *) k_gemv_stream<GGML_TYPE_Q8_0, 4>,
                               (const void *) k_gemv_stream<GGML_TYPE_Q8_0, 1>};
        static bool raised[4] = {false, false, false, false};
        if (lds > 48 * 1024 && !raised[which]) {
            MI_CHECK(hipFuncSetAttribute(fns[which], hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024));
            raised[which] = true;
        }
        const dim3 block(64 * units);
        switch (which) {
            case 0: hipLaunchKernelGGL((k_gemv_stream<GGML_TYPE_Q4_K, 4>), grid, block, lds, stream, a); break;
            case 1: hipLaunchKernelGGL((k_gemv_stream<GGML_TYPE_Q4_K, 1>), grid, block, lds, stream, a); break;
            case 2: hipLaunchKernelGGL((k_gemv_stream<GGML_TYPE_Q8_0, 4>), grid, block, lds, stream, a); break;
            default: hipLaunchKernelGGL((k_gemv_stream<GGML_TYPE_Q8_0, 1>), grid, block, lds, stream, a); break;
        }
        return;
    }
    a.cw = gemv_cols(wtype, M, K, N, W2 != nullptr, mode, n_cu);
    const int waves = gemv_waves(wtype, K, a.cw, W2 != nullptr, mode);
    const int64_t chunks = (N + a.cw - 1) / a.cw;
    // Q4_K without a residual: two tiles a workgroup where one a workgroup
    // would take the CUs more than one round (16 / waves workgroups fit a CU;
    // the Qwen3-1.7B gate/up pair, 384 tiles of 16 waves)
    const int tpw = wtype == GGML_TYPE_Q4_K && !res && (M / 16) % 2 == 0 &&
                            (M / 16) * chunks > (int64_t) n_cu * (16 / waves)
                        ? 2 : 1;
    const dim3 grid((unsigned) (M / 16 / tpw), (unsigned) chunks);
    const dim3 block(64 * waves);
    const size_t lds = mode == kProNone ? 0 : (size_t) gemv_lds_layout(wtype, K, (int) (N < a.cw ? N : a.cw)).total;
    switch (mode) {
        case kProNone: launch_kernel<kProNone>(wtype, grid, block, lds, stream, a, tpw); break;
        case kProQuant: launch_kernel<kProQuant>(wtype, grid, block, lds, stream, a, tpw); break;
        case kProNorm: launch_kernel<kProNorm>(wtype, grid, block, lds, stream, a, tpw); break;
        default: launch_kernel<kProNormBias>(wtype, grid, block, lds, stream, a, tpw); break;
    }
}

}  // namespace mi355x

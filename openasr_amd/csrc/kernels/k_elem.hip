// k_elem.hip -- the small ops of the decoder step that keep the whole graph
// on device (nn/decoder.rs:1850-2145 for the LLM block, whisper
// ggml_decoder_graph.rs:3869-5392 for the seq2seq block): broadcast binary
// ops, scale, unary activations, RMSNorm / LayerNorm (optionally fused with
// the following weight multiply and bias add), RoPE, set_rows into the f16
// KV cache, get_rows from quantized tables, strided copies, soft_max_ext and
// argmax. All are HBM- or latency-bound; each is one pass over its data.
#include "../mi355x_common.h"
#include "../ops.h"

#include <algorithm>
#include "../quant_dev.h"

namespace mi355x {

__device__ __forceinline__ int64_t offs4(const tview & t, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    return i0 * t.nb[0] + i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}

__device__ __forceinline__ void unravel(int64_t idx, const int64_t * ne, int64_t & i0, int64_t & i1, int64_t & i2,
                                        int64_t & i3) {
    i0 = idx % ne[0];
    idx /= ne[0];
    i1 = idx % ne[1];
    idx /= ne[1];
    i2 = idx % ne[2];
    i3 = idx / ne[2];
}

// ------------------------------------------------------------- binary ----

template <int OP>
__device__ __forceinline__ float bin_apply(float x, float y) {
    if (OP == 0) return x + y;
    if (OP == 1) return x - y;
    if (OP == 2) return x * y;
    return x / y;
}

template <int OP>
__global__ void k_binary(tview d, tview a, tview b, int64_t n) {
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(idx, d.ne, i0, i1, i2, i3);
        const float x = *(const float *) (a.data + offs4(a, i0, i1, i2, i3));
        const float y = *(const float *) (b.data + offs4(b, i0 % b.ne[0], i1 % b.ne[1], i2 % b.ne[2], i3 % b.ne[3]));
        *(float *) (d.data + offs4(d, i0, i1, i2, i3)) = bin_apply<OP>(x, y);
    }
}

static unsigned grid_for(int64_t n, int threads, int n_cu) {
    int64_t blocks = (n + threads - 1) / threads;
    const int64_t cap = (int64_t) n_cu * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return (unsigned) blocks;
}

void launch_binary(int op, const tview & d, const tview & a, const tview & b, hipStream_t s, int n_cu) {
    const int64_t n = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    const unsigned g = grid_for(n, 256, n_cu);
    switch (op) {
        case GGML_OP_ADD: hipLaunchKernelGGL(k_binary<0>, dim3(g), dim3(256), 0, s, d, a, b, n); break;
        case GGML_OP_SUB: hipLaunchKernelGGL(k_binary<1>, dim3(g), dim3(256), 0, s, d, a, b, n); break;
        case GGML_OP_MUL: hipLaunchKernelGGL(k_binary<2>, dim3(g), dim3(256), 0, s, d, a, b, n); break;
        default: hipLaunchKernelGGL(k_binary<3>, dim3(g), dim3(256), 0, s, d, a, b, n); break;
    }
}

// -------------------------------------------------------- scale / unary --

__global__ void k_scale(tview d, tview a, float sc, float bias, int64_t n) {
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(idx, d.ne, i0, i1, i2, i3);
        const float x = *(const float *) (a.data + offs4(a, i0, i1, i2, i3));
        *(float *) (d.data + offs4(d, i0, i1, i2, i3)) = x * sc + bias;
    }
}

void launch_scale(const tview & d, const tview & a, float sc, float bias, hipStream_t s, int n_cu) {
    const int64_t n = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    hipLaunchKernelGGL(k_scale, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, d, a, sc, bias, n);
}

// ggml's gelu goes through a 64K-entry f16 table indexed by the f16 bits of
// x (ggml_vec_gelu_f32); the table is built on the host with the same libm
// tanhf and uploaded once, so device and host agree bit for bit.
__device__ __forceinline__ float unary_apply(int op, float x, const uint16_t * gelu_table) {
    switch (op) {
        case GGML_UNARY_OP_SILU: return x / (1.0f + expf_det(-x));
        case GGML_UNARY_OP_GELU: {
            if (x <= -10.0f) return 0.0f;
            if (x >= 10.0f) return x;
            return half_bits_to_float(gelu_table[float_to_half_bits(x)]);
        }
        case GGML_UNARY_OP_GELU_ERF: return gelu_erf_det(x);
        case GGML_UNARY_OP_RELU: return x > 0.0f ? x : 0.0f;
        case GGML_UNARY_OP_TANH: return tanhf(x);
        case GGML_UNARY_OP_SIGMOID: return 1.0f / (1.0f + expf_det(-x));
        case GGML_UNARY_OP_EXP: return expf_det(x);
        case GGML_UNARY_OP_NEG: return -x;
        case GGML_UNARY_OP_ABS: return fabsf(x);
        case kUnarySin:
        case kUnaryCos: {
            float sn, c;
            sincosf_det(x, sn, c);
            return op == kUnarySin ? sn : c;
        }
        default: return x;
    }
}

__global__ void k_unary(tview d, tview a, int op, const uint16_t * gelu_table, int64_t n) {
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(idx, d.ne, i0, i1, i2, i3);
        const float x = *(const float *) (a.data + offs4(a, i0, i1, i2, i3));
        *(float *) (d.data + offs4(d, i0, i1, i2, i3)) = unary_apply(op, x, gelu_table);
    }
}

void launch_unary(const tview & d, const tview & a, int op, const uint16_t * gelu_table, hipStream_t s, int n_cu) {
    const int64_t n = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    hipLaunchKernelGGL(k_unary, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, d, a, op, gelu_table, n);
}

// GGML_OP_CONCAT: d = a joined with b along dim (elements of esize bytes)
__global__ void k_concat(tview d, tview a, tview b, int dim, int esize, int64_t n) {
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t) gridDim.x * blockDim.x) {
        int64_t i[4];
        unravel(idx, d.ne, i[0], i[1], i[2], i[3]);
        const char * src;
        if (i[dim] < a.ne[dim]) {
            src = a.data + offs4(a, i[0], i[1], i[2], i[3]);
        } else {
            i[dim] -= a.ne[dim];
            src = b.data + offs4(b, i[0], i[1], i[2], i[3]);
            i[dim] += a.ne[dim];
        }
        char * dst = d.data + offs4(d, i[0], i[1], i[2], i[3]);
        if (esize == 4) *(uint32_t *) dst = *(const uint32_t *) src;
        else *(uint16_t *) dst = *(const uint16_t *) src;
    }
}

void launch_concat(const tview & d, const tview & a, const tview & b, int dim, int esize, hipStream_t s, int n_cu) {
    const int64_t n = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    hipLaunchKernelGGL(k_concat, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, d, a, b, dim, esize, n);
}

// SwiGLU tail fused: d = silu(g) * u (the gate activation and gate multiply
// of nn/ffn.rs:64-91), one pass instead of two.
__global__ void k_silu_mul(tview d, tview g, tview u, int64_t n) {
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(idx, d.ne, i0, i1, i2, i3);
        const float x = *(const float *) (g.data + offs4(g, i0, i1, i2, i3));
        const float y = *(const float *) (u.data + offs4(u, i0 % u.ne[0], i1 % u.ne[1], i2 % u.ne[2], i3 % u.ne[3]));
        *(float *) (d.data + offs4(d, i0, i1, i2, i3)) = (x / (1.0f + expf_det(-x))) * y;
    }
}

void launch_silu_mul(const tview & d, const tview & g, const tview & u, hipStream_t s, int n_cu) {
    const int64_t n = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    hipLaunchKernelGGL(k_silu_mul, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, d, g, u, n);
}

// ------------------------------------------------------------- norms -----

// One wave per row. mode 0: RMSNorm, 1: LayerNorm. Optional fused weight
// multiply (w broadcast over rows) and bias add, matching the
// rms_norm->mul and norm->mul->add sequences of nn/norm.rs:10-56. PER is the
// number of row elements each lane keeps in registers (the row, its weight
// and bias are read once, all loads issued before the sums); the fused
// weight / bias rows have the norm's width (planner check).
template <int PER>
__global__ __launch_bounds__(256) void k_norm(tview d, tview a, int mode, float eps, tview w, int has_w, tview bias,
                                              int has_b, int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t i1 = row % a.ne[1], i2 = (row / a.ne[1]) % a.ne[2], i3 = row / (a.ne[1] * a.ne[2]);
    const float * x = (const float *) (a.data + i1 * a.nb[1] + i2 * a.nb[2] + i3 * a.nb[3]);
    float * y = (float *) (d.data + i1 * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3]);
    const int n = (int) a.ne[0];
    const float * wr = has_w ? (const float *) (w.data + (i1 % w.ne[1]) * w.nb[1] + (i2 % w.ne[2]) * w.nb[2] +
                                                (i3 % w.ne[3]) * w.nb[3])
                             : nullptr;
    const float * br = has_b ? (const float *) (bias.data + (i1 % bias.ne[1]) * bias.nb[1] +
                                                (i2 % bias.ne[2]) * bias.nb[2] + (i3 % bias.ne[3]) * bias.nb[3])
                             : nullptr;
    float xv[PER], wv[PER], bv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = lane + 64 * k;
        const bool ok = i < n;
        xv[k] = ok ? x[i] : 0.0f;
        wv[k] = ok && has_w ? wr[i] : 1.0f;
        bv[k] = ok && has_b ? br[i] : 0.0f;
    }
    // sums in f64 and one rounding, as ggml-cpu's ggml_float accumulators
    float mean = 0.0f;
    if (mode == 1) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < PER; k++) s += (double) xv[k];
        mean = (float) (wave_sum_d(s) / (double) n);
    }
    double s2 = 0.0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        if (lane + 64 * k < n) {
            const float v = xv[k] - mean;
            s2 += (double) (v * v);
        }
    }
    const float var = (float) (wave_sum_d(s2) / (double) n);
    const float scale = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = lane + 64 * k;
        float v = (xv[k] - mean) * scale;
        if (has_w) v *= wv[k];
        if (has_b) v += bv[k];
        if (i < n) y[i] = v;
    }
}

// Rows whose width is a multiple of 256 with contiguous elements and 1-D
// weight / bias vectors: one workgroup per row, its W waves take the row's
// 256-element chunks round-robin, lane l holding elements 256c + 4l .. +3
// (16-byte loads) -- the layout the activation quantizers expect, so the
// normalised row can also be written as the quantized activations of the
// MUL_MAT that consumes it (qtype: -1 none, Q8_0, or Q4_K for Q8_K). The f32
// row is always written. The waves' f64 partial sums are added in wave order.
template <int C, int W>
__global__ __launch_bounds__(256) void k_norm_rows(tview d, tview a, int mode, float eps, const float * __restrict__ wr,
                                                   const float * __restrict__ br, int qtype, act_buffers act) {
    constexpr int CPW = C / W;  // chunks per wave
    __shared__ double s_part[2][W];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = blockIdx.x;
    const int64_t i1 = row % a.ne[1], i2 = (row / a.ne[1]) % a.ne[2], i3 = row / (a.ne[1] * a.ne[2]);
    const float * x = (const float *) (a.data + i1 * a.nb[1] + i2 * a.nb[2] + i3 * a.nb[3]);
    float * y = (float *) (d.data + i1 * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3]);
    constexpr int n = 256 * C;
    float4 xv[CPW], wv[CPW], bv[CPW];
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        const int i = 256 * (wave + W * k) + 4 * lane;
        xv[k] = *(const float4 *) (x + i);
        wv[k] = wr ? *(const float4 *) (wr + i) : make_float4(1.f, 1.f, 1.f, 1.f);
        bv[k] = br ? *(const float4 *) (br + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mean = 0.0f;
    if (mode == 1) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < CPW; k++) s += (((double) xv[k].x + (double) xv[k].y) + (double) xv[k].z) + (double) xv[k].w;
        s = wave_sum_d(s);
        if (lane == 0) s_part[0][wave] = s;
        __syncthreads();
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < W; w++) t += s_part[0][w];
        mean = (float) (t / (double) n);
    }
    double s2 = 0.0;
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        const float vx = xv[k].x - mean, vy = xv[k].y - mean, vz = xv[k].z - mean, vw = xv[k].w - mean;
        s2 += (((double) (vx * vx) + (double) (vy * vy)) + (double) (vz * vz)) + (double) (vw * vw);
    }
    s2 = wave_sum_d(s2);
    if (lane == 0) s_part[1][wave] = s2;
    __syncthreads();
    double t2 = 0.0;
#pragma unroll
    for (int w = 0; w < W; w++) t2 += s_part[1][w];
    const float var = (float) (t2 / (double) n);
    const float scale = 1.0f / sqrtf(var + eps);
    const int64_t col = row;
#pragma unroll
    for (int k = 0; k < CPW; k++) {
        const int c = wave + W * k;
        float4 v;
        v.x = (xv[k].x - mean) * scale;
        v.y = (xv[k].y - mean) * scale;
        v.z = (xv[k].z - mean) * scale;
        v.w = (xv[k].w - mean) * scale;
        if (wr) {
            v.x *= wv[k].x;
            v.y *= wv[k].y;
            v.z *= wv[k].z;
            v.w *= wv[k].w;
        }
        if (br) {
            v.x += bv[k].x;
            v.y += bv[k].y;
            v.z += bv[k].z;
            v.w += bv[k].w;
        }
        const int e = 256 * c + 4 * lane;
        *(float4 *) (y + e) = v;
        if (qtype == GGML_TYPE_Q4_K) {
            const q8_K_lane o = quantize_q8_K_wave(v, lane);
            *(char4 *) (act.q + col * n + e) = o.q;
            if ((lane & 7) == 0) act.ssum[col * (n / 32) + e / 32] = (int16_t) o.ssum;
            if (lane == 0) act.d[col * C + c] = o.d;
        } else if (qtype == GGML_TYPE_Q8_0) {
            const q8_0_lane o = quantize_q8_0_group(v);
            *(char4 *) (act.q + col * n + e) = o.q;
            if ((lane & 7) == 0) act.d[col * (n / 32) + e / 32] = o.d;
        }
    }
}

bool norm_supported(int64_t ne0) { return ne0 <= 64 * 64; }

// measurement helper: occupies the stream for a bounded time (the loop ends
// when the constant-rate wall clock has advanced by `ticks`)
__global__ void k_spin(uint64_t ticks) {
    const uint64_t t0 = wall_clock64();
    while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

void launch_spin_us(double us, int wall_clock_khz, hipStream_t s) {
    const uint64_t ticks = (uint64_t) (us * (double) wall_clock_khz / 1000.0);
    hipLaunchKernelGGL(k_spin, dim3(1), dim3(64), 0, s, ticks);
}

bool norm_rows_supported(const tview & d, const tview & a, const tview * w, const tview * b) {
    const int64_t n = a.ne[0];
    if (n % 256 != 0 || n / 256 > 16) return false;
    const int c = (int) (n / 256);
    if (c != 1 && c != 2 && c != 4 && c != 6 && c != 8 && c != 12 && c != 16) return false;
    if (a.nb[0] != 4 || d.nb[0] != 4) return false;
    if ((((uintptr_t) a.data) | ((uintptr_t) d.data) | a.nb[1] | a.nb[2] | a.nb[3] | d.nb[1] | d.nb[2] | d.nb[3]) % 16)
        return false;
    for (const tview * v : {w, b}) {
        if (!v) continue;
        if (v->ne[1] != 1 || v->ne[2] != 1 || v->ne[3] != 1 || v->nb[0] != 4 || ((uintptr_t) v->data) % 16) return false;
    }
    return true;
}

void launch_norm(const tview & d, const tview & a, int mode, float eps, const tview * w, const tview * b,
                 hipStream_t s, int qtype, const act_buffers * act) {
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    const dim3 grid((unsigned) ((rows + 3) / 4));
    if (norm_rows_supported(d, a, w, b)) {
        const float * wp = w ? (const float *) w->data : nullptr;
        const float * bp = b ? (const float *) b->data : nullptr;
        const act_buffers ab = act ? *act : act_buffers{nullptr, nullptr, nullptr};
        const int qt = act ? qtype : -1;
        const dim3 g1((unsigned) rows);
        switch (a.ne[0] / 256) {
            case 1: hipLaunchKernelGGL((k_norm_rows<1, 1>), g1, dim3(64), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
            case 2: hipLaunchKernelGGL((k_norm_rows<2, 2>), g1, dim3(128), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
            case 4: hipLaunchKernelGGL((k_norm_rows<4, 4>), g1, dim3(256), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
            case 6: hipLaunchKernelGGL((k_norm_rows<6, 2>), g1, dim3(128), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
            case 8: hipLaunchKernelGGL((k_norm_rows<8, 4>), g1, dim3(256), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
            case 12: hipLaunchKernelGGL((k_norm_rows<12, 4>), g1, dim3(256), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
            default: hipLaunchKernelGGL((k_norm_rows<16, 4>), g1, dim3(256), 0, s, d, a, mode, eps, wp, bp, qt, ab); return;
        }
    }
    const int per = (int) ((a.ne[0] + 63) / 64);
    tview none{};
    const tview wv = w ? *w : none, bv = b ? *b : none;
    const int hw = w ? 1 : 0, hb = b ? 1 : 0;
    if (per <= 2) hipLaunchKernelGGL(k_norm<2>, grid, dim3(256), 0, s, d, a, mode, eps, wv, hw, bv, hb, rows);
    else if (per <= 6) hipLaunchKernelGGL(k_norm<6>, grid, dim3(256), 0, s, d, a, mode, eps, wv, hw, bv, hb, rows);
    else if (per <= 16) hipLaunchKernelGGL(k_norm<16>, grid, dim3(256), 0, s, d, a, mode, eps, wv, hw, bv, hb, rows);
    else if (per <= 32) hipLaunchKernelGGL(k_norm<32>, grid, dim3(256), 0, s, d, a, mode, eps, wv, hw, bv, hb, rows);
    else hipLaunchKernelGGL(k_norm<64>, grid, dim3(256), 0, s, d, a, mode, eps, wv, hw, bv, hb, rows);
}

// RMSNorm * w followed by RoPE NEOX over full 128-wide rows (the per-head
// QK-norm then rotary embedding of nn/decoder.rs:1937-1968): one wave per
// row, lane l holds elements l and l + 64 -- exactly the NEOX pair of
// rotation index l -- so the row is normalised, scaled and rotated in
// registers. Same arithmetic as k_norm followed by k_rope.
// blockIdx.y selects the job: the query and key rows of one layer share a
// launch
__global__ __launch_bounds__(256) void k_rms_norm_rope128(norm_rope_job j0, norm_rope_job j1) {
    const norm_rope_job & j = blockIdx.y == 0 ? j0 : j1;
    const tview & a = j.a;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= j.rows) return;
    const int64_t i1 = row % a.ne[1], i2 = (row / a.ne[1]) % a.ne[2], i3 = row / (a.ne[1] * a.ne[2]);
    const float * x = (const float *) (a.data + i1 * a.nb[1] + i2 * a.nb[2] + i3 * a.nb[3]);
    float * y = (float *) (j.d.data + i1 * j.d.nb[1] + i2 * j.d.nb[2] + i3 * j.d.nb[3]);
    const float x0 = x[lane], x1 = x[lane + 64];
    const float w0 = j.w[lane], w1 = j.w[lane + 64];
    const float p = (float) j.pos[i2];
    const double s2 = wave_sum_d((double) (x0 * x0) + (double) (x1 * x1));
    const float var = (float) (s2 / 128.0);
    const float scale = 1.0f / sqrtf(var + j.eps);
    const float v0 = (x0 * scale) * w0, v1 = (x1 * scale) * w1;
    float theta = p;
    for (int k = 0; k < lane; k++) theta *= j.theta_scale;
    float sn, c;
    sincosf_det(j.freq_scale * theta, sn, c);
    c *= j.attn_factor;
    sn *= j.attn_factor;
    y[lane] = v0 * c - v1 * sn;
    y[lane + 64] = v0 * sn + v1 * c;
}

__global__ __launch_bounds__(64) void k_rope_table(float2 * table, const int32_t * pos, float theta_scale,
                                                   float freq_scale, float attn_factor) {
    const int lane = (int) threadIdx.x, seq = (int) blockIdx.x;
    float theta = (float) pos[seq];
    for (int k = 0; k < lane; k++) theta *= theta_scale;
    float sn, c;
    sincosf_det(freq_scale * theta, sn, c);
    table[seq * 64 + lane] = make_float2(c * attn_factor, sn * attn_factor);
}

void launch_rope_table(float2 * table, const int32_t * pos, int n_seq, float theta_scale, float freq_scale,
                       float attn_factor, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_table, dim3((unsigned) n_seq), dim3(64), 0, s, table, pos, theta_scale, freq_scale,
                       attn_factor);
}

void launch_rms_norm_rope128(const norm_rope_job & j0, const norm_rope_job * j1, hipStream_t s) {
    const int64_t rows = j1 && j1->rows > j0.rows ? j1->rows : j0.rows;
    hipLaunchKernelGGL(k_rms_norm_rope128, dim3((unsigned) ((rows + 3) / 4), j1 ? 2u : 1u), dim3(256), 0, s, j0,
                       j1 ? *j1 : j0);
}

norm_rope_job make_norm_rope_job(const tview & d, const tview & a, float eps, const float * w, const int32_t * pos,
                                 float freq_base, float freq_scale, float attn_factor) {
    norm_rope_job j;
    j.d = d;
    j.a = a;
    j.w = w;
    j.pos = pos;
    j.eps = eps;
    j.theta_scale = powf(freq_base, -2.0f / 128.0f);
    j.freq_scale = freq_scale;
    j.attn_factor = attn_factor;
    j.rows = a.ne[1] * a.ne[2] * a.ne[3];
    return j;
}

// -------------------------------------------------------------- rope -----

// ggml_rope_cache_init with ext_factor 0: theta_i = p * theta_scale^i built by
// repeated f32 multiplication, cos/sin scaled by attn_factor. NEOX rotates
// (x[i], x[i + n_dims/2]); NORMAL rotates (x[2i], x[2i+1]). Dims past n_dims
// pass through. One thread per rotated pair.
__global__ void k_rope(tview d, tview a, const int32_t * pos, int n_dims, int mode, float theta_scale,
                       float freq_scale, float attn_factor, int64_t n_pairs) {
    const int64_t half = n_dims / 2;
    for (int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; idx < n_pairs;
         idx += (int64_t) gridDim.x * blockDim.x) {
        const int64_t ic = idx % half;
        int64_t r = idx / half;
        const int64_t i1 = r % a.ne[1];
        r /= a.ne[1];
        const int64_t i2 = r % a.ne[2];
        const int64_t i3 = r / a.ne[2];
        float theta = (float) pos[i2];
        for (int64_t k = 0; k < ic; k++) theta *= theta_scale;
        const float th = freq_scale * theta;
        float sn, c;
        sincosf_det(th, sn, c);
        c *= attn_factor;
        sn *= attn_factor;
        const int64_t j0 = mode == GGML_ROPE_TYPE_NEOX ? ic : 2 * ic;
        const int64_t j1 = mode == GGML_ROPE_TYPE_NEOX ? ic + half : 2 * ic + 1;
        const char * xr = a.data + i1 * a.nb[1] + i2 * a.nb[2] + i3 * a.nb[3];
        char * yr = d.data + i1 * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3];
        const float x0 = *(const float *) (xr + j0 * a.nb[0]);
        const float x1 = *(const float *) (xr + j1 * a.nb[0]);
        *(float *) (yr + j0 * d.nb[0]) = x0 * c - x1 * sn;
        *(float *) (yr + j1 * d.nb[0]) = x0 * sn + x1 * c;
        if (ic == 0) {
            for (int64_t i = n_dims; i < a.ne[0]; i++) *(float *) (yr + i * d.nb[0]) = *(const float *) (xr + i * a.nb[0]);
        }
    }
}

void launch_rope(const tview & d, const tview & a, const int32_t * pos, int n_dims, int mode, float freq_base,
                 float freq_scale, float attn_factor, hipStream_t s, int n_cu) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    const int64_t n_pairs = (int64_t) (n_dims / 2) * a.ne[1] * a.ne[2] * a.ne[3];
    hipLaunchKernelGGL(k_rope, dim3(grid_for(n_pairs, 256, n_cu)), dim3(256), 0, s, d, a, pos, n_dims, mode,
                       theta_scale, freq_scale, attn_factor, n_pairs);
}

// ----------------------------------------------------------- set_rows ----

// dst[:, idx[i, i2 % ne11, i3 % ne12], i2, i3] = src[:, i, i2, i3], with f32 ->
// f16 round-to-nearest-even when the cache is f16 (KV write, nn/decoder.rs:2031-2036)
struct set_rows_job {
    tview dst, src, idx;
    int dtype, idx_is_i64;
    int64_t n;
};

// blockIdx.y selects the job: the K and V writes of one layer share a launch
__global__ void k_set_rows(set_rows_job j0, set_rows_job j1) {
    const set_rows_job & j = blockIdx.y == 0 ? j0 : j1;
    for (int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; t < j.n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, j.src.ne, i0, i1, i2, i3);
        const char * ip = j.idx.data + i1 * j.idx.nb[0] + (i2 % j.idx.ne[1]) * j.idx.nb[1] + (i3 % j.idx.ne[2]) * j.idx.nb[2];
        const int64_t r = j.idx_is_i64 ? *(const int64_t *) ip : (int64_t) *(const int32_t *) ip;
        const float v = *(const float *) (j.src.data + offs4(j.src, i0, i1, i2, i3));
        char * o = j.dst.data + i0 * j.dst.nb[0] + r * j.dst.nb[1] + i2 * j.dst.nb[2] + i3 * j.dst.nb[3];
        if (j.dtype == GGML_TYPE_F16) *(uint16_t *) o = float_to_half_bits(v);
        else *(float *) o = v;
    }
}

void launch_set_rows(const tview & dst, int dtype, const tview & src, const tview & idx, int idx_is_i64,
                     hipStream_t s, int n_cu, const tview * dst2, int dtype2, const tview * src2) {
    set_rows_job j0{dst, src, idx, dtype, idx_is_i64, src.ne[0] * src.ne[1] * src.ne[2] * src.ne[3]};
    set_rows_job j1 = j0;
    if (dst2) {
        j1.dst = *dst2;
        j1.src = *src2;
        j1.dtype = dtype2;
        j1.n = src2->ne[0] * src2->ne[1] * src2->ne[2] * src2->ne[3];
    }
    const int64_t n = j0.n > j1.n ? j0.n : j1.n;
    hipLaunchKernelGGL(k_set_rows, dim3(grid_for(n, 256, n_cu), dst2 ? 2 : 1), dim3(256), 0, s, j0, j1);
}

// ----------------------------------------------------------- get_rows ----

__device__ __forceinline__ float dequant_elem(int type, const char * row, int64_t K, int64_t i) {
    switch (type) {
        case GGML_TYPE_F32: return ((const float *) row)[i];
        case GGML_TYPE_F16: return half_bits_to_float(((const uint16_t *) row)[i]);
        case GGML_TYPE_Q8_0: {
            // row-split layout: quants first, then f16 scales
            const float dd = half_bits_to_float(((const uint16_t *) (row + K))[i / 32]);
            return dd * (float) ((const int8_t *) row)[i];
        }
        case GGML_TYPE_Q4_K: {
            const char * blk = row + (i / 256) * 144;
            const int e = (int) (i % 256);
            const int c = e / 64, l = e % 64;
            const int j = 2 * c + (l >= 32 ? 1 : 0);
            const uint8_t * s = (const uint8_t *) (blk + 4);
            int sc, m;
            if (j < 4) {
                sc = s[j] & 63;
                m = s[j + 4] & 63;
            } else {
                sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
                m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
            }
            const uint8_t qb = ((const uint8_t *) (blk + 16))[32 * c + (l % 32)];
            const int q = l >= 32 ? (qb >> 4) : (qb & 0xF);
            const float dd = half_bits_to_float(*(const uint16_t *) blk);
            const float dm = half_bits_to_float(*(const uint16_t *) (blk + 2));
            return dd * (float) sc * (float) q - dm * (float) m;
        }
        default: return 0.0f;
    }
}

// dst[:, i10, i11, i12] = src0[:, rows[i10, i11, i12], i11, i12] as f32
__global__ void k_get_rows(tview dst, tview src, int stype, tview idx, int64_t n) {
    for (int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, dst.ne, i0, i1, i2, i3);
        const int64_t r = *(const int32_t *) (idx.data + i1 * idx.nb[0] + i2 * idx.nb[1] + i3 * idx.nb[2]);
        const char * row = src.data + r * src.nb[1] + i2 * src.nb[2] + i3 * src.nb[3];
        float v;
        if (stype == GGML_TYPE_I32) {
            *(int32_t *) (dst.data + offs4(dst, i0, i1, i2, i3)) = ((const int32_t *) row)[i0];
            continue;
        }
        v = dequant_elem(stype, row, src.ne[0], i0);
        *(float *) (dst.data + offs4(dst, i0, i1, i2, i3)) = v;
    }
}

void launch_get_rows(const tview & dst, const tview & src, int stype, const tview & idx, hipStream_t s, int n_cu) {
    const int64_t n = dst.ne[0] * dst.ne[1] * dst.ne[2] * dst.ne[3];
    hipLaunchKernelGGL(k_get_rows, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, dst, src, stype, idx, n);
}

// --------------------------------------------------------------- copy ----

// element-order copy between any two layouts of equal element count, with
// f32 <-> f16 conversion (CPY, CONT, DUP)
__device__ __forceinline__ void copy_elems(const tview & d, int dtype, const tview & a, int atype, int64_t n) {
    for (int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, a.ne, i0, i1, i2, i3);
        const char * ip = a.data + offs4(a, i0, i1, i2, i3);
        int64_t j0, j1, j2, j3;
        unravel(t, d.ne, j0, j1, j2, j3);
        char * op = d.data + offs4(d, j0, j1, j2, j3);
        if (atype == dtype && atype == GGML_TYPE_I32) {
            *(int32_t *) op = *(const int32_t *) ip;
            continue;
        }
        const float v = atype == GGML_TYPE_F16 ? half_bits_to_float(*(const uint16_t *) ip) : *(const float *) ip;
        if (dtype == GGML_TYPE_F16) *(uint16_t *) op = float_to_half_bits(v);
        else *(float *) op = v;
    }
}

__global__ void k_copy(tview d, int dtype, tview a, int atype, int64_t n) { copy_elems(d, dtype, a, atype, n); }

// two such copies of n elements each in one launch (blockIdx.y: which)
__global__ void k_copy_pair(tview d0, tview a0, tview d1, tview a1, int dtype, int atype, int64_t n) {
    if (blockIdx.y == 0) copy_elems(d0, dtype, a0, atype, n);
    else copy_elems(d1, dtype, a1, atype, n);
}

// dense copies: 16 bytes per lane per iteration, grid-stride (same type), or
// four f32 -> four f16 (RNE) per lane
__global__ __launch_bounds__(256) void k_copy_dense(const uint4 * __restrict__ src, uint4 * __restrict__ dst,
                                                    int64_t n16) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t) gridDim.x * blockDim.x)
        dst[i] = src[i];
}

__global__ __launch_bounds__(256) void k_copy_f32_f16_dense(const float4 * __restrict__ src, uint2 * __restrict__ dst,
                                                            int64_t n4) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t) gridDim.x * blockDim.x) {
        const float4 v = src[i];
        dst[i] = make_uint2((uint32_t) float_to_half_bits(v.x) | ((uint32_t) float_to_half_bits(v.y) << 16),
                            (uint32_t) float_to_half_bits(v.z) | ((uint32_t) float_to_half_bits(v.w) << 16));
    }
}

static bool dense(const tview & v, int64_t esize) {
    return v.nb[0] == esize && v.nb[1] == v.ne[0] * v.nb[0] && v.nb[2] == v.ne[1] * v.nb[1] &&
           v.nb[3] == v.ne[2] * v.nb[2];
}

void launch_copy(const tview & d, int dtype, const tview & a, int atype, hipStream_t s, int n_cu) {
    const int64_t n = a.ne[0] * a.ne[1] * a.ne[2] * a.ne[3];
    const int64_t asz = atype == GGML_TYPE_F16 ? 2 : 4, dsz = dtype == GGML_TYPE_F16 ? 2 : 4;
    const bool aligned = ((uintptr_t) a.data | (uintptr_t) d.data) % 16 == 0;
    if (aligned && dense(a, asz) && dense(d, dsz)) {
        const int64_t blocks = 1024 * (int64_t) n_cu;  // one 16-byte piece per lane up to 256 Mi pieces
        if (atype == dtype && (n * asz) % 16 == 0) {
            const int64_t n16 = n * asz / 16;
            hipLaunchKernelGGL(k_copy_dense, dim3((unsigned) std::min<int64_t>(blocks, (n16 + 255) / 256)), dim3(256),
                               0, s, (const uint4 *) a.data, (uint4 *) d.data, n16);
            return;
        }
        if (atype == GGML_TYPE_F32 && dtype == GGML_TYPE_F16 && n % 4 == 0 && (uintptr_t) d.data % 8 == 0) {
            const int64_t n4 = n / 4;
            hipLaunchKernelGGL(k_copy_f32_f16_dense, dim3((unsigned) std::min<int64_t>(blocks, (n4 + 255) / 256)),
                               dim3(256), 0, s, (const float4 *) a.data, (uint2 *) d.data, n4);
            return;
        }
    }
    hipLaunchKernelGGL(k_copy, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, d, dtype, a, atype, n);
}

void launch_copy_pair(const tview & d0, const tview & a0, const tview & d1, const tview & a1, int dtype, int atype,
                      hipStream_t s, int n_cu) {
    const int64_t n = a0.ne[0] * a0.ne[1] * a0.ne[2] * a0.ne[3];
    if (n != a1.ne[0] * a1.ne[1] * a1.ne[2] * a1.ne[3]) {
        launch_copy(d0, dtype, a0, atype, s, n_cu);
        launch_copy(d1, dtype, a1, atype, s, n_cu);
        return;
    }
    hipLaunchKernelGGL(k_copy_pair, dim3(grid_for(n, 256, n_cu), 2), dim3(256), 0, s, d0, a0, d1, a1, dtype, atype, n);
}

// -------------------------------------------------------------- repeat ---

// ggml_repeat: dst[i] = src[i mod src.ne] per dim, elements of esize bytes
__global__ void k_repeat(tview d, tview a, int esize, int64_t n) {
    for (int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (int64_t) gridDim.x * blockDim.x) {
        int64_t i0, i1, i2, i3;
        unravel(t, d.ne, i0, i1, i2, i3);
        const char * ip = a.data + offs4(a, i0 % a.ne[0], i1 % a.ne[1], i2 % a.ne[2], i3 % a.ne[3]);
        char * op = d.data + offs4(d, i0, i1, i2, i3);
        if (esize == 4) *(uint32_t *) op = *(const uint32_t *) ip;
        else *(uint16_t *) op = *(const uint16_t *) ip;
    }
}

void launch_repeat(const tview & d, const tview & src, int esize, hipStream_t s, int n_cu) {
    const int64_t n = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    hipLaunchKernelGGL(k_repeat, dim3(grid_for(n, 256, n_cu)), dim3(256), 0, s, d, src, esize, n);
}

// ------------------------------------------------------------ soft_max ---

// ggml_compute_forward_soft_max_f32, max_bias 0: y = softmax(x*scale + mask)
__global__ __launch_bounds__(256) void k_soft_max(tview d, tview a, tview mask, int has_mask, float scale,
                                                  int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t i1 = row % a.ne[1], i2 = (row / a.ne[1]) % a.ne[2], i3 = row / (a.ne[1] * a.ne[2]);
    const float * x = (const float *) (a.data + i1 * a.nb[1] + i2 * a.nb[2] + i3 * a.nb[3]);
    float * y = (float *) (d.data + i1 * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3]);
    const uint16_t * mp = has_mask ? (const uint16_t *) (mask.data + i1 * mask.nb[1] + (i2 % mask.ne[2]) * mask.nb[2] +
                                                         (i3 % mask.ne[3]) * mask.nb[3])
                                   : nullptr;
    const int64_t n = a.ne[0];
    float mx = -INFINITY;
    for (int64_t i = lane; i < n; i += 64) {
        const float v = x[i] * scale + (mp ? half_bits_to_float(mp[i]) : 0.0f);
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    double sum = 0.0;
    for (int64_t i = lane; i < n; i += 64) {
        const float v = x[i] * scale + (mp ? half_bits_to_float(mp[i]) : 0.0f);
        const float e = expf_det(v - mx);
        y[i] = e;
        sum += (double) e;
    }
    sum = wave_sum_d(sum);
    const float inv = (float) (1.0 / sum);
    for (int64_t i = lane; i < n; i += 64) y[i] *= inv;
}

void launch_soft_max(const tview & d, const tview & a, const tview * mask, float scale, hipStream_t s) {
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    tview none{};
    hipLaunchKernelGGL(k_soft_max, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, s, d, a, mask ? *mask : none,
                       mask ? 1 : 0, scale, rows);
}

// -------------------------------------------------------------- argmax ---

// Two passes over 64-bit keys (order-preserving f32 bits in the high word,
// the index -- or its complement -- in the low word) so the maximum key is the
// wanted element: first == 1 keeps the lowest index of the maximum (OpenASR's
// first-max rule), first == 0 the highest (ggml_vec_argmax_f32). Pass 1: one
// workgroup per (row, 4096-element chunk); pass 2: one wave per row.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i, int first) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t) u << 32) | (first ? (0xFFFFFFFFu - i) : i);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

constexpr int kArgmaxChunk = 4096;

__global__ __launch_bounds__(256) void k_argmax_part(tview a, uint64_t * keys, int first, int chunks) {
    __shared__ uint64_t s_k[4];
    const int64_t row = blockIdx.y;
    const int chunk = blockIdx.x;
    const float * x = (const float *) (a.data + row * a.nb[1]);
    const int64_t n = a.ne[0];
    const int64_t i0 = (int64_t) chunk * kArgmaxChunk;
    const int64_t i1 = i0 + kArgmaxChunk < n ? i0 + kArgmaxChunk : n;
    // every load of the thread requested before the first key (clamped
    // index, masked); the launch is 256 threads, kArgmaxChunk / 256 each
    constexpr int kPer = kArgmaxChunk / 256;
    float v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; u++) {
        const int64_t i = i0 + threadIdx.x + 256 * u;
        v[u] = x[i < i1 ? i : i0];
    }
    uint64_t best = 0;
#pragma unroll
    for (int u = 0; u < kPer; u++) {
        const int64_t i = i0 + threadIdx.x + 256 * u;
        if (i < i1) best = max_u64(best, argmax_key(v[u], (uint32_t) i, first));
    }
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = ((uint64_t) __shfl_xor((unsigned) (best >> 32), off) << 32) |
                           (uint64_t) __shfl_xor((unsigned) best, off);
        best = max_u64(best, o);
    }
    if ((threadIdx.x & 63) == 0) s_k[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) keys[row * chunks + chunk] = max_u64(max_u64(s_k[0], s_k[1]), max_u64(s_k[2], s_k[3]));
}

__global__ void k_argmax_final(const uint64_t * keys, int chunks, int32_t * out, int first) {
    const int64_t row = blockIdx.x;
    uint64_t best = 0;
    for (int c = threadIdx.x; c < chunks; c += 64) best = max_u64(best, keys[row * chunks + c]);
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = ((uint64_t) __shfl_xor((unsigned) (best >> 32), off) << 32) |
                           (uint64_t) __shfl_xor((unsigned) best, off);
        best = max_u64(best, o);
    }
    if (threadIdx.x == 0) {
        const uint32_t lo = (uint32_t) best;
        out[row] = (int32_t) (first ? 0xFFFFFFFFu - lo : lo);
    }
}

size_t argmax_scratch_bytes(int64_t ne0, int64_t rows) {
    return (size_t) rows * (size_t) ((ne0 + kArgmaxChunk - 1) / kArgmaxChunk) * sizeof(uint64_t);
}

void launch_argmax(const tview & a, int32_t * out, int first, void * scratch, hipStream_t s) {
    const int chunks = (int) ((a.ne[0] + kArgmaxChunk - 1) / kArgmaxChunk);
    uint64_t * keys = (uint64_t *) scratch;
    hipLaunchKernelGGL(k_argmax_part, dim3((unsigned) chunks, (unsigned) a.ne[1]), dim3(256), 0, s, a, keys, first,
                       chunks);
    hipLaunchKernelGGL(k_argmax_final, dim3((unsigned) a.ne[1]), dim3(64), 0, s, keys, chunks, out, first);
}

// ---------------------------------------------------- float mul_mat ------

// dst[m, n, i2, i3] = sum_k src0[k, m, i2/r2, i3/r3] * src1[k, n, i2, i3]
// for f16 / f32 src0 (ggml-cpu rounds src1 to f16 for an f16 src0). One wave
// per output element; used by the non-flash attention fallback and small
// float weights, never by the quantized hot path.
__global__ __launch_bounds__(256) void k_mul_mat_float(tview d, tview a, int atype, tview b, int64_t total) {
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= total) return;
    int64_t m, n, i2, i3;
    unravel(wid, d.ne, m, n, i2, i3);
    const int64_t r2 = d.ne[2] / a.ne[2], r3 = d.ne[3] / a.ne[3];
    const char * ar = a.data + m * a.nb[1] + (i2 / r2) * a.nb[2] + (i3 / r3) * a.nb[3];
    const char * br = b.data + n * b.nb[1] + i2 * b.nb[2] + i3 * b.nb[3];
    float s = 0.0f;
    for (int64_t k = lane; k < a.ne[0]; k += 64) {
        float bv = *(const float *) (br + k * b.nb[0]);
        float av;
        if (atype == GGML_TYPE_F16) {
            av = half_bits_to_float(*(const uint16_t *) (ar + k * a.nb[0]));
            bv = round_to_half(bv);
        } else {
            av = *(const float *) (ar + k * a.nb[0]);
        }
        s += av * bv;
    }
    s = wave_sum(s);
    if (lane == 0) *(float *) (d.data + m * d.nb[0] + n * d.nb[1] + i2 * d.nb[2] + i3 * d.nb[3]) = s;
}

void launch_mul_mat_float(const tview & d, const tview & a, int atype, const tview & b, hipStream_t s) {
    const int64_t total = d.ne[0] * d.ne[1] * d.ne[2] * d.ne[3];
    hipLaunchKernelGGL(k_mul_mat_float, dim3((unsigned) ((total + 3) / 4)), dim3(256), 0, s, d, a, atype, b, total);
}

}  // namespace mi355x

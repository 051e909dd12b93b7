// fattn_dev.h -- device helpers shared by the attention kernels
// (k_fattn.hip, k_fattn_dec.hip): the tile a workgroup owns and the
// quantization of its output rows into the activation layout of the
// MUL_MAT that consumes them (the attention output projection).
#pragma once

#include "mi355x_common.h"
#include "ops.h"
#include "quant_dev.h"

namespace mi355x {

struct fa_tile {
    int kvh, seq, g, tq0, ntq, nrows, kv_seq, gti;
};

// the tile's output rows are in LDS (row r at rows + r * D); quantize its
// column segments for the next MUL_MAT (Q8_K for Q4_K weights, Q8_0 for Q8_0
// weights); waves 0 .. NW - 1 of the workgroup take the 256-element pieces
// in turn (waves from NW on take none)
template <int D, int NW = 4>
__device__ __forceinline__ void fa_quantize_out(const fattn_args & a, const fa_tile & t, const float * rows) {
    const int lane = (int) threadIdx.x & 63, wave = (int) threadIdx.x >> 6;
    const int seg = t.g * D;
    const int64_t K = (int64_t) a.hq * D;
    const int64_t e0 = (int64_t) t.kvh * seg;
    for (int tql = 0; tql < t.ntq; tql++) {
        const int64_t col = (int64_t) t.seq * a.n_q + t.tq0 + tql;
        const float * row = rows + (int64_t) tql * t.g * D;
        for (int piece = wave; piece * 256 < seg; piece += NW) {
            const int e = piece * 256 + lane * 4;
            const float4 v = e < seg ? *(const float4 *) (row + e) : make_float4(0.f, 0.f, 0.f, 0.f);
            if (a.qtype == GGML_TYPE_Q4_K) {
                const q8_K_lane o = quantize_q8_K_wave(v, lane);
                *(char4 *) (a.act.q + col * K + e0 + e) = o.q;
                if ((lane & 7) == 0) a.act.ssum[col * (K / 32) + (e0 + e) / 32] = (int16_t) o.ssum;
                if (lane == 0) a.act.d[col * (K / 256) + (e0 + piece * 256) / 256] = o.d;
            } else {
                const q8_0_lane o = quantize_q8_0_group(v);
                if (e < seg) {
                    *(char4 *) (a.act.q + col * K + e0 + e) = o.q;
                    if ((lane & 7) == 0) a.act.d[col * (K / 32) + (e0 + e) / 32] = o.d;
                }
            }
        }
    }
}

// RMS norm * w, then NEOX RoPE by a (cos, sin) pair, of one 128-element row
// held by a wave (lane l: elements l and l + 64, rotation index l) -- the
// arithmetic of k_rms_norm_rope128 with the angle from the rope table
__device__ __forceinline__ void as_norm_rope(float x0, float x1, float w0, float w1, float2 cs, float eps, float & y0,
                                             float & y1) {
    const double s2 = wave_sum_d((double) (x0 * x0) + (double) (x1 * x1));
    const float var = (float) (s2 / 128.0);
    const float scale = 1.0f / sqrtf(var + eps);
    const float v0 = (x0 * scale) * w0, v1 = (x1 * scale) * w1;
    y0 = v0 * cs.x - v1 * cs.y;
    y1 = v0 * cs.y + v1 * cs.x;
}

// STEP: the wave holding this step's position (jn >= 0) writes the new K / V
// rows into the f16 caches (SET_ROWS). Called last: stores issued after the
// K/V burst whose data registers were then reused would make the compiler
// wait for every request of the burst.
__device__ __forceinline__ void fa_decode_set_rows(const attn_step_args & st, int jn, int64_t r_new, int kvh, int seq,
                                                   int lane, uint16_t k0, uint16_t k1, uint16_t v0, uint16_t v1) {
    if (jn < 0) return;
    if (r_new < st.kc_rows) {
        uint16_t * kd = (uint16_t *) (st.kc + r_new * st.kc_nb1 + (int64_t) kvh * st.kc_nb2 + (int64_t) seq * st.kc_nb3);
        kd[lane] = k0;
        kd[lane + 64] = k1;
    }
    if (r_new < st.vc_rows) {
        uint16_t * vd = (uint16_t *) (st.vc + r_new * st.vc_nb1 + (int64_t) kvh * st.vc_nb2 + (int64_t) seq * st.vc_nb3);
        vd[lane] = v0;
        vd[lane + 64] = v1;
    }
}

}  // namespace mi355x

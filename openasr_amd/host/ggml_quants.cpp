// ggml_quants.cpp -- weight quantization of this build's ggml-base:
// ggml_quantize_chunk for Q8_0 and Q4_K (called by the host's pack writer,
// crates/openasr-core/src/ggml_runtime/gguf_write.rs:579-588, with a NULL
// importance matrix), and the f16 conversions.
//
// Q8_0 follows ggml-base's reference rule (d = amax/127, quants rounded half
// away from zero); Q4_K is ggml-base's quantize_row_q4_K_ref (eight 32-weight
// sub-blocks with 6-bit scales and mins under f16 super-block scales, the
// ggml-common.h block_q4_K layout). The ggml fork (pinned revision
// 0db3a287511085fb1564fea3f86839f9e40ca39e, model-registry/catalog.public.json:3941)
// is not part of the reference tree: both are restated from ggml's published
// algorithms.

#include <cmath>
#include <cstdint>
#include <cstring>

#include "ggml_host.h"

namespace {

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t) (sign | (uint32_t) std::nearbyint(a * 16777216.0f));
    }
    const uint32_t mant = ax & 0x7fffffu, rem = mant & 0x1fffu;
    uint32_t h = (((ax >> 23) - 112u) << 10) | (mant >> 13);
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t) (sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float) m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

int rne(float v) { return (int) std::nearbyint(v); }

void quantize_row_q8_0(const float * x, uint8_t * y, int64_t k) {
    for (int64_t b = 0; b < k / 32; b++) {
        const float * xb = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = std::fmax(amax, std::fabs(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = f32_to_f16(d);
        uint8_t * o = y + 34 * b;
        std::memcpy(o, &dh, 2);
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t) (int8_t) std::round(xb[j] * id);
    }
}

// Q4_K: the super-block quantizer ggml_quantize_chunk runs for a NULL
// importance matrix (quantize_row_q4_K_ref, ggml-quants.c of the pinned
// ggml revision), in float arithmetic in ggml's operation order. Per
// 32-weight sub-block, a weighted fit x ~ step * q + low (low <= 0, q in
// 0..15; weights rms + |x|): a first fit from the value range, then 21
// candidate inverse steps (14 + 0.1 i) / range, each rounding q and solving
// the weighted least squares for (step, low) -- low clamped to 0 with the
// step refitted -- the first strictly better weighted squared error
// replacing the current fit.
struct sub_fit {
    float step, neg_low;
};

sub_fit fit_sub_block(const float * x, const float * w, uint8_t * q) {
    constexpr int n = 32, qmax = 15, steps = 20;
    float lo = x[0], hi = x[0], sw = 0.0f, swx = 0.0f;
    for (int i = 0; i < n; i++) {
        lo = x[i] < lo ? x[i] : lo;
        hi = x[i] > hi ? x[i] : hi;
        sw += w[i];
        swx += w[i] * x[i];
    }
    lo = lo > 0.0f ? 0.0f : lo;
    if (hi == lo) {
        std::memset(q, 0, n);
        return {0.0f, -lo};
    }
    auto clamp_q = [](int v) { return (uint8_t) (v < 0 ? 0 : (v > qmax ? qmax : v)); };
    float inv = (float) qmax / (hi - lo);
    float step = 1.0f / inv;
    float err_best = 0.0f;
    for (int i = 0; i < n; i++) {
        q[i] = clamp_q(rne(inv * (x[i] - lo)));
        const float e = step * (float) q[i] + lo - x[i];
        err_best += w[i] * (e * e);
    }
    uint8_t cand[n];
    for (int t = 0; t <= steps; t++) {
        inv = (-1.0f + 0.1f * (float) t + (float) qmax) / (hi - lo);
        float swq = 0.0f, swqq = 0.0f, swqx = 0.0f;
        for (int i = 0; i < n; i++) {
            cand[i] = clamp_q(rne(inv * (x[i] - lo)));
            const float wq = w[i] * (float) cand[i];
            swq += wq;
            swqq += wq * (float) cand[i];
            swqx += wq * x[i];
        }
        const float det = sw * swqq - swq * swq;
        if (!(det > 0.0f)) continue;
        float s = (sw * swqx - swx * swq) / det;
        float low = (swqq * swx - swq * swqx) / det;
        if (low > 0.0f) {
            low = 0.0f;
            s = swqx / swqq;
        }
        float err = 0.0f;
        for (int i = 0; i < n; i++) {
            const float e = s * (float) cand[i] + low - x[i];
            err += w[i] * (e * e);
        }
        if (err < err_best) {
            std::memcpy(q, cand, n);
            err_best = err;
            step = s;
            lo = low;
        }
    }
    return {step, -lo};
}

void quantize_row_q4_K(const float * x, uint8_t * y, int64_t k) {
    for (int64_t sb = 0; sb < k / 256; sb++) {
        const float * xb = x + 256 * sb;
        uint8_t * o = y + 144 * sb;
        uint8_t q[256];
        sub_fit f[8];
        float max_step = 0.0f, max_off = 0.0f;
        for (int j = 0; j < 8; j++) {
            const float * xs = xb + 32 * j;
            float sq = 0.0f;
            for (int l = 0; l < 32; l++) sq += xs[l] * xs[l];
            const float rms = std::sqrt(sq / 32.0f);
            float w[32];
            for (int l = 0; l < 32; l++) w[l] = rms + std::fabs(xs[l]);
            f[j] = fit_sub_block(xs, w, q + 32 * j);
            max_step = f[j].step > max_step ? f[j].step : max_step;
            max_off = f[j].neg_low > max_off ? f[j].neg_low : max_off;
        }
        const float is = max_step > 0 ? 63.0f / max_step : 0.0f;
        const float io = max_off > 0 ? 63.0f / max_off : 0.0f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            const int a = rne(is * f[j].step), b = rne(io * f[j].neg_low);
            ls[j] = (uint8_t) (a > 63 ? 63 : a);
            lm[j] = (uint8_t) (b > 63 ? 63 : b);
        }
        uint8_t * sc = o + 4;
        for (int j = 0; j < 4; j++) {
            sc[j] = (uint8_t) (ls[j] | ((ls[j + 4] >> 4) << 6));
            sc[j + 4] = (uint8_t) (lm[j] | ((lm[j + 4] >> 4) << 6));
            sc[j + 8] = (uint8_t) ((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
        }
        const uint16_t dh = f32_to_f16(max_step / 63.0f), mh = f32_to_f16(max_off / 63.0f);
        std::memcpy(o, &dh, 2);
        std::memcpy(o + 2, &mh, 2);
        const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
        // requantize against the coded step and offset; a sub-block whose
        // coded step is 0 keeps the fit's q
        for (int j = 0; j < 8; j++) {
            const float dd = d * (float) ls[j], dm = dmin * (float) lm[j];
            if (dd == 0.0f) continue;
            for (int l = 0; l < 32; l++) {
                const int v = rne((xb[32 * j + l] + dm) / dd);
                q[32 * j + l] = (uint8_t) (v < 0 ? 0 : (v > 15 ? 15 : v));
            }
        }
        uint8_t * qs = o + 16;
        for (int c = 0; c < 4; c++) {
            for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t) (q[64 * c + l] | (q[64 * c + 32 + l] << 4));
        }
    }
}

}  // namespace

extern "C" {

float ggml_fp16_to_fp32(ggml_fp16_t h) { return f16_to_f32(h); }
ggml_fp16_t ggml_fp32_to_fp16(float f) { return f32_to_f16(f); }

size_t ggml_quantize_chunk(enum ggml_type type, const float * src, void * dst, int64_t start, int64_t nrows,
                           int64_t n_per_row, const float * imatrix) {
    (void) imatrix;
    const int64_t row0 = start / n_per_row;
    const size_t rs = ggml_row_size(type, n_per_row);
    uint8_t * out = (uint8_t *) dst + (size_t) row0 * rs;
    const float * in = src + start;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; r++) {
        const float * xr = in + r * n_per_row;
        uint8_t * yr = out + (size_t) r * rs;
        switch (type) {
            case GGML_TYPE_Q8_0: quantize_row_q8_0(xr, yr, n_per_row); break;
            case GGML_TYPE_Q4_K: quantize_row_q4_K(xr, yr, n_per_row); break;
            case GGML_TYPE_F16:
                for (int64_t i = 0; i < n_per_row; i++) ((uint16_t *) yr)[i] = f32_to_f16(xr[i]);
                break;
            case GGML_TYPE_F32: std::memcpy(yr, xr, (size_t) n_per_row * 4); break;
            default: break;
        }
    }
    return (size_t) nrows * rs;
}

}  // extern "C"

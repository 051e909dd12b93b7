// ggml_quants.cpp -- weight quantization of this build's ggml-base:
// ggml_quantize_chunk for Q8_0 and Q4_K (called by the host's pack writer,
// crates/openasr-core/src/ggml_runtime/gguf_write.rs:579-588, with a NULL
// importance matrix), and the f16 conversions.
//
// Q8_0 follows ggml-base's reference rule (d = amax/127, quants rounded half
// away from zero). Q4_K packs eight 32-weight sub-blocks with 6-bit scales
// and mins under f16 super-block scales (the ggml-common.h block_q4_K
// layout); the per-sub-block (scale, min) is a least-squares fit over a grid
// of candidate step sizes. Kernel parity does not depend on which Q4_K bytes
// a quantizer picks: host and device consume the same bytes.

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

// least-squares (step, offset) for one 32-weight sub-block: x ~ step*q - offset, q in 0..15
void fit_sub_block(const float * x, float & step, float & offset) {
    float lo = x[0], hi = x[0];
    for (int i = 1; i < 32; i++) {
        lo = std::fmin(lo, x[i]);
        hi = std::fmax(hi, x[i]);
    }
    lo = std::fmin(lo, 0.0f);
    if (hi <= lo) {
        step = 0.0f;
        offset = -lo;
        return;
    }
    double best_err = INFINITY;
    float bs = (hi - lo) / 15.0f, bo = -lo;
    for (int t = -10; t <= 10; t++) {
        const float inv = (15.0f + 0.1f * (float) t) / (hi - lo);
        int q[32];
        double sq = 0, sx = 0, sqq = 0, sqx = 0;
        for (int i = 0; i < 32; i++) {
            int v = rne(inv * (x[i] - lo));
            v = v < 0 ? 0 : (v > 15 ? 15 : v);
            q[i] = v;
            sq += v;
            sx += x[i];
            sqq += (double) v * v;
            sqx += (double) v * x[i];
        }
        const double det = 32.0 * sqq - sq * sq;
        if (det <= 0) continue;
        double s = (32.0 * sqx - sq * sx) / det;
        double m = (sx - s * sq) / 32.0;  // x ~ s*q + m with m <= 0
        if (m > 0) {
            m = 0;
            s = sqq > 0 ? sqx / sqq : 0;
        }
        if (s <= 0) continue;
        double err = 0;
        for (int i = 0; i < 32; i++) {
            const double e = s * q[i] + m - x[i];
            err += e * e;
        }
        if (err < best_err) {
            best_err = err;
            bs = (float) s;
            bo = (float) -m;
        }
    }
    step = bs;
    offset = bo;
}

void quantize_row_q4_K(const float * x, uint8_t * y, int64_t k) {
    for (int64_t sb = 0; sb < k / 256; sb++) {
        const float * xb = x + 256 * sb;
        uint8_t * o = y + 144 * sb;
        float step[8], off[8], max_step = 0.0f, max_off = 0.0f;
        for (int j = 0; j < 8; j++) {
            fit_sub_block(xb + 32 * j, step[j], off[j]);
            max_step = std::fmax(max_step, step[j]);
            max_off = std::fmax(max_off, off[j]);
        }
        const float is = max_step > 0 ? 63.0f / max_step : 0.0f;
        const float io = max_off > 0 ? 63.0f / max_off : 0.0f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            const int a = rne(is * step[j]), b = rne(io * off[j]);
            ls[j] = (uint8_t) (a < 0 ? 0 : (a > 63 ? 63 : a));
            lm[j] = (uint8_t) (b < 0 ? 0 : (b > 63 ? 63 : b));
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
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            const float dd = d * ls[j], dm = dmin * lm[j];
            for (int l = 0; l < 32; l++) {
                int v = 0;
                if (dd != 0.0f) {
                    v = rne((xb[32 * j + l] + dm) / dd);
                    v = v < 0 ? 0 : (v > 15 ? 15 : v);
                }
                q[32 * j + l] = (uint8_t) v;
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

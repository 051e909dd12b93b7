// GGML_OP_IM2COL: the column matrix of a 2-D (or 1-D) convolution, the
// first half of ggml_conv_2d as the Qwen audio encoder's stem uses it
// (nn/conv.rs:82-110, cpu_graph.rs:5191-5246). Pure index work: one lane per
// output element, so the f16/f32 stores of consecutive lanes are contiguous;
// the input gathers fall in the few rows a workgroup's outputs touch and are
// served from L2. A tap in the padding is written as zero; an in-range tap is
// copied (f32) or rounded to nearest-even (f16), bit-identical to ggml-cpu.

#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {
namespace {

template <typename DT>
__global__ __launch_bounds__(256) void k_im2col(DT * __restrict__ dst, const char * __restrict__ src, im2col_args a) {
    const int64_t stride = (int64_t) gridDim.x * 256;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < a.total; i += stride) {
        const int64_t k = i % a.K;
        int64_t r = i / a.K;
        const int64_t ow = r % a.OW;
        r /= a.OW;
        const int64_t oh = r % a.OH;
        const int64_t n = r / a.OH;
        const int kw = (int) (k % a.KW);
        const int64_t t = k / a.KW;
        const int kh = (int) (t % a.KH);
        const int64_t ic = t / a.KH;
        const int64_t iw = ow * a.s0 + (int64_t) kw * a.d0 - a.p0;
        const int64_t ih = oh * a.s1 + (int64_t) kh * a.d1 - a.p1;
        float v = 0.0f;
        if (iw >= 0 && iw < a.IW && ih >= 0 && ih < a.IH)
            v = *(const float *) (src + n * a.nb_n + ic * a.nb_c + ih * a.nb_h + iw * 4);
        dst[i] = (DT) v;
    }
}

}  // namespace

void launch_im2col(void * dst, int dst_f16, const char * src, const im2col_args & a, hipStream_t s) {
    if (a.total <= 0) return;
    const int64_t g = std::min<int64_t>((a.total + 255) / 256, 16384);
    if (dst_f16)
        hipLaunchKernelGGL(k_im2col<_Float16>, dim3((unsigned) g), dim3(256), 0, s, (_Float16 *) dst, src, a);
    else
        hipLaunchKernelGGL(k_im2col<float>, dim3((unsigned) g), dim3(256), 0, s, (float *) dst, src, a);
}

}  // namespace mi355x

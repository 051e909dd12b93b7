// k_mmq.hip -- MFMA int8 tile GEMM for GGML_OP_MUL_MAT on quantized weights
// with wide activation batches (prefill, N > 8). Filled in by the MFMA path;
// until then the planner keeps every width on the GEMV kernels.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

bool mmq_supported(int wtype, int64_t M, int64_t K) {
    (void) wtype;
    (void) M;
    (void) K;
    return false;
}

void launch_mmq(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu) {
    launch_mmv(wtype, W, row_bytes, M, K, act, N, dst, dst_nb1, stream, n_cu);
}

}  // namespace mi355x

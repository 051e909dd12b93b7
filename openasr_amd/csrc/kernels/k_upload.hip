// k_upload.hip -- applies staged host uploads: the small per-step inputs a
// host writes with ggml_backend_tensor_set (token ids, positions, KV row
// indices, the attention mask; llm_transformer.rs:5614-5633) are copied into
// pinned host memory by the buffer's set_tensor and written to the device by
// this one launch ahead of the next device use, instead of one synchronous
// copy per tensor.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

// one workgroup per entry; 16-byte pieces when the entry is 16-byte aligned
// (each thread requests up to four pieces before it stores any), bytes otherwise
__global__ __launch_bounds__(256) void k_apply_uploads(upload_batch b) {
    const upload_entry e = b.e[blockIdx.x];
    const char * src = b.src + e.off;
    const int tid = (int) threadIdx.x;
    if ((((uintptr_t) e.dst) | (uintptr_t) src | e.n) % 16 == 0) {
        const uint32_t n16 = e.n / 16;
        const uint4 * s4 = (const uint4 *) src;
        uint4 * d4 = (uint4 *) e.dst;
        for (uint32_t base = 0; base < n16; base += 4 * 256) {
            uint4 v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t i = base + (uint32_t) (k * 256 + tid);
                if (i < n16) v[k] = s4[i];
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t i = base + (uint32_t) (k * 256 + tid);
                if (i < n16) d4[i] = v[k];
            }
        }
    } else {
        for (uint32_t i = (uint32_t) tid; i < e.n; i += 256) e.dst[i] = src[i];
    }
}

void launch_apply_uploads(const upload_batch & b, hipStream_t s) {
    if (b.n <= 0) return;
    hipLaunchKernelGGL(k_apply_uploads, dim3((unsigned) b.n), dim3(256), 0, s, b);
    note_hip_error(hipGetLastError());
}

}  // namespace mi355x

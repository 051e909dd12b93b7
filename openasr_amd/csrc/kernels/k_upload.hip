// k_upload.hip -- applies staged host uploads: the small per-step inputs a
// host writes with ggml_backend_tensor_set (token ids, positions, KV row
// indices, the attention mask; llm_transformer.rs:5614-5633) are copied into
// pinned host memory by the buffer's set_tensor and written to the device by
// this one launch ahead of the next device use, instead of one synchronous
// copy per tensor.
#include "../mi355x_common.h"
#include "../ops.h"

namespace mi355x {

namespace {

// bytes one workgroup copies: one 16-byte piece per thread, so every read of
// host memory is in flight at once and a launch costs one PCIe round trip
// whatever the entry sizes (a 64 KB mask is 16 workgroups, not 16 dependent
// passes of one)
constexpr uint32_t kChunk = 256 * 16;

__host__ __device__ inline uint32_t entry_chunks(uint32_t n) { return n == 0 ? 1u : (n + kChunk - 1) / kChunk; }

}  // namespace

// the workgroups of entry k follow those of entries 0..k-1; 16-byte pieces
// when the entry is 16-byte aligned, bytes otherwise
__global__ __launch_bounds__(256) void k_apply_uploads(upload_batch b) {
    uint32_t blk = blockIdx.x;
    int k = 0;
    for (; k < b.n - 1; k++) {
        const uint32_t c = entry_chunks(b.e[k].n);
        if (blk < c) break;
        blk -= c;
    }
    const upload_entry e = b.e[k];
    const char * src = b.src + e.off;
    const uint32_t lo = blk * kChunk;
    const uint32_t hi = min(e.n, lo + kChunk);
    const uint32_t tid = threadIdx.x;
    if ((((uintptr_t) e.dst) | (uintptr_t) src | e.n) % 16 == 0) {
        const uint32_t i = lo + tid * 16;
        if (i < hi) *(uint4 *) (e.dst + i) = *(const uint4 *) (src + i);
    } else {
        for (uint32_t i = lo + tid; i < hi; i += 256) e.dst[i] = src[i];
    }
}

void launch_apply_uploads(const upload_batch & b, hipStream_t s) {
    if (b.n <= 0) return;
    uint32_t blocks = 0;
    for (int k = 0; k < b.n; k++) blocks += entry_chunks(b.e[k].n);
    hipLaunchKernelGGL(k_apply_uploads, dim3(blocks), dim3(256), 0, s, b);
    note_hip_error(hipGetLastError());
}

}  // namespace mi355x

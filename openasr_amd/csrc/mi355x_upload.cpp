// mi355x_upload.cpp -- staged host uploads. A decode step's host writes a
// handful of small input tensors with ggml_backend_tensor_set (token ids,
// positions, KV row indices, the mask: llm_transformer.rs:5614-5633); each
// synchronous hipMemcpy costs a full host-device round trip (~11 us). Writes
// of up to kStageMax bytes are instead copied into pinned host memory and
// queued; the queue is applied by one launch (k_apply_uploads) on the stream
// of whatever device work comes next -- a graph compute flushes it
// asynchronously ahead of the graph, a buffer operation synchronously -- so
// no reader ever sees the device bytes before the write lands.
//
// The pinned area has two halves: new writes fill one while the launch that
// reads the other may still be in flight (an event per half says when it is
// free again).

#include <cstring>

#include "mi355x_exec.h"

namespace mi355x {

namespace {

constexpr size_t kUploadHalf = 1u << 20;
constexpr size_t kStageMax = 256u << 10;
constexpr size_t kMaxPending = 4 * kUploadBatch;

size_t round16(size_t n) { return (n + 15) & ~(size_t) 15; }

bool ensure_pinned(upload_queue & q) {
    if (q.pinned) return true;
    if (q.tried) return false;
    q.tried = true;
    void * p = nullptr;
    if (hipHostMalloc(&p, 2 * kUploadHalf, hipHostMallocDefault) != hipSuccess) {
        (void) hipGetLastError();
        return false;
    }
    for (hipEvent_t & e : q.done) {
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            (void) hipGetLastError();
            for (hipEvent_t & f : q.done) {
                if (f) (void) hipEventDestroy(f);
                f = nullptr;
            }
            (void) hipHostFree(p);
            return false;
        }
    }
    q.pinned = (char *) p;
    return true;
}

// the caller holds q.mu
void flush_locked(upload_queue & q, hipStream_t s, bool wait) {
    if (q.pending.empty()) return;
    for (size_t i = 0; i < q.pending.size(); i += kUploadBatch) {
        upload_batch b{};
        b.src = q.pinned;
        b.n = (int) std::min<size_t>(kUploadBatch, q.pending.size() - i);
        for (int k = 0; k < b.n; k++) b.e[k] = q.pending[i + (size_t) k];
        launch_apply_uploads(b, s);
    }
    MI_CHECK(hipEventRecord(q.done[q.cur], s));
    q.busy[q.cur] = true;
    if (wait) {
        MI_CHECK(hipEventSynchronize(q.done[q.cur]));
        q.busy[q.cur] = false;
    }
    q.pending.clear();
    q.cur ^= 1;
    q.used = 0;
    if (q.busy[q.cur]) {  // the launch that read this half must be done before it is refilled
        MI_CHECK(hipEventSynchronize(q.done[q.cur]));
        q.busy[q.cur] = false;
    }
}

}  // namespace

bool stage_upload(device_state * dev, char * dst, const void * src, size_t n) {
    if (n == 0) return true;
    if (n > kStageMax) return false;
    upload_queue & q = dev->uploads;
    std::lock_guard<std::mutex> lk(q.mu);
    if (!ensure_pinned(q)) return false;
    // the apply launch writes its entries concurrently: a write that overlaps
    // a queued one goes after the queue has landed
    bool overlap = false;
    for (const upload_entry & e : q.pending) overlap = overlap || (dst < e.dst + e.n && e.dst < dst + n);
    if (overlap || q.pending.size() >= kMaxPending || q.used + round16(n) > kUploadHalf) flush_locked(q, nullptr, true);
    const size_t off = (size_t) q.cur * kUploadHalf + q.used;
    std::memcpy(q.pinned + off, src, n);
    q.pending.push_back(upload_entry{dst, (uint32_t) off, (uint32_t) n});
    q.used += round16(n);
    return true;
}

void flush_uploads(device_state * dev, hipStream_t s, bool wait) {
    upload_queue & q = dev->uploads;
    std::lock_guard<std::mutex> lk(q.mu);
    flush_locked(q, s, wait);
}

void release_uploads(device_state * dev) {
    upload_queue & q = dev->uploads;
    std::lock_guard<std::mutex> lk(q.mu);
    flush_locked(q, nullptr, true);
    for (int h = 0; h < 2; h++) {
        if (q.busy[h]) (void) hipEventSynchronize(q.done[h]);
        q.busy[h] = false;
        if (q.done[h]) (void) hipEventDestroy(q.done[h]);
        q.done[h] = nullptr;
    }
    if (q.pinned) (void) hipHostFree(q.pinned);
    q.pinned = nullptr;
    q.tried = false;
}

}  // namespace mi355x

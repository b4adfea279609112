// Copies that run beside compute, ordered against it with events: the Transfer trait of
// crates/oominf-core/src/backend.rs:945-1018 (CUDA form: crates/oominf-cuda/src/memory.rs:300-380)
// on HIP. A copy queue is a stream of its own (default priority, non-blocking against the
// null stream); expert records move from pinned host memory into device slots on it while
// the compute stream runs the previous layer, and events order the two.
//
// Pinned host memory comes from oom_host_alloc (hipHostMalloc). Registering memory that
// already exists (pin_host) is not offered: callers allocate their host expert tier with
// oom_host_alloc instead.
#include <string>

#include "common.hpp"

namespace oom {
static int hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return OOM_OK;
    (void)hipGetLastError();
    return fail(OOM_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace oom

using oom::hip_ok;

extern "C" int oom_copy_queue_create(void** queue) {
    OOM_REQUIRE(queue != nullptr, "oom_copy_queue_create: null queue");
    hipStream_t s = nullptr;
    if (int rc = hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "oom_copy_queue_create")) return rc;
    *queue = s;
    return OOM_OK;
}

extern "C" int oom_copy_queue_destroy(void* queue) {
    if (!queue) return OOM_OK;
    return hip_ok(hipStreamDestroy(static_cast<hipStream_t>(queue)), "oom_copy_queue_destroy");
}

extern "C" int oom_host_alloc(void** ptr, size_t bytes) {
    OOM_REQUIRE(ptr != nullptr && bytes > 0, "oom_host_alloc: null pointer or zero bytes");
    void* p = nullptr;
    if (int rc = hip_ok(hipHostMalloc(&p, bytes, hipHostMallocDefault), "oom_host_alloc")) return rc;
    *ptr = p;
    return OOM_OK;
}

extern "C" int oom_host_free(void* ptr) {
    if (!ptr) return OOM_OK;
    return hip_ok(hipHostFree(ptr), "oom_host_free");
}

extern "C" int oom_copy_to_device(void* queue, uint64_t dst, const void* src, size_t len) {
    OOM_REQUIRE(queue && dst && src, "oom_copy_to_device: null queue or buffer");
    if (len == 0) return OOM_OK;
    return hip_ok(hipMemcpyAsync(reinterpret_cast<void*>(dst), src, len, hipMemcpyHostToDevice,
                                 static_cast<hipStream_t>(queue)),
                  "oom_copy_to_device");
}

extern "C" int oom_copy_on_device(void* queue, uint64_t dst, uint64_t src, size_t len) {
    OOM_REQUIRE(queue && dst && src, "oom_copy_on_device: null queue or buffer");
    if (len == 0) return OOM_OK;
    return hip_ok(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), len,
                                 hipMemcpyDeviceToDevice, static_cast<hipStream_t>(queue)),
                  "oom_copy_on_device");
}

extern "C" int oom_copy_records_to_device(void* queue, const uint64_t* dst, const void* const* src, size_t bytes,
                                          int n) {
    OOM_REQUIRE(queue && n >= 0 && (n == 0 || (dst && src)), "oom_copy_records_to_device: null queue or table");
    for (int i = 0; i < n; i++)
        if (int rc = oom_copy_to_device(queue, dst[i], src[i], bytes)) return rc;
    return OOM_OK;
}

extern "C" int oom_download_async(void* stream, void* dst, const void* src, size_t len) {
    OOM_REQUIRE(dst && src, "oom_download_async: null buffer");
    if (len == 0) return OOM_OK;
    return hip_ok(hipMemcpyAsync(dst, src, len, hipMemcpyDeviceToHost, oom::as_stream(stream)),
                  "oom_download_async");
}

extern "C" int oom_event_create(void** event) {
    OOM_REQUIRE(event != nullptr, "oom_event_create: null event");
    hipEvent_t e = nullptr;
    if (int rc = hip_ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "oom_event_create")) return rc;
    *event = e;
    return OOM_OK;
}

extern "C" int oom_event_destroy(void* event) {
    if (!event) return OOM_OK;
    return hip_ok(hipEventDestroy(static_cast<hipEvent_t>(event)), "oom_event_destroy");
}

extern "C" int oom_event_record(void* event, void* stream) {
    OOM_REQUIRE(event != nullptr, "oom_event_record: null event");
    return hip_ok(hipEventRecord(static_cast<hipEvent_t>(event), oom::as_stream(stream)), "oom_event_record");
}

extern "C" int oom_stream_wait_event(void* stream, void* event) {
    OOM_REQUIRE(event != nullptr, "oom_stream_wait_event: null event");
    return hip_ok(hipStreamWaitEvent(oom::as_stream(stream), static_cast<hipEvent_t>(event), 0),
                  "oom_stream_wait_event");
}

extern "C" int oom_event_done(void* event) {
    OOM_REQUIRE(event != nullptr, "oom_event_done: null event");
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipSuccess) return 1;
    if (e == hipErrorNotReady) {
        (void)hipGetLastError();
        return 0;
    }
    return hip_ok(e, "oom_event_done");
}

extern "C" int oom_event_wait(void* event) {
    OOM_REQUIRE(event != nullptr, "oom_event_wait: null event");
    return hip_ok(hipEventSynchronize(static_cast<hipEvent_t>(event)), "oom_event_wait");
}

extern "C" int oom_status(void* stream);

// A sync point: waits for `stream`, then reports a bounded wait that gave up inside an
// earlier kernel (OOM_ERR_KERNEL) the way oom_status does.
extern "C" int oom_stream_sync(void* stream) {
    if (int rc = hip_ok(hipStreamSynchronize(oom::as_stream(stream)), "oom_stream_sync")) return rc;
    return oom_status(stream);
}

// kd_runtime.hip - errors, device discovery, memory, copies, stream and events.
//
// Replaces the runtime half of the reference backend (src/cuda/backend.cu:17-32, 73-105):
// same synchronous-at-the-host copy semantics, but every operation is issued on one
// in-order backend stream (the null stream unless kd_set_stream selects another).
#include <atomic>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "kd_internal.h"

namespace kd {

namespace {

thread_local std::string g_error;
std::atomic<hipStream_t> g_stream{nullptr};

struct DeviceState {
    std::atomic<int> checked{0};  // 0 = not probed, 1 = usable, -1 = unusable
    int ordinal = 0;
    int cus = 0;
    std::string arch;
    // Workspace, guarded by g_workspace_mutex: the block, its size, and the stream the last
    // lease enqueued its kernels on (valid once `workspace_used` is set).
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    hipStream_t workspace_stream = nullptr;
    bool workspace_used = false;
};

DeviceState& state() {
    static DeviceState s;
    return s;
}

std::mutex g_mutex;
std::mutex g_workspace_mutex;

} // namespace

int ensure_device() {
    DeviceState& s = state();
    if (s.checked != 0) return s.checked > 0 ? KD_OK : fail(KD_E_NO_DEVICE, "no usable gfx950 device");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (s.checked != 0) return s.checked > 0 ? KD_OK : fail(KD_E_NO_DEVICE, "no usable gfx950 device");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        s.checked = -1;
        (void)hipGetLastError();
        return fail(KD_E_NO_DEVICE, "no HIP device is visible");
    }
    int ordinal = 0;
    if (hipGetDevice(&ordinal) != hipSuccess) ordinal = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, ordinal) != hipSuccess) {
        s.checked = -1;
        return fail(KD_E_NO_DEVICE, "hipGetDeviceProperties failed");
    }
    s.arch = prop.gcnArchName;
    if (s.arch.rfind("gfx950", 0) != 0) {
        s.checked = -1;
        return fail(KD_E_NO_DEVICE, "device is " + s.arch + ", this backend is built for gfx950");
    }
    s.ordinal = ordinal;
    s.cus = prop.multiProcessorCount;
    s.checked = 1;
    return KD_OK;
}

void set_error(const std::string& message) { g_error = message; }

int fail(int status, const std::string& message) {
    g_error = message;
    return status;
}

int hip_fail(hipError_t status, const char* call, const char* file, int line) {
    char buffer[512];
    std::snprintf(buffer, sizeof buffer, "HIP error at %s:%d: %s failed with %s", file, line, call,
                  hipGetErrorString(status));
    g_error = buffer;
    return KD_E_RUNTIME;
}

hipStream_t stream() { return g_stream.load(); }
int device_ordinal() { return state().ordinal; }
int compute_units() { return state().cus > 0 ? state().cus : 256; }

Workspace::~Workspace() {
    if (held) g_workspace_mutex.unlock();
}

int workspace(Workspace& lease, size_t bytes) {
    DeviceState& s = state();
    if (!lease.held) {
        g_workspace_mutex.lock();
        lease.held = true;
    }
    const hipStream_t current = g_stream.load();
    // The previous lease's kernels may still run on another stream: let them finish before this
    // stream reuses (or this call frees) the block.
    if (s.workspace_used && s.workspace_stream != current) KD_HIP(hipStreamSynchronize(s.workspace_stream));
    if (s.workspace_bytes < bytes) {
        if (s.workspace != nullptr) {
            // Kernels queued by earlier leases may still read the old block: drain before freeing.
            KD_HIP(hipStreamSynchronize(current));
            KD_HIP(hipFree(s.workspace));
            s.workspace = nullptr;
            s.workspace_bytes = 0;
        }
        size_t size = 1 << 20;
        while (size < bytes) size <<= 1;
        KD_HIP(hipMalloc(&s.workspace, size));
        s.workspace_bytes = size;
    }
    s.workspace_stream = current;
    s.workspace_used = true;
    lease.ptr = s.workspace;
    return KD_OK;
}

} // namespace kd

using namespace kd;

extern "C" {

const char* kd_last_error(void) { return g_error.c_str(); }

int kd_available(void) { return ensure_device() == KD_OK ? 1 : 0; }

int kd_synchronize(void) {
    if (int rc = ensure_device()) return rc;
    KD_HIP(hipStreamSynchronize(g_stream.load()));
    return KD_OK;
}

int kd_set_stream(void* s) {
    g_stream.store(static_cast<hipStream_t>(s));
    return KD_OK;
}

void* kd_get_stream(void) { return g_stream.load(); }

int kd_malloc(void** out, int64_t bytes) {
    if (out == nullptr || bytes < 0) return fail(KD_E_INVALID, "kd_malloc: bad arguments");
    if (int rc = ensure_device()) return rc;
    *out = nullptr;
    if (bytes == 0) bytes = 1;
    KD_HIP(hipMalloc(out, static_cast<size_t>(bytes)));
    return KD_OK;
}

void kd_free(void* block) {
    if (block != nullptr) {
        // release is noexcept and unchecked in the reference (backend.cu:88-90). hipFree
        // waits for outstanding work on the device, so queued kernels never read freed memory.
        (void)hipFree(block);
    }
}

int kd_copy_h2d(void* target, const void* source, int64_t bytes) {
    if (bytes < 0) return fail(KD_E_INVALID, "kd_copy_h2d: negative size");
    if (bytes == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    KD_HIP(hipMemcpyAsync(target, source, static_cast<size_t>(bytes), hipMemcpyHostToDevice, stream()));
    KD_HIP(hipStreamSynchronize(stream()));
    return KD_OK;
}

int kd_copy_d2h(void* target, const void* source, int64_t bytes) {
    if (bytes < 0) return fail(KD_E_INVALID, "kd_copy_d2h: negative size");
    if (bytes == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    KD_HIP(hipMemcpyAsync(target, source, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, stream()));
    KD_HIP(hipStreamSynchronize(stream()));
    return KD_OK;
}

int kd_copy_d2d(void* target, const void* source, int64_t bytes) {
    if (bytes < 0) return fail(KD_E_INVALID, "kd_copy_d2d: negative size");
    if (bytes == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    KD_HIP(hipMemcpyAsync(target, source, static_cast<size_t>(bytes), hipMemcpyDeviceToDevice, stream()));
    return KD_OK;
}

int kd_event_create(void** event) {
    if (int rc = ensure_device()) return rc;
    hipEvent_t e;
    KD_HIP(hipEventCreate(&e));
    *event = e;
    return KD_OK;
}

int kd_event_destroy(void* event) {
    KD_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return KD_OK;
}

int kd_event_record(void* event) {
    KD_HIP(hipEventRecord(static_cast<hipEvent_t>(event), stream()));
    return KD_OK;
}

int kd_event_elapsed_ms(float* ms, void* start, void* stop) {
    KD_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
    KD_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    return KD_OK;
}

int kd_device_info(int* cus, int* clock_khz, char* arch, int arch_len) {
    if (int rc = ensure_device()) return rc;
    hipDeviceProp_t prop;
    KD_HIP(hipGetDeviceProperties(&prop, state().ordinal));
    if (cus) *cus = prop.multiProcessorCount;
    if (clock_khz) *clock_khz = prop.clockRate;
    if (arch && arch_len > 0) std::snprintf(arch, static_cast<size_t>(arch_len), "%s", prop.gcnArchName);
    return KD_OK;
}

} // extern "C"

// Runtime helpers of libaero_hip.so: error state, device memory, streams,
// events and per-kernel timing. Every entry point returns a status and never
// aborts the process; HIP errors become a refusal plus aero_hip_last_error().
#include "common.hpp"
#include "aero_hip.h"

#include <cstdarg>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <mutex>
#include <string>

namespace aero {

namespace {
thread_local char g_err[512] = {0};
thread_local TimingSlot g_timing;
thread_local Plan* g_recording = nullptr;
}  // namespace

Plan*& recording_plan() { return g_recording; }

bool async_copy(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (Plan* plan = recording_plan()) {
        plan->entries.push_back({"copy", [=](hipStream_t s, hipEvent_t a, hipEvent_t b) {
                                     if (a != nullptr) (void)hipEventRecord(a, s);
                                     (void)hipMemcpyAsync(dst, src, bytes,
                                                          hipMemcpyDeviceToDevice, s);
                                     if (b != nullptr) (void)hipEventRecord(b, s);
                                 }});
        return true;
    }
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream),
                  "hipMemcpyAsync D2D");
}

namespace {
std::mutex g_knob_mu;
std::map<std::string, int>& knobs() {
    static std::map<std::string, int> k;
    return k;
}
void load_knobs() {
    static std::once_flag once;
    std::call_once(once, [] {
        const char* env = std::getenv("AERO_HIP_TUNE");
        if (env == nullptr) return;
        std::string all(env);
        size_t i = 0;
        while (i < all.size()) {
            size_t j = all.find(',', i);
            if (j == std::string::npos) j = all.size();
            const std::string kv = all.substr(i, j - i);
            const size_t eq = kv.find('=');
            if (eq != std::string::npos)
                knobs()[kv.substr(0, eq)] = std::atoi(kv.c_str() + eq + 1);
            i = j + 1;
        }
    });
}
}  // namespace

int tune(const char* key, int dflt) {
    load_knobs();
    std::lock_guard<std::mutex> g(g_knob_mu);
    auto it = knobs().find(key);
    return it == knobs().end() ? dflt : it->second;
}

int cu_count() {
    static std::mutex mu;
    static std::map<int, int> by_dev;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> g(mu);
    auto it = by_dev.find(dev);
    if (it != by_dev.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
        n = 256;
    by_dev[dev] = n;
    return n;
}

bool tune_set(const char* key, int value, bool erase) {
    load_knobs();
    std::lock_guard<std::mutex> g(g_knob_mu);
    if (erase)
        knobs().erase(key);
    else
        knobs()[key] = value;
    return true;
}

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_error("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return false;
}

TimingSlot& timing_slot() { return g_timing; }

}  // namespace aero

using aero::hip_ok;
using aero::set_error;

extern "C" {

const char* aero_hip_last_error(void) { return aero::g_err; }

const char* aero_hip_version(void) { return "aero_hip 0.1 (gfx950)"; }

int aero_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int aero_hip_set_device(int device) {
    return hip_ok(hipSetDevice(device), "hipSetDevice") ? 1 : 0;
}

void* aero_hip_malloc(int64_t bytes) {
    if (bytes <= 0) {
        set_error("aero_hip_malloc: bytes must be > 0 (got %lld)", (long long)bytes);
        return nullptr;
    }
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, (size_t)bytes), "hipMalloc")) return nullptr;
    return p;
}

int aero_hip_free(void* p) {
    if (p == nullptr) return 1;
    return hip_ok(hipFree(p), "hipFree") ? 1 : 0;
}

int aero_hip_tune_set(const char* key, int value, int erase) {
    if (key == nullptr || key[0] == '\0') {
        aero::set_error("aero_hip_tune_set: empty key");
        return 0;
    }
    return aero::tune_set(key, value, erase != 0) ? 1 : 0;
}

int aero_hip_memcpy_htod(void* dst, const void* src, int64_t bytes) {
    if (bytes == 0) return 1;
    if (!dst || !src || bytes < 0) {
        set_error("aero_hip_memcpy_htod: bad arguments");
        return 0;
    }
    return hip_ok(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice),
                  "hipMemcpy H2D") ? 1 : 0;
}

int aero_hip_memcpy_dtoh(void* dst, const void* src, int64_t bytes) {
    if (bytes == 0) return 1;
    if (!dst || !src || bytes < 0) {
        set_error("aero_hip_memcpy_dtoh: bad arguments");
        return 0;
    }
    return hip_ok(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost),
                  "hipMemcpy D2H") ? 1 : 0;
}

int aero_hip_memcpy_dtod(void* dst, const void* src, int64_t bytes, void* stream) {
    if (bytes == 0) return 1;
    if (!dst || !src || bytes < 0) {
        set_error("aero_hip_memcpy_dtod: bad arguments");
        return 0;
    }
    return hip_ok(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice,
                                 (hipStream_t)stream),
                  "hipMemcpyAsync D2D") ? 1 : 0;
}

int aero_hip_memset(void* dst, int value, int64_t bytes) {
    if (bytes == 0) return 1;
    if (!dst || bytes < 0) {
        set_error("aero_hip_memset: bad arguments");
        return 0;
    }
    return hip_ok(hipMemset(dst, value, (size_t)bytes), "hipMemset") ? 1 : 0;
}

void* aero_hip_stream_create(void) {
    hipStream_t s = nullptr;
    // Default flags and priority: the stream orders with the null stream, so
    // the synchronous copies above see its completed work.
    if (!hip_ok(hipStreamCreate(&s), "hipStreamCreate"))
        return nullptr;
    return (void*)s;
}

int aero_hip_stream_destroy(void* stream) {
    if (stream == nullptr) return 1;
    return hip_ok(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy") ? 1 : 0;
}

int aero_hip_stream_synchronize(void* stream) {
    return hip_ok(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize")
               ? 1 : 0;
}

int aero_hip_device_synchronize(void) {
    return hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize") ? 1 : 0;
}

void* aero_hip_event_create(void) {
    hipEvent_t e = nullptr;
    if (!hip_ok(hipEventCreate(&e), "hipEventCreate")) return nullptr;
    return (void*)e;
}

int aero_hip_event_destroy(void* ev) {
    if (ev == nullptr) return 1;
    return hip_ok(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy") ? 1 : 0;
}

int aero_hip_event_record(void* ev, void* stream) {
    if (ev == nullptr) {
        set_error("aero_hip_event_record: null event");
        return 0;
    }
    return hip_ok(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream), "hipEventRecord")
               ? 1 : 0;
}

int aero_hip_event_synchronize(void* ev) {
    if (ev == nullptr) {
        set_error("aero_hip_event_synchronize: null event");
        return 0;
    }
    return hip_ok(hipEventSynchronize((hipEvent_t)ev), "hipEventSynchronize") ? 1 : 0;
}

float aero_hip_event_elapsed_ms(void* start, void* stop) {
    if (start == nullptr || stop == nullptr) {
        set_error("aero_hip_event_elapsed_ms: null event");
        return -1.0f;
    }
    float ms = 0.0f;
    if (!hip_ok(hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop),
                "hipEventElapsedTime"))
        return -1.0f;
    return ms;
}

void* aero_hip_plan_create(void) { return new (std::nothrow) aero::Plan(); }

int aero_hip_plan_destroy(void* plan) {
    if (plan == nullptr) return 1;
    if (aero::recording_plan() == plan) aero::recording_plan() = nullptr;
    delete static_cast<aero::Plan*>(plan);
    return 1;
}

int aero_hip_plan_begin(void* plan) {
    if (plan == nullptr || aero::recording_plan() != nullptr) {
        set_error("plan_begin: null plan or a plan is already recording on this thread");
        return 0;
    }
    aero::recording_plan() = static_cast<aero::Plan*>(plan);
    return 1;
}

int aero_hip_plan_end(void* plan) {
    if (plan == nullptr || aero::recording_plan() != plan) {
        set_error("plan_end: this plan is not recording on this thread");
        return 0;
    }
    aero::recording_plan() = nullptr;
    return 1;
}

int64_t aero_hip_plan_size(void* plan) {
    return plan == nullptr ? 0 : (int64_t)static_cast<aero::Plan*>(plan)->entries.size();
}

int aero_hip_plan_launch(void* plan, void* stream, void** starts, void** stops) {
    if (plan == nullptr || aero::recording_plan() != nullptr) {
        set_error("plan_launch: null plan, or called while a plan records");
        return 0;
    }
    auto& entries = static_cast<aero::Plan*>(plan)->entries;
    for (size_t i = 0; i < entries.size(); ++i) {
        hipEvent_t a = starts ? (hipEvent_t)starts[i] : nullptr;
        hipEvent_t b = stops ? (hipEvent_t)stops[i] : nullptr;
        entries[i].run((hipStream_t)stream, a, b);
    }
    return hip_ok(hipGetLastError(), "plan_launch") ? 1 : 0;
}

int aero_hip_time_next_kernel(void* start, void* stop) {
    if ((start == nullptr) != (stop == nullptr)) {
        set_error("aero_hip_time_next_kernel: give both events or neither");
        return 0;
    }
    aero::timing_slot().start = (hipEvent_t)start;
    aero::timing_slot().stop = (hipEvent_t)stop;
    return 1;
}

}  // extern "C"

// Shared host-runtime pieces of the C ABI: the context object, error reporting, device scoping,
// the scratch arena and small host-to-device uploads.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <exception>
#include <new>
#include <string>

#include "kyro_verify.h"

struct kyro_ctx_s {
    int device = 0;
    int num_cus = 256;      // compute units of the device (hipDeviceAttributeMultiprocessorCount)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    void* arena = nullptr;  // per-call scratch, stream-ordered
    size_t arena_bytes = 0;
    void* noalloc_scratch = nullptr;  // device address of the allocation-free entry point's
                                      // static scratch array on this device
    int* err = nullptr;     // device error word
    int* sched = nullptr;   // kyro::kSchedWords device counters of the balanced attention schedule
                            // (zero between launches: the last workgroup of a launch resets them)
    int* row_cnt = nullptr; // kyro::kSampleRowCounters per-row counters of the one-launch decode
                            // pass (zero between launches, reset by each row's last workgroup)
    // Host staging for small uploads (hipHostMalloc): kStageSlots slots used in turn, each with
    // an event recorded after the copies out of it.
    void* pinned = nullptr;
    void* pinned_dev = nullptr;  // the same memory as the device addresses it
    size_t pinned_slot_bytes = 0;
    int pinned_next = 0;
    hipEvent_t pinned_done[4] = {};
};

namespace kyro {
namespace rt {

// Records the message as the calling thread's last error and returns `code`.
int fail(int code, const char* fmt, ...);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Makes `dev` current for the scope and restores the caller's device afterwards.
struct DeviceGuard {
    int prev = -1;
    hipError_t status = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) status = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

int check_ctx(kyro_ctx ctx);
int ensure_arena(kyro_ctx ctx, size_t bytes);

// One host-to-device copy of an upload.
struct Upload {
    void* dst;        // device
    const void* src;  // host
    size_t bytes;
};

constexpr int kStageSlots = 4;  // slots of the pinned staging ring (kyro_ctx_s::pinned_done)
static_assert(sizeof(kyro_ctx_s::pinned_done) / sizeof(hipEvent_t) == kStageSlots, "staging ring size");

// Queues the copies on the context's stream through the next slot of its pinned staging ring.
// The host data is copied into staging before this returns, so the caller may reuse it at once.
// A slot is reused only after the copies out of it have executed, so the host waits only when
// kStageSlots uploads are still queued ahead.
int stage_uploads(kyro_ctx ctx, const Upload* ups, int n);

template <typename F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return fail(KYRO_EOOM, "host allocation failed");
    } catch (const std::exception& e) {
        return fail(KYRO_EHIP, "internal error: %s", e.what());
    } catch (...) {
        return fail(KYRO_EHIP, "internal error");
    }
}

}  // namespace rt
}  // namespace kyro

#define KYRO_HIP(expr)                                                                          \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            return ::kyro::rt::fail(e_ == hipErrorOutOfMemory ? KYRO_EOOM : KYRO_EHIP,          \
                                    "%s failed: %s", #expr, hipGetErrorString(e_));             \
    } while (0)

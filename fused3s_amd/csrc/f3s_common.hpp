// f3s_common.hpp -- shared helpers of libf3s_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/f3s_capi.h"

namespace f3s {

// Per-thread detail of the last failure (returned by f3s_last_error).
void set_error(const std::string& msg);
void clear_error();

// Turns a HIP error into F3S_EHIP (or F3S_ENOMEM / F3S_ENODEV) and records
// where it happened.
f3s_status hip_fail(hipError_t err, const char* what, const char* file, int line);

// Validates that a device is present and current; F3S_ENODEV otherwise.
f3s_status require_device();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Device-wide exclusive scan of int32 counts into int64 (or int32) prefix
// sums; out has count + 1 entries (out[count] = total).  tmp needs
// scan_tmp_elems(count) int64 elements.
int64_t scan_tmp_elems(int64_t count);
f3s_status exclusive_scan_i32_to_i64(const int32_t* in, int64_t* out, int64_t count,
                                     int64_t* tmp, hipStream_t stream);

// Each translation unit's code object is loaded onto the device at its
// first kernel launch; these launch one empty kernel per unit (f3s_init).
hipError_t warm_runtime(hipStream_t s);
hipError_t warm_convert(hipStream_t s);
hipError_t warm_attention(hipStream_t s);
hipError_t warm_bsf_util(hipStream_t s);
hipError_t warm_naive(hipStream_t s);
// Looks up the current device's address of f3s_attention_fwd_noalloc's
// fixed scratch (attention.hip), so its first call does not.
f3s_status noalloc_setup();

// Device memory of the library, from a caching allocator over hipMalloc:
// freed blocks are kept per device and size class for reuse, so repeated
// conversions, plans and scratch buffers do not pay the driver's allocation
// and page-mapping cost each time.  dev_alloc's block is usable on `stream`
// at once (if it was last used elsewhere, `stream` waits for that use) and
// on other streams once `stream` has been synchronised.
f3s_status dev_alloc(void** ptr, size_t bytes, hipStream_t stream);
// Returns `ptr` for reuse after the work queued on `stream` before this call
// (stream-ordered); `device` is the device it was allocated on.
void dev_free(void* ptr, int device, hipStream_t stream);
// Returns `ptr` for reuse at once: the caller knows no work uses it.
void dev_free_idle(void* ptr, int device);
// Waits for every stream of `device`, then returns `ptr` for reuse: for
// memory whose last users may be on any stream (hipFree's behaviour).
void dev_free_synced(void* ptr, int device);
// Host-pinned staging words of the calling thread (16 x int64), for the small
// device-to-host reads of counts and status that size outputs.
int64_t* host_staging();

// Grow-only device buffer owned by a long-lived object (a plan): allocated on
// the owner's stream, which the owner synchronises before handing the buffer
// out; released after waiting for every stream of its device.
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    int device = -1;
    f3s_status reserve(size_t want, hipStream_t stream);
    void release();
    void release_idle();   // the owner has synchronised the device
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;              // owns its allocation
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() { release(); }
};

// Scratch memory of one call: allocated on the call's stream and returned to
// the cache in stream order when it goes out of scope, so a call that queues
// work on the stream and returns without waiting may still use it on the
// device.  The stream must outlive the object (it does for call-local use).
struct StreamBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    int device = -1;
    hipStream_t stream = nullptr;
    explicit StreamBuffer(hipStream_t s) : stream(s) {}
    f3s_status reserve(size_t want);
    StreamBuffer(const StreamBuffer&) = delete;
    StreamBuffer& operator=(const StreamBuffer&) = delete;
    ~StreamBuffer()
    {
        if (ptr) dev_free(ptr, device, stream);
    }
};

}  // namespace f3s

#define F3S_HIP(call)                                                        \
    do {                                                                     \
        hipError_t f3s_err_ = (call);                                        \
        if (f3s_err_ != hipSuccess)                                          \
            return ::f3s::hip_fail(f3s_err_, #call, __FILE__, __LINE__);     \
    } while (0)

#define F3S_TRY(call)                                                        \
    do {                                                                     \
        f3s_status f3s_st_ = (call);                                         \
        if (f3s_st_ != F3S_OK) return f3s_st_;                               \
    } while (0)

#define F3S_REQUIRE(cond, msg)                                               \
    do {                                                                     \
        if (!(cond)) {                                                       \
            ::f3s::set_error(msg);                                           \
            return F3S_EINVAL;                                               \
        }                                                                    \
    } while (0)

// Orders this wave's LDS traffic: every LDS access issued before completes
// before any issued after, and the compiler may not move memory operations
// across it.  Sufficient for LDS shared between the lanes of one wave.
#define F3S_WAVE_LDS_SYNC() asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory")

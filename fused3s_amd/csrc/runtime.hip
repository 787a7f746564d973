// runtime.hip -- error reporting, device plumbing, fp32->fp16 cast and the
// device-wide scan used by the converter and the planner.
#include <stdio.h>
#include <stdlib.h>

#include <iterator>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

static thread_local std::string g_last_error;

void set_error(const std::string& msg)
{
    try {
        g_last_error = msg;
    } catch (...) {   // keep the old message rather than throw across the C ABI
    }
}
void clear_error() { g_last_error.clear(); }

f3s_status hip_fail(hipError_t err, const char* what, const char* file, int line)
{
    char buf[512];
    snprintf(buf, sizeof buf, "%s failed at %s:%d: %s (%d)", what, file, line,
             hipGetErrorString(err), (int)err);
    set_error(buf);
    if (err == hipErrorOutOfMemory) return F3S_ENOMEM;
    if (err == hipErrorNoDevice || err == hipErrorInvalidDevice) return F3S_ENODEV;
    return F3S_EHIP;
}

f3s_status require_device()
{
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        set_error("no HIP device visible");
        return F3S_ENODEV;
    }
    return F3S_OK;
}

// ------------------------------------------------------------ device memory
//
// A caching allocator over hipMalloc.  Freed blocks go to a per-device cache
// keyed by size class instead of back to the driver, whose large allocations
// and frees cost 0.05-1.7 ms each on MI355X (page mapping; ROCm's
// stream-ordered pools measured no better for large blocks, their frees
// unmapping the memory).  A block freed in stream order carries an event
// recorded on its stream at the free; whoever takes it next waits for that
// event (on the device, through its own stream), so a block is never reused
// while its last user's work may still run.  Idle cached bytes are capped per
// device (1 GiB, or F3S_CACHE_LIMIT_MB read at the first allocation; 0 keeps
// nothing), so a process that shares the GPU with another allocator (torch's)
// holds little idle memory; on an allocation failure the cache is returned to
// the driver and the allocation retried.  (Handing f3s_free's large blocks
// straight back to the driver was measured: the fused pass on memory mapped
// afresh after such frees ran 4.5 % slower, so f3s_free caches them too.)

namespace {

constexpr int kMaxDevices = 64;
constexpr size_t kSmallQuantum = 512;
constexpr size_t kLargeQuantum = (size_t)2 << 20;
constexpr size_t kDefaultCacheCap = (size_t)1 << 30;   // idle cached bytes kept per device

struct CachedBlock {
    void* ptr;
    hipEvent_t last_use;   // recorded where the block was freed (nullptr: no pending use)
};

struct DeviceCache {
    std::multimap<size_t, CachedBlock> idle;   // by size
    std::unordered_map<void*, size_t> live;    // blocks handed out, and their sizes
    std::vector<hipEvent_t> spare_events;
    size_t idle_bytes = 0;
};

std::mutex g_mem_mu;
DeviceCache g_cache[kMaxDevices];

// The idle-byte cap: F3S_CACHE_LIMIT_MB if set to a number, else 1 GiB.
size_t cache_cap()
{
    static const size_t cap = [] {
        const char* v = getenv("F3S_CACHE_LIMIT_MB");
        if (v && *v) {
            char* end = nullptr;
            const unsigned long long mb = strtoull(v, &end, 10);
            if (end && *end == '\0' && mb < ((unsigned long long)1 << 44)) return (size_t)mb << 20;
        }
        return kDefaultCacheCap;
    }();
    return cap;
}

size_t size_class(size_t bytes)
{
    if (bytes < kLargeQuantum / 2) return (bytes + kSmallQuantum - 1) / kSmallQuantum * kSmallQuantum;
    return (bytes + kLargeQuantum - 1) / kLargeQuantum * kLargeQuantum;
}

// Frees one idle block to the driver (its last use must be complete).
void drop_block(DeviceCache& c, void* ptr, hipEvent_t ev)
{
    if (ev) {
        (void)hipEventSynchronize(ev);
        c.spare_events.push_back(ev);
    }
    (void)hipFree(ptr);
}

// Returns every idle block of the current device `dev` to the driver.
void drop_idle(DeviceCache& c)
{
    for (auto& kv : c.idle) drop_block(c, kv.second.ptr, kv.second.last_use);
    c.idle.clear();
    c.idle_bytes = 0;
}

void cache_idle(DeviceCache& c, void* ptr, size_t size, hipEvent_t ev)
{
    c.idle.emplace(size, CachedBlock{ptr, ev});
    c.idle_bytes += size;
    // over the cap: the largest idle blocks go back to the driver
    const size_t cap = cache_cap();
    while (c.idle_bytes > cap && !c.idle.empty()) {
        auto it = std::prev(c.idle.end());
        c.idle_bytes -= it->first;
        drop_block(c, it->second.ptr, it->second.last_use);
        c.idle.erase(it);
    }
}

}  // namespace

f3s_status dev_alloc(void** ptr, size_t bytes, hipStream_t stream)
{
    *ptr = nullptr;
    const size_t size = size_class(bytes ? bytes : 1);
    int dev = 0;
    F3S_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        F3S_HIP(hipMalloc(ptr, size));
        return F3S_OK;
    }
    std::lock_guard<std::mutex> lock(g_mem_mu);
    DeviceCache& c = g_cache[dev];
    // a cached block of this size class, or a close larger one: at most a
    // quarter bigger, plus one 2 MiB quantum for the large classes only (a
    // small request never takes a large block)
    auto it = c.idle.lower_bound(size);
    const size_t slack = size / 4 + (size >= kLargeQuantum / 2 ? kLargeQuantum : 0);
    if (it != c.idle.end() && it->first <= size + slack) {
        const size_t got = it->first;
        const CachedBlock b = it->second;
        c.idle.erase(it);
        c.idle_bytes -= got;
        if (b.last_use) {
            const hipError_t q = hipEventQuery(b.last_use);
            if (q != hipSuccess) {
                (void)hipGetLastError();   // not ready: the new user's stream waits for it
                const hipError_t w = hipStreamWaitEvent(stream, b.last_use, 0);
                if (w != hipSuccess) {
                    c.idle.emplace(got, b);
                    c.idle_bytes += got;
                    return hip_fail(w, "hipStreamWaitEvent", __FILE__, __LINE__);
                }
            }
            c.spare_events.push_back(b.last_use);
        }
        c.live[b.ptr] = got;
        *ptr = b.ptr;
        return F3S_OK;
    }
    hipError_t e = hipMalloc(ptr, size);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        drop_idle(c);
        e = hipMalloc(ptr, size);
    }
    if (e != hipSuccess) {
        *ptr = nullptr;
        return hip_fail(e, "hipMalloc", __FILE__, __LINE__);
    }
    c.live[*ptr] = size;
    return F3S_OK;
}

void dev_free(void* ptr, int device, hipStream_t stream)
{
    if (!ptr) return;
    if (device < 0 || device >= kMaxDevices) {
        (void)hipFree(ptr);
        return;
    }
    std::lock_guard<std::mutex> lock(g_mem_mu);
    DeviceCache& c = g_cache[device];
    auto it = c.live.find(ptr);
    if (it == c.live.end()) {   // not ours: the driver's
        (void)hipFree(ptr);
        return;
    }
    const size_t size = it->second;
    c.live.erase(it);
    hipEvent_t ev = nullptr;
    if (!c.spare_events.empty()) {
        ev = c.spare_events.back();
        c.spare_events.pop_back();
    } else if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        ev = nullptr;
    }
    if (!ev || hipEventRecord(ev, stream) != hipSuccess) {
        // no event to order the reuse by: wait for the stream instead
        (void)hipGetLastError();
        (void)hipStreamSynchronize(stream);
        if (ev) c.spare_events.push_back(ev);
        ev = nullptr;
    }
    cache_idle(c, ptr, size, ev);
}

void dev_free_idle(void* ptr, int device)
{
    if (!ptr) return;
    if (device < 0 || device >= kMaxDevices) {
        (void)hipFree(ptr);
        return;
    }
    std::lock_guard<std::mutex> lock(g_mem_mu);
    DeviceCache& c = g_cache[device];
    auto it = c.live.find(ptr);
    if (it == c.live.end()) {
        (void)hipFree(ptr);
        return;
    }
    const size_t size = it->second;
    c.live.erase(it);
    cache_idle(c, ptr, size, nullptr);
}

void dev_free_synced(void* ptr, int device)
{
    if (!ptr) return;
    int cur = -1;
    const bool switch_dev = hipGetDevice(&cur) == hipSuccess && device >= 0 && cur != device &&
                            hipSetDevice(device) == hipSuccess;
    (void)hipDeviceSynchronize();
    dev_free_idle(ptr, device);
    if (switch_dev) (void)hipSetDevice(cur);
}

int64_t* host_staging()
{
    thread_local int64_t* words = nullptr;   // one small pinned block per host thread
    if (!words) {
        void* p = nullptr;
        if (hipHostMalloc(&p, 16 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            thread_local int64_t fallback[16];
            return fallback;   // pageable: correct, only slower to copy into
        }
        words = static_cast<int64_t*>(p);
    }
    return words;
}

f3s_status DeviceBuffer::reserve(size_t want, hipStream_t stream)
{
    if (want <= bytes && ptr) return F3S_OK;
    release();
    size_t alloc = want ? want : 1;
    F3S_HIP(hipGetDevice(&device));
    F3S_TRY(dev_alloc(&ptr, alloc, stream));
    bytes = alloc;
    return F3S_OK;
}

void DeviceBuffer::release()
{
    if (ptr) dev_free_synced(ptr, device);
    ptr = nullptr;
    bytes = 0;
}

void DeviceBuffer::release_idle()
{
    if (ptr) dev_free_idle(ptr, device);
    ptr = nullptr;
    bytes = 0;
}

f3s_status StreamBuffer::reserve(size_t want)
{
    if (want <= bytes && ptr) return F3S_OK;
    if (ptr) dev_free(ptr, device, stream);
    ptr = nullptr;
    bytes = 0;
    size_t alloc = want ? want : 1;
    F3S_HIP(hipGetDevice(&device));
    F3S_TRY(dev_alloc(&ptr, alloc, stream));
    bytes = alloc;
    return F3S_OK;
}

// ------------------------------------------------------------------ scan

constexpr int kScanThreads = 256;
constexpr int kScanPerThread = 8;
constexpr int kScanTile = kScanThreads * kScanPerThread;

int64_t scan_tmp_elems(int64_t count) { return ceil_div(count, kScanTile) + 1; }

__global__ void __launch_bounds__(kScanThreads)
scan_block_sums(const int32_t* __restrict__ in, int64_t count, int64_t* __restrict__ sums)
{
    __shared__ int64_t lds[kScanThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanPerThread;
    int64_t s = 0;
#pragma unroll
    for (int i = 0; i < kScanPerThread; ++i)
        if (base + i < count) s += in[base + i];
    int64_t total;
    (void)block_exclusive_scan<kScanThreads>(s, lds, total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// One workgroup: exclusive scan of the block sums in place; writes the grand
// total to *total_out.
__global__ void __launch_bounds__(kScanThreads)
scan_sums_single(int64_t* __restrict__ sums, int64_t nblocks, int64_t* __restrict__ total_out)
{
    __shared__ int64_t lds[kScanThreads / kWave];
    int64_t carry = 0;
    for (int64_t b0 = 0; b0 < nblocks; b0 += kScanThreads) {
        int64_t i = b0 + threadIdx.x;
        int64_t v = i < nblocks ? sums[i] : 0;
        int64_t total;
        int64_t ex = block_exclusive_scan<kScanThreads>(v, lds, total);
        if (i < nblocks) sums[i] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0) *total_out = carry;
}

__global__ void __launch_bounds__(kScanThreads)
scan_apply(const int32_t* __restrict__ in, int64_t count, const int64_t* __restrict__ sums,
           int64_t* __restrict__ out)
{
    __shared__ int64_t lds[kScanThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanPerThread;
    int64_t v[kScanPerThread];
    int64_t s = 0;
#pragma unroll
    for (int i = 0; i < kScanPerThread; ++i) {
        v[i] = (base + i < count) ? in[base + i] : 0;
        s += v[i];
    }
    int64_t total;
    int64_t ex = block_exclusive_scan<kScanThreads>(s, lds, total) + sums[blockIdx.x];
#pragma unroll
    for (int i = 0; i < kScanPerThread; ++i) {
        if (base + i < count) out[base + i] = ex;
        ex += v[i];
    }
}

f3s_status exclusive_scan_i32_to_i64(const int32_t* in, int64_t* out, int64_t count,
                                     int64_t* tmp, hipStream_t stream)
{
    if (count <= 0) {
        F3S_HIP(hipMemsetAsync(out, 0, sizeof(int64_t), stream));
        return F3S_OK;
    }
    const int64_t nb = ceil_div(count, kScanTile);
    hipLaunchKernelGGL(scan_block_sums, dim3((unsigned)nb), dim3(kScanThreads), 0, stream,
                       in, count, tmp);
    hipLaunchKernelGGL(scan_sums_single, dim3(1), dim3(kScanThreads), 0, stream, tmp, nb,
                       out + count);
    hipLaunchKernelGGL(scan_apply, dim3((unsigned)nb), dim3(kScanThreads), 0, stream, in,
                       count, tmp, out);
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}

// ------------------------------------------------------------------ cast

// float2half_kernel (tests/test_fused_3s_v2.cu:61-64); 4 elements per thread,
// v_cvt_f16_f32 rounds to nearest even.
__global__ void __launch_bounds__(256)
cast_f32_to_f16_kernel(const float* __restrict__ in, _Float16* __restrict__ out, int64_t count)
{
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 3 < count && ((((uintptr_t)in) | ((uintptr_t)out)) & 15) == 0) {
        float4 v = *reinterpret_cast<const float4*>(in + i);
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        h4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
        *reinterpret_cast<h4*>(out + i) = h;
    } else {
        for (int64_t j = i; j < i + 4 && j < count; ++j) out[j] = (_Float16)in[j];
    }
}

__global__ void warm_runtime_kernel() {}

hipError_t warm_runtime(hipStream_t s)
{
    hipLaunchKernelGGL(warm_runtime_kernel, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

}  // namespace f3s

using namespace f3s;

extern "C" {

const char* f3s_status_string(f3s_status s)
{
    switch (s) {
    case F3S_OK: return "F3S_OK";
    case F3S_EINVAL: return "F3S_EINVAL: invalid argument";
    case F3S_ENOMEM: return "F3S_ENOMEM: device out of memory";
    case F3S_EHIP: return "F3S_EHIP: HIP runtime error";
    case F3S_ENODEV: return "F3S_ENODEV: no GPU device";
    case F3S_EUNSUPPORTED: return "F3S_EUNSUPPORTED: unsupported configuration";
    case F3S_EDATA: return "F3S_EDATA: input violates the format";
    default: return "F3S: unknown status";
    }
}

const char* f3s_last_error(void) { return g_last_error.c_str(); }

int32_t f3s_abi_version(void) { return F3S_ABI_VERSION; }

f3s_status f3s_init(void)
{
    F3S_TRY(require_device());
    F3S_HIP(warm_runtime(nullptr));
    F3S_HIP(warm_convert(nullptr));
    F3S_HIP(warm_attention(nullptr));
    F3S_HIP(warm_bsf_util(nullptr));
    F3S_HIP(warm_naive(nullptr));
    F3S_HIP(hipDeviceSynchronize());
    F3S_TRY(noalloc_setup());
    return F3S_OK;
}

f3s_status f3s_device_count(int32_t* count)
{
    F3S_REQUIRE(count != nullptr, "f3s_device_count: count is NULL");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        c = 0;
    }
    *count = c;
    return F3S_OK;
}

f3s_status f3s_set_device(int32_t device)
{
    F3S_TRY(require_device());
    F3S_HIP(hipSetDevice(device));
    return F3S_OK;
}

f3s_status f3s_device_name(char* buf, int32_t buflen)
{
    F3S_REQUIRE(buf != nullptr && buflen > 0, "f3s_device_name: bad buffer");
    F3S_TRY(require_device());
    int dev = 0;
    F3S_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    F3S_HIP(hipGetDeviceProperties(&p, dev));
    // some drivers leave the marketing name empty: then the architecture alone
    if (p.name[0])
        snprintf(buf, (size_t)buflen, "%s (%s, %d CUs)", p.name, p.gcnArchName,
                 p.multiProcessorCount);
    else
        snprintf(buf, (size_t)buflen, "%s, %d CUs", p.gcnArchName, p.multiProcessorCount);
    return F3S_OK;
}

f3s_status f3s_malloc(void** ptr, uint64_t bytes)
{
    F3S_REQUIRE(ptr != nullptr, "f3s_malloc: ptr is NULL");
    *ptr = nullptr;
    F3S_TRY(require_device());
    // from the device's cache, then usable on every stream (as hipMalloc's memory)
    F3S_TRY(dev_alloc(ptr, bytes, nullptr));
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        dev_free_synced(*ptr, dev);
        *ptr = nullptr;
        return hip_fail(e, "hipStreamSynchronize", __FILE__, __LINE__);
    }
    return F3S_OK;
}

f3s_status f3s_free(void* ptr)
{
    if (!ptr) return F3S_OK;
    int dev = 0;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, ptr) == hipSuccess) {
        dev = attr.device;
    } else {
        (void)hipGetLastError();
        F3S_HIP(hipGetDevice(&dev));
    }
    // as hipFree: waits for the device, so no stream still uses the memory
    dev_free_synced(ptr, dev);
    return F3S_OK;
}

f3s_status f3s_release_cached_memory(void)
{
    int count = 0, cur = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || hipGetDevice(&cur) != hipSuccess) {
        (void)hipGetLastError();
        return F3S_OK;   // nothing was allocated
    }
    std::lock_guard<std::mutex> lock(g_mem_mu);
    for (int d = 0; d < count && d < kMaxDevices; ++d) {
        DeviceCache& c = g_cache[d];
        if (c.idle.empty() && c.spare_events.empty()) continue;
        F3S_HIP(hipSetDevice(d));
        drop_idle(c);
        for (hipEvent_t ev : c.spare_events) (void)hipEventDestroy(ev);
        c.spare_events.clear();
        (void)hipSetDevice(cur);
    }
    return F3S_OK;
}

f3s_status f3s_memcpy_h2d(void* dst, const void* src, uint64_t bytes, void* stream)
{
    if (!bytes) return F3S_OK;
    F3S_REQUIRE(dst && src, "f3s_memcpy_h2d: NULL pointer");
    F3S_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
    F3S_HIP(hipStreamSynchronize(as_stream(stream)));
    return F3S_OK;
}

f3s_status f3s_memcpy_d2h(void* dst, const void* src, uint64_t bytes, void* stream)
{
    if (!bytes) return F3S_OK;
    F3S_REQUIRE(dst && src, "f3s_memcpy_d2h: NULL pointer");
    F3S_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    F3S_HIP(hipStreamSynchronize(as_stream(stream)));
    return F3S_OK;
}

f3s_status f3s_memcpy_d2d(void* dst, const void* src, uint64_t bytes, void* stream)
{
    if (!bytes) return F3S_OK;
    F3S_REQUIRE(dst && src, "f3s_memcpy_d2d: NULL pointer");
    F3S_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return F3S_OK;
}

f3s_status f3s_memset(void* ptr, int32_t value, uint64_t bytes, void* stream)
{
    if (!bytes) return F3S_OK;
    F3S_REQUIRE(ptr != nullptr, "f3s_memset: NULL pointer");
    F3S_HIP(hipMemsetAsync(ptr, value, bytes, as_stream(stream)));
    return F3S_OK;
}

f3s_status f3s_synchronize(void* stream)
{
    F3S_TRY(require_device());
    if (stream) {
        F3S_HIP(hipStreamSynchronize(as_stream(stream)));
    } else {
        F3S_HIP(hipDeviceSynchronize());
    }
    return F3S_OK;
}

f3s_status f3s_stream_create(void** stream)
{
    F3S_REQUIRE(stream != nullptr, "f3s_stream_create: NULL out pointer");
    F3S_TRY(require_device());
    hipStream_t s;
    F3S_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return F3S_OK;
}

f3s_status f3s_stream_destroy(void* stream)
{
    if (!stream) return F3S_OK;
    F3S_HIP(hipStreamDestroy(as_stream(stream)));
    return F3S_OK;
}

f3s_status f3s_event_create(void** event)
{
    F3S_REQUIRE(event != nullptr, "f3s_event_create: NULL out pointer");
    F3S_TRY(require_device());
    hipEvent_t e;
    F3S_HIP(hipEventCreate(&e));
    *event = e;
    return F3S_OK;
}

f3s_status f3s_event_destroy(void* event)
{
    if (!event) return F3S_OK;
    F3S_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return F3S_OK;
}

f3s_status f3s_event_record(void* event, void* stream)
{
    F3S_REQUIRE(event != nullptr, "f3s_event_record: NULL event");
    F3S_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
    return F3S_OK;
}

f3s_status f3s_event_elapsed_ms(void* start, void* stop, float* ms)
{
    F3S_REQUIRE(start && stop && ms, "f3s_event_elapsed_ms: NULL argument");
    F3S_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
    F3S_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                reinterpret_cast<hipEvent_t>(stop)));
    return F3S_OK;
}

f3s_status f3s_cast_f32_to_f16(const float* d_in, uint16_t* d_out, int64_t count, void* stream)
{
    F3S_REQUIRE(count >= 0, "f3s_cast_f32_to_f16: negative count");
    if (count == 0) return F3S_OK;
    F3S_REQUIRE(d_in && d_out, "f3s_cast_f32_to_f16: NULL pointer");
    F3S_TRY(require_device());
    const int64_t threads = ceil_div(count, 4);
    const int64_t blocks = ceil_div(threads, 256);
    F3S_REQUIRE(blocks < (int64_t)1 << 31, "f3s_cast_f32_to_f16: count too large");
    hipLaunchKernelGGL(cast_f32_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       as_stream(stream), d_in, reinterpret_cast<_Float16*>(d_out), count);
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}

}  // extern "C"

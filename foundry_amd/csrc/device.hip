// Device lifecycle, storage, counters, batching and timing entry points of
// the C-ABI (include/foundry_hip.h). The reference counterparts are
// MetalDevice (src/metal/mod.rs:86-149, :527-725) and CommandStream
// (src/metal/stream.rs:29-215).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>

#include "device.hpp"
#include "q4_common.hpp"

namespace fh {

static thread_local char g_error[1024];

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_usable(fh_device *dev, const char *fn) {
    if (dev == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, "%s: device is null", fn);
    if (dev->failed)
        return fail(FH_ERR_FAILED, "%s: an earlier device error is sticky; recreate the device", fn);
    return FH_OK;
}

int set_current(fh_device *dev, const char *fn) {
    hipError_t err = hipSetDevice(dev->ordinal);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipSetDevice");
    return FH_OK;
}

int check_range(const fh_device *dev, const void *ptr, uint64_t nbytes, const char *fn,
                const char *what) {
    if (nbytes == 0) return FH_OK;
    if (ptr == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, "%s: %s is null", fn, what);
    const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
    auto it = dev->allocs.upper_bound(p);
    if (it == dev->allocs.begin())
        return fail(FH_ERR_FOREIGN_STORAGE, "%s: %s is not storage of this device", fn, what);
    --it;
    const uintptr_t base = it->first;
    const uint64_t size = it->second;
    if (p >= base + size)
        return fail(FH_ERR_FOREIGN_STORAGE, "%s: %s is not storage of this device", fn, what);
    if (nbytes > size - (p - base))
        return fail(FH_ERR_OUT_OF_BOUNDS,
                    "%s: %s needs %llu bytes but its allocation has %llu past the pointer", fn,
                    what, (unsigned long long)nbytes, (unsigned long long)(size - (p - base)));
    // a graph being captured retains every allocation its ops touch
    if (dev->capturing) dev->capture_bases.insert(base);
    return FH_OK;
}

int device_error(fh_device *dev, hipError_t err, const char *fn, const char *call) {
    if (err == hipSuccess) return FH_OK;
    if (dev) dev->failed = true;
    return fail(FH_ERR_FAILED, "%s: %s failed: %s", fn, call, hipGetErrorString(err));
}

hipEvent_t take_event(fh_device *dev) {
    if (!dev->event_pool.empty()) {
        hipEvent_t e = dev->event_pool.back();
        dev->event_pool.pop_back();
        return e;
    }
    if (dev->no_alloc) return nullptr;  // profiling skips this dispatch
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void record_profile_begin(fh_device *dev, hipEvent_t *begin) {
    *begin = nullptr;
    if (dev->capturing || dev->profile_mode == FH_PROFILE_OFF) return;
    if (dev->profile_mode == FH_PROFILE_STEPS && !dev->intervals.empty()) return;
    hipEvent_t e = take_event(dev);
    if (e && hipEventRecord(e, dev->stream) == hipSuccess) *begin = e;
}

void record_profile_end(fh_device *dev, hipEvent_t begin) {
    if (begin == nullptr) return;
    if (dev->profile_mode == FH_PROFILE_KERNELS) {
        hipEvent_t e = take_event(dev);
        if (e && hipEventRecord(e, dev->stream) == hipSuccess) {
            dev->intervals.emplace_back(begin, e);
            return;
        }
        dev->event_pool.push_back(begin);
        return;
    }
    // STEPS: one interval opened by the first dispatch, closed at take time
    dev->intervals.emplace_back(begin, nullptr);
}

// 16 bytes per thread: one 16-byte store where the piece is whole and
// aligned, byte stores at an unaligned head or a ragged tail.
__global__ __launch_bounds__(256) void zero_fill_kernel(uint8_t *__restrict__ p, uint64_t n) {
    const uint64_t i = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) * 16;
    if (i >= n) return;
    if (i + 16 <= n && (reinterpret_cast<uintptr_t>(p + i) & 15) == 0) {
        *reinterpret_cast<uint4 *>(p + i) = make_uint4(0, 0, 0, 0);
        return;
    }
    for (uint64_t j = i; j < i + 16 && j < n; ++j) p[j] = 0;
}

int zero_fill(fh_device *dev, const char *fn, void *ptr, uint64_t nbytes) {
    if (nbytes == 0) return FH_OK;
    const uint64_t blocks = (nbytes + 16 * 256 - 1) / (16 * 256);
    if (blocks > 0x7FFFFFFFull) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: fill of %llu bytes", fn,
                                            static_cast<unsigned long long>(nbytes));
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(zero_fill_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, dev->stream,
                           static_cast<uint8_t *>(ptr), nbytes);
    });
}

// The read probe: every thread loads 4 x 16 bytes, contiguous per wavefront
// (all four requested before any is used), with the nontemporal hint the
// decode GEMV's weight loads carry (222 MB read: 37.4 -> 34.1 us); each
// wavefront folds its loads into one XOR word that its lane 0 writes, so no
// block-wide barrier or reduction sits between the last load and the end.
// 512 threads x 4 loads per block was the fastest single-launch read of
// 14.2 MB in a sweep of block sizes (64-1024) and loads per thread (2-16).
constexpr uint32_t kProbeThreads = 512;
constexpr uint32_t kProbeUnroll = 4;
constexpr uint64_t kProbeBlockBytes = kProbeThreads * 16ull * kProbeUnroll;
constexpr uint32_t kProbeWaves = kProbeThreads / 64;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const uint4 *__restrict__ src, uint64_t pieces,
                                                                    uint32_t *__restrict__ out) {
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kProbeThreads * kProbeUnroll + threadIdx.x;
    uint4 v[kProbeUnroll];
#pragma unroll
    for (uint32_t u = 0; u < kProbeUnroll; ++u) {
        const uint64_t i = base + u * kProbeThreads;
        v[u] = load_stream16(src + (i < pieces ? i : pieces - 1));
    }
    uint32_t x = 0;
#pragma unroll
    for (uint32_t u = 0; u < kProbeUnroll; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x ^= __shfl_xor(x, off, 64);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * kProbeWaves + (threadIdx.x >> 6)] = x;
}

// Frees an allocation that is no longer in dev->allocs and that no live graph
// uses, after the work queued on the stream ends.
static hipError_t release(fh_device *dev, uintptr_t base, size_t size) {
    hipError_t err = hipStreamSynchronize(dev->stream);
    hipError_t ferr = hipFree(reinterpret_cast<void *>(base));
    dev->live_bytes -= size;
    return err != hipSuccess ? err : ferr;
}

// Drops one graph's hold on each of its allocations; frees those the caller
// already released once no graph uses them.
static hipError_t drop_graph_refs(fh_device *dev, const fh_graph *g) {
    hipError_t first = hipSuccess;
    for (uintptr_t base : g->bases) {
        auto r = dev->graph_refs.find(base);
        if (r == dev->graph_refs.end()) continue;
        if (--r->second > 0) continue;
        dev->graph_refs.erase(r);
        auto z = dev->retired.find(base);
        if (z == dev->retired.end()) continue;
        const size_t size = z->second;
        dev->retired.erase(z);
        hipError_t err = release(dev, base, size);
        if (first == hipSuccess) first = err;
    }
    return first;
}

// fh_free outside capture: a retained allocation is retired (no longer
// usable by ops, freed with its last graph), any other one freed now.
static int free_now(fh_device *dev, std::map<uintptr_t, size_t>::iterator it, const char *fn) {
    const uintptr_t base = it->first;
    const size_t size = it->second;
    dev->allocs.erase(it);
    if (dev->graph_refs.count(base)) {
        dev->retired[base] = size;
        return FH_OK;
    }
    hipSetDevice(dev->ordinal);
    hipError_t err = release(dev, base, size);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipStreamSynchronize/hipFree");
    return FH_OK;
}

static void note_allocation(fh_device *dev, uint64_t nbytes) {
    dev->live_bytes += nbytes;
    dev->peak_bytes = std::max(dev->peak_bytes, dev->live_bytes);
    dev->run_peak_bytes = std::max(dev->run_peak_bytes, dev->live_bytes);
    dev->counters.allocations += 1;
    dev->counters.allocated_bytes += nbytes;
}

}  // namespace fh

using namespace fh;

extern "C" {

const char *fh_last_error(void) { return g_error; }

int fh_abi_version(void) { return FH_ABI_VERSION; }

int fh_device_count(int *count) {
    if (!count) return fail(FH_ERR_INVALID_ARGUMENT, "fh_device_count: count is null");
    int n = 0;
    hipError_t err = hipGetDeviceCount(&n);
    *count = (err == hipSuccess) ? n : 0;
    return FH_OK;
}

static int create(int ordinal, int mode, fh_device **out, const char *fn) {
    if (!out) return fail(FH_ERR_INVALID_ARGUMENT, "%s: out is null", fn);
    *out = nullptr;
    if (mode < FH_PROFILE_OFF || mode > FH_PROFILE_KERNELS)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: unknown profile mode %d", fn, mode);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: no HIP device is available", fn);
    if (ordinal < 0 || ordinal >= n)
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: ordinal %d outside [0, %d)", fn, ordinal, n);
    if (hipSetDevice(ordinal) != hipSuccess)
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: hipSetDevice(%d) failed", fn, ordinal);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, ordinal) != hipSuccess)
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: hipGetDeviceProperties failed", fn);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(FH_ERR_DEVICE_UNAVAILABLE,
                    "%s: device %d is %s; this library is built for gfx950 only", fn, ordinal,
                    prop.gcnArchName);
    fh_device *dev = new (std::nothrow) fh_device();
    if (!dev) return fail(FH_ERR_ALLOCATION, "%s: out of host memory", fn);
    dev->ordinal = ordinal;
    dev->name = prop.name[0] ? prop.name : prop.gcnArchName;
    dev->compute_units = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    dev->profile_mode = mode;
    // default priority: streams of other priorities are not used anywhere
    if (hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking) != hipSuccess) {
        delete dev;
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: stream creation failed", fn);
    }
    if (hipEventCreate(&dev->timer_begin) != hipSuccess ||
        hipEventCreate(&dev->timer_end) != hipSuccess) {
        hipStreamDestroy(dev->stream);
        delete dev;
        return fail(FH_ERR_DEVICE_UNAVAILABLE, "%s: event creation failed", fn);
    }
    if (hipMalloc(&dev->pack_area, kPackAreaBytes) != hipSuccess ||
        hipMalloc(&dev->partial_area, kPartialAreaBytes) != hipSuccess) {
        hipFree(dev->pack_area);
        hipEventDestroy(dev->timer_begin);
        hipEventDestroy(dev->timer_end);
        hipStreamDestroy(dev->stream);
        delete dev;
        return fail(FH_ERR_ALLOCATION, "%s: the device's %llu-byte work areas could not be allocated", fn,
                    static_cast<unsigned long long>(kPackAreaBytes + kPartialAreaBytes));
    }
    if (int rc = attention_scratch_setup(dev)) {
        hipFree(dev->pack_area);
        hipFree(dev->partial_area);
        hipEventDestroy(dev->timer_begin);
        hipEventDestroy(dev->timer_end);
        hipStreamDestroy(dev->stream);
        delete dev;
        return rc;
    }
    // the work areas are device memory the ops use: counted in the peaks
    dev->live_bytes = kPackAreaBytes + kPartialAreaBytes;
    dev->peak_bytes = dev->run_peak_bytes = dev->live_bytes;
    *out = dev;
    return FH_OK;
}

int fh_device_create(int ordinal, fh_device **out) {
    return create(ordinal, FH_PROFILE_OFF, out, "fh_device_create");
}

int fh_device_create_profiled(int ordinal, int mode, fh_device **out) {
    return create(ordinal, mode, out, "fh_device_create_profiled");
}

int fh_device_destroy(fh_device *dev) {
    if (!dev) return FH_OK;
    hipSetDevice(dev->ordinal);
    if (dev->capturing) {
        hipGraph_t g = nullptr;
        hipStreamEndCapture(dev->stream, &g);
        if (g) hipGraphDestroy(g);
    }
    hipError_t err = hipStreamSynchronize(dev->stream);
    // graphs outlive their device only as handles: they can no longer launch
    for (fh_graph *g : dev->graphs) g->dev = nullptr;
    for (auto &kv : dev->allocs) hipFree(reinterpret_cast<void *>(kv.first));
    for (auto &kv : dev->retired) hipFree(reinterpret_cast<void *>(kv.first));
    hipFree(dev->pack_area);
    hipFree(dev->partial_area);
    for (auto &iv : dev->intervals) {
        if (iv.first) hipEventDestroy(iv.first);
        if (iv.second) hipEventDestroy(iv.second);
    }
    for (hipEvent_t e : dev->event_pool) hipEventDestroy(e);
    hipEventDestroy(dev->timer_begin);
    hipEventDestroy(dev->timer_end);
    hipStreamDestroy(dev->stream);
    delete dev;
    if (err != hipSuccess)
        return fail(FH_ERR_FAILED, "fh_device_destroy: pending work failed: %s",
                    hipGetErrorString(err));
    return FH_OK;
}

int fh_device_name(const fh_device *dev, char *buf, size_t len) {
    if (!dev || !buf || len == 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "fh_device_name: null argument");
    std::snprintf(buf, len, "%s", dev->name.c_str());
    return FH_OK;
}

int fh_synchronize(fh_device *dev) {
    const char *fn = "fh_synchronize";
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: the device is capturing", fn);
    if (int rc = set_current(dev, fn)) return rc;
    return device_error(dev, hipStreamSynchronize(dev->stream), fn, "hipStreamSynchronize");
}

int fh_device_stream(fh_device *dev, void **stream) {
    if (!dev || !stream) return fail(FH_ERR_INVALID_ARGUMENT, "fh_device_stream: null argument");
    *stream = reinterpret_cast<void *>(dev->stream);
    return FH_OK;
}

int fh_alloc(fh_device *dev, size_t nbytes, int zero_fill, void **out) {
    const char *fn = "fh_alloc";
    if (!out) return fail(FH_ERR_INVALID_ARGUMENT, "%s: out is null", fn);
    *out = nullptr;
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: cannot allocate while capturing", fn);
    if (int rc = set_current(dev, fn)) return rc;
    const size_t size = std::max<size_t>(nbytes, 1);
    void *p = nullptr;
    hipError_t err = hipMalloc(&p, size);
    if (err != hipSuccess || p == nullptr) {
        hipGetLastError();  // an out-of-memory refusal is not a device fault
        return fail(FH_ERR_ALLOCATION, "%s: hipMalloc(%zu) failed: %s", fn, size,
                    hipGetErrorString(err));
    }
    if (zero_fill) {
        err = hipMemsetAsync(p, 0, size, dev->stream);
        if (err != hipSuccess) {
            hipFree(p);
            return device_error(dev, err, fn, "hipMemsetAsync");
        }
    }
    dev->allocs[reinterpret_cast<uintptr_t>(p)] = size;
    note_allocation(dev, size);
    *out = p;
    return FH_OK;
}

int fh_free(fh_device *dev, void *ptr) {
    const char *fn = "fh_free";
    if (!dev) return fail(FH_ERR_INVALID_ARGUMENT, "%s: device is null", fn);
    if (!ptr) return FH_OK;
    auto it = dev->allocs.find(reinterpret_cast<uintptr_t>(ptr));
    if (it == dev->allocs.end())
        return fail(FH_ERR_FOREIGN_STORAGE, "%s: pointer is not an allocation of this device", fn);
    if (dev->capturing) {
        // the capture may already use it: decided at fh_capture_end
        for (void *q : dev->deferred_frees)
            if (q == ptr) return FH_OK;
        dev->deferred_frees.push_back(ptr);
        return FH_OK;
    }
    return free_now(dev, it, fn);
}

int fh_upload(fh_device *dev, void *dst, const void *src, size_t nbytes) {
    const char *fn = "fh_upload";
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: cannot copy while capturing", fn);
    if (nbytes == 0) return FH_OK;
    if (!src) return fail(FH_ERR_INVALID_ARGUMENT, "%s: src is null", fn);
    if (int rc = check_range(dev, dst, nbytes, fn, "dst")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    // pageable source: the copy is complete on return, ordered after queued work
    hipError_t err = hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, dev->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(dev->stream);
    return device_error(dev, err, fn, "hipMemcpyAsync");
}

int fh_download(fh_device *dev, void *dst, const void *src, size_t nbytes) {
    const char *fn = "fh_download";
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: cannot copy while capturing", fn);
    if (nbytes == 0) return FH_OK;
    if (!dst) return fail(FH_ERR_INVALID_ARGUMENT, "%s: dst is null", fn);
    if (int rc = check_range(dev, src, nbytes, fn, "src")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    hipError_t err = hipStreamSynchronize(dev->stream);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipStreamSynchronize");
    err = hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, dev->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(dev->stream);
    return device_error(dev, err, fn, "hipMemcpyAsync");
}

int fh_max_memory_allocated(const fh_device *dev, fh_allocated_memory *out) {
    if (!dev || !out) return fail(FH_ERR_INVALID_ARGUMENT, "fh_max_memory_allocated: null");
    out->bytes = dev->peak_bytes;
    out->source = "hip_device_allocations";
    return FH_OK;
}

int fh_reset_run_memory_peak(fh_device *dev) {
    const char *fn = "fh_reset_run_memory_peak";
    if (int rc = check_usable(dev, fn)) return rc;
    if (!dev->capturing) {
        if (int rc = set_current(dev, fn)) return rc;
        hipError_t err = hipStreamSynchronize(dev->stream);
        if (err != hipSuccess) return device_error(dev, err, fn, "hipStreamSynchronize");
    }
    dev->run_peak_bytes = dev->live_bytes;
    dev->peak_bytes = std::max(dev->peak_bytes, dev->run_peak_bytes);
    return FH_OK;
}

int fh_run_memory_peak(const fh_device *dev, fh_allocated_memory *out) {
    if (!dev || !out) return fail(FH_ERR_INVALID_ARGUMENT, "fh_run_memory_peak: null");
    out->bytes = dev->run_peak_bytes;
    out->source = "hip_device_allocations";
    return FH_OK;
}

int fh_take_profile(fh_device *dev, fh_profile *out) {
    const char *fn = "fh_take_profile";
    if (!out) return fail(FH_ERR_INVALID_ARGUMENT, "%s: out is null", fn);
    std::memset(out, 0, sizeof(*out));
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->profile_mode == FH_PROFILE_OFF)
        return fail(FH_ERR_UNSUPPORTED, "%s: the device was not created profiled", fn);
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: the device is capturing", fn);
    if (int rc = set_current(dev, fn)) return rc;
    // close the STEPS span
    for (auto &iv : dev->intervals)
        if (iv.second == nullptr) {
            iv.second = take_event(dev);
            if (iv.second) hipEventRecord(iv.second, dev->stream);
        }
    hipError_t err = hipStreamSynchronize(dev->stream);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipStreamSynchronize");
    // union of [begin, end] intervals, measured from the first begin
    std::vector<std::pair<double, double>> spans;
    if (!dev->intervals.empty()) {
        hipEvent_t epoch = dev->intervals.front().first;
        for (auto &iv : dev->intervals) {
            float a = 0.f, b = 0.f;
            if (!iv.second) continue;
            if (hipEventElapsedTime(&a, epoch, iv.first) != hipSuccess) continue;
            if (hipEventElapsedTime(&b, epoch, iv.second) != hipSuccess) continue;
            spans.emplace_back(a, b);
        }
        std::sort(spans.begin(), spans.end());
    }
    double busy_ms = 0.0, cur_a = 0.0, cur_b = -1.0;
    for (auto &s : spans) {
        if (s.first > cur_b) {
            if (cur_b > cur_a) busy_ms += cur_b - cur_a;
            cur_a = s.first;
            cur_b = s.second;
        } else {
            cur_b = std::max(cur_b, s.second);
        }
    }
    if (cur_b > cur_a) busy_ms += cur_b - cur_a;
    for (auto &iv : dev->intervals) {
        if (iv.first) dev->event_pool.push_back(iv.first);
        if (iv.second) dev->event_pool.push_back(iv.second);
    }
    dev->intervals.clear();
    *out = dev->counters;
    out->gpu_busy_ns = static_cast<uint64_t>(busy_ms * 1e6);
    dev->counters = fh_profile{};
    return FH_OK;
}

int fh_capture_begin(fh_device *dev) {
    const char *fn = "fh_capture_begin";
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: already capturing", fn);
    if (int rc = set_current(dev, fn)) return rc;
    hipError_t err = hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipStreamBeginCapture");
    dev->capturing = true;
    dev->capture_bases.clear();
    return FH_OK;
}

namespace {

// Carries out the frees asked for during a capture that has just ended
// (after the new graph, if any, took its references).
int run_deferred_frees(fh_device *dev, const char *fn) {
    std::vector<void *> pending;
    pending.swap(dev->deferred_frees);
    int rc = FH_OK;
    for (void *p : pending) {
        auto it = dev->allocs.find(reinterpret_cast<uintptr_t>(p));
        if (it == dev->allocs.end()) continue;
        const int r = free_now(dev, it, fn);
        if (rc == FH_OK) rc = r;
    }
    return rc;
}

}  // namespace

int fh_capture_end(fh_device *dev, fh_graph **out) {
    const char *fn = "fh_capture_end";
    if (!out) return fail(FH_ERR_INVALID_ARGUMENT, "%s: out is null", fn);
    *out = nullptr;
    if (!dev) return fail(FH_ERR_INVALID_ARGUMENT, "%s: device is null", fn);
    if (!dev->capturing) return fail(FH_ERR_CAPTURE, "%s: the device is not capturing", fn);
    hipSetDevice(dev->ordinal);
    hipGraph_t graph = nullptr;
    hipError_t err = hipStreamEndCapture(dev->stream, &graph);
    dev->capturing = false;
    std::set<uintptr_t> bases;
    bases.swap(dev->capture_bases);
    if (err != hipSuccess) {
        run_deferred_frees(dev, fn);
        return device_error(dev, err, fn, "hipStreamEndCapture");
    }
    if (dev->failed) {
        if (graph) hipGraphDestroy(graph);
        run_deferred_frees(dev, fn);
        return fail(FH_ERR_FAILED, "%s: a launch failed during capture", fn);
    }
    fh_graph *g = new (std::nothrow) fh_graph();
    if (!g) {
        hipGraphDestroy(graph);
        run_deferred_frees(dev, fn);
        return fail(FH_ERR_ALLOCATION, "%s: out of host memory", fn);
    }
    g->graph = graph;
    g->ordinal = dev->ordinal;
    err = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        hipGraphDestroy(graph);
        delete g;
        run_deferred_frees(dev, fn);
        return device_error(dev, err, fn, "hipGraphInstantiate");
    }
    g->dev = dev;
    g->bases.assign(bases.begin(), bases.end());
    for (uintptr_t b : g->bases) dev->graph_refs[b] += 1;
    dev->graphs.insert(g);
    *out = g;
    return run_deferred_frees(dev, fn);
}

int fh_graph_launch(fh_device *dev, fh_graph *graph) {
    const char *fn = "fh_graph_launch";
    if (int rc = check_usable(dev, fn)) return rc;
    if (!graph) return fail(FH_ERR_INVALID_ARGUMENT, "%s: graph is null", fn);
    if (graph->dev != dev)
        return fail(FH_ERR_FOREIGN_STORAGE, "%s: graph was captured on another device", fn);
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: the device is capturing", fn);
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] { hipGraphLaunch(graph->exec, dev->stream); });
}

int fh_graph_destroy(fh_graph *graph) {
    const char *fn = "fh_graph_destroy";
    if (!graph) return FH_OK;
    hipSetDevice(graph->ordinal);
    fh_device *dev = graph->dev;
    // a replay still queued on the stream reads the exec's nodes and the
    // allocations it retains: let it finish first
    hipError_t err = dev ? hipStreamSynchronize(dev->stream) : hipSuccess;
    if (graph->exec) hipGraphExecDestroy(graph->exec);
    if (graph->graph) hipGraphDestroy(graph->graph);
    hipError_t rerr = hipSuccess;
    if (dev) {
        dev->graphs.erase(graph);
        rerr = drop_graph_refs(dev, graph);
    }
    delete graph;
    if (err != hipSuccess) return device_error(dev, err, fn, "hipStreamSynchronize");
    if (rerr != hipSuccess) return device_error(dev, rerr, fn, "hipFree");
    return FH_OK;
}

int fh_read_probe_blocks(uint64_t nbytes, uint64_t *blocks) {
    if (!blocks) return fail(FH_ERR_INVALID_ARGUMENT, "fh_read_probe_blocks: blocks is null");
    *blocks = (nbytes + kProbeBlockBytes - 1) / kProbeBlockBytes * kProbeWaves;  // output words
    return FH_OK;
}

int fh_read_probe(fh_device *dev, const void *src, uint64_t nbytes, uint32_t *out) {
    const char *fn = "fh_read_probe";
    if (int rc = check_usable(dev, fn)) return rc;
    if (nbytes == 0) return FH_OK;
    if (nbytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
        return fail(FH_ERR_INVALID_ARGUMENT, "%s: src must be 16-byte aligned and nbytes a multiple of 16", fn);
    const uint64_t blocks = (nbytes + kProbeBlockBytes - 1) / kProbeBlockBytes;
    if (blocks > 0x7FFFFFFFull) return fail(FH_ERR_INDEX_TOO_LARGE, "%s: %llu bytes", fn, (unsigned long long)nbytes);
    if (int rc = check_range(dev, src, nbytes, fn, "src")) return rc;
    if (int rc = check_range(dev, out, blocks * kProbeWaves * 4, fn, "out")) return rc;
    if (int rc = set_current(dev, fn)) return rc;
    return dispatch(dev, fn, [&] {
        hipLaunchKernelGGL(read_probe_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kProbeThreads), 0,
                           dev->stream, static_cast<const uint4 *>(src), nbytes / 16, out);
    });
}

int fh_timer_begin(fh_device *dev) {
    const char *fn = "fh_timer_begin";
    if (int rc = check_usable(dev, fn)) return rc;
    if (dev->capturing) return fail(FH_ERR_CAPTURE, "%s: the device is capturing", fn);
    if (int rc = set_current(dev, fn)) return rc;
    hipError_t err = hipEventRecord(dev->timer_begin, dev->stream);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipEventRecord");
    dev->timer_started = true;
    return FH_OK;
}

int fh_timer_end(fh_device *dev, double *elapsed_ms) {
    const char *fn = "fh_timer_end";
    if (!elapsed_ms) return fail(FH_ERR_INVALID_ARGUMENT, "%s: elapsed_ms is null", fn);
    if (int rc = check_usable(dev, fn)) return rc;
    if (!dev->timer_started) return fail(FH_ERR_INVALID_ARGUMENT, "%s: no timer_begin", fn);
    if (int rc = set_current(dev, fn)) return rc;
    hipError_t err = hipEventRecord(dev->timer_end, dev->stream);
    if (err == hipSuccess) err = hipEventSynchronize(dev->timer_end);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipEventRecord/Synchronize");
    float ms = 0.f;
    err = hipEventElapsedTime(&ms, dev->timer_begin, dev->timer_end);
    if (err != hipSuccess) return device_error(dev, err, fn, "hipEventElapsedTime");
    dev->timer_started = false;
    *elapsed_ms = ms;
    return FH_OK;
}

}  // extern "C"

// Internal state of an fh_device and the helpers every op entry point uses:
// error reporting, ownership/bounds checks and the dispatch wrapper.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <map>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/foundry_hip.h"

namespace fh {

// Writes the thread-local message returned by fh_last_error and returns code.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace fh

struct fh_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int ordinal = 0;
    // The device that captured it (null once that device is destroyed) and
    // the base address of every allocation its captured ops touched: the
    // graph retains them, so none is freed while the graph can replay.
    fh_device *dev = nullptr;
    std::vector<uintptr_t> bases;
};

namespace fh {
// Bytes of each device's pack area: the matrix-core GEMV's normalised x image
// (8 rows of up to 16384 values as fragments, two slots, their group sums,
// padding to whole wavefronts), written by the pack kernel and copied by the
// GEMV's prologue in stream order.
constexpr uint64_t kPackAreaBytes = 8ull * 16384 * 2 + (16384 / 64) * 8 * 4 + 2048;
// Bytes of each device's partial area: the f32 partial sums [ranges][rows][n]
// of a GEMV split over K ranges, or [splits][m][n] of a GEMM split over K,
// added in order by the matching combine kernel.
constexpr uint64_t kPartialAreaBytes = 128ull << 20;
// K splits of a prompt-length GEMM at most (their f32 partials share the area).
constexpr uint32_t kMaxGemmSplits = 8;
}  // namespace fh

struct fh_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    std::string name;
    uint32_t compute_units = 0;  // sizes persistent grids
    void *pack_area = nullptr;     // kPackAreaBytes, owned by the device (not in allocs)
    void *partial_area = nullptr;  // kPartialAreaBytes, likewise
    // base address -> size of every live allocation this device made
    std::map<uintptr_t, size_t> allocs;
    uint64_t live_bytes = 0;
    uint64_t peak_bytes = 0;
    uint64_t run_peak_bytes = 0;
    bool failed = false;
    bool capturing = false;
    // Graph lifetime. While capturing, every allocation an op's range check
    // accepts is noted in capture_bases; fh_capture_end hands the set to the
    // new graph and counts it in graph_refs (base -> live graphs that use
    // it). fh_free of a retained allocation moves it to retired (base ->
    // size), freed when its last graph is destroyed; frees asked for during
    // capture wait in deferred_frees until fh_capture_end.
    mutable std::set<uintptr_t> capture_bases;
    std::map<uintptr_t, uint32_t> graph_refs;
    std::map<uintptr_t, size_t> retired;
    std::vector<void *> deferred_frees;
    std::set<fh_graph *> graphs;
    // this GPU's copy of the no-allocation entry point's static workspace
    void *scratch = nullptr;
    // set while an entry point that must not allocate dispatches: profiling
    // then uses pooled events only
    bool no_alloc = false;
    int profile_mode = FH_PROFILE_OFF;
    fh_profile counters{};
    // per-dispatch event pairs (KERNELS mode) or the span of a step (STEPS)
    std::vector<std::pair<hipEvent_t, hipEvent_t>> intervals;
    std::vector<hipEvent_t> event_pool;
    hipEvent_t timer_begin = nullptr;
    hipEvent_t timer_end = nullptr;
    bool timer_started = false;
};

namespace fh {

// Sticky-failure gate at the start of every call that touches the device.
int check_usable(fh_device *dev, const char *fn);

// Makes the device's GPU current for the calling thread.
int set_current(fh_device *dev, const char *fn);

// The operand [ptr, ptr + nbytes) must lie inside one live allocation of dev.
int check_range(const fh_device *dev, const void *ptr, uint64_t nbytes, const char *fn,
                const char *what);

// Records a HIP error from `call`, marks the device failed and returns
// FH_ERR_FAILED; FH_OK when err is hipSuccess.
int device_error(fh_device *dev, hipError_t err, const char *fn, const char *call);

// Launch wrapper: brackets the launch with profiling events when enabled,
// checks the launch status, and counts the dispatch.
template <typename Launch>
int dispatch(fh_device *dev, const char *fn, Launch &&launch);

// Looks up this GPU's address of the static decode-attention workspace
// (attention.hip); called by device creation with the device current.
int attention_scratch_setup(fh_device *dev);

// Writes nbytes of zeros at ptr on the device's stream with a kernel (not
// hipMemsetAsync: a captured memset node is not reliable on replay).
int zero_fill(fh_device *dev, const char *fn, void *ptr, uint64_t nbytes);

hipEvent_t take_event(fh_device *dev);
void record_profile_begin(fh_device *dev, hipEvent_t *begin);
void record_profile_end(fh_device *dev, hipEvent_t begin);

template <typename Launch>
int dispatch(fh_device *dev, const char *fn, Launch &&launch) {
    hipEvent_t begin = nullptr;
    record_profile_begin(dev, &begin);
    launch();
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        dev->failed = true;
        return fail(FH_ERR_LAUNCH, "%s: kernel launch failed: %s", fn, hipGetErrorString(err));
    }
    record_profile_end(dev, begin);
    dev->counters.dispatches += 1;
    return FH_OK;
}

}  // namespace fh

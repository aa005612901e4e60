#pragma once
// Status-returning helpers for host code of the launch layer: device buffers
// that free themselves, HIP calls turned into engine::Error, and event timing
// that reports failures instead of exiting.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <vector>

#include "engine.h"

namespace spmm {
namespace engine {

inline Error hip_error(hipError_t e, const char* what) {
    return Error{kHipError, std::string(what) + ": " + hipGetErrorString(e)};
}

// Returns an Error from the enclosing function when a HIP call fails.
#define SPMM_TRY_HIP(expr, what)                                   \
    do {                                                           \
        const hipError_t spmm_e_ = (expr);                         \
        if (spmm_e_ != hipSuccess) return hip_error(spmm_e_, what); \
    } while (0)

#define SPMM_TRY(expr)                                             \
    do {                                                           \
        Error spmm_err_ = (expr);                                  \
        if (spmm_err_.status != kOk) return spmm_err_;             \
    } while (0)

// hipMalloc'd or hipMallocManaged memory released on scope exit.
struct DeviceBuffer {
    void* p = nullptr;
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() {
        if (p != nullptr) (void)hipFree(p);
    }
    template <typename T>
    T* as() const { return static_cast<T*>(p); }
};

// Median of per-launch times: warmup untimed launches, then iters launches
// each bracketed by events on the null stream (the reference's GpuTimer
// protocol, utils.h:38-56).  launch() returns an Error.
template <typename Launch>
Error time_median_launch(Launch launch, int warmup, int iters, float* ms_out) {
    for (int i = 0; i < warmup; ++i) SPMM_TRY(launch());
    SPMM_TRY_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    SPMM_TRY_HIP(hipEventCreate(&e0), "hipEventCreate");
    const hipError_t c1 = hipEventCreate(&e1);
    if (c1 != hipSuccess) {
        (void)hipEventDestroy(e0);
        return hip_error(c1, "hipEventCreate");
    }
    std::vector<float> times;
    Error err;
    for (int i = 0; i < iters && err.status == kOk; ++i) {
        hipError_t e = hipEventRecord(e0, nullptr);
        if (e == hipSuccess) {
            err = launch();
            if (err.status != kOk) break;
            e = hipEventRecord(e1, nullptr);
        }
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e != hipSuccess) err = hip_error(e, "event timing");
        times.push_back(ms);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (err.status != kOk) return err;
    if (times.empty()) {
        *ms_out = 0.f;
    } else {
        std::vector<float> v = times;
        std::sort(v.begin(), v.end());
        *ms_out = v[v.size() / 2];  // harness.cu:198-201
    }
    return Error{};
}

}  // namespace engine
}  // namespace spmm

#pragma once
// Error macro, ceil_div and an event timer (reference src/utils.h:8-56).
//
// HIP_CHECK keeps the reference's CUDA_CHECK convention: print the failing call
// with file:line and exit(EXIT_FAILURE).  There is no sparse-library check
// macro: nothing in this engine calls a vendor sparse library.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define HIP_CHECK(call)                                                        \
    do {                                                                       \
        hipError_t hip_err_ = (call);                                          \
        if (hip_err_ != hipSuccess) {                                          \
            std::fprintf(stderr, "HIP error %s at %s:%d: %s\n", #call,         \
                         __FILE__, __LINE__, hipGetErrorString(hip_err_));     \
            std::exit(EXIT_FAILURE);                                           \
        }                                                                      \
    } while (0)

constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Event pair on one stream (the null stream by default, as utils.h:32-56).
// stop() waits for the stop event, so elapsed_ms() is valid right after it.
class GpuTimer {
public:
    explicit GpuTimer(hipStream_t stream = nullptr) : stream_(stream) {
        HIP_CHECK(hipEventCreate(&start_));
        HIP_CHECK(hipEventCreate(&stop_));
    }
    ~GpuTimer() {
        (void)hipEventDestroy(start_);
        (void)hipEventDestroy(stop_);
    }
    GpuTimer(const GpuTimer&) = delete;
    GpuTimer& operator=(const GpuTimer&) = delete;

    void start() { HIP_CHECK(hipEventRecord(start_, stream_)); }
    void stop() {
        HIP_CHECK(hipEventRecord(stop_, stream_));
        HIP_CHECK(hipEventSynchronize(stop_));
    }
    float elapsed_ms() {
        float t = 0.f;
        HIP_CHECK(hipEventElapsedTime(&t, start_, stop_));
        return t;
    }

private:
    hipStream_t stream_;
    hipEvent_t  start_;
    hipEvent_t  stop_;
};

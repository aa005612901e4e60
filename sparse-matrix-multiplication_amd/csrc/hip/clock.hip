// Shader-clock trace: the shader clock the GPU delivers, sampled on the
// device from the shader-cycle counter (s_memtime) and the constant 100 MHz
// real-time counter (s_memrealtime), `samples` times `interval` ticks apart,
// by one wave.  Run on a second stream beside a workload, the clock of each
// interval is 100 MHz x delta cycles / delta ticks while that workload runs.
//
// A timing diagnostic, no counterpart in the reference.  On MI355X the DPM
// state reads its top level (2.4 GHz) from the first launch, yet under the
// full load of the SpMM kernels the delivered clock starts near 2.15 GHz
// after an idle period and rises to about 2.39 GHz over some 600 back-to-back
// launches; a lone sampler on an idle GPU reads about 2.4 GHz.
//
// The wave only sleeps between samples and ends after samples x interval
// ticks of real time (bounded by the launcher), whatever else runs.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "engine.h"

namespace spmm {
namespace engine {

namespace {

__global__ __launch_bounds__(64) void shader_clock_kernel(unsigned long long* __restrict__ out,
                                                          int samples, int interval) {
    const unsigned lane = threadIdx.x;
    unsigned long long next = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < samples; ++i) {
        while (__builtin_amdgcn_s_memrealtime() < next) __builtin_amdgcn_s_sleep(2);
        const unsigned long long c = __builtin_amdgcn_s_memtime();
        const unsigned long long r = __builtin_amdgcn_s_memrealtime();
        if (lane < 2) out[2 * i + lane] = lane == 0 ? c : r;  // (cycles, ticks)
        next = r + static_cast<unsigned long long>(interval);
    }
}

}  // namespace

Error launch_shader_clock_trace(unsigned long long* d_out, int samples, int interval_ticks,
                                hipStream_t stream) {
    if (d_out == nullptr) return Error{kInvalid, "null output"};
    if (samples < 2 || samples > (1 << 20) || interval_ticks < 1 || interval_ticks > 100000000) {
        return Error{kInvalid, "samples must be 2 .. 2^20 and interval 1 .. 1e8 ticks"};
    }
    // at most 60 s of real time (100 MHz ticks)
    if (static_cast<long long>(samples - 1) * interval_ticks > 6000000000LL) {
        return Error{kInvalid, "trace longer than 60 s"};
    }
    hipLaunchKernelGGL(shader_clock_kernel, dim3(1), dim3(64), 0, stream, d_out, samples,
                       interval_ticks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return Error{kHipError, hipGetErrorString(e)};
    return Error{};
}

}  // namespace engine
}  // namespace spmm

// spmm_probe: the hardware figures the engine's design and rooflines rest on,
// measured on the GPU it runs on (no counterpart in the reference).
//
//   spmm_probe floor    back-to-back launches of an empty kernel (1 .. 8192
//                       workgroups) and of a kernel that only writes an
//                       M x 128 fp32 C (the fixed cost of every SpMM launch)
//   spmm_probe gather   random 512-byte row gathers from a K x 128 fp32 B, the
//                       CSR engine's access pattern: one row per half-wave
//                       with 16-byte lanes (the engine's form) and one row per
//                       wave with 8-byte lanes, for B of 4 MB (fits one XCD's
//                       L2) and 8 MB
//   spmm_probe copy     device-to-device copy of 256 MiB (measured HBM rate)
//
// Each line: probe=<name> ... value=<number> unit=<unit>.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "spmm/utils.h"

namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRowsPerWave = 256;  // gathered rows per wave

__global__ __launch_bounds__(256) void empty_kernel(int* flag) {
    if (blockIdx.x == 0 && threadIdx.x == 0 && flag[0] == 12345) flag[1] = 1;  // never taken
}

__global__ __launch_bounds__(256) void store_kernel(float* out, long n) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) reinterpret_cast<f32x4*>(out)[i] = f32x4(0.0f);
}

// One B row (128 floats) per half-wave, 16-byte lanes; U rows in flight per lane.
template <int U>
__global__ __launch_bounds__(256) void gather_half_wave(const float* __restrict__ B,
                                                        const int* __restrict__ rows,
                                                        float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const long wave = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int* my = rows + wave * kRowsPerWave;
    const int half = lane >> 5;
    const int col = (lane & 31) * 4;
    f32x4 acc = f32x4(0.0f);
    for (int p = 0; p < kRowsPerWave; p += 2 * U) {
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = my[p + 2 * u + half];
            v[u] = *reinterpret_cast<const f32x4*>(B + static_cast<size_t>(k) * 128 + col);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += v[u];
    }
    reinterpret_cast<f32x4*>(out)[wave * 64 + lane] = acc;
}

// One B row per wave, 8-byte lanes.
template <int U>
__global__ __launch_bounds__(256) void gather_full_wave(const float* __restrict__ B,
                                                        const int* __restrict__ rows,
                                                        float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const long wave = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int* my = rows + wave * kRowsPerWave;
    const int col = lane * 2;
    f32x2 acc = f32x2(0.0f);
    for (int p = 0; p < kRowsPerWave; p += U) {
        f32x2 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = my[p + u];
            v[u] = *reinterpret_cast<const f32x2*>(B + static_cast<size_t>(k) * 128 + col);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += v[u];
    }
    reinterpret_cast<f32x2*>(out)[wave * 64 + lane] = acc;
}

template <typename Launch>
float time_per_launch(Launch launch, int reps) {
    for (int i = 0; i < 5; ++i) launch();
    HIP_CHECK(hipDeviceSynchronize());
    GpuTimer t;
    float best = 1e30f;
    for (int trial = 0; trial < 5; ++trial) {
        t.start();
        for (int i = 0; i < reps; ++i) launch();
        t.stop();
        best = std::min(best, t.elapsed_ms() / reps);
    }
    return best;
}

void probe_floor() {
    int* flag = nullptr;
    HIP_CHECK(hipMalloc(&flag, 2 * sizeof(int)));
    HIP_CHECK(hipMemset(flag, 0, 2 * sizeof(int)));
    for (int grid : {1, 64, 256, 1024, 4096, 8192}) {
        const float ms = time_per_launch(
            [&] { hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(256), 0, nullptr, flag); },
            200);
        std::printf("probe=launch_floor workgroups=%d value=%.3f unit=us\n", grid, ms * 1e3f);
    }
    HIP_CHECK(hipFree(flag));
    for (int m : {4096, 8192, 16384}) {
        const long n4 = static_cast<long>(m) * 128 / 4;  // float4 stores
        float* out = nullptr;
        HIP_CHECK(hipMalloc(&out, sizeof(float) * static_cast<size_t>(m) * 128));
        const unsigned grid = static_cast<unsigned>((n4 + 255) / 256);
        const float ms = time_per_launch(
            [&] { hipLaunchKernelGGL(store_kernel, dim3(grid), dim3(256), 0, nullptr, out, n4); },
            200);
        const double mb = 4.0 * m * 128 / 1e6;
        std::printf("probe=store_only rows=%d mbytes=%.1f value=%.3f unit=us\n", m, mb, ms * 1e3f);
        HIP_CHECK(hipFree(out));
    }
}

void probe_gather() {
    const long waves = 16384;  // 64 per CU
    const long nrows = waves * kRowsPerWave;
    for (int K : {8192, 16384}) {
        std::vector<int> h_rows(static_cast<size_t>(nrows));
        std::mt19937 rng(1234u + K);
        std::uniform_int_distribution<int> pick(0, K - 1);
        for (int& r : h_rows) r = pick(rng);
        std::vector<float> h_B(static_cast<size_t>(K) * 128, 1.0f);
        float *B = nullptr, *out = nullptr;
        int* rows = nullptr;
        HIP_CHECK(hipMalloc(&B, sizeof(float) * h_B.size()));
        HIP_CHECK(hipMalloc(&rows, sizeof(int) * h_rows.size()));
        HIP_CHECK(hipMalloc(&out, sizeof(float) * 4 * 64 * waves));
        HIP_CHECK(hipMemcpy(B, h_B.data(), sizeof(float) * h_B.size(), hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(rows, h_rows.data(), sizeof(int) * h_rows.size(),
                            hipMemcpyHostToDevice));
        const dim3 grid(static_cast<unsigned>(waves / 4));
        const double bytes = 512.0 * nrows;  // gathered B bytes per launch
        const double b_mb = 512.0 * K / 1e6;
        const float half8 = time_per_launch(
            [&] { hipLaunchKernelGGL(gather_half_wave<8>, grid, dim3(256), 0, nullptr, B, rows, out); },
            20);
        const float full8 = time_per_launch(
            [&] { hipLaunchKernelGGL(gather_full_wave<8>, grid, dim3(256), 0, nullptr, B, rows, out); },
            20);
        const float full16 = time_per_launch(
            [&] { hipLaunchKernelGGL(gather_full_wave<16>, grid, dim3(256), 0, nullptr, B, rows, out); },
            20);
        std::printf("probe=gather form=half_wave_16B b_mbytes=%.1f value=%.2f unit=TB/s\n", b_mb,
                    bytes / (half8 * 1e-3) / 1e12);
        std::printf("probe=gather form=full_wave_8B b_mbytes=%.1f value=%.2f unit=TB/s\n", b_mb,
                    bytes / (std::min(full8, full16) * 1e-3) / 1e12);
        HIP_CHECK(hipFree(B));
        HIP_CHECK(hipFree(rows));
        HIP_CHECK(hipFree(out));
    }
}

void probe_copy() {
    const size_t bytes = size_t(256) << 20;
    void *a = nullptr, *b = nullptr;
    HIP_CHECK(hipMalloc(&a, bytes));
    HIP_CHECK(hipMalloc(&b, bytes));
    HIP_CHECK(hipMemset(a, 1, bytes));
    const float ms = time_per_launch(
        [&] { HIP_CHECK(hipMemcpyAsync(b, a, bytes, hipMemcpyDeviceToDevice, nullptr)); }, 20);
    std::printf("probe=copy mbytes=%.0f value=%.2f unit=TB/s (read+write)\n", bytes / 1e6,
                2.0 * bytes / (ms * 1e-3) / 1e12);
    HIP_CHECK(hipFree(a));
    HIP_CHECK(hipFree(b));
}

}  // namespace

int main(int argc, char** argv) {
    const std::string what = argc > 1 ? argv[1] : "all";
    if (what != "floor" && what != "gather" && what != "copy" && what != "all") {
        std::fprintf(stderr, "usage: %s [floor|gather|copy|all]\n", argv[0]);
        return EXIT_FAILURE;
    }
    if (what == "floor" || what == "all") probe_floor();
    if (what == "gather" || what == "all") probe_gather();
    if (what == "copy" || what == "all") probe_copy();
    return 0;
}

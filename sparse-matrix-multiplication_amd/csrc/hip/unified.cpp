// Unified-memory SpMM on one GPU (reference: src/spmm_multigpu.cu:122-182).

#include "spmm/spmm_multigpu.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "engine.h"
#include "hip_status.h"
#include "spmm/utils.h"

namespace spmm {

int gpu_count() {
    int n = 0;
    HIP_CHECK(hipGetDeviceCount(&n));
    return n;
}

namespace engine {

namespace {

// hipMemPrefetchAsync of one managed range.  *moved becomes false when the
// device cannot prefetch (that error is cleared); other failures are errors.
Error prefetch(const void* p, size_t bytes, int dev, bool* moved) {
    const hipError_t e = hipMemPrefetchAsync(p, bytes, dev, nullptr);
    if (e == hipSuccess) return Error{};
    if (e == hipErrorNotSupported || e == hipErrorInvalidDevice) {
        (void)hipGetLastError();
        *moved = false;
        return Error{};
    }
    return hip_error(e, "hipMemPrefetchAsync");
}

}  // namespace

Error run_unified(const CSR& h_A, const float* h_B, float* h_C, int N, int warmup, int iters,
                  float* ms, int* residency) {
    *ms = 0.f;
    *residency = kUnifiedPrefetched;
    const int M = h_A.num_rows;
    const int K = h_A.num_cols;
    if (M < 0 || K < 0 || N < 0 || h_A.nnz < 0) return Error{kInvalid, "negative dimension"};
    // Host arrays are read (and C written) before any launch: refuse missing
    // ones here rather than fault in the copies.
    if (h_A.row_ptr == nullptr ||
        (h_A.nnz > 0 && (h_A.col_idx == nullptr || h_A.values == nullptr)) ||
        (static_cast<size_t>(K) * N > 0 && h_B == nullptr) ||
        (static_cast<size_t>(M) * N > 0 && h_C == nullptr)) {
        return Error{kInvalid, "null host array"};
    }
    int dev = 0;
    SPMM_TRY_HIP(hipGetDevice(&dev), "hipGetDevice");
    int managed = 0;
    SPMM_TRY_HIP(hipDeviceGetAttribute(&managed, hipDeviceAttributeManagedMemory, dev),
                 "hipDeviceGetAttribute");

    const size_t rp_bytes = sizeof(int) * (static_cast<size_t>(M) + 1);
    const size_t nz = static_cast<size_t>(std::max(h_A.nnz, 1));
    const size_t b_bytes = sizeof(float) * std::max<size_t>(static_cast<size_t>(K) * N, 1);
    const size_t c_bytes = sizeof(float) * std::max<size_t>(static_cast<size_t>(M) * N, 1);
    DeviceBuffer rp, ci, va, ub, uc;
    CSR u_A;
    u_A.num_rows = M;
    u_A.num_cols = K;
    u_A.nnz      = h_A.nnz;
    if (!managed) {
        // No managed memory on this device (MI355X with XNACK off): device
        // allocations filled by explicit copies stand in for the managed
        // ranges, which is the state a successful prefetch reaches.  The GPU
        // never touches host memory.
        *residency = kUnifiedDeviceCopies;
        SPMM_TRY_HIP(hipMalloc(&rp.p, rp_bytes), "hipMalloc");
        SPMM_TRY_HIP(hipMalloc(&ci.p, sizeof(int) * nz), "hipMalloc");
        SPMM_TRY_HIP(hipMalloc(&va.p, sizeof(float) * nz), "hipMalloc");
        SPMM_TRY_HIP(hipMalloc(&ub.p, b_bytes), "hipMalloc");
        SPMM_TRY_HIP(hipMalloc(&uc.p, c_bytes), "hipMalloc");
        SPMM_TRY_HIP(hipMemcpy(rp.p, h_A.row_ptr, rp_bytes, hipMemcpyHostToDevice), "hipMemcpy");
        if (h_A.nnz > 0) {
            SPMM_TRY_HIP(hipMemcpy(ci.p, h_A.col_idx, sizeof(int) * h_A.nnz,
                                   hipMemcpyHostToDevice), "hipMemcpy");
            SPMM_TRY_HIP(hipMemcpy(va.p, h_A.values, sizeof(float) * h_A.nnz,
                                   hipMemcpyHostToDevice), "hipMemcpy");
        }
        if (static_cast<size_t>(K) * N > 0) {
            SPMM_TRY_HIP(hipMemcpy(ub.p, h_B, sizeof(float) * static_cast<size_t>(K) * N,
                                   hipMemcpyHostToDevice), "hipMemcpy");
        }
        u_A.row_ptr = rp.as<int>();
        u_A.col_idx = ci.as<int>();
        u_A.values  = va.as<float>();
        SPMM_TRY(time_median_launch(
            [&] { return launch_csr(CsrRole::TiledV3, u_A, ub.as<float>(), uc.as<float>(), N, nullptr); },
            warmup, iters, ms));
        SPMM_TRY_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (static_cast<size_t>(M) * N > 0) {
            SPMM_TRY_HIP(hipMemcpy(h_C, uc.p, sizeof(float) * static_cast<size_t>(M) * N,
                                   hipMemcpyDeviceToHost), "hipMemcpy");
        }
        return Error{};
    }
    SPMM_TRY_HIP(hipMallocManaged(&rp.p, rp_bytes), "hipMallocManaged");
    SPMM_TRY_HIP(hipMallocManaged(&ci.p, sizeof(int) * nz), "hipMallocManaged");
    SPMM_TRY_HIP(hipMallocManaged(&va.p, sizeof(float) * nz), "hipMallocManaged");
    SPMM_TRY_HIP(hipMallocManaged(&ub.p, b_bytes), "hipMallocManaged");
    SPMM_TRY_HIP(hipMallocManaged(&uc.p, c_bytes), "hipMallocManaged");
    std::copy(h_A.row_ptr, h_A.row_ptr + M + 1, rp.as<int>());
    std::copy(h_A.col_idx, h_A.col_idx + h_A.nnz, ci.as<int>());
    std::copy(h_A.values, h_A.values + h_A.nnz, va.as<float>());
    std::copy(h_B, h_B + static_cast<size_t>(K) * N, ub.as<float>());

    bool moved = true;
    SPMM_TRY(prefetch(rp.p, rp_bytes, dev, &moved));
    SPMM_TRY(prefetch(ci.p, sizeof(int) * nz, dev, &moved));
    SPMM_TRY(prefetch(va.p, sizeof(float) * nz, dev, &moved));
    SPMM_TRY(prefetch(ub.p, b_bytes, dev, &moved));
    SPMM_TRY(prefetch(uc.p, c_bytes, dev, &moved));
    SPMM_TRY_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (!moved) *residency = kUnifiedFirstTouch;

    u_A.row_ptr  = rp.as<int>();
    u_A.col_idx  = ci.as<int>();
    u_A.values   = va.as<float>();
    SPMM_TRY(time_median_launch(
        [&] { return launch_csr(CsrRole::TiledV3, u_A, ub.as<float>(), uc.as<float>(), N, nullptr); },
        warmup, iters, ms));
    SPMM_TRY_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    std::copy(uc.as<float>(), uc.as<float>() + static_cast<size_t>(M) * N, h_C);
    return Error{};
}

}  // namespace engine

float spmm_unified(const CSR& h_A, const float* h_B, float* h_C, int N, int warmup, int iters) {
    float ms = 0.f;
    int residency = engine::kUnifiedPrefetched;
    const engine::Error e =
        engine::run_unified(h_A, h_B, h_C, N, warmup, iters, &ms, &residency);
    if (e.status != engine::kOk) {
        std::fprintf(stderr, "spmm_unified: %s\n", e.message.c_str());
        std::exit(EXIT_FAILURE);
    }
    if (residency == engine::kUnifiedFirstTouch) {
        std::fprintf(stderr, "spmm_unified: this device cannot prefetch managed memory; "
                             "pages moved on first touch\n");
    } else if (residency == engine::kUnifiedDeviceCopies) {
        std::fprintf(stderr, "spmm_unified: this device has no managed memory; device copies "
                             "stood in for the prefetched managed ranges\n");
    }
    return ms;
}

}  // namespace spmm

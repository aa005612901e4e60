// Fill-in based dispatch (reference: src/spmm_hybrid.cu:28-125).

#include "spmm/spmm_hybrid.h"

#include <vector>

#include "engine.h"
#include "spmm/bsr.h"
#include "spmm/metrics.h"
#include "spmm/partition.h"
#include "spmm/utils.h"

namespace spmm {

namespace {

void exit_on_error(const engine::Error& e, const char* who) {
    if (e.status == engine::kOk) return;
    std::fprintf(stderr, "%s: %s\n", who, e.message.c_str());
    std::exit(EXIT_FAILURE);
}

// warmup untimed launches, then iters launches each bracketed by events.
template <typename Launch>
float time_median_ms(Launch launch, int warmup, int iters) {
    for (int i = 0; i < warmup; ++i) launch();
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> times(static_cast<size_t>(iters > 0 ? iters : 0));
    GpuTimer timer;
    for (int i = 0; i < iters; ++i) {
        timer.start();
        launch();
        timer.stop();
        times[i] = timer.elapsed_ms();
    }
    return median(times);
}

}  // namespace

const char* backend_name(Backend b) { return b == Backend::TENSOR_WMMA ? "wmma" : "csr"; }

HybridPlan hybrid_choose(const CSR& h_A, int N, float fill_in_threshold) {
    HybridPlan plan;
    plan.threshold = fill_in_threshold;
    plan.n_aligned = N > 0 && N % BSR_BLOCK == 0;
    // The reference builds the whole BSR here only to read its statistics
    // (spmm_hybrid.cu:38); counting blocks gives the same numbers.
    const BSR_stats st = bsr_stats_from_csr_host(h_A);
    plan.fill_in_ratio = st.fill_in_ratio;
    plan.block_density = st.block_density;
    if (plan.n_aligned && st.fill_in_ratio <= fill_in_threshold) {
        plan.backend = Backend::TENSOR_WMMA;
        plan.reason  = "low BSR fill-in and N aligned to 16 -> Tensor Cores";
    } else if (!plan.n_aligned) {
        plan.backend = Backend::CSR_TILED;
        plan.reason  = "N not a multiple of 16 -> CUDA-core CSR";
    } else {
        plan.backend = Backend::CSR_TILED;
        plan.reason  = "high BSR fill-in -> CUDA-core CSR";
    }
    return plan;
}

float spmm_hybrid_run(const HybridPlan& plan, const CSR& h_A, const float* h_B, float* h_C,
                      int N, int warmup, int iters) {
    const int M = h_A.num_rows;
    const int K = h_A.num_cols;
    const size_t b_elems = static_cast<size_t>(K) * N;
    const size_t c_elems = static_cast<size_t>(M) * N;
    if (c_elems == 0) return 0.f;

    float* d_B = nullptr;
    float* d_C = nullptr;
    HIP_CHECK(hipMalloc(&d_B, sizeof(float) * (b_elems > 0 ? b_elems : 1)));
    HIP_CHECK(hipMalloc(&d_C, sizeof(float) * c_elems));
    if (b_elems > 0) {
        HIP_CHECK(hipMemcpy(d_B, h_B, sizeof(float) * b_elems, hipMemcpyHostToDevice));
    }

    float ms = 0.f;
    if (plan.backend == Backend::TENSOR_WMMA) {
        // Upload the CSR (8 bytes per nonzero; the BSR is 512 bytes per block)
        // and build the BSR on the device.  Inputs the device builder does not
        // take (rows with descending column indices, num_cols > 4128768) are
        // built on the host as in the reference (spmm_hybrid.cu:78-80).
        BSR d_bsr;
        {
            CSR d_A = csr_to_device(h_A);
            const engine::Error built = engine::build_bsr_device(d_A, &d_bsr, nullptr);
            csr_free_device(d_A);
            if (built.status == engine::kUnsupported) {
                d_bsr = bsr_to_device(bsr_from_csr_host(h_A));
            } else {
                exit_on_error(built, "spmm_hybrid_run");
            }
        }
        half* d_B16 = nullptr;
        HIP_CHECK(hipMalloc(&d_B16, sizeof(half) * (b_elems > 0 ? b_elems : 1)));
        exit_on_error(engine::launch_float_to_half(d_B, d_B16, static_cast<long>(b_elems), nullptr),
                      "spmm_hybrid_run");
        HIP_CHECK(hipDeviceSynchronize());
        ms = time_median_ms(
            [&] { exit_on_error(engine::launch_bsr(d_bsr, d_B16, d_C, N, nullptr), "spmm_hybrid_run"); },
            warmup, iters);
        HIP_CHECK(hipFree(d_B16));
        bsr_free_device(d_bsr);
    } else {
        CSR d_A = csr_to_device(h_A);
        const int parts = engine::default_partition_parts(M, h_A.nnz);
        const std::vector<int> bounds = nnz_balanced_bounds(h_A, parts);
        int* d_bounds = nullptr;
        HIP_CHECK(hipMalloc(&d_bounds, sizeof(int) * bounds.size()));
        HIP_CHECK(hipMemcpy(d_bounds, bounds.data(), sizeof(int) * bounds.size(),
                            hipMemcpyHostToDevice));
        ms = time_median_ms(
            [&] {
                exit_on_error(engine::launch_csr(engine::CsrRole::TiledV3, d_A, d_B, d_C, N, nullptr,
                                                 d_bounds, parts),
                              "spmm_hybrid_run");
            },
            warmup, iters);
        HIP_CHECK(hipFree(d_bounds));
        csr_free_device(d_A);
    }
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(h_C, d_C, sizeof(float) * c_elems, hipMemcpyDeviceToHost));
    HIP_CHECK(hipFree(d_B));
    HIP_CHECK(hipFree(d_C));
    return ms;
}

}  // namespace spmm

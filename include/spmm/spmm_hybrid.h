#pragma once
// Fill-in based dispatch between the CSR engine and the BSR/MFMA kernel.
//
// Drop-in for the reference's src/spmm_hybrid.h (spmm_hybrid.h:24-64): same
// enum, plan struct, function names, default arguments and reason strings.
// The rule is the reference's (spmm_hybrid.cu:32-56): matrix cores iff
// N % 16 == 0 && N > 0 && fill_in <= threshold.  The default threshold is the
// MI355X crossover (kHybridDefaultThreshold below), measured by timing both
// back ends over a fill-in sweep.

#include "csr.h"

namespace spmm {

enum class Backend {
    CSR_TILED,    // CSR row-block engine (spmm_tiled_v3)
    TENSOR_WMMA   // BSR 16x16 on v_mfma_f32_16x16x32_f16 (spmm_wmma)
};

struct HybridPlan {
    Backend backend       = Backend::CSR_TILED;
    double  fill_in_ratio = 0.0;   // BSR stored elements / nnz
    double  block_density = 0.0;   // non-empty 16x16 blocks / all blocks
    float   threshold     = 0.0f;  // fill-in cut-off used
    bool    n_aligned     = false; // N % 16 == 0
    const char* reason    = "";
};

// Fill-in at or below which the MFMA path wins on MI355X.  Timing both back
// ends (spmm_tiled_v3 and spmm_wmma kernels, warm) on 61 inputs -- uniform
// random 4096^2 .. 16384^2 at fill 10 .. 50, random and banded partially
// filled blocks at fill 10 .. 45, the five BASELINE configs -- at N = 128 and
// 256: any cut-off in 26 .. 32 loses 5.2% on average to the faster back end
// (59 us in total); 18 loses 15.5% (394 us), 45 loses 3.2% but 208 us, most
// of it on large uniform inputs at fill 33 - 50, where the CSR engine is up
// to 2x faster.  The remaining misses are uniform inputs at fill 25 - 33,
// within 15% either way, and partially filled blocks at fill 45, where the
// MFMA kernel is 1.1 - 1.5x faster.  The reference's 2.0 was the crossover of
// a T4, whose tensor cores are far less ahead of its CUDA cores.
constexpr float kHybridDefaultThreshold = 32.0f;

HybridPlan hybrid_choose(const CSR& h_A, int N,
                         float fill_in_threshold = kHybridDefaultThreshold);

// "csr" / "wmma" (spmm_hybrid.cu:28-30).
const char* backend_name(Backend b);

// Host-in / host-out execution of the chosen back end: uploads A (as CSR or
// BSR), B (fp32, converted on the device to fp16 for the MFMA path), runs
// `warmup` untimed and `iters` timed launches (hipEvents per launch on the null
// stream, like spmm_hybrid.cu:87-116), copies C back and returns the median
// per-launch time in milliseconds.  Setup is outside the timed region.
// The CSR branch launches the engine with the host-computed nnz-balanced
// workgroup partition (nnz_balanced_bounds), uploaded once with A.
float spmm_hybrid_run(const HybridPlan& plan,
                      const CSR& h_A, const float* h_B, float* h_C,
                      int N, int warmup, int iters);

}  // namespace spmm

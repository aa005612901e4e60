#pragma once
// Fill-in based dispatch between the CSR engine and the BSR/MFMA kernel.
//
// Drop-in for the reference's src/spmm_hybrid.h (spmm_hybrid.h:24-64): same
// enum, plan struct, function names, default arguments and reason strings.
// The rule is the reference's (spmm_hybrid.cu:32-56): matrix cores iff
// N % 16 == 0 && N > 0 && fill_in <= threshold.  The default threshold is the
// MI355X crossover for the given N (hybrid_default_threshold below), measured
// by timing both back ends over a fill-in sweep.

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

// Fill-in at or below which the MFMA path wins on MI355X for a B of N
// columns.  Timing both back ends as spmm_hybrid_run runs them (the CSR side
// is the engine, its merge-path form or the sub-wave row groups, by the same
// rule) on 33 inputs per N -- uniform random 4096^2 .. 16384^2 at fill
// 10 .. 50, random and banded partially filled blocks at fill 10 .. 45, the
// five BASELINE matrices -- the cut-off that loses least to the faster back
// end is 6 - 8 at N = 16 (0.6% on average), 10 - 14 at N = 32 (2.2%), 16 - 18
// at N = 64 (1.4%), 22 - 24 at N = 128 (1.8%) and 26 - 32 at N = 256 (0.0%).
// Narrow B favours the CSR side: its row groups keep every lane busy there,
// while a 16x16 block costs the MFMA kernel the same whatever N is.  A single
// cut-off of 32 would lose 28% on average at N = 16.  The reference's 2.0 was
// the crossover of a T4, whose tensor cores are far less ahead of its CUDA
// cores.
float hybrid_default_threshold(int N);

// The cut-off for wide B (N >= 256), hybrid_default_threshold's largest value.
constexpr float kHybridDefaultThreshold = 32.0f;

// Default argument of hybrid_choose: any negative threshold selects
// hybrid_default_threshold(N); the plan records the value used.
constexpr float kHybridAutoThreshold = -1.0f;

HybridPlan hybrid_choose(const CSR& h_A, int N,
                         float fill_in_threshold = kHybridAutoThreshold);

// "csr" / "wmma" (spmm_hybrid.cu:28-30).
const char* backend_name(Backend b);

// Host-in / host-out execution of the chosen back end: uploads A (as CSR or
// BSR), B (fp32, converted on the device to fp16 for the MFMA path), runs
// `warmup` untimed and `iters` timed launches (hipEvents per launch on the null
// stream, like spmm_hybrid.cu:87-116), copies C back and returns the median
// per-launch time in milliseconds.  Setup is outside the timed region.
// The CSR branch picks from the host CSR's row lengths: sub-wave row groups
// (narrow B, short rows, N <= 128 on >= 4096 even rows), the merge-path
// partition (a row of more than 2560 entries, its row table and carry
// workspace set up once; split over B-row halves, one per group of four XCDs,
// when B is over one XCD's 4 MiB L2 and half of its rows fit), or the
// row-block engine given the longest row.
float spmm_hybrid_run(const HybridPlan& plan,
                      const CSR& h_A, const float* h_B, float* h_C,
                      int N, int warmup, int iters);

}  // namespace spmm

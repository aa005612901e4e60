#pragma once
// Error statistics, median and the host reference SpMM loops used by the
// drivers to verify a device result.
//
// compare / median / rel_l2 follow harness.cu:173-201 and spmm_run.cu:157-165.
// The reference verifies against cuSPARSE; this engine's drivers verify against
// spmm_host_reference_f64 (CSR, fp64 accumulation) and
// spmm_host_reference_bsr_f32 (fp32 accumulation of the fp16-rounded operands).
// Those loops are verification only: no device entry point ever falls back to
// them.

#include <vector>

#include "bsr.h"
#include "csr.h"

namespace spmm {

struct ErrorStats {
    float max_abs = 0.f;
    float max_rel = 0.f;  // only cells with |ref| > 1e-3 * max|ref|
    float rel_l2  = 0.f;  // ||ours - ref||_2 / ||ref||_2, fp64 sums
};

ErrorStats compare(const std::vector<float>& ours, const std::vector<float>& ref);
float median(std::vector<float> v);  // v[n/2] after sort; 0 for empty input
float rel_l2(const std::vector<float>& ours, const std::vector<float>& ref);

// C (M x N) = A * B with every product and sum in fp64, rows split over
// `threads` std::threads by nnz_balanced_bounds (threads <= 0: hardware
// concurrency).  C is returned rounded to fp32.
std::vector<float> spmm_host_reference_f64(const CSR& h_A, const float* h_B,
                                           int N, int threads);

// C = A_bsr * B16 accumulated in fp32 over the fp16 values of A and of
// fp16(B), block by block in block-column order, k ascending inside a block.
std::vector<float> spmm_host_reference_bsr_f32(const BSR_host& h_A,
                                               const float* h_B, int N,
                                               int threads);

}  // namespace spmm

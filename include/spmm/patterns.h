#pragma once
// Synthetic inputs: the dense B generator of the reference drivers and the
// structured sparsity patterns of scripts/gen_matrices.py restated in C++.
//
// The pattern structure follows gen_matrices.py:37-81; the random streams are
// this engine's own (std::mt19937 seeded as documented per function), not
// numpy's, so matrices are reproducible from C++ alone.

#include <vector>

#include "csr.h"

namespace spmm {

// rows*cols fp32 U[-1,1) from std::mt19937(seed) with
// uniform_real_distribution<float>(-1,1), row-major (harness.cu:114-120,
// spmm_run.cu:99-105).
std::vector<float> generate_dense_row_major(int rows, int cols, int seed);

// Every cell with |r - c| <= half_bandwidth (cols clipped to [0, cols)), as
// gen_matrices.py:37-48.  Values U[-1,1) drawn in CSR order from mt19937(seed).
CSR generate_banded_csr(int rows, int cols, int half_bandwidth, int seed);

// floor(min(rows, cols) / block) dense block x block blocks on the diagonal, as
// gen_matrices.py:51-63.  Values N(0,1) * value_scale in CSR order: Box-Muller
// on two mt19937(seed) doubles in (0, 1], cosine branch only.
CSR generate_block_diagonal_csr(int rows, int cols, int block, int seed,
                                float value_scale = 0.1f);

// The same structure with values U[-1,1) in CSR order from mt19937(seed) (the
// value distribution of gen_matrices.py:62, used by its CLI).
CSR generate_block_diagonal_uniform_csr(int rows, int cols, int block, int seed);

// Power-law rows, as gen_matrices.py:66-81: x_r = (1 - u_r)^(-1/alpha) (Pareto
// with x_m = 1, i.e. numpy's pareto(alpha) + 1), scaled so the sample mean is
// mean_deg, rounded half-to-even, clipped to [1, min(cols, max_row_nnz)].
// Each row's columns are distinct and uniform (Floyd's sampling); values
// U[-1,1) in CSR order.  All draws come from one mt19937(seed).
CSR generate_power_law_csr(int rows, int cols, double mean_deg, double alpha,
                           int max_row_nnz, int seed);

// Round every value of a host CSR through fp16 (RNE) and back, so the CSR and
// BSR back ends multiply identical operands (used for the fp16 configs).
void csr_round_values_to_fp16(CSR& h);
// Same for a dense buffer.
void dense_round_to_fp16(float* v, long n);

}  // namespace spmm

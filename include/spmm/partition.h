#pragma once
// nnz-balanced contiguous row partition.
//
// The reference uses it to split rows over GPUs (spmm_multigpu.cu:26-40); here
// it splits rows over workgroups of the CSR engine (and over host threads in
// the verification loop).  bounds[g]..bounds[g+1] is part g: bounds[0] = 0,
// bounds[parts] = num_rows, bounds[g] is the first row r with
// row_ptr[r] >= nnz * g / parts (64-bit target), then made non-decreasing.

#include <vector>

#include "csr.h"

namespace spmm {

std::vector<int> nnz_balanced_bounds(const CSR& h_A, int parts);

// Row table of the merge-path (nonzero-split) partition used by the CSR
// engine: part g covers nonzeros [nnz*g/parts, nnz*(g+1)/parts) (64-bit); rows[g]
// is the row holding nonzero nnz*g/parts (the last row r < num_rows with
// row_ptr[r] <= that index), rows[0] = 0, rows[parts] = num_rows.  Rows may be
// split between parts.  Requires nnz >= 1.
std::vector<int> nnz_split_rows(const CSR& h_A, int parts);

}  // namespace spmm
